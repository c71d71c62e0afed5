"""aotolith_amd - an MI355X-native (gfx950) kernel backend for aotolith's W4 decoder path.

Target name: ``"hip-gfx950"``. Kernels are hand-written HIP for CDNA4, built into
one gfx950 code object and reached through the C ABI of ``include/aoto_hip.h``
from torch-ROCm tensors.
"""

from __future__ import annotations

from ._version import __version__

TARGET = "hip-gfx950"

__all__ = ["TARGET", "__version__"]
