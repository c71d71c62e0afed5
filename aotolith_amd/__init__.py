"""aotolith_amd - an MI355X-native (gfx950) kernel backend for aotolith's W4 decoder path.

Target name: ``"hip-gfx950"``. Kernels are hand-written HIP for CDNA4, built into
one gfx950 code object and reached through the C ABI of ``include/aoto_hip.h``
from torch-ROCm tensors. The public names mirror the reference's API with
``target="hip-gfx950"``: the static-cache decoders (``compile_qwen2_static_cache``,
``compile_llama_static_cache`` and their bucketed forms) and the general
``compile_callable`` / ``compile_module`` graph compilers.
"""

from __future__ import annotations

from ._version import __version__
from .plan import TARGET

__all__ = [
    "TARGET",
    "__version__",
    "compile_callable",
    "compile_module",
    "compile_decoder_static_cache",
    "compile_decoder_bucketed",
    "compile_llama_bucketed",
    "compile_llama_static_cache",
    "compile_qwen2_bucketed",
    "compile_qwen2_static_cache",
    "load_bucketed",
    "load_compiled_module",
    "load_runtime",
    "read_artifact_manifest",
    "save_compiled",
]


def __getattr__(name: str):
    # The compile entry points import torch-side modules; keep `import aotolith_amd`
    # light for the C-ABI checks that run without a GPU.
    if name in ("compile_qwen2_static_cache", "compile_qwen2_bucketed"):
        from . import qwen2

        return getattr(qwen2, name)
    if name in ("compile_llama_static_cache", "compile_llama_bucketed"):
        from . import llama

        return getattr(llama, name)
    if name in ("compile_decoder_static_cache", "compile_decoder_bucketed"):
        from . import decoder

        return getattr(decoder, name)
    if name in ("compile_callable", "compile_module", "CompiledModulePlan", "CompilationResult"):
        from . import compiler

        return getattr(compiler, name)
    if name in ("load_runtime", "load_bucketed", "load_compiled_module", "read_artifact_manifest",
                "save_compiled"):
        from . import artifact

        return getattr(artifact, name)
    raise AttributeError(name)
