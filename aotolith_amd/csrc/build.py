"""Build the gfx950 code object and the C-ABI host library, in-tree.

Outputs (next to the package, so they travel with the source tree):

* ``aotolith_amd/aoto_gfx950.hsaco`` - every kernel, ``hipcc --genco`` for gfx950;
* ``aotolith_amd/libaoto_hip.so``     - the ``extern "C"`` launchers of
  ``include/aoto_hip.h``.

Run ``python -m aotolith_amd.csrc.build`` or call :func:`build`.
"""

from __future__ import annotations

import os
import subprocess
import sys

CSRC = os.path.dirname(os.path.abspath(__file__))
PACKAGE = os.path.dirname(CSRC)
ROOT = os.path.dirname(PACKAGE)
INCLUDE = os.path.join(ROOT, "include")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ROCM = os.path.dirname(os.path.dirname(HIPCC))

CODE_OBJECT = os.path.join(PACKAGE, "aoto_gfx950.hsaco")
LIBRARY = os.path.join(PACKAGE, "libaoto_hip.so")

# Device flags: gfx950 only; packed-FP32 VALU forms disabled (they are not used
# by hand and the compiler is told not to form them); kernel arguments preloaded
# into SGPRs (up to 14 dwords on gfx950, so a kernel's first loads need not wait
# for a scalar load of its argument buffer; kernels order their arguments for
# it).
DEVICE_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-mllvm",
    "-amdgpu-kernarg-preload-count=16",
    "-I" + CSRC,
    "-I" + INCLUDE,
]


def _run(command: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(command), flush=True)
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        sys.stderr.write(result.stdout + result.stderr)
        raise RuntimeError(f"build step failed ({result.returncode}): {' '.join(command)}")


def build(verbose: bool = False) -> tuple[str, str]:
    """Compile the code object and the host library; return their paths."""

    tmp_obj = CODE_OBJECT + ".tmp"
    _run([HIPCC, *DEVICE_FLAGS, "--genco", "--no-gpu-bundle-output", os.path.join(CSRC, "kernels.hip"), "-o", tmp_obj], verbose)
    os.replace(tmp_obj, CODE_OBJECT)
    tmp_lib = LIBRARY + ".tmp"
    # The host library: the C-ABI launchers, plus noalloc.hip, whose device part is
    # only the static scratch buffer of the allocation-free GEMM entry point.
    _run(
        [
            HIPCC,
            "-O2",
            "-std=c++17",
            "-fPIC",
            "-shared",
            "--offload-arch=gfx950",
            "-Xclang",
            "-target-feature",
            "-Xclang",
            "-packed-fp32-ops",
            "-I" + INCLUDE,
            "-I" + CSRC,
            os.path.join(CSRC, "aoto_hip.cpp"),
            os.path.join(CSRC, "noalloc.hip"),
            "-o",
            tmp_lib,
        ],
        verbose,
    )
    os.replace(tmp_lib, LIBRARY)
    return CODE_OBJECT, LIBRARY


if __name__ == "__main__":
    for path in build(verbose=True):
        print(path, os.path.getsize(path))
