"""The C-ABI library loads on the CPU and exports every symbol the header declares."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "aoto_hip.h")


def _declared() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(aoto_hip_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    assert "aoto_hip_w4_gemv" in names and "aoto_hip_load_code_object" in names


def test_library_exports_every_declared_symbol():
    from aotolith_amd import _lib

    lib = _lib.library()
    for name in _declared():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.aoto_hip_abi_version() == 17


def test_no_code_object_without_a_gpu():
    from aotolith_amd import _lib

    # No HIP device here: the loaded-check must say "not loaded" rather than crash.
    assert _lib.library().aoto_hip_code_object_loaded() == 0


def test_code_object_is_built_for_gfx950():
    from aotolith_amd import _lib

    image = _lib.default_code_object()
    assert image[:4] == b"\x7fELF"
    assert b"gfx950" in image


def test_launcher_rejects_bad_arguments_on_the_host():
    from aotolith_amd import _lib

    lib = _lib.library()
    status = lib.aoto_hip_w4_gemv(None, None, None, None, None, None, 0.0, None, 1.0, 1.0, None,
                                  896, 896, 64, 0, None)
    assert status == _lib.AOTO_ERR_ARGUMENT
    assert "null pointer" in _lib.last_error()


def test_library_plan_matches_the_workspace_queries():
    """ops.library_plan (the Python mirror of the automatic plan's rule) agrees with what the
    C ABI's workspace queries size - host logic only, no device call."""

    from aotolith_amd import _lib, ops

    lib = _lib.library()
    for m in (1, 128, 511, 512, 1023, 1024, 2048):
        for n, k in ((896, 896), (4096, 4096), (1152, 896), (6144, 4096), (4096, 14336), (640, 2048)):
            unpacked = n * k * 2 + m * n * 4
            assert (ops.gemm_workspace_bytes(m, n, k) == unpacked) == ops.library_plan(m, k), (m, n, k)
            assert (ops.gate_up_workspace_bytes(m, n, k) == 2 * n * k * 2 + m * n * 6) == ops.library_plan(m, k)
        for hq, hkv, d, k in ((14, 2, 64, 896), (32, 8, 128, 4096), (8, 2, 128, 2048)):
            n = (hq + 2 * hkv) * d
            got = lib.aoto_hip_w4_gemm_qkv_rope_workspace(m, k, 0, 0, hq, hkv, d)
            assert (got == n * k * 2 + m * n * 4) == ops.library_plan(m, k, qkv=True), (m, hq, k)
    # explicit codes always keep the fused kernel
    assert ops.gemm_workspace_bytes(2048, 4096, 4096, 28, 1) == 0
