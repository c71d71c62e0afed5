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
