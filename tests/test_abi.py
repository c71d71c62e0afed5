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
    assert lib.aoto_hip_abi_version() == 19


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


def test_wide_plan_matches_the_workspace_queries():
    """ops.wide_plan (the Python mirror of the automatic plan's rule) agrees with what the
    C ABI's workspace queries size: from ops.WIDE_ROWS rows (K % 256 == 0) a split plan
    needs splits * M * N f32 partials (twice that for the gate/up pair), an unsplit one
    none - host logic only, no device call."""

    from aotolith_amd import _lib, ops

    lib = _lib.library()
    seen = set()
    for m in (512, 640, 1024, 1100, 2048, 4096):
        assert ops.wide_plan(m, 896, 896) is None  # K % 256 != 0: the 16x16 kernel's plan
        for n, k in ((4096, 4096), (1152, 1024), (6144, 4096), (4096, 14336), (14336, 4096), (640, 2048),
                     (768, 512)):
            plan = ops.wide_plan(m, n, k)
            assert plan is not None, (m, n, k)
            tile, splits = plan
            seen.add(tile)
            want = splits * m * n * 4 if splits > 1 else 0
            assert ops.gemm_workspace_bytes(m, n, k) == want, (m, n, k, plan)
            ptile, psplits = ops.wide_plan(m, n, k, paired=True)
            assert ptile == 241
            assert ops.gate_up_workspace_bytes(m, n, k) == (2 * psplits * m * n * 4 if psplits > 1 else 0), (m, n, k)
        for hq, hkv, d, k in ((32, 8, 128, 4096), (8, 2, 128, 2048), (28, 4, 128, 3584)):
            n = (hq + 2 * hkv) * d
            tile, splits = ops.wide_plan(m, n, k)
            got = lib.aoto_hip_w4_gemm_qkv_rope_workspace(m, k, 0, 0, hq, hkv, d)
            assert got == (splits * m * n * 4 if splits > 1 else 0), (m, hq, k)
    assert seen == {241, 243, 441}, seen
    # below the wide rows, or K % 256 != 0, the 16x16 kernel's plan (no wide plan)
    assert ops.wide_plan(511, 4096, 4096) is None and ops.wide_plan(2048, 896, 896) is None
    # explicit codes are taken as given
    assert ops.gemm_workspace_bytes(2048, 4096, 4096, 28, 1) == 0
    assert ops.gemm_workspace_bytes(2048, 4096, 4096, 441, 2) == 2 * 2048 * 4096 * 4


def test_lds_plan_takes_the_full_rounds_at_long_prompts():
    """ops.lds_plan (the Python mirror of the C ABI's choice of the dequant-once kernel):
    at 2048 rows the Llama-3-8B o, down and paired gate/up projections (256 / 256 / 1792
    blocks: whole rounds of 256) take it, and q/k/v on 192-column blocks (384 blocks of 128
    columns would be 1.5 rounds, 256 of 192 are one); 1024-row o / down grids (128 blocks),
    8-bit codes, gate epilogues and odd group counts do not; at 32-256 rows the paired
    gate/up takes the 128-row forms (64 + 64 columns where that gives 128 blocks, else 32 +
    32 within one round), and single projections with K >= 2048 its split-K form, whose
    partials the automatic workspace query covers; its unsplit tiles need no split-K
    workspace - host logic only."""

    from aotolith_amd import ops

    assert ops.lds_plan(2048, 4096, 4096) == ops.LDS_TILE
    assert ops.lds_plan(2048, 4096, 14336) == ops.LDS_TILE
    assert ops.lds_plan(2048, 14336, 4096, paired=True) == ops.LDS_PAIRED_TILE
    assert ops.lds_plan(2048, 6144, 4096) == ops.LDS_WIDE_TILE
    assert ops.lds_plan(2048, 5120, 4096) is None  # 20 x 8 = 160 blocks of 256 x 128 columns
    assert ops.lds_plan(1024, 4096, 4096) is None and ops.lds_plan(1024, 14336, 4096, paired=True) is None
    assert ops.lds_plan(4096, 4096, 4096) == ops.LDS_TILE
    assert ops.lds_plan(2048, 4096, 4096, bits=8) is None
    assert ops.lds_plan(2048, 4096, 4096, gate=True) is None
    assert ops.lds_plan(2048, 4096, 4096 - 64, group_size=64) is None  # 63 groups per row
    assert ops.lds_plan(2048, 4096, 4096, group_size=96) is None
    # short prompts: the paired gate/up only, 128-row blocks
    assert ops.lds_plan(128, 4864, 896, paired=True) == ops.LDS_SHORT_NARROW_TILE  # 152 blocks of 32 + 32
    assert ops.lds_plan(64, 4864, 896, paired=True) == ops.LDS_SHORT_NARROW_TILE
    assert ops.lds_plan(256, 4864, 896, paired=True) == ops.LDS_SHORT_PAIRED_TILE  # 2 x 76 blocks of 64 + 64
    assert ops.lds_plan(128, 14336, 4096, paired=True) == ops.LDS_SHORT_PAIRED_TILE  # 224 blocks
    assert ops.lds_plan(64, 14336, 4096, paired=True) is None  # 448 blocks of 32 + 32: more than a round
    assert ops.lds_plan(16, 4864, 896, paired=True) is None and ops.lds_plan(300, 4864, 896, paired=True) is None
    assert ops.lds_plan(128, 4864, 896, paired=True, bits=8) is None
    # short prompts, single projections with K >= 2048 and no RoPE: the split-K form
    assert ops.lds_plan(128, 896, 4864) == ops.LDS_SPLIT_NARROW_TILE  # 28 column blocks of 32
    assert ops.lds_plan(128, 4096, 4096) == ops.LDS_SPLIT_TILE  # 64 column blocks of 64
    assert ops.lds_plan(128, 896, 896) is None and ops.lds_plan(128, 4864, 896) is None  # K < 2048
    assert ops.lds_plan(128, 6144, 4096, rope=True) is None and ops.lds_plan(16, 896, 4864) is None
    # the automatic workspace covers the split plan: 232 / 28 -> 8 slices of 10 steps (76 in all)
    assert ops.gemm_workspace_bytes(128, 896, 4864) == 8 * 128 * 896 * 4
    assert ops.gemm_workspace_bytes(128, 896, 4864, ops.LDS_SPLIT_NARROW_TILE, 1) == 128 * 896 * 4
    for tile in (ops.LDS_TILE, ops.LDS_WIDE_TILE, ops.LDS_PAIRED_TILE):
        assert ops.gemm_workspace_bytes(2048, 4096, 4096, tile, 0) == 0
        assert ops.gate_up_workspace_bytes(2048, 4096, 4096, tile, 0) == 0


def test_unload_is_refused_while_captured_graphs_are_held():
    """Host logic only: with a captured graph held, aoto_hip_unload_code_object refuses
    before touching any device (its modules would back the graph's kernel handles); a
    release below zero is refused; after the release the unload no longer names graphs."""

    from aotolith_amd import _lib

    lib = _lib.library()
    assert lib.aoto_hip_graph_holds() == 0
    assert lib.aoto_hip_hold_graphs(1) == _lib.AOTO_OK
    try:
        assert lib.aoto_hip_graph_holds() == 1
        assert lib.aoto_hip_unload_code_object() == _lib.AOTO_ERR_ARGUMENT
        assert "captured graphs still launch kernels" in _lib.last_error()
    finally:
        assert lib.aoto_hip_hold_graphs(-1) == _lib.AOTO_OK
    assert lib.aoto_hip_hold_graphs(-1) == _lib.AOTO_ERR_ARGUMENT
    assert lib.aoto_hip_graph_holds() == 0
    lib.aoto_hip_unload_code_object()  # no GPU here: a device error at most, never the graph refusal
    assert "captured graphs" not in _lib.last_error()


def test_hold_graph_is_released_when_the_graph_is_collected():
    import gc

    from aotolith_amd import _lib

    class Graph:  # stands in for torch.cuda.CUDAGraph (no GPU here)
        pass

    lib = _lib.library()
    graph = Graph()
    _lib.hold_graph(graph)
    assert lib.aoto_hip_graph_holds() == 1
    del graph
    gc.collect()
    assert lib.aoto_hip_graph_holds() == 0
