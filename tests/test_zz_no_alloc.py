"""The allocation-free prefill GEMM entry point, aoto_hip_w4_gemm_noalloc, called through the C ABI.

It is aoto_hip_w4_gemm without the workspace argument: a split-K plan keeps its partials in
the library's static per-device scratch buffer. Its output must be bit-identical to the
workspace entry point's on the same inputs (same kernels, same plan), on two calls in a row,
the second smaller (the buffer keeps the first call's partials, which must not leak into the
second); a plan whose partials exceed the buffer is refused before any launch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.quant import pack_weight_bf16
from tests.helpers import bf16_normal, to_gpu_bf16, to_gpu_bits

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20  # AOTO_HIP_NOALLOC_SCRATCH_BYTES


def _noalloc(x, packed, scales, group, out, *, bias=None, residual=None, tile=0, splits=0):
    from aotolith_amd import _lib, ops

    n, words = packed.shape
    k = words * 8
    m = x.numel() // k
    return _lib.library().aoto_hip_w4_gemm_noalloc(
        ops._ptr(x), ops._ptr(packed), ops._ptr(scales), ops._ptr(bias), ops._ptr(residual), None, ops._ptr(out),
        m, n, k, group, tile, splits, ops._stream(),
    )


def _last_error() -> str:
    import ctypes

    from aotolith_amd import _lib

    buf = ctypes.create_string_buffer(512)
    _lib.library().aoto_hip_last_error(buf, 512)
    return buf.value.decode()


def test_noalloc_gemm_matches_the_workspace_entry_point_on_two_calls():
    from aotolith_amd import ops

    # (M, N, K, epilogue): the Qwen prefill q/k/v projection (7-way split), then a smaller
    # o-projection-like call (fewer rows, a residual) that reuses the same scratch.
    for m, n, k, epilogue in [(128, 1152, 896, "bias"), (64, 896, 896, "residual")]:
        need = ops.gemm_workspace_bytes(m, n, k)
        assert 0 < need <= SCRATCH_BYTES, "the case must split, so the static scratch is used"
        rng = np.random.default_rng(m + n)
        packed, scales = pack_weight_bf16(bf16_normal(rng, (n, k), 0.02), 64)
        gp, gs = torch.from_numpy(packed).cuda(), to_gpu_bits(scales)
        x = to_gpu_bf16(bf16_normal(rng, (m, k)))
        kwargs = {}
        if epilogue == "bias":
            kwargs["bias"] = to_gpu_bf16(bf16_normal(rng, (n,), 0.02))
        else:
            kwargs["residual"] = to_gpu_bf16(bf16_normal(rng, (m, n)))
        want = ops.w4_matmul(x, gp, gs, 64, **kwargs)
        got = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        status = _noalloc(x, gp, gs, 64, got, **kwargs)
        assert status == 0, _last_error()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"M={m} N={n} K={k}"


def test_noalloc_gemm_takes_the_dequant_once_plan_where_the_workspace_entry_point_does():
    """At 2048 rows an o-shaped GEMM (256 blocks of 256 x 128) runs on the dequant-once
    kernel under automatic codes in both entry points - no split, so no scratch - and the
    two outputs are bit-identical."""

    from aotolith_amd import ops

    m, n, k = 2048, 4096, 1024
    assert ops.lds_plan(m, n, k) == ops.LDS_TILE
    rng = np.random.default_rng(95)
    packed, scales = pack_weight_bf16(bf16_normal(rng, (n, k), 0.02), 64)
    gp, gs = torch.from_numpy(packed).cuda(), to_gpu_bits(scales)
    x = to_gpu_bf16(bf16_normal(rng, (m, k)))
    residual = to_gpu_bf16(bf16_normal(rng, (m, n)))
    with ops.recording_launches() as take:
        take()
        want = ops.w4_matmul(x, gp, gs, 64, residual=residual)
        got = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        torch.cuda.synchronize()
        take()
        status = _noalloc(x, gp, gs, 64, got, residual=residual)
        names = take()
    torch.cuda.synchronize()
    assert status == 0, _last_error()
    assert names == ["aoto_w4_gemm_d8w2x2_b0_r1"], names
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_noalloc_gemm_takes_the_short_prompt_split_plan_where_the_workspace_entry_point_does():
    """At 128 rows a down-shaped GEMM (K = 4864 -> 896) runs as the dequant-once split-K
    partials (tile 813) plus the reduce under automatic codes in both entry points, its
    3.7 MB of partials in the static scratch, bit-identical to the workspace entry point;
    then a smaller call (64 rows) on the same scratch."""

    from aotolith_amd import ops

    for m in (128, 64):
        n, k = 896, 4864
        assert ops.lds_plan(m, n, k) == ops.LDS_SPLIT_NARROW_TILE
        assert 0 < ops.gemm_workspace_bytes(m, n, k) <= SCRATCH_BYTES
        rng = np.random.default_rng(96 + m)
        packed, scales = pack_weight_bf16(bf16_normal(rng, (n, k), 0.02), 64)
        gp, gs = torch.from_numpy(packed).cuda(), to_gpu_bits(scales)
        x = to_gpu_bf16(bf16_normal(rng, (m, k)))
        residual = to_gpu_bf16(bf16_normal(rng, (m, n)))
        with ops.recording_launches() as take:
            take()
            want = ops.w4_matmul(x, gp, gs, 64, residual=residual)
            got = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
            torch.cuda.synchronize()
            take()
            status = _noalloc(x, gp, gs, 64, got, residual=residual)
            names = take()
        torch.cuda.synchronize()
        assert status == 0, _last_error()
        assert names == ["aoto_w4_gemm_d4c1w1x1_split", "aoto_w4_gemm_reduce"], names
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), m


def test_noalloc_gemm_refuses_explicit_plans_beyond_its_scratch():
    from aotolith_amd import ops

    m, n, k = 512, 4096, 4096
    assert ops.gemm_workspace_bytes(m, n, k, 28, 4) > SCRATCH_BYTES  # 4 splits: 32 MiB of partials
    x = torch.zeros((m, k), dtype=torch.bfloat16, device="cuda")
    packed = torch.zeros((n, k // 8), dtype=torch.int32, device="cuda")
    scales = torch.zeros((n, k // 64), dtype=torch.bfloat16, device="cuda")
    out = torch.zeros((m, n), dtype=torch.bfloat16, device="cuda")
    status = _noalloc(x, packed, scales, 64, out, tile=28, splits=4)
    assert status == 4, status  # AOTO_ERR_UNSUPPORTED, before any launch
    assert "static scratch" in _last_error()
    torch.cuda.synchronize()
    assert not torch.any(out.view(torch.int16) != 0)


def test_noalloc_gemm_fits_automatic_plans_to_its_scratch():
    """Automatic codes whose split would need more than the scratch run with fewer splits:
    the 16x16 plan at 256 rows (N = 4096, K = 1536: 4 splits, 16.8 MB of partials on its
    own) and a wide plan at 1024 rows both match the workspace entry point under the plan
    the scratch allows, bit for bit; nothing is allocated (the device's free memory is
    unchanged)."""

    from aotolith_amd import ops

    for m, n, k, tile, splits in [(256, 4096, 1536, 0, 0), (1024, 1536, 4096, 241, 0)]:
        assert ops.lds_plan(m, n, k) is None
        rng = np.random.default_rng(90 + m)
        packed, scales = pack_weight_bf16(bf16_normal(rng, (n, k), 0.02), 64)
        gp, gs = torch.from_numpy(packed).cuda(), to_gpu_bits(scales)
        x = to_gpu_bf16(bf16_normal(rng, (m, k)))
        residual = to_gpu_bf16(bf16_normal(rng, (m, n)))
        auto = ops.gemm_workspace_bytes(m, n, k)
        # the largest split count whose partials fit, as the entry point chooses it
        if tile == 0:
            count = auto // (m * n * 4)
            while count > 1 and ops.gemm_workspace_bytes(m, n, k, 0, count) > SCRATCH_BYTES:
                count -= 1
            explicit = (0, count)
        else:
            plan = ops.wide_plan(m, n, k)
            count = plan[1]
            while count > 1 and ops.gemm_workspace_bytes(m, n, k, plan[0], count) > SCRATCH_BYTES:
                count -= 1
            explicit = (plan[0], count)
        want = ops.w4_matmul(x, gp, gs, 64, residual=residual, tile=explicit[0], splits=explicit[1])
        got = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        torch.cuda.synchronize()
        free_before = torch.cuda.mem_get_info()[0]
        status = _noalloc(x, gp, gs, 64, got, residual=residual)
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free_before
        assert status == 0, _last_error()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (m, n, k, explicit)
