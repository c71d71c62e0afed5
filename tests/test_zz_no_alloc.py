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


def test_noalloc_gemm_refuses_plans_beyond_its_scratch():
    from aotolith_amd import ops

    m, n, k = 512, 4096, 4096  # the auto plan splits 4 ways: 32 MiB of partials
    assert ops.gemm_workspace_bytes(m, n, k) > SCRATCH_BYTES
    x = torch.zeros((m, k), dtype=torch.bfloat16, device="cuda")
    packed = torch.zeros((n, k // 8), dtype=torch.int32, device="cuda")
    scales = torch.zeros((n, k // 64), dtype=torch.bfloat16, device="cuda")
    out = torch.zeros((m, n), dtype=torch.bfloat16, device="cuda")
    status = _noalloc(x, packed, scales, 64, out)
    assert status == 4, status  # AOTO_ERR_UNSUPPORTED, before any launch
    assert "static scratch" in _last_error()
    # the same shape unsplit needs no scratch and runs
    assert _noalloc(x, packed, scales, 64, out, splits=1) == 0, _last_error()
    torch.cuda.synchronize()
    assert not torch.any(out.view(torch.int16) != 0)


def test_noalloc_gemm_keeps_the_fused_kernel_for_long_prefills():
    """Automatic codes at 1024+ rows, which send aoto_hip_w4_gemm to the unpacked-weight
    library path, resolve to the fused kernel's own plan here (no room for the weight):
    the result is the workspace entry point's under that explicit plan, bit for bit."""

    from aotolith_amd import ops

    m, n, k = ops.LIBRARY_ROWS, 4096, 896  # 256 output tiles: the fused plan does not split
    rng = np.random.default_rng(90)
    packed, scales = pack_weight_bf16(bf16_normal(rng, (n, k), 0.02), 64)
    gp, gs = torch.from_numpy(packed).cuda(), to_gpu_bits(scales)
    x = to_gpu_bf16(bf16_normal(rng, (m, k)))
    bias = to_gpu_bf16(bf16_normal(rng, (n,), 0.02))
    want = ops.w4_matmul(x, gp, gs, 64, bias=bias, tile=28)  # 128-row, 128-column blocks
    got = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    with ops.recording_launches() as take:
        take()
        status = _noalloc(x, gp, gs, 64, got, bias=bias)
        names = take()
    assert status == 0, _last_error()
    torch.cuda.synchronize()
    assert not any(name.startswith("hipblaslt") for name in names), names
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
