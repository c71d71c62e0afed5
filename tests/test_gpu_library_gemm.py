"""GPU parity of the long-prefill GEMM path: the unpacked weight on hipBLASLt.

From ``ops.LIBRARY_ROWS`` rows on, the prefill GEMMs' automatic plan (tile = splits = 0)
unpacks the packed weight to bf16 with the bit-exact dequant kernel and runs the
product on hipBLASLt (f32 accumulation); each epilogue rounds where the fused
kernels round. Every form is compared with the CPU oracle within one bf16 ulp (two
for the silu_mul products, as for the fused kernels), with the fused kernel under an
explicit plan, and - captured in a HIP graph - replay by replay with its eager result.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ops as oracle
from oracle.bf16 import round_bf16
from oracle.quant import pack_weight_bits_bf16
from tests.helpers import assert_bf16_parity, bf16_normal, from_gpu_bf16, to_gpu_bf16, to_gpu_bits

pytestmark = pytest.mark.gpu


def _ops():
    from aotolith_amd import ops

    return ops


def _weights(rng, n, k, bits, group=64):
    packed, scales = pack_weight_bits_bf16(bf16_normal(rng, (n, k), 0.02), group, bits)
    return packed, scales, torch.from_numpy(packed).cuda(), to_gpu_bits(scales)


def _atol(expected):
    # residuals of std 2 put outputs at |y| ~ 8, where one bf16 ulp (2^-5) exceeds the
    # 2e-2 bar meant for O(1) outputs: scale the bar with |y|
    return 2e-2 * max(1.0, float(np.abs(expected).max()) / 4)


def _traced(fn):
    ops = _ops()
    with ops.recording_launches() as take:
        take()
        out = fn()
        names = take()
    return out, names


def test_library_rows_threshold_matches_the_workspace_query():
    ops = _ops()
    m, n, k = ops.LIBRARY_ROWS, 1152, 1024
    # the library path's workspace: the unpacked weight, then the f32 product
    assert ops.gemm_workspace_bytes(m, n, k) == n * k * 2 + m * n * 4
    assert ops.gate_up_workspace_bytes(m, n, k) == 2 * n * k * 2 + m * n * 4 + m * n * 2
    # one row fewer, or any explicit code, keeps the fused kernel's split-K partials
    assert ops.gemm_workspace_bytes(m - 1, n, k) % ((m - 1) * n * 4) == 0
    assert ops.gemm_workspace_bytes(m, n, k, 28, 0) % (m * n * 4) == 0
    assert ops.gemm_workspace_bytes(m, n, k, 0, 1) == 0


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m", [1024, 1100])
@pytest.mark.parametrize("epilogue", ["none", "bias", "residual", "gate"])
def test_library_gemm_matches_the_oracle_and_the_fused_kernel(epilogue, m, bits):
    ops = _ops()
    n, k = 1152, 1024
    rng = np.random.default_rng(500 + m + bits + len(epilogue))
    packed, scales, gp, gs = _weights(rng, n, k, bits)
    x = bf16_normal(rng, (m, k))
    kwargs = {}
    if epilogue == "bias":
        kwargs["bias"] = bf16_normal(rng, (n,), 0.5)
    elif epilogue == "residual":
        kwargs["residual"] = bf16_normal(rng, (m, n), 2.0)
    elif epilogue == "gate":
        kwargs["gate"] = bf16_normal(rng, (m, n))
    gkw = {key: to_gpu_bf16(value) for key, value in kwargs.items()}
    matmul = ops.w4_matmul if bits == 4 else ops.w8_matmul
    gx = to_gpu_bf16(x)
    y, names = _traced(lambda: matmul(gx, gp, gs, 64, **gkw))
    dequant = "aoto_w4_dequantize" if bits == 4 else "aoto_w8_dequantize"
    product = "hipblaslt_matmul_f32" if epilogue == "gate" else "hipblaslt_matmul_bf16"
    assert names[:2] == [dequant, product], names
    fused, fused_names = _traced(lambda: matmul(gx, gp, gs, 64, tile=28, splits=1, **gkw))
    assert not any(name.startswith("hipblaslt") for name in fused_names)
    ulp = 2.0 if epilogue == "gate" else 1.0
    expected = oracle.w4_matmul(x, packed, scales, 64, bits=bits, **kwargs)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=ulp, atol=_atol(expected))
    assert_bf16_parity(from_gpu_bf16(y), from_gpu_bf16(fused), max_ulp=ulp, atol=_atol(expected))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [32, 128])
def test_library_gemm_other_group_sizes(group, bits):
    """The unpack takes any group size the GEMM accepts: groups of 32 and 128 at 1024 rows."""

    ops = _ops()
    m, n, k = 1024, 640, 1024
    rng = np.random.default_rng(560 + group + bits)
    packed, scales, gp, gs = _weights(rng, n, k, bits, group)
    x = bf16_normal(rng, (m, k))
    bias = bf16_normal(rng, (n,), 0.5)
    matmul = ops.w4_matmul if bits == 4 else ops.w8_matmul
    y, names = _traced(lambda: matmul(to_gpu_bf16(x), gp, gs, group, bias=to_gpu_bf16(bias)))
    assert "hipblaslt_matmul_bf16" in names, names
    expected = oracle.w4_matmul(x, packed, scales, group, bias=bias, bits=bits)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=1.0, atol=_atol(expected))


def test_library_gemm_in_place_residual():
    ops = _ops()
    m, n, k = 1024, 896, 1024
    rng = np.random.default_rng(510)
    packed, scales, gp, gs = _weights(rng, n, k, 4)
    x = bf16_normal(rng, (m, k))
    residual = bf16_normal(rng, (m, n), 2.0)
    buf = to_gpu_bf16(residual)
    ops.w4_matmul(to_gpu_bf16(x), gp, gs, 64, residual=buf, out=buf)
    expected = oracle.w4_matmul(x, packed, scales, 64, residual=residual)
    assert_bf16_parity(from_gpu_bf16(buf), expected, max_ulp=1.0, atol=_atol(expected))


@pytest.mark.parametrize("bits", [4, 8])
def test_library_gate_up_matches_the_oracle(bits):
    """The paired form: the gate GEMM rounded to bf16, then the up GEMM with the gate
    epilogue, y = bf16(up * silu(gate)) - within the bars of the oracle's two-step result."""

    ops = _ops()
    m, n, k = 1024, 1152, 1024
    rng = np.random.default_rng(520 + bits)
    gpk, gsc, g_packed, g_scales = _weights(rng, n, k, bits)
    upk, usc, u_packed, u_scales = _weights(rng, n, k, bits)
    x = bf16_normal(rng, (m, k))
    gate_up = ops.w4_matmul_gate_up if bits == 4 else ops.w8_matmul_gate_up
    gx = to_gpu_bf16(x)
    y, names = _traced(lambda: gate_up(gx, g_packed, g_scales, u_packed, u_scales, 64))
    assert names[2:] == ["hipblaslt_matmul_bf16", "hipblaslt_matmul_f32", "aoto_w4_gemm_reduce"], names
    want_gate = round_bf16(oracle.w4_matmul(x, gpk, gsc, 64, bits=bits))
    expected = oracle.w4_matmul(x, upk, usc, 64, gate=want_gate, bits=bits)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=2.0)
    fused = gate_up(gx, g_packed, g_scales, u_packed, u_scales, 64, tile=18, splits=1)
    assert_bf16_parity(from_gpu_bf16(y), from_gpu_bf16(fused), max_ulp=2.0)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("n", [896, 4096])
def test_library_residual_norm_matches_the_oracle(n, bits):
    ops = _ops()
    m, k = 1024, 1024
    rng = np.random.default_rng(530 + n + bits)
    packed, scales, gp, gs = _weights(rng, n, k, bits)
    x = bf16_normal(rng, (m, k))
    residual = bf16_normal(rng, (m, n), 2.0)
    weight = bf16_normal(rng, (n,), 0.5)
    y = to_gpu_bf16(residual)
    (_, norm), names = _traced(lambda: ops.matmul_residual_norm(to_gpu_bf16(x), gp, gs, 64, y, to_gpu_bf16(weight),
                                                                  1e-6, bits=bits, out=y))
    assert "hipblaslt_matmul_bf16" in names and names[-1] == "aoto_rms_norm", names
    expected = oracle.w4_matmul(x, packed, scales, 64, residual=residual, bits=bits)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=1.0, atol=_atol(expected))
    assert_bf16_parity(from_gpu_bf16(norm), oracle.rms_norm(from_gpu_bf16(y), weight, 1e-6), max_ulp=1.0)


def test_library_qkv_rule_from_512_rows_at_8b_widths():
    """The q/k/v RoPE form takes the library path from 512 rows when K >= 2048 (its fused
    form carries the RoPE epilogue), every other form from 1024."""

    from aotolith_amd import _lib

    ops = _ops()
    lib = _lib.library()
    n = (32 + 2 * 8) * 128
    assert lib.aoto_hip_w4_gemm_qkv_rope_workspace(512, 4096, 0, 0, 32, 8, 128) == n * 4096 * 2 + 512 * n * 4
    assert lib.aoto_hip_w4_gemm_qkv_rope_workspace(511, 4096, 0, 0, 32, 8, 128) < n * 4096 * 2
    assert lib.aoto_hip_w4_gemm_qkv_rope_workspace(512, 896, 0, 0, 14, 2, 64) < 1152 * 896 * 2
    assert ops.gemm_workspace_bytes(512, n, 4096) < n * 4096 * 2  # the plain GEMM keeps the fused kernel
    assert ops.library_plan(512, 4096, qkv=True) and not ops.library_plan(512, 4096)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m,k,hq,hkv,dim,bias", [
    (1024, 512, 8, 2, 128, True),
    (1024, 512, 14, 2, 64, False),
    (512, 2048, 8, 2, 128, True),   # the q/k/v rule's 512-row library plan
])
def test_library_qkv_rope_matches_the_oracle(m, k, hq, hkv, dim, bias, bits):
    ops = _ops()
    slot0 = 9
    n = (hq + 2 * hkv) * dim
    rng = np.random.default_rng(540 + dim + bits + m)
    packed, scales, gp, gs = _weights(rng, n, k, bits)
    x = bf16_normal(rng, (m, k))
    b = bf16_normal(rng, (n,), 0.02) if bias else None
    cap = slot0 + m + 5
    cos, sin = oracle.rope_tables(cap, dim, 1e6)
    positions = rng.integers(0, cap, m)
    gpos = torch.from_numpy(positions).cuda()
    pair = torch.full((2, 1, hkv, cap, dim), 7.0, dtype=torch.bfloat16, device="cuda")
    (y, q), names = _traced(lambda: ops.matmul_qkv_rope(
        to_gpu_bf16(x), gp, gs, 64, gpos, to_gpu_bf16(cos), to_gpu_bf16(sin), pair, query_heads=hq, kv_heads=hkv,
        head_dim=dim, slot0=slot0, bias=to_gpu_bf16(b) if bias else None, bits=bits))
    assert "hipblaslt_matmul_bf16" in names and names[-1] == "aoto_rope_qkv_rows", names
    got_y = from_gpu_bf16(y)
    assert_bf16_parity(got_y, oracle.w4_matmul(x, packed, scales, 64, bias=b, bits=bits), max_ulp=1.0)
    heads = got_y.reshape(m, hq + 2 * hkv, dim).transpose(1, 0, 2)[None]
    c, s_ = cos[positions][None, None], sin[positions][None, None]
    got_pair = from_gpu_bf16(pair)
    assert_bf16_parity(from_gpu_bf16(q), oracle.rope(heads[:, :hq], c, s_), max_ulp=1.0)
    assert_bf16_parity(got_pair[0, :, :, slot0:slot0 + m], oracle.rope(heads[:, hq:hq + hkv], c, s_), max_ulp=1.0)
    np.testing.assert_array_equal(got_pair[1, :, :, slot0:slot0 + m], heads[0, hq + hkv:][None])
    assert np.all(got_pair[:, :, :, :slot0] == 0.0), "slots below slot0 are zeroed"
    assert np.all(got_pair[:, :, :, slot0 + m:] == 7.0), "slots past the prompt are untouched"


def test_library_gemms_replay_in_a_graph_like_eager():
    """A captured long prefill (bias, gate and paired GEMMs, the in-place residual + norm)
    replays three times, with eager work and synchronizations between, bit-identical to
    its eager pass each time: no library node depends on state the capture froze."""

    ops = _ops()
    m, n, k = 1024, 1024, 1024
    rng = np.random.default_rng(550)
    weights = [_weights(rng, n, k, 4)[2:] for _ in range(4)]
    x = to_gpu_bf16(bf16_normal(rng, (m, k)))
    bias = to_gpu_bf16(bf16_normal(rng, (n,), 0.5))
    residual0 = to_gpu_bf16(bf16_normal(rng, (m, n), 2.0))
    norm_w = to_gpu_bf16(bf16_normal(rng, (n,), 0.5))
    outs = {name: torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
            for name in ("bias", "gate", "paired", "norm")}
    residual = residual0.clone()

    def body():
        ops.w4_matmul(x, *weights[0], 64, bias=bias, out=outs["bias"])
        ops.w4_matmul(x, *weights[1], 64, gate=outs["bias"], out=outs["gate"])
        ops.w4_matmul_gate_up(x, *weights[2], *weights[3], 64, out=outs["paired"])
        ops.matmul_residual_norm(outs["paired"], *weights[0], 64, residual, norm_w, 1e-6, out=residual,
                                 norm_out=outs["norm"])

    body()
    torch.cuda.synchronize()
    eager = {name: t.clone() for name, t in outs.items()}
    eager["residual"] = residual.clone()
    residual.copy_(residual0)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        body()
    torch.cuda.synchronize()
    for replay in range(3):
        for t in outs.values():
            t.fill_(float("nan"))
        residual.copy_(residual0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = dict(outs, residual=residual)
        for name, want in eager.items():
            assert torch.equal(got[name].view(torch.int16), want.view(torch.int16)), f"replay {replay}: {name}"
        # eager work between replays
        torch.mm(x[:64].float(), x[:64].float().t()).sum().item()
