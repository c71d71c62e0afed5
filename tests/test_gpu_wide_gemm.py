"""GPU parity of the long-prefill GEMM path: the wide-tile kernel (csrc/w4_gemm_wide.h).

From ``ops.WIDE_ROWS`` rows on (K % 256 == 0) the prefill GEMMs' automatic plan
(tile = splits = 0) runs the 32x32x16-MFMA kernel with the dequant fused in registers,
X and the packed words staged in LDS by direct global->LDS loads. Every form is compared
with the CPU oracle within one bf16 ulp (two for the silu_mul products, as for the
16x16 kernel), with the 16x16 kernel under an explicit plan, and - captured in a HIP
graph - replay by replay with its eager result; two fresh processes give the same
bits (every plan is a fixed function of the shape).
"""

from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from oracle import ops as oracle
from oracle.bf16 import round_bf16
from oracle.quant import pack_weight_bits_bf16
from tests.helpers import assert_bf16_parity, bf16_normal, from_gpu_bf16, to_gpu_bf16, to_gpu_bits

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


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


def _wide(names, bits=4):
    return [name for name in names if name.startswith(f"aoto_w{bits}_gemm_w")]


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m", [512, 1100])
@pytest.mark.parametrize("epilogue", ["none", "bias", "residual", "gate"])
def test_wide_gemm_matches_the_oracle_and_the_16x16_kernel(epilogue, m, bits):
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
    assert len(_wide(names, bits)) == 1, names
    small, small_names = _traced(lambda: matmul(gx, gp, gs, 64, tile=28, splits=1, **gkw))
    assert not _wide(small_names, bits)
    ulp = 2.0 if epilogue == "gate" else 1.0
    expected = oracle.w4_matmul(x, packed, scales, 64, bits=bits, **kwargs)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=ulp, atol=_atol(expected))
    assert_bf16_parity(from_gpu_bf16(y), from_gpu_bf16(small), max_ulp=ulp, atol=_atol(expected))


@pytest.mark.parametrize("bits,tile", [(4, 241), (4, 242), (4, 243), (4, 281), (4, 441), (8, 241), (8, 242),
                                       (8, 441)])
@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("splits", [1, 3])
def test_wide_tiles_explicit(tile, bits, group, splits):
    """Every wide instance under an explicit code: ragged M and N tails, an odd number of
    128-k steps (K = 640: the unrolled loop's extra step adds exactly zero; groups of 128
    need an even count per row, so K = 768 there), groups of 32 / 64 / 128, unsplit and
    split along k."""

    ops = _ops()
    m, n, k = 300, 768, 640 if group < 128 else 768
    rng = np.random.default_rng(600 + tile + group + splits + bits)
    packed, scales, gp, gs = _weights(rng, n, k, bits, group)
    x = bf16_normal(rng, (m, k))
    residual = bf16_normal(rng, (m, n), 2.0)
    matmul = ops.w4_matmul if bits == 4 else ops.w8_matmul
    y, names = _traced(lambda: matmul(to_gpu_bf16(x), gp, gs, group, residual=to_gpu_bf16(residual), tile=tile,
                                      splits=splits))
    assert _wide(names, bits), names
    expected = oracle.w4_matmul(x, packed, scales, group, residual=residual, bits=bits)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=1.0, atol=_atol(expected))


def test_wide_tiles_refuse_what_they_cannot_run():
    from aotolith_amd._lib import HipKernelError, UnsupportedShape

    ops = _ops()
    rng = np.random.default_rng(610)
    packed, scales, gp, gs = _weights(rng, 256, 576, 4)  # K = 576: not a whole number of 128-k steps
    with pytest.raises(UnsupportedShape):
        ops.w4_matmul(to_gpu_bf16(bf16_normal(rng, (64, 576))), gp, gs, 64, tile=242)
    packed, scales, gp, gs = _weights(rng, 256, 512, 8)
    with pytest.raises(HipKernelError, match="no wide tile 243"):
        ops.w8_matmul(to_gpu_bf16(bf16_normal(rng, (64, 512))), gp, gs, 64, tile=243)


def test_wide_gemm_in_place_residual():
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
@pytest.mark.parametrize("m", [512, 1024])
def test_wide_gate_up_matches_the_oracle(bits, m):
    """The paired form: bf16(up * silu(bf16(gate))) in one pass - within the bars of the
    oracle's two-step result (gate GEMM rounded, then the up GEMM's gate epilogue)."""

    ops = _ops()
    n, k = 1152, 1024
    rng = np.random.default_rng(520 + bits + m)
    gpk, gsc, g_packed, g_scales = _weights(rng, n, k, bits)
    upk, usc, u_packed, u_scales = _weights(rng, n, k, bits)
    x = bf16_normal(rng, (m, k))
    gate_up = ops.w4_matmul_gate_up if bits == 4 else ops.w8_matmul_gate_up
    gx = to_gpu_bf16(x)
    y, names = _traced(lambda: gate_up(gx, g_packed, g_scales, u_packed, u_scales, 64))
    assert names[0] == f"aoto_w{bits}_gemm_w4x1x4_paired", names
    want_gate = round_bf16(oracle.w4_matmul(x, gpk, gsc, 64, bits=bits))
    expected = oracle.w4_matmul(x, upk, usc, 64, gate=want_gate, bits=bits)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=2.0)
    small = gate_up(gx, g_packed, g_scales, u_packed, u_scales, 64, tile=18, splits=1)
    assert_bf16_parity(from_gpu_bf16(y), from_gpu_bf16(small), max_ulp=2.0)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("n", [896, 4096])
def test_wide_residual_norm_matches_the_oracle(n, bits):
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
    assert _wide(names, bits) and names[-1] in ("aoto_rms_norm", "aoto_w4_gemm_reduce_norm"), names
    expected = oracle.w4_matmul(x, packed, scales, 64, residual=residual, bits=bits)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=1.0, atol=_atol(expected))
    assert_bf16_parity(from_gpu_bf16(norm), oracle.rms_norm(from_gpu_bf16(y), weight, 1e-6), max_ulp=1.0)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m,k,hq,hkv,dim,bias", [
    (1024, 512, 8, 2, 128, True),    # unsplit: the GEMM, then aoto_rope_qkv_rows
    (512, 2048, 8, 2, 128, True),    # split: aoto_w4_gemm_reduce_rope
    (1024, 512, 14, 2, 64, False),
])
def test_wide_qkv_rope_matches_the_oracle(m, k, hq, hkv, dim, bias, bits):
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
    assert _wide(names, bits) and names[-1] in ("aoto_rope_qkv_rows", "aoto_w4_gemm_reduce_rope"), names
    # y (stored by both plans) is the rounded projection RoPE and the copy start from: a
    # one-ulp difference of y from the oracle's would grow under RoPE's cancellation, so
    # those are checked on y exactly as the kernels saw it
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


def test_wide_gemms_replay_in_a_graph_like_eager():
    """A captured long prefill (bias, gate and paired GEMMs, the in-place residual + norm)
    replays three times, with eager work and synchronizations between, bit-identical to
    its eager pass each time."""

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

    _, names = _traced(body)
    assert len(_wide(names)) == 4, names
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


_CHILD = r"""
import hashlib, sys
import torch
sys.path.insert(0, sys.argv[1])
from aotolith_amd import ops
torch.cuda.set_device(0)
g = torch.Generator(device="cuda"); g.manual_seed(7)
w, s = ops.w4_quantize((torch.randn(4096, 4096, generator=g, device="cuda") * 0.02).to(torch.bfloat16), 64)
x = torch.randn(2048, 4096, generator=g, device="cuda").to(torch.bfloat16)
r = torch.randn(2048, 4096, generator=g, device="cuda").to(torch.bfloat16)
y = ops.w4_matmul(x, w, s, 64, residual=r)
u, us = ops.w4_quantize((torch.randn(4096, 4096, generator=g, device="cuda") * 0.02).to(torch.bfloat16), 64)
p = ops.w4_matmul_gate_up(x, w, s, u, us, 64)
torch.cuda.synchronize()
print(hashlib.sha256(y.view(torch.int16).cpu().numpy().tobytes() + p.view(torch.int16).cpu().numpy().tobytes()).hexdigest())
"""


def test_long_prefill_bits_are_the_same_in_fresh_processes():
    """Two fresh processes run the same 2048-row GEMM and gate/up pair with the automatic
    plan and produce the same output bits (no per-process tuning choice)."""

    digests = []
    for _ in range(2):
        done = subprocess.run([sys.executable, "-c", _CHILD, ROOT], capture_output=True, text=True, timeout=300)
        assert done.returncode == 0, done.stderr[-2000:]
        digests.append(done.stdout.strip().splitlines()[-1])
    assert digests[0] == digests[1], digests
