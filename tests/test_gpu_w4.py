"""GPU parity of the W4 pack/unpack and decode GEMV kernels against the oracle.

Pack and unpack must be bit-exact. The GEMV (f32 accumulation in a different
order than the oracle's exact sum) must land within one bf16 ulp of the oracle,
which also meets the north-star bars (max abs <= 2e-2, cosine >= 0.999).
Shapes: the Qwen2.5-0.5B projections (config 2) and edge cases - a row count
that is not a multiple of a block, a single row, the smallest K, other groups.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.ops import w4_gemv as oracle_gemv
from oracle.quant import dequantize_i4_bf16, pack_weight_bf16
from tests.helpers import assert_bf16_parity, bf16_bits_of, bf16_normal, from_gpu_bf16, to_gpu_bf16, to_gpu_bits

pytestmark = pytest.mark.gpu


def _ops():
    from aotolith_amd import ops

    return ops


def _packed_case(rng, n, k, group=64, std=0.02):
    weight = bf16_normal(rng, (n, k), std)
    packed, scales = pack_weight_bf16(weight, group)
    return weight, packed, scales


@pytest.mark.parametrize("n,k,group", [(1152, 896, 64), (896, 4864, 64), (37, 256, 32), (3, 512, 128)])
@pytest.mark.parametrize("source", ["bf16", "f32"])
def test_quantize_is_bit_exact(n, k, group, source):
    rng = np.random.default_rng(n * 7 + k)
    weight = bf16_normal(rng, (n, k), 0.02)
    if source == "f32":
        weight = rng.standard_normal((n, k)).astype(np.float32) * np.float32(0.02)
        weight[0, :group] = 0.0  # an all-zero group
        tensor = torch.from_numpy(weight).cuda()
    else:
        weight[0, :group] = 0.0
        tensor = to_gpu_bf16(weight)
    packed, scales = _ops().w4_quantize(tensor, group)
    ref_packed, ref_scales = pack_weight_bf16(weight, group)
    np.testing.assert_array_equal(packed.cpu().numpy(), ref_packed)
    np.testing.assert_array_equal(bf16_bits_of(scales), ref_scales)


@pytest.mark.parametrize("n,k,group", [(300, 896, 64), (37, 96, 16), (5, 40, 8)])
def test_dequantize_is_bit_exact(n, k, group):
    rng = np.random.default_rng(5 + group)
    _, packed, scales = _packed_case(rng, n, k, group)
    out = _ops().w4_dequantize(torch.from_numpy(packed).cuda(), to_gpu_bits(scales), group)
    np.testing.assert_array_equal(from_gpu_bf16(out), dequantize_i4_bf16(packed, scales, group))


GEMV_SHAPES = [
    (4864, 896),  # gate / up
    (896, 4864),  # down
    (896, 896),  # o
    (1152, 896),  # packed q/k/v
    (1000, 64),  # ragged rows, tiny K
    (1, 32),  # single row, smallest K
]


@pytest.mark.parametrize("n,k", GEMV_SHAPES)
@pytest.mark.parametrize("lanes", [0, 4, 16, 64])
def test_gemv_plain(n, k, lanes):
    rng = np.random.default_rng(n + k + lanes)
    group = 32 if k < 64 else 64
    _, packed, scales = _packed_case(rng, n, k, group)
    x = bf16_normal(rng, (k,))
    y = _ops().w4_gemv(to_gpu_bf16(x), torch.from_numpy(packed).cuda(), to_gpu_bits(scales), group,
                       lanes_per_row=lanes)
    assert_bf16_parity(from_gpu_bf16(y), oracle_gemv(x, packed, scales, group))


@pytest.mark.parametrize("lanes", [0, 8, 32])
def test_gemv_qkv_norm_and_bias(lanes):
    rng = np.random.default_rng(21 + lanes)
    _, packed, scales = _packed_case(rng, 1152, 896)
    x = bf16_normal(rng, (896,), 3.0)
    norm = bf16_normal(rng, (896,), 0.3) + np.float32(1.0)
    norm = norm.astype(np.float32)
    bias = bf16_normal(rng, (1152,), 0.02)
    from oracle.bf16 import round_bf16

    norm = round_bf16(norm)
    y = _ops().w4_gemv(
        to_gpu_bf16(x), torch.from_numpy(packed).cuda(), to_gpu_bits(scales), 64,
        norm_weight=to_gpu_bf16(norm), eps=1e-6, bias=to_gpu_bf16(bias), lanes_per_row=lanes,
    )
    expected = oracle_gemv(x, packed, scales, 64, norm_weight=norm, eps=1e-6, bias=bias)
    assert_bf16_parity(from_gpu_bf16(y), expected)


@pytest.mark.parametrize("n,k", [(896, 896), (896, 4864)])
def test_gemv_residual(n, k):
    rng = np.random.default_rng(n + 3 * k)
    _, packed, scales = _packed_case(rng, n, k)
    x = bf16_normal(rng, (k,))
    residual = bf16_normal(rng, (n,), 2.0)
    y = _ops().w4_gemv(to_gpu_bf16(x), torch.from_numpy(packed).cuda(), to_gpu_bits(scales), 64,
                       bias=to_gpu_bf16(residual))
    assert_bf16_parity(from_gpu_bf16(y), oracle_gemv(x, packed, scales, 64, bias=residual))


@pytest.mark.parametrize("norm", [False, True])
def test_gemv_paired_gate_up(norm):
    rng = np.random.default_rng(99 + norm)
    _, gate, gate_s = _packed_case(rng, 4864, 896)
    _, up, up_s = _packed_case(rng, 4864, 896)
    x = bf16_normal(rng, (896,))
    norm_w = bf16_normal(rng, (896,), 0.1) if norm else None
    from oracle.bf16 import round_bf16

    if norm_w is not None:
        norm_w = round_bf16(norm_w + np.float32(1.0))
    y = _ops().w4_gemv(
        to_gpu_bf16(x), torch.from_numpy(gate).cuda(), to_gpu_bits(gate_s), 64,
        norm_weight=None if norm_w is None else to_gpu_bf16(norm_w),
        up=(torch.from_numpy(up).cuda(), to_gpu_bits(up_s)),
    )
    expected = oracle_gemv(x, gate, gate_s, 64, norm_weight=norm_w, up_packed=up, up_scales_bits=up_s)
    # Two roundings in series (the gate to bf16, then the product): a gate that
    # lands one ulp away moves the output by up to one more ulp.
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=2.0)


def test_gemv_extreme_codes():
    """Every group holds both +7 and -7 (and a -8 word): a wrong sign extension shows."""

    rng = np.random.default_rng(78)
    n, k = 64, 128
    weight = np.zeros((n, k), dtype=np.float32)
    weight[:, 0::2] = 3.0
    weight[:, 1::2] = -3.0
    packed, scales = pack_weight_bf16(weight, 32)
    packed[:, 0] = np.int32(-2023406815)  # codes 1..7, -8 in the first word of every row
    x = bf16_normal(rng, (k,))
    y = _ops().w4_gemv(to_gpu_bf16(x), torch.from_numpy(packed).cuda(), to_gpu_bits(scales), 32)
    assert_bf16_parity(from_gpu_bf16(y), oracle_gemv(x, packed, scales, 32))


def test_gemv_rejects_unsupported_group():
    from aotolith_amd._lib import UnsupportedShape

    rng = np.random.default_rng(1)
    _, packed, scales = _packed_case(rng, 8, 64, 16)
    with pytest.raises(UnsupportedShape):
        _ops().w4_gemv(to_gpu_bf16(bf16_normal(rng, (64,))), torch.from_numpy(packed).cuda(),
                       to_gpu_bits(scales), 16)


STREAM_SHAPES = [
    (151936 // 8, 896),  # LM-head rows (an eighth of the vocabulary), K = 896
    (1000, 896),          # rows not a multiple of the 64-row tile
    (3, 896),             # fewer rows than one tile
    (1152, 896),          # Qwen qkv (direct x loads, 32 lanes per row)
    (4864, 896),          # Qwen gate/up (paired direct form)
    (8193, 896),          # first output count past the direct-form limit
    (896, 4864),          # Qwen down projection
    (1024, 4096),         # Llama-8B K = 4096 (block-staged x)
    (6144, 4096),         # Llama-8B q/k/v rows
    (20000, 4096),        # past the block-staged limit: per-wave staged x
    (512, 14336),         # Llama-8B down projection K (block-staged, 64 lanes x 7 chunks)
    (4096, 14336),        # Llama-8B down projection
]


@pytest.mark.parametrize("n,k", STREAM_SHAPES)
@pytest.mark.parametrize("variant", ["plain", "norm_bias", "paired"])
def test_gemv_stream_shapes(n, k, variant):
    """The persistent streaming kernels (chosen for these K) against the oracle."""

    from oracle.bf16 import round_bf16

    rng = np.random.default_rng(n + k + len(variant))
    _, packed, scales = _packed_case(rng, n, k)
    x = bf16_normal(rng, (k,))
    kwargs, gpu_kwargs = {}, {}
    if variant == "norm_bias":
        norm = round_bf16(np.float32(1.0) + bf16_normal(rng, (k,), 0.2))
        bias = bf16_normal(rng, (n,), 0.5)
        kwargs = {"norm_weight": norm, "eps": 1e-6, "bias": bias}
        gpu_kwargs = {"norm_weight": to_gpu_bf16(norm), "eps": 1e-6, "bias": to_gpu_bf16(bias)}
    elif variant == "paired":
        _, up, up_s = _packed_case(rng, n, k)
        kwargs = {"up_packed": up, "up_scales_bits": up_s}
        gpu_kwargs = {"up": (torch.from_numpy(up).cuda(), to_gpu_bits(up_s))}
    y = _ops().w4_gemv(to_gpu_bf16(x), torch.from_numpy(packed).cuda(), to_gpu_bits(scales), 64, **gpu_kwargs)
    expected = oracle_gemv(x, packed, scales, 64, **kwargs)
    # Long reductions (K = 14336) give |y| up to ~8 (paired), where one bf16 ulp
    # exceeds the 2e-2 bar meant for O(1) outputs: scale the bar with |y|.
    atol = 2e-2 * max(1.0, float(np.abs(expected).max()) / 4)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=2.0 if variant == "paired" else 1.0, atol=atol)


ARGMAX_SHAPES = [
    (151936, 896, 64),   # Qwen LM head (staged 8x4 form)
    (128256, 4096, 64),  # Llama-8B LM head (staged 32x4 form)
    (3000, 4864, 64),    # direct 64x3 form
    (512, 256, 64),      # direct 64x1 form (the small decoder tests' head)
    (100, 896, 32),      # fewer rows than waves; group 32
]


@pytest.mark.parametrize("n,k,group", ARGMAX_SHAPES)
@pytest.mark.parametrize("norm", [True, False])
def test_gemv_argmax_matches_gemv_then_first_index_argmax(n, k, group, norm):
    """Fused LM head + argmax: same logits as w4_gemv, the first maximal index, and the loop bookkeeping."""

    from oracle.ops import argmax_first

    ops = _ops()
    count = ops.argmax_key_count(k, n, group)
    assert count > 0
    gen = torch.Generator(device="cuda").manual_seed(n + k + group)
    x = torch.randn(k, generator=gen, device="cuda").to(torch.bfloat16)
    weight = (torch.randn((n, k), generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    # Row n//3 aligned with x gets the largest logit; its copy at n-1 ties it.
    top = n // 3
    weight[top] = (torch.sign(x.float()) * 0.05).to(torch.bfloat16)
    weight[n - 1] = weight[top]
    packed, scales = ops.w4_quantize(weight, group)
    normw = (1.0 + 0.1 * torch.randn(k, generator=gen, device="cuda")).to(torch.bfloat16) if norm else None
    keys = torch.full((count,), -7, dtype=torch.int64, device="cuda")
    y = ops.w4_gemv_argmax(x, packed, scales, group, keys, norm_weight=normw, eps=1e-6)
    ref = ops.w4_gemv(x, packed, scales, group, norm_weight=normw, eps=1e-6)
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))

    logits = y.float().cpu().numpy()[None]
    want = int(argmax_first(logits)[0])
    assert want == top
    cap = 8
    token = torch.zeros((1,), dtype=torch.int64, device="cuda")
    history = torch.zeros((4,), dtype=torch.int64, device="cuda")
    history_len = torch.ones((1,), dtype=torch.int32, device="cuda")
    step = torch.tensor([5, 6, cap - 1, cap - 1], dtype=torch.int32, device="cuda")
    embed = torch.randn((n, 64), generator=gen, device="cuda").to(torch.bfloat16)
    hidden = torch.empty(64, dtype=torch.bfloat16, device="cuda")
    error = torch.zeros((1,), dtype=torch.int32, device="cuda")
    cos_t = torch.randn((cap, 64), generator=gen, device="cuda").to(torch.bfloat16)
    sin_t = torch.randn((cap, 64), generator=gen, device="cuda").to(torch.bfloat16)
    rope_rows = torch.zeros((2, 64), dtype=torch.bfloat16, device="cuda")
    ops.argmax_finish(keys, count, out=token, history=history, history_len=history_len, step_state=step,
                      capacity=cap, embedding=embed, hidden_out=hidden, error=error, rope_tables=(cos_t, sin_t),
                      rope_rows=rope_rows)
    assert int(token.item()) == want
    assert history.cpu().tolist()[1] == want and int(history_len.item()) == 2
    assert step.cpu().tolist() == [6, 7, 0, 0]
    assert torch.equal(rope_rows[0].view(torch.int16), cos_t[6].view(torch.int16))
    assert torch.equal(rope_rows[1].view(torch.int16), sin_t[6].view(torch.int16))
    assert torch.equal(hidden.view(torch.int16), embed[want].view(torch.int16))
    assert int(error.item()) == 0

    # A token outside the embedding table: zero row and the error flag, no fault.
    short = embed[:top].contiguous()
    ops.argmax_finish(keys, count, out=token, embedding=short, hidden_out=hidden, error=error)
    assert int(token.item()) == want
    assert int(error.item()) == 1 and not bool(hidden.float().abs().sum().item())


def test_gemv_argmax_refuses_unsupported_shapes():
    from aotolith_amd._lib import HipKernelError, UnsupportedShape

    ops = _ops()
    assert ops.argmax_key_count(96, 64, 32) == 0      # three groups per row: scale pairs do not fit
    assert ops.argmax_key_count(8192, 64, 64) == 0    # K beyond the direct forms
    keys = torch.empty((4,), dtype=torch.int64, device="cuda")
    x = torch.zeros(896, dtype=torch.bfloat16, device="cuda")
    packed = torch.zeros((1000, 112), dtype=torch.int32, device="cuda")
    scales = torch.zeros((1000, 14), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(HipKernelError):   # too few keys for the launch
        ops.w4_gemv_argmax(x, packed, scales, 64, keys)
    with pytest.raises(UnsupportedShape):
        ops.w4_gemv_argmax(torch.zeros(96, dtype=torch.bfloat16, device="cuda"),
                           torch.zeros((64, 12), dtype=torch.int32, device="cuda"),
                           torch.zeros((64, 3), dtype=torch.bfloat16, device="cuda"), 32, keys)


# (LM-head rows, K, q/k/v rows, bias): the Qwen2.5-0.5B and Llama-3-8B q/k/v shapes,
# each after an LM head whose launch writes 2048 argmax keys
FINISH_SHAPES = [(20000, 896, 1152, True), (8192, 4096, 6144, False)]


@pytest.mark.parametrize("lm_n,k,n,bias", FINISH_SHAPES)
def test_gemv_finish_matches_finish_then_gemv(lm_n, k, n, bias):
    """The finish folded into the next q/k/v GEMV: the same token, history, step state, RoPE
    rows and residual row as argmax_finish, and bit-identical GEMV output to w4_gemv on that
    row; a token outside the embedding table stages zeros and sets the error flag."""

    ops = _ops()
    group = 64
    count = ops.argmax_key_count(k, lm_n, group)
    assert 0 < count <= 2048 and ops.gemv_finish_supported(k, n, group, count)
    gen = torch.Generator(device="cuda").manual_seed(lm_n + k + n)
    x = torch.randn(k, generator=gen, device="cuda").to(torch.bfloat16)
    head = (torch.randn((lm_n, k), generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    top = lm_n // 5
    head[top] = (torch.sign(x.float()) * 0.05).to(torch.bfloat16)
    hp, hs = ops.w4_quantize(head, group)
    keys = torch.full((count,), -7, dtype=torch.int64, device="cuda")
    ops.w4_gemv_argmax(x, hp, hs, group, keys, eps=1e-6)
    embed = torch.randn((lm_n, k), generator=gen, device="cuda").to(torch.bfloat16)
    qkv = (torch.randn((n, k), generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    qp, qs = ops.w4_quantize(qkv, group)
    normw = (1.0 + 0.1 * torch.randn(k, generator=gen, device="cuda")).to(torch.bfloat16)
    qbias = (torch.randn(n, generator=gen, device="cuda") * 0.02).to(torch.bfloat16) if bias else None
    cap, hd = 16, 64
    cos_t = torch.randn((cap, hd), generator=gen, device="cuda").to(torch.bfloat16)
    sin_t = torch.randn((cap, hd), generator=gen, device="cuda").to(torch.bfloat16)

    def state():
        return dict(token=torch.zeros((1,), dtype=torch.int64, device="cuda"),
                    history=torch.zeros((8,), dtype=torch.int64, device="cuda"),
                    history_len=torch.full((1,), 3, dtype=torch.int32, device="cuda"),
                    step=torch.tensor([9, 10, cap - 1, 4], dtype=torch.int32, device="cuda"),
                    rope=torch.zeros((2, hd), dtype=torch.bfloat16, device="cuda"),
                    hidden=torch.full((k,), float("nan"), dtype=torch.bfloat16, device="cuda"),
                    error=torch.zeros((1,), dtype=torch.int32, device="cuda"))

    for table in (embed, embed[:top].contiguous()):
        a, b = state(), state()
        ops.argmax_finish(keys, count, out=a["token"], history=a["history"], history_len=a["history_len"],
                          step_state=a["step"], capacity=cap, embedding=table, hidden_out=a["hidden"],
                          error=a["error"], rope_tables=(cos_t, sin_t), rope_rows=a["rope"])
        want = ops.w4_gemv(a["hidden"], qp, qs, group, norm_weight=normw, eps=1e-6, bias=qbias)
        got = torch.full((n,), float("nan"), dtype=torch.bfloat16, device="cuda")
        ops.w4_gemv_finish(keys, count, table, qp, qs, group, norm_weight=normw, eps=1e-6, bias=qbias, out=got,
                           token_out=b["token"], hidden_out=b["hidden"], history=b["history"],
                           history_len=b["history_len"], step_state=b["step"], capacity=cap, error=b["error"],
                           rope_tables=(cos_t, sin_t), rope_rows=b["rope"])
        torch.cuda.synchronize()
        assert int(a["token"].item()) == top
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        for name in ("token", "history", "history_len", "step", "error"):
            assert torch.equal(a[name], b[name]), name
        for name in ("rope", "hidden"):
            assert torch.equal(a[name].view(torch.int16), b[name].view(torch.int16)), name
        assert b["step"].cpu().tolist() == [10, 11, 0, 5]
        assert int(b["error"].item()) == (0 if table is embed else 1)


def test_gemv_finish_refuses_other_shapes():
    from aotolith_amd._lib import UnsupportedShape

    ops = _ops()
    assert not ops.gemv_finish_supported(1024, 1024, 64, 2048)   # not a block-staged q/k/v shape
    assert not ops.gemv_finish_supported(896, 1152, 64, 4096)    # more keys than the prologue reads
    keys = torch.zeros((2048,), dtype=torch.int64, device="cuda")
    embed = torch.zeros((16, 896), dtype=torch.bfloat16, device="cuda")
    packed = torch.zeros((20000, 112), dtype=torch.int32, device="cuda")  # a long output: the LM-head form
    scales = torch.zeros((20000, 14), dtype=torch.bfloat16, device="cuda")
    normw = torch.ones(896, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(UnsupportedShape):
        ops.w4_gemv_finish(keys, 2048, embed, packed, scales, 64, norm_weight=normw, eps=1e-6,
                           out=torch.empty(20000, dtype=torch.bfloat16, device="cuda"),
                           token_out=torch.zeros((1,), dtype=torch.int64, device="cuda"),
                           hidden_out=torch.empty(896, dtype=torch.bfloat16, device="cuda"))
