"""Pin the oracle's fused ops: closed forms, brute force, and independent torch fp32 evaluations.

Each check is chosen so a plausible mistake in ``oracle/ops.py`` fails it: a
flipped rotate-half sign, a GQA head map of ``h % Hkv`` instead of ``h // G``, a
norm over the wrong axis, a dropped epsilon, a transposed weight, a gate rounded
at the wrong point. None of them re-types the oracle's own formula.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ops
from oracle.bf16 import round_bf16
from oracle.quant import dequantize_i4_bf16, dequantize_i4_exact, pack_weight_bf16
from tests.helpers import bf16_normal


# ------------------------------------------------------------------ RoPE
def test_rope_tables_match_the_reference_torch_recipe():
    """The runtime builds the tables with the reference's torch ops; the oracle with NumPy."""

    from aotolith_amd.decoder import rope_tables as runtime_tables

    for capacity, dim, theta in ((192, 64, 1e6), (2304, 128, 5e5), (40, 16, 1e4)):
        cos, sin = runtime_tables(capacity, dim, theta, "cpu")
        ocos, osin = ops.rope_tables(capacity, dim, theta)
        np.testing.assert_array_equal(cos.float().numpy(), ocos)
        np.testing.assert_array_equal(sin.float().numpy(), osin)


def test_rope_tables_round_the_angle_before_cos():
    """The tables take cos/sin of the bf16-rounded angle (models/decoder.py:323-334), not the f32 one."""

    theta, dim = 1e6, 64
    cos, sin = ops.rope_tables(192, dim, theta)
    inverse = np.power(np.float32(theta), np.arange(0, dim, 2, dtype=np.float32) / np.float32(dim))
    differing = 0
    for pos in (129, 150, 191):
        for i in range(dim // 2):
            angle = float(np.float32(pos) / inverse[i])
            rounded = float(round_bf16(np.array([angle], dtype=np.float32))[0])
            want = round_bf16(np.array([math.cos(rounded), math.sin(rounded)]))
            assert cos[pos, i] == want[0] and sin[pos, i] == want[1]
            naive = round_bf16(np.array([math.cos(angle), math.sin(angle)]))
            differing += int(naive[0] != want[0] or naive[1] != want[1])
    assert differing > 0, "the bf16 angle rounding must be visible at these positions"


def test_rope_at_position_zero_is_the_identity():
    rng = np.random.default_rng(0)
    cos, sin = ops.rope_tables(8, 64, 1e6)
    x = bf16_normal(rng, (1, 3, 1, 64))
    np.testing.assert_array_equal(ops.rope(x, cos[0], sin[0]), x)


def test_rope_is_the_pairwise_rotation():
    """Brute force: pair (d, d + D/2) rotates by the table angle, first half takes -partner."""

    rng = np.random.default_rng(1)
    dim = 16
    cos, sin = ops.rope_tables(32, dim, 1e4)
    x = bf16_normal(rng, (dim,))
    pos = 27
    got = ops.rope(x, cos[pos], sin[pos])
    half = dim // 2
    want = np.empty(dim)
    for d in range(half):
        c, s = float(cos[pos, d]), float(sin[pos, d])
        a, b = float(x[d]), float(x[d + half])
        want[d] = a * c - b * s
        want[d + half] = b * c + a * s
    np.testing.assert_array_equal(got, round_bf16(want))
    # and the rotation keeps each pair's norm (to the tables' bf16 precision)
    for d in range(half):
        before = x[d] ** 2 + x[d + half] ** 2
        after = got[d] ** 2 + got[d + half] ** 2
        assert abs(after - before) <= 0.03 * before + 1e-6


# ------------------------------------------------------------------ RMSNorm
def test_rms_norm_of_a_constant_row():
    w = round_bf16(np.linspace(0.5, 1.5, 64).astype(np.float32))
    x = np.full((1, 64), 3.0, dtype=np.float32)
    eps = 1e-6
    want = round_bf16((np.float32(3.0) / np.sqrt(np.float32(9.0) + np.float32(eps))) * w)
    np.testing.assert_array_equal(ops.rms_norm(x, w, eps)[0], want)


def test_rms_norm_matches_torch_fp32():
    rng = np.random.default_rng(2)
    x = bf16_normal(rng, (5, 896), 2.0)
    w = round_bf16(np.float32(1.0) + bf16_normal(rng, (896,), 0.2))
    ref = F.rms_norm(torch.from_numpy(x), (896,), torch.from_numpy(w), eps=1e-6).numpy()
    got = ops.rms_norm(x, w, 1e-6)
    # torch rounds nothing; the oracle rounds once to bf16 -> within one bf16 ulp
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-30)


# ------------------------------------------------------------------ attention
def _sdpa_fp32(q, k, v, mask, group):
    kk = torch.from_numpy(np.repeat(k, group, axis=1).astype(np.float32))
    vv = torch.from_numpy(np.repeat(v, group, axis=1).astype(np.float32))
    qq = torch.from_numpy(q.astype(np.float32))
    m = None if mask is None else torch.from_numpy(np.asarray(mask, dtype=bool))
    return F.scaled_dot_product_attention(qq, kk, vv, attn_mask=m).numpy()


def test_attention_matches_torch_sdpa_with_gqa():
    rng = np.random.default_rng(3)
    q = bf16_normal(rng, (1, 14, 9, 64))
    k = bf16_normal(rng, (1, 2, 9, 64))
    v = bf16_normal(rng, (1, 2, 9, 64))
    mask = ops.prefill_mask(9, 9)
    got = ops.attention(q, k, v, mask)
    ref = _sdpa_fp32(q, k, v, mask, 7)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6)


def test_attention_gqa_uses_h_floor_div_group():
    """kv head j holds the constant value j: query head h must read h // G, not h % Hkv."""

    rng = np.random.default_rng(4)
    q = bf16_normal(rng, (1, 6, 1, 8))
    k = bf16_normal(rng, (1, 2, 5, 8))
    v = np.zeros((1, 2, 5, 8), dtype=np.float32)
    v[0, 1] = 1.0
    out = ops.attention(q, k, v)
    np.testing.assert_array_equal(out[0, :3], 0.0)
    np.testing.assert_array_equal(out[0, 3:], 1.0)


def test_attention_closed_forms():
    rng = np.random.default_rng(5)
    q = bf16_normal(rng, (1, 2, 1, 16))
    k = bf16_normal(rng, (1, 1, 1, 16))
    v = bf16_normal(rng, (1, 1, 1, 16))
    # one key: the output is that key's value
    np.testing.assert_array_equal(ops.attention(q, k, v)[0, 0, 0], v[0, 0, 0])
    # all-ones values: softmax rows sum to one
    k5 = bf16_normal(rng, (1, 1, 5, 16))
    ones = np.ones((1, 1, 5, 16), dtype=np.float32)
    np.testing.assert_array_equal(ops.attention(q, k5, ones), 1.0)
    # a fully masked row gives zero (safe_softmax)
    masked = np.zeros((1, 1, 1, 5), dtype=bool)
    np.testing.assert_array_equal(ops.attention(q, k5, ones, masked), 0.0)


def test_masks():
    np.testing.assert_array_equal(ops.prefill_mask(6, 6)[0, 0], np.tril(np.ones((6, 6), dtype=bool)))
    m = ops.prefill_mask(4, 6)[0, 0]
    assert not m[:2].any() and m[5, 2:].all() and not m[5, :2].any()
    d = ops.decode_mask(3, 8)[0, 0, 0]
    np.testing.assert_array_equal(d, [False] * 5 + [True] * 3)


def test_argmax_first_index_on_ties():
    assert int(ops.argmax_first(np.array([1.0, 3.0, 2.0, 3.0]))) == 1


# ------------------------------------------------------------------ W4 GEMV / GEMM
def _packed(rng, n, k, group=32):
    w = bf16_normal(rng, (n, k), 0.05)
    return pack_weight_bf16(w, group)


def test_w4_gemv_matches_torch_on_the_unrounded_dequant():
    rng = np.random.default_rng(6)
    packed, scales = _packed(rng, 24, 64)
    x = bf16_normal(rng, (64,))
    w = torch.from_numpy(dequantize_i4_exact(packed, scales, 32).astype(np.float64))
    ref = (w @ torch.from_numpy(x.astype(np.float64))).numpy()
    np.testing.assert_array_equal(ops.w4_gemv(x, packed, scales, 32), round_bf16(ref))


def test_w4_gemv_prologue_and_epilogues_against_torch():
    rng = np.random.default_rng(7)
    gate, gs = _packed(rng, 16, 64)
    up, us = _packed(rng, 16, 64)
    x = bf16_normal(rng, (64,), 3.0)
    nw = round_bf16(np.float32(1.0) + bf16_normal(rng, (64,), 0.2))
    bias = bf16_normal(rng, (16,), 0.1)
    xn = F.rms_norm(torch.from_numpy(x), (64,), torch.from_numpy(nw), eps=1e-6).to(torch.bfloat16).double()
    wg = torch.from_numpy(dequantize_i4_exact(gate, gs, 32).astype(np.float64))
    wu = torch.from_numpy(dequantize_i4_exact(up, us, 32).astype(np.float64))
    # norm + bias
    got = ops.w4_gemv(x, gate, gs, 32, norm_weight=nw, eps=1e-6, bias=bias)
    ref = (wg @ xn + torch.from_numpy(bias).double()).numpy()
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-6)
    # paired: silu of the bf16-rounded gate times up
    got = ops.w4_gemv(x, gate, gs, 32, norm_weight=nw, eps=1e-6, up_packed=up, up_scales_bits=us)
    g = (wg @ xn).to(torch.bfloat16).double()
    ref = ((wu @ xn) * F.silu(g)).numpy()
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -6 + 1e-6)


def test_w4_matmul_uses_the_rounded_dequant_and_epilogues():
    rng = np.random.default_rng(8)
    packed, scales = _packed(rng, 32, 64)
    x = bf16_normal(rng, (5, 64))
    w = torch.from_numpy(dequantize_i4_bf16(packed, scales, 32).astype(np.float64))
    xt = torch.from_numpy(x.astype(np.float64))
    np.testing.assert_array_equal(ops.w4_matmul(x, packed, scales, 32), round_bf16((xt @ w.T).numpy()))
    res = bf16_normal(rng, (5, 32))
    np.testing.assert_array_equal(ops.w4_matmul(x, packed, scales, 32, residual=res),
                                  round_bf16((xt @ w.T).numpy() + res))
    gate = bf16_normal(rng, (5, 32))
    ref = (xt @ w.T) * F.silu(torch.from_numpy(gate.astype(np.float64)))
    got = ops.w4_matmul(x, packed, scales, 32, gate=gate)
    assert np.all(np.abs(got - ref.numpy()) <= np.abs(ref.numpy()) * 2.0 ** -7 + 1e-6)


@pytest.mark.parametrize("layout", ["weight_rows_are_outputs"])
def test_w4_gemv_rows_are_output_features(layout):
    """A transposed weight would mix rows: one-hot x picks column k of every row."""

    rng = np.random.default_rng(9)
    packed, scales = _packed(rng, 8, 32)
    x = np.zeros(32, dtype=np.float32)
    x[5] = 1.0
    w = dequantize_i4_exact(packed, scales, 32)
    np.testing.assert_array_equal(ops.w4_gemv(x, packed, scales, 32), round_bf16(w[:, 5]))


# ------------------------------------------------------------------ RoPE + KV append (decode)
def _tiny_decoder(seed=5, capacity=12):
    from oracle.decoder import DecoderShape, OracleDecoder
    from tests.helpers import random_oracle_state

    shape = DecoderShape(vocab=48, hidden=64, intermediate=96, layers=2, heads=4, kv_heads=2, head_dim=16, eps=1e-6,
                         theta=1e6, group_size=32)
    return shape, OracleDecoder(shape, random_oracle_state(shape, seed=seed), capacity)


def test_rope_kv_cache_append_is_the_decoders_cache_update():
    """rope_kv_cache_append rolls layer 0's window exactly as the oracle decoder's decode
    step does (the decoder is pinned against HuggingFace eager in test_oracle_decoder.py),
    from the same projection row, at the step's position."""

    shape, dec = _tiny_decoder()
    ids = np.array([3, 17, 40, 9, 22], dtype=np.int64)
    _, compact = dec.prefill(ids)
    cache = dec.pad_cache(compact)
    token, valid = 11, ids.shape[0] + 1
    _, next_cache = dec.decode(token, valid, cache)
    layer = dec.state["layers"][0]
    row = dec._gemv(dec.state["embed"][token], layer["qkv"], norm=layer["input_norm"], bias=layer.get("qkv_bias"))
    qd, kd = shape.heads * shape.head_dim, shape.kv_heads * shape.head_dim
    q, pair = ops.rope_kv_cache_append(cache, row[None], dec.cos[valid - 1], dec.sin[valid - 1], layer=0,
                                       query_heads=shape.heads, query_start=0, key_start=qd, value_start=qd + kd)
    np.testing.assert_array_equal(pair, next_cache[0])
    assert q.shape == (1, shape.heads, 1, shape.head_dim)


def test_rope_kv_cache_append_closed_forms():
    """The window moves down one slot bit for bit, the value lands unrotated in the last
    slot, and at position 0 (cos 1, sin 0) q and k are the projection row's own values;
    at another position q and k keep each rotated pair's norm (to bf16 rounding)."""

    rng = np.random.default_rng(8)
    layers, batch, hkv, cap, d, hq = 3, 1, 2, 7, 16, 4
    cache = bf16_normal(rng, (layers, 2, batch, hkv, cap, d))
    width = (hq + 2 * hkv) * d
    row = bf16_normal(rng, (batch, width))
    cos, sin = ops.rope_tables(16, d, 1e6)
    kw = dict(layer=1, query_heads=hq, query_start=0, key_start=hq * d, value_start=(hq + hkv) * d)
    q, pair = ops.rope_kv_cache_append(cache, row, cos[0], sin[0], **kw)
    np.testing.assert_array_equal(pair[:, :, :, :-1], cache[1][:, :, :, 1:])
    np.testing.assert_array_equal(pair[1, :, :, -1], row[:, (hq + hkv) * d:].reshape(batch, hkv, d))
    np.testing.assert_array_equal(pair[0, :, :, -1], row[:, hq * d:(hq + hkv) * d].reshape(batch, hkv, d))
    np.testing.assert_array_equal(q.reshape(batch, hq, d), row[:, :hq * d].reshape(batch, hq, d))
    q, pair = ops.rope_kv_cache_append(cache, row, cos[9], sin[9], **kw)
    k_in = row[:, hq * d:(hq + hkv) * d].reshape(batch, hkv, d).astype(np.float64)
    k_out = pair[0, :, :, -1].astype(np.float64)
    half = d // 2
    pair_norm_in = np.hypot(k_in[..., :half], k_in[..., half:])
    pair_norm_out = np.hypot(k_out[..., :half], k_out[..., half:])
    np.testing.assert_allclose(pair_norm_out, pair_norm_in, rtol=2 ** -7, atol=1e-3)
    assert not np.array_equal(k_out, k_in), "position 9 rotates"
    # the other layers' windows are not part of the result
    assert pair.shape == (2, batch, hkv, cap, d)
