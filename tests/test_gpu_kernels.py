"""GPU parity of the prefill GEMM, norms, RoPE, cache append, attention, embedding and argmax.

Every kernel runs through the C ABI (``aotolith_amd.ops`` -> ``libaoto_hip.so``) on
seeded inputs at the configs' shapes and is compared with the CPU oracle. Index
and copy work (cache roll/ring writes, embedding rows, argmax, the value half of
the cache) must be bit-exact; arithmetic lands within the north-star bars
(max abs <= 2e-2, cosine >= 0.999) and within a small number of bf16 ulps.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ops as oracle
from oracle.bf16 import round_bf16
from oracle.quant import pack_weight_bf16
from tests.helpers import assert_bf16_parity, bf16_bits_of, bf16_normal, from_gpu_bf16, to_gpu_bf16, to_gpu_bits

pytestmark = pytest.mark.gpu


def _ops():
    from aotolith_amd import ops

    return ops


def _packed(rng, n, k, group=64, std=0.02):
    weight = bf16_normal(rng, (n, k), std)
    packed, scales = pack_weight_bf16(weight, group)
    return packed, scales


def _gpu_packed(packed, scales):
    return torch.from_numpy(packed).cuda(), to_gpu_bits(scales)


# ---------------------------------------------------------------- prefill GEMM
GEMM_CASES = [
    (128, 4864, 896, 64),   # gate / up at the Qwen prefill length
    (128, 896, 4864, 64),   # down
    (16, 4864, 896, 64),    # config 2, M = 16: 896 -> 4864
    (16, 896, 4864, 64),    # config 2, M = 16: 4864 -> 896
    (1, 896, 896, 64),      # a single row through the GEMM
    (200, 1152, 896, 32),   # ragged M, group 32
    (300, 2048, 512, 128),  # group 128, several m blocks
    (40, 640, 192, 64),     # K = 64 mod 128: the last 128-k step is half
    (130, 1152, 960, 32),   # half last step with group 32, ragged M
]


@pytest.mark.parametrize("m,n,k,group", GEMM_CASES)
@pytest.mark.parametrize("tile", [0, 12, 14, 28])
def test_w4_matmul_plain(m, n, k, group, tile):
    rng = np.random.default_rng(m + n + k + tile)
    packed, scales = _packed(rng, n, k, group)
    x = bf16_normal(rng, (m, k))
    y = _ops().w4_matmul(to_gpu_bf16(x), *_gpu_packed(packed, scales), group, tile=tile)
    assert_bf16_parity(from_gpu_bf16(y), oracle.w4_matmul(x, packed, scales, group), max_ulp=1.0)


@pytest.mark.parametrize("m", [128, 16])  # config 2's M: the bias form is the packed q/k/v 896 -> 1152
@pytest.mark.parametrize("epilogue", ["bias", "residual", "gate"])
def test_w4_matmul_epilogues(epilogue, m):
    rng = np.random.default_rng({"bias": 1, "residual": 2, "gate": 3}[epilogue] + m)
    n, k = 1152 if epilogue == "bias" else 896, 896
    packed, scales = _packed(rng, n, k)
    x = bf16_normal(rng, (m, k))
    kwargs = {}
    if epilogue == "bias":
        kwargs["bias"] = bf16_normal(rng, (n,), 0.02)
    elif epilogue == "residual":
        kwargs["residual"] = bf16_normal(rng, (m, n), 2.0)
    else:
        kwargs["gate"] = bf16_normal(rng, (m, n))
    gpu_kwargs = {key: to_gpu_bf16(value) for key, value in kwargs.items()}
    y = _ops().w4_matmul(to_gpu_bf16(x), *_gpu_packed(packed, scales), 64, **gpu_kwargs)
    expected = oracle.w4_matmul(x, packed, scales, 64, **kwargs)
    # silu_mul rounds once after a product of two inexact terms; allow one more ulp there.
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=2.0 if epilogue == "gate" else 1.0)


def test_w4_matmul_rejects_unsupported_k():
    from aotolith_amd._lib import UnsupportedShape

    rng = np.random.default_rng(4)
    packed, scales = _packed(rng, 64, 96, 32)
    with pytest.raises(UnsupportedShape):
        _ops().w4_matmul(to_gpu_bf16(bf16_normal(rng, (4, 96))), *_gpu_packed(packed, scales), 32)


# ---------------------------------------------------------------- RMSNorm / RoPE
@pytest.mark.parametrize("rows,hidden,eps", [(128, 896, 1e-6), (7, 4096, 1e-5), (1, 64, 1e-6)])
def test_rms_norm(rows, hidden, eps):
    rng = np.random.default_rng(rows * hidden)
    x = bf16_normal(rng, (rows, hidden), 3.0)
    w = round_bf16(np.float32(1.0) + bf16_normal(rng, (hidden,), 0.2))
    y = _ops().rms_norm(to_gpu_bf16(x), to_gpu_bf16(w), eps)
    assert_bf16_parity(from_gpu_bf16(y), oracle.rms_norm(x, w, eps), max_ulp=1.0)


def _tables(capacity, head_dim, theta):
    cos, sin = oracle.rope_tables(capacity, head_dim, theta)
    return cos, sin, to_gpu_bf16(cos), to_gpu_bf16(sin)


@pytest.mark.parametrize("heads,seq,dim,theta", [(14, 128, 64, 1e6), (8, 40, 128, 5e5)])
def test_rope(heads, seq, dim, theta):
    rng = np.random.default_rng(seq)
    cos, sin, gcos, gsin = _tables(192, dim, theta)
    x = bf16_normal(rng, (1, heads, seq, dim))
    positions = np.arange(seq) + 5
    y = _ops().rope(to_gpu_bf16(x), gcos, gsin, torch.from_numpy(positions).cuda())
    expected = oracle.rope(x, cos[positions][None, None], sin[positions][None, None])
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=1.0)


def test_rope_qkv_prefill_fills_queries_and_cache():
    rng = np.random.default_rng(8)
    hq, hkv, dim, m, cap = 14, 2, 64, 128, 192
    cos, sin, gcos, gsin = _tables(cap, dim, 1e6)
    qkv = bf16_normal(rng, (1, m, (hq + 2 * hkv) * dim))
    positions = np.arange(m)
    pair = torch.full((2, 1, hkv, cap, dim), 7.0, dtype=torch.bfloat16, device="cuda")
    q = _ops().rope_qkv_prefill(to_gpu_bf16(qkv), torch.from_numpy(positions).cuda(), gcos, gsin, pair,
                                query_heads=hq, kv_heads=hkv, head_dim=dim, slot0=cap - m)
    qd, kd = hq * dim, hkv * dim
    rows = qkv[0]
    ref_q = oracle.rope(rows[:, :qd].reshape(m, hq, dim).transpose(1, 0, 2)[None], cos[:m][None, None], sin[:m][None, None])
    ref_k = oracle.rope(rows[:, qd:qd + kd].reshape(m, hkv, dim).transpose(1, 0, 2)[None], cos[:m][None, None], sin[:m][None, None])
    ref_v = rows[:, qd + kd:].reshape(m, hkv, dim).transpose(1, 0, 2)[None]
    assert_bf16_parity(from_gpu_bf16(q), ref_q, max_ulp=1.0)
    got = from_gpu_bf16(pair)
    assert np.all(got[:, :, :, : cap - m] == 0.0), "left pad must be zero"
    assert_bf16_parity(got[0, :, :, cap - m:], ref_k[0][None][0], max_ulp=1.0)
    np.testing.assert_array_equal(got[1, :, :, cap - m:], ref_v)


# ---------------------------------------------------------------- decode cache append
@pytest.mark.parametrize("mode", ["roll", "ring"])
def test_rope_kv_cache_append(mode):
    rng = np.random.default_rng(11)
    layers, hq, hkv, dim, cap = 3, 14, 2, 64, 192
    cos, sin, gcos, gsin = _tables(cap, dim, 1e6)
    cache = bf16_normal(rng, (layers, 2, 1, hkv, cap, dim))
    row = bf16_normal(rng, (1, (hq + 2 * hkv) * dim))
    position, layer = 150, 1
    ref_q, ref_pair = oracle.rope_kv_cache_append(
        cache, row, cos[position], sin[position], layer=layer, query_heads=hq,
        query_start=0, key_start=hq * dim, value_start=(hq + hkv) * dim,
    )
    gcache = to_gpu_bf16(cache)
    if mode == "roll":
        out_pair = torch.empty_like(gcache[layer])
        q = _ops().rope_kv_cache_append(to_gpu_bf16(row), gcos, gsin, position, out_pair, pair_in=gcache[layer],
                                        query_heads=hq, query_start=0, key_start=hq * dim,
                                        value_start=(hq + hkv) * dim)
        got = from_gpu_bf16(out_pair)
        np.testing.assert_array_equal(got[:, :, :, : cap - 1], ref_pair[:, :, :, : cap - 1])
        np.testing.assert_array_equal(got[1, :, :, cap - 1], ref_pair[1, :, :, cap - 1])
        assert_bf16_parity(got[0, :, :, cap - 1], ref_pair[0, :, :, cap - 1], max_ulp=1.0)
    else:
        slot = 37
        pair = gcache[layer]
        q = _ops().rope_kv_cache_append(to_gpu_bf16(row), gcos, gsin, position, pair, pair_in=None,
                                        query_heads=hq, query_start=0, key_start=hq * dim,
                                        value_start=(hq + hkv) * dim, ring_slot=slot)
        got = from_gpu_bf16(pair)
        untouched = np.ones(cap, dtype=bool)
        untouched[slot] = False
        np.testing.assert_array_equal(got[:, :, :, untouched], cache[layer][:, :, :, untouched])
        np.testing.assert_array_equal(got[1, :, :, slot], ref_pair[1, :, :, cap - 1])
        assert_bf16_parity(got[0, :, :, slot], ref_pair[0, :, :, cap - 1], max_ulp=1.0)
        # the other layers of the cache are not touched
        np.testing.assert_array_equal(from_gpu_bf16(gcache[0]), cache[0])
    assert_bf16_parity(from_gpu_bf16(q).reshape(ref_q.shape), ref_q, max_ulp=1.0)


# ---------------------------------------------------------------- attention
DECODE_CASES = [
    # (hq, hkv, dim, cap, valid, splits)
    (14, 2, 64, 192, 129, 0),
    (14, 2, 64, 192, 191, 1),
    (14, 2, 64, 192, 150, 3),
    (32, 8, 128, 768, 600, 0),
    (32, 8, 128, 2304, 2300, 0),
    (4, 4, 64, 64, 1, 1),
]


@pytest.mark.parametrize("hq,hkv,dim,cap,valid,splits", DECODE_CASES)
def test_decode_attention_last_valid_slots(hq, hkv, dim, cap, valid, splits):
    rng = np.random.default_rng(cap + valid)
    q = bf16_normal(rng, (1, hq, 1, dim))
    k = bf16_normal(rng, (1, hkv, cap, dim))
    v = bf16_normal(rng, (1, hkv, cap, dim))
    keep = oracle.decode_mask(valid, cap)
    expected = oracle.attention(q, k, v, keep)
    ops = _ops()
    workspace = None
    if splits != 1:
        workspace = ops.decode_attention_workspace(1, hq, hkv, cap, dim, splits, device="cuda")
    for _ in range(2):  # the split counters must return to zero between calls
        out = ops.decode_attention(to_gpu_bf16(q[:, :, 0]), to_gpu_bf16(k), to_gpu_bf16(v), valid=valid,
                                   workspace=workspace, splits=splits)
        assert_bf16_parity(from_gpu_bf16(out), expected.reshape(1, hq, dim), max_ulp=2.0)


def test_decode_attention_ring_and_mask_agree_with_the_roll():
    rng = np.random.default_rng(5)
    hq, hkv, dim, cap, valid, offset = 14, 2, 64, 192, 140, 61
    q = bf16_normal(rng, (1, hq, dim))
    k = bf16_normal(rng, (1, hkv, cap, dim))
    v = bf16_normal(rng, (1, hkv, cap, dim))
    # physical slot p holds logical slot (p - offset) mod cap
    logical = (np.arange(cap) - offset) % cap
    keep_phys = logical >= cap - valid
    expected = oracle.attention(q[:, :, None], k, v, keep_phys[None, None, None, :])
    ops = _ops()
    ring = ops.decode_attention(to_gpu_bf16(q), to_gpu_bf16(k), to_gpu_bf16(v), valid=valid, ring_offset=offset)
    masked = ops.decode_attention(to_gpu_bf16(q), to_gpu_bf16(k), to_gpu_bf16(v),
                                  mask=torch.from_numpy(keep_phys).cuda())
    assert_bf16_parity(from_gpu_bf16(ring), expected.reshape(1, hq, dim), max_ulp=2.0)
    np.testing.assert_array_equal(bf16_bits_of(ring), bf16_bits_of(masked))


def test_decode_attention_fully_masked_gives_zero():
    rng = np.random.default_rng(6)
    q = bf16_normal(rng, (1, 14, 64))
    k = bf16_normal(rng, (1, 2, 192, 64))
    out = _ops().decode_attention(to_gpu_bf16(q), to_gpu_bf16(k), to_gpu_bf16(k), valid=0)
    assert np.all(from_gpu_bf16(out) == 0.0)


PREFILL_CASES = [
    # (hq, hkv, dim, m, length)
    (14, 2, 64, 128, 128),   # config 3 prefill, causal
    (14, 2, 64, 128, 77),    # left-padded bucket
    (32, 8, 128, 200, 200),  # Llama heads, ragged length
    (4, 4, 64, 64, 64),      # MHA
    (4, 2, 64, 16, 16),      # one key tile: the block's second key group has none
    (4, 2, 64, 16, 11),      # ... left-padded
    (32, 8, 128, 40, 40),    # ... at D = 128
    # D = 64 grids of at most a quarter (half) of the CUs take 32-query (64-query) blocks
    # of two 1-wave (2-wave) key groups:
    (14, 2, 64, 256, 256),   # 32-query blocks; the last sees four key tiles: prefetched trips, then the last
    (14, 2, 64, 200, 150),   # 32-query blocks, ragged query tiles with a left pad
    (14, 2, 64, 1024, 1000), # 64-query blocks, up to 16 key tiles, left pad
    (32, 8, 128, 512, 500),  # D = 128 64-query blocks (Llama-8B 512 bucket), left pad
]


@pytest.mark.parametrize("hq,hkv,dim,m,length", PREFILL_CASES)
def test_prefill_attention_causal_left_pad(hq, hkv, dim, m, length):
    rng = np.random.default_rng(m + length + dim)
    q = bf16_normal(rng, (1, hq, m, dim))
    k = bf16_normal(rng, (1, hkv, m, dim))
    v = bf16_normal(rng, (1, hkv, m, dim))
    mask = oracle.prefill_mask(length, m)
    expected = oracle.attention(q, k, v, mask)
    out = _ops().prefill_attention(to_gpu_bf16(q), to_gpu_bf16(k), to_gpu_bf16(v), causal=True, key_start=m - length)
    got = from_gpu_bf16(out).reshape(1, m, hq, dim).transpose(0, 2, 1, 3)
    # P is rounded to bf16 before the P.V product, as the reference's flash kernel
    # does (codegen/attention.py:367-371): the error scales with |v|, not with the
    # output, so the bound is absolute - 2^-6 for N(0,1) values - and not in ulps.
    assert_bf16_parity(got, expected, max_ulp=None, atol=2.0 ** -6)
    if length < m:
        assert np.all(got[:, :, : m - length] == 0.0), "fully masked pad rows must be zero"


def test_prefill_attention_single_tile_ignores_stale_lds():
    """A block with one key tile leaves its second key group without tiles; that
    group's masked trip must compute on a staged tile, not on LDS an earlier launch
    left behind - here NaN values, which P = 0 would turn into a NaN output."""
    rng = np.random.default_rng(12)
    ops = _ops()
    # an earlier launch of the same kernel (8-wave blocks on every CU) with NaN values
    hq, hkv, dim, m = 32, 8, 64, 1024
    q = bf16_normal(rng, (1, hq, m, dim))
    k = bf16_normal(rng, (1, hkv, m, dim))
    v = np.full((1, hkv, m, dim), np.nan, dtype=np.float32)
    ops.prefill_attention(to_gpu_bf16(q), to_gpu_bf16(k), to_gpu_bf16(v), causal=True)
    torch.cuda.synchronize()
    hq, hkv, m = 4, 2, 16
    q = bf16_normal(rng, (1, hq, m, dim))
    k = bf16_normal(rng, (1, hkv, m, dim))
    v = bf16_normal(rng, (1, hkv, m, dim))
    expected = oracle.attention(q, k, v, oracle.prefill_mask(m, m))
    out = ops.prefill_attention(to_gpu_bf16(q), to_gpu_bf16(k), to_gpu_bf16(v), causal=True)
    got = from_gpu_bf16(out).reshape(1, m, hq, dim).transpose(0, 2, 1, 3)
    assert not np.isnan(got).any()
    assert_bf16_parity(got, expected, max_ulp=None, atol=2.0 ** -6)


def test_prefill_attention_explicit_mask_matches_the_implicit_one():
    rng = np.random.default_rng(9)
    hq, hkv, dim, m, length = 14, 2, 64, 128, 90
    q = bf16_normal(rng, (1, hq, m, dim))
    k = bf16_normal(rng, (1, hkv, m, dim))
    mask = oracle.prefill_mask(length, m)
    ops = _ops()
    implicit = ops.prefill_attention(to_gpu_bf16(q), to_gpu_bf16(k), to_gpu_bf16(k), causal=True, key_start=m - length)
    explicit = ops.prefill_attention(to_gpu_bf16(q), to_gpu_bf16(k), to_gpu_bf16(k),
                                     mask=torch.from_numpy(mask.copy()).cuda())
    np.testing.assert_array_equal(bf16_bits_of(implicit), bf16_bits_of(explicit))


# ---------------------------------------------------------------- embedding / argmax
def test_embedding_is_exact_and_flags_bad_ids():
    rng = np.random.default_rng(10)
    table = bf16_normal(rng, (1000, 896))
    ids = np.array([0, 999, 17, 17, 500], dtype=np.int64)
    ops = _ops()
    error = torch.zeros((1,), dtype=torch.int32, device="cuda")
    out = ops.embedding(to_gpu_bf16(table), torch.from_numpy(ids).cuda(), error=error)
    np.testing.assert_array_equal(from_gpu_bf16(out), table[ids])
    assert int(error.item()) == 0
    bad = ops.embedding(to_gpu_bf16(table), torch.tensor([3, 1000], device="cuda"), error=error)
    assert int(error.item()) == 1
    assert np.all(from_gpu_bf16(bad)[1] == 0.0)


def test_argmax_first_index_on_ties():
    rng = np.random.default_rng(12)
    logits = bf16_normal(rng, (3, 151936))
    logits[1, 5] = logits[1, 100] = logits[1, 150000] = 50.0   # tie: the first wins
    logits[2, :] = -1.0
    logits[2, 151935] = -0.5
    got = _ops().argmax(to_gpu_bf16(logits)).cpu().numpy()
    np.testing.assert_array_equal(got, oracle.argmax_first(logits))
    assert got[1] == 5


def test_argmax_records_history():
    ops = _ops()
    history = torch.zeros((4,), dtype=torch.int64, device="cuda")
    length = torch.zeros((1,), dtype=torch.int32, device="cuda")
    for token in (3, 9, 1):
        logits = torch.zeros((1, 64), dtype=torch.bfloat16, device="cuda")
        logits[0, token] = 1.0
        ops.argmax(logits, history=history, history_len=length)
    assert history.cpu().tolist()[:3] == [3, 9, 1]
    assert int(length.item()) == 3


@pytest.mark.parametrize("hq,hkv,dim,cap,valid,offset,slot,splits", [
    (14, 2, 64, 192, 140, 61, 60, 0),      # Qwen shape, one block per kv head
    (14, 2, 64, 192, 191, 0, 191, 3),     # rolled layout, 3 splits + merge
    (32, 8, 128, 2304, 1500, 700, 699, 0),  # Llama-8B window, split-K + merge
    (32, 8, 128, 768, 640, 0, 639, 0),       # Llama-8B 512 bucket window, slot in the last split
    (32, 8, 128, 768, 300, 100, 99, 0),      # ... partly filled, wrapped ring
    (32, 8, 128, 2304, 2304, 5, 4, 72),      # 72 splits: the merge's records past its 40 register columns
])
@pytest.mark.parametrize("rows", [False, True])
def test_decode_rope_attention_matches_append_then_attend(hq, hkv, dim, cap, valid, offset, slot, splits, rows):
    """The fused ring step equals rope_kv_cache_append's rotation + attention over the ring.

    With ``rows`` the cos/sin rows come from a [2, D] buffer and the table
    position passed is wrong on purpose: the buffer must be what is used.
    """

    rng = np.random.default_rng(cap + slot)
    cos, sin, gcos, gsin = _tables(cap, dim, 1e6)
    pair = bf16_normal(rng, (2, 1, hkv, cap, dim))
    row = bf16_normal(rng, (1, (hq + 2 * hkv) * dim))
    position = valid - 1
    cache = pair[None]  # one layer
    ref_q, ref_pair = oracle.rope_kv_cache_append(
        cache, row, cos[position], sin[position], layer=0, query_heads=hq,
        query_start=0, key_start=hq * dim, value_start=(hq + hkv) * dim,
    )
    ring = pair.copy()
    ring[:, :, :, slot] = ref_pair[:, :, :, cap - 1]
    logical = (np.arange(cap) - offset) % cap
    keep = (logical >= cap - valid)[None, None, None, :]
    expected = oracle.attention(ref_q, ring[0], ring[1], keep)
    ops = _ops()
    gpair = to_gpu_bf16(pair)
    workspace = ops.decode_attention_workspace(1, hq, hkv, cap, dim, splits, device="cuda")
    rope_rows = torch.stack([gcos[position], gsin[position]]).contiguous() if rows else None
    out = ops.decode_rope_attention(to_gpu_bf16(row), gcos, gsin, gpair, query_heads=hq, query_start=0,
                                    key_start=hq * dim, value_start=(hq + hkv) * dim,
                                    position=(position + 7) % cap if rows else position, slot=slot, valid=valid,
                                    ring_offset=offset, workspace=workspace, splits=splits, rope_rows=rope_rows)
    assert_bf16_parity(from_gpu_bf16(out), expected.reshape(1, hq, dim), max_ulp=2.0)
    got = from_gpu_bf16(gpair)
    others = np.ones(cap, dtype=bool)
    others[slot] = False
    np.testing.assert_array_equal(got[:, :, :, others], pair[:, :, :, others])
    np.testing.assert_array_equal(got[1, :, :, slot], ref_pair[1, :, :, cap - 1])
    assert_bf16_parity(got[0, :, :, slot], ref_pair[0, :, :, cap - 1], max_ulp=1.0)


@pytest.mark.parametrize("epilogue", ["none", "bias", "residual", "gate"])
@pytest.mark.parametrize("splits", [1, 5])
def test_w4_matmul_split_k_matches_single_pass(epilogue, splits):
    """Split-K (partials + reduce launch) gives the oracle's result for every epilogue."""

    rng = np.random.default_rng(40 + splits)
    m, n, k = 96, 896, 4864
    packed, scales = _packed(rng, n, k)
    x = bf16_normal(rng, (m, k))
    kwargs = {}
    if epilogue == "bias":
        kwargs["bias"] = bf16_normal(rng, (n,), 0.5)
    elif epilogue == "residual":
        kwargs["residual"] = bf16_normal(rng, (m, n), 2.0)
    elif epilogue == "gate":
        kwargs["gate"] = bf16_normal(rng, (m, n))
    gpu_kwargs = {key: to_gpu_bf16(value) for key, value in kwargs.items()}
    ops = _ops()
    assert (ops.gemm_workspace_bytes(m, n, k, 0, splits) > 0) == (splits > 1)
    y = ops.w4_matmul(to_gpu_bf16(x), *_gpu_packed(packed, scales), 64, splits=splits, **gpu_kwargs)
    expected = oracle.w4_matmul(x, packed, scales, 64, **kwargs)
    # K = 4864 with N(0,1) activations puts outputs at |y| ~ 4-16, where one bf16
    # ulp exceeds the 2e-2 bar meant for O(1) outputs: scale the bar with |y|.
    atol = 2e-2 * max(1.0, float(np.abs(expected).max()) / 4)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=2.0 if epilogue == "gate" else 1.0, atol=atol)


def test_w4_matmul_in_place_residual_with_split_k():
    rng = np.random.default_rng(44)
    m, n, k = 128, 896, 896
    packed, scales = _packed(rng, n, k)
    x = bf16_normal(rng, (m, k))
    residual = bf16_normal(rng, (m, n), 2.0)
    buf = to_gpu_bf16(residual)
    _ops().w4_matmul(to_gpu_bf16(x), *_gpu_packed(packed, scales), 64, residual=buf, out=buf, splits=4)
    assert_bf16_parity(from_gpu_bf16(buf), oracle.w4_matmul(x, packed, scales, 64, residual=residual), max_ulp=1.0)


GATE_UP_CASES = [
    (128, 4864, 896, 64, 0),    # Qwen prefill MLP (auto plan: split-K)
    (16, 4864, 896, 64, 0),     # config 2, M = 16
    (200, 1152, 896, 32, 0),    # ragged M, group 32
    (512, 2048, 512, 128, 0),   # several m blocks, no split
    (96, 896, 4864, 64, 5),     # forced 5-way split
    (64, 512, 256, 64, 1),      # forced single pass
    (72, 512, 320, 64, 0),      # half last 128-k step
    (64, 640, 960, 64, 3),      # half last step inside a 3-way split
]


@pytest.mark.parametrize("m,n,k,group,splits", GATE_UP_CASES)
@pytest.mark.parametrize("bits", [4, 8])
def test_gemm_gate_up_matches_gate_then_up(m, n, k, group, splits, bits):
    """The paired prefill MLP GEMM: bit-identical to the gate GEMM followed by the up
    GEMM with the silu_mul epilogue under the same plan, and within the bars of the
    oracle's two-step result. Where the automatic paired plan is the dequant-once kernel
    (4-bit, 32-256 rows; a summation order of its own) the identity is checked on the
    16x16 kernel's explicit tile 14 and the automatic result against the oracle."""

    from oracle.quant import pack_weight_bits_bf16

    rng = np.random.default_rng(m * 3 + n + k + bits + splits)
    gate_w = bf16_normal(rng, (n, k), 0.02)
    up_w = bf16_normal(rng, (n, k), 0.02)
    gp, gs = pack_weight_bits_bf16(gate_w, group, bits)
    upk, us = pack_weight_bits_bf16(up_w, group, bits)
    x = bf16_normal(rng, (m, k))
    ops = _ops()
    matmul = ops.w4_matmul if bits == 4 else ops.w8_matmul
    gate_up = ops.w4_matmul_gate_up if bits == 4 else ops.w8_matmul_gate_up
    xg = to_gpu_bf16(x)
    g_gpu, u_gpu = _gpu_packed(gp, gs), _gpu_packed(upk, us)
    lds = bits == 4 and splits == 0 and ops.lds_plan(m, n, k, group_size=group, paired=True) is not None
    plan = {"tile": 14} if lds else {}
    y = gate_up(xg, *g_gpu, *u_gpu, group, splits=splits, **plan)
    gate = matmul(xg, *g_gpu, group, splits=splits, **plan)
    two_step = matmul(xg, *u_gpu, group, gate=gate, splits=splits, **plan)
    assert torch.equal(y.view(torch.int16), two_step.view(torch.int16))
    if lds:
        y = gate_up(xg, *g_gpu, *u_gpu, group)
    want_gate = round_bf16(oracle.w4_matmul(x, gp, gs, group, bits=bits))
    expected = oracle.w4_matmul(x, upk, us, group, gate=want_gate, bits=bits)
    atol = 2e-2 * max(1.0, float(np.abs(expected).max()) / 4)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=2.0, atol=atol)


def test_gemm_gate_up_rejects_mismatched_weights():
    ops = _ops()
    x = torch.zeros((4, 256), dtype=torch.bfloat16, device="cuda")
    gp = torch.zeros((64, 32), dtype=torch.int32, device="cuda")
    gs = torch.zeros((64, 4), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        ops.w4_matmul_gate_up(x, gp, gs, torch.zeros((32, 32), dtype=torch.int32, device="cuda"), gs, 64)


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m,n,k,splits", [
    (128, 896, 896, 0),     # Qwen o projection at the prefill length (auto plan: split-K)
    (128, 896, 4864, 0),    # Qwen down projection (split)
    (96, 896, 896, 1),      # forced single pass: GEMM then the row norm
    (40, 4096, 512, 3),     # 4096-wide rows, forced split
])
def test_matmul_residual_norm_equals_matmul_then_norm(m, n, k, splits, bits):
    """The fused o/down projection + RMSNorm gives the two-launch path's y bit for bit, in
    place over the residual, and its norm within one bf16 rounding of the two-launch norm
    and of the oracle's (the fused sum of squares is a block sum). The y half is also
    checked against the oracle's matmul, for either code width."""

    from oracle.quant import pack_weight_bits_bf16

    rng = np.random.default_rng(70 + m + k + bits)
    packed, scales = pack_weight_bits_bf16(bf16_normal(rng, (n, k), 0.02), 64, bits)
    x = bf16_normal(rng, (m, k))
    residual = bf16_normal(rng, (m, n), 2.0)
    weight = bf16_normal(rng, (n,), 0.5)
    ops = _ops()
    matmul = ops.w4_matmul if bits == 4 else ops.w8_matmul
    gp, gs = _gpu_packed(packed, scales)
    gx, gw = to_gpu_bf16(x), to_gpu_bf16(weight)
    y_ref = matmul(gx, gp, gs, 64, residual=to_gpu_bf16(residual), splits=splits)
    norm_ref = ops.rms_norm(y_ref, gw, 1e-6)
    y = to_gpu_bf16(residual)  # in place: out aliases the residual
    y_out, norm = ops.matmul_residual_norm(gx, gp, gs, 64, y, gw, 1e-6, bits=bits, out=y, splits=splits)
    assert y_out.data_ptr() == y.data_ptr()
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
    assert_bf16_parity(from_gpu_bf16(y), oracle.w4_matmul(x, packed, scales, 64, residual=residual, bits=bits),
                       max_ulp=1.0)
    assert_bf16_parity(from_gpu_bf16(norm), from_gpu_bf16(norm_ref), max_ulp=1.0)
    expected_norm = oracle.rms_norm(from_gpu_bf16(y_ref), weight, 1e-6)
    assert_bf16_parity(from_gpu_bf16(norm), expected_norm, max_ulp=1.0)


@pytest.mark.gpu
def test_matmul_residual_norm_rejects_wide_rows_and_aliasing():
    rng = np.random.default_rng(77)
    packed, scales = _packed(rng, 4104, 64)
    ops = _ops()
    gp, gs = _gpu_packed(packed, scales)
    x = to_gpu_bf16(bf16_normal(rng, (4, 64)))
    res = to_gpu_bf16(bf16_normal(rng, (4, 4104)))
    with pytest.raises(Exception, match="4096"):
        ops.matmul_residual_norm(x, gp, gs, 64, res, to_gpu_bf16(bf16_normal(rng, (4104,))), 1e-6)
    packed, scales = _packed(rng, 512, 64)
    gp, gs = _gpu_packed(packed, scales)
    res = to_gpu_bf16(bf16_normal(rng, (4, 512)))
    with pytest.raises(Exception, match="alias"):
        ops.matmul_residual_norm(x, gp, gs, 64, res, to_gpu_bf16(bf16_normal(rng, (512,))), 1e-6, norm_out=res)


# ---------------------------------------------------------------- q/k/v projection + RoPE + cache fill
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m,hq,hkv,dim,k,splits,bias,slot0,tile", [
    (128, 14, 2, 64, 896, 0, True, 64, 0),   # Qwen prefill, auto plan
    (128, 14, 2, 64, 896, 7, True, 64, 0),   # split 7 ways: the split-K sum with RoPE and the fill
    (128, 14, 2, 64, 896, 1, True, 0, 0),    # unsplit 64-column blocks: RoPE in the GEMM epilogue
    (128, 14, 2, 64, 896, 1, True, 64, 0),   # the same with a zeroed prefix
    (128, 14, 2, 64, 896, 1, True, 9, 14),   # 64-row blocks (the auto plan takes 32-row ones)
    (72, 14, 2, 64, 896, 1, False, 5, 12),   # 32-row blocks, ragged M
    (40, 8, 2, 128, 512, 3, False, 9, 0),    # head_dim 128, no bias, ragged M, forced split
    (40, 8, 2, 128, 512, 1, False, 9, 24),   # 128-column blocks hold one 128-wide head: epilogue
    (40, 8, 2, 128, 512, 1, True, 9, 14),    # 64-column blocks split a head: GEMM, then the RoPE kernel
    (40, 8, 2, 64, 512, 1, True, 3, 24),     # two 64-wide heads per block
    (200, 8, 2, 128, 512, 1, True, 5, 28),   # 128x128 blocks, ragged M
])
def test_matmul_qkv_rope_equals_matmul_then_rope(m, hq, hkv, dim, k, splits, bias, slot0, tile, bits):
    """The fused q/k/v projection + RoPE + cache fill gives the projection of w4_matmul bit for bit,
    and q / keys / values within one bf16 rounding of rope_qkv_prefill over it (and of the oracle)."""

    from oracle.quant import pack_weight_bits_bf16

    ops = _ops()
    rng = np.random.default_rng(m + dim + splits + bits + tile)
    n = (hq + 2 * hkv) * dim
    packed, scales = pack_weight_bits_bf16(bf16_normal(rng, (n, k), 0.02), 64, bits)
    gp, gs = _gpu_packed(packed, scales)
    x = bf16_normal(rng, (m, k))
    b = bf16_normal(rng, (n,), 0.02) if bias else None
    cap = slot0 + m + 5
    cos, sin = oracle.rope_tables(cap, dim, 1e6)
    positions = rng.integers(0, cap, m)
    gx, gb = to_gpu_bf16(x), (to_gpu_bf16(b) if bias else None)
    gcos, gsin = to_gpu_bf16(cos), to_gpu_bf16(sin)
    gpos = torch.from_numpy(positions).cuda()
    matmul = ops.w4_matmul if bits == 4 else ops.w8_matmul
    # the projection of the same plan: with splits=0 the q/k/v form prefers the unsplit
    # epilogue, whose plan needs no workspace
    from aotolith_amd import _lib
    auto_unsplit = _lib.library().aoto_hip_w4_gemm_qkv_rope_workspace(m, k, tile, 0, hq, hkv, dim) == 0
    y_ref = matmul(gx, gp, gs, 64, bias=gb, tile=tile, splits=splits or (1 if auto_unsplit else 0))
    pair_ref = torch.full((2, 1, hkv, cap, dim), 7.0, dtype=torch.bfloat16, device="cuda")
    q_ref = ops.rope_qkv_prefill(y_ref.view(1, m, n), gpos.view(1, m), gcos, gsin, pair_ref, query_heads=hq,
                                 kv_heads=hkv, head_dim=dim, slot0=slot0, zero_prefix=True)
    pair = torch.full((2, 1, hkv, cap, dim), 7.0, dtype=torch.bfloat16, device="cuda")
    y, q = ops.matmul_qkv_rope(gx, gp, gs, 64, gpos, gcos, gsin, pair, query_heads=hq, kv_heads=hkv, head_dim=dim,
                               slot0=slot0, bias=gb, bits=bits, tile=tile, splits=splits)
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
    assert_bf16_parity(from_gpu_bf16(q), from_gpu_bf16(q_ref), max_ulp=1.0)
    assert_bf16_parity(from_gpu_bf16(pair), from_gpu_bf16(pair_ref), max_ulp=1.0)
    got_pair = from_gpu_bf16(pair)
    assert np.all(got_pair[:, :, :, :slot0] == 0.0), "slots below slot0 are zeroed"
    assert np.all(got_pair[:, :, :, slot0 + m:] == 7.0), "slots past the prompt are untouched"
    # against the oracle: the projection within one rounding of the oracle's, and RoPE of the
    # projection the GPU stored within one rounding of the oracle's RoPE of it
    assert_bf16_parity(from_gpu_bf16(y), oracle.w4_matmul(x, packed, scales, 64, bias=b, bits=bits), max_ulp=1.0)
    heads = from_gpu_bf16(y).reshape(m, hq + 2 * hkv, dim).transpose(1, 0, 2)[None]
    c, s_ = cos[positions][None, None], sin[positions][None, None]
    assert_bf16_parity(from_gpu_bf16(q), oracle.rope(heads[:, :hq], c, s_), max_ulp=1.0)
    assert_bf16_parity(got_pair[0, :, :, slot0:slot0 + m], oracle.rope(heads[:, hq:hq + hkv], c, s_), max_ulp=1.0)
    np.testing.assert_array_equal(got_pair[1, :, :, slot0:slot0 + m], from_gpu_bf16(y).reshape(
        m, hq + 2 * hkv, dim).transpose(1, 0, 2)[None, hq + hkv:])
