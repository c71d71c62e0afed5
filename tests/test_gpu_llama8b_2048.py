"""Config 5 at its long bucket: prompt 2048, cache 2304 (reference ``compile_llama_bucketed``,
``models/llama.py:103-129``; bucket tests ``tests/test_llama_static_cache.py:361-440``).

Three levels, each against the CPU oracle on the same seeded inputs:

* the prefill flash attention at M = 2048, head_dim 128, 32 query / 8 kv heads (causal, and
  causal with a left pad);
* the prefill W4 GEMM at M = 2048 on the plan the decoder picks for that length (128x128
  tiles, no split-K), an N slice of the 8B q/k/v and down shapes, plain and with the
  residual epilogue;
* the 2-layer 8B-width decoder compiled as a 2048-token bucket with 256 new tokens:
  prefill logits, and greedy tokens through the ring loop (the decode attention over a
  2304-slot window splits and merges).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ops as oracle
from oracle.decoder import DecoderShape, OracleDecoder
from oracle.quant import pack_weight_bf16
from tests.helpers import (
    assert_bf16_parity,
    bf16_normal,
    first_divergence,
    from_gpu_bf16,
    near_tie,
    state_to_oracle,
    to_gpu_bf16,
    to_gpu_bits,
)

pytestmark = pytest.mark.gpu

M = 2048


@pytest.mark.timeout(300)
@pytest.mark.parametrize("length", [M, M - 300])
def test_prefill_attention_2048_tokens_d128(length):
    from aotolith_amd import ops

    rng = np.random.default_rng(length)
    hq, hkv, dim = 32, 8, 128
    q = bf16_normal(rng, (1, hq, M, dim))
    k = bf16_normal(rng, (1, hkv, M, dim))
    v = bf16_normal(rng, (1, hkv, M, dim))
    expected = oracle.attention(q, k, v, oracle.prefill_mask(length, M))
    out = ops.prefill_attention(to_gpu_bf16(q), to_gpu_bf16(k), to_gpu_bf16(v), causal=True, key_start=M - length)
    got = from_gpu_bf16(out).reshape(1, M, hq, dim).transpose(0, 2, 1, 3)
    # P is rounded to bf16 before P.V (codegen/attention.py:367-371), so the error is
    # absolute in |v| (N(0,1) values), as in the shorter cases.
    stats = assert_bf16_parity(got, expected, max_ulp=None, atol=2.0 ** -6)
    print(f"prefill attention M={M} length={length}: {stats}")
    if length < M:
        assert np.all(got[:, :, : M - length] == 0.0), "fully masked pad rows must be zero"


@pytest.mark.timeout(300)
@pytest.mark.parametrize("plan", ["fused", "wide"])
@pytest.mark.parametrize("n,k,full_n,epilogue", [
    (1024, 4096, 6144, None),        # a slice of the 8B q/k/v projection
    (1024, 4096, 4096, "residual"),  # a slice of the o projection, residual epilogue
    (512, 14336, 4096, "residual"),  # a slice of the down projection
])
def test_w4_matmul_2048_rows_on_the_decoder_plan(n, k, full_n, epilogue, plan):
    """An N slice at 2048 rows on either plan: the automatic one the decoder takes (the
    wide-tile 32x32x16 kernel) and the 16x16 kernel's own at this length (128x128 block
    tiles, tile code 28, no split-K)."""

    from aotolith_amd import ops

    assert ops.wide_plan(M, full_n, k) is not None, "the automatic plan takes the wide kernel"
    assert ops.gemm_workspace_bytes(M, full_n, k, tile=28, splits=1) == 0
    rng = np.random.default_rng(n + k)
    packed, scales = pack_weight_bf16(bf16_normal(rng, (n, k), 0.02), 64)
    x = bf16_normal(rng, (M, k))
    kwargs = {}
    if epilogue == "residual":
        kwargs["residual"] = bf16_normal(rng, (M, n))
    gpu_kwargs = {key: to_gpu_bf16(value) for key, value in kwargs.items()}
    codes = {"tile": 28, "splits": 1} if plan == "fused" else {}
    with ops.recording_launches() as take:
        take()
        y = ops.w4_matmul(to_gpu_bf16(x), torch.from_numpy(packed).cuda(), to_gpu_bits(scales), 64, **codes,
                          **gpu_kwargs)
        names = take()
    assert any(name.startswith("aoto_w4_gemm_w") for name in names) == (plan == "wide"), names
    expected = oracle.w4_matmul(x, packed, scales, 64, **kwargs)
    # Outputs reach ~6 with the N(0,1) residual, where one bf16 ulp is 2^-5: the bar is
    # one ulp of each value (and the absolute bar one ulp of the largest).
    top_ulp = 2.0 ** (np.floor(np.log2(np.abs(expected).max())) - 7)
    stats = assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=1.0, atol=max(2e-2, top_ulp))
    print(f"w4 matmul {plan} M={M} N={n} K={k} {epilogue}: {stats}")


def _spec(layers=2):
    from aotolith_amd.decoder import DecoderSpec

    return DecoderSpec(family="llama", vocab=128256, hidden=4096, intermediate=14336, layers=layers, heads=32,
                       kv_heads=8, head_dim=128, eps=1e-5, theta=5e5, qkv_bias=False, max_position=131072)


@pytest.mark.timeout(900)
def test_llama8b_width_bucket_2048_prefill_and_greedy_match_the_oracle():
    from aotolith_amd.decoder import compile_decoder_bucketed_state, random_state

    spec = _spec()
    state = random_state(spec, 64, seed=5, norm_std=0.1)
    runtime = compile_decoder_bucketed_state(spec, state, prompt_lengths=[M], max_new_tokens=256)
    bucket = runtime.buckets[0]
    assert bucket.cache_capacity == M + 256
    shape = DecoderShape(vocab=spec.vocab, hidden=spec.hidden, intermediate=spec.intermediate, layers=spec.layers,
                         heads=spec.heads, kv_heads=spec.kv_heads, head_dim=spec.head_dim, eps=spec.eps,
                         theta=spec.theta)
    oracle_decoder = OracleDecoder(shape, state_to_oracle(state), M + 256)
    ids = np.random.default_rng(6).integers(0, spec.vocab, M)
    logits, cache = bucket.prefill_ids(ids)
    ref_logits, ref_cache = oracle_decoder.prefill(ids)
    scale = float(np.abs(ref_logits).max())
    # Two 8B-width layers compound bf16 roundings (one per residual add, the flash
    # kernel's bf16 P): the bar is relative to the logits' range, plus the cosine bar.
    stats = assert_bf16_parity(from_gpu_bf16(logits), ref_logits, max_ulp=None, atol=0.02 * scale, min_cos=0.9999)
    print(f"bucket {M} prefill logits: max|ref| {scale:.3f}, {stats}")
    cache_stats = assert_bf16_parity(from_gpu_bf16(cache), ref_cache, max_ulp=None, atol=2e-2 * float(
        np.abs(ref_cache).max()), min_cos=0.9999)
    print(f"bucket {M} prefill cache: {cache_stats}")
    steps = 9
    tokens = runtime.greedy_generate(ids, max_new_tokens=steps).cpu().numpy()
    want, history = oracle_decoder.greedy_generate(ids, steps, record_logits=True)
    print(f"bucket {M} greedy: gpu {tokens.reshape(-1).tolist()} oracle {want.tolist()}")
    divergence = first_divergence(tokens, want, history)
    if divergence is not None:
        assert near_tie(divergence, history), divergence
