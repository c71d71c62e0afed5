"""Config 5 shapes on the GPU: Llama-3-8B widths (hidden 4096, intermediate 14336, 32/8 heads,
head_dim 128, vocab 128256) at two layers, bucket 512 with 256 new tokens (cache 768, so the
decode attention splits and merges), against the CPU oracle on the same packed state."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.decoder import DecoderShape, OracleDecoder
from tests.helpers import assert_bf16_parity, first_divergence, from_gpu_bf16, state_to_oracle

pytestmark = pytest.mark.gpu


def _spec(layers=2):
    from aotolith_amd.decoder import DecoderSpec

    return DecoderSpec(family="llama", vocab=128256, hidden=4096, intermediate=14336, layers=layers, heads=32,
                       kv_heads=8, head_dim=128, eps=1e-5, theta=5e5, qkv_bias=False, max_position=131072)


@pytest.mark.timeout(600)
def test_llama8b_width_prefill_and_greedy_match_the_oracle():
    from aotolith_amd.decoder import compile_decoder_bucketed_state, random_state

    spec = _spec()
    state = random_state(spec, 64, seed=3, norm_std=0.1)
    runtime = compile_decoder_bucketed_state(spec, state, prompt_lengths=[512], max_new_tokens=256)
    bucket = runtime.buckets[0]
    shape = DecoderShape(vocab=spec.vocab, hidden=spec.hidden, intermediate=spec.intermediate, layers=spec.layers,
                         heads=spec.heads, kv_heads=spec.kv_heads, head_dim=spec.head_dim, eps=spec.eps,
                         theta=spec.theta)
    oracle = OracleDecoder(shape, state_to_oracle(state), 512 + 256)
    ids = np.random.default_rng(4).integers(0, spec.vocab, 512)
    logits, _ = bucket.prefill_ids(ids)
    ref_logits, _ = oracle.prefill(ids)
    # End to end through two 8B-width layers the bf16 roundings compound (the flash
    # kernel's bf16 P, one rounding per residual add): the per-op 2e-2 bar becomes
    # a bar relative to the logits' range, plus the cosine bar.
    scale = float(np.abs(ref_logits).max())
    stats = assert_bf16_parity(from_gpu_bf16(logits), ref_logits, max_ulp=None, atol=0.02 * scale)
    print(f"llama8b-width prefill logits: max|ref| {scale:.3f}, {stats}")
    steps = 6
    tokens = runtime.greedy_generate(ids, max_new_tokens=steps).cpu().numpy()
    want, history = oracle.greedy_generate(ids, steps, record_logits=True)
    divergence = first_divergence(tokens, want, history)
    if divergence is not None:
        scale = float(np.abs(history[divergence["step"]]).max())
        assert divergence["margin"] <= 2 * 2.0 ** -7 * max(abs(divergence["want_logit"]), scale / 16), divergence
