"""The eight-bit (``quantize_bits=8``) decoder end to end on the GPU against the oracle.

Counterparts of the reference's int8 model tests
(tests/test_quantized_qwen2.py:224-320): greedy decode of an int8-packed model
agrees with the oracle decoder run on the same packed state, and every packed
input is twice as wide as at four bits (four codes a word). The state is
uploaded bit for bit from the oracle's eight-bit packer; prefill logits/cache
and a functional decode step meet the per-op bf16 bars and greedy tokens are
identical up to near-ties of the oracle's logits.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from oracle.decoder import DecoderShape, OracleDecoder
from tests.helpers import (
    assert_bf16_parity,
    first_divergence,
    from_gpu_bf16,
    random_oracle_state,
    runtime_spec,
    state_to_device,
    to_gpu_bf16,
)

pytestmark = pytest.mark.gpu

TINY8 = DecoderShape(vocab=512, hidden=256, intermediate=512, layers=2, heads=4, kv_heads=2, head_dim=64,
                     eps=1e-6, theta=1e6, bits=8)
PROMPT, NEW = 16, 10


def _pair(seed=0, bias=True, prompt=PROMPT, new=NEW):
    from aotolith_amd.decoder import compile_decoder_state

    ostate = random_oracle_state(TINY8, seed, bias=bias)
    state = state_to_device(ostate, TINY8.group_size, bits=8)
    runtime = compile_decoder_state(runtime_spec(TINY8, "qwen2", bias), state, prompt_length=prompt,
                                    max_new_tokens=new)
    return runtime, OracleDecoder(TINY8, ostate, prompt + new)


def test_w8_prefill_logits_and_cache():
    runtime, oracle = _pair(seed=31)
    assert runtime.quantize_bits == 8
    ids = np.random.default_rng(32).integers(0, TINY8.vocab, PROMPT)
    logits, cache = runtime.prefill_ids(ids)
    ref_logits, ref_cache = oracle.prefill(ids)
    assert_bf16_parity(from_gpu_bf16(logits), ref_logits, max_ulp=None)
    assert_bf16_parity(from_gpu_bf16(cache), ref_cache, max_ulp=None)


def test_w8_decode_token_matches_the_oracle():
    runtime, oracle = _pair(seed=33)
    ids = np.random.default_rng(34).integers(0, TINY8.vocab, PROMPT)
    ref_logits, ref_compact = oracle.prefill(ids)
    ref_cache = oracle.pad_cache(ref_compact)
    cache = runtime.pad_cache(to_gpu_bf16(ref_compact))
    token = int(np.argmax(ref_logits))
    logits, next_cache = runtime.decode_token(torch.tensor([[token]]), cache, PROMPT + 1)
    want_logits, want_cache = oracle.decode(token, PROMPT + 1, ref_cache)
    assert_bf16_parity(from_gpu_bf16(logits), want_logits, max_ulp=None)
    cap = PROMPT + NEW
    assert_bf16_parity(from_gpu_bf16(next_cache)[..., cap - 1, :], want_cache[..., cap - 1, :], max_ulp=None)


@pytest.mark.parametrize("use_graph", [True, False])
def test_w8_greedy_tokens_match_the_oracle(use_graph):
    runtime, oracle = _pair(seed=35)
    # no fused argmax tail at eight bits: the loop runs GEMV + argmax + step advance
    assert runtime.engine.keys is None
    ids = np.random.default_rng(36).integers(0, TINY8.vocab, PROMPT)
    tokens = runtime.greedy_generate(ids, use_graph=use_graph).cpu().numpy()
    want, history = oracle.greedy_generate(ids, NEW, record_logits=True)
    divergence = first_divergence(tokens, want, history)
    if divergence is not None:
        scale = float(np.abs(history[divergence["step"]]).max())
        limit = 2 * 2.0 ** -7 * max(abs(divergence["want_logit"]), scale * 2.0 ** -4)
        assert divergence["margin"] <= limit, divergence
    if use_graph:
        assert runtime.engine.graph_error is None, runtime.engine.graph_error
        assert runtime.engine.prefill_graph_error is None, runtime.engine.prefill_graph_error


def test_w8_selections_name_the_eight_bit_kernels():
    runtime, _ = _pair(seed=37)
    decode_kinds = {s.kind for s in runtime.decode.selections}
    prefill_kinds = {s.kind for s in runtime.prefill.selections}
    assert "w8_gemv" in decode_kinds and "w4_gemv" not in decode_kinds
    assert "w8_gemm" in prefill_kinds and "w4_gemm" not in prefill_kinds
    assert all(s.is_native for s in runtime.decode.selections + runtime.prefill.selections)


def test_w8_state_is_twice_as_wide_as_w4():
    """tests/test_quantized_qwen2.py:263-296: every packed input doubles in width at eight bits."""

    four = random_oracle_state(dataclasses.replace(TINY8, bits=4), 38)
    eight = random_oracle_state(TINY8, 38)
    for key in ("qkv", "o", "gate", "up", "down"):
        p4, s4 = four["layers"][0][key]
        p8, s8 = eight["layers"][0][key]
        assert p8.shape == (p4.shape[0], 2 * p4.shape[1])
        assert s8.shape == s4.shape


def test_w8_artifact_round_trip(tmp_path):
    from aotolith_amd import load_runtime, read_artifact_manifest

    runtime, _ = _pair(seed=39)
    ids = np.random.default_rng(40).integers(0, TINY8.vocab, PROMPT)
    tokens = runtime.greedy_generate(ids).cpu()
    _, decode_path = runtime.save(tmp_path / "w8")
    manifest = read_artifact_manifest(decode_path)
    assert manifest["compile_options"]["quantize_bits"] == 8
    loaded = load_runtime(tmp_path / "w8")
    assert loaded.quantize_bits == 8
    assert loaded.engine.state.lm_head.bits == 8
    assert torch.equal(loaded.greedy_generate(ids).cpu(), tokens)


def test_w8_compile_from_a_hf_module():
    """compile_qwen2_static_cache(quantize_bits=8) packs on the GPU bit for bit with the oracle's packer."""

    import aotolith_amd as aoto
    from oracle.quant import pack_weight_bits_bf16

    from tests.test_gpu_hf import _f32, _model

    model = _model("qwen2", 41)
    runtime = aoto.compile_qwen2_static_cache(model, prompt_length=16, max_new_tokens=4, quantize=64,
                                              quantize_bits=8, target="hip-gfx950")
    assert runtime.quantize_bits == 8
    down = model.model.layers[1].mlp.down_proj.weight
    want_packed, want_scales = pack_weight_bits_bf16(_f32(down), 64, 8)
    got = runtime.engine.state.layers[1].down
    np.testing.assert_array_equal(got.packed.cpu().numpy(), want_packed)
    np.testing.assert_array_equal(got.scales.cpu().view(torch.int16).numpy().view(np.uint16), want_scales)
    tokens = runtime.greedy_generate(np.arange(16)).cpu().numpy()
    assert tokens.shape == (1, 4)
