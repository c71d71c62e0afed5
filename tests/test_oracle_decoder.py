"""Pin the oracle decoder against HuggingFace torch eager on round-tripped weights.

The reference checks its quantized plans the same way: greedy tokens of the
compiled plan against a torch run whose weights went through the int4 round trip
(``tests/test_quantized_qwen2.py:107-123``). Here the HF model runs in fp32 with
every projection set to the bf16 dequantized weight the oracle multiplies, so
the two differ only in the oracle's bf16 rounding points (and its bf16 RoPE
angles): prefill logits must agree to bf16-level tolerance and greedy tokens
must be identical or flip only where the oracle's top two logits nearly tie.
A wrong layer order, residual, norm placement, RoPE convention or GQA mapping
in the oracle breaks this by far more than bf16 noise.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.bf16 import round_bf16
from oracle.decoder import DecoderShape, OracleDecoder
from oracle.quant import dequantize_i4_bf16, pack_weight_bf16

GROUP = 16


def _hf(family: str, seed: int):
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen2Config, Qwen2ForCausalLM

    common = dict(vocab_size=96, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                  num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64,
                  tie_word_embeddings=False)
    torch.manual_seed(seed)
    if family == "qwen2":
        config = Qwen2Config(rms_norm_eps=1e-6, rope_parameters={"rope_type": "default", "rope_theta": 1e6},
                             **common)
        model = Qwen2ForCausalLM(config)
    else:
        config = LlamaConfig(rms_norm_eps=1e-5, rope_parameters={"rope_type": "default", "rope_theta": 5e5},
                             **common)
        model = LlamaForCausalLM(config)
    return model.eval().float()


def _round_trip(model, seed: int):
    """Give the model bf16-exact random weights, quantize its projections, return (oracle state, shape)."""

    rng = np.random.default_rng(seed)
    cfg = model.config
    h = cfg.hidden_size

    def bf(shape, std):
        return round_bf16(rng.standard_normal(shape).astype(np.float32) * np.float32(std))

    def setp(param, value):
        with torch.no_grad():
            param.copy_(torch.from_numpy(np.asarray(value, dtype=np.float32)).reshape(param.shape))

    def packed(param):
        weight = bf(tuple(param.shape), 0.08)
        pair = pack_weight_bf16(weight, GROUP)
        setp(param, dequantize_i4_bf16(pair[0], pair[1], GROUP))
        return pair

    embed = bf((cfg.vocab_size, h), 1.0)
    setp(model.model.embed_tokens.weight, embed)
    layers = []
    for layer in model.model.layers:
        att, mlp = layer.self_attn, layer.mlp
        q, k, v = (packed(p.weight) for p in (att.q_proj, att.k_proj, att.v_proj))
        qkv = (np.concatenate([q[0], k[0], v[0]]), np.concatenate([q[1], k[1], v[1]]))
        bias = None
        if att.q_proj.bias is not None:
            parts = [bf((p.bias.shape[0],), 0.05) for p in (att.q_proj, att.k_proj, att.v_proj)]
            for p, value in zip((att.q_proj, att.k_proj, att.v_proj), parts):
                setp(p.bias, value)
            bias = np.concatenate(parts)
        in_norm = round_bf16(np.float32(1.0) + bf((h,), 0.1))
        post_norm = round_bf16(np.float32(1.0) + bf((h,), 0.1))
        setp(layer.input_layernorm.weight, in_norm)
        setp(layer.post_attention_layernorm.weight, post_norm)
        layers.append({"qkv": qkv, "o": packed(att.o_proj.weight), "gate": packed(mlp.gate_proj.weight),
                       "up": packed(mlp.up_proj.weight), "down": packed(mlp.down_proj.weight),
                       "qkv_bias": bias, "input_norm": in_norm, "post_norm": post_norm})
    final = round_bf16(np.float32(1.0) + bf((h,), 0.1))
    setp(model.model.norm.weight, final)
    state = {"embed": embed, "final_norm": final, "lm_head": packed(model.lm_head.weight), "layers": layers}
    theta = float(cfg.rope_parameters["rope_theta"])
    shape = DecoderShape(vocab=cfg.vocab_size, hidden=h, intermediate=cfg.intermediate_size,
                         layers=cfg.num_hidden_layers, heads=cfg.num_attention_heads,
                         kv_heads=cfg.num_key_value_heads, head_dim=h // cfg.num_attention_heads,
                         eps=float(cfg.rms_norm_eps), theta=theta, group_size=GROUP)
    return state, shape


def _hf_greedy(model, ids: np.ndarray, steps: int):
    seq = torch.from_numpy(ids)[None]
    tokens, logits_hist = [], []
    with torch.no_grad():
        for _ in range(steps):
            logits = model(seq).logits[0, -1].double().numpy()
            tok = int(np.argmax(logits))
            tokens.append(tok)
            logits_hist.append(logits)
            seq = torch.cat([seq, torch.tensor([[tok]])], dim=1)
    return np.array(tokens), logits_hist


@pytest.mark.parametrize("family", ["qwen2", "llama"])
def test_oracle_prefill_logits_match_hf_eager(family):
    model = _hf(family, 1)
    state, shape = _round_trip(model, 2)
    ids = np.random.default_rng(3).integers(0, shape.vocab, 12)
    oracle = OracleDecoder(shape, state, 24)
    logits, cache = oracle.prefill(ids)
    with torch.no_grad():
        ref = model(torch.from_numpy(ids)[None]).logits[0, -1].double().numpy()
    got = np.asarray(logits, dtype=np.float64).reshape(-1)
    cosine = float(got @ ref / (np.linalg.norm(got) * np.linalg.norm(ref)))
    assert cosine >= 0.999, cosine
    assert np.abs(got - ref).max() <= 0.03 * np.abs(ref).max() + 1e-3
    assert cache.shape == (shape.layers, 2, 1, shape.kv_heads, 12, shape.head_dim)


@pytest.mark.parametrize("family", ["qwen2", "llama"])
def test_oracle_greedy_tokens_match_hf_eager(family):
    model = _hf(family, 4)
    state, shape = _round_trip(model, 5)
    ids = np.random.default_rng(6).integers(0, shape.vocab, 10)
    steps = 8
    oracle = OracleDecoder(shape, state, 10 + steps)
    got, hist = oracle.greedy_generate(ids, steps, record_logits=True)
    want, want_hist = _hf_greedy(model, ids, steps)
    for step in range(steps):
        if got[step] != want[step]:
            ref = want_hist[step]
            top = np.sort(ref)[-2:]
            margin = float(top[1] - top[0])
            # a flip is only acceptable on a near-tie of the fp32 reference
            assert margin <= 0.02 * np.abs(ref).max(), (step, got.tolist(), want.tolist(), margin)
            break


def test_oracle_decode_step_equals_a_longer_prefill():
    """Decode at position p with the rolled cache gives the prefill's last-token logits of p + 1 tokens."""

    model = _hf("qwen2", 7)
    state, shape = _round_trip(model, 8)
    ids = np.random.default_rng(9).integers(0, shape.vocab, 9)
    cap = 16
    oracle = OracleDecoder(shape, state, cap)
    _, compact = oracle.prefill(ids[:8])
    cache = oracle.pad_cache(compact)
    step_logits, next_cache = oracle.decode(int(ids[8]), 9, cache)
    full_logits, full_compact = oracle.prefill(ids)
    a = np.asarray(step_logits, dtype=np.float64).reshape(-1)
    b = np.asarray(full_logits, dtype=np.float64).reshape(-1)
    # decode rounds at the GEMV's points, prefill at the GEMM's: bf16-level agreement
    assert float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b))) >= 0.999
    # the rolled window holds the same nine keys/values at its end
    np.testing.assert_allclose(next_cache[..., cap - 9:, :], full_compact, atol=0.1, rtol=0.05)
