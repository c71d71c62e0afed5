"""The public entry points on real HuggingFace modules: GPU packing, adapter, tokens vs the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.bf16 import round_bf16
from oracle.decoder import DecoderShape, OracleDecoder
from oracle.quant import pack_weight_bf16
from tests.helpers import first_divergence

pytestmark = pytest.mark.gpu


def _model(family: str, seed: int):
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen2Config, Qwen2ForCausalLM

    common = dict(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                  num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=128)
    torch.manual_seed(seed)
    if family == "qwen2":
        model = Qwen2ForCausalLM(Qwen2Config(rms_norm_eps=1e-6, tie_word_embeddings=True,
                                             rope_parameters={"rope_type": "default", "rope_theta": 1e6},
                                             **common))
    else:
        model = LlamaForCausalLM(LlamaConfig(rms_norm_eps=1e-5, tie_word_embeddings=False,
                                             rope_parameters={"rope_type": "default", "rope_theta": 5e5},
                                             **common))
    model = model.to(torch.bfloat16).eval()
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" in name:
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g))
            elif name.endswith("bias"):
                p.copy_(0.05 * torch.randn(p.shape, generator=g))
            elif "embed" in name:
                p.copy_(torch.randn(p.shape, generator=g))
            else:
                p.copy_(0.05 * torch.randn(p.shape, generator=g))
    return model


def _f32(t):
    return t.detach().float().cpu().numpy()


def _oracle_state(model):
    layers = []
    for layer in model.model.layers:
        att, mlp = layer.self_attn, layer.mlp
        qkv = torch.cat((att.q_proj.weight, att.k_proj.weight, att.v_proj.weight))
        bias = None if att.q_proj.bias is None else _f32(torch.cat((att.q_proj.bias, att.k_proj.bias,
                                                                     att.v_proj.bias)))
        layers.append({
            "qkv": pack_weight_bf16(_f32(qkv), 64), "o": pack_weight_bf16(_f32(att.o_proj.weight), 64),
            "gate": pack_weight_bf16(_f32(mlp.gate_proj.weight), 64),
            "up": pack_weight_bf16(_f32(mlp.up_proj.weight), 64),
            "down": pack_weight_bf16(_f32(mlp.down_proj.weight), 64), "qkv_bias": bias,
            "input_norm": _f32(layer.input_layernorm.weight), "post_norm": _f32(layer.post_attention_layernorm.weight),
        })
    return {"embed": _f32(model.model.embed_tokens.weight), "final_norm": _f32(model.model.norm.weight),
            "lm_head": pack_weight_bf16(_f32(model.lm_head.weight), 64), "layers": layers}


@pytest.mark.parametrize("family", ["qwen2", "llama"])
def test_compile_static_cache_from_a_hf_module(family):
    import aotolith_amd as aoto

    model = _model(family, 3 if family == "qwen2" else 5)
    compile_fn = aoto.compile_qwen2_static_cache if family == "qwen2" else aoto.compile_llama_static_cache
    runtime = compile_fn(model, prompt_length=16, max_new_tokens=8, quantize=64, target="hip-gfx950")
    ostate = _oracle_state(model)
    # the GPU packer reproduces the oracle's packing bit for bit
    layer0 = runtime.engine.state.layers[0]
    np.testing.assert_array_equal(layer0.qkv.packed.cpu().numpy(), ostate["layers"][0]["qkv"][0])
    np.testing.assert_array_equal(
        layer0.down.scales.cpu().view(torch.int16).numpy().view(np.uint16), ostate["layers"][0]["down"][1])
    cfg = model.config
    shape = DecoderShape(vocab=cfg.vocab_size, hidden=cfg.hidden_size, intermediate=cfg.intermediate_size,
                         layers=cfg.num_hidden_layers, heads=cfg.num_attention_heads,
                         kv_heads=cfg.num_key_value_heads, head_dim=64, eps=float(cfg.rms_norm_eps),
                         theta=float(cfg.rope_parameters["rope_theta"]))
    oracle = OracleDecoder(shape, ostate, 24)
    ids = np.random.default_rng(7).integers(0, cfg.vocab_size, 16)
    tokens = runtime.greedy_generate(ids).cpu().numpy()
    want, history = oracle.greedy_generate(ids, 8, record_logits=True)
    divergence = first_divergence(tokens, want, history)
    if divergence is not None:
        scale = float(np.abs(history[divergence["step"]]).max())
        assert divergence["margin"] <= 2 * 2.0 ** -7 * max(abs(divergence["want_logit"]), scale / 16), divergence
    assert runtime.family == family
    assert all(s.is_native for s in runtime.decode.selections)


def test_bucketed_llama_from_a_hf_module():
    import aotolith_amd as aoto

    model = _model("llama", 11)
    runtime = aoto.compile_llama_bucketed(model, prompt_lengths=[8, 16], max_new_tokens=4, quantize=64)
    assert runtime.family == "llama" and runtime.prompt_lengths == (8, 16)
    assert runtime.buckets[0].engine.state is runtime.buckets[1].engine.state
    short = runtime.greedy_generate(np.arange(5))
    long = runtime.greedy_generate(np.arange(12))
    assert short.shape == (1, 4) and long.shape == (1, 4)


def test_fp32_module_is_refused():
    import aotolith_amd as aoto
    from aotolith_amd.errors import UnsupportedDTypeError

    model = _model("qwen2", 13).float()
    with pytest.raises(UnsupportedDTypeError):
        aoto.compile_qwen2_static_cache(model, prompt_length=8, max_new_tokens=4, quantize=64)
