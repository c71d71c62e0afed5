"""Host-side adapter checks that need no GPU: family, config reading, refusals, API errors."""

from __future__ import annotations

import pytest
import torch


def _qwen(**overrides):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = dict(vocab_size=64, hidden_size=128, intermediate_size=256, num_hidden_layers=1,
               num_attention_heads=2, num_key_value_heads=1, max_position_embeddings=64,
               rope_parameters={"rope_type": "default", "rope_theta": 1e6}, tie_word_embeddings=True)
    cfg.update(overrides)
    return Qwen2ForCausalLM(Qwen2Config(**cfg)).eval()


def _llama(**overrides):
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = dict(vocab_size=64, hidden_size=128, intermediate_size=256, num_hidden_layers=1,
               num_attention_heads=2, num_key_value_heads=2, max_position_embeddings=64,
               rope_parameters={"rope_type": "default", "rope_theta": 5e5})
    cfg.update(overrides)
    return LlamaForCausalLM(LlamaConfig(**cfg)).eval()


def test_spec_reads_transformers5_configs():
    from aotolith_amd.decoder import spec_from_model

    spec = spec_from_model(_qwen())
    assert (spec.family, spec.hidden, spec.heads, spec.kv_heads, spec.head_dim) == ("qwen2", 128, 2, 1, 64)
    assert spec.theta == 1e6 and spec.qkv_bias and spec.tied and spec.eps == pytest.approx(1e-6)
    lspec = spec_from_model(_llama())
    assert lspec.family == "llama" and lspec.theta == 5e5 and not lspec.qkv_bias


def test_family_pinning_and_refusals():
    from aotolith_amd.decoder import family_for, spec_from_model
    from aotolith_amd.errors import UnsupportedModelError

    with pytest.raises(UnsupportedModelError):
        family_for(_qwen(), require="llama")
    with pytest.raises(UnsupportedModelError):
        spec_from_model(_llama(rope_parameters={"rope_type": "linear", "factor": 2.0, "rope_theta": 5e5}))
    with pytest.raises(UnsupportedModelError):
        spec_from_model(_llama(hidden_act="gelu"))


def test_compile_entry_points_refuse_before_touching_a_gpu():
    import aotolith_amd as aoto
    from aotolith_amd.errors import CompilationError, DynamicShapeError, UnsupportedModelError

    with pytest.raises(CompilationError):
        aoto.compile_qwen2_static_cache(_qwen(), prompt_length=8, max_new_tokens=4, quantize=64,
                                        target="apple-metal")
    with pytest.raises(CompilationError):
        aoto.compile_qwen2_static_cache(_qwen(), prompt_length=8, max_new_tokens=4, quantize=None)
    with pytest.raises(CompilationError):
        aoto.compile_qwen2_static_cache(_qwen(), prompt_length=8, max_new_tokens=4, quantize=64,
                                        quantize_bits=3)
    with pytest.raises(UnsupportedModelError):
        aoto.compile_llama_static_cache(_qwen(), prompt_length=8, max_new_tokens=4, quantize=64)
    with pytest.raises(DynamicShapeError):
        aoto.compile_qwen2_static_cache(_qwen(), prompt_length=60, max_new_tokens=8, quantize=64)
    train = _qwen().train()
    with pytest.raises(CompilationError):
        aoto.compile_qwen2_static_cache(train, prompt_length=8, max_new_tokens=4, quantize=64)


def test_kernel_limits_are_checked_at_compile_time():
    from aotolith_amd.decoder import DecoderSpec, _check_kernel_limits
    from aotolith_amd.errors import CompilationError

    good = DecoderSpec("qwen2", 64, 896, 4864, 1, 14, 2, 64, 1e-6, 1e6, True)
    _check_kernel_limits(good, 64)
    with pytest.raises(CompilationError):
        _check_kernel_limits(DecoderSpec("qwen2", 64, 896, 4864, 1, 7, 1, 128 - 32, 1e-6, 1e6, True), 64)
    with pytest.raises(CompilationError):
        _check_kernel_limits(good, 48)


def test_no_gpu_means_a_device_error():
    from aotolith_amd.decoder import DecoderSpec, random_state
    from aotolith_amd.errors import DeviceError

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(DeviceError):
        random_state(DecoderSpec("qwen2", 64, 128, 256, 1, 2, 1, 64, 1e-6, 1e6, True))


def test_kernel_limits_refuse_per_node_with_reasons():
    """A shape outside the kernels' limits is refused node by node (reference backends/apple.py:719-740);
    the compile error carries each refused node's selection record."""

    from aotolith_amd.decoder import DecoderSpec, _check_kernel_limits, kernel_refusals
    from aotolith_amd.errors import CompilationError

    assert kernel_refusals(DecoderSpec("qwen2", 64, 896, 4864, 2, 14, 2, 64, 1e-6, 1e6, True), 64) == ()
    bad = DecoderSpec("llama", 64, 896, 4864, 2, 14, 2, 96, 1e-6, 1e6, False)   # head_dim 96
    refused = kernel_refusals(bad, 64)
    assert [s.output_id for s in refused] == ["attention_0", "attention_1"]
    assert all(s.implementation == "unsupported" and not s.is_native and "head_dim 96" in s.reason for s in refused)
    with pytest.raises(CompilationError) as info:
        _check_kernel_limits(bad, 64)
    assert info.value.refused == refused
    odd = DecoderSpec("qwen2", 64, 896, 4864, 1, 14, 2, 64, 1e-6, 1e6, True)
    by_node = {s.output_id: s.reason for s in kernel_refusals(odd, 48)}
    assert set(by_node) == {"qkv_0", "hidden_0a", "mlp_0", "hidden_0b", "logits"}
    assert all("group size 48" in reason for reason in by_node.values())


def test_backend_seam_registry():
    """The target registry and backend object of the reference's seam (backends/__init__.py:38-55)."""

    from aotolith_amd.backends import TARGETS, HipGfx950Backend, backend_for
    from aotolith_amd.errors import CompilationError

    assert TARGETS == ("hip-gfx950",)
    assert isinstance(backend_for("hip-gfx950"), HipGfx950Backend)
    assert backend_for("hip-gfx950").name == "hip-gfx950"
    with pytest.raises(CompilationError, match="unsupported target"):
        backend_for("apple-metal")
    with pytest.raises(CompilationError, match="autotune"):
        backend_for("hip-gfx950", autotune=True)
