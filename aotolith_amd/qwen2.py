"""Qwen2/Qwen2.5 frontend of the static-cache adapter (the reference's models/qwen2.py:60-127)."""

from __future__ import annotations

from collections.abc import Sequence

import torch

from .decoder import (
    TARGET,
    DecoderBucketedRuntime,
    DecoderStaticCacheRuntime,
    compile_decoder_bucketed,
    compile_decoder_static_cache,
    family_for,
    prefill_mask,
)

FAMILY = "qwen2"

__all__ = ["check_qwen2_model", "compile_qwen2_bucketed", "compile_qwen2_static_cache", "prefill_mask"]


def check_qwen2_model(model: torch.nn.Module) -> None:
    """Raise unless ``model`` is a Qwen2 checkpoint this adapter covers."""

    family_for(model, require=FAMILY)


def compile_qwen2_static_cache(
    model: torch.nn.Module,
    *,
    prompt_length: int,
    max_new_tokens: int,
    codegen_matmul: bool = False,
    codegen_attention: bool = False,
    autotune: bool = False,
    quantize: int | None = None,
    quantize_bits: int = 4,
    target: str = TARGET,
    memory: str = "latency",
) -> DecoderStaticCacheRuntime:
    """Compile a Qwen2/Qwen2.5 causal LM for greedy single-request generation."""

    check_qwen2_model(model)
    return compile_decoder_static_cache(
        model, prompt_length=prompt_length, max_new_tokens=max_new_tokens, codegen_matmul=codegen_matmul,
        codegen_attention=codegen_attention, autotune=autotune, quantize=quantize, quantize_bits=quantize_bits,
        family=FAMILY, target=target, memory=memory,
    )


def compile_qwen2_bucketed(
    model: torch.nn.Module,
    *,
    prompt_lengths: Sequence[int],
    max_new_tokens: int,
    codegen_matmul: bool = False,
    codegen_attention: bool = False,
    autotune: bool = False,
    quantize: int | None = None,
    quantize_bits: int = 4,
    target: str = TARGET,
) -> DecoderBucketedRuntime:
    """Compile one Qwen2 plan pair per prompt-length bucket."""

    check_qwen2_model(model)
    return compile_decoder_bucketed(
        model, prompt_lengths=prompt_lengths, max_new_tokens=max_new_tokens, codegen_matmul=codegen_matmul,
        codegen_attention=codegen_attention, autotune=autotune, quantize=quantize, quantize_bits=quantize_bits,
        family=FAMILY, target=target,
    )
