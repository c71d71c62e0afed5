"""Llama frontend of the static-cache adapter (the reference's models/llama.py:60-129)."""

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

FAMILY = "llama"

__all__ = ["check_llama_model", "compile_llama_bucketed", "compile_llama_static_cache", "prefill_mask"]


def check_llama_model(model: torch.nn.Module) -> None:
    """Check the family of ``model`` before any packing: a config whose ``model_type`` is not
    ``llama`` is refused with ``UnsupportedModelError`` naming the entry point to use instead."""

    family_for(model, require=FAMILY)


def compile_llama_static_cache(
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
    """Pack a Llama model's projections on the GPU and build its prefill / decode plan pair
    for one prompt length (cache capacity ``prompt_length + max_new_tokens``), batch 1."""

    check_llama_model(model)
    return compile_decoder_static_cache(
        model, prompt_length=prompt_length, max_new_tokens=max_new_tokens, codegen_matmul=codegen_matmul,
        codegen_attention=codegen_attention, autotune=autotune, quantize=quantize, quantize_bits=quantize_bits,
        family=FAMILY, target=target, memory=memory,
    )


def compile_llama_bucketed(
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
    """Pack the Llama weights once and build a prefill / decode plan pair for every width in
    ``prompt_lengths`` over that one device state; a prompt runs in the narrowest bucket it fits."""

    check_llama_model(model)
    return compile_decoder_bucketed(
        model, prompt_lengths=prompt_lengths, max_new_tokens=max_new_tokens, codegen_matmul=codegen_matmul,
        codegen_attention=codegen_attention, autotune=autotune, quantize=quantize, quantize_bits=quantize_bits,
        family=FAMILY, target=target,
    )
