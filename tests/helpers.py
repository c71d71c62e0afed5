"""Shared test helpers: seeded bf16 data, parity metrics, GPU gating."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.bf16 import from_bf16_bits, round_bf16, to_bf16_bits


def gpu_available() -> bool:
    return torch.cuda.is_available()


requires_gpu = pytest.mark.skipif(not gpu_available(), reason="needs an MI355X")


def bf16_normal(rng: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    """bf16-representable N(0, std) values as f32."""

    return round_bf16(rng.standard_normal(shape).astype(np.float32) * np.float32(std))


def to_gpu_bf16(values: np.ndarray) -> torch.Tensor:
    bits = to_bf16_bits(values)
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).cuda()


def to_gpu_bits(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).copy()).view(torch.bfloat16).cuda()


def from_gpu_bf16(tensor: torch.Tensor) -> np.ndarray:
    return from_bf16_bits(tensor.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16))


def bf16_bits_of(tensor: torch.Tensor) -> np.ndarray:
    return tensor.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def parity(actual: np.ndarray, expected: np.ndarray) -> dict:
    a = np.asarray(actual, dtype=np.float64).reshape(-1)
    e = np.asarray(expected, dtype=np.float64).reshape(-1)
    diff = np.abs(a - e)
    denom = np.linalg.norm(a) * np.linalg.norm(e)
    cosine = float(a @ e / denom) if denom > 0 else (1.0 if np.all(a == e) else 0.0)
    # Distance in bf16 ulps (1 ulp = 2^-7 relative to the leading bit) of the larger
    # of the two values: an f32 sum that lands on the other side of a binade edge
    # rounds to a neighbour one ulp away in the wider binade. Values far below the
    # row's scale (cancellation) are measured against 2^-10 of the largest value,
    # where f32 accumulation noise, not the final rounding, sets the error.
    floor = max(float(np.abs(e).max()) * 2.0 ** -10 if e.size else 0.0, 2.0 ** -126)
    scale = np.maximum(np.maximum(np.abs(e), np.abs(a)), floor)
    ulp = 2.0 ** (np.floor(np.log2(scale)) - 7)
    return {
        "max_abs": float(diff.max()) if diff.size else 0.0,
        "cosine": cosine,
        "max_ulp": float((diff / ulp).max()) if diff.size else 0.0,
        "mismatch": int((diff > 0).sum()),
    }


def assert_bf16_parity(
    actual, expected, *, max_ulp: float | None = 1.0, atol: float = 2e-2, min_cos: float = 0.999
) -> dict:
    """North-star bars (max abs <= 2e-2, cosine >= 0.999) plus an ulp bound (None: no ulp bound)."""

    stats = parity(actual, expected)
    assert stats["max_abs"] <= atol, stats
    assert stats["cosine"] >= min_cos, stats
    if max_ulp is not None:
        assert stats["max_ulp"] <= max_ulp, stats
    return stats
