"""bfloat16 helpers for the oracle: round-to-nearest-even on raw bits.

The reference stores every activation, scale and cache entry in the model's
compute dtype, bf16 (``models/quantized.py:149-152``, ``models/decoder.py:323-334``),
so the oracle needs the exact RNE cast torch and MLX perform. NumPy has no bf16
dtype; values travel as ``uint16`` bit patterns and widen losslessly to f32.
"""

from __future__ import annotations

import numpy as np


def to_bf16_bits(values) -> np.ndarray:
    """Round f32 (or wider) values to bf16, returned as ``uint16`` bits (RNE)."""

    f32 = np.ascontiguousarray(np.asarray(values, dtype=np.float32))
    bits = f32.view(np.uint32)
    lsb = (bits >> 16) & np.uint32(1)
    rounded = (bits + np.uint32(0x7FFF) + lsb) >> 16
    nan = np.isnan(f32)
    out = rounded.astype(np.uint16)
    if nan.any():
        out = np.where(nan, np.uint16(0x7FC0), out)
    return out


def from_bf16_bits(bits) -> np.ndarray:
    """Widen ``uint16`` bf16 bits to f32 (exact)."""

    b = np.asarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(values) -> np.ndarray:
    """Round to the nearest bf16 and return it as f32 (the value a bf16 store keeps)."""

    return from_bf16_bits(to_bf16_bits(values))
