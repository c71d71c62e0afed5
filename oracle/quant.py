"""Oracle for the symmetric int4 / int8 group quantizers, packers and unpacks.

Restates ``quantize.py:64-268`` and ``models/quantized.py:61-172`` of the
reference. The int4 format (int8 differs only where noted):

* a weight is ``[out, in]``; the reduction axis is cut into groups of
  ``group_size`` columns sharing one scale;
* ``scale = max|w| / 7`` in f32, an all-zero group takes ``1 / 7``;
* ``code = clip(rint(w / scale), -8, 7)``, f32 division, round half to even;
* eight codes per ``int32`` word, code ``8j + k`` at bits ``4k`` of word ``j``;
* the stored scale is ``scale`` rounded to the weight dtype (bf16, RNE), while
  the codes come from the f32 scale (``models/quantized.py:149-163``).

int8 (``quantize_int8``, ``quantize.py:155-172``): ``scale = max|w| / 127``
(all-zero group ``1 / 127``), ``code = clip(rint(w / scale), -128, 127)``, four
codes per word, code ``4j + k`` at bits ``8k`` of word ``j``; the group size
must be a multiple of 4 (``check_group_size(..., 4)``).
"""

from __future__ import annotations

import numpy as np

from .bf16 import from_bf16_bits, round_bf16, to_bf16_bits

INT4_MIN = -8
INT4_MAX = 7
INT4_MAGNITUDE = 7
NIBBLES_PER_WORD = 8
INT8_MIN = -128
INT8_MAGNITUDE = 127
BYTES_PER_WORD = 4


def check_group_size(group_size: int, inner: int, packed_width: int = NIBBLES_PER_WORD) -> int:
    """Validate a group size (``quantize.py:64-92``)."""

    if group_size <= 0:
        raise ValueError(f"quantization group size must be positive, got {group_size}")
    if group_size % packed_width != 0:
        raise ValueError(
            f"quantization group size must be a multiple of {packed_width}, got {group_size}"
        )
    if inner % group_size != 0:
        raise ValueError(
            f"quantization group size {group_size} does not divide the reduction length {inner}"
        )
    return group_size


def _quantize(weight, group_size: int, per_word: int, lowest: int, magnitude: int, shift: int):
    """Group scales, round half to even, clip, pack (``quantize.py:95-132``, shared by both widths)."""

    matrix = np.asarray(weight, dtype=np.float32)
    if matrix.ndim != 2:
        raise ValueError(f"quantization expects a 2-D weight, got {matrix.shape}")
    rows, inner = matrix.shape
    check_group_size(group_size, inner, per_word)
    groups = inner // group_size
    blocks = matrix.reshape(rows, groups, group_size)
    widest = np.abs(blocks).max(axis=-1)
    scale = (np.where(widest > np.float32(0.0), widest, np.float32(1.0)) / np.float32(magnitude)).astype(np.float32)
    codes = np.clip(np.rint(blocks / scale[:, :, None]), lowest, magnitude)
    codes = codes.astype(np.int32).reshape(rows, inner)
    packed = np.zeros((rows, inner // per_word), dtype=np.int32)
    mask = (1 << shift) - 1
    for position in range(per_word):
        field = (codes[:, position::per_word] & mask).astype(np.int64)
        packed |= (field << (shift * position)).astype(np.uint32).astype(np.int32)
    return packed, scale


def quantize_int4(weight, group_size: int = 64) -> tuple[np.ndarray, np.ndarray]:
    """``(packed int32 [out, in/8], scales f32 [out, in/group])`` (``quantize.py:95-152``)."""

    return _quantize(weight, group_size, NIBBLES_PER_WORD, INT4_MIN, INT4_MAGNITUDE, 4)


def quantize_int8(weight, group_size: int = 64) -> tuple[np.ndarray, np.ndarray]:
    """``(packed int32 [out, in/4], scales f32 [out, in/group])`` (``quantize.py:155-172``)."""

    return _quantize(weight, group_size, BYTES_PER_WORD, INT8_MIN, INT8_MAGNITUDE, 8)


def unpack_codes(packed) -> np.ndarray:
    """Signed codes ``int8 [out, in]`` from packed words (``quantize.py:175-187``)."""

    words = np.asarray(packed).astype(np.int64)
    rows, count = words.shape
    codes = np.empty((rows, count * NIBBLES_PER_WORD), dtype=np.int8)
    for nibble in range(NIBBLES_PER_WORD):
        field = ((words >> (4 * nibble)) & 0xF).astype(np.int8)
        codes[:, nibble::NIBBLES_PER_WORD] = np.where(field >= 8, field - 16, field)
    return codes


def unpack_codes_int8(packed) -> np.ndarray:
    """Signed codes ``int8 [out, in]`` from eight-bit packed words (``quantize.py:190-202``)."""

    words = np.asarray(packed).astype(np.int64)
    rows, count = words.shape
    codes = np.empty((rows, count * BYTES_PER_WORD), dtype=np.int8)
    for byte in range(BYTES_PER_WORD):
        field = ((words >> (8 * byte)) & 0xFF).astype(np.int16)
        codes[:, byte::BYTES_PER_WORD] = np.where(field >= 128, field - 256, field).astype(np.int8)
    return codes


def dequantize_int8(packed, scales, group_size: int) -> np.ndarray:
    """f32 weights ``code * scale`` of an eight-bit pack (``quantize.py:237-248``)."""

    codes = unpack_codes_int8(packed)
    return codes.astype(np.float32) * np.repeat(np.asarray(scales, dtype=np.float32), group_size, axis=-1)


def codes_of(packed, bits: int) -> np.ndarray:
    """Signed codes of a four- or eight-bit pack."""

    if bits == 4:
        return unpack_codes(packed)
    if bits == 8:
        return unpack_codes_int8(packed)
    raise ValueError(f"bits must be 4 or 8, got {bits}")


def dequantize_int4(packed, scales, group_size: int) -> np.ndarray:
    """f32 weights ``code * scale`` (``quantize.py:201-213``)."""

    codes = unpack_codes(packed)
    return codes.astype(np.float32) * np.repeat(np.asarray(scales, dtype=np.float32), group_size, axis=-1)


def pack_weight_bf16(weight, group_size: int = 64) -> tuple[np.ndarray, np.ndarray]:
    """Pack a weight held in bf16 and store bf16 scales (``models/quantized.py:133-163``).

    ``weight`` is f32 values that are already bf16-representable (the model's
    parameters widened), or ``uint16`` bf16 bits. Returns ``(packed int32,
    scales uint16 bf16 bits)``.
    """

    return pack_weight_bits_bf16(weight, group_size, 4)


def pack_weight_bits_bf16(weight, group_size: int = 64, bits: int = 4) -> tuple[np.ndarray, np.ndarray]:
    """``pack_weight_bf16`` for either width (``models/quantized.py:133-172``)."""

    w = np.asarray(weight)
    if w.dtype == np.uint16:
        w = from_bf16_bits(w)
    quantizer = {4: quantize_int4, 8: quantize_int8}[bits]
    packed, scales = quantizer(w.astype(np.float32), group_size)
    return packed, to_bf16_bits(scales)


def dequantize_i4_bf16(packed, scales_bf16_bits, group_size: int) -> np.ndarray:
    """The torch op in the scales' dtype: ``bf16(code * scale_bf16)`` as f32.

    ``models/quantized.py:61-76``: codes are cast to the scale dtype (exact for
    -8..7) and multiplied in bf16, so each weight is the product rounded once.
    """

    return dequantize_bits_bf16(packed, scales_bf16_bits, group_size, 4)


def dequantize_bits_bf16(packed, scales_bf16_bits, group_size: int, bits: int = 4) -> np.ndarray:
    """``bf16(code * scale_bf16)`` for either width (``models/quantized.py:61-107``)."""

    codes = codes_of(packed, bits).astype(np.float32)
    scales = from_bf16_bits(scales_bf16_bits)
    return round_bf16(codes * np.repeat(scales, group_size, axis=-1))


def dequantize_i4_exact(packed, scales_bf16_bits, group_size: int) -> np.ndarray:
    """``code * scale_bf16`` without a rounding step (exact in f32: 4 x 8 bits).

    This is the weight the decode GEMV multiplies by: it never materializes a
    rounded weight and accumulates ``code * (x * scale)`` in f32
    (``codegen/matmul.py:696-704``); ``x * scale`` of two bf16 values is exact in
    f32, so every product is exact and only the summation rounds.
    """

    return dequantize_bits_exact(packed, scales_bf16_bits, group_size, 4)


def dequantize_bits_exact(packed, scales_bf16_bits, group_size: int, bits: int = 4) -> np.ndarray:
    """``code * scale_bf16`` for either width; exact in f32 (at most 8 x 8 bits)."""

    codes = codes_of(packed, bits).astype(np.float32)
    scales = from_bf16_bits(scales_bf16_bits)
    return codes * np.repeat(scales, group_size, axis=-1)
