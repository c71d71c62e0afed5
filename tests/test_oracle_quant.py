"""Pin the int4 oracle: known answers, closed forms, round trips, torch cross-check.

The intent of the reference's ``tests/test_quantize.py`` (nibble order, negative
codes, scale closed form, zero group, error bound, group validation) plus the
checks that fix what those leave open: half-to-even rounding, the bf16 RNE cast
against torch's, the bf16 dequant against torch's bf16 multiply.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from oracle.bf16 import from_bf16_bits, round_bf16, to_bf16_bits
from oracle.quant import (
    check_group_size,
    dequantize_i4_bf16,
    dequantize_i4_exact,
    dequantize_int4,
    pack_weight_bf16,
    quantize_int4,
    unpack_codes,
)

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quantize_kats.json")


def _cases() -> dict:
    with open(GOLDEN) as handle:
        return {case["name"]: case for case in json.load(handle)["cases"]}


def _weight(rows: int, inner: int, seed: int = 0) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal((rows, inner)).astype(np.float32)


def test_nibble_order_known_answer() -> None:
    case = _cases()["nibble_order"]
    packed = np.array([[case["word"]]], dtype=np.int32)
    np.testing.assert_array_equal(unpack_codes(packed), np.array([case["codes"]], dtype=np.int8))


@pytest.mark.parametrize("name", ["negative_codes", "half_to_even", "zero_group"])
def test_pack_known_answers(name: str) -> None:
    case = _cases()[name]
    weight = np.array([case["weight"]], dtype=np.float32)
    packed, scales = quantize_int4(weight, case["group_size"])
    np.testing.assert_array_equal(unpack_codes(packed)[0], np.array(case["codes"], dtype=np.int8))
    assert int(packed[0, 0]) == case["word"]
    assert scales.dtype == np.float32
    assert float(scales[0, 0]) == case["scale_f32"]


def test_packed_shape_is_an_eighth_of_the_codes() -> None:
    packed, scales = quantize_int4(_weight(8, 32), 32)
    assert packed.dtype == np.int32 and packed.shape == (8, 4)
    assert scales.shape == (8, 1)


def test_scale_closed_form() -> None:
    weight = _weight(2, 64, seed=3)
    weight[0, :32] *= 7.0
    _, scales = quantize_int4(weight, 32)
    assert scales[0, 0] == np.float32(np.abs(weight[0, :32]).max()) / np.float32(7.0)
    assert scales[0, 1] == np.float32(np.abs(weight[0, 32:]).max()) / np.float32(7.0)


def test_codes_are_rint_of_the_f32_quotient() -> None:
    weight = _weight(16, 128, seed=9)
    packed, scales = quantize_int4(weight, 64)
    expected = np.clip(
        np.rint(weight.reshape(16, 2, 64) / scales[:, :, None]), -8, 7
    ).reshape(16, 128)
    np.testing.assert_array_equal(unpack_codes(packed), expected.astype(np.int8))
    # The symmetric quantizer never produces the spare code.
    assert int(unpack_codes(packed).min()) >= -7


def test_error_bounded_by_half_the_scale() -> None:
    weight = _weight(32, 128, seed=4)
    packed, scales = quantize_int4(weight, 32)
    restored = dequantize_int4(packed, scales, 32)
    bound = np.repeat(scales, 32, axis=1) / 2 + 1e-6
    assert np.all(np.abs(restored - weight) <= bound)


def test_round_trip_and_idempotence() -> None:
    weight = _weight(64, 256, seed=5)
    packed, scales = quantize_int4(weight, 64)
    np.testing.assert_array_equal(unpack_codes(packed), unpack_codes(unpack_codes_to_words(unpack_codes(packed))))
    again, _ = quantize_int4(dequantize_int4(packed, scales, 64), 64)
    np.testing.assert_array_equal(again, packed)


def unpack_codes_to_words(codes: np.ndarray) -> np.ndarray:
    """Independent re-pack in Python integers (row by row) for the round trip."""

    rows, inner = codes.shape
    out = np.zeros((rows, inner // 8), dtype=np.int32)
    for r in range(rows):
        for j in range(inner // 8):
            word = 0
            for k in range(8):
                word |= (int(codes[r, 8 * j + k]) & 0xF) << (4 * k)
            out[r, j] = word - (1 << 32) if word >= 1 << 31 else word
    return out


@pytest.mark.parametrize("group_size", [0, -8, 3, 12])
def test_rejects_group_sizes_that_do_not_cover_whole_words(group_size: int) -> None:
    with pytest.raises(ValueError):
        check_group_size(group_size, 32)


def test_rejects_a_group_that_does_not_divide_the_reduction() -> None:
    with pytest.raises(ValueError):
        check_group_size(48, 32)
    with pytest.raises(ValueError):
        quantize_int4(_weight(2, 12), 4)


def test_bf16_rne_matches_torch() -> None:
    rng = np.random.default_rng(11)
    values = np.concatenate(
        [
            rng.standard_normal(20000).astype(np.float32) * np.float32(3.0),
            rng.standard_normal(2000).astype(np.float32) * np.float32(1e-30),
            np.array([0.0, -0.0, 1.0, 65504.0, 3.0e38, -3.0e38], dtype=np.float32),
            # exact ties: bf16 value + half an ulp
            (from_bf16_bits(np.arange(0x3F80, 0x3F90, dtype=np.uint16)).view(np.uint32) + 0x8000).view(np.float32),
        ]
    )
    expected = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(to_bf16_bits(values), expected)


def test_dequant_exhaustive_codes_against_torch_bf16_multiply() -> None:
    """All 16 codes x many bf16 scales: ``bf16(code * s)`` as torch computes it."""

    rng = np.random.default_rng(12)
    scales = to_bf16_bits(np.abs(rng.standard_normal(512)).astype(np.float32) * np.float32(0.01))
    codes = np.arange(-8, 8, dtype=np.int32)
    words = np.zeros((512, 2), dtype=np.int32)
    for j in range(2):
        word = 0
        for k in range(8):
            word |= (int(codes[8 * j + k]) & 0xF) << (4 * k)
        words[:, j] = word - (1 << 32) if word >= 1 << 31 else word
    ours = dequantize_i4_bf16(words, scales[:, None], 16)
    code_t = torch.from_numpy(np.tile(codes, (512, 1))).to(torch.bfloat16)
    scale_t = torch.from_numpy(scales.view(np.int16)).view(torch.bfloat16)[:, None]
    theirs = (code_t * scale_t.repeat_interleave(16, dim=-1)).float().numpy()
    np.testing.assert_array_equal(ours, theirs)
    exact = dequantize_i4_exact(words, scales[:, None], 16)
    np.testing.assert_array_equal(round_bf16(exact), ours)


def test_pack_weight_bf16_scales_are_rne_of_f32_scales() -> None:
    weight = round_bf16(_weight(8, 128, seed=13) * np.float32(0.02))
    packed, scales_bits = pack_weight_bf16(weight, 64)
    ref_packed, ref_scales = quantize_int4(weight, 64)
    np.testing.assert_array_equal(packed, ref_packed)
    torch_scales = torch.from_numpy(ref_scales).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(scales_bits, torch_scales)


# --- eight bits (quantize.py:155-268, models/quantized.py:84-107, 165-172) ---------------


def test_int8_byte_order_known_answer() -> None:
    from oracle.quant import unpack_codes_int8

    case = _cases()["int8_byte_order"]
    packed = np.array([[case["word"]]], dtype=np.int32)
    np.testing.assert_array_equal(unpack_codes_int8(packed), np.array([case["codes"]], dtype=np.int8))


@pytest.mark.parametrize("name", ["int8_group_scale", "int8_half_to_even", "int8_zero_group"])
def test_int8_pack_known_answers(name: str) -> None:
    from oracle.quant import quantize_int8, unpack_codes_int8

    case = _cases()[name]
    weight = np.array([case["weight"]], dtype=np.float32)
    packed, scales = quantize_int8(weight, case["group_size"])
    np.testing.assert_array_equal(unpack_codes_int8(packed)[0], np.array(case["codes"], dtype=np.int8))
    assert [int(w) for w in packed[0]] == case["words"]
    assert float(scales[0, 0]) == case["scale_f32"]


def test_int8_shape_scale_and_error_bound() -> None:
    from oracle.quant import dequantize_int8, quantize_int8

    weight = _weight(16, 64, seed=11)
    weight[0, :32] *= 7.0
    packed, scales = quantize_int8(weight, 32)
    assert packed.dtype == np.int32 and packed.shape == (16, 16) and packed.nbytes * 4 == weight.nbytes
    np.testing.assert_allclose(scales[0, 0], np.abs(weight[0, :32]).max() / np.float32(127.0), rtol=0)
    error = np.abs(dequantize_int8(packed, scales, 32) - weight)
    assert (error <= np.repeat(scales, 32, axis=1) / 2 * (1 + 1e-6)).all()
    # 127 levels instead of 7: the residual is more than 15x smaller (reference test :205-214)
    coarse = np.abs(dequantize_int4(*quantize_int4(weight, 32), 32) - weight).max()
    assert error.max() < coarse / 15


def test_int8_round_trip_and_idempotence() -> None:
    from oracle.quant import dequantize_int8, quantize_int8, unpack_codes_int8

    weight = _weight(8, 128, seed=12)
    packed, scales = quantize_int8(weight, 64)
    codes = unpack_codes_int8(packed)
    assert codes.min() >= -128 and codes.max() <= 127
    again, again_scales = quantize_int8(dequantize_int8(packed, scales, 64), 64)
    np.testing.assert_array_equal(again, packed)


@pytest.mark.parametrize("group_size", [0, 6, 10])
def test_int8_rejects_groups_that_split_a_word(group_size: int) -> None:
    from oracle.quant import quantize_int8

    with pytest.raises(ValueError):
        quantize_int8(_weight(2, 60), group_size)


def test_int8_unpack_matches_a_torch_shift_and_wrap() -> None:
    """The reference's torch op (models/quantized.py:84-107) restated in torch ops."""

    from oracle.quant import dequantize_bits_bf16, pack_weight_bits_bf16

    weight = round_bf16(_weight(6, 64, seed=13) * np.float32(0.05))
    packed, scales_bits = pack_weight_bits_bf16(weight, 32, 8)
    words = torch.from_numpy(packed).to(torch.int64) & 0xFFFFFFFF
    fields = [((words >> (8 * b)) & 0xFF) for b in range(4)]
    codes = torch.stack([torch.where(f >= 128, f - 256, f) for f in fields], dim=-1).reshape(6, -1)
    scales = torch.from_numpy(from_bf16_bits(scales_bits)).to(torch.bfloat16)
    ref = (codes.to(torch.bfloat16) * scales.repeat_interleave(32, dim=-1)).float().numpy()
    np.testing.assert_array_equal(dequantize_bits_bf16(packed, scales_bits, 32, 8), ref)
