"""Write ``quantize_kats.json``: known-answer vectors for the int4 and int8 formats.

The vectors come from the reference's own known-answer tests and from the format
definition worked by hand in pure Python integers - nothing here calls the
oracle, so the oracle can be checked against them:

* ``tests/test_quantize.py:66-74`` (reference): codes ``[1..7, -8]`` pack to the
  word with nibble ``k`` at bits ``4k``;
* ``tests/test_quantize.py:77-83``: the row ``[-1, -0.5, 0, 0.5, 1, 1.5, -1.5,
  0.25]`` at group 8 (scale ``1.5 / 7``); its codes are worked out below from
  ``rint(w * 7 / 1.5)``;
* half-to-even rounding at scale 1 (``quantize.py:119-121`` uses ``np.rint``);
* an all-zero group (``tests/test_quantize.py:103-107``): scale ``1 / 7``,
  codes 0;
* int8 (``"bits": 8``): byte order ``[-128, -1, 0, 127]`` with byte ``k`` at
  bits ``8k`` (``tests/test_quantize.py:194-202``), a row at group 8 with scale
  ``max|w| / 127`` (``:217-223``), half-to-even at scale 1 and an all-zero group
  (scale ``1 / 127``).

Run ``python tests/golden/make_kats.py`` to regenerate.
"""

from __future__ import annotations

import json
import os
import struct
from fractions import Fraction


def pack_word(codes: list[int]) -> int:
    """Pack eight signed codes into a signed 32-bit word, nibble k at bits 4k."""

    word = 0
    for position, code in enumerate(codes):
        word |= (code & 0xF) << (4 * position)
    return word - (1 << 32) if word >= 1 << 31 else word


def pack_word8(codes: list[int]) -> int:
    """Pack four signed byte codes into a signed 32-bit word, byte k at bits 8k."""

    word = 0
    for position, code in enumerate(codes):
        word |= (code & 0xFF) << (8 * position)
    return word - (1 << 32) if word >= 1 << 31 else word


def rint_half_even(value: Fraction) -> int:
    floor = value.numerator // value.denominator
    rest = value - floor
    if rest > Fraction(1, 2):
        return floor + 1
    if rest < Fraction(1, 2):
        return floor
    return floor if floor % 2 == 0 else floor + 1


def f32(value: float) -> float:
    return struct.unpack("<f", struct.pack("<f", value))[0]


def main() -> None:
    cases = []

    codes = [1, 2, 3, 4, 5, 6, 7, -8]
    cases.append({"name": "nibble_order", "codes": codes, "word": pack_word(codes)})

    row = [-1.0, -0.5, 0.0, 0.5, 1.0, 1.5, -1.5, 0.25]
    # scale = 1.5 / 7; w / scale = w * 7 / 1.5 exactly in rationals. The f32
    # division the quantizer performs lands on the same side of every .5 here
    # (the nearest ties are 7/3-ish values), so the rational rint is the answer.
    scale = Fraction(3, 2) / 7
    row_codes = [max(-8, min(7, rint_half_even(Fraction(w) / scale))) for w in row]
    cases.append(
        {
            "name": "negative_codes",
            "weight": row,
            "group_size": 8,
            "codes": row_codes,
            "word": pack_word(row_codes),
            "scale_f32": f32(1.5 / 7.0),
        }
    )

    ties = [7.0, 3.5, 2.5, 0.5, -0.5, -2.5, 1.5, -1.5]
    tie_codes = [rint_half_even(Fraction(w)) for w in ties]
    cases.append(
        {
            "name": "half_to_even",
            "weight": ties,
            "group_size": 8,
            "codes": tie_codes,
            "word": pack_word(tie_codes),
            "scale_f32": 1.0,
        }
    )

    cases.append(
        {
            "name": "zero_group",
            "weight": [0.0] * 16,
            "group_size": 16,
            "codes": [0] * 16,
            "word": 0,
            "scale_f32": f32(1.0 / 7.0),
        }
    )

    codes8 = [-128, -1, 0, 127]
    cases.append({"name": "int8_byte_order", "bits": 8, "codes": codes8, "word": pack_word8(codes8)})

    row8 = [-1.0, -0.5, 0.0, 0.5, 1.0, 1.5, -1.5, 0.25]
    scale8 = Fraction(3, 2) / 127
    row8_codes = [max(-128, min(127, rint_half_even(Fraction(w) / scale8))) for w in row8]
    cases.append(
        {
            "name": "int8_group_scale",
            "bits": 8,
            "weight": row8,
            "group_size": 8,
            "codes": row8_codes,
            "words": [pack_word8(row8_codes[:4]), pack_word8(row8_codes[4:])],
            "scale_f32": f32(1.5 / 127.0),
        }
    )

    ties8 = [100.5, 3.5, 2.5, 0.5, -0.5, -2.5, 127.0, -127.0]
    tie8_codes = [rint_half_even(Fraction(w)) for w in ties8]
    # with max |w| = 127 the scale is exactly 1
    cases.append(
        {
            "name": "int8_half_to_even",
            "bits": 8,
            "weight": ties8,
            "group_size": 8,
            "codes": tie8_codes,
            "words": [pack_word8(tie8_codes[:4]), pack_word8(tie8_codes[4:])],
            "scale_f32": 1.0,
        }
    )

    cases.append(
        {
            "name": "int8_zero_group",
            "bits": 8,
            "weight": [0.0] * 8,
            "group_size": 8,
            "codes": [0] * 8,
            "words": [0, 0],
            "scale_f32": f32(1.0 / 127.0),
        }
    )

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "quantize_kats.json")
    with open(path, "w") as handle:
        json.dump({"source": "reference tests/test_quantize.py + format definition", "cases": cases}, handle, indent=1)
        handle.write("\n")


if __name__ == "__main__":
    main()
