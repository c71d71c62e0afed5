"""GPU parity of the eight-bit (``quantize_bits=8``) pack, unpack, decode GEMV and prefill GEMM.

The int8 format is the reference's ``quantize_int8`` / ``pack_weight_int8``
(quantize.py:155-172, models/quantized.py:166-172): four codes per int32 word,
scale max|w|/127. Pack and unpack are bit-exact with the oracle; the GEMV and
GEMM land within the north-star bars and one bf16 ulp (two for the silu_mul
epilogues), as the four-bit kernels do. The reference's own test of both code
widths at the ends of the code range
(tests/test_quantized_matmul.py:75-120) has its counterpart in the extreme-code
cases here, and its paired gate/up test (:123-170) in the paired cases.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ops as oracle
from oracle.bf16 import round_bf16
from oracle.quant import dequantize_bits_bf16, pack_weight_bits_bf16
from tests.helpers import assert_bf16_parity, bf16_bits_of, bf16_normal, from_gpu_bf16, to_gpu_bf16, to_gpu_bits

pytestmark = pytest.mark.gpu


def _ops():
    from aotolith_amd import ops

    return ops


def _packed(rng, n, k, group=64, std=0.02):
    weight = bf16_normal(rng, (n, k), std)
    return pack_weight_bits_bf16(weight, group, 8)


def _gpu(packed, scales):
    return torch.from_numpy(packed).cuda(), to_gpu_bits(scales)


@pytest.mark.parametrize("n,k,group", [(1152, 896, 64), (896, 4864, 64), (37, 256, 32), (5, 64, 4), (3, 512, 128)])
@pytest.mark.parametrize("source", ["bf16", "f32"])
def test_w8_quantize_is_bit_exact(n, k, group, source):
    rng = np.random.default_rng(n * 11 + k + group)
    if source == "f32":
        weight = rng.standard_normal((n, k)).astype(np.float32) * np.float32(0.02)
        weight[0, :group] = 0.0  # an all-zero group takes scale 1/127
        tensor = torch.from_numpy(weight).cuda()
    else:
        weight = bf16_normal(rng, (n, k), 0.02)
        weight[0, :group] = 0.0
        tensor = to_gpu_bf16(weight)
    packed, scales = _ops().w8_quantize(tensor, group)
    ref_packed, ref_scales = pack_weight_bits_bf16(weight, group, 8)
    assert tuple(packed.shape) == (n, k // 4)
    np.testing.assert_array_equal(packed.cpu().numpy(), ref_packed)
    np.testing.assert_array_equal(bf16_bits_of(scales), ref_scales)


@pytest.mark.parametrize("n,k,group", [(300, 896, 64), (37, 96, 8), (5, 20, 4)])
def test_w8_dequantize_is_bit_exact(n, k, group):
    rng = np.random.default_rng(6 + group)
    packed, scales = _packed(rng, n, k, group)
    out = _ops().w8_dequantize(*_gpu(packed, scales), group)
    np.testing.assert_array_equal(from_gpu_bf16(out), dequantize_bits_bf16(packed, scales, group, 8))


def _extreme_case(n, k, group):
    """Every group holds +127 and -127 and every row's first word -128, 127, 1, -1."""

    weight = np.zeros((n, k), dtype=np.float32)
    weight[:, 0::2] = 3.0
    weight[:, 1::2] = -3.0
    packed, scales = pack_weight_bits_bf16(weight, group, 8)
    word = (0x80) | (0x7F << 8) | (0x01 << 16) | (0xFF << 24)
    packed[:, 0] = np.int64(word).astype(np.uint32).astype(np.int32)
    return packed, scales


def test_w8_extreme_codes_unpack_gemv_and_gemm():
    rng = np.random.default_rng(79)
    n, k, group = 64, 128, 32
    packed, scales = _extreme_case(n, k, group)
    out = _ops().w8_dequantize(*_gpu(packed, scales), group)
    np.testing.assert_array_equal(from_gpu_bf16(out), dequantize_bits_bf16(packed, scales, group, 8))
    x = bf16_normal(rng, (k,))
    y = _ops().w8_gemv(to_gpu_bf16(x), *_gpu(packed, scales), group)
    assert_bf16_parity(from_gpu_bf16(y), oracle.w4_gemv(x, packed, scales, group, bits=8))
    xm = bf16_normal(rng, (16, k))
    ym = _ops().w8_matmul(to_gpu_bf16(xm), *_gpu(packed, scales), group)
    assert_bf16_parity(from_gpu_bf16(ym), oracle.w4_matmul(xm, packed, scales, group, bits=8), max_ulp=1.0)


GEMV_SHAPES = [
    (4864, 896),    # Qwen gate / up (4 rows per wave, one chunk per lane)
    (151936 // 8, 896),  # an eighth of the Qwen LM head
    (1152, 896),    # Qwen packed q/k/v
    (896, 4864),    # Qwen down (4 chunks per lane, two passes)
    (1000, 1536),   # 2 rows x 2 chunks form
    (4096, 14336),  # Llama-8B down projection
    (6144, 4096),   # Llama-8B q/k/v
    (3, 64),        # fewer rows than a wave's share, tiny K
    (1, 16),        # a single row, the smallest K
]


@pytest.mark.parametrize("n,k", GEMV_SHAPES)
@pytest.mark.parametrize("variant", ["plain", "norm_bias", "paired"])
def test_w8_gemv(n, k, variant):
    rng = np.random.default_rng(n + 3 * k + len(variant))
    group = 64 if k % 64 == 0 else 16
    packed, scales = _packed(rng, n, k, group)
    x = bf16_normal(rng, (k,))
    kwargs, gpu_kwargs = {}, {}
    if variant == "norm_bias":
        norm = round_bf16(np.float32(1.0) + bf16_normal(rng, (k,), 0.2))
        bias = bf16_normal(rng, (n,), 0.5)
        kwargs = {"norm_weight": norm, "eps": 1e-6, "bias": bias}
        gpu_kwargs = {"norm_weight": to_gpu_bf16(norm), "eps": 1e-6, "bias": to_gpu_bf16(bias)}
    elif variant == "paired":
        up, up_s = _packed(rng, n, k, group)
        kwargs = {"up_packed": up, "up_scales_bits": up_s}
        gpu_kwargs = {"up": _gpu(up, up_s)}
    y = _ops().w8_gemv(to_gpu_bf16(x), *_gpu(packed, scales), group, **gpu_kwargs)
    expected = oracle.w4_gemv(x, packed, scales, group, bits=8, **kwargs)
    atol = 2e-2 * max(1.0, float(np.abs(expected).max()) / 4)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=2.0 if variant == "paired" else 1.0, atol=atol)


def test_w8_gemv_in_place_residual():
    """The decoder's o/down projections add into the buffer they overwrite."""

    rng = np.random.default_rng(12)
    n, k = 896, 4864
    packed, scales = _packed(rng, n, k)
    x = bf16_normal(rng, (k,))
    residual = bf16_normal(rng, (n,), 2.0)
    buf = to_gpu_bf16(residual)
    _ops().w8_gemv(to_gpu_bf16(x), *_gpu(packed, scales), 64, bias=buf, out=buf)
    expected = oracle.w4_gemv(x, packed, scales, 64, bias=residual, bits=8)
    assert_bf16_parity(from_gpu_bf16(buf), expected, atol=2e-2 * max(1.0, float(np.abs(expected).max()) / 4))


def test_w8_gemv_rejects_unsupported_group():
    from aotolith_amd._lib import UnsupportedShape

    rng = np.random.default_rng(2)
    packed, scales = _packed(rng, 8, 64, 8)
    with pytest.raises(UnsupportedShape):
        _ops().w8_gemv(to_gpu_bf16(bf16_normal(rng, (64,))), *_gpu(packed, scales), 8)


GEMM_CASES = [
    (128, 4864, 896, 64),   # Qwen gate / up at the prefill length
    (128, 896, 4864, 64),   # Qwen down
    (16, 1152, 896, 32),    # M = 16, group 32
    (1, 896, 896, 64),      # a single row
    (300, 2048, 512, 128),  # several m blocks, group 128
]


@pytest.mark.parametrize("m,n,k,group", GEMM_CASES)
@pytest.mark.parametrize("tile", [0, 12, 28])
def test_w8_matmul_plain(m, n, k, group, tile):
    rng = np.random.default_rng(m + n + k + tile + 8)
    packed, scales = _packed(rng, n, k, group)
    x = bf16_normal(rng, (m, k))
    y = _ops().w8_matmul(to_gpu_bf16(x), *_gpu(packed, scales), group, tile=tile)
    expected = oracle.w4_matmul(x, packed, scales, group, bits=8)
    atol = 2e-2 * max(1.0, float(np.abs(expected).max()) / 4)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=1.0, atol=atol)


@pytest.mark.parametrize("epilogue", ["bias", "residual", "gate"])
@pytest.mark.parametrize("splits", [1, 4])
def test_w8_matmul_epilogues(epilogue, splits):
    rng = np.random.default_rng({"bias": 21, "residual": 22, "gate": 23}[epilogue] + splits)
    m, n, k = 96, 1152 if epilogue == "bias" else 896, 896
    packed, scales = _packed(rng, n, k)
    x = bf16_normal(rng, (m, k))
    kwargs = {}
    if epilogue == "bias":
        kwargs["bias"] = bf16_normal(rng, (n,), 0.5)
    elif epilogue == "residual":
        kwargs["residual"] = bf16_normal(rng, (m, n), 2.0)
    else:
        kwargs["gate"] = bf16_normal(rng, (m, n))
    gpu_kwargs = {key: to_gpu_bf16(value) for key, value in kwargs.items()}
    y = _ops().w8_matmul(to_gpu_bf16(x), *_gpu(packed, scales), 64, splits=splits, **gpu_kwargs)
    expected = oracle.w4_matmul(x, packed, scales, 64, bits=8, **kwargs)
    atol = 2e-2 * max(1.0, float(np.abs(expected).max()) / 4)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=2.0 if epilogue == "gate" else 1.0, atol=atol)
