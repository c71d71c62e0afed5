"""Oracle for the fused decoder ops, at the reference kernels' rounding points.

Each function takes and returns f32 arrays whose values are bf16-representable
(the compute dtype of every config on this path) and rounds exactly where the
reference's native kernels round; accumulation is f64, which is the exact sum
the kernels' f32 accumulators approximate. The functions cite the reference's
interpreter semantics (``runtime/mlx_ops``) and the kernel emitters whose
rounding points they keep.
"""

from __future__ import annotations

import numpy as np

from .bf16 import round_bf16
from .quant import dequantize_bits_bf16, dequantize_bits_exact


def _f32(values) -> np.ndarray:
    return np.asarray(values, dtype=np.float32)


def rms_scale(x, eps: float) -> np.ndarray:
    """``rsqrt(mean(x^2) + eps)`` per row in f32 (``codegen/norm.py:45-72``)."""

    x64 = _f32(x).astype(np.float64)
    mean = np.float32((x64 * x64).sum(axis=-1, keepdims=True) / x64.shape[-1])
    return (np.float32(1.0) / np.sqrt(mean + np.float32(eps))).astype(np.float32)


def rms_norm(x, weight, eps: float) -> np.ndarray:
    """Row RMSNorm: ``bf16(x * rsqrt(mean(x^2) + eps) * w)``.

    ``runtime/mlx_ops/normalization.py:73-119``: statistics in f32, the
    normalized value times the weight in f32, one rounding to the output dtype.
    """

    x32 = _f32(x)
    scale = rms_scale(x32, eps)
    return round_bf16((x32 * scale) * _f32(weight))


def w4_gemv(
    x,
    packed,
    scales_bits,
    group_size: int,
    *,
    norm_weight=None,
    eps: float = 1e-6,
    bias=None,
    alpha: float = 1.0,
    beta: float = 1.0,
    up_packed=None,
    up_scales_bits=None,
    bits: int = 4,
) -> np.ndarray:
    """Packed W4 (``bits=8``: W8, ``codegen/matmul.py:742-929``) GEMV with its prologue and
    epilogues, one output row ``[N]``.

    Follows ``codegen/matmul.py:542-739`` (semantics
    ``runtime/mlx_ops/__init__.py:563-619``):

    * optional RMSNorm prologue: ``x' = bf16(ns * x * w)``, ``ns`` from
      ``rms_scale`` (``codegen/matmul.py:677-695``, ``codegen/norm.py:45-72``);
    * ``acc = sum_k code[n,k] * (x[k] * s[n,k/g])`` - every product is exact in
      f32, so the f64 sum here is the value the f32 accumulators round toward;
    * ``addmm`` epilogue ``bf16(beta * bias + alpha * acc)`` (``:588-594``);
    * paired gate/up epilogue: ``g = bf16(acc_gate)``,
      ``out = bf16(acc_up * g / (1 + exp(-g)))`` (``:598-602, 722-729``).
    """

    xv = _f32(x).reshape(-1)
    if norm_weight is not None:
        ns = rms_scale(xv, eps)[0]
        xv = round_bf16((ns * xv) * _f32(norm_weight).reshape(-1))
    weight = dequantize_bits_exact(packed, scales_bits, group_size, bits).astype(np.float64)
    acc = weight @ xv.astype(np.float64)
    if up_packed is not None:
        up = dequantize_bits_exact(up_packed, up_scales_bits, group_size, bits).astype(np.float64)
        acc_up = up @ xv.astype(np.float64)
        gate = round_bf16(np.float32(1.0) * acc.astype(np.float32)).astype(np.float64)
        return round_bf16(acc_up.astype(np.float32).astype(np.float64) * (gate / (1.0 + np.exp(-gate))))
    if bias is not None:
        acc = beta * _f32(bias).reshape(-1).astype(np.float64) + alpha * acc
    return round_bf16(acc)


def w4_matmul(
    x,
    packed,
    scales_bits,
    group_size: int,
    *,
    bias=None,
    residual=None,
    gate=None,
    bits: int = 4,
) -> np.ndarray:
    """Prefill W4 (or W8) matmul ``[M, K] -> [M, N]`` with its fused epilogue.

    The reference keeps the unpack for ``M > 1`` (``passes/quantize.py:58-71``):
    the dequant kernel writes ``bf16(code * scale)`` (``codegen/quantize.py:27-63``,
    ``models/quantized.py:61-76``), then the GEMM accumulates bf16 x bf16 in f32
    and rounds once after the epilogue (``codegen/matmul.py:1443-1471, 1721-1742``):

    * ``bias`` ``[N]`` (packed q/k/v bias): ``bf16(bias + acc)``;
    * ``residual`` ``[M, N]`` (``fuse_residual_epilogue``): ``bf16(res + acc)``;
    * ``gate`` ``[M, N]`` (``fuse_activation_epilogue``, the up projection):
      ``bf16(acc * g / (1 + exp(-g)))`` with ``g`` the stored bf16 gate.
    """

    x64 = _f32(x).astype(np.float64)
    weight = dequantize_bits_bf16(packed, scales_bits, group_size, bits).astype(np.float64)
    acc = x64 @ weight.T
    if bias is not None:
        acc = acc + _f32(bias).astype(np.float64)[None, :]
    if residual is not None:
        acc = acc + _f32(residual).astype(np.float64)
    if gate is not None:
        g = _f32(gate).astype(np.float64)
        acc = acc.astype(np.float32).astype(np.float64) * (g / (1.0 + np.exp(-g)))
    return round_bf16(acc)


def rope_tables(capacity: int, head_dim: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """bf16 cos/sin tables ``[capacity, head_dim]`` (``models/decoder.py:323-334``).

    The angle ``pos / theta^(2i/D)`` is formed in f32, duplicated across the two
    halves, **rounded to bf16 before** ``cos``/``sin``, and the results are
    rounded to bf16 again.
    """

    positions = np.arange(capacity, dtype=np.float32)[:, None]
    exponents = np.arange(0, head_dim, 2, dtype=np.float32)[None, :] / np.float32(head_dim)
    inverse = np.power(np.float32(theta), exponents).astype(np.float32)
    angles = (positions / inverse).astype(np.float32)
    angles = np.concatenate((angles, angles), axis=-1)
    angles = round_bf16(angles).astype(np.float64)
    return round_bf16(np.cos(angles)), round_bf16(np.sin(angles))


def rope(x, cos, sin) -> np.ndarray:
    """``bf16(x * cos + rotate_half(x) * sin)``, one rounding.

    ``runtime/mlx_ops/__init__.py:276-280`` with the rotate-half of
    ``models/decoder.py:213-223``: the first half takes ``-x[d + D/2]``, the
    second ``x[d - D/2]``. ``cos``/``sin`` broadcast against ``x``.
    """

    x64 = _f32(x).astype(np.float64)
    half = x64.shape[-1] // 2
    rotated = np.concatenate((-x64[..., half:], x64[..., :half]), axis=-1)
    return round_bf16(x64 * _f32(cos).astype(np.float64) + rotated * _f32(sin).astype(np.float64))


def rope_kv_cache_append(
    cache,
    row,
    cos,
    sin,
    *,
    layer: int,
    query_heads: int,
    query_start: int,
    key_start: int,
    value_start: int,
) -> tuple[np.ndarray, np.ndarray]:
    """Rotate the step's q and k out of the projection row, roll one layer's window.

    ``runtime/mlx_ops/__init__.py:207-236`` (kernel ``codegen/kv_cache.py:96-215``):
    ``cache`` is ``[L, 2, B, Hkv, cap, D]``, ``row`` the ``[B, W]`` projection
    row, ``cos``/``sin`` the ``[D]`` table rows at the step's position. Returns
    ``q [B, Hq, 1, D]`` and the new pair ``[2, B, Hkv, cap, D]``: the old window
    shifted down one slot with ``(k_rot, v)`` in the last slot.
    """

    cache = _f32(cache)
    row = _f32(row)
    batch, heads, head_dim = cache.shape[2], cache.shape[3], cache.shape[5]

    def take(start: int, count: int) -> np.ndarray:
        return row[:, start : start + count * head_dim].reshape(batch, count, 1, head_dim)

    query = rope(take(query_start, query_heads), cos, sin)
    key = rope(take(key_start, heads), cos, sin)
    value = take(value_start, heads)
    pair = cache[layer]
    new_pair = np.concatenate((pair[:, :, :, 1:, :], np.stack((key, value), axis=0)), axis=3)
    return query, new_pair


def attention(query, key, value, mask=None, scale: float | None = None) -> np.ndarray:
    """GQA softmax attention with a boolean keep-mask, ``[B, Hq, Sq, D]``.

    ``runtime/mlx_ops/attention.py:73-122`` and the decode kernel
    ``codegen/attention.py:447-656``: ``scale = D^-0.5``
    (``legalize/attention.py:146-147``), key/value head ``h // (Hq / Hkv)``,
    mask ``True`` keeps, f32 scores and softmax, a fully masked row yields 0
    (``safe_softmax``), one rounding of the output.
    """

    q = _f32(query).astype(np.float64)
    k = _f32(key).astype(np.float64)
    v = _f32(value).astype(np.float64)
    batch, query_heads, query_len, head_dim = q.shape
    kv_heads, key_len = k.shape[1], k.shape[2]
    if scale is None:
        scale = float(np.float32(head_dim ** -0.5))
    group = query_heads // kv_heads
    if mask is None:
        keep = np.ones((query_len, key_len), dtype=bool)
    else:
        keep = np.broadcast_to(np.asarray(mask, dtype=bool), (batch, query_heads, query_len, key_len))
    out = np.zeros((batch, query_heads, query_len, v.shape[-1]), dtype=np.float64)
    for b in range(batch):
        for h in range(query_heads):
            kv = h // group
            scores = (q[b, h] @ k[b, kv].T) * scale
            m = keep if mask is None else keep[b, h]
            scores = np.where(m, scores, -np.inf)
            row_max = scores.max(axis=-1, keepdims=True)
            finite = np.isfinite(row_max)
            shifted = np.where(finite, scores - np.where(finite, row_max, 0.0), -np.inf)
            p = np.exp(shifted)
            total = p.sum(axis=-1, keepdims=True)
            p = np.where(total > 0, p / np.where(total > 0, total, 1.0), 0.0)
            out[b, h] = p @ v[b, kv]
    return round_bf16(out)


def embedding(weight, ids) -> np.ndarray:
    """Row gather ``weight[ids]`` (``runtime/bounds.py:104-107``)."""

    return _f32(weight)[np.asarray(ids, dtype=np.int64)]


def argmax_first(logits) -> np.ndarray:
    """Greedy token: the first index of the maximum (``models/decoder.py:1069, 1080``)."""

    return np.argmax(_f32(logits), axis=-1).astype(np.int64)


def prefill_mask(length: int, bucket: int) -> np.ndarray:
    """``[1, 1, bucket, bucket]`` keep-mask: causal and not a left pad (``models/decoder.py:226-247``)."""

    query = np.arange(bucket)[:, None]
    key = np.arange(bucket)[None, :]
    return ((key <= query) & (key >= bucket - length))[None, None]


def decode_mask(valid_length: int, capacity: int) -> np.ndarray:
    """``[1, 1, 1, cap]`` keep-mask: the last ``valid_length`` slots (``models/decoder.py:960-979``)."""

    return (np.arange(capacity) >= capacity - valid_length).reshape(1, 1, 1, capacity)
