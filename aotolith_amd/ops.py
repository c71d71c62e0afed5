"""torch-ROCm front of the C ABI: shape/dtype checks, output allocation, launch.

Every function takes device tensors, checks them against what the kernel and
its grid assume (on the host, before anything is enqueued), allocates the
outputs with torch (Python owns all buffers), and enqueues the kernel on the
current stream. No function here computes anything on the CPU.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

BF16 = torch.bfloat16


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(tensor: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())


def _expect(tensor: torch.Tensor, name: str, dtype: torch.dtype, shape: tuple[int, ...] | None = None) -> None:
    if not isinstance(tensor, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(tensor).__name__}")
    if tensor.device.type != "cuda":
        raise ValueError(f"{name} must be on the GPU, got {tensor.device}")
    if tensor.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {tensor.dtype}")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(tensor.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(tensor.shape)}")


def _ready(tensor: torch.Tensor) -> None:
    _lib.ensure_code_object(tensor.device.index)


def w4_quantize(weight: torch.Tensor, group_size: int = 64) -> tuple[torch.Tensor, torch.Tensor]:
    """Pack a ``[out, in]`` bf16/f32 weight: ``(int32 [out, in/8], bf16 scales [out, in/group])``.

    Bit-exact with the reference packer (``quantize.py:95-152``,
    ``models/quantized.py:133-163``).
    """

    if weight.dim() != 2:
        raise ValueError(f"a quantized weight must be 2-D, got {tuple(weight.shape)}")
    if weight.dtype not in (BF16, torch.float32):
        raise TypeError(f"weight must be bf16 or f32, got {weight.dtype}")
    _expect(weight, "weight", weight.dtype)
    rows, inner = weight.shape
    if group_size <= 0 or group_size % 8 or inner % group_size:
        raise ValueError(f"group size {group_size} must be a positive multiple of 8 dividing {inner}")
    _ready(weight)
    packed = torch.empty((rows, inner // 8), dtype=torch.int32, device=weight.device)
    scales = torch.empty((rows, inner // group_size), dtype=BF16, device=weight.device)
    _lib.check(
        _lib.library().aoto_hip_w4_quantize(
            _ptr(weight), int(weight.dtype == torch.float32), rows, inner, group_size,
            _ptr(packed), _ptr(scales), None, _stream(),
        )
    )
    return packed, scales


def w4_dequantize(packed: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """``bf16(code * scale)`` ``[out, in]`` (``models/quantized.py:61-82``)."""

    _expect(packed, "packed", torch.int32)
    if packed.dim() != 2:
        raise ValueError("packed must be 2-D")
    rows, words = packed.shape
    inner = words * 8
    _expect(scales, "scales", BF16, (rows, inner // group_size))
    _ready(packed)
    out = torch.empty((rows, inner), dtype=BF16, device=packed.device)
    _lib.check(
        _lib.library().aoto_hip_w4_dequantize(
            _ptr(packed), _ptr(scales), rows, inner, group_size, _ptr(out), _stream()
        )
    )
    return out


def w4_gemv(
    x: torch.Tensor,
    packed: torch.Tensor,
    scales: torch.Tensor,
    group_size: int,
    *,
    norm_weight: torch.Tensor | None = None,
    eps: float = 1e-6,
    bias: torch.Tensor | None = None,
    alpha: float = 1.0,
    beta: float = 1.0,
    up: tuple[torch.Tensor, torch.Tensor] | None = None,
    out: torch.Tensor | None = None,
    lanes_per_row: int = 0,
) -> torch.Tensor:
    """Decode GEMV ``y[N] = W4[N, K] @ x[K]`` with the fused prologue/epilogues.

    ``norm_weight``: RMSNorm prologue; ``bias``: addmm epilogue
    ``bf16(beta * bias + alpha * acc)``; ``up``: ``(packed, scales)`` of the up
    projection for the paired ``silu_mul`` epilogue (``packed`` is then gate).
    """

    _expect(packed, "packed", torch.int32)
    if packed.dim() != 2:
        raise ValueError("packed must be 2-D [N, K/8]")
    n, words = packed.shape
    k = words * 8
    if x.numel() != k:
        raise ValueError(f"x has {x.numel()} elements, the weight reduces over {k}")
    _expect(x, "x", BF16)
    if group_size <= 0 or k % group_size:
        raise ValueError(f"group size {group_size} does not divide K={k}")
    _expect(scales, "scales", BF16, (n, k // group_size))
    up_packed = up_scales = None
    if up is not None:
        up_packed, up_scales = up
        _expect(up_packed, "up packed", torch.int32, (n, words))
        _expect(up_scales, "up scales", BF16, (n, k // group_size))
    if norm_weight is not None:
        _expect(norm_weight, "norm_weight", BF16)
        if norm_weight.numel() != k:
            raise ValueError(f"norm_weight has {norm_weight.numel()} elements, expected {k}")
    if bias is not None:
        _expect(bias, "bias", BF16)
        if bias.numel() != n:
            raise ValueError(f"bias has {bias.numel()} elements, expected {n}")
    if out is None:
        out = torch.empty((n,), dtype=BF16, device=x.device)
    else:
        _expect(out, "out", BF16)
        if out.numel() != n:
            raise ValueError(f"out has {out.numel()} elements, expected {n}")
    _ready(x)
    _lib.check(
        _lib.library().aoto_hip_w4_gemv(
            _ptr(x), _ptr(packed), _ptr(scales), _ptr(up_packed), _ptr(up_scales), _ptr(norm_weight),
            float(eps), _ptr(bias), float(alpha), float(beta), _ptr(out), k, n, group_size,
            int(lanes_per_row), _stream(),
        )
    )
    return out
