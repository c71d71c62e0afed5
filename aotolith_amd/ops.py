"""torch-ROCm front of the C ABI: shape/dtype checks, output allocation, launch.

Every function takes device tensors, checks them against what the kernel and
its grid assume (on the host, before anything is enqueued), allocates the
outputs with torch (Python owns all buffers), and enqueues the kernel on the
current stream. No function here computes anything on the CPU.
"""

from __future__ import annotations

import contextlib
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


#: codes per packed int32 word of each width
CODES_PER_WORD = {4: 8, 8: 4}


def take_launches() -> list[str]:
    """Kernel symbols this thread launched since the last call, while :func:`recording_launches`
    is active (``aoto_hip_take_launches``)."""

    lib = _lib.library()
    size = int(lib.aoto_hip_take_launches(None, 0))
    if size == 0:
        return []
    buf = ctypes.create_string_buffer(size + 1)
    lib.aoto_hip_take_launches(buf, size + 1)
    return buf.value.decode().split()


@contextlib.contextmanager
def recording_launches():
    """Record the kernel symbols this thread launches (read them with :func:`take_launches`)."""

    lib = _lib.library()
    previous = int(lib.aoto_hip_trace_launches(1))
    try:
        yield take_launches
    finally:
        if not previous:
            take_launches()
        lib.aoto_hip_trace_launches(previous)


def _quantize(weight: torch.Tensor, group_size: int, bits: int) -> tuple[torch.Tensor, torch.Tensor]:
    per_word = CODES_PER_WORD[bits]
    if weight.dim() != 2:
        raise ValueError(f"a quantized weight must be 2-D, got {tuple(weight.shape)}")
    if weight.dtype not in (BF16, torch.float32):
        raise TypeError(f"weight must be bf16 or f32, got {weight.dtype}")
    _expect(weight, "weight", weight.dtype)
    rows, inner = weight.shape
    if group_size <= 0 or group_size % per_word or inner % group_size:
        raise ValueError(f"group size {group_size} must be a positive multiple of {per_word} dividing {inner}")
    _ready(weight)
    packed = torch.empty((rows, inner // per_word), dtype=torch.int32, device=weight.device)
    scales = torch.empty((rows, inner // group_size), dtype=BF16, device=weight.device)
    entry = _lib.library().aoto_hip_w4_quantize if bits == 4 else _lib.library().aoto_hip_w8_quantize
    _lib.check(
        entry(
            _ptr(weight), int(weight.dtype == torch.float32), rows, inner, group_size,
            _ptr(packed), _ptr(scales), None, _stream(),
        )
    )
    return packed, scales


def w4_quantize(weight: torch.Tensor, group_size: int = 64) -> tuple[torch.Tensor, torch.Tensor]:
    """Pack a ``[out, in]`` bf16/f32 weight: ``(int32 [out, in/8], bf16 scales [out, in/group])``.

    Bit-exact with the reference packer (``quantize.py:95-152``,
    ``models/quantized.py:133-163``).
    """

    return _quantize(weight, group_size, 4)


def w8_quantize(weight: torch.Tensor, group_size: int = 64) -> tuple[torch.Tensor, torch.Tensor]:
    """Eight-bit pack: ``(int32 [out, in/4], bf16 scales [out, in/group])``.

    Bit-exact with ``quantize_int8`` (``quantize.py:155-172``) and
    ``pack_weight_int8`` (``models/quantized.py:166-172``).
    """

    return _quantize(weight, group_size, 8)


def quantize(weight: torch.Tensor, group_size: int = 64, bits: int = 4) -> tuple[torch.Tensor, torch.Tensor]:
    """:func:`w4_quantize` or :func:`w8_quantize` by width."""

    if bits not in CODES_PER_WORD:
        raise ValueError(f"bits must be 4 or 8, got {bits!r}")
    return _quantize(weight, group_size, bits)


def _dequantize(packed: torch.Tensor, scales: torch.Tensor, group_size: int, bits: int) -> torch.Tensor:
    _expect(packed, "packed", torch.int32)
    if packed.dim() != 2:
        raise ValueError("packed must be 2-D")
    rows, words = packed.shape
    inner = words * CODES_PER_WORD[bits]
    if group_size <= 0 or inner % group_size:
        raise ValueError(f"group size {group_size} does not divide {inner}")
    _expect(scales, "scales", BF16, (rows, inner // group_size))
    _ready(packed)
    out = torch.empty((rows, inner), dtype=BF16, device=packed.device)
    entry = _lib.library().aoto_hip_w4_dequantize if bits == 4 else _lib.library().aoto_hip_w8_dequantize
    _lib.check(entry(_ptr(packed), _ptr(scales), rows, inner, group_size, _ptr(out), _stream()))
    return out


def w4_dequantize(packed: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """``bf16(code * scale)`` ``[out, in]`` (``models/quantized.py:61-82``)."""

    return _dequantize(packed, scales, group_size, 4)


def w8_dequantize(packed: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """``bf16(code * scale)`` of an eight-bit pack (``models/quantized.py:84-107``)."""

    return _dequantize(packed, scales, group_size, 8)


def _gemv(
    bits: int,
    x: torch.Tensor,
    packed: torch.Tensor,
    scales: torch.Tensor,
    group_size: int,
    norm_weight: torch.Tensor | None,
    eps: float,
    bias: torch.Tensor | None,
    alpha: float,
    beta: float,
    up: tuple[torch.Tensor, torch.Tensor] | None,
    out: torch.Tensor | None,
    lanes_per_row: int = 0,
) -> torch.Tensor:
    per_word = CODES_PER_WORD[bits]
    _expect(packed, "packed", torch.int32)
    if packed.dim() != 2:
        raise ValueError(f"packed must be 2-D [N, K/{per_word}]")
    n, words = packed.shape
    k = words * per_word
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
    lib = _lib.library()
    args = (_ptr(x), _ptr(packed), _ptr(scales), _ptr(up_packed), _ptr(up_scales), _ptr(norm_weight),
            float(eps), _ptr(bias), float(alpha), float(beta), _ptr(out), k, n, group_size)
    if bits == 4:
        _lib.check(lib.aoto_hip_w4_gemv(*args, int(lanes_per_row), _stream()))
    else:
        _lib.check(lib.aoto_hip_w8_gemv(*args, _stream()))
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

    return _gemv(4, x, packed, scales, group_size, norm_weight, eps, bias, alpha, beta, up, out, lanes_per_row)


def w8_gemv(
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
) -> torch.Tensor:
    """:func:`w4_gemv` over an eight-bit pack ``int32 [N, K/4]``
    (``codegen/matmul.py:742-929``)."""

    return _gemv(8, x, packed, scales, group_size, norm_weight, eps, bias, alpha, beta, up, out)


def _i64(tensor: torch.Tensor, name: str) -> None:
    _expect(tensor, name, torch.int64)


def _matmul(
    bits: int,
    x: torch.Tensor,
    packed: torch.Tensor,
    scales: torch.Tensor,
    group_size: int,
    bias: torch.Tensor | None,
    residual: torch.Tensor | None,
    gate: torch.Tensor | None,
    out: torch.Tensor | None,
    tile: int,
    splits: int,
    workspace: torch.Tensor | None,
) -> torch.Tensor:
    per_word = CODES_PER_WORD[bits]
    _expect(packed, "packed", torch.int32)
    if packed.dim() != 2:
        raise ValueError(f"packed must be 2-D [N, K/{per_word}]")
    n, words = packed.shape
    k = words * per_word
    _expect(x, "x", BF16)
    if x.shape[-1] != k:
        raise ValueError(f"x has last dimension {x.shape[-1]}, the weight reduces over {k}")
    m = x.numel() // k
    if group_size <= 0 or k % group_size:
        raise ValueError(f"group size {group_size} does not divide K={k}")
    _expect(scales, "scales", BF16, (n, k // group_size))
    for name, tensor, numel in (("bias", bias, n), ("residual", residual, m * n), ("gate", gate, m * n)):
        if tensor is not None:
            _expect(tensor, name, BF16)
            if tensor.numel() != numel:
                raise ValueError(f"{name} has {tensor.numel()} elements, expected {numel}")
    shape = tuple(x.shape[:-1]) + (n,)
    if out is None:
        out = torch.empty(shape, dtype=BF16, device=x.device)
    else:
        _expect(out, "out", BF16)
        if out.numel() != m * n:
            raise ValueError(f"out has {out.numel()} elements, expected {m * n}")
    _ready(x)
    need = gemm_workspace_bytes(m, n, k, tile, splits)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty((need // 4,), dtype=torch.float32, device=x.device)
    entry = _lib.library().aoto_hip_w4_gemm if bits == 4 else _lib.library().aoto_hip_w8_gemm
    _lib.check(
        entry(
            _ptr(x), _ptr(packed), _ptr(scales), _ptr(bias), _ptr(residual), _ptr(gate), _ptr(out),
            m, n, k, group_size, int(tile), int(splits), _ptr(workspace if need else None), _stream(),
        )
    )
    return out


def w4_matmul(
    x: torch.Tensor,
    packed: torch.Tensor,
    scales: torch.Tensor,
    group_size: int,
    *,
    bias: torch.Tensor | None = None,
    residual: torch.Tensor | None = None,
    gate: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    tile: int = 0,
    splits: int = 0,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """Prefill W4 matmul ``[M, K] -> [M, N]`` on MFMA with one fused epilogue.

    ``bias`` ``[N]`` (q/k/v bias), ``residual`` ``[M, N]`` or ``gate`` ``[M, N]``
    (``silu_mul``: ``bf16(acc * silu(gate))``), as the reference's prefill GEMM.
    """

    return _matmul(4, x, packed, scales, group_size, bias, residual, gate, out, tile, splits, workspace)


def w8_matmul(
    x: torch.Tensor,
    packed: torch.Tensor,
    scales: torch.Tensor,
    group_size: int,
    *,
    bias: torch.Tensor | None = None,
    residual: torch.Tensor | None = None,
    gate: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    tile: int = 0,
    splits: int = 0,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """:func:`w4_matmul` over an eight-bit pack ``int32 [N, K/4]``."""

    return _matmul(8, x, packed, scales, group_size, bias, residual, gate, out, tile, splits, workspace)


#: From this many rows (with K % 256 == 0) the prefill GEMMs' automatic plan
#: (tile = splits = 0) takes the wide-tile 32x32x16-MFMA kernel (the C ABI's kWideRows).
WIDE_ROWS = 512


def wide_plan(m: int, n: int, k: int, *, paired: bool = False) -> tuple[int, int] | None:
    """The automatic plan's ``(tile, splits)`` for ``m`` rows of an ``[n, k]`` weight when
    it takes the wide kernel, else None: the Python mirror of the C ABI's
    ``wide_auto_plan`` (``csrc/aoto_hip.cpp``), for labels and host-side checks."""

    if m < WIDE_ROWS or k % 256:
        return None
    mb = (m + 127) // 128

    def blocks(bn):
        return -(-n // bn) * mb

    tile = 241
    if not paired and n % 384 == 0 and blocks(384) >= 224:
        tile = 243
    elif not paired and blocks(256) >= 224:
        tile = 441
    count = {243: blocks(384), 441: blocks(256), 241: blocks(128)}[tile]
    splits = -(-256 // count) if count < 160 else 1
    most = (k // 128) // 2
    splits = max(1, min(splits, most))
    # the launch cuts K into slices of whole 128-k steps: the count it actually runs
    steps = k // 128
    per = -(-steps // splits)
    return tile, -(-steps // per)


#: Tile codes of the dequant-once long-prefill kernel (``csrc/w4_gemm_lds.h``): the
#: single forms (256 x 128 and 256 x 192 blocks) and the paired gate/up form (256 x (64 + 64)).
LDS_TILE, LDS_WIDE_TILE, LDS_PAIRED_TILE = 822, 823, 821
#: the paired dequant-once forms for short prompts (128-row blocks of 4 waves):
#: 64 + 64 and 32 + 32 columns per block
LDS_SHORT_PAIRED_TILE, LDS_SHORT_NARROW_TILE = 812, 811
#: the single form's split-K partials for short prompts: 128 x 64 and 128 x 32 blocks
LDS_SPLIT_TILE, LDS_SPLIT_NARROW_TILE = 814, 813


def lds_plan(m: int, n: int, k: int, *, group_size: int = 64, paired: bool = False, bits: int = 4,
             gate: bool = False, rope: bool = False) -> int | None:
    """The tile code the automatic plan runs on the dequant-once kernel for this shape, else
    None: the Python mirror of the C ABI's ``lds_auto`` (4-bit codes, no gate epilogue,
    K % 64 == 0, a power-of-two group with an even count per row; from 1024 rows a grid
    of at least 256 blocks whose last round of 256 is at least 90% full: 128 columns per
    block where that fills the rounds, else 192; for a paired gate/up of 32-256 rows the
    128-row forms: 64 + 64 columns where that gives at least 128 blocks from 65 rows,
    else 32 + 32 where that fits 256 blocks; for a single projection of 32-256 rows with
    K >= 2048 and no RoPE epilogue (``rope``) the split-K form, 128 x 64 blocks where
    those give at least 64 column blocks, else 128 x 32)."""

    if bits != 4 or gate or k % 64 or group_size < 32 or group_size & (group_size - 1):
        return None
    if (k // group_size) % 2 or m * k * 2 >= 2 ** 31 or n * k // 2 >= 2 ** 31:
        return None
    if m < 1024:
        if m < 32 or m > 256:
            return None
        mb = -(-m // 128)
        if not paired:
            if rope or k < 2048:
                return None
            return LDS_SPLIT_TILE if -(-n // 64) * mb >= 64 else LDS_SPLIT_NARROW_TILE
        if m > 64 and -(-n // 64) * mb >= 128:
            return LDS_SHORT_PAIRED_TILE
        return LDS_SHORT_NARROW_TILE if -(-n // 32) * mb <= 256 else None
    def fills(bn):
        blocks = -(-n // bn) * -(-m // 256)
        rounds = -(-blocks // 256)
        return blocks >= 256 and blocks * 10 >= rounds * 256 * 9

    if paired:
        return LDS_PAIRED_TILE if fills(64) else None
    return LDS_TILE if fills(128) else LDS_WIDE_TILE if fills(192) else None


def gemm_workspace_bytes(m: int, n: int, k: int, tile: int = 0, splits: int = 0) -> int:
    """Workspace bytes :func:`w4_matmul` needs for this shape: split-K partials (0: no split)."""

    return int(_lib.library().aoto_hip_w4_gemm_workspace(int(m), int(n), int(k), int(tile), int(splits)))


def gate_up_workspace_bytes(m: int, n: int, k: int, tile: int = 0, splits: int = 0) -> int:
    """Workspace bytes :func:`w4_matmul_gate_up` needs (gate and up partials, 0: no split)."""

    return int(_lib.library().aoto_hip_w4_gemm_gate_up_workspace(int(m), int(n), int(k), int(tile), int(splits)))


def _matmul_gate_up(bits, x, gate_packed, gate_scales, up_packed, up_scales, group_size, out, tile, splits,
                    workspace):
    per_word = CODES_PER_WORD[bits]
    _expect(gate_packed, "gate_packed", torch.int32)
    if gate_packed.dim() != 2:
        raise ValueError(f"gate_packed must be 2-D [N, K/{per_word}]")
    n, words = gate_packed.shape
    k = words * per_word
    _expect(up_packed, "up_packed", torch.int32, (n, words))
    _expect(x, "x", BF16)
    if x.shape[-1] != k:
        raise ValueError(f"x has last dimension {x.shape[-1]}, the weights reduce over {k}")
    m = x.numel() // k
    if group_size <= 0 or k % group_size:
        raise ValueError(f"group size {group_size} does not divide K={k}")
    _expect(gate_scales, "gate_scales", BF16, (n, k // group_size))
    _expect(up_scales, "up_scales", BF16, (n, k // group_size))
    shape = tuple(x.shape[:-1]) + (n,)
    if out is None:
        out = torch.empty(shape, dtype=BF16, device=x.device)
    else:
        _expect(out, "out", BF16)
        if out.numel() != m * n:
            raise ValueError(f"out has {out.numel()} elements, expected {m * n}")
    _ready(x)
    need = gate_up_workspace_bytes(m, n, k, tile, splits)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty((need // 4,), dtype=torch.float32, device=x.device)
    lib = _lib.library()
    entry = lib.aoto_hip_w4_gemm_gate_up if bits == 4 else lib.aoto_hip_w8_gemm_gate_up
    _lib.check(
        entry(
            _ptr(x), _ptr(gate_packed), _ptr(gate_scales), _ptr(up_packed), _ptr(up_scales), _ptr(out),
            m, n, k, group_size, int(tile), int(splits), _ptr(workspace if need else None), _stream(),
        )
    )
    return out


def w4_matmul_gate_up(x, gate_packed, gate_scales, up_packed, up_scales, group_size, *, out=None, tile=0,
                      splits=0, workspace=None):
    """Prefill MLP ``bf16(up(x) * silu(bf16(gate(x))))`` ``[M, K] -> [M, N]`` in one pass over x.

    The same values as ``w4_matmul(x, gate)`` followed by ``w4_matmul(x, up, gate=...)``
    (the reference's gate GEMM and silu_mul-epilogue up GEMM), up to the f32
    summation order of the split reduction.
    """

    return _matmul_gate_up(4, x, gate_packed, gate_scales, up_packed, up_scales, group_size, out, tile, splits,
                           workspace)


def w8_matmul_gate_up(x, gate_packed, gate_scales, up_packed, up_scales, group_size, *, out=None, tile=0,
                      splits=0, workspace=None):
    """:func:`w4_matmul_gate_up` over int8 packs (words ``[N, K/4]``)."""

    return _matmul_gate_up(8, x, gate_packed, gate_scales, up_packed, up_scales, group_size, out, tile, splits,
                           workspace)


def matmul_residual_norm(x, packed, scales, group_size, residual, norm_weight, eps, *, bits=4, out=None,
                         norm_out=None, tile=0, splits=0, workspace=None):
    """``y = bf16(x @ W^T + residual)`` then ``norm_out = rms_norm(y, norm_weight, eps)``.

    A decoder layer's o / down projection and the next block's RMSNorm: the same
    values as :func:`w4_matmul` (``residual=``) followed by :func:`rms_norm`, with the
    split-K sum and the norm in one launch. ``out`` may be ``residual`` (in place).
    Returns ``(y, norm_out)``.
    """

    per_word = CODES_PER_WORD[bits]
    _expect(packed, "packed", torch.int32)
    if packed.dim() != 2:
        raise ValueError(f"packed must be 2-D [N, K/{per_word}]")
    n, words = packed.shape
    k = words * per_word
    _expect(x, "x", BF16)
    if x.shape[-1] != k:
        raise ValueError(f"x has last dimension {x.shape[-1]}, the weight reduces over {k}")
    m = x.numel() // k
    if group_size <= 0 or k % group_size:
        raise ValueError(f"group size {group_size} does not divide K={k}")
    _expect(scales, "scales", BF16, (n, k // group_size))
    _expect(residual, "residual", BF16)
    _expect(norm_weight, "norm_weight", BF16, (n,))
    if residual.numel() != m * n:
        raise ValueError(f"residual has {residual.numel()} elements, expected {m * n}")
    shape = tuple(x.shape[:-1]) + (n,)
    out = torch.empty(shape, dtype=BF16, device=x.device) if out is None else out
    norm_out = torch.empty(shape, dtype=BF16, device=x.device) if norm_out is None else norm_out
    for name, t in (("out", out), ("norm_out", norm_out)):
        _expect(t, name, BF16)
        if t.numel() != m * n:
            raise ValueError(f"{name} has {t.numel()} elements, expected {m * n}")
    _ready(x)
    need = gemm_workspace_bytes(m, n, k, tile, splits)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty((need // 4,), dtype=torch.float32, device=x.device)
    lib = _lib.library()
    entry = lib.aoto_hip_w4_gemm_residual_norm if bits == 4 else lib.aoto_hip_w8_gemm_residual_norm
    _lib.check(
        entry(
            _ptr(x), _ptr(packed), _ptr(scales), _ptr(residual), _ptr(out), m, n, k, group_size, int(tile),
            int(splits), _ptr(workspace if need else None), _ptr(norm_weight), float(eps), _ptr(norm_out),
            _stream(),
        )
    )
    return out, norm_out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """Row RMSNorm over the last dimension, ``bf16((x * rsqrt(mean(x^2) + eps)) * w)``."""

    _expect(x, "x", BF16)
    hidden = x.shape[-1]
    _expect(weight, "weight", BF16, (hidden,))
    rows = x.numel() // hidden
    if out is None:
        out = torch.empty_like(x)
    else:
        _expect(out, "out", BF16, tuple(x.shape))
    _ready(x)
    _lib.check(_lib.library().aoto_hip_rms_norm(_ptr(x), _ptr(weight), float(eps), _ptr(out), rows, hidden, _stream()))
    return out


def rope(
    x: torch.Tensor, cos_table: torch.Tensor, sin_table: torch.Tensor, positions: torch.Tensor
) -> torch.Tensor:
    """RoPE of ``x [B, H, S, D]`` with table rows ``positions [B, S]`` (int64)."""

    _expect(x, "x", BF16)
    if x.dim() != 4:
        raise ValueError("x must be [B, H, S, D]")
    batch, heads, seq, dim = x.shape
    _expect(cos_table, "cos_table", BF16)
    _expect(sin_table, "sin_table", BF16, tuple(cos_table.shape))
    if cos_table.shape[-1] != dim:
        raise ValueError("table width must equal the head dimension")
    _i64(positions, "positions")
    if positions.numel() != batch * seq:
        raise ValueError(f"positions must hold B*S = {batch * seq} entries")
    if batch != 1:
        raise ValueError("rope takes one batch row (positions are per token)")
    out = torch.empty_like(x)
    _ready(x)
    _lib.check(
        _lib.library().aoto_hip_rope(
            _ptr(x), _ptr(cos_table), _ptr(sin_table), _ptr(positions), 1, seq, _ptr(out),
            batch * heads * seq, dim, _stream(),
        )
    )
    return out


def rope_qkv_prefill(
    qkv: torch.Tensor,
    positions: torch.Tensor,
    cos_table: torch.Tensor,
    sin_table: torch.Tensor,
    pair: torch.Tensor,
    *,
    query_heads: int,
    kv_heads: int,
    head_dim: int,
    slot0: int,
    zero_prefix: bool = True,
    q_out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Rotate q/k of ``qkv [B, M, W]`` into ``q [B, Hq, M, D]`` and fill ``pair [2, B, Hkv, cap, D]``."""

    _expect(qkv, "qkv", BF16)
    batch, tokens, width = qkv.shape
    if width != (query_heads + 2 * kv_heads) * head_dim:
        raise ValueError("qkv width does not match the head counts")
    _i64(positions, "positions")
    if positions.numel() != batch * tokens:
        raise ValueError("positions must be [B, M]")
    _expect(pair, "pair", BF16)
    if pair.dim() != 5 or tuple(pair.shape[:3]) != (2, batch, kv_heads) or pair.shape[4] != head_dim:
        raise ValueError(f"pair must be [2, {batch}, {kv_heads}, cap, {head_dim}], got {tuple(pair.shape)}")
    capacity = pair.shape[3]
    if q_out is None:
        q_out = torch.empty((batch, query_heads, tokens, head_dim), dtype=BF16, device=qkv.device)
    else:
        _expect(q_out, "q_out", BF16, (batch, query_heads, tokens, head_dim))
    _ready(qkv)
    _lib.check(
        _lib.library().aoto_hip_rope_qkv_prefill(
            _ptr(qkv), _ptr(positions), _ptr(cos_table), _ptr(sin_table), _ptr(q_out), _ptr(pair), batch,
            tokens, query_heads, kv_heads, head_dim, capacity, int(slot0), int(bool(zero_prefix)), _stream(),
        )
    )
    return q_out


def matmul_qkv_rope(
    x: torch.Tensor,
    packed: torch.Tensor,
    scales: torch.Tensor,
    group_size: int,
    positions: torch.Tensor,
    cos_table: torch.Tensor,
    sin_table: torch.Tensor,
    pair: torch.Tensor,
    *,
    query_heads: int,
    kv_heads: int,
    head_dim: int,
    slot0: int,
    bias: torch.Tensor | None = None,
    zero_prefix: bool = True,
    bits: int = 4,
    out: torch.Tensor | None = None,
    q_out: torch.Tensor | None = None,
    tile: int = 0,
    splits: int = 0,
    workspace: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """The packed q/k/v projection ``out = bf16(x @ W^T + bias)`` ``[M, W]`` with RoPE of q into
    ``q_out [1, Hq, M, D]`` and the rotated keys / values into ``pair [2, 1, Hkv, cap, D]`` at
    ``slot0``: :func:`w4_matmul` then :func:`rope_qkv_prefill` (batch 1) in one launch - RoPE in
    the GEMM's epilogue when unsplit (``splits=0`` prefers it whenever a block's columns are
    whole heads), in the split-K sum's launch when split. Returns ``(out, q_out)``."""

    per_word = CODES_PER_WORD[bits]
    _expect(packed, "packed", torch.int32)
    if packed.dim() != 2:
        raise ValueError(f"packed must be 2-D [N, K/{per_word}]")
    n, words = packed.shape
    k = words * per_word
    if n != (query_heads + 2 * kv_heads) * head_dim:
        raise ValueError("the projection's rows do not match the head counts")
    _expect(x, "x", BF16)
    if x.shape[-1] != k:
        raise ValueError(f"x has last dimension {x.shape[-1]}, the weight reduces over {k}")
    m = x.numel() // k
    if group_size <= 0 or k % group_size:
        raise ValueError(f"group size {group_size} does not divide K={k}")
    _expect(scales, "scales", BF16, (n, k // group_size))
    if bias is not None:
        _expect(bias, "bias", BF16, (n,))
    _i64(positions, "positions")
    if positions.numel() != m:
        raise ValueError("positions must hold one entry per row of x")
    _expect(pair, "pair", BF16)
    if pair.dim() != 5 or tuple(pair.shape[:3]) != (2, 1, kv_heads) or pair.shape[4] != head_dim \
            or not pair.is_contiguous():
        raise ValueError(f"pair must be a contiguous [2, 1, {kv_heads}, cap, {head_dim}], got {tuple(pair.shape)}")
    capacity = pair.shape[3]
    if out is None:
        out = torch.empty((m, n), dtype=BF16, device=x.device)
    elif out.numel() != m * n:
        raise ValueError(f"out has {out.numel()} elements, expected {m * n}")
    if q_out is None:
        q_out = torch.empty((1, query_heads, m, head_dim), dtype=BF16, device=x.device)
    else:
        _expect(q_out, "q_out", BF16, (1, query_heads, m, head_dim))
    _ready(x)
    lib = _lib.library()
    need = int(lib.aoto_hip_w4_gemm_qkv_rope_workspace(m, k, int(tile), int(splits), query_heads, kv_heads, head_dim))
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty((need // 4,), dtype=torch.float32, device=x.device)
    entry = lib.aoto_hip_w4_gemm_qkv_rope if bits == 4 else lib.aoto_hip_w8_gemm_qkv_rope
    _lib.check(
        entry(
            _ptr(x), _ptr(packed), _ptr(scales), _ptr(bias), _ptr(out), m, k, group_size, int(tile), int(splits),
            _ptr(workspace if need else None), _ptr(positions), _ptr(cos_table), _ptr(sin_table), _ptr(q_out),
            _ptr(pair), query_heads, kv_heads, head_dim, capacity, int(slot0), int(bool(zero_prefix)), _stream(),
        )
    )
    return out, q_out


def rope_kv_cache_append(
    row: torch.Tensor,
    cos_table: torch.Tensor,
    sin_table: torch.Tensor,
    position: int,
    pair_out: torch.Tensor,
    *,
    pair_in: torch.Tensor | None,
    query_heads: int,
    query_start: int,
    key_start: int,
    value_start: int,
    ring_slot: int | None = None,
    step_state: torch.Tensor | None = None,
    q_out: torch.Tensor | None = None,
) -> torch.Tensor:
    """The decode ``rope_kv_cache_append``: returns ``q [B, Hq, D]``.

    ``pair_in`` given: the reference's roll into ``pair_out``. ``ring_slot``
    given instead: the new key/value is written in place at that slot.
    """

    _expect(row, "row", BF16)
    batch, width = row.shape[0], row.shape[-1]
    _expect(pair_out, "pair_out", BF16)
    _, b2, kv_heads, capacity, head_dim = pair_out.shape
    if b2 != batch:
        raise ValueError("row and pair batch differ")
    mode = 1 if (ring_slot is not None or step_state is not None) else 0
    if mode == 0:
        if pair_in is None:
            raise ValueError("the roll needs pair_in")
        _expect(pair_in, "pair_in", BF16, tuple(pair_out.shape))
    if q_out is None:
        q_out = torch.empty((batch, query_heads, head_dim), dtype=BF16, device=row.device)
    _ready(row)
    _lib.check(
        _lib.library().aoto_hip_rope_kv_cache_append(
            _ptr(row), width, _ptr(cos_table), _ptr(sin_table), int(position), _ptr(pair_in), _ptr(pair_out),
            _ptr(q_out), batch, query_heads, kv_heads, capacity, head_dim, query_start, key_start, value_start,
            mode, int(ring_slot or 0), _ptr(step_state), _stream(),
        )
    )
    return q_out


def decode_attention_workspace(batch: int, query_heads: int, kv_heads: int, capacity: int, head_dim: int,
                               splits: int = 0, device=None) -> torch.Tensor:
    """A workspace for the split-K records of :func:`decode_attention` with these shapes."""

    size = _lib.library().aoto_hip_decode_attention_workspace(batch, query_heads, kv_heads, capacity, head_dim, splits)
    return torch.zeros((max(size, 16),), dtype=torch.uint8, device=device)


def decode_attention(
    q: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    *,
    valid: int | None = None,
    ring_offset: int = 0,
    mask: torch.Tensor | None = None,
    scale: float | None = None,
    workspace: torch.Tensor | None = None,
    splits: int = 0,
    step_state: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Single-query GQA attention: ``q [B, Hq, D]`` over ``keys/values [B, Hkv, cap, D]``."""

    _expect(q, "q", BF16)
    batch, query_heads, head_dim = q.shape
    if keys.dtype != BF16 or values.dtype != BF16 or keys.shape != values.shape or keys.dim() != 4:
        raise ValueError("keys/values must be bf16 [B, Hkv, cap, D] of one shape")
    if keys.stride(-1) != 1 or keys.stride(-2) != head_dim or values.stride() != keys.stride():
        raise ValueError("keys/values rows must be contiguous with matching strides")
    _, kv_heads, capacity, _ = keys.shape
    if scale is None:
        scale = float(torch.tensor(head_dim ** -0.5, dtype=torch.float32))
    mask_ptr = None
    mask_stride = 0
    if mask is not None:
        if mask.dtype != torch.bool:
            raise TypeError("mask must be bool")
        mask = mask.reshape(-1, capacity).to(torch.uint8).contiguous()
        mask_stride = capacity if mask.shape[0] == batch else 0
        mask_ptr = mask
    elif valid is None and step_state is None:
        raise ValueError("pass valid=, mask= or step_state=")
    if out is None:
        out = torch.empty_like(q)
    _ready(q)
    _lib.check(
        _lib.library().aoto_hip_decode_attention(
            _ptr(q), _ptr(keys), _ptr(values), keys.stride(0), keys.stride(1), _ptr(mask_ptr), mask_stride,
            int(valid or 0), int(ring_offset), batch, query_heads, kv_heads, capacity, head_dim, float(scale),
            int(splits), _ptr(workspace), _ptr(step_state), _ptr(out), _stream(),
        )
    )
    return out


def decode_rope_attention(
    row: torch.Tensor,
    cos_table: torch.Tensor,
    sin_table: torch.Tensor,
    pair: torch.Tensor,
    *,
    query_heads: int,
    query_start: int,
    key_start: int,
    value_start: int,
    position: int = 0,
    slot: int = 0,
    valid: int = 0,
    ring_offset: int = 0,
    step_state: torch.Tensor | None = None,
    scale: float | None = None,
    workspace: torch.Tensor | None = None,
    splits: int = 0,
    rope_rows: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """RoPE + in-place KV write at ``slot`` + single-query attention over ``pair [2, B, Hkv, cap, D]``.

    ``rope_rows`` (bf16 ``[2, D]``: cos row, sin row of the current position) replaces the table lookup.
    """

    _expect(row, "row", BF16)
    _expect(pair, "pair", BF16)
    _, batch, kv_heads, capacity, head_dim = pair.shape
    width = row.shape[-1]
    if row.numel() != batch * width:
        raise ValueError("row must be [B, W]")
    if scale is None:
        scale = float(torch.tensor(head_dim ** -0.5, dtype=torch.float32))
    if out is None:
        out = torch.empty((batch, query_heads, head_dim), dtype=BF16, device=row.device)
    if rope_rows is not None:
        _expect(rope_rows, "rope_rows", BF16, (2, head_dim))
    keys, values = pair[0], pair[1]
    _ready(row)
    _lib.check(
        _lib.library().aoto_hip_decode_rope_attention(
            _ptr(row), width, query_start, key_start, value_start, _ptr(cos_table), _ptr(sin_table), _ptr(keys),
            _ptr(values), keys.stride(0), keys.stride(1), int(position), int(slot), int(valid), int(ring_offset),
            batch, query_heads, kv_heads, capacity, head_dim, float(scale), int(splits), _ptr(workspace),
            _ptr(step_state), _ptr(rope_rows), _ptr(out), _stream(),
        )
    )
    return out


def prefill_attention(
    q: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    *,
    causal: bool = True,
    key_start: int = 0,
    mask: torch.Tensor | None = None,
    scale: float | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Prefill GQA attention: ``q [B, Hq, M, D]``, ``keys/values [B, Hkv, Mk, D]`` (rows contiguous)
    -> ``[B, M, Hq*D]``."""

    _expect(q, "q", BF16)
    batch, query_heads, tokens, head_dim = q.shape
    if keys.dtype != BF16 or values.dtype != BF16 or keys.shape != values.shape or keys.dim() != 4:
        raise ValueError("keys/values must be bf16 [B, Hkv, Mk, D] of one shape")
    if keys.stride(-1) != 1 or keys.stride(-2) != head_dim or values.stride() != keys.stride():
        raise ValueError("keys/values rows must be contiguous with matching strides")
    _, kv_heads, key_tokens, _ = keys.shape
    if scale is None:
        scale = float(torch.tensor(head_dim ** -0.5, dtype=torch.float32))
    mask_ptr = None
    mask_stride = 0
    if mask is not None:
        if mask.dtype != torch.bool:
            raise TypeError("mask must be bool")
        mask = mask.reshape(-1, tokens, key_tokens).to(torch.uint8).contiguous()
        mask_stride = tokens * key_tokens if mask.shape[0] == batch and batch > 1 else 0
        mask_ptr = mask
    if out is None:
        out = torch.empty((batch, tokens, query_heads * head_dim), dtype=BF16, device=q.device)
    _ready(q)
    _lib.check(
        _lib.library().aoto_hip_prefill_attention(
            _ptr(q), _ptr(keys), _ptr(values), keys.stride(0), keys.stride(1), _ptr(mask_ptr), mask_stride,
            int(bool(causal)), int(key_start), batch, tokens, key_tokens, query_heads, kv_heads, head_dim,
            float(scale), _ptr(out), _stream(),
        )
    )
    return out


def embedding(weight: torch.Tensor, ids: torch.Tensor, *, out: torch.Tensor | None = None,
              error: torch.Tensor | None = None) -> torch.Tensor:
    """``weight[ids]`` for int64 device ``ids``; out-of-range ids give zero rows and set ``error``."""

    _expect(weight, "weight", BF16)
    _i64(ids, "ids")
    vocab, hidden = weight.shape
    count = ids.numel()
    if out is None:
        out = torch.empty(tuple(ids.shape) + (hidden,), dtype=BF16, device=weight.device)
    if error is not None:
        _expect(error, "error", torch.int32)
    _ready(weight)
    _lib.check(
        _lib.library().aoto_hip_embedding(
            _ptr(weight), _ptr(ids), count, hidden, vocab, _ptr(out), _ptr(error), _stream()
        )
    )
    return out


def argmax(logits: torch.Tensor, *, out: torch.Tensor | None = None, history: torch.Tensor | None = None,
           history_len: torch.Tensor | None = None) -> torch.Tensor:
    """First-index argmax over the last dimension of bf16 ``logits`` -> int64 ``[rows]``."""

    _expect(logits, "logits", BF16)
    n = logits.shape[-1]
    rows = logits.numel() // n
    if out is None:
        out = torch.empty((rows,), dtype=torch.int64, device=logits.device)
    _ready(logits)
    _lib.check(
        _lib.library().aoto_hip_argmax(
            _ptr(logits), rows, n, n, _ptr(out), _ptr(history), _ptr(history_len), _stream()
        )
    )
    return out


def argmax_key_count(k: int, n: int, group_size: int) -> int:
    """Keys ``w4_gemv_argmax`` writes for a ``[n, k]`` weight; 0 when the fused form does not take the shape."""

    return int(_lib.library().aoto_hip_w4_gemv_argmax_keys(int(k), int(n), int(group_size)))


def w4_gemv_argmax(
    x: torch.Tensor,
    packed: torch.Tensor,
    scales: torch.Tensor,
    group_size: int,
    keys: torch.Tensor,
    *,
    norm_weight: torch.Tensor | None = None,
    eps: float = 1e-6,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """LM-head GEMV (optional RMSNorm prologue) that also writes greedy-argmax keys for ``argmax_finish``.

    ``keys`` is an int64 device buffer of at least ``argmax_key_count(K, N, group)`` entries.
    Returns the bf16 logits ``[N]`` (identical to ``w4_gemv``'s).
    """

    _expect(packed, "packed", torch.int32)
    if packed.dim() != 2:
        raise ValueError("packed must be 2-D [N, K/8]")
    n, words = packed.shape
    k = words * 8
    _expect(x, "x", BF16)
    if x.numel() != k:
        raise ValueError(f"x has {x.numel()} elements, the weight reduces over {k}")
    if group_size <= 0 or k % group_size:
        raise ValueError(f"group size {group_size} does not divide K={k}")
    _expect(scales, "scales", BF16, (n, k // group_size))
    _i64(keys, "keys")
    if norm_weight is not None:
        _expect(norm_weight, "norm_weight", BF16)
        if norm_weight.numel() != k:
            raise ValueError(f"norm_weight has {norm_weight.numel()} elements, expected {k}")
    if out is None:
        out = torch.empty((n,), dtype=BF16, device=x.device)
    else:
        _expect(out, "out", BF16)
        if out.numel() != n:
            raise ValueError(f"out has {out.numel()} elements, expected {n}")
    _ready(x)
    _lib.check(
        _lib.library().aoto_hip_w4_gemv_argmax(
            _ptr(x), _ptr(packed), _ptr(scales), _ptr(norm_weight), float(eps), _ptr(out), k, n, group_size,
            _ptr(keys), keys.numel(), _stream(),
        )
    )
    return out


def argmax_finish(
    keys: torch.Tensor,
    count: int,
    *,
    out: torch.Tensor,
    history: torch.Tensor | None = None,
    history_len: torch.Tensor | None = None,
    step_state: torch.Tensor | None = None,
    capacity: int = 0,
    embedding: torch.Tensor | None = None,
    hidden_out: torch.Tensor | None = None,
    error: torch.Tensor | None = None,
    rope_tables: tuple[torch.Tensor, torch.Tensor] | None = None,
    rope_rows: torch.Tensor | None = None,
) -> torch.Tensor:
    """Reduce ``count`` argmax keys to the greedy token ``out[0]``; optionally append it to ``history``,
    advance ``step_state``, gather its ``embedding`` row into ``hidden_out`` and copy the advanced
    position's rows of ``rope_tables`` (cos, sin ``[capacity, D]``) into ``rope_rows`` ``[2, D]``."""

    _i64(keys, "keys")
    _i64(out, "out")
    if not 0 < count <= keys.numel():
        raise ValueError(f"count {count} is outside (0, {keys.numel()}]")
    if step_state is not None:
        _expect(step_state, "step_state", torch.int32, (4,))
    hidden = rows = 0
    if embedding is not None:
        _expect(embedding, "embedding", BF16)
        rows, hidden = embedding.shape
        if hidden_out is None or hidden_out.numel() != hidden:
            raise ValueError("hidden_out must hold one embedding row")
        _expect(hidden_out, "hidden_out", BF16)
    if error is not None:
        _expect(error, "error", torch.int32)
    cos_table = sin_table = None
    head_dim = 0
    if rope_rows is not None:
        if rope_tables is None or step_state is None:
            raise ValueError("rope_rows needs rope_tables and step_state")
        cos_table, sin_table = rope_tables
        head_dim = cos_table.shape[-1]
        _expect(cos_table, "cos table", BF16, (int(capacity), head_dim))
        _expect(sin_table, "sin table", BF16, (int(capacity), head_dim))
        _expect(rope_rows, "rope_rows", BF16, (2, head_dim))
    _ready(keys)
    _lib.check(
        _lib.library().aoto_hip_argmax_finish(
            _ptr(keys), int(count), _ptr(out), _ptr(history), _ptr(history_len), _ptr(step_state), int(capacity),
            _ptr(embedding), int(rows), int(hidden), _ptr(hidden_out), _ptr(error), _ptr(cos_table),
            _ptr(sin_table), int(head_dim), _ptr(rope_rows), _stream(),
        )
    )
    return out


def gemv_finish_supported(k: int, n: int, group_size: int, key_count: int) -> bool:
    """Whether ``w4_gemv_finish`` takes a ``[n, k]`` weight and ``key_count`` keys (a shape check, no launch)."""

    if not 0 < key_count <= int(_lib.library().aoto_hip_w4_gemv_finish_max_keys()):
        return False
    if group_size < 32 or group_size & (group_size - 1) or k % group_size or (k // group_size) % 2:
        return False
    return (k == 896 and n <= 8192) or (k == 4096 and n <= 16384)


def w4_gemv_finish(
    keys: torch.Tensor,
    count: int,
    embedding: torch.Tensor,
    packed: torch.Tensor,
    scales: torch.Tensor,
    group_size: int,
    *,
    norm_weight: torch.Tensor,
    eps: float,
    out: torch.Tensor,
    token_out: torch.Tensor,
    hidden_out: torch.Tensor,
    bias: torch.Tensor | None = None,
    history: torch.Tensor | None = None,
    history_len: torch.Tensor | None = None,
    step_state: torch.Tensor | None = None,
    capacity: int = 0,
    error: torch.Tensor | None = None,
    rope_tables: tuple[torch.Tensor, torch.Tensor] | None = None,
    rope_rows: torch.Tensor | None = None,
) -> torch.Tensor:
    """``argmax_finish`` of ``count`` keys folded into the next step's first W4 GEMV.

    The greedy token's ``embedding`` row is the GEMV's x (RMSNorm prologue with
    ``norm_weight``, optional ``bias``): ``out`` [N] equals ``w4_gemv`` of that row.
    The token, history, step state, RoPE rows and the raw row (into ``hidden_out``)
    are recorded as ``argmax_finish`` records them.
    """

    _i64(keys, "keys")
    _i64(token_out, "token_out")
    _expect(packed, "packed", torch.int32)
    if packed.dim() != 2:
        raise ValueError("packed must be 2-D [N, K/8]")
    n, words = packed.shape
    k = words * 8
    _expect(embedding, "embedding", BF16)
    rows, hidden = embedding.shape
    if hidden != k:
        raise ValueError(f"embedding rows have {hidden} elements, the weight reduces over {k}")
    if group_size <= 0 or k % group_size:
        raise ValueError(f"group size {group_size} does not divide K={k}")
    _expect(scales, "scales", BF16, (n, k // group_size))
    _expect(norm_weight, "norm_weight", BF16)
    if norm_weight.numel() != k:
        raise ValueError(f"norm_weight has {norm_weight.numel()} elements, expected {k}")
    if bias is not None:
        _expect(bias, "bias", BF16)
        if bias.numel() != n:
            raise ValueError(f"bias has {bias.numel()} elements, expected {n}")
    _expect(out, "out", BF16)
    if out.numel() != n:
        raise ValueError(f"out has {out.numel()} elements, expected {n}")
    _expect(hidden_out, "hidden_out", BF16)
    if hidden_out.numel() != k:
        raise ValueError("hidden_out must hold one embedding row")
    if not 0 < count <= keys.numel():
        raise ValueError(f"count {count} is outside (0, {keys.numel()}]")
    if step_state is not None:
        _expect(step_state, "step_state", torch.int32, (4,))
    if error is not None:
        _expect(error, "error", torch.int32)
    cos_table = sin_table = None
    head_dim = 0
    if rope_rows is not None:
        if rope_tables is None or step_state is None:
            raise ValueError("rope_rows needs rope_tables and step_state")
        cos_table, sin_table = rope_tables
        head_dim = cos_table.shape[-1]
        _expect(cos_table, "cos table", BF16, (int(capacity), head_dim))
        _expect(sin_table, "sin table", BF16, (int(capacity), head_dim))
        _expect(rope_rows, "rope_rows", BF16, (2, head_dim))
    _ready(keys)
    _lib.check(
        _lib.library().aoto_hip_w4_gemv_finish(
            _ptr(keys), int(count), _ptr(embedding), int(rows), _ptr(packed), _ptr(scales), _ptr(norm_weight),
            float(eps), _ptr(bias), 1.0, 1.0, _ptr(out), k, n, int(group_size), _ptr(token_out), _ptr(history),
            _ptr(history_len), _ptr(step_state), int(capacity), _ptr(cos_table), _ptr(sin_table), int(head_dim),
            _ptr(rope_rows), _ptr(hidden_out), _ptr(error), _stream(),
        )
    )
    return out


def step_advance(step_state: torch.Tensor, capacity: int) -> None:
    """Advance the int32 device step state ``{position, valid, ring_offset, slot}`` by one token."""

    _expect(step_state, "step_state", torch.int32, (4,))
    _ready(step_state)
    _lib.check(_lib.library().aoto_hip_step_advance(_ptr(step_state), int(capacity), _stream()))
