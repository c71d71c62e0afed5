"""ctypes binding of ``libaoto_hip.so`` and the code-object lifecycle.

The library is the C ABI of ``include/aoto_hip.h``. Loading it needs nothing
from a GPU; installing a code object (``ensure_code_object``) needs the HIP
runtime on the current device, which torch initializes. There is no fallback:
a missing library or code object raises :class:`HipBackendUnavailable`.
"""

from __future__ import annotations

import ctypes
import hashlib
import os
import threading
import weakref

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(PACKAGE_DIR, "libaoto_hip.so")
CODE_OBJECT_PATH = os.path.join(PACKAGE_DIR, "aoto_gfx950.hsaco")
ARCH = "gfx950"

AOTO_OK = 0
AOTO_ERR_ARGUMENT = 1
AOTO_ERR_NO_CODE_OBJECT = 2
AOTO_ERR_HIP = 3
AOTO_ERR_UNSUPPORTED = 4

_c_int = ctypes.c_int
_c_float = ctypes.c_float
_c_size = ctypes.c_size_t
_i64 = ctypes.c_int64
_p = ctypes.c_void_p

#: Every exported entry point with its argument types, in header order.
SIGNATURES: dict[str, tuple] = {
    "aoto_hip_abi_version": (),
    "aoto_hip_trace_launches": (_c_int,),
    "aoto_hip_take_launches": (ctypes.c_char_p, _c_size),
    "aoto_hip_last_error": (ctypes.c_char_p, _c_size),
    "aoto_hip_load_code_object": (_p, _c_size),
    "aoto_hip_unload_code_object": (),
    "aoto_hip_hold_graphs": (_c_int,),
    "aoto_hip_graph_holds": (),
    "aoto_hip_code_object_loaded": (),
    "aoto_hip_w4_quantize": (_p, _c_int, _c_int, _c_int, _c_int, _p, _p, _p, _p),
    "aoto_hip_w4_dequantize": (_p, _p, _c_int, _c_int, _c_int, _p, _p),
    "aoto_hip_w4_gemv": (
        _p, _p, _p, _p, _p, _p, _c_float, _p, _c_float, _c_float, _p,
        _c_int, _c_int, _c_int, _c_int, _p,
    ),
    "aoto_hip_w4_gemm": (_p, _p, _p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _p, _p),
    "aoto_hip_w4_gemm_workspace": (_c_int, _c_int, _c_int, _c_int, _c_int),
    "aoto_hip_w8_quantize": (_p, _c_int, _c_int, _c_int, _c_int, _p, _p, _p, _p),
    "aoto_hip_w8_dequantize": (_p, _p, _c_int, _c_int, _c_int, _p, _p),
    "aoto_hip_w8_gemv": (
        _p, _p, _p, _p, _p, _p, _c_float, _p, _c_float, _c_float, _p,
        _c_int, _c_int, _c_int, _p,
    ),
    "aoto_hip_w8_gemm": (_p, _p, _p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _p, _p),
    "aoto_hip_w4_gemm_gate_up": (_p, _p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _p, _p),
    "aoto_hip_w4_gemm_residual_norm": (_p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _p, _p,
                                       _c_float, _p, _p),
    "aoto_hip_w8_gemm_residual_norm": (_p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _p, _p,
                                       _c_float, _p, _p),
    "aoto_hip_w8_gemm_gate_up": (_p, _p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _p, _p),
    "aoto_hip_w4_gemm_gate_up_workspace": (_c_int, _c_int, _c_int, _c_int, _c_int),
    "aoto_hip_rms_norm": (_p, _p, _c_float, _p, _c_int, _c_int, _p),
    "aoto_hip_rope": (_p, _p, _p, _p, _c_int, _c_int, _p, _i64, _c_int, _p),
    "aoto_hip_rope_qkv_prefill": (
        _p, _p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _p,
    ),
    "aoto_hip_rope_kv_cache_append": (
        _p, _c_int, _p, _p, _c_int, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
        _c_int, _c_int, _c_int, _p, _p,
    ),
    "aoto_hip_w4_gemm_qkv_rope": (
        _p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _p, _p, _p, _p, _p, _p, _c_int, _c_int, _c_int,
        _c_int, _c_int, _c_int, _p,
    ),
    "aoto_hip_w8_gemm_qkv_rope": (
        _p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _p, _p, _p, _p, _p, _p, _c_int, _c_int, _c_int,
        _c_int, _c_int, _c_int, _p,
    ),
    "aoto_hip_w4_gemm_qkv_rope_workspace": (_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int),
    "aoto_hip_w4_gemm_noalloc": (_p, _p, _p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _p),
    "aoto_hip_decode_attention_workspace": (_c_int, _c_int, _c_int, _c_int, _c_int, _c_int),
    "aoto_hip_decode_attention": (
        _p, _p, _p, _i64, _i64, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
        _c_float, _c_int, _p, _p, _p, _p,
    ),
    "aoto_hip_decode_rope_attention": (
        _p, _c_int, _c_int, _c_int, _c_int, _p, _p, _p, _p, _i64, _i64, _c_int, _c_int, _c_int, _c_int, _c_int,
        _c_int, _c_int, _c_int, _c_int, _c_float, _c_int, _p, _p, _p, _p, _p,
    ),
    "aoto_hip_step_advance": (_p, _c_int, _p),
    "aoto_hip_prefill_attention": (
        _p, _p, _p, _i64, _i64, _p, _i64, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
        _c_float, _p, _p,
    ),
    "aoto_hip_embedding": (_p, _p, _c_int, _c_int, _i64, _p, _p, _p),
    "aoto_hip_argmax": (_p, _c_int, _c_int, _i64, _p, _p, _p, _p),
    "aoto_hip_w4_gemv_argmax_keys": (_c_int, _c_int, _c_int),
    "aoto_hip_w4_gemv_argmax": (_p, _p, _p, _p, _c_float, _p, _c_int, _c_int, _c_int, _p, _c_size, _p),
    "aoto_hip_argmax_finish": (
        _p, _c_int, _p, _p, _p, _p, _c_int, _p, _i64, _c_int, _p, _p, _p, _p, _c_int, _p, _p,
    ),
    "aoto_hip_w4_gemv_finish_max_keys": (),
    "aoto_hip_w4_gemv_finish": (
        _p, _c_int, _p, _i64, _p, _p, _p, _c_float, _p, _c_float, _c_float, _p, _c_int, _c_int, _c_int,
        _p, _p, _p, _p, _c_int, _p, _p, _c_int, _p, _p, _p, _p,
    ),
    "aoto_hip_generic_elementwise": (_c_int, _p, _p, _p, _p, ctypes.c_double, _p),
    "aoto_hip_generic_reduce": (_c_int, _p, _p, _p),
    "aoto_hip_generic_matmul": (_p, _p, _p, _p, _c_float, _c_float, _p),
    "aoto_hip_generic_index": (_p, _p, _c_int, _p, _p, _p),
    "aoto_hip_generic_copy": (_p, _p, _p),
    "aoto_hip_generic_fill": (_p, ctypes.c_double, ctypes.c_double, _p),
    "aoto_hip_generic_rms_norm": (_p, _p, _p, _c_float, _c_int, _p),
    "aoto_hip_generic_attention": (_p, _p, _p, _p, _p, _c_int, _c_float, _p),
}

#: Entry points returning a size rather than a status.
SIZE_RETURNING = {"aoto_hip_last_error", "aoto_hip_take_launches", "aoto_hip_decode_attention_workspace",
                  "aoto_hip_w4_gemm_workspace", "aoto_hip_w4_gemm_gate_up_workspace", "aoto_hip_w4_gemm_qkv_rope_workspace",
                  "aoto_hip_w4_gemv_argmax_keys", "aoto_hip_w4_gemv_finish_max_keys"}


class HipBackendUnavailable(RuntimeError):
    """The HIP library or its gfx950 code object cannot be used here."""


class HipKernelError(RuntimeError):
    """A launcher refused its arguments or HIP reported an error."""

    def __init__(self, status: int, message: str) -> None:
        super().__init__(f"[aoto_hip status {status}] {message}")
        self.status = status


class UnsupportedShape(HipKernelError):
    """The shape is outside a kernel's limits (status AOTO_ERR_UNSUPPORTED)."""


_lock = threading.RLock()
_lib: ctypes.CDLL | None = None
_loaded_devices: dict[int, str] = {}
_loaded_images: dict[int, bytes] = {}


def library() -> ctypes.CDLL:
    """Load the C-ABI library once; raise if it was never built."""

    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIBRARY_PATH):
                raise HipBackendUnavailable(
                    f"{LIBRARY_PATH} is missing: build it with `python -m aotolith_amd.csrc.build`"
                )
            lib = ctypes.CDLL(LIBRARY_PATH)
            for name, argtypes in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = list(argtypes)
                fn.restype = _c_size if name in SIZE_RETURNING else _c_int
            _lib = lib
    return _lib


def last_error() -> str:
    buf = ctypes.create_string_buffer(1024)
    library().aoto_hip_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(status: int) -> None:
    if status == AOTO_OK:
        return
    message = last_error()
    if status == AOTO_ERR_UNSUPPORTED:
        raise UnsupportedShape(status, message)
    raise HipKernelError(status, message)


def default_code_object() -> bytes:
    if not os.path.exists(CODE_OBJECT_PATH):
        raise HipBackendUnavailable(
            f"{CODE_OBJECT_PATH} is missing: build it with `python -m aotolith_amd.csrc.build`"
        )
    with open(CODE_OBJECT_PATH, "rb") as handle:
        return handle.read()


def code_object_digest(image: bytes) -> str:
    return hashlib.sha256(image).hexdigest()


def install_code_object(image: bytes, device: int | None = None) -> str:
    """Install ``image`` as the module of ``device`` (default: current); return its digest."""

    import torch

    if not torch.cuda.is_available():
        raise HipBackendUnavailable("no ROCm GPU visible: the hip-gfx950 target needs an MI355X")
    device = torch.cuda.current_device() if device is None else device
    digest = code_object_digest(image)
    torch.cuda.init()
    with torch.cuda.device(device):
        buffer = ctypes.create_string_buffer(image, len(image))
        check(library().aoto_hip_load_code_object(buffer, len(image)))
    _loaded_devices[device] = digest
    _loaded_images[device] = bytes(image)
    return digest


def _release_graph_hold() -> None:
    library().aoto_hip_hold_graphs(-1)


def hold_graph(graph) -> None:
    """Count a captured graph whose nodes launch this library's kernels until it is
    garbage-collected: while any is held, a code-object reload keeps the replaced
    module loaded and ``aoto_hip_unload_code_object`` refuses (the graph launches
    kernels by handle)."""

    check(library().aoto_hip_hold_graphs(1))
    weakref.finalize(graph, _release_graph_hold)


def ensure_code_object(device: int | None = None) -> str:
    """Install the packaged code object on ``device`` unless one is installed."""

    import torch

    if not torch.cuda.is_available():
        raise HipBackendUnavailable("no ROCm GPU visible: the hip-gfx950 target needs an MI355X")
    device = torch.cuda.current_device() if device is None else device
    digest = _loaded_devices.get(device)
    if digest is not None:
        return digest
    with _lock:
        digest = _loaded_devices.get(device)
        if digest is None:
            digest = install_code_object(default_code_object(), device)
    return digest


def installed_digest(device: int) -> str | None:
    return _loaded_devices.get(device)


def installed_image(device: int) -> bytes | None:
    """The code object installed on ``device`` by this process, if any."""

    return _loaded_images.get(device)
