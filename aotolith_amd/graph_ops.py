"""gfx950 lowering of a :class:`~aotolith_amd.graph.LoweredGraph`: one launch per compute node.

Each node of the captured graph maps to a generic kernel of the C ABI
(``aoto_hip_generic_*``): elementwise, reduction/scan, strided batched GEMM,
advanced indexing, strided copy, fill/arange, and the two legalized patterns
(RMSNorm, scaled-dot-product attention). View nodes (view, permute, expand,
slice, unsqueeze, ...) change only the strides the next kernel reads through;
when a view cannot be expressed by strides, a copy kernel materializes it.

The node set and its semantics follow what the reference's ``mlx-reference``
target executes per node (``runtime/mlx_ops/__init__.py:239-620``); torch's
ATen semantics decide dtypes and broadcasting (they are recorded on every node
at capture). A node this module cannot lower is a compile-time error: there is
no torch or CPU fallback.
"""

from __future__ import annotations

import ctypes
import math
from collections.abc import Callable

import torch

from . import _lib
from .errors import CompilationError, PlanInputError
from .graph import RMS_NORM, LoweredGraph, Node, Ref
from .plan import ARCHITECTURE, CompiledPlan, PlanNode
from .selection import KernelSelection

MAX_DIMS = 8

DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.int64: 2, torch.int32: 3, torch.bool: 4, torch.uint8: 5,
               torch.int8: 6}


class AotoTensor(ctypes.Structure):
    """``aoto_tensor`` of include/aoto_hip.h."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * MAX_DIMS),
        ("strides", ctypes.c_int64 * MAX_DIMS),
        ("value", ctypes.c_double),
    ]


def describe(value) -> AotoTensor:
    """The descriptor of a device tensor, or of a Python scalar (data NULL, ndim 0)."""

    d = AotoTensor()
    if isinstance(value, torch.Tensor):
        if value.dtype not in DTYPE_CODES:
            raise CompilationError(f"element type {value.dtype} has no gfx950 kernel here")
        if value.dim() > MAX_DIMS:
            raise CompilationError(f"tensors of rank {value.dim()} exceed the kernels' {MAX_DIMS} dims")
        d.data = value.data_ptr() if value.numel() else 1  # a non-null pointer for empty tensors
        d.dtype = DTYPE_CODES[value.dtype]
        d.ndim = value.dim()
        for i, (n, s) in enumerate(zip(value.shape, value.stride())):
            d.shape[i] = n
            d.strides[i] = s
        return d
    d.data = None
    d.ndim = 0
    d.value = float(value)
    return d


def _p(desc: AotoTensor | None):
    """The address of a descriptor (kept alive by the caller for the call)."""

    return None if desc is None else ctypes.addressof(desc)


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


# ----------------------------------------------------------------------------- launches
# Every launcher binds its descriptors to locals before the call: the C side
# reads them through their addresses, so they must outlive the call.
def launch_elementwise(op: int, out: torch.Tensor, a, b=None, c=None, alpha: float = 1.0) -> torch.Tensor:
    do, da = describe(out), describe(a)
    db = None if b is None else describe(b)
    dc = None if c is None else describe(c)
    _lib.check(_lib.library().aoto_hip_generic_elementwise(op, _p(do), _p(da), _p(db), _p(dc), float(alpha),
                                                           _stream()))
    return out


def launch_copy(dst: torch.Tensor, src: torch.Tensor) -> torch.Tensor:
    dd, ds = describe(dst), describe(src)
    _lib.check(_lib.library().aoto_hip_generic_copy(_p(dd), _p(ds), _stream()))
    return dst


def launch_fill(dst: torch.Tensor, start: float, step: float = 0.0) -> torch.Tensor:
    dd = describe(dst)
    _lib.check(_lib.library().aoto_hip_generic_fill(_p(dd), float(start), float(step), _stream()))
    return dst


def launch_reduce(op: int, out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    do, dx = describe(out), describe(x)
    _lib.check(_lib.library().aoto_hip_generic_reduce(op, _p(do), _p(dx), _stream()))
    return out


def launch_matmul(out: torch.Tensor, a: torch.Tensor, b: torch.Tensor, bias=None, alpha=1.0, beta=1.0):
    do, da, db = describe(out), describe(a), describe(b)
    dbias = None if bias is None else describe(bias)
    _lib.check(_lib.library().aoto_hip_generic_matmul(_p(do), _p(da), _p(db), _p(dbias), float(alpha), float(beta),
                                                      _stream()))
    return out


def launch_index(out: torch.Tensor, src: torch.Tensor, indices: list, error: torch.Tensor | None):
    descs = [describe(ix) for ix in indices]
    array = (ctypes.c_void_p * len(descs))(*[ctypes.addressof(d) for d in descs])
    err = None if error is None else ctypes.c_void_p(error.data_ptr())
    do, ds = describe(out), describe(src)
    _lib.check(_lib.library().aoto_hip_generic_index(_p(do), _p(ds), len(descs), ctypes.addressof(array), err,
                                                     _stream()))
    return out


def launch_rms_norm(out: torch.Tensor, x: torch.Tensor, weight, eps: float, mid_dtype) -> torch.Tensor:
    do, dx = describe(out), describe(x)
    dw = None if weight is None else describe(weight)
    _lib.check(_lib.library().aoto_hip_generic_rms_norm(_p(do), _p(dx), _p(dw), float(eps), DTYPE_CODES[mid_dtype],
                                                        _stream()))
    return out


def launch_attention(out, q, k, v, mask, causal: bool, scale: float) -> torch.Tensor:
    do, dq, dk, dv = describe(out), describe(q), describe(k), describe(v)
    dm = None if mask is None else describe(mask)
    _lib.check(_lib.library().aoto_hip_generic_attention(_p(do), _p(dq), _p(dk), _p(dv), _p(dm), int(bool(causal)),
                                                         float(scale), _stream()))
    return out


# ----------------------------------------------------------------------------- helpers
EW = {  # op -> (code, arity)
    "cast": 0, "neg": 1, "abs": 2, "reciprocal": 3, "sqrt": 4, "rsqrt": 5, "exp": 6, "log": 7, "sigmoid": 8,
    "silu": 9, "tanh": 10, "cos": 11, "sin": 12, "relu": 13, "gelu": 14, "gelu_tanh": 15, "erf": 16, "floor": 17,
    "ceil": 18, "log1p": 19, "expm1": 20, "logical_not": 21, "bitwise_not": 22, "add": 32, "sub": 33, "mul": 34,
    "div": 35, "div_trunc": 36, "div_floor": 37, "pow": 38, "maximum": 39, "minimum": 40, "remainder": 41,
    "bitwise_and": 42, "bitwise_or": 43, "bitwise_xor": 44, "logical_and": 45, "logical_or": 46, "eq": 48, "ne": 49,
    "lt": 50, "le": 51, "gt": 52, "ge": 53, "isnan": 54, "where": 64,
}
RED = {"sum": 0, "mean": 1, "amax": 2, "amin": 3, "any": 4, "all": 5, "argmax": 6, "argmin": 7, "softmax": 8,
       "log_softmax": 9, "cumsum": 10}

UNARY_OPS = {
    "aten.neg.default": "neg", "aten.abs.default": "abs", "aten.reciprocal.default": "reciprocal",
    "aten.sqrt.default": "sqrt", "aten.rsqrt.default": "rsqrt", "aten.exp.default": "exp", "aten.log.default": "log",
    "aten.sigmoid.default": "sigmoid", "aten.silu.default": "silu", "aten.tanh.default": "tanh",
    "aten.cos.default": "cos", "aten.sin.default": "sin", "aten.relu.default": "relu", "aten.erf.default": "erf",
    "aten.floor.default": "floor", "aten.ceil.default": "ceil", "aten.log1p.default": "log1p",
    "aten.expm1.default": "expm1", "aten.logical_not.default": "logical_not",
    "aten.bitwise_not.default": "bitwise_not", "aten.isnan.default": "isnan",
}
BINARY_OPS = {}
for _name in ("add", "sub", "mul", "div", "eq", "ne", "lt", "le", "gt", "ge", "bitwise_and", "bitwise_or",
              "bitwise_xor", "remainder"):
    BINARY_OPS[f"aten.{_name}.Tensor"] = _name
    BINARY_OPS[f"aten.{_name}.Scalar"] = _name
BINARY_OPS.update({"aten.maximum.default": "maximum", "aten.minimum.default": "minimum",
                   "aten.logical_and.default": "logical_and", "aten.logical_or.default": "logical_or",
                   "aten.pow.Tensor_Scalar": "pow", "aten.pow.Tensor_Tensor": "pow", "aten.pow.Scalar": "pow"})
REDUCE_OPS = {"aten.sum.dim_IntList": "sum", "aten.sum.default": "sum", "aten.mean.dim": "mean",
              "aten.mean.default": "mean", "aten.amax.default": "amax", "aten.amin.default": "amin",
              "aten.any.dim": "any", "aten.any.dims": "any", "aten.any.default": "any", "aten.all.dim": "all",
              "aten.all.dims": "all", "aten.all.default": "all", "aten.argmax.default": "argmax",
              "aten.argmin.default": "argmin"}
FILL_OPS = {"aten.full.default", "aten.full_like.default", "aten.zeros.default", "aten.zeros_like.default",
            "aten.ones.default", "aten.ones_like.default", "aten.empty.memory_format", "aten.empty_like.default",
            "aten.scalar_tensor.default", "aten.arange.start_step", "aten.arange.default", "aten.arange.start",
            "aten.new_zeros.default", "aten.new_ones.default", "aten.new_full.default", "aten.new_empty.default"}
COPY_OPS = {"aten.clone.default", "aten._to_copy.default", "aten.lift_fresh_copy.default", "aten.copy.default",
            "aten.cat.default", "aten.contiguous.default"}
MATMUL_OPS = {"aten.mm.default", "aten.bmm.default", "aten.addmm.default", "aten.baddbmm.default"}
INDEX_OPS = {"aten.embedding.default", "aten.index.Tensor", "aten.index_select.default"}
OTHER_OPS = {"aten._softmax.default": "softmax", "aten._log_softmax.default": "log_softmax",
             "aten.cumsum.default": "cumsum", "aten.where.self": "where", "aten.clamp.default": "clamp",
             "aten.clamp_min.default": "clamp", "aten.clamp_max.default": "clamp",
             "aten.masked_fill.Scalar": "masked_fill", "aten.gelu.default": "gelu",
             "aten.scaled_dot_product_attention.default": "attention", RMS_NORM: "rms_norm",
             "aten.div.Tensor_mode": "div_mode", "aten.rsub.Scalar": "rsub", "aten.rsub.Tensor": "rsub"}

FAMILIES = {}
for _op in UNARY_OPS:
    FAMILIES[_op] = "elementwise"
for _op in BINARY_OPS:
    FAMILIES[_op] = "elementwise"
for _op in ("aten.where.self", "aten.clamp.default", "aten.clamp_min.default", "aten.clamp_max.default",
            "aten.masked_fill.Scalar", "aten.gelu.default", "aten.div.Tensor_mode", "aten.rsub.Scalar",
            "aten.rsub.Tensor"):
    FAMILIES[_op] = "elementwise"
for _op in REDUCE_OPS:
    FAMILIES[_op] = "reduction"
for _op in ("aten._softmax.default", "aten._log_softmax.default", "aten.cumsum.default"):
    FAMILIES[_op] = "reduction"
for _op in FILL_OPS:
    FAMILIES[_op] = "fill"
for _op in COPY_OPS:
    FAMILIES[_op] = "copy"
for _op in MATMUL_OPS:
    FAMILIES[_op] = "matmul"
for _op in INDEX_OPS:
    FAMILIES[_op] = "gather"
FAMILIES["aten.scaled_dot_product_attention.default"] = "attention"
FAMILIES[RMS_NORM] = "rms_norm"

KERNELS = {"elementwise": "aoto_generic_elementwise", "reduction": "aoto_generic_reduce",
           "matmul": "aoto_generic_gemm", "gather": "aoto_generic_index", "copy": "aoto_generic_copy",
           "fill": "aoto_generic_fill", "rms_norm": "aoto_generic_rms_norm", "attention": "aoto_generic_attention"}
REASONS = {
    "elementwise": "strided broadcasting elementwise kernel, f32 compute, one rounding to the output type",
    "reduction": "row reduction / scan over the (permuted) last dim, f32 or int64 accumulation",
    "matmul": "strided batched GEMM, LDS-staged 64x64 tiles, f32 accumulation",
    "gather": "advanced indexing gather with bounds flag",
    "copy": "strided copy with element-type conversion",
    "fill": "device fill / arange",
    "rms_norm": "legalized HF RMSNorm chain in one kernel",
    "attention": "legalized scaled-dot-product attention (bool/float mask, causal, GQA), f32 softmax",
}


def _empty(shape, dtype, device) -> torch.Tensor:
    return torch.empty(tuple(shape), dtype=dtype, device=device)


def _contiguous(x: torch.Tensor) -> torch.Tensor:
    """``x`` itself when contiguous, else a contiguous copy made by the copy kernel."""

    if x.is_contiguous():
        return x
    return launch_copy(_empty(x.shape, x.dtype, x.device), x)


def _norm_dims(dims, rank: int) -> list[int]:
    if dims is None:
        return list(range(rank))
    if isinstance(dims, int):
        dims = [dims]
    out = sorted({d % rank if rank else 0 for d in dims})
    return out if out else list(range(rank))


def _value(env, arg):
    if isinstance(arg, Ref):
        return env[arg.name]
    if isinstance(arg, (list, tuple)):
        return type(arg)(_value(env, a) for a in arg)
    return arg


class GraphRunner:
    """Runs a lowered graph's nodes on the current GPU, one generic kernel per compute node."""

    def __init__(self, graph: LoweredGraph, device: torch.device):
        self.graph = graph
        self.device = device
        self.state = {name: tensor.detach().to(device).contiguous() if isinstance(tensor, torch.Tensor) else tensor
                      for name, tensor in graph.state.items()}
        self.handlers: list[tuple[Node, Callable]] = []
        for node in graph.nodes:
            self.handlers.append((node, self._handler(node)))
        self.error = None

    # -- selection records --------------------------------------------------------
    def selections(self, device_name: str | None) -> tuple[KernelSelection, ...]:
        out = []
        for node in self.graph.nodes:
            if node.is_view:
                continue
            family = FAMILIES[node.op]
            out.append(KernelSelection(
                op_index=len(out), op=node.op.split(".")[1] if node.op.startswith("aten.") else node.op,
                output_id=node.name, implementation="hip_kernel", kind=family, reason=REASONS[family],
                artifact_name=KERNELS[family], device_name=device_name, device_architecture=ARCHITECTURE,
            ))
        return tuple(out)

    # -- execution ------------------------------------------------------------------
    def run(self, inputs: dict[str, torch.Tensor], *, verify_index_bounds: bool = True):
        env: dict = dict(self.state)
        env.update(inputs)
        self.error = torch.empty((1,), dtype=torch.int32, device=self.device)
        launch_fill(self.error, 0)
        for node, handler in self.handlers:
            env[node.name] = handler(env, node)
        outputs = []
        state_ptrs = {t.data_ptr() for t in self.state.values() if isinstance(t, torch.Tensor)}
        for out in self.graph.outputs:
            value = _value(env, out)
            aliased = isinstance(out, Ref) and out.name in inputs
            if isinstance(value, torch.Tensor) and (value.data_ptr() in state_ptrs or aliased):
                value = launch_copy(_empty(value.shape, value.dtype, self.device), value)
            outputs.append(value)
        if verify_index_bounds and int(self.error.item()) != 0:
            raise PlanInputError("an index input is out of range for the tensor it indexes",
                                 hint="embedding ids / gather indices must lie in [-size, size)")
        return tuple(outputs)

    # -- node handlers ----------------------------------------------------------------
    def _handler(self, node: Node) -> Callable:
        op = node.op
        if node.is_view:
            return self._view
        if op in UNARY_OPS:
            return self._unary
        if op in BINARY_OPS:
            return self._binary
        if op in REDUCE_OPS:
            return self._reduce
        if op in FILL_OPS:
            return self._fill
        if op in COPY_OPS:
            return self._cat if op == "aten.cat.default" else self._copy
        if op in MATMUL_OPS:
            return self._matmul
        if op in INDEX_OPS:
            return self._index
        if op in OTHER_OPS:
            return getattr(self, "_" + OTHER_OPS[op])
        raise CompilationError(f"node {node.name}: {op} has no gfx950 kernel in this backend",
                               hint="compile_callable/compile_module lower core-ATen graphs of the supported op set")

    def _out(self, node: Node) -> torch.Tensor:
        if node.shape is None or node.dtype is None:
            raise CompilationError(f"node {node.name} ({node.op}) has no static tensor output")
        return _empty(node.shape, node.dtype, self.device)

    def _view(self, env, node: Node):
        x = _value(env, node.args[0])
        rest = [_value(env, a) for a in node.args[1:]]
        op = node.op
        if op in ("aten.view.default", "aten._unsafe_view.default", "aten.reshape.default"):
            try:
                return x.view(node.shape)
            except RuntimeError:
                return _contiguous(x).view(node.shape)
        if op == "aten.permute.default":
            return x.permute(rest[0])
        if op == "aten.transpose.int":
            return x.transpose(rest[0], rest[1])
        if op == "aten.t.default":
            return x.t()
        if op == "aten.expand.default":
            return x.expand(node.shape)
        if op == "aten.slice.Tensor":
            dim = rest[0] if len(rest) > 0 else 0
            start = rest[1] if len(rest) > 1 else None
            end = rest[2] if len(rest) > 2 else None
            step = rest[3] if len(rest) > 3 else 1
            dim = dim % x.dim()
            index = [slice(None)] * x.dim()
            index[dim] = slice(start, end, step)
            return x[tuple(index)]
        if op == "aten.select.int":
            return x.select(rest[0], rest[1])
        if op == "aten.unsqueeze.default":
            return x.unsqueeze(rest[0])
        if op in ("aten.squeeze.dim", "aten.squeeze.dims", "aten.squeeze.default"):
            return x.view(node.shape)
        if op in ("aten.alias.default", "aten.detach.default"):
            return x
        if op == "aten.lift_fresh_copy.default":
            return launch_copy(self._out(node), x)
        raise CompilationError(f"view {op} is not handled")

    def _unary(self, env, node: Node):
        x = _value(env, node.args[0])
        name = UNARY_OPS[node.op]
        return launch_elementwise(EW[name], self._out(node), x)

    def _binary(self, env, node: Node):
        a = _value(env, node.args[0])
        b = _value(env, node.args[1])
        name = BINARY_OPS[node.op]
        alpha = node.kwargs.get("alpha", 1)
        if len(node.args) > 2 and name in ("add", "sub"):
            alpha = node.args[2]
        if name == "div" and node.dtype is not None and not node.dtype.is_floating_point:
            name = "div_trunc"
        return launch_elementwise(EW[name], self._out(node), a, b, alpha=alpha)

    def _rsub(self, env, node: Node):
        a = _value(env, node.args[0])
        b = _value(env, node.args[1])
        alpha = node.kwargs.get("alpha", 1)
        if alpha != 1:
            scaled = launch_elementwise(EW["mul"], self._out(node), a, alpha)
            return launch_elementwise(EW["sub"], self._out(node), b, scaled)
        return launch_elementwise(EW["sub"], self._out(node), b, a)

    def _div_mode(self, env, node: Node):
        a = _value(env, node.args[0])
        b = _value(env, node.args[1])
        mode = node.kwargs.get("rounding_mode")
        name = {"trunc": "div_trunc", "floor": "div_floor"}.get(mode, "div")
        return launch_elementwise(EW[name], self._out(node), a, b)

    def _gelu(self, env, node: Node):
        x = _value(env, node.args[0])
        approximate = node.kwargs.get("approximate", node.args[1] if len(node.args) > 1 else "none")
        return launch_elementwise(EW["gelu_tanh" if approximate == "tanh" else "gelu"], self._out(node), x)

    def _where(self, env, node: Node):
        cond, a, b = (_value(env, x) for x in node.args[:3])
        return launch_elementwise(EW["where"], self._out(node), cond, a, b)

    def _masked_fill(self, env, node: Node):
        x, mask, value = (_value(env, v) for v in node.args[:3])
        return launch_elementwise(EW["where"], self._out(node), mask, value, x)

    def _clamp(self, env, node: Node):
        x = _value(env, node.args[0])
        if node.op == "aten.clamp_min.default":
            lo, hi = _value(env, node.args[1]), None
        elif node.op == "aten.clamp_max.default":
            lo, hi = None, _value(env, node.args[1])
        else:
            lo = _value(env, node.args[1]) if len(node.args) > 1 else node.kwargs.get("min")
            hi = _value(env, node.args[2]) if len(node.args) > 2 else node.kwargs.get("max")
        out = x
        if lo is not None:
            out = launch_elementwise(EW["maximum"], self._out(node), out, lo)
        if hi is not None:
            out = launch_elementwise(EW["minimum"], self._out(node), out, hi)
        if out is x:
            out = launch_copy(self._out(node), x)
        return out

    def _fill(self, env, node: Node):
        op = node.op
        out = self._out(node)
        args = [_value(env, a) for a in node.args]
        if op.startswith("aten.arange"):
            if op == "aten.arange.default":
                start, step = 0, 1
            elif op == "aten.arange.start":
                start, step = args[0], 1
            else:
                start = args[0]
                step = args[2] if len(args) > 2 else node.kwargs.get("step", 1)
            return launch_fill(out, start, step)
        if op in ("aten.full.default",):
            value = args[1]
        elif op in ("aten.full_like.default", "aten.new_full.default"):
            value = args[1] if op == "aten.full_like.default" else args[2]
        elif op == "aten.scalar_tensor.default":
            value = args[0]
        elif "ones" in op:
            value = 1
        else:
            value = 0
        if isinstance(value, bool):
            value = int(value)
        return launch_fill(out, value)

    def _copy(self, env, node: Node):
        src = _value(env, node.args[0])
        if node.op == "aten.copy.default":
            src = _value(env, node.args[1])
        out = self._out(node)
        if tuple(src.shape) != tuple(out.shape):
            src = src.expand(out.shape)
        return launch_copy(out, src)

    def _cat(self, env, node: Node):
        parts = [_value(env, a) for a in node.args[0]]
        dim = node.args[1] if len(node.args) > 1 else node.kwargs.get("dim", 0)
        out = self._out(node)
        dim = dim % out.dim()
        offset = 0
        for part in parts:
            if part.dim() == 1 and part.shape[0] == 0 and out.dim() > 1:
                continue  # torch's legacy empty-tensor rule
            size = part.shape[dim]
            if size:
                launch_copy(out.narrow(dim, offset, size), part)
            offset += size
        return out

    #: reductions whose second argument lists the reduced dims (the others reduce everything)
    _DIM_REDUCTIONS = frozenset({"aten.sum.dim_IntList", "aten.mean.dim", "aten.amax.default", "aten.amin.default",
                                 "aten.any.dim", "aten.any.dims", "aten.all.dim", "aten.all.dims"})

    def _reduce(self, env, node: Node):
        x = _value(env, node.args[0])
        name = REDUCE_OPS[node.op]
        rank = x.dim()
        if name in ("argmax", "argmin"):
            dim = node.args[1] if len(node.args) > 1 else node.kwargs.get("dim")
            dims = list(range(rank)) if dim is None else [dim % max(rank, 1)]
        elif node.op in self._DIM_REDUCTIONS:
            raw = node.args[1] if len(node.args) > 1 else node.kwargs.get("dim")
            if raw is None or (isinstance(raw, (list, tuple)) and len(raw) == 0):
                dims = list(range(rank))
            else:
                dims = sorted({d % max(rank, 1) for d in (raw if isinstance(raw, (list, tuple)) else [raw])})
        else:
            dims = list(range(rank))
        if rank == 0:
            x = x.reshape(1)
            dims = [0]
        keep = [d for d in range(x.dim()) if d not in dims]
        length = 1
        for d in dims:
            length *= x.shape[d]
        moved = _contiguous(x.permute(keep + dims))
        rows = moved.view([x.shape[d] for d in keep] + [length])
        out = self._out(node)
        launch_reduce(RED[name], out, rows)
        return out

    def _scan_like(self, env, node: Node, name: str):
        x = _value(env, node.args[0])
        dim = (node.args[1] if len(node.args) > 1 else node.kwargs.get("dim", -1)) % max(1, x.dim())
        out = self._out(node)
        if x.dim() == 0:
            return launch_reduce(RED[name], out.view(1, 1), x.reshape(1, 1))
        order = [d for d in range(x.dim()) if d != dim] + [dim]
        moved = x.permute(order)
        moved_out = out.permute(order)
        if moved_out.is_contiguous():
            src = moved if moved.is_contiguous() else _contiguous(moved)
            launch_reduce(RED[name], moved_out, src)
            return out
        tmp = _empty(moved.shape, out.dtype, self.device)
        launch_reduce(RED[name], tmp, _contiguous(moved))
        launch_copy(moved_out, tmp)
        return out

    def _softmax(self, env, node: Node):
        return self._scan_like(env, node, "softmax")

    def _log_softmax(self, env, node: Node):
        return self._scan_like(env, node, "log_softmax")

    def _cumsum(self, env, node: Node):
        return self._scan_like(env, node, "cumsum")

    def _matmul(self, env, node: Node):
        out = self._out(node)
        op = node.op
        if op == "aten.mm.default":
            a, b = (_value(env, x) for x in node.args[:2])
            launch_matmul(out.unsqueeze(0), a.unsqueeze(0), b.unsqueeze(0))
            return out
        if op == "aten.bmm.default":
            a, b = (_value(env, x) for x in node.args[:2])
            launch_matmul(out, a, b)
            return out
        bias, a, b = (_value(env, x) for x in node.args[:3])
        beta = node.kwargs.get("beta", 1)
        alpha = node.kwargs.get("alpha", 1)
        if op == "aten.addmm.default":
            bias3 = bias.unsqueeze(0) if isinstance(bias, torch.Tensor) else bias
            if not isinstance(bias3, torch.Tensor):
                raise CompilationError("addmm with a scalar bias is not lowered")
            launch_matmul(out.unsqueeze(0), a.unsqueeze(0), b.unsqueeze(0), bias3, alpha, beta)
            return out
        launch_matmul(out, a, b, bias, alpha, beta)
        return out

    def _index(self, env, node: Node):
        out = self._out(node)
        if node.op == "aten.embedding.default":
            weight, ids = (_value(env, x) for x in node.args[:2])
            return launch_index(out, _contiguous(weight), [ids], self.error)
        if node.op == "aten.index_select.default":
            x, dim, idx = (_value(env, a) for a in node.args[:3])
            indices = [None] * (dim % x.dim()) + [idx]
        else:
            x = _value(env, node.args[0])
            indices = list(_value(env, node.args[1]))
        positions = [i for i, ix in enumerate(indices) if ix is not None]
        if not positions:
            return launch_copy(out, x)
        if any(ix.dtype == torch.bool for ix in indices if ix is not None):
            raise CompilationError("boolean mask indexing has a data-dependent shape")
        adjacent = positions == list(range(positions[0], positions[-1] + 1))
        rest = [d for d in range(x.dim()) if d not in positions]
        src = _contiguous(x.permute(positions + rest))
        tensors = [indices[i] for i in positions]
        bshape = torch.broadcast_shapes(*[t.shape for t in tensors])
        gathered_shape = list(bshape) + [x.shape[d] for d in rest]
        if adjacent and positions[0] > 0:
            # torch keeps the indexed block where it was: [pre, bshape, post]
            tmp = _empty(gathered_shape, x.dtype, self.device)
            launch_index(tmp, src, tensors, self.error)
            nb, pre = len(bshape), positions[0]
            order = list(range(nb, nb + pre)) + list(range(nb)) + list(range(nb + pre, len(gathered_shape)))
            return launch_copy(out, tmp.permute(order))
        return launch_index(out.view(gathered_shape), src, tensors, self.error)

    def _rms_norm(self, env, node: Node):
        x, weight, eps, mid_dtype = node.args
        x = _contiguous(_value(env, x))
        weight = None if weight is None else _contiguous(_value(env, weight))
        return launch_rms_norm(self._out(node), x, weight, eps, mid_dtype)

    def _attention(self, env, node: Node):
        q, k, v = (_value(env, x) for x in node.args[:3])
        names = ("attn_mask", "dropout_p", "is_causal", "scale", "enable_gqa")
        extra = dict(zip(names, [_value(env, a) for a in node.args[3:]]))
        extra.update({key: _value(env, val) for key, val in node.kwargs.items()})
        mask = extra.get("attn_mask")
        if extra.get("dropout_p", 0.0):
            raise CompilationError("attention dropout is not part of an inference plan")
        scale = extra.get("scale")
        if scale is None:
            scale = 1.0 / math.sqrt(q.shape[-1])
        out = self._out(node)
        if q.dim() != 4:
            raise CompilationError("attention lowers 4-D [batch, heads, tokens, dim] operands")
        return launch_attention(out, q, k, v, mask, bool(extra.get("is_causal", False)), scale)


def build_graph_plan(graph: LoweredGraph, name: str = "graph") -> tuple[CompiledPlan, GraphRunner]:
    """A :class:`CompiledPlan` whose nodes are the graph's kernel launches."""

    if not torch.cuda.is_available():
        from .errors import DeviceError

        raise DeviceError("the hip-gfx950 target needs a ROCm GPU (MI355X, gfx950); none is visible",
                          hint="run on the GPU host")
    device = torch.device("cuda", torch.cuda.current_device())
    _lib.ensure_code_object(device.index)
    runner = GraphRunner(graph, device)
    selections = runner.selections(torch.cuda.get_device_name(device))

    def run(*inputs, verify_index_bounds: bool = True, memory: str = "latency"):
        if len(inputs) != len(graph.inputs):
            raise PlanInputError(f"expected {len(graph.inputs)} inputs, received {len(inputs)}")
        bound = {}
        for key, value in zip(graph.inputs, inputs):
            shape, dtype = graph.input_meta[key]
            if not isinstance(value, torch.Tensor):
                value = torch.as_tensor(value)
            if tuple(value.shape) != shape or value.dtype != dtype:
                raise PlanInputError(f"input {key!r}: expected {dtype} {shape}, got {value.dtype} "
                                     f"{tuple(value.shape)}", hint="a compiled plan has static shapes")
            bound[key] = value.to(device)
        return runner.run(bound, verify_index_bounds=verify_index_bounds)

    plan = CompiledPlan(name, tuple(PlanNode(s) for s in selections), run, input_names=tuple(graph.inputs),
                        output_names=tuple(o.name if isinstance(o, Ref) else str(o) for o in graph.outputs))
    return plan, runner
