"""Oracle interpreter of a captured graph (test infrastructure only).

A NumPy restatement of the per-node semantics the reference's ``mlx-reference``
target executes (``runtime/mlx_ops/__init__.py:239-620``; attention
``runtime/mlx_ops/attention.py:89-122``; RMSNorm
``runtime/mlx_ops/normalization.py:73-119``) over the node records of a
``LoweredGraph`` (``aotolith_amd.graph``): ATen op names, static shapes and
dtypes recorded at capture. Float work is f32 with one rounding per node to
the node's element type (bf16 by round-to-nearest-even), reductions accumulate
in f64 and round once, integer work is int64. It is the checker of the gfx950
graph lowering, never part of it.

Pinning: ``tests/test_graph_capture.py`` runs this interpreter against torch's
own CPU execution of every captured test function and of the tiny Llama /
Qwen2 modules (independent implementations), so a wrong broadcast, dtype rule,
index placement or rounding point fails there.
"""

from __future__ import annotations

import math

import numpy as np

from .bf16 import round_bf16

_NP = {"torch.float32": np.float32, "torch.bfloat16": np.float32, "torch.int64": np.int64, "torch.int32": np.int32,
       "torch.bool": np.bool_, "torch.uint8": np.uint8, "torch.int8": np.int8}
_FLOAT = {"torch.float32", "torch.bfloat16"}


def _is_ref(x) -> bool:
    return type(x).__name__ == "Ref"


def _cast(values, dtype) -> np.ndarray:
    """Round/convert to a torch dtype's values (bf16 kept as f32 bf16 values; float -> int truncates)."""

    key = str(dtype)
    arr = np.asarray(values)
    if key == "torch.bfloat16":
        return round_bf16(arr.astype(np.float32))
    if key == "torch.float32":
        return arr.astype(np.float32)
    if key == "torch.bool":
        return arr != 0
    if np.issubdtype(arr.dtype, np.floating):
        arr = np.trunc(arr)
    return arr.astype(_NP[key])


def _f32(x) -> np.ndarray:
    return np.asarray(x).astype(np.float32) if not isinstance(x, (int, float, bool)) else np.float32(x)


def _pow(a, e):
    if isinstance(e, (int, float)) and float(e) == 2.0:
        return a * a
    return np.power(a, e)


_UNARY = {
    "neg": lambda x: -x, "abs": np.abs, "reciprocal": lambda x: np.float32(1.0) / x, "sqrt": np.sqrt,
    "rsqrt": lambda x: np.float32(1.0) / np.sqrt(x), "exp": np.exp, "log": np.log,
    "sigmoid": lambda x: np.float32(1.0) / (np.float32(1.0) + np.exp(-x)),
    "silu": lambda x: x / (np.float32(1.0) + np.exp(-x)), "tanh": np.tanh, "cos": np.cos, "sin": np.sin,
    "relu": lambda x: np.maximum(x, np.float32(0)), "floor": np.floor, "ceil": np.ceil, "log1p": np.log1p,
    "expm1": np.expm1,
}
_BINARY_F = {
    "add": lambda a, b: a + b, "sub": lambda a, b: a - b, "mul": lambda a, b: a * b, "div": lambda a, b: a / b,
    "pow": _pow, "maximum": np.maximum, "minimum": np.minimum,
    "remainder": lambda a, b: a - np.floor(a / b) * b,
}
_BINARY_I = {
    "add": lambda a, b: a + b, "sub": lambda a, b: a - b, "mul": lambda a, b: a * b,
    "maximum": np.maximum, "minimum": np.minimum, "bitwise_and": lambda a, b: a & b,
    "bitwise_or": lambda a, b: a | b, "bitwise_xor": lambda a, b: a ^ b,
    "logical_and": lambda a, b: (a != 0) & (b != 0), "logical_or": lambda a, b: (a != 0) | (b != 0),
    "remainder": lambda a, b: np.mod(a, b), "div": lambda a, b: np.trunc(a / b),
}
_COMPARE = {"eq": np.equal, "ne": np.not_equal, "lt": np.less, "le": np.less_equal, "gt": np.greater,
            "ge": np.greater_equal}


def _op_parts(op: str) -> tuple[str, str]:
    parts = op.split(".")
    return (parts[1], parts[2]) if op.startswith("aten.") else (op, "")


class GraphOracle:
    """Interprets ``graph.nodes`` over NumPy arrays."""

    def __init__(self, graph):
        self.graph = graph

    def run(self, inputs: dict, state: dict | None = None):
        env = {}
        for name, value in (state if state is not None else self.graph.state).items():
            env[name] = self._host(value)
        for name, value in inputs.items():
            env[name] = self._host(value)
        for node in self.graph.nodes:
            env[node.name] = self.node(env, node)
        return tuple(self._get(env, o) for o in self.graph.outputs)

    @staticmethod
    def _host(value):
        if hasattr(value, "detach"):
            import torch

            t = value.detach().cpu()
            if t.dtype == torch.bfloat16:
                return t.float().numpy()
            return t.numpy()
        return np.asarray(value)

    def _get(self, env, x):
        if _is_ref(x):
            return env[x.name]
        if isinstance(x, (list, tuple)):
            return type(x)(self._get(env, v) for v in x)
        return x

    # ------------------------------------------------------------------ one node
    def node(self, env, node):  # noqa: C901 - one dispatch table, read top to bottom
        name, overload = _op_parts(node.op)
        args = [self._get(env, a) for a in node.args]
        kw = {k: self._get(env, v) for k, v in node.kwargs.items()}
        out_dt = str(node.dtype) if node.dtype is not None else None
        shape = node.shape
        # views
        if name in ("view", "_unsafe_view", "reshape"):
            return np.reshape(args[0], shape)
        if name == "permute":
            return np.transpose(args[0], args[1])
        if name == "transpose":
            return np.swapaxes(args[0], args[1], args[2])
        if name == "t":
            return np.transpose(args[0])
        if name == "expand":
            return np.broadcast_to(args[0], shape)
        if name == "slice":
            x = args[0]
            dim = (args[1] if len(args) > 1 else 0) % x.ndim
            start = args[2] if len(args) > 2 else None
            end = args[3] if len(args) > 3 else None
            step = args[4] if len(args) > 4 else 1
            index = [slice(None)] * x.ndim
            index[dim] = slice(start, end, step)
            return x[tuple(index)]
        if name == "select":
            return np.take(args[0], args[2], axis=args[1])
        if name == "unsqueeze":
            return np.expand_dims(args[0], args[1] % (np.ndim(args[0]) + 1))
        if name == "squeeze":
            return np.reshape(args[0], shape)
        if name in ("alias", "detach", "lift_fresh_copy", "clone", "contiguous"):
            return np.array(args[0], copy=True)
        # casts and copies
        if name == "_to_copy":
            return _cast(args[0], node.dtype)
        if name == "copy":
            return _cast(np.broadcast_to(args[1], shape), node.dtype)
        if name == "cat":
            dim = args[1] if len(args) > 1 else kw.get("dim", 0)
            parts = [p for p in args[0] if not (np.ndim(p) == 1 and np.shape(p)[0] == 0)]
            return _cast(np.concatenate(parts, axis=dim), node.dtype)
        # fills
        if name == "arange":
            if overload == "default":
                start, step = 0, 1
            elif overload == "start":
                start, step = args[0], 1
            else:
                start, step = args[0], (args[2] if len(args) > 2 else kw.get("step", 1))
            n = int(np.prod(shape))
            return _cast(np.float64(start) + np.arange(n, dtype=np.float64) * step, node.dtype)
        if name in ("full", "full_like", "new_full", "scalar_tensor", "zeros", "zeros_like", "ones", "ones_like",
                    "empty", "empty_like", "new_zeros", "new_ones", "new_empty"):
            value = {"full": lambda: args[1], "full_like": lambda: args[1], "new_full": lambda: args[2],
                     "scalar_tensor": lambda: args[0]}.get(name, lambda: 1 if "ones" in name else 0)()
            return _cast(np.full(shape, float(value)), node.dtype)
        # elementwise
        if name in _UNARY:
            if out_dt in _FLOAT:
                return _cast(_UNARY[name](_f32(args[0])), node.dtype)
            if name == "neg":
                return _cast(-np.asarray(args[0]).astype(np.int64), node.dtype)
            if name == "abs":
                return _cast(np.abs(np.asarray(args[0]).astype(np.int64)), node.dtype)
        if name == "logical_not":
            return np.asarray(args[0]) == 0
        if name == "bitwise_not":
            a = np.asarray(args[0])
            return ~a if a.dtype != np.bool_ else ~a
        if name == "isnan":
            return np.isnan(_f32(args[0]))
        if name == "erf":
            return _cast(np.vectorize(math.erf, otypes=[np.float64])(_f32(args[0])), node.dtype)
        if name == "gelu":
            x = _f32(args[0]).astype(np.float64)
            approximate = kw.get("approximate", args[1] if len(args) > 1 else "none")
            if approximate == "tanh":
                y = 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))
            else:
                y = 0.5 * x * (1.0 + np.vectorize(math.erf)(x / math.sqrt(2.0)))
            return _cast(y, node.dtype)
        if name in _COMPARE:
            a, b = args[0], args[1]
            return _COMPARE[name](np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64))
        if name == "rsub":
            alpha = kw.get("alpha", 1)
            return self._binary("sub", args[1], args[0] if alpha == 1 else np.asarray(args[0]) * alpha, out_dt,
                                node.dtype)
        if name == "div" and overload == "Tensor_mode":
            mode = kw.get("rounding_mode")
            q = np.asarray(args[0], dtype=np.float64) / np.asarray(args[1], dtype=np.float64)
            if out_dt in _FLOAT:
                q = _f32(args[0]) / _f32(args[1])
            q = np.trunc(q) if mode == "trunc" else (np.floor(q) if mode == "floor" else q)
            return _cast(q, node.dtype)
        if name in _BINARY_F or name in _BINARY_I:
            alpha = kw.get("alpha", args[2] if len(args) > 2 and name in ("add", "sub") else 1)
            b = args[1]
            if alpha != 1:
                b = np.asarray(b) * alpha
            return self._binary(name, args[0], b, out_dt, node.dtype)
        if name == "where":
            return _cast(np.where(np.asarray(args[0]) != 0, args[1], args[2]), node.dtype)
        if name == "masked_fill":
            return _cast(np.where(np.asarray(args[1]) != 0, args[2], args[0]), node.dtype)
        if name in ("clamp", "clamp_min", "clamp_max"):
            x = _f32(args[0]) if out_dt in _FLOAT else np.asarray(args[0])
            lo = args[1] if name in ("clamp", "clamp_min") and len(args) > 1 else kw.get("min")
            hi = (args[2] if len(args) > 2 else kw.get("max")) if name == "clamp" else (
                args[1] if name == "clamp_max" else None)
            if lo is not None:
                x = np.maximum(x, lo)
            if hi is not None:
                x = np.minimum(x, hi)
            return _cast(x, node.dtype)
        # reductions
        if name in ("sum", "mean", "amax", "amin", "any", "all", "argmax", "argmin"):
            return self._reduce(name, overload, args, kw, node)
        if name in ("_softmax", "_log_softmax"):
            x = _f32(args[0])
            dim = args[1]
            m = np.max(x, axis=dim, keepdims=True)
            e = np.exp(x - m)
            s = e.sum(axis=dim, keepdims=True, dtype=np.float32)
            y = e / s if name == "_softmax" else (x - m) - np.log(s)
            return _cast(y, node.dtype)
        if name == "cumsum":
            dim = args[1]
            x = np.asarray(args[0])
            if out_dt in _FLOAT:
                return _cast(np.cumsum(x.astype(np.float64), axis=dim), node.dtype)
            return _cast(np.cumsum(x.astype(np.int64), axis=dim), node.dtype)
        # products
        if name in ("mm", "bmm"):
            return _cast(np.matmul(np.asarray(args[0], np.float64), np.asarray(args[1], np.float64)), node.dtype)
        if name in ("addmm", "baddbmm"):
            beta, alpha = kw.get("beta", 1), kw.get("alpha", 1)
            prod = np.matmul(np.asarray(args[1], np.float64), np.asarray(args[2], np.float64))
            return _cast(beta * np.asarray(args[0], np.float64) + alpha * prod, node.dtype)
        # indexing
        if name == "embedding":
            return np.asarray(args[0])[np.asarray(args[1])]
        if name == "index_select":
            return np.take(args[0], np.asarray(args[2]), axis=args[1])
        if name == "index" and overload == "Tensor":
            x = np.asarray(args[0])
            index = tuple(slice(None) if ix is None else np.asarray(ix) for ix in args[1])
            return x[index]
        # legalized patterns
        if node.op == "aoto.rms_norm":
            x, weight, eps, mid = args
            x32 = _f32(x)
            ms = (x32.astype(np.float64) ** 2).mean(axis=-1, keepdims=True).astype(np.float32)
            y = x32 * (np.float32(1.0) / np.sqrt(ms + np.float32(eps)))
            y = _cast(y, mid)
            if weight is not None:
                y = _f32(weight) * y
            return _cast(y, node.dtype)
        if name == "scaled_dot_product_attention":
            return self._attention(args, kw, node)
        raise NotImplementedError(f"oracle has no rule for {node.op}")

    def _binary(self, name, a, b, out_dt, dtype):
        if out_dt in _FLOAT:
            return _cast(_BINARY_F[name](_f32(a), _f32(b)), dtype)
        ai = np.asarray(a).astype(np.int64)
        bi = np.asarray(b).astype(np.int64)
        return _cast(_BINARY_I[name](ai, bi), dtype)

    def _reduce(self, name, overload, args, kw, node):
        x = np.asarray(args[0])
        if name in ("argmax", "argmin"):
            dim = args[1] if len(args) > 1 else kw.get("dim")
            keep = args[2] if len(args) > 2 else kw.get("keepdim", False)
            f = np.argmax if name == "argmax" else np.argmin
            r = f(x.reshape(-1)) if dim is None else f(x, axis=dim)
            return np.reshape(np.asarray(r, dtype=np.int64), node.shape)
        if overload in ("dim_IntList", "dim", "dims") or name in ("amax", "amin"):
            dims = args[1] if len(args) > 1 else kw.get("dim")
        else:
            dims = None
        if isinstance(dims, int):
            dims = [dims]
        axis = None if dims is None or len(dims) == 0 else tuple(d % max(x.ndim, 1) for d in dims)
        if name in ("any", "all"):
            r = (np.any if name == "any" else np.all)(x != 0, axis=axis)
        elif name in ("amax", "amin"):
            r = (np.max if name == "amax" else np.min)(x, axis=axis)
        elif str(node.dtype) in _FLOAT:
            total = np.sum(np.asarray(x, np.float64), axis=axis)
            if name == "mean":
                count = x.size if axis is None else int(np.prod([x.shape[a] for a in axis]))
                total = total / count
            r = total
        else:
            r = np.sum(x.astype(np.int64), axis=axis)
        return _cast(np.reshape(r, node.shape), node.dtype)

    def _attention(self, args, kw, node):
        names = ("attn_mask", "dropout_p", "is_causal", "scale", "enable_gqa")
        extra = dict(zip(names, args[3:]))
        extra.update(kw)
        q, k, v = (np.asarray(a, np.float64) for a in args[:3])
        b, h, lq, d = q.shape
        hk, lk = k.shape[1], k.shape[2]
        scale = extra.get("scale") or 1.0 / math.sqrt(d)
        group = h // hk
        k = np.repeat(k, group, axis=1)
        v = np.repeat(v, group, axis=1)
        scores = np.einsum("bhqd,bhkd->bhqk", q, k) * scale
        keep = np.ones((b, h, lq, lk), dtype=bool)
        mask = extra.get("attn_mask")
        if mask is not None:
            mask = np.broadcast_to(np.asarray(mask), (b, h, lq, lk))
            if mask.dtype == np.bool_:
                keep &= mask
            else:
                scores = scores + mask.astype(np.float64)
        if extra.get("is_causal"):
            keep &= np.tril(np.ones((lq, lk), dtype=bool))[None, None]
        scores = np.where(keep, scores, -np.inf)
        m = scores.max(axis=-1, keepdims=True)
        m = np.where(np.isfinite(m), m, 0.0)
        e = np.where(keep, np.exp(scores - m), 0.0)
        s = e.sum(axis=-1, keepdims=True)
        p = np.where(s > 0, e / np.where(s > 0, s, 1.0), 0.0)
        return _cast(np.einsum("bhqk,bhkd->bhqd", p, v), node.dtype)
