"""Graph capture and legalization for ``compile_callable`` / ``compile_module``.

The reference traces a callable or module into its own IR
(``frontend`` capture, ``compiler.py:301-405``), rewrites it
(``passes/driver.py``, legalizers such as the RMSNorm chain and SDPA of
``legalize/attention.py:105-170, 332-525``) and lowers every node to a kernel
or an MLX op. Here the capture is ``torch.export`` followed by the core-ATen
decompositions (SDPA kept whole), and the result is a flat, static-shape
:class:`LoweredGraph` of :class:`Node` records in ATen vocabulary. Two
legalizations fold patterns into one node each:

* ``aoto.rms_norm`` - the HF RMSNorm chain ``w * cast(x * rsqrt(mean(x^2) + eps))``;
* ``aten.scaled_dot_product_attention`` stays one node (not decomposed into
  bmm/softmax/bmm).

Nothing here touches a GPU: capture and legalization run on the CPU, and the
graph is what both the gfx950 lowering (``graph_ops``) and the CPU oracle
interpret.
"""

from __future__ import annotations

import operator
from dataclasses import dataclass, field
from typing import Any

import torch

from .errors import CompilationError

#: Node ops whose output is a view of an input (metadata only, no kernel).
VIEW_OPS = frozenset({
    "aten.view.default", "aten._unsafe_view.default", "aten.reshape.default", "aten.permute.default",
    "aten.transpose.int", "aten.t.default", "aten.expand.default", "aten.slice.Tensor", "aten.select.int",
    "aten.unsqueeze.default", "aten.squeeze.dim", "aten.squeeze.dims", "aten.squeeze.default",
    "aten.alias.default", "aten.detach.default", "aten.lift_fresh_copy.default",
})

#: Node ops that only assert and produce nothing.
NO_OPS = frozenset({"aten._assert_tensor_metadata.default", "aten._assert_scalar.default",
                    "aten.sym_constrain_range_for_size.default"})

RMS_NORM = "aoto.rms_norm"


@dataclass(frozen=True)
class Ref:
    """A reference to a graph value (an input, a bound state tensor or a node output)."""

    name: str


@dataclass
class Node:
    name: str
    op: str
    args: tuple
    kwargs: dict
    shape: tuple[int, ...] | None
    dtype: torch.dtype | None

    @property
    def is_view(self) -> bool:
        return self.op in VIEW_OPS


@dataclass
class LoweredGraph:
    """A static-shape graph: user inputs, bound state, nodes in order, outputs."""

    inputs: list[str]
    input_meta: dict[str, tuple[tuple[int, ...], torch.dtype]]
    state_names: list[str]
    state: dict[str, torch.Tensor]
    nodes: list[Node]
    outputs: list[Any]
    #: user-facing names of the bound state (module parameter / buffer names)
    state_labels: dict[str, str] = field(default_factory=dict)

    def describe(self) -> str:
        lines = [f"inputs: {', '.join(self.inputs)}"]
        for node in self.nodes:
            lines.append(f"  {node.name} = {node.op}{node.args} -> {node.shape} {node.dtype}")
        lines.append(f"outputs: {self.outputs}")
        return "\n".join(lines)


def _op_name(target) -> str:
    if target is operator.getitem:
        return "getitem"
    if isinstance(target, torch._ops.OpOverload):
        return f"aten.{target._opname}.{target._overloadname}" if target.namespace == "aten" else str(target)
    return getattr(target, "__name__", str(target))


def _decompositions():
    table = torch.export.default_decompositions()
    for key in list(table):
        if "scaled_dot_product" in str(key):
            table.pop(key)
    return table


class _CallableModule(torch.nn.Module):
    def __init__(self, fn):
        super().__init__()
        self.fn = fn

    def forward(self, *args):
        return self.fn(*args)


def export_program(fn_or_module, example_inputs, kwargs=None):
    """``torch.export`` the callable/module on its example inputs, then decompose to core ATen."""

    module = fn_or_module if isinstance(fn_or_module, torch.nn.Module) else _CallableModule(fn_or_module)
    try:
        with torch.no_grad():
            program = torch.export.export(module, tuple(example_inputs), kwargs or {}, strict=False)
            program = program.run_decompositions(_decompositions())
    except Exception as error:  # noqa: BLE001 - report capture failures as compile errors
        raise CompilationError(
            f"could not capture the graph: {type(error).__name__}: {error}",
            hint="compile_callable/compile_module need a static-shape, data-independent forward",
        ) from error
    return program


# ----------------------------------------------------------------------------- legalization
def _single_user(node) -> bool:
    return len(node.users) == 1


def _is(node, name: str) -> bool:
    return getattr(node, "op", None) == "call_function" and _op_name(node.target) == name


def _scalar_arg(node, index: int):
    value = node.args[index] if len(node.args) > index else None
    return value if isinstance(value, (int, float)) else None


def _rms_norm_marker(x, weight, eps, mid_dtype):  # pragma: no cover - a graph marker, never called
    raise RuntimeError("aoto.rms_norm is a graph marker")


_rms_norm_marker.__name__ = RMS_NORM


def fold_rms_norm(graph: torch.fx.Graph) -> int:
    """Fold ``w * cast(x * rsqrt(mean(x^2, -1, keepdim) + eps))`` chains; return how many.

    The chain is the one HF's Llama/Qwen2 RMSNorm modules trace to
    (``legalize/attention.py:332-525`` matches the same shape). Intermediate
    nodes must feed only the chain; the normalized input may have other users.
    """

    folded = 0
    for mean in list(graph.nodes):
        if not _is(mean, "aten.mean.dim") or not _single_user(mean):
            continue
        dims = mean.args[1] if len(mean.args) > 1 else mean.kwargs.get("dim")
        keepdim = mean.args[2] if len(mean.args) > 2 else mean.kwargs.get("keepdim", False)
        rank = len(mean.meta["val"].shape)
        if not keepdim or list(dims) not in ([-1], [rank - 1]):
            continue
        square = mean.args[0]
        if not (_is(square, "aten.pow.Tensor_Scalar") and _scalar_arg(square, 1) == 2 and _single_user(square)):
            continue
        x32 = square.args[0]
        add = next(iter(mean.users))
        if not (_is(add, "aten.add.Tensor") or _is(add, "aten.add.Scalar")) or not _single_user(add):
            continue
        eps = _scalar_arg(add, 1)
        if eps is None or add.args[0] is not mean:
            continue
        rsqrt = next(iter(add.users))
        if not _is(rsqrt, "aten.rsqrt.default") or not _single_user(rsqrt):
            continue
        scaled = next(iter(rsqrt.users))
        if not _is(scaled, "aten.mul.Tensor") or set(scaled.args[:2]) != {x32, rsqrt}:
            continue
        x_val = x32.meta["val"]
        if x_val.dtype != torch.float32:
            continue
        tail = scaled
        mid_dtype = torch.float32
        if _single_user(tail):
            user = next(iter(tail.users))
            if _is(user, "aten._to_copy.default") and set(user.kwargs) <= {"dtype"} and len(user.args) == 1:
                tail = user
                mid_dtype = user.kwargs.get("dtype", torch.float32)
        weight = None
        if _single_user(tail):
            user = next(iter(tail.users))
            if _is(user, "aten.mul.Tensor"):
                other = user.args[0] if user.args[1] is tail else user.args[1]
                other_val = getattr(other, "meta", {}).get("val")
                hidden = x_val.shape[-1]
                if isinstance(other_val, torch.Tensor) and tuple(other_val.shape) == (hidden,) \
                        and other_val.dtype in (torch.float32, torch.bfloat16):
                    weight = other
                    tail = user
        # source of the normalized value: the pre-cast input when x32 is an f32 cast
        source = x32
        if _is(x32, "aten._to_copy.default") and set(x32.kwargs) <= {"dtype"} \
                and x32.args[0].meta["val"].dtype in (torch.float32, torch.bfloat16):
            source = x32.args[0]
        with graph.inserting_after(tail):
            fused = graph.call_function(_rms_norm_marker, (source, weight, float(eps), mid_dtype))
        fused.meta["val"] = tail.meta["val"]
        tail.replace_all_uses_with(fused)
        graph.eliminate_dead_code()
        folded += 1
    return folded


# ----------------------------------------------------------------------------- conversion
def _convert(value, names: dict):
    if isinstance(value, torch.fx.Node):
        return Ref(names[value.name])
    if isinstance(value, (list, tuple)):
        return type(value)(_convert(v, names) for v in value)
    if isinstance(value, dict):
        return {k: _convert(v, names) for k, v in value.items()}
    return value


def lower_program(program) -> LoweredGraph:
    """Legalize an exported program and convert it to a :class:`LoweredGraph`."""

    from torch.export.graph_signature import InputKind

    gm = program.graph_module
    graph = gm.graph
    # metadata asserts only restate what the node metadata already holds
    for node in list(graph.nodes):
        if node.op == "call_function" and _op_name(node.target) in NO_OPS and not node.users:
            graph.erase_node(node)
    fold_rms_norm(graph)
    graph.eliminate_dead_code()

    sig = program.graph_signature
    kinds = {spec.arg.name: spec for spec in sig.input_specs}
    inputs: list[str] = []
    input_meta: dict = {}
    state_names: list[str] = []
    state: dict[str, torch.Tensor] = {}
    labels: dict[str, str] = {}
    names: dict[str, str] = {}
    nodes: list[Node] = []
    outputs: list = []
    for node in graph.nodes:
        names[node.name] = node.name
        if node.op == "placeholder":
            spec = kinds[node.name]
            val = node.meta.get("val")
            if spec.kind == InputKind.USER_INPUT:
                if not isinstance(val, torch.Tensor):
                    raise CompilationError(f"input {node.name!r} is not a tensor",
                                           hint="pass non-tensor arguments as static keywords")
                inputs.append(node.name)
                input_meta[node.name] = (tuple(int(d) for d in val.shape), val.dtype)
            else:
                target = spec.target
                if spec.kind in (InputKind.PARAMETER, InputKind.BUFFER):
                    tensor = program.state_dict[target] if target in program.state_dict else program.constants[target]
                else:
                    tensor = program.constants[target]
                state_names.append(node.name)
                state[node.name] = tensor.detach()
                labels[node.name] = target
        elif node.op == "call_function":
            op = _op_name(node.target)
            if op in NO_OPS:
                continue
            val = node.meta.get("val")
            shape = tuple(int(d) for d in val.shape) if isinstance(val, torch.Tensor) else None
            dtype = val.dtype if isinstance(val, torch.Tensor) else None
            if isinstance(val, (tuple, list)):
                shape, dtype = None, None
            nodes.append(Node(node.name, op, _convert(tuple(node.args), names), _convert(dict(node.kwargs), names),
                              shape, dtype))
        elif node.op == "output":
            outputs = list(_convert(node.args[0], names))
        elif node.op == "get_attr":
            raise CompilationError(f"unexpected get_attr node {node.name}")
    return LoweredGraph(inputs, input_meta, state_names, state, nodes, outputs, labels)


def capture(fn_or_module, example_inputs, kwargs=None) -> LoweredGraph:
    return lower_program(export_program(fn_or_module, example_inputs, kwargs))
