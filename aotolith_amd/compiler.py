"""``compile_callable`` and ``compile_module`` for ``target="hip-gfx950"``.

Mirror of the reference's entry points (``compiler.py:301-405``): a callable
or an ``nn.Module`` with example inputs is captured once, legalized, and lowered
to a :class:`~aotolith_amd.plan.CompiledPlan` whose every node is a gfx950
kernel (``graph_ops``). A module's parameters and buffers become bound plan
state on the GPU, so the plan does not keep the module; Python keyword values
are baked in at compile time and tensor keyword values become named inputs
(``compiler.py:356-404``). The plan's call returns a tuple of device tensors,
as the reference's returns a tuple of arrays.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping, Sequence
from dataclasses import dataclass, field
from typing import Any

import torch

from .backends import backend_for
from .errors import CompilationError, PlanInputError
from .graph import LoweredGraph, capture
from .plan import TARGET, CompiledPlan

MEMORY_POLICIES = ("latency", "balanced", "minimal")


@dataclass(frozen=True)
class CompilationResult:
    """The reference's ``CompilationResult`` (``compiler.py:25-47``) for the hip target."""

    plan: CompiledPlan
    input_graph: LoweredGraph
    lowered_graph: LoweredGraph
    codegen_matmul: bool = True
    codegen_attention: bool = True
    autotune: bool = False
    target: str = TARGET

    def __call__(self, *inputs, verify_index_bounds: bool = True, memory: str = "latency"):
        return self.plan(*inputs, verify_index_bounds=verify_index_bounds, memory=memory)

    def save(self, path):
        """Write the plan as a ``.aoto`` artifact (gfx950 code object, graph, bound state)."""

        from .artifact import save_compiled

        return save_compiled(self, path)

    def prepare(self, memory: str = "latency") -> dict:
        """Everything is built at compile time; report what a call does."""

        if memory not in MEMORY_POLICIES:
            raise CompilationError(f"unknown memory policy {memory!r}")
        return {"memory": memory, "kernels": len(self.plan.nodes)}


@dataclass(frozen=True)
class CompiledModulePlan:
    """An executable plan with the module's parameters bound as device state (``compiler.py:88-218``)."""

    compilation: CompilationResult
    input_count: int
    state_names: tuple[str, ...]
    tensor_kwarg_names: tuple[str, ...] = ()
    _runner: Any = field(default=None, repr=False, compare=False)

    @property
    def plan(self) -> CompiledPlan:
        return self.compilation.plan

    @property
    def target(self) -> str:
        return self.compilation.target

    @property
    def input_graph(self) -> LoweredGraph:
        return self.compilation.input_graph

    @property
    def lowered_graph(self) -> LoweredGraph:
        return self.compilation.lowered_graph

    @property
    def selections(self):
        return self.plan.selections

    def prepare(self, memory: str = "latency") -> dict:
        return self.compilation.prepare(memory)

    def save(self, path):
        """Write the plan as a ``.aoto`` artifact; ``load_compiled_module`` reloads it in any process."""

        from .artifact import save_compiled

        return save_compiled(self, path)

    def __call__(self, *inputs, verify_index_bounds: bool = True, memory: str = "latency", **tensor_kwargs):
        if len(inputs) != self.input_count:
            raise PlanInputError(
                f"expected {self.input_count} inputs, received {len(inputs)}",
                hint="positional inputs come first, then the promoted tensor keywords by name",
            )
        missing = [name for name in self.tensor_kwarg_names if name not in tensor_kwargs]
        if missing:
            raise PlanInputError("missing tensor keyword inputs: " + ", ".join(missing))
        unexpected = sorted(set(tensor_kwargs) - set(self.tensor_kwarg_names))
        if unexpected:
            raise PlanInputError("unexpected keyword inputs: " + ", ".join(unexpected),
                                 hint="Python-valued keywords were baked in at compile time")
        if memory not in MEMORY_POLICIES:
            raise PlanInputError(f"unknown memory policy {memory!r}")
        values = list(inputs) + [tensor_kwargs[name] for name in self.tensor_kwarg_names]
        return self.plan(*values, verify_index_bounds=verify_index_bounds, memory=memory)


def _tensor_leaves(value) -> list[torch.Tensor] | None:
    """Depth-first tensor leaves of nested tuples/lists (``None`` entries dropped); ``None``
    when some leaf is neither a tensor nor ``None``."""

    if value is None:
        return []
    if isinstance(value, torch.Tensor):
        return [value]
    if not isinstance(value, (tuple, list)):
        return None
    out: list[torch.Tensor] = []
    for item in value:
        found = _tensor_leaves(item)
        if found is None:
            return None
        out += found
    return out


def _pick_by_key(output: Any, key: str):
    """``output[key]`` for a mapping (``KeyError`` when absent), else the attribute ``key``
    (``ValueError`` when absent)."""

    if isinstance(output, Mapping):
        if key in output:
            return output[key]
        raise KeyError(f"output_key {key!r} is not among the module's outputs {sorted(map(str, output))}")
    if hasattr(output, key):
        return getattr(output, key)
    raise ValueError(f"output_key {key!r}: the module's {type(output).__name__} output has no such attribute")


def _select_output(output: Any, output_key: str | None):
    """Which part of a module's return value a plan returns (reference ``compiler.py:843-889``).

    An explicit ``output_key`` wins. Otherwise a tensor is returned as is; a model
    output object gives its ``logits``; a one-entry mapping gives its value; a tuple or
    list gives its tensor leaves, flattened in order. Anything else is refused.
    """

    chosen = output
    if output_key is not None:
        chosen = _pick_by_key(output, output_key)
    elif not isinstance(output, torch.Tensor):
        if hasattr(output, "logits"):
            chosen = output.logits
        elif isinstance(output, Mapping) and len(output) == 1:
            (chosen,) = output.values()
    if isinstance(chosen, torch.Tensor):
        return chosen
    if isinstance(chosen, (tuple, list)):
        leaves = _tensor_leaves(chosen)
        if leaves:
            return tuple(leaves)
        raise ValueError(f"cannot compile a {type(chosen).__name__} output holding no tensors or a non-tensor leaf; "
                         "return tensors (possibly nested in tuples/lists)")
    raise ValueError(f"cannot compile a module returning {type(chosen).__name__}: return a tensor or tensors, "
                     "or pass output_key to select one")


class _ModuleCall(torch.nn.Module):
    """forward(*inputs, *tensor_kwargs) -> the selected output of ``module(*inputs, **kwargs)``."""

    def __init__(self, module, input_count, static_kwargs, tensor_kwarg_names, output_key):
        super().__init__()
        self.module = module
        self.input_count = input_count
        self.static_kwargs = dict(static_kwargs)
        self.tensor_kwarg_names = tuple(tensor_kwarg_names)
        self.output_key = output_key

    def forward(self, *args):
        inputs = args[: self.input_count]
        kwargs = dict(self.static_kwargs)
        kwargs.update(zip(self.tensor_kwarg_names, args[self.input_count:]))
        return _select_output(self.module(*inputs, **kwargs), self.output_key)


def compile_callable(
    fn: Callable[..., Any],
    example_inputs: Sequence[Any],
    *,
    target: str = TARGET,
    codegen_matmul: bool = False,
    codegen_attention: bool = False,
    autotune: bool = False,
) -> CompilationResult:
    """Capture ``fn`` on ``example_inputs`` and lower it to gfx950 kernels (``compiler.py:301-321``)."""

    backend = backend_for(target, codegen_matmul=codegen_matmul, codegen_attention=codegen_attention,
                          autotune=autotune)
    graph = capture(fn, tuple(example_inputs))
    plan = backend.compile(graph, plan_name=getattr(fn, "__name__", "callable"))
    return CompilationResult(plan=plan, input_graph=graph, lowered_graph=graph)


def compile_module(
    module: Any,
    example_inputs: Sequence[Any],
    *,
    example_kwargs: Mapping[str, Any] | None = None,
    output_key: str | None = None,
    target: str = TARGET,
    codegen_matmul: bool = False,
    codegen_attention: bool = False,
    autotune: bool = False,
) -> CompiledModulePlan:
    """Compile an ``nn.Module`` with its parameters and buffers bound as plan state (``compiler.py:324-405``)."""

    backend = backend_for(target, codegen_matmul=codegen_matmul, codegen_attention=codegen_attention,
                          autotune=autotune)
    if not isinstance(module, torch.nn.Module):
        raise TypeError(f"expected torch.nn.Module, got {type(module).__name__}")
    if getattr(module, "training", False):
        raise CompilationError(
            "compile_module requires module.eval()",
            hint="a graph traced in training mode holds dropout and batchnorm updates a static plan cannot replay",
        )
    static_kwargs: dict[str, Any] = {}
    tensor_names: list[str] = []
    tensor_values: list[torch.Tensor] = []
    for name, value in dict(example_kwargs or {}).items():
        if isinstance(value, torch.Tensor):
            tensor_names.append(name)
            tensor_values.append(value)
        elif isinstance(value, (list, tuple, dict)) and _holds_tensor(value):
            raise CompilationError(f"keyword {name!r} nests tensors; pass each tensor as its own keyword")
        else:
            static_kwargs[name] = value
    clashes = sorted({"verify_index_bounds", "memory"} & set(tensor_names))
    if clashes:
        raise CompilationError(f"a tensor keyword input cannot be named {clashes[0]!r}: the plan uses that name")
    wrapper = _ModuleCall(module, len(example_inputs), static_kwargs, tensor_names, output_key).eval()
    graph = capture(wrapper, tuple(example_inputs) + tuple(tensor_values))
    plan = backend.compile(graph, plan_name=type(module).__name__)
    runner = plan._keepalive
    result = CompilationResult(plan=plan, input_graph=graph, lowered_graph=graph)
    labels = tuple(graph.state_labels.get(n, n).removeprefix("module.") for n in graph.state_names)
    return CompiledModulePlan(compilation=result, input_count=len(example_inputs), state_names=labels,
                              tensor_kwarg_names=tuple(tensor_names), _runner=runner)


def _holds_tensor(value) -> bool:
    if isinstance(value, torch.Tensor):
        return True
    if isinstance(value, Mapping):
        return any(_holds_tensor(v) for v in value.values())
    if isinstance(value, (list, tuple, set)):
        return any(_holds_tensor(v) for v in value)
    return False
