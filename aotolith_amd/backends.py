"""The backend seam for ``target="hip-gfx950"``.

The reference's compiler picks a ``Backend`` by target name (``TARGETS``,
``backends/__init__.py:38``; ``compiler.backend_for``, ``compiler.py:219-258``) and
asks it to ``compile(graph, *, tune_inputs=None) -> CompiledPlan``
(``backends/__init__.py:41-55``). This module is that seam for this target: the
registry and the backend object that lowers a captured, legalized graph to a plan
whose every node is a gfx950 kernel (``graph_ops``). ``compile_callable`` and
``compile_module`` reach their kernels through it.
"""

from __future__ import annotations

from collections.abc import Sequence
from typing import Any, Protocol

from .errors import CompilationError
from .graph import LoweredGraph
from .plan import TARGET, CompiledPlan

#: Target names this package compiles for (the reference registers "apple-metal"
#: and "mlx-reference"; a build of the reference with this backend adds this one).
TARGETS: tuple[str, ...] = (TARGET,)


class Backend(Protocol):
    """What the compiler asks of a target (``backends/__init__.py:41-55``)."""

    name: str

    def compile(self, graph: LoweredGraph, *, tune_inputs: Sequence[Any] | None = None) -> CompiledPlan: ...


class HipGfx950Backend:
    """Lowers a captured graph to gfx950 kernel launches, one selection per launched kernel.

    There is one kernel per node family and no candidate search, so ``tune_inputs``
    (the reference's autotuning samples) are checked against the graph's input count
    and otherwise unused.
    """

    name = TARGET

    def compile(self, graph: LoweredGraph, *, tune_inputs: Sequence[Any] | None = None,
                plan_name: str = "graph") -> CompiledPlan:
        if tune_inputs is not None and len(tune_inputs) != len(graph.inputs):
            raise CompilationError(f"tune_inputs has {len(tune_inputs)} values for a graph of "
                                   f"{len(graph.inputs)} inputs")
        from .graph_ops import build_graph_plan

        plan, runner = build_graph_plan(graph, name=plan_name)
        plan._keepalive = runner
        return plan


def backend_for(target: str, *, codegen_matmul: bool = False, codegen_attention: bool = False,
                autotune: bool = False) -> HipGfx950Backend:
    """The backend of ``target`` (``compiler.py:219-258``); refuses targets this package does not build."""

    if target not in TARGETS:
        raise CompilationError(
            f"unsupported target: {target}",
            hint=f"this package implements {TARGET!r}; 'apple-metal' and 'mlx-reference' run on Apple silicon",
        )
    if autotune:
        raise CompilationError(f"target {TARGET!r} has one kernel per node family and nothing to autotune",
                               hint="drop autotune=True")
    del codegen_matmul, codegen_attention  # every node is a generated kernel on this target
    return HipGfx950Backend()
