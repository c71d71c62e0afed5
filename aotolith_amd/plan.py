"""Compiled plans of the hip-gfx950 target: an ordered list of kernel launches.

A plan is what the reference's ``CompiledPlan`` is to its backend
(``runtime/plan.py:200-260``): a fixed sequence of nodes, each with the
``KernelSelection`` that says which kernel runs it and why, and a runner that
executes them in submission order on one stream. Here every node is a
hand-written gfx950 kernel launched through the C ABI; there is no interpreter
fallback, so a node that no kernel covers is a compile-time error.
"""

from __future__ import annotations

import threading
import weakref
from collections.abc import Callable, Sequence
from dataclasses import dataclass, field

from .errors import CompilationError
from .selection import KernelSelection

TARGET = "hip-gfx950"
ARCHITECTURE = "gfx950"


@dataclass(frozen=True)
class PlanNode:
    """One lowered operation: its selection record and the launch that runs it."""

    selection: KernelSelection
    launch: Callable[..., None] | None = None


@dataclass
class CompiledPlan:
    """An executable plan: nodes in order plus the callable that runs them.

    ``run`` takes the plan's inputs and returns its outputs; it is built by
    the lowering that made the nodes and closes over their launches.
    """

    name: str
    nodes: tuple[PlanNode, ...]
    run: Callable[..., object]
    target: str = TARGET
    input_names: tuple[str, ...] = ()
    output_names: tuple[str, ...] = ()
    _lock: threading.Lock = field(default_factory=threading.Lock, repr=False)
    _runtime_ref: object | None = field(default=None, repr=False, compare=False)
    _keepalive: object | None = field(default=None, repr=False, compare=False)

    @property
    def runtime(self):
        """The runtime this plan belongs to (held weakly: a runtime owns its plans)."""

        return None if self._runtime_ref is None else self._runtime_ref()

    @runtime.setter
    def runtime(self, value) -> None:
        self._runtime_ref = None if value is None else weakref.ref(value)

    @property
    def selections(self) -> tuple[KernelSelection, ...]:
        return tuple(node.selection for node in self.nodes)

    @property
    def native_count(self) -> int:
        return sum(1 for node in self.nodes if node.selection.is_native)

    def kernel_names(self) -> tuple[str, ...]:
        """Distinct kernel symbols this plan launches, in first-use order."""

        seen: dict[str, None] = {}
        for node in self.nodes:
            if node.selection.artifact_name:
                seen.setdefault(node.selection.artifact_name, None)
        return tuple(seen)

    def save(self, path):
        """Write this plan as a ``.aoto`` artifact (the reference's ``CompiledModulePlan.save``)."""

        from .artifact import save_compiled

        return save_compiled(self, path)

    def __call__(self, *inputs, **kwargs):
        # Launches are enqueued in order on the caller's current stream; the lock
        # only keeps two host threads from interleaving one plan's buffers.
        with self._lock:
            return self.run(*inputs, **kwargs)


def require_native(selections: Sequence[KernelSelection], what: str) -> None:
    """Refuse a plan with a node no hip kernel covers (no CPU or torch fallback)."""

    missing = [s for s in selections if not s.is_native]
    if missing:
        detail = "; ".join(f"{s.op} ({s.output_id}): {s.reason}" for s in missing)
        raise CompilationError(
            f"{what}: {len(missing)} node(s) have no {TARGET} kernel: {detail}",
            hint="the hip-gfx950 target runs every node as a gfx950 kernel and has no fallback",
        )
