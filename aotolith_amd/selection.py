"""Per-node kernel selection records of a compiled plan.

Same record as the reference's ``selection.py:6-34`` (field names and order),
so tooling that reads ``plan.selections`` reads ours. ``is_native`` is widened
from the reference's single ``"metal_kernel"`` to every implementation that
runs a kernel this backend emitted, here ``"hip_kernel"``.
"""

from __future__ import annotations

from dataclasses import dataclass

#: Implementations that run kernels a backend emitted itself (no CPU, torch or
#: vendor-library fallback): this target's gfx950 code object and the Metal kernels
#: of the reference's Apple backend.
NATIVE_IMPLEMENTATIONS = frozenset({"hip_kernel", "metal_kernel"})


@dataclass(frozen=True, slots=True)
class KernelBenchmark:
    candidate: str
    artifact_name: str | None
    warmup_iterations: int
    iterations: int
    samples_seconds: tuple[float, ...]
    median_seconds: float | None
    min_seconds: float | None
    error: str | None = None


@dataclass(frozen=True, slots=True)
class KernelSelection:
    op_index: int
    op: str
    output_id: str
    implementation: str
    kind: str
    reason: str
    artifact_name: str | None = None
    benchmarks: tuple[KernelBenchmark, ...] = ()
    autotuned: bool = False
    device_name: str | None = None
    device_architecture: str | None = None

    @property
    def is_native(self) -> bool:
        return self.implementation in NATIVE_IMPLEMENTATIONS
