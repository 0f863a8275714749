"""Executor base class, the COpNode ctypes mirror and profiling records.

``COpNode`` is field-for-field the reference's ctypes mirror
(runtime/executor/common.py:125-141) of the C ``OpNode`` (csrc/runtime.h:60-69,
include/lbr_executor.h); the device library checks ``sizeof`` at load.
"""

from __future__ import annotations

import ctypes
from abc import ABC, abstractmethod
from collections import defaultdict
from dataclasses import dataclass, field

import numpy as np

from ..planner import MemoryPlan

MAX_INPUTS = 12
MAX_DIMS = 24


class COpNode(ctypes.Structure):
    _fields_ = [
        ("op", ctypes.c_int),
        ("n_inputs", ctypes.c_int),
        ("inputs", ctypes.c_void_p * MAX_INPUTS),
        ("output", ctypes.c_void_p),
        ("out_shape", ctypes.c_int * MAX_DIMS),
        ("n_dims", ctypes.c_int),
        ("elem_size", ctypes.c_int),
        ("extra", ctypes.c_int * MAX_DIMS),
    ]


@dataclass
class OpTiming:
    node_id: int
    op: str
    time_ns: int
    output_name: str
    output_shape: tuple[int, ...]


@dataclass
class RunProfile:
    op_timings: list[OpTiming] = field(default_factory=list)
    total_ns: int = 0

    def __str__(self) -> str:
        total_ms = self.total_ns / 1e6
        if not self.op_timings:
            return f"Execution Profile:\n  Total: {total_ms:.2f} ms (no per-op breakdown)"
        by_op: dict[str, list[int]] = defaultdict(list)
        for t in self.op_timings:
            by_op[t.op].append(t.time_ns)
        lines = ["Execution Profile:", f"  Total: {total_ms:.2f} ms ({len(self.op_timings)} ops)"]
        rows = sorted(((op, sum(v), len(v)) for op, v in by_op.items()), key=lambda r: r[1], reverse=True)
        for op, ns, cnt in rows:
            pct = ns / self.total_ns * 100 if self.total_ns > 0 else 0.0
            lines.append(f"  {op:<20} {ns / 1e6:7.2f} ms ({pct:5.1f}%)  {cnt} ops")
        return "\n".join(lines)


class Executor(ABC):
    """compile() once per plan, run() many times."""

    def __init__(self, profile: bool = False) -> None:
        self._profile = profile
        self._last_profile: RunProfile | None = None

    @abstractmethod
    def compile(self, plan: MemoryPlan) -> None:
        ...

    @abstractmethod
    def run(self, inputs: dict[str, np.ndarray]) -> dict[str, np.ndarray]:
        ...
