"""TEST INFRASTRUCTURE ONLY — runs a memory plan on the CPU oracle.

Builds the same OpNode array the device executor builds (via
runtime.executor.nodes.build_nodes), but with host addresses: a numpy arena
of ``plan.arena_size`` bytes, the constants' numpy buffers and the caller's
input arrays — i.e. what the reference's CompiledExecutor hands to
``execute`` (runtime/executor/compiled.py:34-99) — and calls
``oracle_execute`` from liboracle.so (oracle_executor.c).

Used by tests/ (as the checker), by bench.py's cpu_baseline leg, and by
__graft_entry__.smoke(); never by the product path.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build(force: bool = True) -> Path:
    """Compile liboracle.so with the Makefile beside this file."""
    cmd = ["make", "-C", str(HERE)] + (["-B"] if force else []) + ["liboracle.so"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    return LIB_PATH


def load():
    global _lib
    if _lib is None:
        from runtime.executor.common import COpNode
        if not LIB_PATH.exists():
            build(force=False)
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.oracle_execute.argtypes = [ctypes.POINTER(COpNode), ctypes.c_int]
        lib.oracle_execute.restype = ctypes.c_int
        lib.oracle_last_error.restype = ctypes.c_char_p
        lib.oracle_num_threads.restype = ctypes.c_int
        lib.oracle_set_num_threads.argtypes = [ctypes.c_int]
        _lib = lib
    return _lib


def num_threads() -> int:
    return load().oracle_num_threads()


def set_num_threads(n: int) -> None:
    load().oracle_set_num_threads(int(n))


class OracleRun:
    """A plan compiled against the oracle: host arena + node array."""

    def __init__(self, plan) -> None:
        from runtime.executor.nodes import build_nodes
        self.plan = plan
        graph = plan.graph
        self.arena = np.zeros(max(plan.arena_size, 1), dtype=np.uint8)
        external = set(graph.inputs) | set(graph.constants)
        self._inputs = {name: np.zeros(graph.tensors[name].shape, dtype=np.dtype(graph.tensors[name].dtype))
                        for name in graph.inputs}
        self._consts = {}
        for name in graph.constants:
            buf = graph.tensors[name].buffer
            if buf is not None:
                self._consts[name] = np.ascontiguousarray(buf)
        base = self.arena.ctypes.data

        def addr(name: str) -> int:
            if name in self._inputs:
                return self._inputs[name].ctypes.data
            if name in self._consts:
                return self._consts[name].ctypes.data
            if name in plan.offsets and name not in external:
                return base + plan.offsets[name]
            raise RuntimeError(f"oracle: tensor '{name}' has no host address")

        self.nodes, self.order = build_nodes(plan, addr, lambda off, size: base + off)
        self._addr = addr

    def run(self, inputs: dict[str, np.ndarray]) -> dict[str, np.ndarray]:
        graph = self.plan.graph
        for name, buf in self._inputs.items():
            if name not in inputs:
                raise ValueError(f"Missing input tensor: '{name}'")
            src = np.asarray(inputs[name], dtype=buf.dtype).reshape(buf.shape)
            np.copyto(buf, src)
        lib = load()
        rc = lib.oracle_execute(self.nodes, len(self.order))
        if rc != 0:
            raise RuntimeError(lib.oracle_last_error().decode())
        out = {}
        for name in graph.outputs:
            t = graph.tensors[name]
            n = int(np.prod(t.shape)) * np.dtype(t.dtype).itemsize
            raw = (ctypes.c_char * n).from_address(self._addr(name))
            out[name] = np.frombuffer(bytes(raw), dtype=np.dtype(t.dtype)).reshape(t.shape).copy()
        return out


def run_plan(plan, inputs: dict[str, np.ndarray]) -> dict[str, np.ndarray]:
    return OracleRun(plan).run(inputs)


if __name__ == "__main__":
    os.environ.setdefault("OMP_NUM_THREADS", str(os.cpu_count() or 1))
    print(build())
