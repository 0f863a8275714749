"""Compiled executor on the MI355X: the whole plan as one hipGraph replay.

Drop-in for the reference's CompiledExecutor (runtime/executor/compiled.py:
20-157): ``compile(plan)`` once, ``run(inputs) -> outputs`` many times, same
node filtering and OpNode contents.  What changes is where memory lives:

* the arena is one device allocation of ``plan.arena_size`` bytes; every
  intermediate is at ``arena + plan.offsets[name]`` and every scratch slot
  at ``arena + plan.scratch[id][0]`` — the planner's layout, byte for byte;
* constants are uploaded once into one device block (256-byte aligned
  slots);
* each graph input gets a fixed device staging buffer, so node pointers
  never change after compile and the launch sequence can be captured into a
  hipGraph once and replayed (``run`` = H2D inputs, graph launch, D2H
  outputs).

``launch()`` / ``synchronize()`` / ``time_launches()`` / ``profile_nodes()``
run the plan on device-resident data for benchmarking.  There is no CPU
fallback: a missing library or GPU raises at compile.
"""

from __future__ import annotations

import ctypes
import os
import time

import numpy as np

from ..ir import Graph, OpType
from ..planner import MemoryPlan
from .common import Executor, OpTiming, RunProfile
from .hip_lib import FUSE_KINDS, HipLibrary, live_arrays, load_library
from .nodes import build_nodes, check_extents, dispatch_order

_ALIGN = 256


def _align(n: int) -> int:
    return (n + _ALIGN - 1) // _ALIGN * _ALIGN


class DeviceWeights:
    """Constants resident in one device block, keyed by tensor name."""

    def __init__(self, lib: HipLibrary, graph: Graph, names: list[str]) -> None:
        self._lib = lib
        self.offsets: dict[str, int] = {}
        self.keys: dict[str, tuple[int, int]] = {}
        total = 0
        for n in names:
            buf = graph.tensors[n].buffer
            if buf is None:
                raise ValueError(f"constant '{n}' has no data")
            self.offsets[n] = total
            total += _align(buf.nbytes)
        self.nbytes = total
        self.base = lib.alloc(total) if total else 0
        for n in names:
            buf = np.ascontiguousarray(graph.tensors[n].buffer)
            if buf.nbytes:
                lib.h2d(self.base + self.offsets[n], buf.ctypes.data, buf.nbytes)
            self.keys[n] = (id(graph.tensors[n].buffer), buf.nbytes)

    def covers(self, graph: Graph, names: list[str]) -> bool:
        """True if every named constant is resident with the same buffer object."""
        for n in names:
            t = graph.tensors.get(n)
            if n not in self.keys or t is None or t.buffer is None or self.keys[n] != (id(t.buffer), t.buffer.nbytes):
                return False
        return True

    def addr(self, name: str) -> int:
        return self.base + self.offsets[name]

    def free(self) -> None:
        if self.base:
            self._lib.free(self.base)
            self.base = 0


class _PinnedBlock:
    """Pinned host memory lent to one returned output array.  numpy keeps this object as the
    array's base, so the block goes back to its pool when the last view of it is dropped."""

    __slots__ = ("ptr", "nbytes", "pool")

    def __init__(self, pool: "PinnedPool", ptr: int, nbytes: int) -> None:
        self.ptr, self.nbytes, self.pool = ptr, nbytes, pool

    @property
    def __array_interface__(self):
        return {"shape": (self.nbytes,), "typestr": "|u1", "data": (self.ptr, False), "version": 3}

    def __del__(self):
        try:
            self.pool.give_back(self.ptr, self.nbytes)
        except Exception:
            pass


class PinnedPool:
    """Output buffers in pinned host memory, so device→host copies run at DMA speed straight
    into the arrays run() returns.  Each array is the caller's own (as the reference's
    compiled executor returns copies, runtime/executor/compiled.py:94-98); its block is
    reused only after the caller drops it.  Beyond ``cap_bytes`` of blocks out at once,
    arrays fall back to ordinary memory."""

    def __init__(self, lib: HipLibrary, cap_bytes: int = 1 << 30) -> None:
        self._lib = lib
        self._free: dict[int, list[int]] = {}
        self._out = 0
        self._cap = cap_bytes
        self._closed = False

    def array(self, shape, dtype) -> np.ndarray:
        dtype = np.dtype(dtype)
        nbytes = int(np.prod(shape)) * dtype.itemsize
        free = self._free.get(nbytes)
        if not nbytes or self._closed or (not free and self._out + nbytes > self._cap):
            return np.empty(shape, dtype=dtype)
        ptr = free.pop() if free else self._host_alloc(nbytes)
        self._out += nbytes
        return np.asarray(_PinnedBlock(self, ptr, nbytes)).view(dtype).reshape(shape)

    def _host_alloc(self, nbytes: int) -> int:
        p = ctypes.c_void_p()
        self._lib.check(self._lib.lbr_host_alloc(nbytes, ctypes.byref(p)), f"pinned host alloc {nbytes} B")
        return int(p.value)

    def give_back(self, ptr: int, nbytes: int) -> None:
        self._out -= nbytes
        if self._closed:
            self._lib.lbr_host_free(ctypes.c_void_p(ptr))
        else:
            self._free.setdefault(nbytes, []).append(ptr)

    def close(self) -> None:
        for ptrs in self._free.values():
            for ptr in ptrs:
                self._lib.lbr_host_free(ctypes.c_void_p(ptr))
        self._free = {}
        self._closed = True


class CompiledExecutor(Executor):
    """Plan → device OpNode array → hipGraph, replayed per run()."""

    def __init__(self, profile: bool = False, use_graph: bool = True, device: int = 0,
                 weights: DeviceWeights | None = None, fuse: bool | None = None) -> None:
        super().__init__(profile=profile)
        self._use_graph = use_graph
        # peephole fusion in the device library (LBR_FUSE=0 turns it off)
        self._fuse = os.environ.get("LBR_FUSE", "1") != "0" if fuse is None else fuse
        self._device = device
        self._lib: HipLibrary | None = None
        self._graph: Graph | None = None
        self._plan_handle = ctypes.c_void_p()
        self._nodes = None
        self._order = []
        self._arena = 0
        # weights passed in (Session's shared block) are borrowed: used when they cover the
        # graph's constants, never freed here; weights this executor uploads itself it owns
        self._weights: DeviceWeights | None = weights
        self._owns_weights = weights is None
        self._inputs: dict[str, tuple[int, int]] = {}   # name -> (device ptr, nbytes)
        self._addr: dict[str, int] = {}
        self._pinned: PinnedPool | None = None

    # ------------------------------------------------------------------ compile
    def compile(self, plan: MemoryPlan) -> None:
        self.close()
        lib = load_library(self._device)
        self._lib = lib
        graph = plan.graph
        self._graph = graph
        external = set(graph.inputs) | set(graph.constants)

        # constants referenced by dispatched nodes (and constant outputs)
        order = dispatch_order(plan)
        check_extents(order, graph)
        for node in order:
            if not lib.lbr_op_supported(node.op.value):
                raise RuntimeError(f"Op {node.op.name} (node {node.id}) has no device kernel")
        used_consts: list[str] = []
        seen = set()
        for node in order:
            for t in node.inputs:
                if t in graph.constants and t not in seen:
                    seen.add(t)
                    used_consts.append(t)
        for t in graph.outputs:
            if t in graph.constants and t not in seen:
                seen.add(t)
                used_consts.append(t)

        if self._weights is None or not self._weights.covers(graph, used_consts):
            if self._weights is not None and self._owns_weights:
                self._weights.free()
            self._weights = DeviceWeights(lib, graph, used_consts)
            self._owns_weights = True

        self._arena = lib.alloc(max(plan.arena_size, 1))
        self._inputs = {}
        for name in graph.inputs:
            t = graph.tensors[name]
            nb = int(np.prod(t.shape)) * np.dtype(t.dtype).itemsize
            self._inputs[name] = (lib.alloc(max(nb, 1)), nb)

        addr: dict[str, int] = {}
        for name, off in plan.offsets.items():
            if name not in external:
                addr[name] = self._arena + off
        for name, (ptr, _) in self._inputs.items():
            addr[name] = ptr
        for name in used_consts:
            addr[name] = self._weights.addr(name)
        self._addr = addr

        def resolve(name: str) -> int:
            if name not in addr:
                raise RuntimeError(f"tensor '{name}' has no device address (not an input, constant or "
                                   f"planned intermediate)")
            return addr[name]

        arr, order = build_nodes(plan, resolve, lambda off, size: self._arena + off)
        for i, node in enumerate(order):
            if node.op == OpType.EMBEDDING:
                # device kernel bounds-checks ids against the table's row count
                arr[i].extra[1] = graph.tensors[node.inputs[1]].shape[0]
        self._nodes = arr
        self._order = order
        self._pinned = PinnedPool(lib)
        handle = ctypes.c_void_p()
        if self._fuse:
            live = self.live_outs()
            lp, lb = live_arrays(live)
            lib.check(lib.lbr_plan_create_fused(arr, len(order), 1 if self._use_graph else 0, lp, lb, len(live),
                                                ctypes.byref(handle)), "lbr_plan_create_fused")
        else:
            lib.check(lib.lbr_plan_create(arr, len(order), 1 if self._use_graph else 0, ctypes.byref(handle)),
                      "lbr_plan_create")
        self._plan_handle = handle

    def live_outs(self) -> list[tuple[int, int]]:
        """(device address, bytes) of every graph output: what the caller reads after a launch."""
        out = []
        for name in self._graph.outputs:
            t = self._graph.tensors[name]
            out.append((self._addr[name], int(np.prod(t.shape)) * np.dtype(t.dtype).itemsize))
        return out

    def fused_runs(self) -> list[tuple[int, int, str]]:
        """(first node, node count, kind) of every fused step of the compiled plan."""
        runs = []
        first, count, kind = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        for st in range(self._lib.lbr_plan_num_steps(self._plan_handle)):
            self._lib.check(self._lib.lbr_plan_step_info(self._plan_handle, st, ctypes.byref(first),
                                                         ctypes.byref(count), ctypes.byref(kind)),
                            "lbr_plan_step_info")
            if count.value > 1:
                runs.append((first.value, count.value, FUSE_KINDS.get(kind.value, "?")))
        return runs

    def step_params(self) -> list[dict]:
        """Every kernel step of the compiled plan: its kernel (and full step name, with the
        fused parts), the nodes it covers, and the schedule its launch arguments encode
        (attention: causal fold, key-range split workgroups, deferred output, key-quartered
        16-row kernel and whether it reads K fragment-major; GEMM: DMA tile
        index, K ranges, norm prologue, norm in the split-K reduce and whether the split was
        made for it, head splits it stores fragment-major (bit mask), head-prologue parts
        its epilogue applies; head prologue: float4 kernel or one wavefront per row, and
        how many Q/K parts one launch covers)."""
        lib, h = self._lib, self._plan_handle
        first, count, kind = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        ints = (ctypes.c_longlong * 40)()
        names = self.kernel_names()
        out = []
        for st in range(lib.lbr_plan_num_steps(h)):
            lib.check(lib.lbr_plan_step_info(h, st, ctypes.byref(first), ctypes.byref(count), ctypes.byref(kind)),
                      "lbr_plan_step_info")
            lib.check(lib.lbr_plan_step_args(h, st, ints, 40), "lbr_plan_step_args")
            d = {"kernel": names[first.value].split("+")[0], "name": names[first.value], "first": first.value,
                 "count": count.value, "kind": FUSE_KINDS.get(kind.value, "?")}
            if d["kernel"].startswith(("attn_fwd_mfma16", "attn_fwd_kq")):
                d.update(fold=bool(ints[6]), split_wg=int(ints[7]), defer=bool(ints[14]), kq=bool(ints[15]),
                         k_frag=bool(ints[15]) and bool(ints[16]),
                         block_rows=16 if ints[15] else 64 if ints[18] else 128)
            elif d["kernel"].startswith("gemm_"):
                d.update(m=int(ints[0]), n=int(ints[1]), k=int(ints[2]),
                         tile=lib.lbr_gemm_tile_name(int(ints[14]) - 1).decode() or "legacy",
                         ksplit=max(1, int(ints[10])), dma_tile=int(ints[14]) - 1, norm=int(ints[15]),
                         reduce_norm=int(ints[16]), split_for_norm=bool(int(ints[17]) & 256),
                         frag_splits=int(ints[5]) if int(ints[19]) > 0 else 0,
                         head_parts=int(ints[18]))
            elif d["kind"] == "head_prologue":
                d.update(vec=bool(ints[13]), parts=int(ints[14]) if ints[13] else 1)
            out.append(d)
        return out

    # ------------------------------------------------------------------ run
    def _upload_inputs(self, inputs: dict[str, np.ndarray]) -> None:
        """Enqueue the input copies on the library stream (through its pinned ring); the
        caller's arrays may change once this returns."""
        graph = self._graph
        for name, (ptr, nb) in self._inputs.items():
            if name not in inputs:
                raise ValueError(f"Missing input tensor: '{name}'")
            t = graph.tensors[name]
            arr = np.ascontiguousarray(inputs[name])
            if arr.dtype != np.dtype(t.dtype):
                raise ValueError(f"input '{name}' is {arr.dtype}, graph expects {t.dtype}")
            if arr.nbytes != nb:
                raise ValueError(f"input '{name}' has shape {arr.shape}, graph expects {t.shape}")
            self._lib.check(self._lib.lbr_upload_async(ctypes.c_void_p(ptr), ctypes.c_void_p(arr.ctypes.data), nb),
                            "upload")

    def _enqueue_downloads(self) -> dict[str, np.ndarray]:
        """Arrays for the graph outputs (pinned where possible) with their device→host copies
        enqueued on the library stream; valid after synchronize()."""
        graph = self._graph
        out = {}
        for name in graph.outputs:
            t = graph.tensors[name]
            host = self._pinned.array(t.shape, t.dtype)
            if host.nbytes:
                self._lib.check(self._lib.lbr_download_async(ctypes.c_void_p(host.ctypes.data),
                                                             ctypes.c_void_p(self._addr[name]), host.nbytes),
                                "download")
            out[name] = host
        return out

    def _download_outputs(self) -> dict[str, np.ndarray]:
        out = self._enqueue_downloads()
        self.synchronize()
        return out

    def run(self, inputs: dict[str, np.ndarray]) -> dict[str, np.ndarray]:
        if self._lib is None:
            raise RuntimeError("CompiledExecutor.run() before compile()")
        self._upload_inputs(inputs)
        if self._profile:
            times = self.profile_nodes(1)
            self._last_profile = RunProfile(
                op_timings=[OpTiming(node.id, node.op.name, int(ms * 1e6), node.output,
                                     tuple(self._graph.tensors[node.output].shape))
                            for node, ms in zip(self._order, times)],
                total_ns=int(sum(times) * 1e6))
        else:
            # inputs in, one graph replay, outputs out: all in stream order, one wait
            t0 = time.perf_counter_ns()
            self.launch()
            out = self._enqueue_downloads()
            self.synchronize()
            self._last_profile = RunProfile(total_ns=time.perf_counter_ns() - t0)
            return out
        return self._download_outputs()

    # ------------------------------------------------------------------ device-resident API
    def upload_inputs(self, inputs: dict[str, np.ndarray]) -> None:
        self._upload_inputs(inputs)
        self.synchronize()

    def download_outputs(self) -> dict[str, np.ndarray]:
        return self._download_outputs()

    def launch(self) -> None:
        self._lib.check(self._lib.lbr_plan_launch(self._plan_handle), "lbr_plan_launch")

    def synchronize(self) -> None:
        self._lib.check(self._lib.lbr_synchronize(), "lbr_synchronize")

    def time_launches(self, iters: int) -> float:
        """Milliseconds for ``iters`` back-to-back launches (hipEvents on the library stream)."""
        ms = ctypes.c_float()
        self._lib.check(self._lib.lbr_plan_time(self._plan_handle, int(iters), ctypes.byref(ms)), "lbr_plan_time")
        return float(ms.value)

    def profile_nodes(self, iters: int = 1) -> list[float]:
        """Mean milliseconds per dispatched node: each step launched ``iters`` times back to
        back between one hipEvent pair (eager launches on the library stream)."""
        n = len(self._order)
        buf = (ctypes.c_float * max(n, 1))()
        self._lib.check(self._lib.lbr_plan_profile(self._plan_handle, int(iters), buf, max(n, 1)),
                        "lbr_plan_profile")
        return [float(buf[i]) for i in range(n)]

    def kernel_names(self) -> list[str]:
        names = []
        for i in range(len(self._order)):
            b = ctypes.create_string_buffer(64)
            self._lib.check(self._lib.lbr_plan_node_kernel(self._plan_handle, i, b, 64), "lbr_plan_node_kernel")
            names.append(b.value.decode())
        return names

    @property
    def dispatch_order(self):
        return list(self._order)

    @property
    def weights(self) -> DeviceWeights | None:
        return self._weights

    def device_address(self, name: str) -> int:
        return self._addr[name]

    # ------------------------------------------------------------------ teardown
    def close(self) -> None:
        lib = self._lib
        if lib is None:
            return
        if self._plan_handle:
            lib.lbr_plan_destroy(self._plan_handle)
            self._plan_handle = ctypes.c_void_p()
        for ptr, _ in self._inputs.values():
            lib.free(ptr)
        self._inputs = {}
        if self._pinned is not None:
            self._pinned.close()    # blocks still held by returned arrays are freed when those go
            self._pinned = None
        if self._arena:
            lib.free(self._arena)
            self._arena = 0
        if self._weights is not None and self._owns_weights:
            self._weights.free()
            self._weights = None

    def release_weights(self) -> DeviceWeights | None:
        """Hand the resident weights to the caller (Session, which shares them between cached
        plans and frees them); this executor stops owning them."""
        self._owns_weights = False
        return self._weights

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
