"""Memory planner: execution order, tensor lifetimes and arena offsets.

Restates runtime/planner.py:160-569 of the reference; the device arena is
laid out with exactly these offsets, so the algorithm is kept step for step:

1. order: memory-aware Kahn (V1) — among ready nodes pop the one whose
   inputs it would free the most bytes of, ties to the lower node id
   (planner.py:160-217);
2. lifetimes: one pass that makes alias outputs (RESHAPE, dim-0 SLICE) and
   in-place outputs (element-wise ops over a dying, same-sized first input)
   share their root's slot and extend the root's death (planner.py:285-377);
3. scratch: single-step lifetimes for ops with a scratch calculator
   (planner.py:384-418);
4. offsets: step-ordered first-fit (or best-fit) over the live set
   (planner.py:425-477), then shared tensors take root offset + alias byte
   offset (planner.py:520-533).

On the GPU the arena is one hipMalloc of ``arena_size`` bytes and every
intermediate lives at ``base + offsets[name]``.
"""

from __future__ import annotations

import heapq
from collections import defaultdict, deque
from dataclasses import dataclass, field
from enum import Enum, auto

import numpy as np

from .ir import Graph, Node
from .ops import OP_REGISTRY


class OrderStrategy(Enum):
    NAIVE = auto()            # FIFO Kahn
    MEMORY_AWARE_V1 = auto()  # freed-bytes heap (default)
    MEMORY_AWARE_V2 = auto()  # not provided by this backend
    MEMORY_AWARE_V3 = auto()  # not provided by this backend


class FitStrategy(Enum):
    FIRST_FIT = auto()
    BEST_FIT = auto()


@dataclass(frozen=True)
class PlannerConfig:
    order: OrderStrategy = OrderStrategy.MEMORY_AWARE_V1
    fit: FitStrategy = FitStrategy.FIRST_FIT
    enable_inplace: bool = True
    enable_aliases: bool = True


def _fmt_bytes(n: int) -> str:
    if n >= 1024 * 1024:
        return f"{n / (1024 * 1024):.1f} MB"
    if n >= 1024:
        return f"{n / 1024:.1f} KB"
    return f"{n} B"


@dataclass
class PlanStats:
    arena_bytes: int
    naive_bytes: int
    n_intermediates: int
    n_allocated: int
    n_shared: int
    scratch_bytes: int
    weight_bytes: int

    @property
    def reuse_savings_bytes(self) -> int:
        return self.naive_bytes - self.arena_bytes

    @property
    def reuse_savings_pct(self) -> float:
        return 0.0 if self.naive_bytes == 0 else self.reuse_savings_bytes / self.naive_bytes * 100

    def __str__(self) -> str:
        return "\n".join([
            "Memory Plan:",
            f"  Arena:          {_fmt_bytes(self.arena_bytes)}",
            f"  Naive (no reuse): {_fmt_bytes(self.naive_bytes)}",
            f"  Savings:        {_fmt_bytes(self.reuse_savings_bytes)} ({self.reuse_savings_pct:.1f}%)",
            f"  Intermediates:  {self.n_intermediates} tensors ({self.n_allocated} allocated, "
            f"{self.n_shared} shared)",
            f"  Scratch:        {_fmt_bytes(self.scratch_bytes)}",
            f"  Weights:        {_fmt_bytes(self.weight_bytes)}",
        ])


@dataclass
class MemoryPlan:
    """Planner output: order, arena size, per-tensor offsets, per-node scratch."""
    graph: Graph
    order: list[Node]
    arena_size: int
    offsets: dict[str, int] = field(default_factory=dict)
    scratch: dict[int, tuple[int, int]] = field(default_factory=dict)  # node id -> (offset, bytes)
    stats: PlanStats | None = None

    def allocate_arena(self) -> np.ndarray:
        return np.zeros(self.arena_size, dtype=np.uint8)


@dataclass
class ExecutionPlan:
    """Memory plan plus the dispatch target (what PRE_EXECUTE validators see)."""
    graph: Graph
    memory: MemoryPlan
    executor_type: str
    backend: str


@dataclass
class Lifetime:
    tensor_name: str
    size_bytes: int
    born: int
    dies: int


def _tensor_size(graph: Graph, name: str) -> int:
    t = graph.tensors[name]
    return int(np.prod(t.shape)) * np.dtype(t.dtype).itemsize


# ---------------------------------------------------------------- ordering

def _memory_aware_order(graph: Graph) -> list[Node]:
    indeg = {nid: sum(1 for t in n.inputs if t in graph._producer) for nid, n in graph.nodes.items()}
    uses_left: dict[str, int] = defaultdict(int)
    for n in graph.nodes.values():
        for t in n.inputs:
            uses_left[t] += 1
    external = set(graph.inputs) | set(graph.constants)

    def freed(n: Node) -> int:
        return sum(_tensor_size(graph, t) for t in n.inputs if t not in external and uses_left[t] == 1)

    heap: list[tuple[int, int]] = []
    for nid, d in indeg.items():
        if d == 0:
            heapq.heappush(heap, (-freed(graph.nodes[nid]), nid))
    order: list[Node] = []
    while heap:
        _, nid = heapq.heappop(heap)
        node = graph.nodes[nid]
        order.append(node)
        for t in node.inputs:
            uses_left[t] -= 1
        for cid in graph._consumers.get(node.output, []):
            indeg[cid] -= 1
            if indeg[cid] == 0:
                heapq.heappush(heap, (-freed(graph.nodes[cid]), cid))
    return order


def _naive_toposort(graph: Graph) -> list[Node]:
    indeg = {nid: sum(1 for t in n.inputs if t in graph._producer) for nid, n in graph.nodes.items()}
    q = deque(nid for nid, d in indeg.items() if d == 0)
    order: list[Node] = []
    while q:
        node = graph.nodes[q.popleft()]
        order.append(node)
        for cid in graph._consumers.get(node.output, []):
            indeg[cid] -= 1
            if indeg[cid] == 0:
                q.append(cid)
    return order


def _get_order(graph: Graph, strategy: OrderStrategy) -> list[Node]:
    if strategy == OrderStrategy.NAIVE:
        return _naive_toposort(graph)
    if strategy == OrderStrategy.MEMORY_AWARE_V1:
        return _memory_aware_order(graph)
    raise NotImplementedError(f"ordering strategy {strategy.name} is not provided by this backend "
                              "(only NAIVE and MEMORY_AWARE_V1)")


# ---------------------------------------------------------------- lifetimes

def _resolve_alias(name: str, graph: Graph) -> str:
    """Follow graph-level alias producers (RESHAPE, dim-0 SLICE) to the owning tensor."""
    while True:
        prod = graph.producer(name)
        if prod is None:
            return name
        op_def = OP_REGISTRY.get(prod.op)
        if op_def is None or not op_def.is_alias(prod):
            return name
        name = prod.inputs[0]


def _compute_lifetimes(graph: Graph, order: list[Node],
                       config: PlannerConfig | None = None) -> tuple[dict[str, Lifetime], dict[str, str]]:
    config = config or PlannerConfig()
    external = set(graph.inputs) | set(graph.constants)
    memory_root: dict[str, str] = {}

    def root_of(name: str) -> str:
        while name in memory_root:
            name = memory_root[name]
        return name

    total_uses: dict[str, int] = defaultdict(int)
    for node in order:
        for t in node.inputs:
            total_uses[_resolve_alias(t, graph)] += 1

    seen_uses: dict[str, int] = defaultdict(int)
    born: dict[str, int] = {}
    dies: dict[str, int] = {}

    for step, node in enumerate(order):
        for t in node.inputs:
            seen_uses[_resolve_alias(t, graph)] += 1
        for t in node.inputs:
            r = root_of(t)
            if r not in external:
                dies[r] = step
        if node.output in external:
            continue
        op_def = OP_REGISTRY.get(node.op)
        if config.enable_aliases and op_def is not None and op_def.is_alias(node):
            r = root_of(_resolve_alias(node.inputs[0], graph))
            if r not in external:
                memory_root[node.output] = r
                continue
        if config.enable_inplace and op_def is not None and op_def.inplace and node.inputs:
            src = _resolve_alias(node.inputs[0], graph)
            if (src not in external and seen_uses[src] == total_uses[src]
                    and _tensor_size(graph, src) == _tensor_size(graph, node.output)):
                memory_root[node.output] = root_of(src)
                continue
        born[node.output] = step

    lifetimes = {name: Lifetime(name, _tensor_size(graph, name), b, dies.get(name, b)) for name, b in born.items()}
    return lifetimes, memory_root


def _compute_scratch(order: list[Node], graph: Graph) -> tuple[dict[str, Lifetime], dict[int, tuple[str, int]]]:
    lifetimes: dict[str, Lifetime] = {}
    info: dict[int, tuple[str, int]] = {}
    for step, node in enumerate(order):
        op_def = OP_REGISTRY.get(node.op)
        if op_def is None or op_def.scratch is None:
            continue
        size = op_def.scratch([graph.tensors[t].shape for t in node.inputs], graph.tensors[node.output].shape,
                              node.attrs)
        if size <= 0:
            continue
        name = f"__scratch_{node.id}"
        lifetimes[name] = Lifetime(name, size, step, step)
        info[node.id] = (name, size)
    return lifetimes, info


# ---------------------------------------------------------------- offsets

def _first_fit(live: list[tuple[int, int]], size: int) -> int:
    cand = 0
    for off, sz in live:
        if cand + size <= off:
            return cand
        cand = max(cand, off + sz)
    return cand


def _best_fit(live: list[tuple[int, int]], size: int) -> int:
    best, waste = -1, float("inf")
    cand = 0
    for off, sz in live:
        gap = off - cand
        if gap >= size and gap - size < waste:
            best, waste = cand, gap - size
        cand = max(cand, off + sz)
    return cand if best < 0 else best


def _assign_offsets(lifetimes: dict[str, Lifetime], n_steps: int,
                    fit: FitStrategy = FitStrategy.FIRST_FIT) -> tuple[dict[str, int], int]:
    choose = _best_fit if fit == FitStrategy.BEST_FIT else _first_fit
    births: dict[int, list[str]] = defaultdict(list)
    evictions: dict[int, list[str]] = defaultdict(list)
    for name, lt in lifetimes.items():
        births[lt.born].append(name)
        evictions[lt.dies + 1].append(name)
    live: dict[str, tuple[int, int]] = {}
    offsets: dict[str, int] = {}
    arena = 0
    for step in range(n_steps):
        for name in evictions.get(step, []):
            live.pop(name, None)
        for name in births.get(step, []):
            size = lifetimes[name].size_bytes
            off = choose(sorted(live.values()), size)
            offsets[name] = off
            live[name] = (off, size)
            arena = max(arena, off + size)
    return offsets, arena


# ---------------------------------------------------------------- plan

def plan(graph: Graph, config: PlannerConfig | None = None) -> MemoryPlan:
    """Order the graph and lay its intermediates out in one arena."""
    config = config or PlannerConfig()
    order = _get_order(graph, config.order)
    lifetimes, memory_root = _compute_lifetimes(graph, order, config)
    scratch_lt, scratch_info = _compute_scratch(order, graph)
    offsets_all, arena_size = _assign_offsets({**lifetimes, **scratch_lt}, n_steps=len(order), fit=config.fit)

    for name, root in memory_root.items():
        while root in memory_root:
            root = memory_root[root]
        if root not in offsets_all:
            continue
        base = offsets_all[root]
        prod = graph.producer(name)
        if prod is not None:
            op_def = OP_REGISTRY.get(prod.op)
            if op_def is not None and op_def.alias_offset is not None:
                base += op_def.alias_offset(prod)
        offsets_all[name] = base

    scratch_names = {n for n, _ in scratch_info.values()}
    offsets = {k: v for k, v in offsets_all.items() if k not in scratch_names}
    scratch = {nid: (offsets_all[n], size) for nid, (n, size) in scratch_info.items()}

    external = set(graph.inputs) | set(graph.constants)
    inter = [n for n in graph.tensors if n not in external]
    stats = PlanStats(
        arena_bytes=arena_size,
        naive_bytes=sum(_tensor_size(graph, n) for n in inter),
        n_intermediates=len(inter),
        n_allocated=len(lifetimes),
        n_shared=len(memory_root),
        scratch_bytes=sum(s for _, s in scratch_info.values()),
        weight_bytes=sum(_tensor_size(graph, n) for n in graph.constants),
    )
    return MemoryPlan(graph=graph, order=order, arena_size=arena_size, offsets=offsets, scratch=scratch,
                      stats=stats)
