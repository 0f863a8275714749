"""Graph IR: op codes, tensor metadata, nodes and the Graph container.

Mirrors the reference's single-level IR (runtime/ir.py:21-484).  The pieces
that other layers depend on bit-for-bit are kept alike on purpose:

* ``OpType`` values are the ABI op codes of ``include/lbr_executor.h``
  (= csrc/runtime.h:11-55, runtime/ir.py:36-90).
* Node ids are handed out sequentially by ``add_node``; consumer lists grow
  in insertion order; the topological order is Kahn's algorithm seeded in
  node-dict order with a FIFO queue (runtime/ir.py:226-249).  The planner's
  memory-aware order breaks ties on node id, so these details decide arena
  offsets and must match the reference for the same export.

Everything else (summary text, serialisation layout) follows the reference's
format so graphs saved by either side load in the other
(runtime/ir.py:309-447).
"""

from __future__ import annotations

import json
from collections import Counter, deque
from dataclasses import dataclass, field
from enum import Enum
from pathlib import Path
from typing import Any, Iterator

import numpy as np


class OpType(Enum):
    """Operator codes (value = the C ABI op code).

    Ranges: 100-199 unary, 200-299 binary, 300-399 reductions, 400-499
    matmul, 500-599 data movement, 600-699 normalisation, 1000-1499 fused,
    5000+ fold-only (evaluated by constant folding, never dispatched).
    """
    RELU = 100
    EXP = 101
    TANH = 102
    POW = 103            # attrs["scalar"] = exponent
    GELU = 104           # tanh approximation
    RSQRT = 105
    SILU = 106
    NEG = 107
    COS = 108
    SIN = 109

    ADD = 200
    SUB = 201
    MUL = 202
    DIV = 203

    MAX = 300            # attrs["axis", "keepdim"]
    SUM = 301            # attrs["axis", "keepdim"]
    SOFTMAX = 302        # attrs["axis"]

    MATMUL = 400         # attrs["transpose_b", "alpha"]

    RESHAPE = 500        # attrs["shape"]
    TRANSPOSE = 501      # attrs["dim0", "dim1"]
    PERMUTE = 502        # attrs["axes"]
    SLICE = 503          # attrs["dim", "start", "end", "byte_offset"]
    EMBEDDING = 504      # inputs [indices, table]
    CAT = 505            # attrs["dim"]

    LAYERNORM = 600      # inputs [x, weight, bias], attrs["eps"]
    RMSNORM = 601        # inputs [x, weight], attrs["eps"]

    MATMUL_ADD = 1000    # inputs [A, B, bias]
    FUSED_BIAS_RELU = 1001
    ATTENTION = 1002     # inputs [Q, K, V(, mask)], attrs["causal", "group_size"]
    GATED_ACT = 1003     # inputs [x, up] / [x, bias, up], attrs["act", "has_bias"]

    CAST = 5000
    EXPAND = 5001
    ARANGE = 5002
    DIFF = 5003
    CMP_NE = 5004
    CMP_LE = 5005
    CMP_EQ = 5006
    CUMSUM = 5007
    BITWISE_AND = 5008
    INDEX = 5009


# Op codes at or above this value are fold-only.
FOLD_ONLY_BASE = 5000


@dataclass
class TensorInfo:
    """A named tensor: static shape/dtype plus the buffer bound before execution.

    ``buffer`` holds weight data for constants; executors bind intermediates
    and inputs themselves.
    """
    name: str
    shape: tuple[int, ...]
    dtype: str = "float32"
    buffer: np.ndarray | None = None


@dataclass
class Node:
    """One operation: op code, input tensor names, one output tensor name."""
    id: int
    op: OpType
    inputs: list[str]
    output: str
    attrs: dict[str, Any] = field(default_factory=dict)


class Graph:
    """Nodes by id, tensors by name, and the graph's input/output/constant roles."""

    def __init__(self) -> None:
        self.nodes: dict[int, Node] = {}
        self.tensors: dict[str, TensorInfo] = {}
        self.inputs: list[str] = []
        self.outputs: list[str] = []
        self.constants: list[str] = []
        self._producer: dict[str, int] = {}
        self._consumers: dict[str, list[int]] = {}
        # symbol -> [(input tensor name, dim index)], set by the exporter
        self.dynamic_dims: dict[str, list[tuple[str, int]]] = {}
        self._next_id = 0
        self._order: list[Node] | None = None

    # ------------------------------------------------------------ building
    def add_tensor(self, name: str, shape: tuple[int, ...], dtype: str = "float32") -> TensorInfo:
        if name in self.tensors:
            raise ValueError(f"Duplicate tensor name: {name}")
        info = TensorInfo(name=name, shape=shape, dtype=dtype)
        self.tensors[name] = info
        self._consumers[name] = []
        return info

    def add_node(self, op: OpType, inputs: list[str], output: str,
                 attrs: dict[str, Any] | None = None) -> Node:
        missing = [t for t in inputs if t not in self.tensors]
        if missing:
            raise ValueError(f"Input tensor '{missing[0]}' not registered")
        if output not in self.tensors:
            raise ValueError(f"Output tensor '{output}' not registered")
        node = Node(id=self._next_id, op=op, inputs=inputs, output=output, attrs=attrs or {})
        self._next_id += 1
        self.nodes[node.id] = node
        self._producer[output] = node.id
        for t in inputs:
            self._consumers[t].append(node.id)
        self._order = None
        return node

    # ------------------------------------------------------------ lookups
    def producer(self, tensor_name: str) -> Node | None:
        nid = self._producer.get(tensor_name)
        return None if nid is None else self.nodes[nid]

    def consumers(self, tensor_name: str) -> list[Node]:
        return [self.nodes[i] for i in self._consumers.get(tensor_name, [])]

    # ------------------------------------------------------------ ordering
    def _toposort(self) -> list[Node]:
        """Kahn's algorithm, FIFO, seeded in node-dict order."""
        pending = {nid: sum(1 for t in n.inputs if t in self._producer) for nid, n in self.nodes.items()}
        ready = deque(nid for nid, deg in pending.items() if deg == 0)
        order: list[Node] = []
        while ready:
            node = self.nodes[ready.popleft()]
            order.append(node)
            for cid in self._consumers.get(node.output, []):
                pending[cid] -= 1
                if pending[cid] == 0:
                    ready.append(cid)
        return order

    def __iter__(self) -> Iterator[Node]:
        if self._order is not None:
            yield from self._order
            return
        order = self._toposort()
        if len(order) != len(self.nodes):
            raise ValueError("Graph has a cycle")
        yield from order

    # ------------------------------------------------------------ reporting
    def summary(self) -> str:
        head = (f"Graph: {len(self.nodes)} nodes, {len(self.tensors)} tensors "
                f"({len(self.inputs)} inputs, {len(self.constants)} constants, "
                f"{len(self.outputs)} outputs)")
        counts = Counter(n.op.name for n in self.nodes.values())
        lines = [head, "  Ops:     " + ", ".join(f"{k}: {v}" for k, v in counts.most_common())]

        def desc(name: str) -> str:
            t = self.tensors[name]
            return f"{name} [{'x'.join(str(d) for d in t.shape)}] {t.dtype}"

        if self.inputs:
            lines.append("  Inputs:  " + ", ".join(desc(n) for n in self.inputs))
        if self.outputs:
            lines.append("  Outputs: " + ", ".join(desc(n) for n in self.outputs))
        return "\n".join(lines)

    def dump(self) -> str:
        lines = [self.summary(), ""]
        for node in self._toposort():
            shape = "x".join(str(d) for d in self.tensors[node.output].shape)
            attrs = ("  " + ", ".join(f"{k}={v}" for k, v in node.attrs.items())) if node.attrs else ""
            lines.append(f"  [{node.id:>3}] {node.op.name:<20} {', '.join(node.inputs)} -> "
                         f"{node.output} ({shape}){attrs}")
        return "\n".join(lines)

    # ------------------------------------------------------------ serialisation
    def to_dict(self) -> dict:
        """Structure only (no weight data); nodes in topological order."""
        return {
            "nodes": [{"id": n.id, "op": n.op.name, "inputs": n.inputs, "output": n.output, "attrs": n.attrs}
                      for n in self._toposort()],
            "tensors": {name: {"shape": list(t.shape), "dtype": t.dtype} for name, t in self.tensors.items()},
            "inputs": self.inputs,
            "constants": self.constants,
            "outputs": self.outputs,
        }

    @classmethod
    def from_dict(cls, d: dict) -> "Graph":
        g = cls()
        for name, info in d["tensors"].items():
            g.add_tensor(name, tuple(info["shape"]), info["dtype"])
        g.inputs = d["inputs"]
        g.constants = d["constants"]
        g.outputs = d["outputs"]
        for nd in d["nodes"]:
            g.add_node(OpType[nd["op"]], nd["inputs"], nd["output"], nd.get("attrs"))
        return g

    def save(self, path: str | Path) -> None:
        """Write ``{path}.json`` (structure + weight manifest) and ``{path}.weights``."""
        path = Path(path)

        def encode(obj):
            if isinstance(obj, np.integer):
                return int(obj)
            if isinstance(obj, np.floating):
                return float(obj)
            if isinstance(obj, tuple):
                return list(obj)
            raise TypeError(f"Not JSON serializable: {type(obj)}")

        d = self.to_dict()
        manifest: dict[str, dict] = {}
        blobs: list[bytes] = []
        offset = 0
        for name in self.constants:
            buf = self.tensors[name].buffer
            if buf is None:
                continue
            raw = np.ascontiguousarray(buf).tobytes()
            manifest[name] = {"offset": offset, "size": len(raw)}
            blobs.append(raw)
            offset += len(raw)
        d["weights"] = manifest
        with open(path.with_suffix(".json"), "w") as f:
            json.dump(d, f, indent=2, default=encode)
        if blobs:
            with open(path.with_suffix(".weights"), "wb") as f:
                for b in blobs:
                    f.write(b)

    @classmethod
    def load(cls, path: str | Path) -> "Graph":
        """Read a graph written by ``save``; constants get buffers if the weights file exists."""
        path = Path(path)
        with open(path.with_suffix(".json")) as f:
            d = json.load(f)
        g = cls.from_dict(d)
        wpath = path.with_suffix(".weights")
        manifest = d.get("weights", {})
        if wpath.exists() and manifest:
            raw = wpath.read_bytes()
            for name, entry in manifest.items():
                info = g.tensors.get(name)
                if info is None:
                    continue
                count = int(np.prod(info.shape))
                info.buffer = np.frombuffer(raw, dtype=np.dtype(info.dtype), offset=entry["offset"],
                                            count=count).reshape(info.shape).copy()
        return g

    # ------------------------------------------------------------ mutation (passes)
    def rewire_input(self, node_id: int, old_tensor: str, new_tensor: str) -> None:
        """Point every occurrence of ``old_tensor`` in the node's inputs at ``new_tensor``."""
        node = self.nodes[node_id]
        for i, name in enumerate(node.inputs):
            if name == old_tensor:
                node.inputs[i] = new_tensor
                self._consumers[old_tensor].remove(node_id)
                self._consumers[new_tensor].append(node_id)
        self._order = None

    def remove_node(self, node_id: int) -> None:
        """Drop a node and its connectivity (its output tensor stays registered)."""
        node = self.nodes.pop(node_id)
        self._producer.pop(node.output, None)
        for name in node.inputs:
            users = self._consumers.get(name, [])
            if node_id in users:
                users.remove(node_id)
        self._order = None

    def remove_tensor(self, name: str) -> None:
        self.tensors.pop(name, None)
        self._consumers.pop(name, None)
        self._producer.pop(name, None)
        self._order = None
