"""Model exporters (framework → graph IR) and an export summary.

Same entry points as the reference (runtime/exporter/__init__.py:25-61):
``export_pytorch``, its alias ``export_model`` and ``summary``.
"""

from collections import Counter

from ..ir import Graph
from .torch import export_pytorch

export_model = export_pytorch


def summary(graph: Graph) -> str:
    """Inputs, outputs, parameter count and op histogram of an exported graph."""
    lines = [f"Inputs ({len(graph.inputs)}):"]
    lines += [f"  {n}: {graph.tensors[n].shape} {graph.tensors[n].dtype}" for n in graph.inputs]
    lines.append(f"Outputs ({len(graph.outputs)}):")
    lines += [f"  {n}: {graph.tensors[n].shape} {graph.tensors[n].dtype}" for n in graph.outputs]
    params = 0
    for n in graph.constants:
        p = 1
        for d in graph.tensors[n].shape:
            p *= d
        params += int(p)
    lines.append(f"Constants: {len(graph.constants)} ({params:,} parameters)")
    lines.append(f"Nodes: {len(graph.nodes)}")
    for op, cnt in Counter(n.op.name for n in graph.nodes.values()).most_common():
        lines.append(f"  {op}: {cnt}")
    return "\n".join(lines)
