"""Write graph_tiny.{json,weights}: a small exported graph saved with the
reference's own Graph.save (runtime/ir.py:363-447), the on-disk format a
user of the reference ships.

    python tests/golden/make_graph_fixture.py

Runs in the build container only (it imports the reference from
/root/reference).  The model is the toy pre-norm block of
lets-build-a-runtime_amd/workloads.py at d_model 32, 2 heads, seq 8, with the
workloads' seeded N(0, 0.02) weights, but with nonzero biases and norm
parameters so every constant carries distinct bytes.  The graph is saved as
exported (before the optimisation passes), as the reference's exporter
returns it.  tests/test_graph_files.py loads it with this repository's
Graph.load and checks it against its own export of the same model;
tests/test_gpu_workloads.py runs it on the GPU.
"""

from __future__ import annotations

import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
REFERENCE = Path("/root/reference")

D_MODEL, HEADS, SEQ = 32, 2, 8


def tiny_model():
    """The fixture's model (shared with the tests, which rebuild it)."""
    import torch
    from workloads import CausalGeluBlock, init_weights
    m = init_weights(CausalGeluBlock(D_MODEL, HEADS), seed=0)
    g = torch.Generator().manual_seed(1)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if p.dim() == 1:
                p.copy_(torch.randn(p.shape, generator=g) * 0.1 + (1.0 if "ln" in name and name.endswith("weight")
                                                                   else 0.0))
    return m.eval()


def tiny_input():
    import numpy as np
    return np.random.default_rng(0).standard_normal((1, SEQ, D_MODEL)).astype(np.float32)


def main() -> None:
    sys.path.insert(0, str(REPO / "lets-build-a-runtime_amd"))
    sys.path.insert(0, str(REFERENCE))           # `runtime` = the reference's package
    import torch
    import runtime
    assert str(REFERENCE) in runtime.__file__, runtime.__file__
    from runtime.exporter import export_model
    g = export_model(tiny_model(), (torch.from_numpy(tiny_input()),))
    g.save(HERE / "graph_tiny")
    print(f"wrote {HERE / 'graph_tiny.json'} and .weights: {len(g.nodes)} nodes, {len(g.constants)} constants")


if __name__ == "__main__":
    main()
