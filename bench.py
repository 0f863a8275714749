#!/usr/bin/env python3
"""Benchmark: fp32 forward of a BASELINE workload through Session on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config KEY]

A step is one forward pass (Session's compiled plan, replayed as a hipGraph)
over one batch of synthetic input that is already resident in HBM.  W
untimed warm-up steps, then exactly K steps between two device
synchronisations; ms_per_step is host wall time / K (hipEvent time on the
library stream is reported beside it).  value = tokens/s = batch·seq /
(ms_per_step/1000).

With no --config the headline is the 7B-shaped block at S=4096 (BASELINE
configs[3]) and `configs` carries the same measurement for every BASELINE
shape in order (toy, gpt2w, gpt2, 7b4k, qwen3_4b), then the two full language
models the reference publishes latencies for (gpt2_lm: GPT-2 with embeddings
and LM head, qwen3_4b_lm: the Qwen3-4B-shaped body with embeddings and LM
head, both at S=1024), each with its own latency, roofline, kernel table,
schedule (GEMM tiles and K ranges, attention kernel), parity and CPU
baseline; --config KEY measures one workload only.

Also reported, on the same JSON line:
  roofline      dominant kernel (largest share of device time): algorithmic
                FLOPs (or bytes) per launch ÷ its mean launch duration,
                measured with hipEvent pairs on the library stream over K
                eager steps, against MI355X peak (fp32 MFMA 157.3 TFLOP/s,
                HBM 8 TB/s); `traffic` = HBM bytes per launch from the
                committed rocprofv3 counter summary when one exists;
  kernels       the same per-kernel figures for every kernel in the step;
  parity        GPU output vs the CPU oracle on the same plan and input;
  cpu_baseline  the oracle (C restatement of the reference CPU executor),
                the median of three whole forwards of the same workload after
                a warm-up, on the host's cores; `host` states nproc, the CPU
                model, OMP_NUM_THREADS and which sgemm ran;
  latency       single-replay median and the end-to-end Session.run time
                (input and output copies included).

Only one GPU is used; --gpus above 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT / "lets-build-a-runtime_amd"), str(ROOT)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
METRIC = "fp32 forward latency (ms) + tokens/s per shape; MFMA % and HBM GB/s of roofline"
HEADLINE = "7b4k"   # BASELINE configs[3], the north star's named target


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------- per-node work

def node_work(node, graph) -> tuple[float, float]:
    """(algorithmic FLOPs, algorithmic HBM bytes) of one dispatched node.

    GEMM: 2·M·N·K flops, bytes = A + B + C (+ bias).  Attention: 4·bh·S²·hd,
    halved when causal; bytes = Q + K + V + O.  Memory-bound ops: minimum
    traffic, every input element read once and the output written once.
    """
    from runtime.ir import OpType
    from runtime.ops import OP_REGISTRY

    def numel(name):
        n = 1
        for d in graph.tensors[name].shape:
            n *= d
        return n

    def nbytes(name):
        return numel(name) * np.dtype(graph.tensors[name].dtype).itemsize

    out_b = nbytes(node.output)
    op = node.op
    if op in (OpType.MATMUL, OpType.MATMUL_ADD):
        ex = OP_REGISTRY[op].extras(node, graph)
        K = ex[0]
        shape = graph.tensors[node.output].shape
        flops = 2.0 * numel(node.output) * K
        return flops, float(sum(nbytes(t) for t in node.inputs) + out_b)
    if op == OpType.ATTENTION:
        q = graph.tensors[node.inputs[0]].shape
        bh = int(np.prod(q[:-2]))
        s, hd = q[-2], q[-1]
        flops = 4.0 * bh * s * s * hd * (0.5 if node.attrs.get("causal") else 1.0)
        return flops, float(sum(nbytes(t) for t in node.inputs[:3]) + out_b)
    if op == OpType.EMBEDDING:
        # a gather: the ids, the table rows it reads (as many bytes as it writes) and the output
        return 0.0, float(nbytes(node.inputs[0]) + 2 * out_b)
    return 0.0, float(sum(nbytes(t) for t in node.inputs) + out_b)


def step_units(names, order, graph, ms, runs):
    """One entry per kernel step: fused runs (first, count, kind) become one unit.

    A fused run's work: the flops of its GEMM/attention nodes; bytes = what it
    reads from outside the run (for a SLICE of an outside tensor, only the
    sliced part) plus the outputs that leave the run (read by a later node or
    graph outputs).  Views (RESHAPE, dim-0 SLICE: never dispatched, they alias
    their input, runtime/ops.py:411-415) are resolved to the tensor that owns
    the memory, so a view of a tensor made inside the run is not an outside
    read, and a later read through a view still takes the run's output."""
    from runtime.planner import _resolve_alias

    def nbytes(t):
        return float(np.prod(graph.tensors[t].shape)) * np.dtype(graph.tensors[t].dtype).itemsize

    start = {f: c for f, c, _ in runs}
    units, i = [], 0
    while i < len(order):
        c = start.get(i, 1)
        nodes = order[i:i + c]
        if c == 1:
            f, b = node_work(nodes[0], graph)
        else:
            inside = {_resolve_alias(n.output, graph) for n in nodes}
            later = {_resolve_alias(t, graph) for n in order[i + c:] for t in n.inputs}
            later |= {_resolve_alias(t, graph) for t in graph.outputs}
            f, b = 0.0, 0.0
            seen = set()
            for n in nodes:
                nf, _ = node_work(n, graph)
                f += nf
                for t in n.inputs:
                    root = _resolve_alias(t, graph)
                    if root in inside:
                        continue
                    # a view as large as its root reads the same bytes as the root
                    key = root if nbytes(t) == nbytes(root) else t
                    if key in seen:
                        continue
                    seen.add(key)
                    b += nbytes(n.output) if n.op.name == "SLICE" else nbytes(t)
            for n in nodes:
                if _resolve_alias(n.output, graph) in later:
                    b += nbytes(n.output)
        units.append({"name": names[i], "nodes": nodes, "ms": ms[i], "flops": f, "bytes": float(b)})
        i += c
    return units


def kernel_table(units):
    """Aggregate per-step device times by device kernel: a fused step is named
    `<kernel>+<epilogue>` and runs `<kernel>`, so it counts under `<kernel>`
    (the grouping rocprofv3 reports, by kernel function)."""
    agg: dict[str, dict] = {}
    for u in units:
        base = u["name"].split("+")[0]
        a = agg.setdefault(base, {"kernel": base, "launches": 0, "ms": 0.0, "flops": 0.0, "bytes": 0.0})
        a["launches"] += 1
        a["ms"] += u["ms"]
        a["flops"] += u["flops"]
        a["bytes"] += u["bytes"]
    rows = []
    total = sum(a["ms"] for a in agg.values()) or 1.0
    for a in agg.values():
        sec = max(a["ms"], 1e-9) / 1e3
        mfma = a["flops"] > 0
        achieved = (a["flops"] / sec / 1e12) if mfma else (a["bytes"] / sec / 1e9)
        peak = PEAK_FP32_MFMA_TFLOPS if mfma else PEAK_HBM_GBS
        rows.append({
            "kernel": a["kernel"], "launches": a["launches"], "ms_per_step": round(a["ms"], 4),
            "share": round(a["ms"] / total, 4), "bound": "mfma" if mfma else "hbm",
            "achieved": round(achieved, 2), "unit": "TFLOP/s" if mfma else "GB/s", "frac": round(achieved / peak, 4),
            "flops_per_launch": a["flops"] / a["launches"], "bytes_per_launch": a["bytes"] / a["launches"],
            "mean_launch_us": round(a["ms"] * 1e3 / a["launches"], 2),
        })
    rows.sort(key=lambda r: r["ms_per_step"], reverse=True)
    return rows


def committed_traffic(kernel: str, workload: str):
    """HBM bytes per launch from profiles/traffic_<kernel>_<workload>.json (rocprofv3 --pmc), if committed."""
    p = ROOT / "profiles" / f"traffic_{kernel}_{workload}.json"
    if p.exists():
        try:
            return json.loads(p.read_text()).get("bytes_per_launch")
        except Exception:
            return None
    return None


def calibrate_copy(mib: int) -> int:
    """Run the device copy kernel (a RESHAPE node through lbr_execute) over `mib` MiB, 5 times.

    Under ``rocprofv3 --pmc FETCH_SIZE`` / ``WRITE_SIZE`` its per-dispatch
    counters read ≈ mib·1024 KiB each; the ratio scales the counters of the
    benchmarked kernels to bytes.
    """
    from runtime.executor.common import COpNode
    from runtime.executor.hip_lib import load_library
    lib = load_library(0)
    n = mib * 2**20
    src, dst = lib.alloc(n), lib.alloc(n)
    host = np.arange(n // 4, dtype=np.float32)
    lib.h2d(src, host.ctypes.data, n)
    node = (COpNode * 1)()
    node[0].op = 500  # RESHAPE of an external buffer = plain copy
    node[0].n_inputs = 1
    node[0].inputs[0] = src
    node[0].output = dst
    node[0].n_dims = 1
    node[0].out_shape[0] = n // 4
    node[0].elem_size = 4
    for _ in range(5):
        lib.check(lib.lbr_execute(node, 1), "lbr_execute(copy)")
    back = np.empty_like(host)
    lib.d2h(back.ctypes.data, dst, n)
    ok = bool(np.array_equal(back, host))
    lib.free(src)
    lib.free(dst)
    print(json.dumps({"calibration": "copy", "bytes_read": n, "bytes_written": n, "dispatches": 5, "ok": ok}))
    return 0 if ok else 1


def memory_floor(rows: int = 1024, cols: int = 2560, reps: int = 20) -> int:
    """The memory-bound floor beside the norms, in one process: the library's float4
    copy (a RESHAPE of an external buffer) of rows·cols floats, then RMSNORM and
    LAYERNORM over the same [rows, cols] (Qwen3-4B's hidden rows at S=1024), each
    launched `reps` times through lbr_execute.  Under ``rocprofv3 --kernel-trace``
    the three kernels' mean durations compare the norms' one read + one write of
    the rows with a plain copy of the same bytes."""
    import struct
    from runtime.executor.common import COpNode
    from runtime.executor.hip_lib import load_library
    lib = load_library(0)
    n = rows * cols * 4
    r = np.random.default_rng(0)
    x_h = r.standard_normal(rows * cols).astype(np.float32)
    w_h = r.standard_normal(cols).astype(np.float32)
    x, y, w, b = lib.alloc(n), lib.alloc(n), lib.alloc(cols * 4), lib.alloc(cols * 4)
    lib.h2d(x, x_h.ctypes.data, n)
    lib.h2d(w, w_h.ctypes.data, cols * 4)
    lib.h2d(b, w_h.ctypes.data, cols * 4)

    def node(op, inputs, eps=None):
        nd = (COpNode * 1)()
        nd[0].op = op
        nd[0].n_inputs = len(inputs)
        for k, p_ in enumerate(inputs):
            nd[0].inputs[k] = p_
        nd[0].output = y
        if op == 500:   # RESHAPE: a flat copy
            nd[0].n_dims, nd[0].out_shape[0] = 1, rows * cols
        else:
            nd[0].n_dims, nd[0].out_shape[0], nd[0].out_shape[1] = 2, rows, cols
            nd[0].extra[0] = struct.unpack("<i", struct.pack("<f", eps))[0]
        nd[0].elem_size = 4
        return nd

    out = {"memory_floor": {"rows": rows, "cols": cols, "reps": reps, "bytes_read": n, "bytes_written": n}}
    for name, nd in (("copy", node(500, [x])), ("rmsnorm", node(601, [x, w], 1e-6)),
                     ("layernorm", node(600, [x, w, b], 1e-5))):
        for _ in range(reps):
            lib.check(lib.lbr_execute(nd, 1), f"lbr_execute({name})")
        out["memory_floor"][name] = "ok"
    for p_ in (x, y, w, b):
        lib.free(p_)
    print(json.dumps(out))
    return 0


# ---------------------------------------------------------------- host facts

def host_facts() -> dict:
    """What the CPU baseline ran on: core counts, CPU model, thread settings, sgemm."""
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    return {"nproc": affinity, "cpu_count": os.cpu_count(), "cpu_model": model,
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS"),
            "sgemm": "the oracle's own cache-blocked OpenMP fp32 sgemm (no CBLAS library is linked; the reference "
                     "links OpenBLAS cblas_sgemm, csrc/Makefile:10-13, which this image does not have)"}


# ---------------------------------------------------------------- one workload

def measure(key: str, args, graph_stem: str | None = None, min_timed_ms: float = 0.0) -> dict:
    """Export (or load) one workload, compile it through Session, and measure it.

    min_timed_ms > 0 (the non-headline configs): time at least --steps steps and
    enough more that the timed region covers that many milliseconds, so that
    host-side jitter does not dominate a step of a few µs; the headline times
    exactly --steps."""
    from runtime.session import Session
    from workloads import WORKLOADS, export_workload

    t0 = time.time()
    if graph_stem:
        # a saved graph: seeded N(0,1) input of the graph's input shape
        from runtime.ir import Graph
        graph = Graph.load(graph_stem)
        shape = tuple(graph.tensors[graph.inputs[0]].shape)
        x = np.random.default_rng(0).standard_normal(shape).astype(np.float32)
        title, d_model = f"saved graph {Path(graph_stem).name}", int(shape[-1])
    else:
        wl = WORKLOADS[key]
        model, x, graph = export_workload(key)
        del model
        title, d_model = wl.title, int(x.shape[2]) if x.ndim == 3 else int(getattr(wl, "d_model", 0))
    sess = Session(graph)
    sess.create(use_graph=not args.eager)
    ex = sess.executor
    log(f"[bench] {title}: export+optimise+plan+compile {time.time() - t0:.1f}s, "
        f"{len(ex.dispatch_order)} nodes/step, {len(ex.fused_runs())} fused runs, "
        f"arena {sess.plan_stats.arena_bytes / 2**20:.1f} MiB")

    ex.upload_inputs({graph.inputs[0]: x})
    for _ in range(args.warmup):
        ex.launch()
    ex.synchronize()
    steps = args.steps
    if min_timed_ms > 0:
        est = ex.time_launches(max(1, args.warmup)) / max(1, args.warmup)
        steps = max(steps, int(np.ceil(min_timed_ms / max(est, 1e-3))))
    t_start = time.perf_counter()
    for _ in range(steps):
        ex.launch()
    ex.synchronize()
    wall_ms = (time.perf_counter() - t_start) * 1e3 / steps
    event_ms = ex.time_launches(steps) / steps
    tokens = x.shape[0] * x.shape[1]
    log(f"[bench] {steps} steps: {wall_ms:.3f} ms/step wall, {event_ms:.3f} ms/step hipEvent")
    # median of single replays (hipEvent pair around each graph launch), and the end-to-end
    # Session.run wall time with the input H2D and output D2H copies included
    replays = max(20, args.steps)
    replay_ms = float(np.median([ex.time_launches(1) for _ in range(replays)]))
    run_wall = []
    for _ in range(6):
        t1 = time.perf_counter()
        sess.run({graph.inputs[0]: x})
        run_wall.append((time.perf_counter() - t1) * 1e3)
    session_run_ms = float(np.median(run_wall[1:]))      # the first run also allocates pinned output memory
    io_bytes = x.nbytes + sum(int(np.prod(sess.resolved_graph.tensors[o].shape)) * 4 for o in graph.outputs)
    log(f"[bench] replay median {replay_ms:.3f} ms; Session.run (H2D + replay + D2H) median {session_run_ms:.3f} ms")

    # per-kernel device time (eager launches, hipEvent pairs on the library stream)
    names = ex.kernel_names()
    node_ms = ex.profile_nodes(max(1, min(args.steps, 20)))
    rg = sess.resolved_graph
    runs = ex.fused_runs()
    units = step_units(names, ex.dispatch_order, rg, node_ms, runs)
    rows = kernel_table(units)
    dom = rows[0]
    if args.nodes:
        for u in units:
            node, t, f, b = u["nodes"][0], u["ms"], u["flops"], u["bytes"]
            rate = f"{f / t / 1e9:8.1f} TF/s {100 * f / t / 1e9 / PEAK_FP32_MFMA_TFLOPS:5.1f}%" if f else \
                f"{b / t / 1e6:8.1f} GB/s {100 * b / t / 1e6 / PEAK_HBM_GBS:5.1f}%"
            ops = "+".join(n.op.name for n in u["nodes"]) if len(u["nodes"]) <= 3 else \
                f"{u['nodes'][0].op.name}+{len(u['nodes']) - 1} nodes"
            log(f"[node] {node.id:>4} {ops:<24} {u['name']:<24} {str(rg.tensors[node.output].shape):<22} "
                f"{t * 1e3:9.1f} us {rate}")
    for r in rows:
        log(f"[bench]   {r['kernel']:<22} x{r['launches']:<3} {r['ms_per_step']:8.3f} ms "
            f"({100 * r['share']:5.1f}%)  {r['achieved']:9.2f} {r['unit']:<8} {100 * r['frac']:5.1f}% of peak")

    y = ex.download_outputs()[graph.outputs[0]]
    parity = cpu = None
    if not (args.no_parity and args.no_cpu):
        from oracle.host_exec import OracleRun, num_threads
        orc = OracleRun(sess.memory_plan)
        times = []
        runs_cpu = 1 if args.no_cpu else 4          # one warm-up (also the parity run), then three timed
        for _ in range(runs_cpu):
            t1 = time.perf_counter()
            o = orc.run({graph.inputs[0]: x})[graph.outputs[0]]
            times.append(time.perf_counter() - t1)
        err = float(np.abs(y.astype(np.float64) - o).max())
        rel = err / float(np.abs(o).max())
        parity = {"vs": "cpu oracle, same plan and input", "max_abs_err": err, "normwise_rel_err": rel,
                  "tolerance": 1e-3, "ok": bool(np.isfinite(y).all() and rel <= 1e-3)}
        log(f"[bench] parity vs oracle: normwise rel {rel:.3e}, max abs {err:.3e}")
        if not args.no_cpu:
            cpu_s = float(np.median(times[1:]))
            cpu = {"value": round(tokens / cpu_s, 2), "unit": "tokens/s", "cores": num_threads(),
                   "kind": "port", "ms_per_step": round(cpu_s * 1e3, 2), "runs": len(times) - 1,
                   "statistic": "median of 3 forwards after 1 warm-up",
                   "sample": f"whole forward of the same workload ({title}) on the CPU oracle, same plan and "
                             f"input: a C restatement of the reference compiled executor that differs from its "
                             f"Linux schedule in two ways: the attention batch x head loop runs in parallel "
                             f"(OpenMP; the reference's Linux loop is serial, csrc/ops.h:56-57) and the GEMMs use "
                             f"the oracle's own cache-blocked OpenMP sgemm, not OpenBLAS cblas_sgemm"}
            log(f"[bench] cpu oracle: {cpu_s * 1e3:.2f} ms/forward (median of {len(times) - 1}) on "
                f"{num_threads()} threads")

    traffic = committed_traffic(dom["kernel"], key)
    ms_per_step = wall_ms
    result = {
        "workload": key, "title": title, "batch": int(x.shape[0]), "seq_len": int(x.shape[1]),
        "d_model": d_model, "tokens_per_s": round(tokens / (ms_per_step / 1e3), 2),
        "ms_per_step": round(ms_per_step, 4), "event_ms_per_step": round(event_ms, 4), "steps": steps,
        "latency": {"replay_median_ms": round(replay_ms, 4), "replays": replays,
                    "session_run_median_ms": round(session_run_ms, 4), "session_runs": len(run_wall) - 1,
                    "session_run_io_bytes": int(io_bytes),
                    "session_run_includes": "input H2D copy (pinned ring), graph replay, output D2H copy "
                                            "(into pinned memory); median after one run that allocates"},
        "graph": "hipGraph replay" if not args.eager else "eager launches",
        "nodes_per_step": len(ex.dispatch_order), "kernels_per_step": len(units), "fused_runs": len(runs),
        "roofline": {"kernel": dom["kernel"], "bound": dom["bound"], "achieved": dom["achieved"],
                     "peak": PEAK_FP32_MFMA_TFLOPS if dom["bound"] == "mfma" else PEAK_HBM_GBS,
                     "unit": dom["unit"], "frac": dom["frac"], "traffic": traffic,
                     "mean_launch_us": dom["mean_launch_us"], "launches_per_step": dom["launches"],
                     "work_per_launch": dom["flops_per_launch"] if dom["bound"] == "mfma"
                     else dom["bytes_per_launch"]},
        "kernels": [{k: r[k] for k in ("kernel", "launches", "ms_per_step", "share", "achieved", "unit", "frac",
                                       "mean_launch_us")} for r in rows],
        "schedule": [{k: v for k, v in p.items() if k not in ("first", "count", "kernel")}
                     for p in ex.step_params() if p["kernel"].startswith(("gemm_", "attn_"))],
        "parity": parity,
        "cpu_baseline": cpu,
    }
    sess.close()
    return result


# ---------------------------------------------------------------- main

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default=None,
                    help="measure only this workload (toy, gpt2w, gpt2, 7b4k, qwen3_4b, gpt2_lm, qwen3_4b_lm); "
                         "default: the 7b4k headline plus every BASELINE config in `configs`")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-parity", action="store_true", help="skip the GPU-vs-oracle output check")
    ap.add_argument("--eager", action="store_true", help="launch node by node instead of replaying a hipGraph")
    ap.add_argument("--nodes", action="store_true", help="log every node's device time and roofline fraction")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run the library's copy kernel over MIB MiB, 5 times (reference for HBM counters)")
    ap.add_argument("--memory-floor", action="store_true",
                    help="only run the copy kernel, RMSNORM and LAYERNORM over the same 1024x2560 rows, 20 times "
                         "each (the memory-bound floor beside the norms, for rocprofv3 --kernel-trace)")
    ap.add_argument("--save-graph", metavar="STEM",
                    help="only export the --config workload and write STEM.json + STEM.weights")
    ap.add_argument("--graph", metavar="STEM",
                    help="run a saved graph (STEM.json + STEM.weights) instead of exporting --config")
    args = ap.parse_args()
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy)
    if args.memory_floor:
        return memory_floor()
    if args.save_graph:
        from workloads import export_workload
        _, _, graph = export_workload(args.config or HEADLINE)
        graph.save(args.save_graph)
        log(f"[bench] wrote {args.save_graph}.json/.weights ({len(graph.nodes)} nodes, {len(graph.constants)} "
            f"constants) for workload {args.config or HEADLINE}")
        return 0

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(the multi-GPU sharding is a design note only; nothing here launches collectives)",
              file=sys.stderr)
        return 2

    from workloads import CONFIG_ORDER, LM_ORDER
    if args.graph:
        head = measure(Path(args.graph).name, args, graph_stem=args.graph)
        others = []
    else:
        head_key = args.config or HEADLINE
        head = measure(head_key, args)
        others = [] if args.config else [k for k in CONFIG_ORDER + LM_ORDER if k != head_key]
    per_shape = []
    for k in others:
        per_shape.append(measure(k, args, min_timed_ms=30.0))
    if per_shape:
        by_key = {r["workload"]: r for r in per_shape}
        by_key[head["workload"]] = dict(head, headline=True)
        per_shape = [by_key[k] for k in CONFIG_ORDER + LM_ORDER if k in by_key]

    cpu = head["cpu_baseline"]
    if cpu is not None:
        cpu = dict(cpu, host=host_facts())
    result = {
        "metric": METRIC,
        "value": head["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "event_ms_per_step": head["event_ms_per_step"],
        "latency": head["latency"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) input, random-init N(0,0.02) weights)"
                if not head["workload"].endswith("_lm") else
                "synthetic (seeded uniform token ids, random-init N(0,0.02) weights)",
        "config": {"workload": head["workload"], "title": head["title"], "batch": head["batch"],
                   "seq_len": head["seq_len"], "d_model": head["d_model"], "graph": head["graph"],
                   "nodes_per_step": head["nodes_per_step"], "kernels_per_step": head["kernels_per_step"],
                   "fused_runs": head["fused_runs"]},
        "roofline": head["roofline"],
        "kernels": head["kernels"],
        "schedule": head["schedule"],
        "parity": head["parity"],
        "cpu_baseline": cpu,
    }
    if per_shape:
        result["configs"] = per_shape
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
