"""Session: optimise → (resolve) → plan → compile → run.

Same API as the reference (runtime/session.py:79-229):

    graph = export_model(model, (x,))
    session = Session(graph)
    session.create()                       # compiled executor, on the GPU
    out = session.run({"x": x_numpy})
    session.rebind({"L": 64})              # new shapes, passes not re-run

``execution_mode="compiled"`` builds the device executor; its weights stay
resident across ``rebind`` calls when the constants are unchanged.
``execution_mode="interpreted"`` (the reference's per-node CPU debug path)
is not provided by this backend and raises.

``rebind`` keeps the last ``plan_cache`` compiled plans (arena, node array,
hipGraph) keyed by their bindings: returning to a shape seen before switches
to its plan without re-planning or re-capturing.  All cached plans share one
device copy of the weights.
"""

from __future__ import annotations

from collections import OrderedDict

import numpy as np

from .executor.common import Executor, RunProfile
from .ir import Graph
from .ops import resolve_graph
from .passes.passes import Pass, PassResult, run_pipeline, run_until_stable
from .planner import ExecutionPlan, PlanStats, plan
from .validation import Phase, Severity, run_validators


class Session:
    def __init__(self, graph: Graph) -> None:
        self._graph = graph
        self._resolved: Graph | None = None
        self._executor: Executor | None = None
        self._plan_stats: PlanStats | None = None
        self._pass_log: list[PassResult] | None = None
        self._optimized = False
        self._execution_mode = "compiled"
        self._backend = "hip"
        self._profile = False
        self._memory_plan = None
        # rebind cache: bindings key → (executor, resolved graph, memory plan), least recent first
        self._plans: OrderedDict = OrderedDict()
        self._plan_cache = 8
        self._key = None
        self._weights: list = []      # device weight blocks shared by the cached executors

    @staticmethod
    def _bindings_key(bindings: dict[str, int] | None):
        return tuple(sorted((bindings or {}).items()))

    @property
    def cached_plans(self) -> list:
        """Bindings of the compiled plans kept for rebind, least recently used first."""
        return [dict(k) for k in self._plans]

    @property
    def graph(self) -> Graph:
        return self._graph

    @property
    def resolved_graph(self) -> Graph | None:
        return self._resolved

    @property
    def memory_plan(self):
        return self._memory_plan

    @property
    def executor(self) -> Executor | None:
        return self._executor

    @property
    def plan_stats(self) -> PlanStats | None:
        return self._plan_stats

    @property
    def pass_log(self) -> list[PassResult] | None:
        return self._pass_log

    @property
    def last_profile(self) -> RunProfile | None:
        return None if self._executor is None else self._executor._last_profile

    def create(self, execution_mode: str = "compiled", backend: str = "hip", optimization: str = "default",
               pipeline: list[Pass] | None = None, verbose: bool = False, profile: bool = False,
               bindings: dict[str, int] | None = None, validation: str = "normal",
               use_graph: bool = True, plan_cache: int = 8) -> None:
        """Optimise (once), resolve ``bindings``, plan, validate and compile.

        optimization: "none" | "default" (pipeline once) | "aggressive" (until stable)
        validation:   "strict" (fail on warnings) | "normal" (fail on errors) | "none"
        use_graph:    capture the launch sequence into a hipGraph (default) or launch eagerly
        plan_cache:   compiled plans kept for rebind (≥ 1)
        """
        self.close()
        self._execution_mode = execution_mode
        self._backend = backend
        self._profile = profile
        self._use_graph = use_graph
        self._plan_cache = max(1, int(plan_cache))
        fail_on = _validation_severity(validation)
        self._check_mode(execution_mode)

        if not self._optimized:
            if verbose:
                print(self._graph.summary())
                print()
            log = [] if verbose else None
            if optimization == "default":
                run_pipeline(self._graph, pipeline, log=log)
            elif optimization == "aggressive":
                run_until_stable(self._graph, pipeline, log=log)
            if verbose and log:
                for entry in log:
                    print(entry)
                print()
                print(self._graph.summary())
                print()
            self._pass_log = log
            self._optimized = True
            self._validate(Phase.POST_OPTIMIZE, self._graph, fail_on, verbose)

        self._resolved = resolve_graph(self._graph, bindings) if bindings else self._graph
        self._validate(Phase.POST_RESOLVE_OPTIMIZE, self._resolved, fail_on, verbose)

        mem = plan(self._resolved)
        self._memory_plan = mem
        self._plan_stats = mem.stats
        if verbose and self._plan_stats:
            print(self._plan_stats)
            print()
        self._validate(Phase.POST_PLAN, mem, fail_on, verbose)
        self._validate(Phase.PRE_EXECUTE, ExecutionPlan(self._resolved, mem, execution_mode, backend), fail_on,
                       verbose)

        ex = self._make_executor(execution_mode, backend, profile)
        ex.compile(mem)
        self._adopt(self._bindings_key(bindings), ex)

    def rebind(self, bindings: dict[str, int]) -> None:
        """Switch to new symbol values (passes are not re-run): the cached plan for these
        bindings if there is one, else re-resolve, re-plan and re-compile (session.py:187-207
        of the reference), sharing the resident weights."""
        key = self._bindings_key(bindings)
        if key == self._key and self._executor is not None:
            return
        if key in self._plans:
            self._plans.move_to_end(key)
            self._executor, self._resolved, self._memory_plan = self._plans[key]
            self._plan_stats = self._memory_plan.stats
            self._key = key
            return
        self._resolved = resolve_graph(self._graph, bindings)
        mem = plan(self._resolved)
        self._memory_plan = mem
        self._plan_stats = mem.stats
        ex = self._make_executor(self._execution_mode, self._backend, self._profile,
                                 weights=self._weights[-1] if self._weights else None)
        ex.compile(mem)
        self._adopt(key, ex)

    def run(self, inputs: dict[str, np.ndarray], profile: bool = False) -> dict[str, np.ndarray]:
        if self._executor is None:
            raise RuntimeError("Session not created — call create() first")
        if profile:
            self._executor._profile = True
        try:
            return self._executor.run(inputs)
        finally:
            if profile:
                self._executor._profile = self._profile

    def close(self) -> None:
        """Free every cached plan's device memory and the weights now (otherwise freed when
        the session is collected)."""
        execs = [e for e, _, _ in self._plans.values()]
        if self._executor is not None and all(self._executor is not e for e in execs):
            execs.append(self._executor)
        for e in execs:
            if hasattr(e, "close"):
                e.close()
        for w in self._weights:
            w.free()
        self._plans.clear()
        self._weights = []
        self._executor = None
        self._key = None

    # ------------------------------------------------------------------ internals
    def _adopt(self, key, ex: Executor) -> None:
        """Make `ex` current and cache it under `key`; the session takes over its weights
        (shared with later plans) and evicts the least recently used plan beyond the cache size."""
        if hasattr(ex, "release_weights"):
            w = ex.release_weights()
            if w is not None and all(w is not v for v in self._weights):
                self._weights.append(w)
        self._executor = ex
        self._key = key
        self._plans[key] = (ex, self._resolved, self._memory_plan)
        self._plans.move_to_end(key)
        while len(self._plans) > self._plan_cache:
            _, (old, _, _) = self._plans.popitem(last=False)
            if old is not ex and hasattr(old, "close"):
                old.close()

    @staticmethod
    def _check_mode(execution_mode: str) -> None:
        if execution_mode == "interpreted":
            raise NotImplementedError("execution_mode='interpreted' (per-node CPU dispatch) is not provided by "
                                      "the MI355X backend; use execution_mode='compiled'")
        if execution_mode != "compiled":
            raise ValueError(f"Unknown execution_mode '{execution_mode}' (expected 'compiled' or 'interpreted')")

    @staticmethod
    def _validate(phase: Phase, target, fail_on: Severity | None, verbose: bool) -> None:
        if fail_on is None:
            return
        results = run_validators(phase, target, fail_on=fail_on)
        if verbose and results:
            for r in results:
                print(r)

    def _make_executor(self, execution_mode: str, backend: str, profile: bool = False, weights=None) -> Executor:
        self._check_mode(execution_mode)
        from .executor.compiled import CompiledExecutor
        return CompiledExecutor(profile=profile, use_graph=getattr(self, "_use_graph", True), weights=weights)


def _validation_severity(validation: str) -> Severity | None:
    if validation == "strict":
        return Severity.WARNING
    if validation == "normal":
        return Severity.ERROR
    if validation == "none":
        return None
    raise ValueError(f"Unknown validation '{validation}' (expected 'strict', 'normal', or 'none')")
