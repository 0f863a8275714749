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
"""

from __future__ import annotations

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
               use_graph: bool = True) -> None:
        """Optimise (once), resolve ``bindings``, plan, validate and compile.

        optimization: "none" | "default" (pipeline once) | "aggressive" (until stable)
        validation:   "strict" (fail on warnings) | "normal" (fail on errors) | "none"
        use_graph:    capture the launch sequence into a hipGraph (default) or launch eagerly
        """
        self._execution_mode = execution_mode
        self._backend = backend
        self._profile = profile
        self._use_graph = use_graph
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
        self._replace_executor(ex)

    def rebind(self, bindings: dict[str, int]) -> None:
        """Re-resolve, re-plan and re-compile for new symbol values (passes are not re-run)."""
        self._resolved = resolve_graph(self._graph, bindings)
        mem = plan(self._resolved)
        self._memory_plan = mem
        self._plan_stats = mem.stats
        weights = None
        if self._executor is not None and hasattr(self._executor, "release_weights"):
            weights = self._executor.release_weights()
        ex = self._make_executor(self._execution_mode, self._backend, self._profile, weights=weights)
        ex.compile(mem)
        self._replace_executor(ex)

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
        """Free the executor's device memory now (otherwise freed when the session is collected)."""
        if self._executor is not None and hasattr(self._executor, "close"):
            self._executor.close()
        self._executor = None

    # ------------------------------------------------------------------ internals
    def _replace_executor(self, ex: Executor) -> None:
        old = self._executor
        self._executor = ex
        if old is not None and old is not ex and hasattr(old, "close"):
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
