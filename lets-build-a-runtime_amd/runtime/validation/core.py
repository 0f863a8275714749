"""Validation phases, severities, the validator registry and its runner.

Same contract as runtime/validation/core.py:12-131 of the reference:
validators are tagged with a pipeline phase, return ``ValidationResult``s,
and ``run_validators`` raises ``ValidationError`` when any result is at or
above ``fail_on`` severity.
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum, auto
from typing import Any, Callable


class Phase(Enum):
    POST_EXPORT = auto()            # Graph
    POST_OPTIMIZE = auto()          # Graph
    POST_RESOLVE = auto()           # Graph
    POST_RESOLVE_OPTIMIZE = auto()  # Graph
    POST_PLAN = auto()              # MemoryPlan
    PRE_EXECUTE = auto()            # ExecutionPlan


class Severity(Enum):
    ERROR = auto()
    WARNING = auto()
    INFO = auto()


@dataclass
class ValidationResult:
    validator: str
    severity: Severity
    message: str

    def __str__(self) -> str:
        return f"[{self.severity.name}] {self.validator}: {self.message}"


class ValidationError(Exception):
    def __init__(self, phase: Phase, results: list[ValidationResult]) -> None:
        self.phase = phase
        self.results = results
        errors = [r for r in results if r.severity == Severity.ERROR]
        super().__init__(f"Validation failed at {phase.name} ({len(errors)} error(s)):\n"
                         + "\n".join(f"  {r}" for r in errors))


@dataclass
class Validator:
    name: str
    phase: Phase
    check: Callable[..., list[ValidationResult]]


VALIDATORS: list[Validator] = []


def register_validator(name: str, phase: Phase):
    def deco(fn):
        VALIDATORS.append(Validator(name=name, phase=phase, check=fn))
        return fn
    return deco


def run_validators(phase: Phase, target: Any, *, fail_on: Severity | None = Severity.ERROR) -> list[ValidationResult]:
    results: list[ValidationResult] = []
    for v in VALIDATORS:
        if v.phase == phase:
            results.extend(v.check(target))
    if fail_on is not None and any(r.severity.value <= fail_on.value for r in results):
        raise ValidationError(phase, results)
    return results
