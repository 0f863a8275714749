"""Pipeline validators: phase-tagged checks over graphs, memory plans and
execution plans (same framework as runtime/validation/ of the reference)."""

from .core import (  # noqa: F401
    Phase,
    Severity,
    ValidationResult,
    ValidationError,
    Validator,
    VALIDATORS,
    register_validator,
    run_validators,
)
from . import graph, plan, execution  # noqa: F401,E402
