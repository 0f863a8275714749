"""Host layer of the MI355X compiled-executor backend.

Same package layout and public API as the reference runtime (exporter →
passes → planner → Session → executor); the compiled executor runs the plan
on a gfx950 GPU through liblbr_executor.so.
"""
