"""The library's host code (node decoders, the fusion matcher, plan joins,
launch planning) under AddressSanitizer and UndefinedBehaviorSanitizer, on the
CPU: the fusion-matcher (with malformed node arrays) and host-layer tests run
in a subprocess against the
sanitized build (build_native.build(sanitize=True), made by the graft build),
with the shared ASan runtime preloaded.  A planted out-of-bounds read of a node
array shows that the sanitizer is live in that setting.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "lets-build-a-runtime_amd"))


def _san_env():
    import build_native
    if not build_native.SAN_LIB.exists():
        pytest.skip("sanitized library not built (build_native.py --sanitize)")
    rt = build_native.asan_runtime()
    if not rt or not Path(rt).exists():
        pytest.skip("ASan runtime not found")
    env = dict(os.environ)
    env["LD_PRELOAD"] = rt + (":" + env["LD_PRELOAD"] if env.get("LD_PRELOAD") else "")
    env["LBR_EXECUTOR_LIB"] = str(build_native.SAN_LIB)
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    return env


def _run(args, env, timeout=900):
    return subprocess.run([sys.executable, *args], cwd=ROOT, env=env, capture_output=True, text=True,
                          timeout=timeout)


def test_host_layer_tests_pass_under_asan_and_ubsan():
    env = _san_env()
    res = _run(["-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "tests/test_fusion.py",
                "tests/test_fusion_fuzz.py", "tests/test_host_layer.py", "-k",
                "not stream_counts and not plan_integrity and not graph_save_load and not dynamic_seq"], env)
    out = res.stdout + res.stderr
    print(out[-2000:])
    assert res.returncode == 0, out[-4000:]
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out
    assert " passed" in out


def test_sanitizer_is_live():
    # a node array of 2 records handed over as 3: the matcher reads past its end
    env = _san_env()
    code = (
        "import sys; sys.path.insert(0, 'lets-build-a-runtime_amd')\n"
        "from runtime.executor.common import COpNode\n"
        "from runtime.executor.hip_lib import open_library\n"
        "lib = open_library()\n"
        "assert lib.path.name == 'liblbr_executor_san.so', lib.path\n"
        "arr = (COpNode * 2)()\n"
        "for n in arr:\n"
        "    n.op = 600; n.n_dims = 1; n.out_shape[0] = 4; n.elem_size = 4\n"
        "print(lib.fusion_windows(arr, 3, []))\n")
    res = _run(["-c", code], env, timeout=300)
    out = res.stdout + res.stderr
    assert res.returncode != 0 and "AddressSanitizer" in out and "overflow" in out, out[-3000:]
