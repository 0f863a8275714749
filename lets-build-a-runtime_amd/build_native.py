"""Build liblbr_executor.so (the gfx950 compiled-executor library) in-tree.

    python lets-build-a-runtime_amd/build_native.py [--sanitize]

Compiles every csrc/*.hip translation unit with hipcc for gfx950 (in
parallel) and links them into csrc/liblbr_executor.so.  Always rebuilds.
Packed-FP32 instruction selection is disabled for all device code.

--sanitize builds the same sources with AddressSanitizer and
UndefinedBehaviorSanitizer on the host code only (node decoders, the fusion
matcher, plan joins, launchers; the device code is built as usual) into
_build_san/liblbr_executor_san.so, for CPU tests of the host layer: load it
with LBR_EXECUTOR_LIB and the shared ASan runtime preloaded (asan_runtime()).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = CSRC / "liblbr_executor.so"
BUILD = HERE / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# host-only sanitizers (each -fsanitize= applies to the host compilation alone)
SAN_FLAGS = "-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined".split() + [
    "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer", "-g1"]
SAN_BUILD = HERE / "_build_san"
SAN_LIB = SAN_BUILD / "liblbr_executor_san.so"


def asan_runtime() -> str:
    """Path of the shared ASan runtime the sanitized library links against."""
    res = subprocess.run([HIPCC, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    return res.stdout.strip()


def _compile(src: Path, sanitize: bool = False) -> Path:
    obj = (SAN_BUILD if sanitize else BUILD) / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *(SAN_FLAGS if sanitize else []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    # hipcc's host pass does not know the packed-fp32 feature; drop that noise
    noise = [ln for ln in res.stderr.splitlines()
             if ln.strip() and "packed-fp32-ops" not in ln and "warning generated" not in ln]
    if noise:
        sys.stderr.write(f"[{src.name}]\n" + "\n".join(noise) + "\n")
    return obj


def build(verbose: bool = True, sanitize: bool = False) -> Path:
    """Compile and link; returns the path of the shared library (the sanitized
    variant with sanitize=True)."""
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    out_dir, lib = (SAN_BUILD, SAN_LIB) if sanitize else (BUILD, LIB)
    out_dir.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda src: _compile(src, sanitize), sources))
    tmp = lib.with_suffix(".so.tmp")
    link_san = "-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined -shared-libsan".split()
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *(link_san if sanitize else []), *map(str, objs),
           "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib.relative_to(HERE.parent)} from {len(sources)} sources")
    return lib


if __name__ == "__main__":
    build(sanitize="--sanitize" in sys.argv[1:])
