"""ctypes binding of liblbr_executor.so (include/lbr_executor.h).

Plays the role of the reference's ``_load_c_executor``
(runtime/executor/common.py:148-163), extended to the device library's
lifecycle calls.  Every call's int status is checked; a failure raises
``HipExecutorError`` carrying ``lbr_last_error()``.  There is no fallback:
if the library is missing the executor refuses to compile.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

from .common import COpNode

_DEFAULT_LIB = Path(__file__).resolve().parents[2] / "csrc" / "liblbr_executor.so"


class HipExecutorError(RuntimeError):
    """A call into the device library returned a nonzero status."""

    def __init__(self, what: str, status: int, message: str) -> None:
        self.status = status
        super().__init__(f"{what} failed (status {status}): {message}")


def library_path() -> Path:
    return Path(os.environ.get("LBR_EXECUTOR_LIB", _DEFAULT_LIB))


class LbrWindow(ctypes.Structure):
    """lbr_window: one fused run of consecutive nodes."""
    _fields_ = [("first", ctypes.c_int), ("count", ctypes.c_int), ("kind", ctypes.c_int)]


FUSE_KINDS = {0: "none", 1: "gemm_resid", 2: "gemm_heads", 3: "head_prologue", 4: "attn_transpose",
              5: "gemm_act", 6: "gemm_gated", 7: "transpose_gemm", 8: "attn_sliced_v", 10: "norm_gemm",
              11: "mlp", 12: "add_norm", 13: "gemm_head_prologue"}


class HipLibrary:
    """Loaded device library with typed entry points."""

    def __init__(self, path: Path) -> None:
        self.path = path
        lib = ctypes.CDLL(str(path))
        c_int, c_size, c_vp, c_char_p = ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_char_p
        P = ctypes.POINTER
        sig = {
            "lbr_last_error": ([], c_char_p),
            "lbr_version": ([], c_char_p),
            "lbr_opnode_size": ([], c_int),
            "lbr_init": ([c_int], c_int),
            "lbr_op_supported": ([c_int], c_int),
            "lbr_device_alloc": ([c_size, P(c_vp)], c_int),
            "lbr_device_free": ([c_vp], c_int),
            "lbr_memcpy_h2d": ([c_vp, c_vp, c_size], c_int),
            "lbr_memcpy_d2h": ([c_vp, c_vp, c_size], c_int),
            "lbr_memcpy_d2d": ([c_vp, c_vp, c_size], c_int),
            "lbr_memset": ([c_vp, c_int, c_size], c_int),
            "lbr_host_alloc": ([c_size, P(c_vp)], c_int),
            "lbr_host_free": ([c_vp], c_int),
            "lbr_upload_async": ([c_vp, c_vp, c_size], c_int),
            "lbr_download_async": ([c_vp, c_vp, c_size], c_int),
            "lbr_execute": ([P(COpNode), c_int], c_int),
            "lbr_execute_workspace_bytes": ([P(c_size)], c_int),
            "lbr_execute_noalloc": ([P(COpNode), c_int], c_int),
            "lbr_plan_create": ([P(COpNode), c_int, c_int, P(c_vp)], c_int),
            "lbr_plan_destroy": ([c_vp], c_int),
            "lbr_plan_num_nodes": ([c_vp], c_int),
            "lbr_plan_launch": ([c_vp], c_int),
            "lbr_synchronize": ([], c_int),
            "lbr_plan_time": ([c_vp, c_int, P(ctypes.c_float)], c_int),
            "lbr_plan_profile": ([c_vp, c_int, P(ctypes.c_float), c_int], c_int),
            "lbr_plan_node_kernel": ([c_vp, c_int, ctypes.c_char_p, c_int], c_int),
            "lbr_fusion_windows": ([P(COpNode), c_int, P(c_vp), P(c_size), c_int, P(LbrWindow), c_int, P(c_int)],
                                   c_int),
            "lbr_plan_create_fused": ([P(COpNode), c_int, c_int, P(c_vp), P(c_size), c_int, P(c_vp)], c_int),
            "lbr_check_nodes": ([P(COpNode), c_int, c_int, P(c_vp), P(c_size), c_int, P(c_int)], c_int),
            "lbr_plan_num_steps": ([c_vp], c_int),
            "lbr_plan_step_info": ([c_vp, c_int, P(c_int), P(c_int), P(c_int)], c_int),
            "lbr_plan_step_args": ([c_vp, c_int, P(ctypes.c_longlong), c_int], c_int),
            "lbr_fast_div": ([ctypes.c_uint, ctypes.c_uint], ctypes.c_uint),
            "lbr_gemm_tile_name": ([c_int], c_char_p),
            "lbr_attn_kq_grid": ([ctypes.c_longlong, c_int, c_int, c_int, P(c_int), P(c_int), c_int], c_int),
        }
        for name, (args, res) in sig.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        self._lib = lib
        size = lib.lbr_opnode_size()
        if size != ctypes.sizeof(COpNode):
            raise RuntimeError(f"{path}: OpNode is {size} bytes in the library, {ctypes.sizeof(COpNode)} in ctypes")

    def __getattr__(self, name):
        return getattr(self._lib, name)

    def last_error(self) -> str:
        msg = self._lib.lbr_last_error()
        return msg.decode() if msg else ""

    def check(self, status: int, what: str) -> None:
        if status != 0:
            raise HipExecutorError(what, status, self.last_error())

    # convenience wrappers -------------------------------------------------
    def alloc(self, nbytes: int) -> int:
        ptr = ctypes.c_void_p()
        self.check(self._lib.lbr_device_alloc(max(int(nbytes), 1), ctypes.byref(ptr)), f"device alloc {nbytes} B")
        return int(ptr.value)

    def free(self, ptr: int) -> None:
        if ptr:
            self.check(self._lib.lbr_device_free(ctypes.c_void_p(ptr)), "device free")

    def h2d(self, dst: int, src_ptr: int, nbytes: int) -> None:
        self.check(self._lib.lbr_memcpy_h2d(ctypes.c_void_p(dst), ctypes.c_void_p(src_ptr), nbytes), "memcpy H2D")

    def d2h(self, dst_ptr: int, src: int, nbytes: int) -> None:
        self.check(self._lib.lbr_memcpy_d2h(ctypes.c_void_p(dst_ptr), ctypes.c_void_p(src), nbytes), "memcpy D2H")


    def fusion_windows(self, nodes, n: int, live: list[tuple[int, int]]) -> list[tuple[int, int, str]]:
        """(first, count, kind) of every run lbr_plan_create_fused would fuse; needs no device."""
        lp, lb = live_arrays(live)
        cap = max(n, 1)
        out = (LbrWindow * cap)()
        n_out = ctypes.c_int(0)
        self.check(self._lib.lbr_fusion_windows(nodes, n, lp, lb, len(live), out, cap, ctypes.byref(n_out)),
                   "lbr_fusion_windows")
        return [(out[k].first, out[k].count, FUSE_KINDS.get(out[k].kind, "?")) for k in range(n_out.value)]

    def check_nodes(self, nodes, n: int, live: list[tuple[int, int]], fuse: bool = True) -> int:
        """Kernel steps lbr_plan_create[_fused] would build from `nodes`, or its error; needs no device."""
        lp, lb = live_arrays(live)
        steps = ctypes.c_int(0)
        self.check(self._lib.lbr_check_nodes(nodes, n, int(fuse), lp, lb, len(live), ctypes.byref(steps)),
                   "lbr_check_nodes")
        return steps.value


def live_arrays(live: list[tuple[int, int]]):
    """ctypes (pointer, byte count) arrays of live-out ranges."""
    n = max(len(live), 1)
    lp = (ctypes.c_void_p * n)(*[ctypes.c_void_p(p) for p, _ in live])
    lb = (ctypes.c_size_t * n)(*[b for _, b in live])
    return lp, lb


_LIB: HipLibrary | None = None


def open_library() -> HipLibrary:
    """Load (once) the device library without touching a device."""
    global _LIB
    if _LIB is None:
        path = library_path()
        if not path.exists():
            raise RuntimeError(f"HIP executor library not found at {path} — build it with "
                               "lets-build-a-runtime_amd/build_native.py first")
        _LIB = HipLibrary(path)
    return _LIB


def load_library(device: int = 0) -> HipLibrary:
    """Load (once) and initialise the device library; raises if it is absent or no gfx950 GPU is usable."""
    lib = open_library()
    lib.check(lib.lbr_init(device), f"lbr_init({device})")
    return lib


def loaded_library() -> HipLibrary | None:
    return _LIB
