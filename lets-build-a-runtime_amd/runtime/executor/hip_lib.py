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
            "lbr_execute": ([P(COpNode), c_int], c_int),
            "lbr_plan_create": ([P(COpNode), c_int, c_int, P(c_vp)], c_int),
            "lbr_plan_destroy": ([c_vp], c_int),
            "lbr_plan_num_nodes": ([c_vp], c_int),
            "lbr_plan_launch": ([c_vp], c_int),
            "lbr_synchronize": ([], c_int),
            "lbr_plan_time": ([c_vp, c_int, P(ctypes.c_float)], c_int),
            "lbr_plan_profile": ([c_vp, c_int, P(ctypes.c_float), c_int], c_int),
            "lbr_plan_node_kernel": ([c_vp, c_int, ctypes.c_char_p, c_int], c_int),
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


_LIB: HipLibrary | None = None


def load_library(device: int = 0) -> HipLibrary:
    """Load (once) and initialise the device library; raises if it is absent or no gfx950 GPU is usable."""
    global _LIB
    if _LIB is None:
        path = library_path()
        if not path.exists():
            raise RuntimeError(f"HIP executor library not found at {path} — build it with "
                               "lets-build-a-runtime_amd/build_native.py first")
        _LIB = HipLibrary(path)
    _LIB.check(_LIB.lbr_init(device), f"lbr_init({device})")
    return _LIB


def loaded_library() -> HipLibrary | None:
    return _LIB
