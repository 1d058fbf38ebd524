"""volta_amd -- MI355X (gfx950) drop-in for Volta's compile-train MLP step.

The product is the shared library volta_amd/libvolta_hip.so (hand-written
HIP kernels + C++ runtime) exporting the C ABI of include/volta_train.h.
This package only loads it (`load_hip`) and offers the ctypes mirror of the
ABI (`volta_amd.abi`).  There is no CPU fallback: without the built library
or a GPU, `load_hip` / `Trainer` raise.
"""
from __future__ import annotations

import ctypes as C
import os

from .abi import HEADER_SYMBOLS, MlpSpec, Trainer, TrainLibrary  # noqa: F401

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
HIP_LIB = os.path.join(PKG_DIR, "libvolta_hip.so")

_F = C.POINTER(C.c_float)

# Kernel-level entry points of libvolta_hip.so used by the GPU tests; they
# take device pointers and run synchronously (volta_hip_gemm_plan makes no
# device call: the CPU tests use it).
HIP_EXTRA = {
    "volta_hip_gemm": (C.c_int32, [C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p,
                                   C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32]),
    "volta_hip_gemm_plan": (C.c_int32, [C.c_int32] * 7 + [C.POINTER(C.c_int32)]),
    "volta_hip_arena_bytes": (C.c_int64, [C.c_void_p]),
    "volta_hip_optimizer": (C.c_int32, [C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64]
                            + [C.c_float] * 7),
    "volta_hip_profile_step": (C.c_int32, [C.c_void_p, C.c_int32, C.c_char_p, C.c_int32]),
    "volta_hip_time_kernel": (C.c_int32, [C.c_void_p, C.c_int32, C.c_int32, C.POINTER(C.c_float), C.c_char_p,
                                          C.c_int32]),
    "volta_hip_calibration_copy": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_int64, C.c_int32]),
    "volta_hip_device_alloc": (C.c_void_p, [C.c_int64]),
    "volta_hip_device_free": (C.c_int32, [C.c_void_p]),
    "volta_hip_copy": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_int64, C.c_int32]),
    "volta_hip_rt_graph_replays": (C.c_int64, []),
}


class DeviceArray:
    """A float32/int32 device buffer owned through libvolta_hip.so (tests and
    benchmarks use it instead of a second GPU runtime)."""

    def __init__(self, host, lib=None):
        import numpy as np

        self.lib = lib or load_hip()
        self.host = np.ascontiguousarray(host)
        self.nbytes = max(int(self.host.nbytes), 4)
        p = self.lib.lib.volta_hip_device_alloc(self.nbytes)
        if not p:
            raise MemoryError("volta_hip_device_alloc failed")
        self.ptr = int(p)
        if self.lib.lib.volta_hip_copy(self.ptr, self.host.ctypes.data, int(self.host.nbytes), 1) != 0:
            raise RuntimeError("host->device copy failed")

    def numpy(self):
        import numpy as np

        out = np.empty_like(self.host)
        if self.lib.lib.volta_hip_copy(out.ctypes.data, self.ptr, int(out.nbytes), 2) != 0:
            raise RuntimeError("device->host copy failed")
        return out

    def free(self):
        if self.ptr:
            self.lib.lib.volta_hip_device_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

_loaded = {}


class HipLibraryMissing(RuntimeError):
    pass


def load_hip(path: str = HIP_LIB) -> TrainLibrary:
    """Load the HIP product library.  Raises if it has not been built."""
    if path not in _loaded:
        if not os.path.exists(path):
            raise HipLibraryMissing(
                f"{path} is not built; run `python -m volta_amd.build` (or __graft_entry__.build())")
        from .abi import VT_SIGNATURES

        _loaded[path] = TrainLibrary(path, extra={**HIP_EXTRA, **VT_SIGNATURES})
    return _loaded[path]
