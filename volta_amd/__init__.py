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
# take device pointers and run synchronously.
HIP_EXTRA = {
    "volta_hip_gemm": (C.c_int32, [C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p,
                                   C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32]),
    "volta_hip_arena_bytes": (C.c_int64, [C.c_void_p]),
}

_loaded = {}


class HipLibraryMissing(RuntimeError):
    pass


def load_hip(path: str = HIP_LIB) -> TrainLibrary:
    """Load the HIP product library.  Raises if it has not been built."""
    if path not in _loaded:
        if not os.path.exists(path):
            raise HipLibraryMissing(
                f"{path} is not built; run `python -m volta_amd.build` (or __graft_entry__.build())")
        _loaded[path] = TrainLibrary(path, extra=HIP_EXTRA)
    return _loaded[path]
