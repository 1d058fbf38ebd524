"""Host mirror of Volta's runtime Backend for the HIP library: capabilities()
and apply_gradients() of the Backend trait (src/engine/ir/backend.rs:24-69),
whose update is optimizer::apply_gradients (src/engine/ir/optimizer.rs:
36-178), over the volta_rt_* C ABI (include/volta_backend.h).

The same RtOptimizer drives libvolta_hip.so (device pointers) and the CPU
oracle (host pointers, tests only).  Parameters and gradients are keyed by
integer ids as the reference keys them by ValueId; the state follows a fixed
list of ids.
"""
from __future__ import annotations

import ctypes as C
from typing import Dict, Optional, Sequence

import numpy as np

KINDS = {"sgd": 0, "adam": 1, "adamw": 2, "rmsprop": 3, "adagrad": 4, "lars": 5}
BUFFERS = {"adam_m": 0, "adam_v": 1, "rms_v": 2, "rms_buf": 3, "adagrad_acc": 4, "lars_vel": 5}


class RtConfig(C.Structure):
    """OptimizerConfig (optimizer.rs:37-79) as volta_rt_config."""
    _fields_ = [("kind", C.c_int32), ("lr", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float),
                ("epsilon", C.c_float), ("weight_decay", C.c_float), ("alpha", C.c_float),
                ("momentum", C.c_float), ("trust_coeff", C.c_float)]


class RtCapabilities(C.Structure):
    _fields_ = [("backend", C.c_int32), ("device_class", C.c_int32), ("vendor", C.c_int32),
                ("maturity", C.c_int32), ("supports_inference", C.c_uint8), ("supports_training", C.c_uint8),
                ("supports_runtime_execution", C.c_uint8), ("supports_gradient_updates", C.c_uint8),
                ("supports_adam", C.c_uint8), ("supports_strict_determinism", C.c_uint8),
                ("supports_balanced_determinism", C.c_uint8), ("supports_fast_determinism", C.c_uint8),
                ("default_determinism", C.c_int32)]


def config(kind: str, lr: float, beta1: float = 0.9, beta2: float = 0.999, epsilon: float = 1e-8,
           weight_decay: float = 0.0, alpha: float = 0.99, momentum: float = 0.0,
           trust_coeff: float = 0.001) -> RtConfig:
    """An OptimizerConfig of variant `kind` (fields it lacks are ignored)."""
    return RtConfig(KINDS[kind], lr, beta1, beta2, epsilon, weight_decay, alpha, momentum, trust_coeff)


class OptimizerError(RuntimeError):
    """OptimizerError (optimizer.rs:95-98): the reference's message."""


_SIGS = {
    "volta_rt_optimizer_new": (C.c_void_p, [C.c_int32, C.POINTER(C.c_int64)]),
    "volta_rt_optimizer_free": (None, [C.c_void_p]),
    "volta_rt_apply_gradients": (C.c_int32, [C.c_void_p, C.POINTER(RtConfig), C.POINTER(C.c_void_p),
                                             C.POINTER(C.c_void_p)]),
    "volta_rt_step": (C.c_int64, [C.c_void_p]),
    "volta_rt_get_state": (C.c_int32, [C.c_void_p, C.c_int32, C.c_int32, C.POINTER(C.c_float)]),
    "volta_rt_last_error": (C.c_char_p, []),
    "volta_rt_capabilities_get": (None, [C.POINTER(RtCapabilities)]),
}


def bind(cdll: C.CDLL) -> C.CDLL:
    """Declare the volta_rt_* signatures on a loaded library."""
    for name, (res, args) in _SIGS.items():
        fn = getattr(cdll, name)
        fn.restype = res
        fn.argtypes = args
    return cdll


class RtOptimizer:
    """OptimizerState for tensors of `counts` elements in library `cdll`."""

    def __init__(self, cdll: C.CDLL, counts: Sequence[int]):
        self.lib = bind(cdll)
        self.counts = [int(c) for c in counts]
        arr = (C.c_int64 * len(self.counts))(*self.counts)
        self.h = self.lib.volta_rt_optimizer_new(len(self.counts), arr)
        if not self.h:
            raise OptimizerError(self.lib.volta_rt_last_error().decode())

    def apply(self, cfg: RtConfig, params: Sequence[int], grads: Sequence[Optional[int]]) -> None:
        """apply_gradients with params[i] / grads[i] as raw addresses (None: no gradient)."""
        n = len(self.counts)
        if len(params) != n or len(grads) != n:
            raise ValueError("one parameter and one gradient slot per tensor")
        pp = (C.c_void_p * n)(*[int(p) for p in params])
        gp = (C.c_void_p * n)(*[int(g) if g else None for g in grads])
        if self.lib.volta_rt_apply_gradients(self.h, C.byref(cfg), pp, gp) != 0:
            raise OptimizerError(self.lib.volta_rt_last_error().decode())

    @property
    def step(self) -> int:
        return int(self.lib.volta_rt_step(self.h))

    def state(self, which: str, i: int) -> Optional[np.ndarray]:
        """State buffer `which` of tensor i, or None when the reference would have no entry."""
        out = np.empty(self.counts[i], np.float32)
        rc = self.lib.volta_rt_get_state(self.h, BUFFERS[which], i, out.ctypes.data_as(C.POINTER(C.c_float)))
        return out if rc == 0 else None

    def close(self) -> None:
        if self.h:
            self.lib.volta_rt_optimizer_free(self.h)
            self.h = None

    def __del__(self):
        self.close()


def capabilities(cdll: C.CDLL) -> Dict[str, int]:
    """BackendCapabilities of the library as a dict."""
    out = RtCapabilities()
    bind(cdll).volta_rt_capabilities_get(C.byref(out))
    return {f: int(getattr(out, f)) for f, _ in RtCapabilities._fields_}


class HipBackend:
    """The HIP backend's side of the Backend trait for training updates:
    capabilities() and apply_gradients(parameters, gradients, config, state)
    with parameters/gradients as {id: DeviceArray} (gradients may omit ids,
    as the reference skips parameters without a gradient)."""

    def __init__(self, lib=None):
        from volta_amd import load_hip

        self.lib = lib or load_hip()

    def capabilities(self) -> Dict[str, int]:
        return capabilities(self.lib.lib)

    def new_state(self, parameters: Dict[int, "object"]) -> RtOptimizer:
        """OptimizerState::default() for these parameters (ids in sorted order)."""
        ids = sorted(parameters)
        st = RtOptimizer(self.lib.lib, [parameters[i].host.size for i in ids])
        st.ids = ids
        return st

    def apply_gradients(self, parameters: Dict[int, "object"], gradients: Dict[int, "object"], cfg: RtConfig,
                        state: RtOptimizer) -> None:
        for i in state.ids:
            g = gradients.get(i)
            if g is not None and g.host.size != parameters[i].host.size:
                raise OptimizerError(f"Shape mismatch for ValueId {i}: {parameters[i].host.shape} vs "
                                     f"{g.host.shape}")
        state.apply(cfg, [parameters[i].ptr for i in state.ids],
                    [gradients[i].ptr if i in gradients else None for i in state.ids])
