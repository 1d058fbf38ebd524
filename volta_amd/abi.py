"""ctypes view of the C ABI in include/volta_train.h.

`TrainLibrary` wraps any shared library that exports that ABI (the HIP
product library or the CPU oracle) and `Trainer` mirrors one handle of it,
method for method, with the reference's entry points
(mlp_train_rust_codegen.rs:640-994):

    init(batch)               -> Trainer(lib, spec, batch)
    step(X, Y, lr)            -> Trainer.step
    loss()                    -> Trainer.loss
    get_params()              -> Trainer.get_params  (copies of W_i, b_i)
    set_params(li, w, b)      -> Trainer.set_params
    free()                    -> Trainer.close

Arrays are numpy float32/int32, row-major, as in the reference.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Tuple

import numpy as np

MAX_LAYER_SIZES = 17

ACTIVATIONS = {"relu": 0, "sigmoid": 1, "tanh": 2, "leaky_relu": 3, "silu": 4, "gelu": 5, "softmax": 6}
OPTIMIZERS = {"sgd": 0, "adam": 1, "adamw": 2, "adagrad": 3}
LOSSES = {"mse": 0, "ce": 1}

STATUS_NONFINITE_LOSS = 1
STATUS_BAD_ARGUMENT = 2
STATUS_DEVICE_ERROR = 4


class CSpec(C.Structure):
    _fields_ = [
        ("n_sizes", C.c_int32),
        ("sizes", C.c_int32 * MAX_LAYER_SIZES),
        ("activation", C.c_int32),
        ("optimizer", C.c_int32),
        ("loss", C.c_int32),
        ("beta1", C.c_float),
        ("beta2", C.c_float),
        ("eps", C.c_float),
        ("weight_decay", C.c_float),
        ("clip_grad", C.c_float),
        ("dropout_p", C.c_float),
        ("layernorm", C.c_int32),
    ]


@dataclass
class MlpSpec:
    """Topology + optimizer constants (the reference bakes these into the
    generated library; defaults from mlp_train_rust_codegen.rs:807-813)."""

    sizes: Sequence[int]
    activation: str = "relu"
    optimizer: str = "sgd"
    loss: str = "mse"
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    weight_decay: Optional[float] = None  # None -> 0.01 for adamw, else 0
    clip_grad: float = 0.0    # codegen extras (0 / False: off)
    dropout_p: float = 0.0
    layernorm: bool = False

    def to_c(self) -> CSpec:
        s = CSpec()
        if not 2 <= len(self.sizes) <= MAX_LAYER_SIZES:
            raise ValueError(f"need 2..{MAX_LAYER_SIZES} layer sizes, got {len(self.sizes)}")
        s.n_sizes = len(self.sizes)
        for i, v in enumerate(self.sizes):
            s.sizes[i] = int(v)
        s.activation = ACTIVATIONS[self.activation]
        s.optimizer = OPTIMIZERS[self.optimizer]
        s.loss = LOSSES[self.loss]
        s.beta1 = self.beta1
        s.beta2 = self.beta2
        s.eps = self.eps
        wd = self.weight_decay
        if wd is None:
            wd = 0.01 if self.optimizer == "adamw" else 0.0
        s.weight_decay = wd
        s.clip_grad = self.clip_grad
        s.dropout_p = self.dropout_p
        s.layernorm = 1 if self.layernorm else 0
        return s

    @property
    def has_extras(self) -> bool:
        return self.clip_grad > 0 or self.dropout_p > 0 or bool(self.layernorm)

    @property
    def n_layers(self) -> int:
        return len(self.sizes) - 1

    def shapes(self) -> List[Tuple[int, int]]:
        return [(self.sizes[i], self.sizes[i + 1]) for i in range(self.n_layers)]

    def text(self) -> str:
        t = "-".join(str(s) for s in self.sizes) + f":{self.activation}:{self.optimizer}:{self.loss}"
        if self.clip_grad > 0:
            t += f":clip={self.clip_grad!r}"
        if self.dropout_p > 0:
            t += f":dropout={self.dropout_p!r}"
        if self.layernorm:
            t += ":ln"
        return t


_P = C.c_void_p
_F = C.POINTER(C.c_float)
_I = C.POINTER(C.c_int32)

_SIGNATURES = {
    "volta_train_init": (_P, [C.c_int32]),
    "volta_train_init_spec": (_P, [C.POINTER(CSpec), C.c_int32]),
    "volta_train_step": (None, [_P, _F, _F, C.c_float]),
    "volta_train_step_labels": (None, [_P, _F, _I, C.c_float]),
    "volta_train_step_device": (C.c_int32, [_P, _P, _P, C.c_float]),
    "volta_train_batch_buffers": (C.c_int32, [_P, C.POINTER(_P), C.POINTER(_P)]),
    "volta_train_loss": (C.c_float, [_P]),
    "volta_train_get_params": (None, [_P, C.POINTER(_F), C.POINTER(_F)]),
    "volta_train_set_params": (None, [_P, C.c_int32, _F, _F]),
    "volta_train_free": (None, [_P]),
    "volta_train_sync": (C.c_int32, [_P]),
    "volta_train_status": (C.c_int32, [_P]),
    "volta_train_clear_status": (None, [_P]),
    "volta_train_last_error": (C.c_char_p, []),
    "volta_train_num_layers": (C.c_int32, [_P]),
    "volta_train_batch": (C.c_int32, [_P]),
    "volta_train_configure": (C.c_int32, [C.POINTER(CSpec)]),
    "volta_mlp_spec_default": (None, [C.POINTER(CSpec), C.c_int32, _I, C.c_int32, C.c_int32, C.c_int32]),
    "volta_mlp_spec_parse": (C.c_int32, [C.c_char_p, C.POINTER(CSpec)]),
    "volta_train_state_size": (C.c_int64, [_P]),
    "volta_train_get_state": (C.c_int32, [_P, _F, C.POINTER(C.c_int64)]),
    "volta_train_set_state": (C.c_int32, [_P, _F, C.c_int64]),
    "volta_train_get_dropout_rng": (C.c_int32, [_P, C.POINTER(C.c_uint64)]),
    "volta_train_set_dropout_rng": (C.c_int32, [_P, C.c_uint64]),
    "volta_train_debug_buffer": (C.c_int64, [_P, C.c_int32, C.c_int32, _F]),
    "volta_train_set_hparams": (C.c_int32, [_P, C.c_float, C.c_float, C.c_float, C.c_float]),
    "volta_train_infer": (C.c_int32, [_P, _F, C.c_int64, _F]),
    "volta_train_infer_device_noalloc": (C.c_int32, [_P, C.c_void_p, C.c_int64, C.c_void_p]),
    "volta_infer_bind": (C.c_int32, [_P]),
    "volta_infer": (None, [_F, C.c_int64, _F, C.c_int64]),
    "volta_infer_model_create": (_P, [C.c_int32, C.POINTER(C.c_int32), C.c_int32, _F]),
}

# include/volta_vt.h (the .vt front end; GPU library only)
VT_SIGNATURES = {
    "volta_vt_compile_train_spec": (C.c_int32, [C.c_char_p, C.POINTER(CSpec), C.c_char_p, C.c_int32]),
    "volta_vt_compile_train_spec_path": (C.c_int32, [C.c_char_p, C.c_int32, C.POINTER(CSpec), C.c_char_p,
                                                     C.c_int32]),
}

BUF_ACT, BUF_DELTA, BUF_GRAD_W, BUF_GRAD_B = 0, 1, 2, 3
BUF_LN_GAMMA, BUF_LN_BETA, BUF_DROPOUT_MASK, BUF_PRE = 4, 5, 6, 7
BUF_LN_DGAMMA, BUF_LN_DBETA, BUF_CLIP_SCALE = 8, 9, 10

# Every symbol include/volta_train.h declares (checked by the CPU tests).
HEADER_SYMBOLS = tuple(_SIGNATURES)


def fptr(a: np.ndarray):
    return a.ctypes.data_as(_F)


def iptr(a: np.ndarray):
    return a.ctypes.data_as(_I)


class TrainLibrary:
    """A loaded library exporting the volta_train_* ABI."""

    def __init__(self, path: str, extra: Optional[dict] = None):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.path = path
        self.lib = C.CDLL(path)
        for name, (res, args) in list(_SIGNATURES.items()) + list((extra or {}).items()):
            fn = getattr(self.lib, name)
            fn.restype = res
            fn.argtypes = args

    def last_error(self) -> str:
        msg = self.lib.volta_train_last_error()
        return msg.decode() if msg else ""

    def parse_spec(self, text: str) -> CSpec:
        s = CSpec()
        if self.lib.volta_mlp_spec_parse(text.encode(), C.byref(s)) != 0:
            raise ValueError(self.last_error())
        return s


class Trainer:
    """One handle of a TrainLibrary."""

    def __init__(self, lib: TrainLibrary, spec: MlpSpec, batch: int, handle=None):
        self.lib = lib
        self.spec = spec
        self.batch = batch
        self._cspec = spec.to_c()
        h = handle if handle is not None else lib.lib.volta_train_init_spec(C.byref(self._cspec), batch)
        if not h:
            raise RuntimeError(f"volta_train_init_spec failed: {lib.last_error()}")
        self.h = C.c_void_p(h)

    # -- reference ABI -------------------------------------------------------
    def step(self, X: np.ndarray, Y: np.ndarray, lr: float) -> None:
        X = np.ascontiguousarray(X, dtype=np.float32)
        if self.spec.loss == "ce":
            Y = np.ascontiguousarray(Y, dtype=np.int32)
            self._check(X, Y)
            self.lib.lib.volta_train_step_labels(self.h, fptr(X), iptr(Y), lr)
        else:
            Y = np.ascontiguousarray(Y, dtype=np.float32)
            self._check(X, Y)
            self.lib.lib.volta_train_step(self.h, fptr(X), fptr(Y), lr)

    def _check(self, X, Y):
        n0, nl = self.spec.sizes[0], self.spec.sizes[-1]
        if X.size != self.batch * n0:
            raise ValueError(f"X has {X.size} elements, expected {self.batch}x{n0}")
        want = self.batch if self.spec.loss == "ce" else self.batch * nl
        if Y.size != want:
            raise ValueError(f"Y has {Y.size} elements, expected {want}")

    def loss(self) -> float:
        return float(self.lib.lib.volta_train_loss(self.h))

    def get_params(self) -> Tuple[List[np.ndarray], List[np.ndarray]]:
        n = self.spec.n_layers
        wo = (_F * n)()
        bo = (_F * n)()
        self.lib.lib.volta_train_get_params(self.h, wo, bo)
        ws, bs = [], []
        for i, (r, c) in enumerate(self.spec.shapes()):
            ws.append(np.ctypeslib.as_array(wo[i], shape=(r, c)).copy())
            bs.append(np.ctypeslib.as_array(bo[i], shape=(c,)).copy())
        return ws, bs

    def set_params(self, li: int, w: np.ndarray, b: np.ndarray) -> None:
        w = np.ascontiguousarray(w, dtype=np.float32)
        b = np.ascontiguousarray(b, dtype=np.float32)
        if 0 <= li < self.spec.n_layers:
            r, c = self.spec.shapes()[li]
            if w.size != r * c or b.size != c:
                raise ValueError(f"layer {li}: expected W {r}x{c} and b {c}")
        self.lib.lib.volta_train_set_params(self.h, li, fptr(w), fptr(b))

    def close(self) -> None:
        if self.h:
            self.lib.lib.volta_train_free(self.h)
            self.h = C.c_void_p(None)

    # -- extensions ----------------------------------------------------------
    def set_all_params(self, ws, bs) -> None:
        for i, (w, b) in enumerate(zip(ws, bs)):
            self.set_params(i, w, b)

    def sync(self) -> int:
        return int(self.lib.lib.volta_train_sync(self.h))

    def status(self) -> int:
        return int(self.lib.lib.volta_train_status(self.h))

    def clear_status(self) -> None:
        self.lib.lib.volta_train_clear_status(self.h)

    def step_device(self, x_ptr: int, y_ptr: int, lr: float) -> int:
        return int(self.lib.lib.volta_train_step_device(self.h, C.c_void_p(x_ptr), C.c_void_p(y_ptr), lr))

    def batch_buffers(self) -> Tuple[int, int]:
        x = C.c_void_p()
        y = C.c_void_p()
        rc = self.lib.lib.volta_train_batch_buffers(self.h, C.byref(x), C.byref(y))
        if rc != 0:
            raise RuntimeError(self.lib.last_error())
        return int(x.value or 0), int(y.value or 0)

    def state_size(self) -> int:
        return int(self.lib.lib.volta_train_state_size(self.h))

    def get_state(self) -> Tuple[np.ndarray, int]:
        n = self.state_size()
        buf = np.zeros(max(n, 1), dtype=np.float32)
        step = C.c_int64()
        if self.lib.lib.volta_train_get_state(self.h, fptr(buf), C.byref(step)) != 0:
            raise RuntimeError(self.lib.last_error())
        return buf[:n], int(step.value)

    def set_state(self, state: np.ndarray, step: int) -> None:
        state = np.ascontiguousarray(state, dtype=np.float32)
        if state.size != self.state_size():
            raise ValueError("state size mismatch")
        buf = state if state.size else np.zeros(1, np.float32)
        if self.lib.lib.volta_train_set_state(self.h, fptr(buf), step) != 0:
            raise RuntimeError(self.lib.last_error())

    def get_dropout_rng(self) -> int:
        v = C.c_uint64()
        if self.lib.lib.volta_train_get_dropout_rng(self.h, C.byref(v)) != 0:
            raise RuntimeError(self.lib.last_error())
        return int(v.value)

    def set_dropout_rng(self, rng: int) -> None:
        if self.lib.lib.volta_train_set_dropout_rng(self.h, C.c_uint64(rng)) != 0:
            raise RuntimeError(self.lib.last_error())

    def set_hparams(self, beta1: float, beta2: float, eps: float, weight_decay: float) -> None:
        if self.lib.lib.volta_train_set_hparams(self.h, beta1, beta2, eps, weight_decay) != 0:
            raise ValueError(self.lib.last_error())

    def infer(self, X: np.ndarray) -> np.ndarray:
        """Forward pass only: the output layer's pre-activation for X [rows x L0]."""
        X = np.ascontiguousarray(X, dtype=np.float32)
        rows = X.shape[0]
        if X.ndim != 2 or X.shape[1] != self.spec.sizes[0] or rows == 0:
            raise ValueError(f"X must be [rows x {self.spec.sizes[0]}]")
        out = np.zeros((rows, self.spec.sizes[-1]), np.float32)
        if self.lib.lib.volta_train_infer(self.h, fptr(X), rows, fptr(out)) != 0:
            raise RuntimeError(self.lib.last_error())
        return out

    def debug_buffer(self, kind: int, layer: int) -> np.ndarray:
        """An intermediate buffer of the last step (see volta_train_debug_buffer)."""
        sizes = self.spec.sizes
        B = self.batch
        count = {BUF_ACT: lambda i: B * sizes[i], BUF_DELTA: lambda i: B * sizes[i + 1],
                 BUF_GRAD_W: lambda i: sizes[i] * sizes[i + 1], BUF_GRAD_B: lambda i: sizes[i + 1],
                 BUF_LN_GAMMA: lambda i: sizes[i + 1], BUF_LN_BETA: lambda i: sizes[i + 1],
                 BUF_DROPOUT_MASK: lambda i: B * sizes[i + 1], BUF_PRE: lambda i: B * sizes[i + 1],
                 BUF_LN_DGAMMA: lambda i: sizes[i + 1], BUF_LN_DBETA: lambda i: sizes[i + 1],
                 BUF_CLIP_SCALE: lambda i: 1}[kind](layer)
        out = np.zeros(count, np.float32)
        n = self.lib.lib.volta_train_debug_buffer(self.h, kind, layer, fptr(out))
        if n != count:
            raise RuntimeError(f"debug_buffer({kind}, {layer}) failed: {self.lib.last_error()}")
        return out

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
