"""GPU parity of the codegen extras (LayerNorm, dropout, gradient clipping;
mlp_train_rust_codegen.rs:745-788, :829-892, :936-955) against the CPU
oracle, through the C ABI.

Bar: losses and LayerNorm gamma/beta within rel 1e-4 / abs 1e-5 of the
oracle after several steps on the same seeded inputs; weights and biases
likewise for SGD; dropout masks and the dropout LCG state bit-exact
(integer work); two GPU runs bit-identical.  Adam/AdamW/Adagrad turn the
rounding of a near-zero gradient into a +-lr update flip (lr * g / (|g| +
eps) on the first step), so for them at most 1e-3 of a layer's parameters
may leave that tolerance, each by at most a few lr per step, and the HIP
run must be no further from the oracle's fp64 twin than the fp32 oracle is
(per-layer RMS).
"""
import ctypes as C
import sys

import numpy as np
import pytest

from tests.oracle_lib import load_oracle
from tests.test_oracle import oracle_trainer
from volta_amd import data, load_hip
from volta_amd.abi import BUF_DELTA, BUF_DROPOUT_MASK, BUF_LN_BETA, BUF_LN_GAMMA, MlpSpec, Trainer

RTOL = 1e-4
ATOL = 1e-5

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def close_enough(got, want, rtol=RTOL, atol=ATOL):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    ok = err <= atol + rtol * np.abs(want)
    return bool(ok.all()), float(err.max()) if err.size else 0.0, int((~ok).sum())


def assert_close(got, want, label, rtol=RTOL, atol=ATOL):
    ok, mx, bad = close_enough(got, want, rtol, atol)
    assert ok, f"{label}: {bad} elements out of tolerance, max abs err {mx:.3e}"


def gnorm_of_first_step(spec, B, seed):
    """Global norm of the first step's deltas (oracle, clipping off)."""
    base = MlpSpec(spec.sizes, spec.activation, spec.optimizer, spec.loss, dropout_p=spec.dropout_p,
                   layernorm=spec.layernorm)
    ws, bs = data.he_uniform(seed, spec.sizes)
    X, Y = data.batch(seed, spec.sizes, B, spec.loss)
    t = Trainer(load_oracle(), base, B)
    t.set_all_params(ws, bs)
    t.step(X, Y, 1e-3)
    g = sum(float(np.sum(t.debug_buffer(BUF_DELTA, i).astype(np.float64) ** 2)) for i in range(spec.n_layers))
    t.close()
    return float(np.sqrt(g))


ADAPTIVE = ("adam", "adamw", "adagrad")


def flat64(lib, t, spec):
    out = []
    for i, (r, c) in enumerate(spec.shapes()):
        w = np.zeros(r * c)
        b = np.zeros(c)
        lib.lib.volta_oracle_get_params_f64(t.h, i, w.ctypes.data_as(C.POINTER(C.c_double)),
                                            b.ctypes.data_as(C.POINTER(C.c_double)))
        out.append(np.concatenate([w, b]))
    return out


def flat(params):
    return [np.concatenate([w.ravel(), b]).astype(np.float64) for w, b in zip(*params)]


def run(lib, spec, B, seed, lr, steps, f64=False):
    ws, bs = data.he_uniform(seed, spec.sizes)
    batches = [data.batch(seed + k, spec.sizes, B, spec.loss) for k in range(2)]
    t = oracle_trainer(lib, spec, B, f64=True) if f64 else Trainer(lib, spec, B)
    t.set_all_params(ws, bs)
    losses = []
    for s in range(steps):
        X, Y = batches[s % 2]
        t.step(X, Y, lr)
        losses.append(t.loss())
    out = {"loss": np.array(losses, np.float32), "params": t.get_params(), "status": t.status()}
    if f64:
        out["flat64"] = flat64(lib, t, spec)
    nh = spec.n_layers - 1
    if spec.layernorm:
        out["gamma"] = [t.debug_buffer(BUF_LN_GAMMA, i) for i in range(nh)]
        out["beta"] = [t.debug_buffer(BUF_LN_BETA, i) for i in range(nh)]
    if spec.dropout_p > 0:
        out["mask"] = [t.debug_buffer(BUF_DROPOUT_MASK, i) for i in range(nh)]
        out["rng"] = t.get_dropout_rng()
    t.close()
    return out


def compare(g, o, label, spec=None, lr=0.0, steps=0, twin=None):
    assert g["status"] == 0, f"{label}: GPU status {g['status']}"
    assert_close(g["loss"], o["loss"], f"{label} loss")
    if spec is not None and spec.optimizer in ADAPTIVE:
        for i, (a, b, t) in enumerate(zip(flat(g["params"]), flat(o["params"]), twin["flat64"])):
            err = np.abs(a - b)
            out = err > ATOL + RTOL * np.abs(b)
            worst = float(err[out].max()) if out.any() else 0.0
            rh = float(np.sqrt(np.mean((a - t) ** 2)))
            ro = float(np.sqrt(np.mean((b - t) ** 2)))
            say(f"  layer {i}: {int(out.sum())} of {a.size} outside tolerance (worst {worst:.2e}); "
                f"rms vs fp64 hip {rh:.2e} oracle {ro:.2e}")
            assert out.mean() <= 1e-3, f"{label} layer {i}: {int(out.sum())} parameters out of tolerance"
            assert worst <= 4 * lr * steps + ATOL, f"{label} layer {i}: outlier {worst:.3e}"
            assert rh <= 3 * ro + 1e-7, f"{label} layer {i}: hip rms error {rh:.3e} vs oracle {ro:.3e}"
    else:
        for i, (a, b) in enumerate(zip(g["params"][0], o["params"][0])):
            assert_close(a, b, f"{label} W{i}")
        for i, (a, b) in enumerate(zip(g["params"][1], o["params"][1])):
            assert_close(a, b, f"{label} b{i}")
    for key in ("gamma", "beta"):
        for i, (a, b) in enumerate(zip(g.get(key, []), o.get(key, []))):
            assert_close(a, b, f"{label} {key}{i}")
    for i, (a, b) in enumerate(zip(g.get("mask", []), o.get("mask", []))):
        np.testing.assert_array_equal(a, b, err_msg=f"{label} dropout mask {i}")
    assert g.get("rng") == o.get("rng"), f"{label}: dropout LCG state differs"


# (label, spec, batch, lr); shapes cover the narrow output kernels (Ln <= 16),
# the GEMM loss head (Ln <= 64), the stand-alone loss (Ln > 64), split-K
# (K >= 1024 over few tiles) and row widths that are not multiples of 4.
CASES = [
    ("ln_relu_sgd", MlpSpec([16, 64, 48, 4], "relu", "sgd", layernorm=True), 32, 0.05),
    ("ln_gelu_adam", MlpSpec([32, 96, 80, 24], "gelu", "adam", layernorm=True), 64, 1e-3),
    ("ln_tanh_adamw", MlpSpec([24, 130, 70, 100], "tanh", "adamw", layernorm=True), 48, 1e-3),
    ("ln_sigmoid_ce", MlpSpec([20, 64, 10], "sigmoid", "adam", "ce", layernorm=True), 40, 1e-3),
    ("drop_relu_sgd", MlpSpec([16, 64, 48, 4], "relu", "sgd", dropout_p=0.3), 32, 0.05),
    ("drop_silu_adam", MlpSpec([32, 96, 80, 24], "silu", "adam", dropout_p=0.1), 64, 1e-3),
    ("drop_leaky_adagrad", MlpSpec([24, 130, 70, 100], "leaky_relu", "adagrad", dropout_p=0.5), 48, 1e-2),
    ("clip_tanh_sgd", MlpSpec([16, 64, 48, 4], "tanh", "sgd", clip_grad=-1.0), 32, 0.05),
    ("clip_relu_adam", MlpSpec([32, 96, 80, 24], "relu", "adam", clip_grad=-1.0), 64, 1e-3),
    ("clip_gelu_adagrad_wide", MlpSpec([24, 130, 70, 100], "gelu", "adagrad", clip_grad=-1.0), 48, 1e-2),
    ("all_gelu_adam", MlpSpec([48, 128, 96, 10], "gelu", "adam", layernorm=True, dropout_p=0.2, clip_grad=-1.0),
     64, 1e-3),
    ("all_relu_sgd_splitk", MlpSpec([1024, 256, 128, 8], "relu", "sgd", layernorm=True, dropout_p=0.25,
                                    clip_grad=-1.0), 64, 0.02),
    ("all_tanh_adamw_ce", MlpSpec([64, 200, 120, 30], "tanh", "adamw", "ce", layernorm=True, dropout_p=0.15,
                                  clip_grad=-1.0), 96, 1e-3),
    # softmax as the hidden activation (a row operation, :727-740, :898-906)
    ("softmax_sgd", MlpSpec([16, 64, 48, 4], "softmax", "sgd"), 32, 0.5),
    ("softmax_adam_ce", MlpSpec([32, 96, 80, 24], "softmax", "adam", "ce"), 64, 1e-3),
    ("softmax_drop_clip_adagrad", MlpSpec([24, 130, 70, 100], "softmax", "adagrad", dropout_p=0.2,
                                          clip_grad=-1.0), 48, 1e-2),
    ("softmax_ln_sgd", MlpSpec([20, 64, 10], "softmax", "sgd", layernorm=True), 32, 0.05),
    ("softmax_all_adam", MlpSpec([32, 96, 12], "softmax", "adam", layernorm=True, dropout_p=0.1, clip_grad=-1.0),
     64, 1e-3),
]
# (LayerNorm over the outputs of a softmax divides by their small spread, so
# its backward multiplies deltas by 1/sigma, ~50 per layer here; with two such
# layers the fp32 oracle itself leaves the tolerance of its fp64 twin, so the
# combined softmax cases use one hidden layer.)


def resolve(spec, B, seed):
    """clip_grad = -1 marks 'half the first step's delta norm' (so the clip
    is taken on every step of the run)."""
    if spec.clip_grad < 0:
        spec = MlpSpec(spec.sizes, spec.activation, spec.optimizer, spec.loss, clip_grad=0.0,
                       dropout_p=spec.dropout_p, layernorm=spec.layernorm)
        spec.clip_grad = float(np.float32(0.5 * gnorm_of_first_step(spec, B, seed)))
    return spec


@pytest.mark.parametrize("label,spec,B,lr", CASES, ids=[c[0] for c in CASES])
def test_extras_match_oracle(label, spec, B, lr):
    seed = 11
    spec = resolve(spec, B, seed)
    say(f"extras {label}: {spec.text()} B={B}")
    g = run(load_hip(), spec, B, seed, lr, 4)
    o = run(load_oracle(), spec, B, seed, lr, 4)
    twin = run(load_oracle(), spec, B, seed, lr, 4, f64=True) if spec.optimizer in ADAPTIVE else None
    compare(g, o, label, spec, lr, 4, twin)


def test_extras_two_gpu_runs_bit_identical():
    spec = resolve(CASES[-2][1], 64, 5)
    say(f"extras determinism: {spec.text()}")
    a = run(load_hip(), spec, 64, 5, 1e-3, 3)
    b = run(load_hip(), spec, 64, 5, 1e-3, 3)
    np.testing.assert_array_equal(a["loss"], b["loss"])
    for x, y in zip(a["params"][0] + a["params"][1] + a["gamma"] + a["beta"],
                    b["params"][0] + b["params"][1] + b["gamma"] + b["beta"]):
        np.testing.assert_array_equal(x, y)


def test_extras_state_resume_matches_uninterrupted_run():
    """get_state (optimizer moments, LayerNorm gamma/beta) and the dropout
    LCG state moved to a fresh handle continue the run exactly."""
    spec = MlpSpec([32, 96, 80, 24], "gelu", "adam", layernorm=True, dropout_p=0.2)
    B, lr = 32, 1e-3
    say(f"extras resume: {spec.text()}")
    lib = load_hip()
    ws, bs = data.he_uniform(3, spec.sizes)
    X, Y = data.batch(3, spec.sizes, B, "mse")
    full = Trainer(lib, spec, B)
    full.set_all_params(ws, bs)
    for _ in range(4):
        full.step(X, Y, lr)
    want = full.get_params()
    first = Trainer(lib, spec, B)
    first.set_all_params(ws, bs)
    for _ in range(2):
        first.step(X, Y, lr)
    w, b = first.get_params()
    state, step = first.get_state()
    rng = first.get_dropout_rng()
    assert state.size == first.state_size() == 2 * sum(r * c + c for r, c in spec.shapes()) + 2 * (96 + 80)
    second = Trainer(lib, spec, B)
    second.set_all_params(w, b)
    second.set_state(state, step)
    second.set_dropout_rng(rng)
    for _ in range(2):
        second.step(X, Y, lr)
    got = second.get_params()
    for x, y in zip(got[0] + got[1], want[0] + want[1]):
        np.testing.assert_array_equal(x, y)
    for t in (full, first, second):
        t.close()


@pytest.mark.parametrize("act,rows", [("relu", 1), ("relu", 37), ("relu", 200), ("softmax", 45)])
def test_infer_with_layernorm_matches_oracle(act, rows):
    """Inference applies the activation and LayerNorm with the trained
    gamma/beta and no dropout (and leaves the dropout stream untouched)."""
    spec = MlpSpec([24, 64, 48, 6], act, "adam", layernorm=True, dropout_p=0.2)
    B = 32
    say(f"extras infer rows={rows}: {spec.text()}")
    outs = []
    for lib in (load_hip(), load_oracle()):
        ws, bs = data.he_uniform(9, spec.sizes)
        X, Y = data.batch(9, spec.sizes, B, "mse")
        t = Trainer(lib, spec, B)
        t.set_all_params(ws, bs)
        for _ in range(3):
            t.step(X, Y, 1e-3)
        rng = t.get_dropout_rng()
        Xi = data.normal(77, (rows, spec.sizes[0]))
        outs.append(t.infer(Xi))
        assert t.get_dropout_rng() == rng
        t.close()
    assert_close(outs[0], outs[1], "infer")
