"""Pins the CPU oracle (CPU only, no GPU).

Each check is chosen so that a plausible mistake in the oracle (a dropped
term, a wrong sign or index, a transposed operand) fails one of them:
  * torch-float64 goldens (independent autograd + torch.optim), including the
    reference's own tiny-MLP literals (tests/pytorch_parity.rs:120-243);
  * the reference's Adam known-answer test (optimizer.rs:831-862);
  * closed forms: Adagrad step 1, CE on uniform logits = ln C;
  * central finite differences of the loss against the fp64 twin's gradient;
  * the reference's own C GEMM (gemm_shim.c, built into oracle/_ref/);
  * exact integer GEMMs;
  * the LCG Xavier stream's range, moments and continuity across layers.
"""
import ctypes as C
import json
import math
import os

import numpy as np
import pytest

from tests.oracle_lib import load_ref_shim
from volta_amd.abi import (BUF_DELTA, BUF_DROPOUT_MASK, BUF_LN_BETA, BUF_LN_GAMMA, HEADER_SYMBOLS, MlpSpec, Trainer,
                           fptr)

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = json.load(open(os.path.join(HERE, "golden", "train_step_golden.json")))["cases"]
KAT = json.load(open(os.path.join(HERE, "golden", "optimizer_kat.json")))


def spec_of(case):
    return MlpSpec(case["sizes"], case["activation"], case["optimizer"], case["loss"],
                   eps=case["eps"], weight_decay=case["weight_decay"])


def oracle_trainer(lib, spec, batch, f64=False):
    if f64:
        cs = spec.to_c()
        h = lib.lib.volta_oracle_init_f64(C.byref(cs), batch)
        return Trainer(lib, spec, batch, handle=h)
    return Trainer(lib, spec, batch)


def load_inputs(case):
    inp = case["inputs"]
    sizes = case["sizes"]
    ws = [np.array(w, np.float32).reshape(sizes[i], sizes[i + 1]) for i, w in enumerate(inp["w"])]
    bs = [np.array(b, np.float32) for b in inp["b"]]
    B = case["batch"]
    Xs = [np.array(x, np.float32).reshape(B, sizes[0]) for x in inp["X"]]
    if case["loss"] == "ce":
        Ys = [np.array(y, np.int32) for y in inp["Y"]]
    else:
        Ys = [np.array(y, np.float32).reshape(B, sizes[-1]) for y in inp["Y"]]
    return ws, bs, Xs, Ys


def run_oracle_case(lib, case, f64=False):
    spec = spec_of(case)
    ws, bs, Xs, Ys = load_inputs(case)
    t = oracle_trainer(lib, spec, case["batch"], f64=f64)
    t.set_all_params(ws, bs)
    losses = []
    for s in range(case["steps"]):
        t.step(Xs[s % len(Xs)], Ys[s % len(Ys)], case["lr"])
        if f64:
            losses.append(lib.lib.volta_oracle_loss_f64(t.h))
        else:
            losses.append(t.loss())
    if f64:
        out_w, out_b = [], []
        for i, (r, c) in enumerate(spec.shapes()):
            w = np.zeros(r * c, np.float64)
            b = np.zeros(c, np.float64)
            lib.lib.volta_oracle_get_params_f64(t.h, i, w.ctypes.data_as(C.POINTER(C.c_double)),
                                                b.ctypes.data_as(C.POINTER(C.c_double)))
            out_w.append(w)
            out_b.append(b)
    else:
        ws2, bs2 = t.get_params()
        out_w = [w.ravel().astype(np.float64) for w in ws2]
        out_b = [b.astype(np.float64) for b in bs2]
    t.close()
    return np.array(losses), out_w, out_b


@pytest.mark.parametrize("case", GOLDEN, ids=[c["name"] for c in GOLDEN])
def test_oracle_f64_matches_torch_golden(oracle, case):
    """The fp64 twin must agree with torch-float64 to ~1e-9: any wrong term in
    the forward, backward, loss or optimizer shows up far above that."""
    losses, ws, bs = run_oracle_case(oracle, case, f64=True)
    exp = case["expected"]
    np.testing.assert_allclose(losses, exp["losses"], rtol=1e-8, atol=1e-10)
    for i in range(len(ws)):
        np.testing.assert_allclose(ws[i], exp["w"][i], rtol=1e-8, atol=1e-10, err_msg=f"W{i}")
        np.testing.assert_allclose(bs[i], exp["b"][i], rtol=1e-8, atol=1e-10, err_msg=f"b{i}")


@pytest.mark.parametrize("case", GOLDEN, ids=[c["name"] for c in GOLDEN])
def test_oracle_f32_matches_torch_golden(oracle, case):
    """The fp32 oracle (reference arithmetic) stays within fp32 rounding of the
    float64 result."""
    losses, ws, bs = run_oracle_case(oracle, case, f64=False)
    exp = case["expected"]
    np.testing.assert_allclose(losses, exp["losses"], rtol=2e-5, atol=1e-6)
    for i in range(len(ws)):
        np.testing.assert_allclose(ws[i], exp["w"][i], rtol=2e-5, atol=2e-6, err_msg=f"W{i}")
        np.testing.assert_allclose(bs[i], exp["b"][i], rtol=2e-5, atol=2e-6, err_msg=f"b{i}")


def test_tiny_fixture_single_sgd_step_gradients(oracle):
    """Reference parity fixture, one SGD step: recover the gradient from the
    update (g = (w0 - w1)/lr) and compare with torch's step-0 gradients."""
    case = next(c for c in GOLDEN if c["name"] == "tiny_relu_sgd_mse")
    spec = spec_of(case)
    ws, bs, Xs, Ys = load_inputs(case)
    t = oracle_trainer(oracle, spec, 2, f64=True)
    t.set_all_params(ws, bs)
    t.step(Xs[0], Ys[0], case["lr"])
    lr = float(np.float32(case["lr"]))  # the ABI takes lr as float32
    g = case["expected"]["grads_step0"]
    for i, (r, c) in enumerate(spec.shapes()):
        w = np.zeros(r * c)
        b = np.zeros(c)
        oracle.lib.volta_oracle_get_params_f64(t.h, i, w.ctypes.data_as(C.POINTER(C.c_double)),
                                               b.ctypes.data_as(C.POINTER(C.c_double)))
        np.testing.assert_allclose((ws[i].ravel().astype(np.float64) - w) / lr, g["w"][i], rtol=1e-8, atol=1e-10)
        np.testing.assert_allclose((bs[i].astype(np.float64) - b) / lr, g["b"][i], rtol=1e-8, atol=1e-10)
    t.close()


def test_adam_reference_kat(oracle):
    """optimizer.rs:831-862: w=0.5, g=0.1, lr=1e-3, step 1 -> 0.499000."""
    k = KAT["adam_step1"]
    w = np.array([k["w"]], np.float32)
    m = np.zeros(1, np.float32)
    v = np.zeros(1, np.float32)
    g = np.array([k["g"]], np.float32)
    bc1 = np.float32(1.0) - np.float32(0.9) ** 1
    bc2 = np.float32(1.0) - np.float32(0.999) ** 1
    oracle.lib.volta_oracle_adam(fptr(w), fptr(m), fptr(v), fptr(g), 1, 0.9, 0.999, float(bc1), float(bc2),
                                 k["lr"], 1e-8, 0.0)
    assert abs(float(w[0]) - k["expected"]) < k["tol"]


def test_adagrad_step1_closed_form(oracle):
    """Adagrad from G=0: w -= lr*g/(|g|+eps), i.e. ~lr*sign(g)."""
    rng = np.random.default_rng(0)
    g = rng.standard_normal(1000).astype(np.float32)
    w = rng.standard_normal(1000).astype(np.float32)
    G = np.zeros(1000, np.float32)
    w0 = w.copy()
    oracle.lib.volta_oracle_adagrad(fptr(w), fptr(G), fptr(g), 1000, 0.01, 1e-10)
    np.testing.assert_allclose(G, g * g, rtol=1e-7)
    np.testing.assert_allclose(w0 - w, 0.01 * np.sign(g), rtol=1e-5)


def test_adam_vector_tail_split(oracle):
    """adam_update_slice (mlp_train_rust_codegen.rs:341-388) computes v with
    (1-b2)*(g*g) in its 8-wide loop and ((1-b2)*g)*g in the scalar tail; the
    oracle follows both.  Checked against numpy float32 arithmetic."""
    n = 13
    rng = np.random.default_rng(1)
    g = rng.standard_normal(n).astype(np.float32) * np.float32(3.3)
    v = np.abs(rng.standard_normal(n)).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    m = rng.standard_normal(n).astype(np.float32)
    b2 = np.float32(0.999)
    one = np.float32(1)
    v_vec = b2 * v + (one - b2) * (g * g)
    v_tail = b2 * v + ((one - b2) * g) * g
    oracle.lib.volta_oracle_adam(fptr(w), fptr(m), fptr(v), fptr(g), n, 0.9, 0.999, 0.1, 0.001, 1e-3, 1e-8, 0.0)
    np.testing.assert_array_equal(v[:8], v_vec[:8])
    np.testing.assert_array_equal(v[8:], v_tail[8:])


def test_ce_uniform_logits_closed_form(oracle):
    """All-zero weights/biases give uniform logits: loss = ln C exactly in
    float64 and the output-bias gradient is (1/C - onehot)/B summed over B."""
    sizes = [4, 3, 5]
    B = 4
    spec = MlpSpec(sizes, "relu", "sgd", "ce")
    t = oracle_trainer(oracle, spec, B, f64=True)
    for i, (r, c) in enumerate(spec.shapes()):
        t.set_params(i, np.zeros((r, c), np.float32), np.zeros(c, np.float32))
    X = np.ones((B, 4), np.float32)
    lab = np.array([0, 1, 1, 4], np.int32)
    t.step(X, lab, 1.0)
    assert abs(oracle.lib.volta_oracle_loss_f64(t.h) - math.log(5)) < 1e-15
    b = np.zeros(5)
    w = np.zeros(15)
    oracle.lib.volta_oracle_get_params_f64(t.h, 1, w.ctypes.data_as(C.POINTER(C.c_double)),
                                           b.ctypes.data_as(C.POINTER(C.c_double)))
    onehot = np.eye(5)[lab]
    expected_db = ((0.2 - onehot) / B).sum(axis=0)
    np.testing.assert_allclose(-b, expected_db, atol=1e-15)
    t.close()


@pytest.mark.parametrize("act", ["relu", "sigmoid", "tanh", "leaky_relu", "silu", "gelu", "softmax"])
@pytest.mark.parametrize("loss", ["mse", "ce"])
def test_f64_gradient_matches_finite_differences(oracle, act, loss):
    """Gradient recovered from one SGD step (lr=1) of the fp64 twin equals the
    central finite difference of its loss (evaluated with lr=0 steps)."""
    sizes = [3, 5, 4, 3]
    B = 3
    spec = MlpSpec(sizes, act, "sgd", loss)
    rng = np.random.default_rng(7)
    ws = [(rng.standard_normal((r, c)) * 0.7).astype(np.float32) for r, c in spec.shapes()]
    bs = [(rng.standard_normal(c) * 0.2).astype(np.float32) for _, c in spec.shapes()]
    X = rng.standard_normal((B, 3)).astype(np.float32)
    Y = rng.integers(0, 3, B).astype(np.int32) if loss == "ce" else rng.standard_normal((B, 3)).astype(np.float32)

    def loss_at(wlist, blist):
        t = oracle_trainer(oracle, spec, B, f64=True)
        for i in range(len(wlist)):
            t.set_params(i, wlist[i], blist[i])
        t.step(X, Y, 0.0)
        val = oracle.lib.volta_oracle_loss_f64(t.h)
        t.close()
        return val

    t = oracle_trainer(oracle, spec, B, f64=True)
    t.set_all_params(ws, bs)
    t.step(X, Y, 1.0)
    grads_w = []
    for i, (r, c) in enumerate(spec.shapes()):
        w = np.zeros(r * c)
        b = np.zeros(c)
        oracle.lib.volta_oracle_get_params_f64(t.h, i, w.ctypes.data_as(C.POINTER(C.c_double)),
                                               b.ctypes.data_as(C.POINTER(C.c_double)))
        grads_w.append((ws[i].ravel().astype(np.float64) - w, bs[i].astype(np.float64) - b))
    t.close()
    # Perturbations must be float32-representable (set_params takes float32):
    # use h = 2^-10 on weights that are multiples of 2^-10 after rounding.
    h = 2.0 ** -10
    for li in range(len(ws)):
        for idx in [0, ws[li].size // 2, ws[li].size - 1]:
            wp = [w.copy() for w in ws]
            wm = [w.copy() for w in ws]
            wp[li].ravel()[idx] += np.float32(h)
            wm[li].ravel()[idx] -= np.float32(h)
            hp = float(wp[li].ravel()[idx]) - float(ws[li].ravel()[idx])
            hm = float(ws[li].ravel()[idx]) - float(wm[li].ravel()[idx])
            fd = (loss_at(wp, bs) - loss_at(wm, bs)) / (hp + hm)
            g = grads_w[li][0][idx]
            # relu/leaky kinks are avoided by the random data; tolerance is
            # the O(h^2) truncation error.
            assert abs(fd - g) <= 2e-5 + 1e-3 * abs(g), (li, idx, fd, g)
        bp = [b.copy() for b in bs]
        bm = [b.copy() for b in bs]
        bp[li][0] += np.float32(h)
        bm[li][0] -= np.float32(h)
        fd = (loss_at(ws, bp) - loss_at(ws, bm)) / (float(bp[li][0]) - float(bm[li][0]))
        g = grads_w[li][1][0]
        assert abs(fd - g) <= 2e-5 + 1e-3 * abs(g), (li, "b", fd, g)


@pytest.mark.parametrize("m,k,n", [(5, 7, 3), (64, 33, 17), (70, 129, 96)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1)])
def test_oracle_gemm_integer_exact(oracle, m, k, n, ta, tb):
    """Integer-valued operands: every summation order gives the exact result."""
    rng = np.random.default_rng(m * 1000 + k)
    A = rng.integers(-8, 9, (k, m) if ta else (m, k)).astype(np.float32)
    B = rng.integers(-8, 9, (n, k) if tb else (k, n)).astype(np.float32)
    Cm = np.zeros((m, n), np.float32)
    oracle.lib.volta_oracle_gemm(fptr(Cm), fptr(A), fptr(B), m, k, n, ta, tb)
    ref = (A.T if ta else A).astype(np.int64) @ (B.T if tb else B).astype(np.int64)
    np.testing.assert_array_equal(Cm, ref.astype(np.float32))


def test_oracle_gemm_matches_reference_gemm_shim(oracle):
    """The reference's own C GEMM (gemm_shim.c) vs the oracle on random
    float32 data; skipped where oracle/_ref was not built."""
    shim = load_ref_shim()
    if shim is None:
        pytest.skip("oracle/_ref/libvolta_gemm_shim.so not built (reference tree absent)")
    rng = np.random.default_rng(3)
    m, k, n = 64, 256, 96
    A = rng.standard_normal((m, k)).astype(np.float32)
    B = rng.standard_normal((k, n)).astype(np.float32)
    At = np.ascontiguousarray(A.T)
    c_ref = np.zeros((m, n), np.float32)
    c_or = np.zeros((m, n), np.float32)
    shim.volta_gemm_f32(fptr(c_ref), fptr(A), fptr(B), m, k, n)
    oracle.lib.volta_oracle_gemm(fptr(c_or), fptr(A), fptr(B), m, k, n, 0, 0)
    exact = A.astype(np.float64) @ B.astype(np.float64)
    bound = 2 * k * np.finfo(np.float32).eps * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64))
    assert np.all(np.abs(c_ref - exact) <= bound)
    assert np.all(np.abs(c_or - exact) <= bound)
    np.testing.assert_allclose(c_or, c_ref, rtol=1e-4, atol=1e-4)
    # transposed-A (dW) and transposed-B (dX) forms
    c_ref.fill(0)
    shim.volta_gemm_tn_f32(fptr(c_ref), fptr(At), fptr(B), m, k, n)
    oracle.lib.volta_oracle_gemm(fptr(c_or), fptr(At), fptr(B), m, k, n, 1, 0)
    np.testing.assert_allclose(c_or, c_ref, rtol=1e-4, atol=1e-4)
    Bt = np.ascontiguousarray(B.T)  # [n x k]
    shim.volta_gemm_nt_f32(fptr(c_ref), fptr(A), fptr(B), m, k, n)  # takes B^T pre-transposed = B
    oracle.lib.volta_oracle_gemm(fptr(c_or), fptr(A), fptr(Bt), m, k, n, 0, 1)
    np.testing.assert_allclose(c_or, c_ref, rtol=1e-4, atol=1e-4)


def test_lcg_xavier_stream(oracle):
    """volta_train_init draws W_i from one LCG stream seeded 42
    (mlp_train_rust_codegen.rs:629-658): values in [-lim, lim), mean ~0,
    variance ~lim^2/3, biases 0, and layer 1 continues layer 0's stream."""
    sizes = [64, 128, 32]
    spec = MlpSpec(sizes, "relu", "sgd")
    t = Trainer(oracle, spec, 4)
    ws, bs = t.get_params()
    t.close()
    for (r, c), w, b in zip(spec.shapes(), ws, bs):
        lim = math.sqrt(6.0 / (r + c))
        assert w.min() >= -lim and w.max() < lim
        assert abs(w.mean()) < 0.02 * lim
        assert abs(w.var() / (lim * lim / 3) - 1) < 0.03
        assert not b.any()
    rng = C.c_uint64(42)
    w0 = np.zeros(64 * 128, np.float32)
    oracle.lib.volta_oracle_lcg_xavier(fptr(w0), w0.size, 64, 128, C.byref(rng))
    np.testing.assert_array_equal(w0.reshape(64, 128), ws[0])
    # first draw from an independent big-integer evaluation of the recurrence
    x = (42 * 6364136223846793005 + 1442695040888963407) % (1 << 64)
    f = np.float32((x >> 11) & ((1 << 53) - 1)) / np.float32(1 << 53)
    lim0 = np.sqrt(np.float32(6.0) / np.float32(192.0))
    assert ws[0][0, 0] == (f * np.float32(2) - np.float32(1)) * lim0
    w1 = np.zeros(128 * 32, np.float32)
    oracle.lib.volta_oracle_lcg_xavier(fptr(w1), w1.size, 128, 32, C.byref(rng))
    np.testing.assert_array_equal(w1.reshape(128, 32), ws[1])


def test_spec_parse(oracle):
    s = oracle.parse_spec("512-1024-1024-512-256-1:relu:adam")
    assert s.n_sizes == 6 and list(s.sizes[:6]) == [512, 1024, 1024, 512, 256, 1]
    assert s.optimizer == 1 and s.loss == 0
    assert abs(s.beta1 - 0.9) < 1e-7 and abs(s.eps - 1e-8) < 1e-15 and s.weight_decay == 0.0
    s = oracle.parse_spec("1024-4096-4096-1024-10:relu:adagrad:ce:eps=1e-10")
    assert s.loss == 1 and abs(s.eps - 1e-10) < 1e-17
    s = oracle.parse_spec("512-2048-2048-512-1:gelu:adamw")
    assert abs(s.weight_decay - 0.01) < 1e-9
    for bad in ["", "3-4", "3-4:relu", "3-0-2:relu:sgd", "3-4:swish:sgd", "3-4:relu:lamb",
                "3-1:relu:sgd:ce", "3-4:relu:sgd:eps=0", "3-4:relu:sgd:foo=1"]:
        with pytest.raises(ValueError):
            oracle.parse_spec(bad)


def test_oracle_exports_header_symbols(oracle):
    for name in HEADER_SYMBOLS:
        assert hasattr(oracle.lib, name), name


def test_oracle_status_and_bad_args(oracle):
    # tanh, because ReLU maps a NaN input to 0 (pre > 0 is false)
    spec = MlpSpec([3, 4, 2], "tanh", "sgd")
    t = Trainer(oracle, spec, 2)
    t.set_params(5, np.zeros((3, 4), np.float32), np.zeros(4, np.float32))  # ignored, flagged
    assert t.status() & 2
    t.clear_status()
    X = np.full((2, 3), np.nan, np.float32)
    t.step(X, np.zeros((2, 2), np.float32), 0.1)
    assert t.status() & 1
    t.close()


def test_oracle_state_roundtrip(oracle):
    """get_state/set_state lets an Adam run resume bit-identically."""
    spec = MlpSpec([5, 7, 3], "tanh", "adam")
    rng = np.random.default_rng(11)
    X = rng.standard_normal((4, 5)).astype(np.float32)
    Y = rng.standard_normal((4, 3)).astype(np.float32)
    a = Trainer(oracle, spec, 4)
    for _ in range(3):
        a.step(X, Y, 1e-2)
    st, step = a.get_state()
    ws, bs = a.get_params()
    assert step == 3 and st.size == a.state_size()
    b = Trainer(oracle, spec, 4)
    b.set_all_params(ws, bs)
    b.set_state(st, step)
    for _ in range(2):
        a.step(X, Y, 1e-2)
        b.step(X, Y, 1e-2)
    wa, ba = a.get_params()
    wb, bb = b.get_params()
    for x, y in zip(wa + ba, wb + bb):
        np.testing.assert_array_equal(x, y)


# ---------------------------------------------------------------------------
# Forward-only entry points and live hyperparameters
# ---------------------------------------------------------------------------
def _np_act(name, x):
    """Activation closed forms (mlp_train_rust_codegen.rs:563-596), float64."""
    if name == "relu":
        return np.maximum(x, 0.0)
    if name == "leaky_relu":
        return np.where(x > 0, x, 0.01 * x)
    if name == "sigmoid":
        return 1.0 / (1.0 + np.exp(-x))
    if name == "tanh":
        return np.tanh(x)
    if name == "silu":
        return x / (1.0 + np.exp(-x))
    if name == "gelu":
        return 0.5 * x * (1.0 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))
    raise ValueError(name)


def _np_forward(ws, bs, X, act):
    a = X.astype(np.float64)
    for i, (w, b) in enumerate(zip(ws, bs)):
        z = a @ w.astype(np.float64) + b.astype(np.float64)
        a = z if i == len(ws) - 1 else _np_act(act, z)
    return a


@pytest.mark.parametrize("act", ["relu", "sigmoid", "tanh", "leaky_relu", "silu", "gelu"])
def test_oracle_infer_matches_closed_form_forward(oracle, act):
    """volta_train_infer = the model's forward (output pre-activation) for any
    row count: the fp64 twin equals a numpy float64 forward, the fp32 oracle
    is within fp32 rounding; rows below, at and above the batch (chunks)."""
    spec = MlpSpec([12, 20, 16, 5], act, "adam")
    rng = np.random.default_rng(3)
    ws = [rng.uniform(-0.5, 0.5, (r, c)).astype(np.float32) for r, c in spec.shapes()]
    bs = [rng.uniform(-0.1, 0.1, c).astype(np.float32) for _, c in spec.shapes()]
    for rows in (3, 8, 21):
        X = rng.standard_normal((rows, 12)).astype(np.float32)
        want = _np_forward(ws, bs, X, act)
        for f64, tol in ((True, 1e-6), (False, 1e-5)):
            t = oracle_trainer(oracle, spec, 8, f64=f64)
            t.set_all_params(ws, bs)
            got = t.infer(X)
            np.testing.assert_allclose(got, want, rtol=tol, atol=tol)
            t.close()


def test_oracle_volta_infer_symbol(oracle):
    """The reference's inference signature volta_infer(in, in_n, out, out_n)
    runs the bound model; bad sizes and an unbound model leave out alone."""
    spec = MlpSpec([6, 10, 3], "tanh", "sgd")
    t = Trainer(oracle, spec, 4)
    X = np.random.default_rng(1).standard_normal((7, 6)).astype(np.float32)
    want = t.infer(X)
    f = oracle.lib
    out = np.full(7 * 3, -7.0, np.float32)
    f.volta_infer_bind(None)
    f.volta_infer(fptr(X), X.size, fptr(out), out.size)
    assert (out == -7.0).all() and b"bound" in f.volta_train_last_error()
    f.volta_infer_bind(t.h)
    f.volta_infer(fptr(X), X.size - 1, fptr(out), out.size)
    assert (out == -7.0).all()
    f.volta_infer(fptr(X), X.size, fptr(out), out.size)
    np.testing.assert_array_equal(out.reshape(7, 3), want)
    f.volta_infer_bind(None)
    t.close()


def test_oracle_set_hparams_equals_spec_from_start(oracle):
    """set_hparams before the first step gives the same bits as a handle
    created with those hyperparameters; out-of-range values are rejected."""
    base = MlpSpec([8, 16, 4], "relu", "adamw")
    new = MlpSpec([8, 16, 4], "relu", "adamw", beta1=0.8, beta2=0.99, eps=1e-6, weight_decay=0.05)
    rng = np.random.default_rng(5)
    X = rng.standard_normal((4, 8)).astype(np.float32)
    Y = rng.standard_normal((4, 4)).astype(np.float32)
    a, b = Trainer(oracle, base, 4), Trainer(oracle, new, 4)
    a.set_hparams(0.8, 0.99, 1e-6, 0.05)
    for _ in range(3):
        a.step(X, Y, 1e-2)
        b.step(X, Y, 1e-2)
    wa, ba = a.get_params()
    wb, bb = b.get_params()
    for p, q in zip(wa + ba, wb + bb):
        np.testing.assert_array_equal(p, q)
    with pytest.raises(ValueError):
        a.set_hparams(1.5, 0.99, 1e-6, 0.0)
    a.close()
    b.close()


# ---------------------------------------------------------------------------
# Codegen extras: dropout, LayerNorm, gradient clipping
# ---------------------------------------------------------------------------
def _lcg_keep(n, p, state=12345678):
    """The dropout stream written out with Python integers: state' = state*A
    + C mod 2^64, r = f32(state >> 33) / 2^31, keep when r >= p."""
    A, Cc, M = 6364136223846793005, 1442695040888963407, 1 << 64
    keep = np.zeros(n, bool)
    for k in range(n):
        state = (state * A + Cc) % M
        r = np.float32(state >> 33) / np.float32(2147483648.0)
        keep[k] = r >= np.float32(p)
    return keep, state


def test_oracle_dropout_mask_follows_the_lcg_stream(oracle):
    """act_1 after a zero-lr step = relu(pre_0) * mask / (1 - p), with the
    mask drawn from the reference's LCG in row-major order; the stream
    continues across layers and steps."""
    spec = MlpSpec([5, 12, 9, 2], "relu", "sgd", dropout_p=0.3)
    B = 4
    t = Trainer(oracle, spec, B)
    rng = np.random.default_rng(9)
    X = rng.standard_normal((B, 5)).astype(np.float32)
    Y = rng.standard_normal((B, 2)).astype(np.float32)
    keep_scale = np.float32(1.0) / (np.float32(1.0) - np.float32(0.3))
    state = 12345678
    from volta_amd.abi import BUF_ACT
    for step in range(2):
        t.step(X, Y, 0.0)
        k1, state = _lcg_keep(B * 12, 0.3, state)
        k2, state = _lcg_keep(B * 9, 0.3, state)
        a1 = t.debug_buffer(BUF_ACT, 1).reshape(B, 12)
        ws, bs = t.get_params()
        pre0 = X @ ws[0] + bs[0]
        want1 = np.maximum(pre0, 0) * (k1.reshape(B, 12).astype(np.float32) * keep_scale)
        np.testing.assert_allclose(a1, want1, rtol=1e-5, atol=1e-6)
        assert ((a1 == 0) | k1.reshape(B, 12)).all()
        a2 = t.debug_buffer(BUF_ACT, 2).reshape(B, 9)
        assert (a2[~k2.reshape(B, 9)] == 0).all()
    t.close()


def test_oracle_softmax_forward_closed_form(oracle):
    """Softmax as the hidden activation (:727-740): each row of act_1 is
    exp(pre - max) / sum, rows sum to 1, and the fp32 oracle agrees with the
    float64 closed form to fp32 rounding."""
    spec = MlpSpec([6, 9, 3], "softmax", "sgd")
    B = 5
    rng = np.random.default_rng(8)
    X = (rng.standard_normal((B, 6)) * 3).astype(np.float32)
    from volta_amd.abi import BUF_ACT
    ws = [rng.uniform(-0.8, 0.8, (r, c)).astype(np.float32) for r, c in spec.shapes()]
    bs = [rng.uniform(-0.3, 0.3, c).astype(np.float32) for _, c in spec.shapes()]
    # (the debug buffer hands out float32 copies, so the twin is compared to
    # float32 rounding too)
    for f64, rtol in ((True, 1.2e-7), (False, 1e-6)):
        t = oracle_trainer(oracle, spec, B, f64=f64)
        t.set_all_params(ws, bs)
        t.step(X, np.zeros((B, 3), np.float32), 0.0)
        pre = X.astype(np.float64) @ ws[0].astype(np.float64) + bs[0]
        e = np.exp(pre - pre.max(axis=1, keepdims=True))
        want = e / e.sum(axis=1, keepdims=True)
        got = t.debug_buffer(BUF_ACT, 1).reshape(B, 9)
        np.testing.assert_allclose(got, want, rtol=rtol, atol=1e-12)
        np.testing.assert_allclose(got.sum(axis=1), 1.0, atol=1e-6)
        t.close()


def test_oracle_layernorm_forward_closed_form(oracle):
    """With gamma = 1 and beta = 0 (init), each row of act_1 is the
    standardised relu(pre_0): mean 0 and variance v/(v + 1e-5)."""
    spec = MlpSpec([6, 32, 3], "relu", "sgd", layernorm=True)
    B = 5
    t = oracle_trainer(oracle, spec, B, f64=True)
    rng = np.random.default_rng(4)
    X = rng.standard_normal((B, 6)).astype(np.float32)
    t.step(X, np.zeros((B, 3), np.float32), 0.0)
    from volta_amd.abi import BUF_ACT
    ws, bs = t.get_params()
    h = np.maximum(X.astype(np.float64) @ ws[0].astype(np.float64) + bs[0], 0)
    mu = h.mean(axis=1, keepdims=True)
    var = ((h - mu) ** 2).mean(axis=1, keepdims=True)
    want = (h - mu) / np.sqrt(var + np.float64(np.float32(1e-5)))
    np.testing.assert_allclose(t.debug_buffer(BUF_ACT, 1).reshape(B, 32), want, rtol=1e-6, atol=1e-6)
    t.close()


@pytest.mark.parametrize("act", ["relu", "gelu", "silu"])
def test_f64_layernorm_gradient_matches_finite_differences(oracle, act):
    """dW through the LayerNorm backward equals the finite-difference
    gradient of the fp64 twin's loss (derivatives that use the
    pre-activation; sigmoid/tanh with LayerNorm use the reference's own
    post-LayerNorm derivative, :908-914, which is not the true gradient)."""
    spec = MlpSpec([4, 7, 6, 2], act, "sgd", layernorm=True)
    B = 3
    rng = np.random.default_rng(12)
    ws = [rng.uniform(-0.6, 0.6, (r, c)).astype(np.float32) for r, c in spec.shapes()]
    bs = [rng.uniform(-0.2, 0.2, c).astype(np.float32) for _, c in spec.shapes()]
    X = rng.standard_normal((B, 4)).astype(np.float32)
    Y = rng.standard_normal((B, 2)).astype(np.float32)
    lr = 1e-3

    def loss_at(wsx):
        t = oracle_trainer(oracle, spec, B, f64=True)
        t.set_all_params(wsx, bs)
        t.step(X, Y, 0.0)
        v = float(oracle.lib.volta_oracle_loss_f64(t.h))
        t.close()
        return v

    t = oracle_trainer(oracle, spec, B, f64=True)
    t.set_all_params(ws, bs)
    t.step(X, Y, lr)
    w_after, _ = t.get_params()
    t.close()
    for li in range(3):
        grad = (ws[li].astype(np.float64) - w_after[li].astype(np.float64)) / lr
        for (a, b) in [(0, 0), (ws[li].shape[0] - 1, ws[li].shape[1] - 1), (1, 1)]:
            h = 1e-3
            wp = [w.copy() for w in ws]
            wm = [w.copy() for w in ws]
            wp[li][a, b] += h
            wm[li][a, b] -= h
            fd = (loss_at(wp) - loss_at(wm)) / (2 * (np.float64(wp[li][a, b]) - np.float64(ws[li][a, b])))
            assert abs(fd - grad[a, b]) <= 2e-3 * max(1.0, abs(fd)), (li, a, b, fd, grad[a, b])


def _buf64(oracle, t, kind, layer, n):
    out = np.zeros(n, np.float64)
    got = oracle.lib.volta_oracle_debug_buffer_f64(t.h, kind, layer, out.ctypes.data_as(C.POINTER(C.c_double)))
    assert got == n, (kind, layer, got)
    return out


def _textbook_layernorm(a):
    """Per-row standardisation with eps 1e-5 (gamma 1, beta 0): x-hat and
    1/sigma."""
    mu = a.mean(axis=1, keepdims=True)
    var = ((a - mu) ** 2).mean(axis=1, keepdims=True)
    inv = 1.0 / np.sqrt(var + np.float64(np.float32(1e-5)))
    return (a - mu) * inv, inv


@pytest.mark.parametrize("act", ["sigmoid", "tanh"])
def test_f64_sigmoid_tanh_layernorm_derivative_at_the_layernorm_output(oracle, act):
    """Sigmoid/tanh followed by LayerNorm (mlp_train_rust_codegen.rs:908-914):
    the reference multiplies the LayerNorm backward by the activation's
    derivative written in its output -- y(1 - y), 1 - y^2 -- evaluated at the
    LayerNorm output y, not at the activation's own output.  With one hidden
    layer, no dropout and B = 1 its LayerNorm backward is the textbook one, so
    the hidden delta must equal the true gradient with respect to the
    pre-activation (central differences of the fp64 twin's loss over b_0)
    times g(y_j) / f'(z_j), unit by unit -- z the pre-activation, y the
    textbook LayerNorm of f(z).  The true derivative would fail: the ratio
    is far from 1 here."""
    spec = MlpSpec([4, 6, 2], act, "sgd", layernorm=True)
    rng = np.random.default_rng(31)
    ws = [rng.uniform(-0.9, 0.9, (r, c)).astype(np.float32) for r, c in spec.shapes()]
    bs = [rng.uniform(-0.3, 0.3, c).astype(np.float32) for _, c in spec.shapes()]
    X = rng.standard_normal((1, 4)).astype(np.float32)
    Y = rng.standard_normal((1, 2)).astype(np.float32)

    def loss_at(b0):
        t = oracle_trainer(oracle, spec, 1, f64=True)
        t.set_all_params(ws, [b0] + bs[1:])
        t.step(X, Y, 0.0)
        v = float(oracle.lib.volta_oracle_loss_f64(t.h))
        t.close()
        return v

    t = oracle_trainer(oracle, spec, 1, f64=True)
    t.set_all_params(ws, bs)
    t.step(X, Y, 0.0)
    delta = _buf64(oracle, t, BUF_DELTA, 0, 6)
    t.close()
    z = (X.astype(np.float64) @ ws[0].astype(np.float64) + bs[0])[0]
    a = 1.0 / (1.0 + np.exp(-z)) if act == "sigmoid" else np.tanh(z)
    fprime = a * (1.0 - a) if act == "sigmoid" else 1.0 - a * a
    y = _textbook_layernorm(a[None, :])[0][0]
    g = y * (1.0 - y) if act == "sigmoid" else 1.0 - y * y
    assert np.abs(g / fprime - 1.0).max() > 0.1
    for j in range(6):
        bp, bm = bs[0].copy(), bs[0].copy()
        bp[j] += np.float32(1e-4)
        bm[j] -= np.float32(1e-4)
        fd = (loss_at(bp) - loss_at(bm)) / (np.float64(bp[j]) - np.float64(bm[j]))
        want = fd * g[j] / fprime[j]
        assert abs(delta[j] - want) <= 1e-5 * abs(want) + 1e-9, (j, delta[j], want, fd)


def test_f64_layernorm_then_dropout_backward(oracle):
    """LayerNorm followed by dropout (:742-790 forward, :829-880 backward):
    the reference runs the LayerNorm backward on the gradient with respect
    to the dropout output g, with x-hat recomputed from the stored output
    after dropout d = s * mask * x-hat (s = 1/(1-p)), then applies the mask,
    then ReLU's derivative; dgamma = g * d and dbeta = g.  Pinned with one
    hidden layer and B = 1 against quantities fixed independently: the mask
    (the LCG written out with Python integers), the textbook LayerNorm
    forward, and g itself -- for a kept unit g = u / s with u the true
    gradient over beta (central differences of the fp64 twin's loss, which is
    quadratic in beta, so they are exact), and each dropped unit's outgoing
    weights are set to a kept unit's so its g is that unit's.  The textbook
    order (mask first, x-hat from the LayerNorm output) gives another delta
    here."""
    H, p = 8, 0.3
    spec = MlpSpec([4, H, 2], "relu", "sgd", layernorm=True, dropout_p=p)
    keep, _ = _lcg_keep(H, p)  # B = 1: the first step's mask of the hidden layer
    kept, dropped = np.flatnonzero(keep), np.flatnonzero(~keep)
    assert kept.size and dropped.size
    rng = np.random.default_rng(41)
    ws = [rng.uniform(-0.8, 0.8, (r, c)).astype(np.float32) for r, c in spec.shapes()]
    bs = [rng.uniform(-0.2, 0.4, c).astype(np.float32) for _, c in spec.shapes()]
    partner = {int(j): int(kept[i % kept.size]) for i, j in enumerate(dropped)}
    for j, k in partner.items():
        ws[1][j] = ws[1][k]
    X = rng.standard_normal((1, 4)).astype(np.float32)
    Y = rng.standard_normal((1, 2)).astype(np.float32)
    s = np.float64(np.float32(1.0) / (np.float32(1.0) - np.float32(p)))  # the reference's f32 literal

    def run(beta, lr):
        t = oracle_trainer(oracle, spec, 1, f64=True)
        t.set_all_params(ws, bs)
        t.set_state(np.concatenate([np.ones(H, np.float32), beta.astype(np.float32)]), 0)
        t.set_dropout_rng(12345678)
        t.step(X, Y, lr)
        return t

    u = np.zeros(H)
    for j in range(H):
        bp, bm = np.zeros(H, np.float32), np.zeros(H, np.float32)
        bp[j], bm[j] = np.float32(1e-2), np.float32(-1e-2)
        lv = []
        for beta in (bp, bm):
            t = run(beta, 0.0)
            lv.append(float(oracle.lib.volta_oracle_loss_f64(t.h)))
            t.close()
        u[j] = (lv[0] - lv[1]) / (np.float64(bp[j]) - np.float64(bm[j]))
    assert np.abs(u[dropped]).max() < 1e-12  # a dropped unit does not reach the loss
    g = np.zeros(H)
    g[kept] = u[kept] / s
    for j, k in partner.items():
        g[j] = g[k]
    z = (X.astype(np.float64) @ ws[0].astype(np.float64) + bs[0])[0]
    xhat, inv = _textbook_layernorm(np.maximum(z, 0.0)[None, :])
    xhat, inv = xhat[0], float(inv[0, 0])
    d = s * keep * xhat
    want = keep * s * inv * (g - g.mean() - d * (g * d).mean()) * (z > 0)
    t = run(np.zeros(H, np.float32), 1.0)
    np.testing.assert_array_equal(_buf64(oracle, t, BUF_DROPOUT_MASK, 0, H), keep.astype(np.float64))
    delta = _buf64(oracle, t, BUF_DELTA, 0, H)
    dgamma = 1.0 - _buf64(oracle, t, BUF_LN_GAMMA, 0, H)
    dbeta = -_buf64(oracle, t, BUF_LN_BETA, 0, H)
    t.close()
    np.testing.assert_allclose(delta, want, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(dbeta, g, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(dgamma, g * d, rtol=1e-9, atol=1e-12)
    textbook = keep * inv * ((s * keep * g) - (s * keep * g).mean() - xhat * (s * keep * g * xhat).mean()) * (z > 0)
    assert np.abs(textbook - want).max() > 1e-3 * np.abs(want).max()


def test_oracle_clip_scales_dw_but_not_db(oracle):
    """With clipping the weight step shrinks by clip/||deltas|| (norm over
    every layer's deltas) while the bias step keeps the unscaled deltas
    (db is formed before the clip, :931-955)."""
    base = MlpSpec([6, 10, 8, 3], "tanh", "sgd")
    B = 4
    rng = np.random.default_rng(21)
    ws = [rng.uniform(-0.5, 0.5, (r, c)).astype(np.float32) for r, c in base.shapes()]
    bs = [rng.uniform(-0.1, 0.1, c).astype(np.float32) for _, c in base.shapes()]
    X = rng.standard_normal((B, 6)).astype(np.float32)
    Y = rng.standard_normal((B, 3)).astype(np.float32)
    from volta_amd.abi import BUF_DELTA
    out = {}

    def run(name, spec):
        t = oracle_trainer(oracle, spec, B, f64=True)
        t.set_all_params(ws, bs)
        t.step(X, Y, 0.5)
        out[name] = t.get_params() + ([t.debug_buffer(BUF_DELTA, i) for i in range(3)],)
        t.close()

    run("base", base)
    deltas = out["base"][2]
    gnorm = np.sqrt(sum(float((d.astype(np.float64) ** 2).sum()) for d in deltas))
    clip_val = float(np.float32(0.4 * gnorm))
    run("clip", MlpSpec([6, 10, 8, 3], "tanh", "sgd", clip_grad=clip_val))
    scale = clip_val / gnorm
    assert scale < 1
    for i in range(3):
        dw_base = ws[i].astype(np.float64) - out["base"][0][i]
        dw_clip = ws[i].astype(np.float64) - out["clip"][0][i]
        # weights come back as float32: allow their rounding
        np.testing.assert_allclose(dw_clip, dw_base * scale, rtol=1e-4, atol=2e-7)
        np.testing.assert_array_equal(out["clip"][1][i], out["base"][1][i])  # bias step unscaled


def test_division_by_a_constant_through_double_is_the_fp32_quotient():
    """The GPU's Adam divides m/bc1 and v/bc2 as float(double(x) * (1/double(c)))
    (device_common.h div_by_const).  That equals IEEE fp32 division x/c for
    every fp32 x, c: the exact quotient is never an fp32 midpoint and is at
    least 2^-49 (relative) away from one, the double product within ~2^-52.
    Checked here on 4M pairs over the whole exponent range (subnormals,
    zeros, infinities, overflow) and on the bias corrections the step uses."""
    rng = np.random.default_rng(1234)
    n = 1 << 22
    bits = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    c = np.abs(rng.standard_normal(x.size).astype(np.float32) * np.float32(2.0) ** rng.integers(-30, 30, x.size)
               .astype(np.float32)).astype(np.float32)
    c[c == 0] = np.float32(1)
    corr = []
    for b in (0.9, 0.999, 0.5, 0.95, 0.99):
        for t in list(range(1, 300)) + [1000, 5000, 17000, 20000]:
            corr.append(np.float32(1) - np.float32(b) ** np.float32(t))
    corr = np.array([v for v in corr if v > 0], np.float32)
    c[: corr.size * 64] = np.repeat(corr, 64)[: min(corr.size * 64, c.size)]
    x = np.concatenate([x, np.float32([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, 3.4e38, -3.4e38])])
    c = np.concatenate([c, np.float32([0.1, 0.1, 0.1, 0.1, 0.1, 0.1, 0.1, 0.1])])
    with np.errstate(over="ignore", under="ignore", invalid="ignore"):
        want = x / c
        got = (x.astype(np.float64) * (1.0 / c.astype(np.float64))).astype(np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("hidden_act", [0, -1], ids=["relu", "linear"])
def test_oracle_inference_model_graph(oracle, hidden_act):
    """volta_infer_model_create (the `volta compile` library's model): the
    graph of lower_model_to_graph (lowering.rs:87-140) -- x W_i + b_i per
    layer, ReLU after each hidden layer (hidden_act VOLTA_ACT_RELU = 0) or
    nothing (-1) -- on the embedded [W_0|b_0|W_1|b_1|...] parameters.
    Against the float64 numpy forward within the fp32 summation bound
    2(K+1) eps |x||W| + |b| per layer (with the bound carried through the
    later layers), and a ReLU model differs from the linear one."""
    sizes = [24, 40, 33, 5]
    rng = np.random.default_rng(8)
    ws = [rng.standard_normal((sizes[i], sizes[i + 1])).astype(np.float32) / 4 for i in range(3)]
    bs = [rng.standard_normal(sizes[i + 1]).astype(np.float32) for i in range(3)]
    blob = np.concatenate([np.concatenate([w.ravel(), b]) for w, b in zip(ws, bs)]).astype(np.float32)
    arr = (C.c_int32 * 4)(*sizes)
    F = C.POINTER(C.c_float)
    h = oracle.lib.volta_infer_model_create(4, arr, hidden_act, blob.ctypes.data_as(F))
    assert h
    rows = 70  # more rows than the model's 64-row chunk
    X = rng.standard_normal((rows, sizes[0])).astype(np.float32)
    out = np.zeros((rows, sizes[-1]), np.float32)
    assert oracle.lib.volta_train_infer(h, X.ctypes.data_as(F), rows, out.ctypes.data_as(F)) == 0
    oracle.lib.volta_train_free(h)
    eps = 2.0 ** -24
    a = X.astype(np.float64)
    err = np.zeros_like(a)
    for i in range(3):
        W = ws[i].astype(np.float64)
        z = a @ W + bs[i]
        err = err @ np.abs(W) + 2 * (sizes[i] + 1) * eps * (np.abs(a) @ np.abs(W) + np.abs(bs[i]))
        if i < 2 and hidden_act == 0:
            z = np.maximum(z, 0.0)
        a = z
    assert np.all(np.abs(out - a) <= err * (1 + 1e-6) + 1e-30)
    # the two graphs differ (the ReLU is applied or not)
    relu_differs = np.any(np.maximum(X.astype(np.float64) @ ws[0] + bs[0], 0) != X.astype(np.float64) @ ws[0] + bs[0])
    assert relu_differs
    assert oracle.lib.volta_infer_model_create(4, arr, 3, blob.ctypes.data_as(F)) is None  # tanh: refused
