"""The oracle's restatement of Volta's runtime optimizer (oracle/rt_optimizer.cpp,
following src/engine/ir/optimizer.rs) pinned by the reference's own tests of
that file (optimizer.rs:676-1045) and by closed forms.  CPU only."""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import pytest

from tests.oracle_lib import load_oracle
from volta_amd.backend import OptimizerError, RtOptimizer, capabilities, config

F32 = np.float32


def _lib():
    lib = load_oracle().lib
    lib.volta_oracle_powi.restype = C.c_float
    lib.volta_oracle_powi.argtypes = [C.c_float, C.c_int32]
    return lib


class Host:
    """Host tensors driven through the oracle's volta_rt_* ABI."""

    def __init__(self, params, grads):
        self.p = [np.ascontiguousarray(p, F32) for p in params]
        self.g = [None if g is None else np.ascontiguousarray(g, F32) for g in grads]
        self.opt = RtOptimizer(_lib(), [p.size for p in self.p])

    def apply(self, cfg):
        self.opt.apply(cfg, [p.ctypes.data for p in self.p], [None if g is None else g.ctypes.data for g in self.g])


# --- the reference's tests (optimizer.rs:676-1045) ---------------------------
def test_sgd_updates_parameter_values():  # :677-703
    h = Host([[1.0]], [[0.5]])
    h.apply(config("sgd", 0.1))
    assert abs(h.p[0][0] - 0.95) < 1e-6


@pytest.mark.parametrize("bad_lr", [0.0, -0.01, float("nan"), float("inf")])
def test_sgd_rejects_non_positive_learning_rate(bad_lr):  # :706-733
    h = Host([[1.0]], [[1.0]])
    with pytest.raises(OptimizerError, match="learning rate"):
        h.apply(config("sgd", bad_lr))


def test_adam_rejects_beta_equal_to_one():  # :736-766
    h = Host([[1.0]], [[1.0]])
    with pytest.raises(OptimizerError, match="beta1"):
        h.apply(config("adam", 0.001, beta1=1.0))


def test_adagrad_reduces_loss_over_steps():  # :769-795
    h = Host([[1.0, -1.0]], [[0.5, -0.5]])
    prev = 1.0
    for _ in range(3):
        h.apply(config("adagrad", 0.1, epsilon=1e-8))
        assert h.p[0][0] < prev
        prev = h.p[0][0]


def test_adam_rejects_non_positive_epsilon():  # :798-828
    h = Host([[1.0]], [[1.0]])
    with pytest.raises(OptimizerError, match="epsilon"):
        h.apply(config("adam", 0.001, epsilon=0.0))


def test_adam_updates_parameter_numerically_correct():  # :831-862
    h = Host([[0.5]], [[0.1]])
    h.apply(config("adam", 0.001))
    assert abs(h.p[0][0] - 0.499) < 1e-5


@pytest.mark.parametrize("kw,word", [({"beta1": 1.0}, "beta1"), ({"epsilon": 0.0}, "epsilon"),
                                     ({"weight_decay": -0.01}, "weight_decay")])
def test_adamw_rejects_invalid_hyperparameters(kw, word):  # :865-922
    h = Host([[1.0]], [[1.0]])
    args = dict(weight_decay=0.01)
    args.update(kw)
    with pytest.raises(OptimizerError, match=word):
        h.apply(config("adamw", 0.001, **args))


@pytest.mark.parametrize("kw,word", [({"alpha": 1.0}, "alpha"), ({"epsilon": 0.0}, "epsilon")])
def test_rmsprop_rejects_invalid_hyperparameters(kw, word):  # :925-967
    h = Host([[1.0]], [[1.0]])
    with pytest.raises(OptimizerError, match=word):
        h.apply(config("rmsprop", 0.01, **kw))


@pytest.mark.parametrize("kw,word", [({"epsilon": 0.0}, "epsilon"), ({"weight_decay": -0.01}, "weight_decay")])
def test_adagrad_rejects_invalid_hyperparameters(kw, word):  # :970-1008
    h = Host([[1.0]], [[1.0]])
    with pytest.raises(OptimizerError, match=word):
        h.apply(config("adagrad", 0.1, **kw))


def test_three_sgd_steps_and_step_counter():  # :1011-1045
    h = Host([[1.0]], [[0.5]])
    for _ in range(3):
        h.apply(config("sgd", 0.1))
    assert h.opt.step == 3
    assert abs(h.p[0][0] - 0.85) < 1e-6


# --- semantics the reference fixes beyond its tests --------------------------
def test_step_advances_before_validation():
    """apply_gradients increments the step first (optimizer.rs:114), so a
    rejected configuration still counts."""
    h = Host([[1.0]], [[1.0]])
    with pytest.raises(OptimizerError):
        h.apply(config("adam", 0.001, beta2=1.5))
    assert h.opt.step == 1
    assert h.p[0][0] == 1.0


def test_rust_style_messages():
    h = Host([[1.0]], [[1.0]])
    for lr, text in ((float("nan"), "got NaN"), (float("inf"), "got inf"), (-0.01, "got -0.01")):
        with pytest.raises(OptimizerError) as e:
            h.apply(config("sgd", lr))
        assert str(e.value) == "SGD learning rate must be a finite positive number, " + text


def test_parameters_without_gradient_are_skipped():
    h = Host([[1.0, 2.0], [3.0]], [None, [0.5]])
    h.apply(config("adam", 0.01))
    np.testing.assert_array_equal(h.p[0], [1.0, 2.0])
    assert h.opt.state("adam_m", 0) is None
    assert h.opt.state("adam_m", 1) is not None


def test_state_entries_created_as_the_reference_creates_them():
    h = Host([[1.0]], [[0.5]])
    h.apply(config("rmsprop", 0.01, momentum=0.0))
    assert h.opt.state("rms_v", 0) is not None and h.opt.state("rms_buf", 0) is None
    h.apply(config("rmsprop", 0.01, momentum=0.9))
    assert h.opt.state("rms_buf", 0) is not None
    assert h.opt.state("adagrad_acc", 0) is None and h.opt.state("lars_vel", 0) is None


def test_adam_and_adamw_share_moments():
    """AdamW reads the m/v entries Adam wrote (both use adam_m/adam_v)."""
    h = Host([[1.0]], [[0.5]])
    h.apply(config("adam", 0.01))
    m1 = h.opt.state("adam_m", 0)[0]
    h.apply(config("adamw", 0.01, weight_decay=0.0))
    assert h.opt.state("adam_m", 0)[0] == F32(F32(0.9) * m1 + F32(1 - F32(0.9)) * F32(0.5))


# --- powi (compiler-rt square-and-multiply) ------------------------------------
def test_powi_square_and_multiply():
    lib = _lib()
    b = F32(0.9)
    assert lib.volta_oracle_powi(b, 1) == b
    assert lib.volta_oracle_powi(b, 2) == F32(b * b)
    b2 = F32(b * b)
    b4 = F32(b2 * b2)
    assert lib.volta_oracle_powi(b, 5) == F32(b * b4)          # e=5: r=b, a=b^2, a=b^4, r=b*b^4
    assert lib.volta_oracle_powi(b, 6) == F32(b2 * b4)         # e=6: a=b^2, r=b^2, a=b^4, r=b^2*b^4
    assert lib.volta_oracle_powi(2.0, 10) == 1024.0
    assert lib.volta_oracle_powi(0.5, -2) == 4.0
    assert lib.volta_oracle_powi(0.999, 0) == 1.0


def test_adam_moments_after_three_steps():
    """With a constant gradient m_t = (1 - b1^t) g and v_t = (1 - b2^t) g^2
    (b1, b2 the f32 values of 0.9 and 0.999; 1 - b is exact in f32)."""
    g = 0.25
    b1, b2 = float(F32(0.9)), float(F32(0.999))
    h = Host([[1.0]], [[g]])
    for _ in range(3):
        h.apply(config("adam", 0.001))
    assert math.isclose(h.opt.state("adam_m", 0)[0], (1 - b1 ** 3) * g, rel_tol=1e-6)
    assert math.isclose(h.opt.state("adam_v", 0)[0], (1 - b2 ** 3) * g * g, rel_tol=1e-6)


# --- closed forms ---------------------------------------------------------------
@pytest.mark.parametrize("g", [0.1, -2.5, 1e-3])
def test_adam_step_one_closed_form(g):
    """m_hat = g and v_hat = g^2 at step 1, so p -= lr*g/(|g|+eps)."""
    p0, lr, eps = 0.75, 0.01, 1e-8
    h = Host([[p0]], [[g]])
    h.apply(config("adam", lr, epsilon=eps))
    want = p0 - lr * g / (abs(g) + eps)
    assert abs(h.p[0][0] - want) <= 2 * np.spacing(F32(p0))


def test_adamw_step_one_closed_form():
    p0, g, lr, wd = 2.0, 0.3, 0.01, 0.1
    h = Host([[p0]], [[g]])
    h.apply(config("adamw", lr, weight_decay=wd))
    want = p0 - lr * (g / (abs(g) + 1e-8) + wd * p0)
    assert abs(h.p[0][0] - want) <= 2 * np.spacing(F32(p0))


def test_adagrad_constant_gradient_closed_form():
    """acc_k = k g^2, so p_n = p0 - lr*g*sum_k 1/(sqrt(k)|g| + eps)."""
    p0, g, lr, eps, n = 1.0, 0.2, 0.05, 1e-8, 6
    h = Host([[p0]], [[g]])
    for _ in range(n):
        h.apply(config("adagrad", lr, epsilon=eps))
    want = p0 - lr * g * sum(1.0 / (math.sqrt(k) * abs(g) + eps) for k in range(1, n + 1))
    assert math.isclose(h.p[0][0], want, rel_tol=1e-6)


def test_rmsprop_constant_gradient_closed_form():
    """v_k = (1 - alpha^k) g^2 without momentum or decay."""
    p0, g, lr, al, eps, n = 1.0, -0.4, 0.01, 0.9, 1e-8, 5
    h = Host([[p0]], [[g]])
    for _ in range(n):
        h.apply(config("rmsprop", lr, alpha=al, epsilon=eps))
    want = p0 - lr * g * sum(1.0 / (math.sqrt(1 - al ** k) * abs(g) + eps) for k in range(1, n + 1))
    assert math.isclose(h.p[0][0], want, rel_tol=1e-5)


def test_rmsprop_momentum_geometric_series():
    """alpha = 0 makes v_k = g^2, so buf_k = c(1 + mo + ... + mo^(k-1)) with
    c = lr*g/(|g|+eps) and p_n = p0 - c * sum_k (1 - mo^k)/(1 - mo)."""
    p0, g, lr, mo, eps, n = 0.5, 0.8, 0.02, 0.5, 1e-8, 4
    h = Host([[p0]], [[g]])
    for _ in range(n):
        h.apply(config("rmsprop", lr, alpha=0.0, epsilon=eps, momentum=mo))
    c = lr * g / (abs(g) + eps)
    want = p0 - c * sum((1 - mo ** k) / (1 - mo) for k in range(1, n + 1))
    assert math.isclose(h.p[0][0], want, rel_tol=1e-5)


def test_rmsprop_weight_decay_enters_the_gradient():
    """gwd = g + wd*p: with g = 0 the update is driven by wd*p alone."""
    p0, wd, lr = 2.0, 0.5, 0.01
    h = Host([[p0]], [[0.0]])
    h.apply(config("rmsprop", lr, alpha=0.0, weight_decay=wd))
    gwd = wd * p0
    assert math.isclose(h.p[0][0], p0 - lr * gwd / (abs(gwd) + 1e-8), rel_tol=1e-6)


def test_lars_local_rate_and_momentum():
    """p = (3, 4), g = (0.6, 0.8): |p| = 5, |g| = 1, so the local rate is
    lr*tc*5/(1 + 5wd + eps); velocity accumulates with momentum."""
    lr, tc, wd, mo, eps = 0.1, 0.01, 0.0, 0.9, 1e-8
    h = Host([[3.0, 4.0]], [[0.6, 0.8]])
    h.apply(config("lars", lr, weight_decay=wd, momentum=mo, trust_coeff=tc, epsilon=eps))
    local = lr * tc * 5.0 / (1.0 + eps)
    np.testing.assert_allclose(h.p[0], [3.0 - local * 0.6, 4.0 - local * 0.8], rtol=1e-6)
    np.testing.assert_allclose(h.opt.state("lars_vel", 0), [local * 0.6, local * 0.8], rtol=1e-6)


def test_lars_zero_norm_uses_base_rate():
    h = Host([[0.0, 0.0]], [[1.0, -2.0]])
    h.apply(config("lars", 0.1, momentum=0.0))
    np.testing.assert_allclose(h.p[0], [-0.1, 0.2], rtol=1e-6)


def test_oracle_capabilities_are_the_cpu_backend():
    caps = capabilities(_lib())
    assert caps["backend"] == 0 and caps["device_class"] == 0 and caps["supports_adam"] == 1
