"""The gradient-level checker (tests/grad_check.py) on the CPU: the fp32
oracle as the candidate against its fp64 twin passes at small config-like
shapes, and mistakes planted in the candidate's buffers -- a gradient off
by 10% in magnitude, a dropped bias term, a transposed operand, a wrong
loss scale, an optimizer step with a perturbed learning rate -- fail it."""
import numpy as np
import pytest

from tests import grad_check as gc
from tests.oracle_lib import load_oracle
from tests.test_oracle import oracle_trainer
from volta_amd import data
from volta_amd.abi import MlpSpec, Trainer

CASES = {
    "relu_adam_mse": (MlpSpec([96, 128, 64, 1], "relu", "adam"), 32, 1e-3),
    "gelu_adamw_mse": (MlpSpec([64, 96, 96, 1], "gelu", "adamw"), 16, 1e-3),
    "relu_adagrad_ce": (MlpSpec([64, 128, 10], "relu", "adagrad", "ce", eps=1e-10), 48, 1e-2),
}


def _one_step(name, steps_before=3):
    spec, B, lr = CASES[name]
    orc = load_oracle()
    ws, bs = data.he_uniform(3, spec.sizes)
    X, Y = data.batch(3, spec.sizes, B, spec.loss)
    to = Trainer(orc, spec, B)
    to.set_all_params(ws, bs)
    for _ in range(steps_before):
        to.step(X, Y, lr)
    W0, b0 = to.get_params()
    st0, t0 = to.get_state()
    tt = oracle_trainer(orc, spec, B, f64=True)
    tt.set_all_params(W0, b0)
    tt.set_state(st0, t0)
    to.step(X, Y, lr)
    tt.step(X, Y, lr)
    cand = gc.read_candidate(to, spec, B)
    twin = gc.read_twin(orc, tt, spec, B)
    W1, b1 = to.get_params()
    st1, t1 = to.get_state()
    to.close()
    tt.close()
    return spec, B, lr, X, Y, W0, b0, st0, t0, cand, twin, W1, b1, st1, t1


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_fp32_passes_checker(name):
    spec, B, lr, X, Y, W0, b0, st0, t0, cand, twin, W1, b1, st1, t1 = _one_step(name)
    rep = gc.check_step(load_oracle(), spec, B, X, Y, W0, b0, cand, twin, name)
    assert not rep.failures, "\n".join(rep.failures) + "\n" + rep.summary()
    if spec.optimizer in ("adam", "adamw"):
        assert t1 == t0 + 1  # the Adam step counter (Adagrad keeps none)
    We, be, ste = gc.expected_update(load_oracle(), spec, lr, t1, W0, b0, st0, cand.dw, cand.db)
    for i in range(spec.n_layers):
        assert gc.bits_equal(We[i], W1[i]) and gc.bits_equal(be[i], b1[i]), f"layer {i}"
    assert gc.bits_equal(ste, st1)


def _fails(name, mutate):
    spec, B, lr, X, Y, W0, b0, st0, t0, cand, twin, *_ = _one_step(name)
    mutate(spec, cand)
    rep = gc.check_step(load_oracle(), spec, B, X, Y, W0, b0, cand, twin, name)
    return rep.failures


@pytest.mark.parametrize("name", sorted(CASES))
def test_checker_sees_gradient_magnitude_error(name):
    def m(spec, cand):
        cand.dw[0] = cand.dw[0] * 1.1
    assert any("dw0" in f for f in _fails(name, m))


@pytest.mark.parametrize("name", sorted(CASES))
def test_checker_sees_delta_magnitude_error(name):
    def m(spec, cand):
        cand.delta[0] = cand.delta[0] * 0.9
    f = _fails(name, m)
    assert any("dx1" in x for x in f) and any("dw0" in x for x in f)


def test_checker_sees_dropped_bias_term():
    def m(spec, cand):
        cand.db[1] = cand.db[1] - cand.delta[1][0]  # one batch row left out of the sum
    assert any("db1" in f for f in _fails("relu_adam_mse", m))


def test_checker_sees_transposed_operand():
    def m(spec, cand):
        w = cand.dw[1]
        k = min(w.shape)
        w[:k, :k] = w[:k, :k].T.copy()
    assert any("dw1" in f for f in _fails("gelu_adamw_mse", m))


@pytest.mark.parametrize("name", ["relu_adam_mse", "relu_adagrad_ce"])
def test_checker_sees_wrong_loss_scale(name):
    def m(spec, cand):
        cand.delta[spec.n_layers - 1] = cand.delta[spec.n_layers - 1] * 2.0
    assert any("loss grad" in f for f in _fails(name, m))


def test_checker_sees_wrong_forward():
    def m(spec, cand):
        cand.act[1] = cand.act[1] * 1.01
    assert any("fwd0" in f for f in _fails("relu_adam_mse", m))


@pytest.mark.parametrize("name", sorted(CASES))
def test_expected_update_sees_perturbed_lr(name):
    spec, B, lr, X, Y, W0, b0, st0, t0, cand, twin, W1, b1, st1, t1 = _one_step(name)
    We, be, ste = gc.expected_update(load_oracle(), spec, lr * (1 + 1e-3), t1, W0, b0, st0, cand.dw, cand.db)
    assert not all(gc.bits_equal(We[i], W1[i]) for i in range(spec.n_layers))
