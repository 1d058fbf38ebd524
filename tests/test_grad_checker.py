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


# ---------------------------------------------------------------------------
# The extras checker (check_step_ext / expected_update_ext): the fp32 oracle
# as the candidate passes, and mistakes in the wiring only the extras path
# uses fail it -- the bias updated from the clipped deltas, dW from the
# unclipped ones, a wrong clip scale, a LayerNorm gradient or a hidden delta
# off in magnitude, gamma's SGD step with another learning rate.
# ---------------------------------------------------------------------------

EXT_CASES = {
    "clip_relu_adam": (MlpSpec([32, 96, 80, 24], "relu", "adam", clip_grad=-1.0), 64, 1e-3),
    "all_tanh_adamw_ce": (MlpSpec([64, 200, 120, 30], "tanh", "adamw", "ce", layernorm=True, dropout_p=0.15,
                                  clip_grad=-1.0), 96, 1e-3),
    "drop_leaky_adagrad": (MlpSpec([24, 130, 70, 100], "leaky_relu", "adagrad", dropout_p=0.5), 48, 1e-2),
    "softmax_all_adam": (MlpSpec([32, 96, 12], "softmax", "adam", layernorm=True, dropout_p=0.1, clip_grad=-1.0),
                         64, 1e-3),
}


def _ext_step(name, steps_before=3):
    from tests.test_gpu_extras import resolve
    from tests.test_gpu_extras_grad import ln_from_state

    spec, B, lr = EXT_CASES[name]
    spec = resolve(spec, B, 11)
    orc = load_oracle()
    ws, bs = data.he_uniform(11, spec.sizes)
    batches = [data.batch(11 + j, spec.sizes, B, spec.loss) for j in range(2)]
    to = Trainer(orc, spec, B)
    to.set_all_params(ws, bs)
    for s in range(steps_before):
        to.step(*batches[s % 2], lr)
    X, Y = batches[steps_before % 2]
    W0, b0 = to.get_params()
    st0, t0 = to.get_state()
    rng0 = to.get_dropout_rng()
    g0, be0 = ln_from_state(spec, st0)
    tt = oracle_trainer(orc, spec, B, f64=True)
    tt.set_all_params(W0, b0)
    tt.set_state(st0, t0)
    tt.set_dropout_rng(rng0)
    to.step(X, Y, lr)
    tt.step(X, Y, lr)
    cand = gc.read_candidate_ext(to, spec, B)
    twin = gc.read_twin_ext(orc, tt, spec, B)
    W1, b1 = to.get_params()
    st1, t1 = to.get_state()
    to.close()
    tt.close()
    return dict(spec=spec, B=B, lr=lr, X=X, Y=Y, W0=W0, b0=b0, st0=st0, t0=t0, g0=g0, be0=be0, cand=cand,
                twin=twin, W1=W1, b1=b1, st1=st1, t1=t1)


def _ext_check(r, cand=None):
    import copy

    spec, B = r["spec"], r["B"]
    yard = r["cand"]
    cand = cand if cand is not None else copy.deepcopy(yard)
    # the oracle sums the clip's squares sequentially over every delta
    terms = B * sum(spec.sizes[1:])
    return gc.check_step_ext(load_oracle(), spec, B, r["X"], r["Y"], r["W0"], r["b0"], r["g0"], r["be0"], cand,
                             r["twin"], yard, "ext", clip_terms=terms)


def _ext_update(r, lr=None, db=None, dg=None):
    spec, cand = r["spec"], r["cand"]
    t_next = r["t0"] + 1 if spec.optimizer in ("adam", "adamw") else r["t0"]
    return gc.expected_update_ext(load_oracle(), spec, r["lr"] if lr is None else lr, t_next, r["W0"], r["b0"],
                                  r["st0"], cand.dw, cand.db if db is None else db, r["g0"], r["be0"],
                                  cand.dg if dg is None else dg, cand.dbe)


def _ext_bits_equal(r, upd):
    We, be, ste = upd
    n = r["spec"].n_layers
    return all(gc.bits_equal(We[i], r["W1"][i]) and gc.bits_equal(be[i], r["b1"][i]) for i in range(n)) and \
        gc.bits_equal(ste, r["st1"])


@pytest.mark.parametrize("name", sorted(EXT_CASES))
def test_oracle_fp32_passes_extras_checker(name):
    r = _ext_step(name)
    rep = _ext_check(r)
    assert not rep.failures, "\n".join(rep.failures) + "\n" + rep.summary()
    assert _ext_bits_equal(r, _ext_update(r))


def test_extras_checker_without_stored_pre_activation():
    """The HIP library keeps no pre-activation for ReLU with clipping only
    (the derivative comes from the output): the forward is then checked on
    the activation output; a 1% error there still fails."""
    import copy

    r = _ext_step("clip_relu_adam")
    cand = copy.deepcopy(r["cand"])
    cand.pre = [None] * len(cand.pre)
    rep = _ext_check(r, cand)
    assert not rep.failures, "\n".join(rep.failures)
    assert any(name.startswith("fwd0 vs fp64 (act)") for name, *_ in rep.rows)
    cand.act[1] = cand.act[1] * 1.01
    assert any("fwd0 vs fp64 (act)" in f for f in _ext_check(r, cand).failures)


def _ext_mutated(name, mutate):
    import copy

    r = _ext_step(name)
    cand = copy.deepcopy(r["cand"])
    mutate(r["spec"], cand)
    return _ext_check(r, cand).failures


@pytest.mark.parametrize("name", ["clip_relu_adam", "all_tanh_adamw_ce", "softmax_all_adam"])
def test_extras_checker_sees_bias_gradient_from_clipped_deltas(name):
    r = _ext_step(name)
    assert r["cand"].scale < 1.0, "the case must clip on this step"
    import copy

    cand = copy.deepcopy(r["cand"])
    cand.db = [d * cand.scale for d in cand.db]
    assert any("db" in f for f in _ext_check(r, cand).failures)
    # and a bias updated from the clipped sums is not the candidate's update
    assert not _ext_bits_equal(r, _ext_update(r, db=[np.float32(d) * np.float32(r["cand"].scale)
                                                     for d in r["cand"].db]))


@pytest.mark.parametrize("name", ["clip_relu_adam", "all_tanh_adamw_ce"])
def test_extras_checker_sees_weight_gradient_from_unclipped_deltas(name):
    def m(spec, cand):
        cand.dw[0] = cand.dw[0] / cand.scale
    assert any("dw0" in f for f in _ext_mutated(name, m))


@pytest.mark.parametrize("name", ["clip_relu_adam", "softmax_all_adam"])
def test_extras_checker_sees_wrong_applied_clip_factor(name):
    # every delta, dW and the recorded factor scaled alike: only the norm of
    # the scaled deltas (clip, when the step clips) tells
    def m(spec, cand):
        cand.scale = cand.scale * 1.001
        cand.delta = [d * 1.001 for d in cand.delta]
        cand.dw = [d * 1.001 for d in cand.dw]
    assert any("clip scale" in f for f in _ext_mutated(name, m))


@pytest.mark.parametrize("name", ["clip_relu_adam", "softmax_all_adam"])
def test_extras_checker_sees_misrecorded_clip_scale(name):
    # the deltas scaled right but another factor recorded: the unscaled
    # deltas the checks rebuild (loss gradient, db) are off
    def m(spec, cand):
        cand.scale = cand.scale * 1.001
    f = _ext_mutated(name, m)
    assert any("loss grad" in x for x in f) and any("db" in x for x in f)


@pytest.mark.parametrize("name", ["all_tanh_adamw_ce", "softmax_all_adam"])
def test_extras_checker_sees_layernorm_gradient_magnitude_error(name):
    def mg(spec, cand):
        cand.dg[0] = cand.dg[0] * 1.01

    def mb(spec, cand):
        cand.dbe[0] = cand.dbe[0] * 1.01
    assert any("dgamma0" in f for f in _ext_mutated(name, mg))
    assert any("dbeta0" in f for f in _ext_mutated(name, mb))


@pytest.mark.parametrize("name", sorted(EXT_CASES))
def test_extras_checker_sees_hidden_delta_magnitude_error(name):
    def m(spec, cand):
        cand.delta[0] = cand.delta[0] * 0.999
    f = _ext_mutated(name, m)
    assert any("delta0" in x for x in f) and any("dw0" in x for x in f)


def test_extras_checker_sees_dropout_mask_error():
    def m(spec, cand):
        cand.mask[0] = cand.mask[0].copy()
        cand.mask[0][0, 0] = 1.0 - cand.mask[0][0, 0]
    assert any("dropout mask" in f for f in _ext_mutated("drop_leaky_adagrad", m))


@pytest.mark.parametrize("name", ["all_tanh_adamw_ce", "softmax_all_adam"])
def test_extras_expected_update_sees_layernorm_step(name):
    r = _ext_step(name)
    assert not _ext_bits_equal(r, _ext_update(r, dg=[d * np.float32(1.0001) for d in r["cand"].dg]))
    assert not _ext_bits_equal(r, _ext_update(r, lr=r["lr"] * (1 + 1e-3)))
