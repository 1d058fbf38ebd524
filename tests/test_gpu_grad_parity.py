"""Gradient-level parity of single HIP steps at the adaptive configurations'
shapes (C2 Adam, C3 AdamW, C5 Adagrad), teacher-forced from the fp32
oracle's exact state at points along its 50-step trajectory.

At each point one HIP step (VOLTA_KEEP_GRADS=1, so the fused dW kernels also
store the gradient they apply) and one fp64-twin step run from the same
parameters, optimizer state and step counter on the same batch; then
  * every product of the HIP step -- forward pre-activations and outputs, the
    loss gradient, every delta, every dW and db -- is within the elementwise
    bound of tests/grad_check.py, both on the HIP step's own operands (the
    fp32 summation bound 2 K eps |A||B|) and against the fp64 twin (that
    bound plus the measured deviation of the operands);
  * the HIP step's updated parameters and optimizer state equal, bit for bit,
    the oracle's fp32 optimizer (mlp_train_rust_codegen.rs:957-985) applied
    to the HIP step's own gradients from the same starting state.
Together these pin the step's gradients in magnitude, not only in sign (an
adaptive update lr*m^/sqrt(v^) is near +-lr whatever the gradient's size).
"""
import os
import sys

import numpy as np
import pytest

from tests import grad_check as gc
from tests.oracle_lib import load_oracle
from tests.test_gpu_parity import CONFIGS, config_inputs
from volta_amd import load_hip
from volta_amd.abi import Trainer

pytestmark = pytest.mark.gpu

POINTS = {
    "c2_mlp512_relu_adam_b64": [0, 10, 25, 49],
    "c3_mlp512w_gelu_adamw_b64": [0, 10, 25, 49],
    "c5_wide_ce_adagrad_b4096": [0, 1, 2, 3, 4],
}
CASES = [(name, k) for name, ks in POINTS.items() for k in ks]

_traj = {}  # config -> [oracle trainer, steps taken]


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _oracle_at(name, k):
    """The fp32 oracle's trainer after k steps of the config (one trajectory
    per config, advanced as the points are visited in order)."""
    spec, B, lr, _ = CONFIGS[name]
    ws, bs, batches = config_inputs(spec, B)
    X, Y = batches[0]
    t, done = _traj.get(name, (None, 0))
    if t is None or done > k:
        if t is not None:
            t.close()
        t = Trainer(load_oracle(), spec, B)
        t.set_all_params(ws, bs)
        done = 0
    while done < k:
        t.step(X, Y, lr)
        done += 1
    _traj[name] = (t, done)
    return t


@pytest.mark.parametrize("name,k", CASES, ids=[f"{n.split('_')[0]}-step{k + 1}" for n, k in CASES])
def test_teacher_forced_step_gradients(name, k):
    from tests.test_oracle import oracle_trainer

    spec, B, lr, _ = CONFIGS[name]
    say(f"gradient parity {name} step {k + 1}: {spec.text()} B={B}")
    _, _, batches = config_inputs(spec, B)
    X, Y = batches[0]
    orc, hip = load_oracle(), load_hip()
    to = _oracle_at(name, k)
    W0, b0 = to.get_params()
    st0, t0 = to.get_state()

    old = os.environ.get("VOLTA_KEEP_GRADS")
    os.environ["VOLTA_KEEP_GRADS"] = "1"
    try:
        th = Trainer(hip, spec, B)
    finally:
        if old is None:
            os.environ.pop("VOLTA_KEEP_GRADS", None)
        else:
            os.environ["VOLTA_KEEP_GRADS"] = old
    tt = oracle_trainer(orc, spec, B, f64=True)
    for t in (th, tt):
        t.set_all_params(W0, b0)
        t.set_state(st0, t0)
    th.step(X, Y, lr)
    assert th.status() == 0, f"HIP step status {th.status()}"
    say("  hip step done; fp64 twin step")
    tt.step(X, Y, lr)
    cand = gc.read_candidate(th, spec, B)
    twin = gc.read_twin(orc, tt, spec, B)
    W1, b1 = th.get_params()
    st1, t1 = th.get_state()
    th.close()
    tt.close()

    say("  product checks")
    rep = gc.check_step(orc, spec, B, X, Y, W0, b0, cand, twin, f"step {k + 1}")
    say(rep.summary())
    assert not rep.failures, "\n".join(rep.failures)

    say("  optimizer on the HIP gradients")
    t_next = t0 + 1 if spec.optimizer in ("adam", "adamw") else t0
    assert t1 == t_next
    We, be, ste = gc.expected_update(orc, spec, lr, t_next, W0, b0, st0, cand.dw, cand.db)
    for i in range(spec.n_layers):
        assert gc.bits_equal(W1[i], We[i]), f"W{i} differs from the oracle's update of the HIP gradient"
        assert gc.bits_equal(b1[i], be[i]), f"b{i} differs from the oracle's update of the HIP gradient"
    assert gc.bits_equal(st1, ste), "optimizer state differs from the oracle's update of the HIP gradient"


@pytest.mark.parametrize("step", [25, 50])
def test_c5_late_step_gradients_from_hip_state(step):
    """C5 (B=4096, softmax-CE, Adagrad eps 1e-10) over its 50 steps
    the HIP run's own parameters and Adagrad
    sums after step-1 steps, then step `step` checked as above -- every
    product against the fp32 summation bound and the fp64 twin's step from
    the same state, and the update bit-equal to the oracle's Adagrad applied
    to the HIP gradients.  Teacher-forced from the HIP state, so no 50-step
    CPU trajectory is needed."""
    from tests.test_oracle import oracle_trainer

    name = "c5_wide_ce_adagrad_b4096"
    spec, B, lr, _ = CONFIGS[name]
    say(f"gradient parity {name} step {step} from the HIP run's state")
    ws, bs, batches = config_inputs(spec, B)
    X, Y = batches[0]
    orc = load_oracle()
    old = os.environ.get("VOLTA_KEEP_GRADS")
    os.environ["VOLTA_KEEP_GRADS"] = "1"
    try:
        th = Trainer(load_hip(), spec, B)
    finally:
        if old is None:
            os.environ.pop("VOLTA_KEEP_GRADS", None)
        else:
            os.environ["VOLTA_KEEP_GRADS"] = old
    th.set_all_params(ws, bs)
    for _ in range(step - 1):
        th.step(X, Y, lr)
    assert th.status() == 0
    W0, b0 = th.get_params()
    W0 = [w.copy() for w in W0]
    b0 = [b.copy() for b in b0]
    st0, t0 = th.get_state()
    th.step(X, Y, lr)
    assert th.status() == 0, f"HIP step status {th.status()}"
    say(f"  {step} hip steps done; fp64 twin step")
    tt = oracle_trainer(orc, spec, B, f64=True)
    tt.set_all_params(W0, b0)
    tt.set_state(st0, t0)
    tt.step(X, Y, lr)
    cand = gc.read_candidate(th, spec, B)
    twin = gc.read_twin(orc, tt, spec, B)
    W1, b1 = th.get_params()
    st1, t1 = th.get_state()
    th.close()
    tt.close()

    say("  product checks")
    rep = gc.check_step(orc, spec, B, X, Y, W0, b0, cand, twin, f"step {step}")
    say(rep.summary())
    assert not rep.failures, "\n".join(rep.failures)
    say("  optimizer on the HIP gradients")
    We, be, ste = gc.expected_update(orc, spec, lr, t1, W0, b0, st0, cand.dw, cand.db)
    for i in range(spec.n_layers):
        assert gc.bits_equal(W1[i], We[i]), f"W{i} differs from the oracle's update of the HIP gradient"
        assert gc.bits_equal(b1[i], be[i]), f"b{i} differs from the oracle's update of the HIP gradient"
    assert gc.bits_equal(st1, ste), "Adagrad sums differ from the oracle's update of the HIP gradient"


@pytest.mark.parametrize("name,k,tn", [("c2_mlp512_relu_adam_b64", 0, "32"), ("c2_mlp512_relu_adam_b64", 10, "32"),
                                       ("c3_mlp512w_gelu_adamw_b64", 10, "64")])
def test_dw_group_width_forced_step_gradients(name, k, tn):
    """The dW group with the tile width the library would not pick for the
    configuration (VOLTA_DW_GROUP_TN: C2 picks 32x64 tiles, C3 32x32): the
    same gradient-level checks and the bit-equal update."""
    old = os.environ.get("VOLTA_DW_GROUP_TN")
    os.environ["VOLTA_DW_GROUP_TN"] = tn
    try:
        test_teacher_forced_step_gradients(name, k)
    finally:
        if old is None:
            os.environ.pop("VOLTA_DW_GROUP_TN", None)
        else:
            os.environ["VOLTA_DW_GROUP_TN"] = old
