"""Gradient-level parity of single HIP steps with the codegen extras and an
adaptive optimizer (Adam, AdamW, Adagrad with LayerNorm, dropout, gradient
clipping and softmax hidden rows; mlp_train_rust_codegen.rs:727-788,
:829-993), teacher-forced from the fp32 oracle's exact state after 0 and 3
steps.

At each point one HIP step (VOLTA_KEEP_GRADS=1: the fused dW kernels and the
clip-mode bias update also store the gradient they apply), one fp64-twin
step and one more fp32-oracle step run from the same parameters, optimizer
state, LayerNorm gamma/beta, step counter and dropout stream on the same
batch.  Then (tests/grad_check.py, check_step_ext):
  * every product of the HIP step is within the fp32 summation bound of its
    own operands -- forward products, the loss gradient, dW_i from the
    clipped deltas, db_i from the unclipped ones, dgamma/dbeta as batch sums
    of the upstream gradient -- and the clip scale is clip / ||delta||;
  * the same products are within the triangle bound of the fp64 twin's, the
    dropout masks equal the twin's, and the hidden activations and deltas
    (LayerNorm / softmax rows) are no further from the twin than the fp32
    oracle is (4x in norm, 8x in the largest element, plus 16 eps);
  * the HIP step's parameters, Adam moments / Adagrad sums and LayerNorm
    gamma/beta equal, bit for bit, the oracle's optimizer (and LayerNorm's
    SGD step) applied to the HIP step's own gradients.
The last pins the wiring only the extras path uses -- the bias update from
the unclipped deltas under clipping (bias_update_kernel) and the phase-2
dW launches without a bias -- in magnitude, not only in sign.
"""
import os
import sys

import numpy as np
import pytest

from tests import grad_check as gc
from tests.oracle_lib import load_oracle
from tests.test_gpu_extras import ADAPTIVE, CASES, resolve
from tests.test_oracle import oracle_trainer
from volta_amd import data, load_hip
from volta_amd.abi import Trainer

pytestmark = pytest.mark.gpu

SEED = 11
POINTS = (0, 3)
ADAPTIVE_CASES = [c for c in CASES if c[1].optimizer in ADAPTIVE]
PARAMS = [(c, k) for c in ADAPTIVE_CASES for k in POINTS]


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def ln_from_state(spec, st):
    """gamma_i, beta_i of each hidden layer from the state's tail."""
    if not spec.layernorm:
        return [], []
    L = spec.sizes
    widths = L[1:-1]
    off = st.size - 2 * sum(widths)
    g, b = [], []
    for c in widths:
        g.append(st[off:off + c].copy())
        b.append(st[off + c:off + 2 * c].copy())
        off += 2 * c
    return g, b


def hip_trainer(spec, B):
    old = os.environ.get("VOLTA_KEEP_GRADS")
    os.environ["VOLTA_KEEP_GRADS"] = "1"
    try:
        return Trainer(load_hip(), spec, B)
    finally:
        if old is None:
            os.environ.pop("VOLTA_KEEP_GRADS", None)
        else:
            os.environ["VOLTA_KEEP_GRADS"] = old


@pytest.mark.parametrize("case,k", PARAMS, ids=[f"{c[0]}-step{k + 1}" for c, k in PARAMS])
def test_extras_teacher_forced_step_gradients(case, k):
    label, spec, B, lr = case
    spec = resolve(spec, B, SEED)
    say(f"extras gradient parity {label} step {k + 1}: {spec.text()} B={B}")
    orc = load_oracle()
    ws, bs = data.he_uniform(SEED, spec.sizes)
    batches = [data.batch(SEED + j, spec.sizes, B, spec.loss) for j in range(2)]
    to = Trainer(orc, spec, B)
    to.set_all_params(ws, bs)
    for s in range(k):
        to.step(*batches[s % 2], lr)
    X, Y = batches[k % 2]
    W0, b0 = to.get_params()
    st0, t0 = to.get_state()
    rng0 = to.get_dropout_rng()
    g0, be0 = ln_from_state(spec, st0)

    th = hip_trainer(spec, B)
    tt = oracle_trainer(orc, spec, B, f64=True)
    for t in (th, tt):
        t.set_all_params(W0, b0)
        t.set_state(st0, t0)
        t.set_dropout_rng(rng0)
    th.step(X, Y, lr)
    assert th.status() == 0, f"HIP step status {th.status()}"
    say("  hip step done; fp64 twin and fp32 oracle steps")
    tt.step(X, Y, lr)
    to.step(X, Y, lr)
    cand = gc.read_candidate_ext(th, spec, B)
    twin = gc.read_twin_ext(orc, tt, spec, B)
    yard = gc.read_candidate_ext(to, spec, B)
    W1, b1 = th.get_params()
    st1, t1 = th.get_state()
    assert th.get_dropout_rng() == to.get_dropout_rng(), "dropout stream differs after the step"
    for t in (th, tt, to):
        t.close()

    say("  product checks")
    rep = gc.check_step_ext(orc, spec, B, X, Y, W0, b0, g0, be0, cand, twin, yard, f"{label} step {k + 1}")
    say(rep.summary())
    assert not rep.failures, "\n".join(rep.failures)

    say("  optimizer and LayerNorm update on the HIP gradients")
    t_next = t0 + 1 if spec.optimizer in ("adam", "adamw") else t0
    assert t1 == t_next
    We, be, ste = gc.expected_update_ext(orc, spec, lr, t_next, W0, b0, st0, cand.dw, cand.db, g0, be0,
                                         cand.dg, cand.dbe)
    for i in range(spec.n_layers):
        assert gc.bits_equal(W1[i], We[i]), f"W{i} differs from the oracle's update of the HIP gradient"
        assert gc.bits_equal(b1[i], be[i]), f"b{i} differs from the oracle's update of the HIP gradient"
    assert gc.bits_equal(st1, ste), "optimizer state / gamma / beta differ from the update of the HIP gradients"
    for i, (g, b) in enumerate(zip(cand.gamma, cand.beta)):
        gs, bst = ln_from_state(spec, st1)
        assert gc.bits_equal(g, gs[i]) and gc.bits_equal(b, bst[i]), f"gamma/beta {i}: state export differs"
