"""The runtime optimizer on the GPU (volta_rt_*, include/volta_backend.h)
against the CPU oracle's restatement of optimizer.rs, through the same C ABI:
every parameter and state buffer bit for bit (LARS: its norms are a
fixed-order tree instead of the reference's sequential sums, so parameters
within rel 1e-6 and velocities within the sequential sum's error), the same
error messages and step counts."""
from __future__ import annotations

import numpy as np
import pytest

from tests.oracle_lib import load_oracle
from volta_amd import DeviceArray, load_hip
from volta_amd.backend import BUFFERS, HipBackend, OptimizerError, RtOptimizer, config

pytestmark = pytest.mark.gpu

SIZES = [1, 5, 1000, 1023, 1025, 4099, 65536 + 7]

CONFIGS = {
    "sgd": config("sgd", 0.05),
    "adam": config("adam", 1e-3),
    "adamw": config("adamw", 1e-3, weight_decay=0.01),
    "rmsprop": config("rmsprop", 1e-2, alpha=0.99, weight_decay=1e-4),
    "rmsprop_momentum": config("rmsprop", 1e-2, alpha=0.9, momentum=0.9),
    "adagrad": config("adagrad", 1e-2, epsilon=1e-10, weight_decay=1e-3),
    "lars": config("lars", 0.1, momentum=0.9, weight_decay=1e-4, trust_coeff=1e-3, epsilon=1e-8),
}


def say(msg):
    print(msg, flush=True)


def _tensors(seed, skip=()):
    rng = np.random.default_rng(seed)
    params = [rng.standard_normal(n).astype(np.float32) for n in SIZES]
    grads = [None if i in skip else (rng.standard_normal(n) * 0.1).astype(np.float32)
             for i, n in enumerate(SIZES)]
    return params, grads


def _run_oracle(params, grads, cfgs):
    ps = [p.copy() for p in params]
    opt = RtOptimizer(load_oracle().lib, [p.size for p in ps])
    for cfg in cfgs:
        opt.apply(cfg, [p.ctypes.data for p in ps], [None if g is None else g.ctypes.data for g in grads])
    return ps, opt


def _run_hip(params, grads, cfgs):
    lib = load_hip()
    dp = [DeviceArray(p, lib) for p in params]
    dg = [None if g is None else DeviceArray(g, lib) for g in grads]
    opt = RtOptimizer(lib.lib, [p.size for p in params])
    for cfg in cfgs:
        opt.apply(cfg, [d.ptr for d in dp], [None if d is None else d.ptr for d in dg])
    return [d.numpy() for d in dp], opt


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_matches_oracle_over_steps(name):
    say(f"runtime optimizer {name}")
    params, grads = _tensors(7, skip=(2,))
    cfgs = [CONFIGS[name]] * 5
    hp, ho = _run_hip(params, grads, cfgs)
    op, oo = _run_oracle(params, grads, cfgs)
    assert ho.step == oo.step == 5
    for i, (a, b) in enumerate(zip(hp, op)):
        if name == "lars":
            np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7, err_msg=f"tensor {i}")
        else:
            np.testing.assert_array_equal(a, b, err_msg=f"tensor {i}")
    np.testing.assert_array_equal(hp[2], params[2])  # no gradient: untouched
    for which in BUFFERS:
        for i in range(len(SIZES)):
            sh, so = ho.state(which, i), oo.state(which, i)
            assert (sh is None) == (so is None), (which, i)
            if sh is None:
                continue
            if name == "lars":
                # the velocity carries the local rate's error: the oracle's
                # (and the reference's) sequential f32 norm of n squares is
                # off by O(sqrt(n) eps) relative (1.5e-5 at n = 65543), the
                # GPU's tree by O(log n eps)
                n = SIZES[i]
                np.testing.assert_allclose(sh, so, rtol=max(1e-6, 8 * np.sqrt(n) * 6e-8), atol=1e-9)
            else:
                np.testing.assert_array_equal(sh, so, err_msg=f"{which}[{i}]")


def test_switching_configurations_shares_state_like_the_reference():
    """Adam then AdamW reuse adam_m/adam_v; RMSprop without, then with
    momentum creates the momentum buffer on first use."""
    say("runtime optimizer: configuration switches")
    params, grads = _tensors(11)
    cfgs = [CONFIGS["adam"], CONFIGS["adamw"], CONFIGS["rmsprop"], CONFIGS["rmsprop_momentum"], CONFIGS["sgd"]]
    hp, ho = _run_hip(params, grads, cfgs)
    op, oo = _run_oracle(params, grads, cfgs)
    for a, b in zip(hp, op):
        np.testing.assert_array_equal(a, b)
    for which in ("adam_m", "adam_v", "rms_v", "rms_buf"):
        np.testing.assert_array_equal(ho.state(which, 0), oo.state(which, 0))


@pytest.mark.parametrize("cfg", [config("sgd", 0.0), config("adam", 1e-3, beta1=1.0),
                                 config("adamw", 1e-3, weight_decay=-1.0), config("rmsprop", 1e-2, alpha=1.0),
                                 config("adagrad", 0.1, epsilon=0.0), config("lars", float("nan"))])
def test_rejections_match_oracle(cfg):
    say(f"runtime optimizer rejection kind={cfg.kind}")
    params, grads = _tensors(3)
    msgs = []
    for run in (_run_hip, _run_oracle):
        with pytest.raises(OptimizerError) as e:
            run(params, grads, [cfg])
        msgs.append(str(e.value))
    assert msgs[0] == msgs[1]


def test_rejected_step_still_counts():
    """After a rejected call the step has advanced (optimizer.rs:114): the
    next Adam step uses bias corrections of step 2, as the oracle's does."""
    say("runtime optimizer: rejected step counts")
    params, grads = _tensors(5)
    res = []
    for lib_run in ("hip", "oracle"):
        lib = load_hip() if lib_run == "hip" else None
        ps = [p.copy() for p in params]
        if lib:
            dp = [DeviceArray(p, lib) for p in ps]
            dg = [DeviceArray(g, lib) for g in grads]
            opt = RtOptimizer(lib.lib, [p.size for p in ps])
            pp, gp = [d.ptr for d in dp], [d.ptr for d in dg]
        else:
            opt = RtOptimizer(load_oracle().lib, [p.size for p in ps])
            pp, gp = [p.ctypes.data for p in ps], [g.ctypes.data for g in grads]
        with pytest.raises(OptimizerError):
            opt.apply(config("adam", -1.0), pp, gp)
        opt.apply(CONFIGS["adam"], pp, gp)
        assert opt.step == 2
        res.append([d.numpy() for d in dp] if lib else ps)
    for a, b in zip(*res):
        np.testing.assert_array_equal(a, b)


def test_hip_backend_apply_gradients_by_id():
    """The Backend-shaped mirror: parameters and gradients keyed by id,
    missing gradients skipped, shape mismatches rejected."""
    say("runtime optimizer: backend mirror")
    backend = HipBackend()
    caps = backend.capabilities()
    assert caps["supports_training"] == 1 and caps["supports_gradient_updates"] == 1
    rng = np.random.default_rng(2)
    host = {7: rng.standard_normal(300).astype(np.float32), 3: rng.standard_normal(64).astype(np.float32)}
    params = {k: DeviceArray(v) for k, v in host.items()}
    grads = {7: DeviceArray(np.full(300, 0.5, np.float32))}
    state = backend.new_state(params)
    backend.apply_gradients(params, grads, config("sgd", 0.1), state)
    np.testing.assert_array_equal(params[7].numpy(), host[7] - np.float32(0.1) * np.float32(0.5))
    np.testing.assert_array_equal(params[3].numpy(), host[3])
    with pytest.raises(OptimizerError, match="Shape mismatch"):
        backend.apply_gradients(params, {3: DeviceArray(np.ones(5, np.float32))}, config("sgd", 0.1), state)


def test_two_runs_bit_identical_lars():
    say("runtime optimizer: LARS determinism")
    params, grads = _tensors(13)
    a, _ = _run_hip(params, grads, [CONFIGS["lars"]] * 3)
    b, _ = _run_hip(params, grads, [CONFIGS["lars"]] * 3)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
