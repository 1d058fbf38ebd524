"""Write the committed golden fixtures for the compile-train MLP step.

Expected values come from PyTorch in float64 -- autograd for the gradients,
torch.optim for the updates, torch.nn.functional for losses and
activations -- i.e. from an implementation that shares no code with the
oracle.  Each case uses the semantics of the step Volta's `compile-train`
generates (mlp_train_rust_codegen.rs:698-994):

  * forward  act_{i+1} = f(act_i W_i + b_i), last layer linear;
  * MSE      mean over B*Ln (:792-798);
  * softmax-CE mean over B (interpreter.rs:762-812, autograd.rs:467-534);
  * SGD      W -= lr*dW, b -= lr*db (:986-991);
  * Adam     torch.optim.Adam (same formula as adam_update, :326-388);
  * AdamW    torch.optim.AdamW with decay on W only -- the generated step
             passes wd=0 for biases (:966);
  * Adagrad  torch.optim.Adagrad, accumulator starting at 0 (:967-985).

Case "tiny_mlp_sgd" is the reference's own parity fixture: the literals of
tests/pytorch_parity.rs:120-243 (x[2x3], w1[3x4], b1[4], w2[4x2], b2[2],
two samples), with lr 0.05 as in examples/pytorch_parity.py:613-668.

Run:  python tests/golden/make_golden.py   (writes tests/golden/*.json)
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from volta_amd import data  # noqa: E402

torch.set_default_dtype(torch.float64)

ACT = {
    "relu": torch.relu,
    "sigmoid": torch.sigmoid,
    "tanh": torch.tanh,
    "leaky_relu": lambda x: F.leaky_relu(x, 0.01),
    "silu": F.silu,
    "gelu": lambda x: F.gelu(x, approximate="tanh"),
}


def f32r(x):
    return float(np.float32(x))


def run_case(sizes, activation, optimizer, loss, ws, bs, batches, lr, steps, eps=1e-8, wd=0.01,
             keep_grads=True):
    # The step takes float32 constants (lr argument, baked eps/betas/wd), so
    # the float64 run uses the same float32-rounded values.
    lr, eps, wd = f32r(lr), f32r(eps), f32r(wd)
    betas = (f32r(0.9), f32r(0.999))
    W = [torch.tensor(w.astype(np.float64), requires_grad=True) for w in ws]
    Bv = [torch.tensor(b.astype(np.float64), requires_grad=True) for b in bs]
    if optimizer == "sgd":
        opt = torch.optim.SGD(W + Bv, lr=lr)
    elif optimizer == "adam":
        opt = torch.optim.Adam(W + Bv, lr=lr, betas=betas, eps=eps)
    elif optimizer == "adamw":
        opt = torch.optim.AdamW(
            [{"params": W, "weight_decay": wd}, {"params": Bv, "weight_decay": 0.0}],
            lr=lr, betas=betas, eps=eps)
    elif optimizer == "adagrad":
        opt = torch.optim.Adagrad(W + Bv, lr=lr, eps=eps, initial_accumulator_value=0.0)
    else:
        raise ValueError(optimizer)
    losses = []
    grads0 = None
    n = len(W)
    for s in range(steps):
        X, Y = batches[s % len(batches)]
        h = torch.tensor(X.astype(np.float64))
        for i in range(n):
            h = h @ W[i] + Bv[i]
            if i < n - 1:
                h = ACT[activation](h)
        if loss == "mse":
            L = F.mse_loss(h, torch.tensor(Y.astype(np.float64)))
        else:
            L = F.cross_entropy(h, torch.tensor(Y.astype(np.int64)))
        opt.zero_grad()
        L.backward()
        if s == 0 and keep_grads:
            grads0 = {
                "w": [w.grad.detach().numpy().ravel().tolist() for w in W],
                "b": [b.grad.detach().numpy().ravel().tolist() for b in Bv],
            }
        opt.step()
        losses.append(float(L.detach()))
    return {
        "losses": losses,
        "grads_step0": grads0,
        "w": [w.detach().numpy().ravel().tolist() for w in W],
        "b": [b.detach().numpy().ravel().tolist() for b in Bv],
    }


def tiny_fixture_case():
    # Literals of tests/pytorch_parity.rs:189-243.
    w1 = np.array([0.1, -0.2, 0.3, 0.4, 0.5, 0.6, -0.7, 0.8, -0.9, 1.0, 0.2, -0.3], np.float32).reshape(3, 4)
    b1 = np.array([0.05, -0.1, 0.15, 0.2], np.float32)
    w2 = np.array([0.2, -0.4, 0.1, 0.3, -0.5, 0.7, 0.6, -0.2], np.float32).reshape(4, 2)
    b2 = np.array([0.25, -0.35], np.float32)
    batches = [
        (np.array([[0.2, -0.1, 0.3], [0.7, 0.5, -0.4]], np.float32),
         np.array([[0.1, -0.2], [0.3, 0.4]], np.float32)),
        (np.array([[0.4, 0.2, -0.5], [-0.3, 0.6, 0.8]], np.float32),
         np.array([[0.2, 0.05], [-0.1, 0.6]], np.float32)),
    ]
    return [w1, w2], [b1, b2], batches


def f32_list(a):
    # 9 significant digits round-trip every float32 exactly.
    a = np.asarray(a)
    if a.dtype.kind in "iu":
        return a.ravel().tolist()
    return [float("%.9g" % v) for v in a.astype(np.float32).ravel()]


def encode_inputs(ws, bs, batches):
    return {
        "w": [f32_list(w) for w in ws],
        "b": [f32_list(b) for b in bs],
        "X": [f32_list(x) for x, _ in batches],
        "Y": [f32_list(y) for _, y in batches],
    }


def round12(v):
    # 12 significant digits: far below every tolerance the tests apply.
    if isinstance(v, float):
        return float("%.12g" % v)
    if isinstance(v, list):
        return [round12(x) for x in v]
    if isinstance(v, dict):
        return {k: round12(x) for k, x in v.items()}
    return v


def main():
    cases = []
    # 1. The reference's tiny fixture, every optimizer x activation, MSE.
    ws, bs, batches = tiny_fixture_case()
    for opt, lr in (("sgd", 0.05), ("adam", 1e-2), ("adamw", 1e-2), ("adagrad", 1e-1)):
        for act in ACT:
            steps = 6
            cases.append({
                "name": f"tiny_{act}_{opt}_mse",
                "sizes": [3, 4, 2], "batch": 2, "activation": act, "optimizer": opt,
                "loss": "mse", "lr": lr, "eps": 1e-8, "weight_decay": 0.01 if opt == "adamw" else 0.0,
                "steps": steps, "inputs": encode_inputs(ws, bs, batches),
                "expected": run_case([3, 4, 2], act, opt, "mse", ws, bs, batches, lr, steps),
            })
    # 2. Small seeded MLPs (3 weight layers so hidden->hidden backprop is
    #    covered), MSE and softmax-CE, every optimizer; Adagrad also with
    #    the eps=1e-10 that the benchmark's wide classifier asks for.
    sizes_mse = [12, 20, 16, 3]
    sizes_ce = [12, 20, 16, 5]
    B = 6
    combos = []
    for act in ACT:
        combos.append((act, "sgd", "mse", 0.05, 1e-8))
    for opt, lr in (("adam", 1e-2), ("adamw", 1e-2), ("adagrad", 5e-2)):
        combos.append(("relu", opt, "mse", lr, 1e-8))
        combos.append(("gelu", opt, "mse", lr, 1e-8))
    for act, opt, lr, eps in (("relu", "sgd", 0.1, 1e-8), ("relu", "adagrad", 1e-2, 1e-10),
                              ("tanh", "adam", 1e-2, 1e-8), ("silu", "adamw", 1e-2, 1e-8)):
        combos.append((act, opt, "ce", lr, eps))
    for k, (act, opt, loss, lr, eps) in enumerate(combos):
        sizes = sizes_ce if loss == "ce" else sizes_mse
        seed = 100 + k
        ws, bs = data.he_uniform(seed, sizes)
        # small nonzero biases so the bias path is exercised from step 0
        bs = [(0.05 * data.normal(seed + 50 + i, (b.size,))).astype(np.float32) for i, b in enumerate(bs)]
        batches = [data.batch(seed + j, sizes, B, loss) for j in range(2)]
        steps = 8
        cases.append({
            "name": f"mlp_{act}_{opt}_{loss}" + ("_eps1e-10" if eps == 1e-10 else ""),
            "sizes": sizes, "batch": B, "activation": act, "optimizer": opt, "loss": loss,
            "lr": lr, "eps": eps, "weight_decay": 0.01 if opt == "adamw" else 0.0,
            "steps": steps, "inputs": encode_inputs(ws, bs, batches),
            "expected": run_case(sizes, act, opt, loss, ws, bs, batches, lr, steps, eps=eps,
                                 keep_grads=(k == 0)),
        })
    for c in cases:
        c["expected"] = round12(c["expected"])
    out = os.path.join(HERE, "train_step_golden.json")
    with open(out, "w") as f:
        json.dump({"generator": "tests/golden/make_golden.py (torch float64, torch " + torch.__version__.split("+")[0] + ")",
                   "cases": cases}, f, separators=(",", ":"))
    print(f"wrote {len(cases)} cases to {out} ({os.path.getsize(out)} bytes)")

    # 3. Reference optimizer known-answer test (optimizer.rs:831-862):
    #    w=0.5, g=0.1, Adam lr=1e-3 step 1 -> 0.499000 (+-1e-5).
    kat = {"adam_step1": {"w": 0.5, "g": 0.1, "lr": 1e-3, "expected": 0.499, "tol": 1e-5}}
    with open(os.path.join(HERE, "optimizer_kat.json"), "w") as f:
        json.dump(kat, f, indent=1)


if __name__ == "__main__":
    main()
