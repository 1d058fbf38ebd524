"""Gradient-level checks of one training step (test infrastructure).

A candidate step (the HIP library, or the fp32 oracle when the checker itself
is tested) is compared with the fp64 twin of the oracle run from the same
state on the same batch.  Every product of the step is checked elementwise
against a bound built by the triangle inequality from quantities the test
measures:

  C = op(A) . op(B) computed in fp32 from the candidate's own operands
  A_c, B_c, against the twin's C_t = A_t . B_t:

    |C_c - C_t| <= |A_c - A_t| . |B_c| + |A_t| . |B_c - B_t|      (input deviation)
                 + 2 K eps |A_c| . |B_c|                          (fp32 summation of K terms)

with eps = 2^-24 and the products of absolute values taken in float64.  The
same bound with zero input deviation is the local check of each product on
the candidate's own operands (the bound the GEMM kernel tests use).  The
activation derivative, the loss gradient and the bias-gradient sum get the
analogous bounds.  A gradient that is wrong in magnitude (a dropped term, a
wrong scale, a transposed operand) exceeds them; rounding in another
summation order, and ReLU masks that flip at a pre-activation within
rounding of zero, stay inside because the measured input deviation carries
them.

The step's formulas are those of mlp_train_rust_codegen.rs:698-994: forward
act_{i+1} = f(act_i W_i + b_i) (:719-743), MSE delta 2(y^ - y)/(B L_n)
(:792-798) or softmax-CE (softmax - onehot)/B (interpreter.rs:762-812),
delta_{i-1} = (delta_i W_i^T) * f'(pre_{i-1}) (:893-929), dW_i = act_i^T
delta_i (:315-317), db_i = sum_b delta_i (:931-933).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from volta_amd.abi import ACTIVATIONS, BUF_ACT, BUF_DELTA, BUF_GRAD_B, BUF_GRAD_W, BUF_PRE

EPS = 2.0 ** -24
# max |f'| of each hidden activation (bounds |f(a) - f(b)| by L |a - b|)
LIPSCHITZ = {"relu": 1.0, "leaky_relu": 1.0, "sigmoid": 0.25, "tanh": 1.0, "silu": 1.1, "gelu": 1.13}
RELU_LIKE = ("relu",)

_D = C.POINTER(C.c_double)


class StepBuffers:
    """The buffers of one step: act_0..act_n, delta_0..delta_{n-1},
    pre_0..pre_{n-2} (None where the library keeps none), dW_i, db_i, all
    float64 arrays shaped as matrices."""

    def __init__(self, act, delta, pre, dw, db):
        self.act, self.delta, self.pre, self.dw, self.db = act, delta, pre, dw, db


def read_candidate(t, spec, B) -> StepBuffers:
    """Buffers of a Trainer's last step through volta_train_debug_buffer
    (fp32 values widened)."""
    n, L = spec.n_layers, spec.sizes
    act = [t.debug_buffer(BUF_ACT, i).astype(np.float64).reshape(B, L[i]) for i in range(n + 1)]
    delta = [t.debug_buffer(BUF_DELTA, i).astype(np.float64).reshape(B, L[i + 1]) for i in range(n)]
    pre = []
    for i in range(n - 1):
        try:
            pre.append(t.debug_buffer(BUF_PRE, i).astype(np.float64).reshape(B, L[i + 1]))
        except RuntimeError:
            pre.append(None)
    dw = [t.debug_buffer(BUF_GRAD_W, i).astype(np.float64).reshape(L[i], L[i + 1]) for i in range(n)]
    db = [t.debug_buffer(BUF_GRAD_B, i).astype(np.float64) for i in range(n)]
    return StepBuffers(act, delta, pre, dw, db)


def read_twin(orc, t, spec, B) -> StepBuffers:
    """Buffers of the fp64 twin's last step, unrounded."""
    n, L = spec.n_layers, spec.sizes
    fn = orc.lib.volta_oracle_debug_buffer_f64

    def get(kind, i, shape):
        out = np.zeros(int(np.prod(shape)), np.float64)
        got = fn(t.h, kind, i, out.ctypes.data_as(_D))
        if got != out.size:
            return None
        return out.reshape(shape)

    act = [get(BUF_ACT, i, (B, L[i])) for i in range(n + 1)]
    delta = [get(BUF_DELTA, i, (B, L[i + 1])) for i in range(n)]
    pre = [get(BUF_PRE, i, (B, L[i + 1])) for i in range(n - 1)]
    dw = [get(BUF_GRAD_W, i, (L[i], L[i + 1])) for i in range(n)]
    db = [get(BUF_GRAD_B, i, (L[i + 1],)) for i in range(n)]
    return StepBuffers(act, delta, pre, dw, db)


def act_derivative(orc, spec, pre, y):
    """f'(pre) in float64 by the oracle's activation derivative (y is the
    layer output, which sigmoid/tanh derive from)."""
    pre = np.ascontiguousarray(pre, np.float64)
    y = np.ascontiguousarray(y, np.float64)
    out = np.empty_like(pre)
    orc.lib.volta_oracle_act_bwd_f64_n(ACTIVATIONS[spec.activation], pre.ctypes.data_as(_D),
                                       y.ctypes.data_as(_D), out.ctypes.data_as(_D), pre.size)
    return out


class Report:
    def __init__(self, label):
        self.label = label
        self.rows = []
        self.failures = []

    def check(self, name, got, want, bound):
        got, want, bound = (np.asarray(x, np.float64) for x in (got, want, bound))
        # the bounds are exact up to the float64 rounding of computing them
        # and of the twin itself (K * 2^-53 relative): equality cases (a sum
        # whose terms all have one sign, a gradient the candidate rounds to
        # exactly zero) need that slack
        bound = bound * (1.0 + 1e-6)
        err = np.abs(got - want)
        bad = ~(err <= bound)
        ratio = float(np.max(err / np.maximum(bound, 1e-300))) if err.size else 0.0
        self.rows.append((name, ratio, int(bad.sum()), err.size))
        if bad.any():
            k = int(np.flatnonzero(bad.ravel())[0])
            self.failures.append(f"{self.label} {name}: {int(bad.sum())} of {err.size} elements beyond the bound "
                                 f"(first at flat index {k}: got {got.ravel()[k]:.9g} want {want.ravel()[k]:.9g} "
                                 f"bound {bound.ravel()[k]:.3g})")

    def summary(self):
        return "\n".join(f"  {self.label} {n}: max err/bound {r:.3f} ({b} of {s} beyond)" for n, r, b, s in self.rows)


def check_step(orc, spec, B, X, Y, W0, b0, cand: StepBuffers, twin: StepBuffers, label, local=True) -> Report:
    """All product checks of one step.  W0/b0: the parameters the step
    started from (float32 arrays), X/Y the batch."""
    n, L = spec.n_layers, spec.sizes
    rep = Report(label)
    W = [np.asarray(w, np.float64).reshape(L[i], L[i + 1]) for i, w in enumerate(W0)]
    bvec = [np.asarray(b, np.float64) for b in b0]
    aW = [np.abs(w) for w in W]
    lip = LIPSCHITZ.get(spec.activation, 1.0)

    rep.check("act0 (input)", cand.act[0], np.asarray(X, np.float64).reshape(B, L[0]), np.zeros((B, L[0])))
    # forward: z_i = act_i W_i + b_i (K = r terms plus the bias)
    for i in range(n):
        r = L[i]
        A_c, A_t = cand.act[i], twin.act[i]
        rnd = 2 * (r + 1) * EPS * (np.abs(A_c) @ aW[i] + np.abs(bvec[i]))
        zdev = np.abs(A_c - A_t) @ aW[i] + rnd
        if local:
            z_own = A_c @ W[i] + bvec[i]
            if i == n - 1:
                rep.check(f"fwd{i} local (output)", cand.act[n], z_own, rnd)
            elif cand.pre[i] is not None:
                rep.check(f"fwd{i} local (pre)", cand.pre[i], z_own, rnd)
        if i == n - 1:
            rep.check(f"fwd{i} vs fp64 (output)", cand.act[n], twin.act[n], zdev)
        else:
            if cand.pre[i] is not None and twin.pre[i] is not None:
                rep.check(f"fwd{i} vs fp64 (pre)", cand.pre[i], twin.pre[i], zdev)
            # fp32 evaluation of f: relative to the larger of |f| and |z|
            # (GELU's 1 + tanh cancels in the negative tail)
            f_rnd = 16 * EPS * (np.abs(twin.act[i + 1]) + np.abs(twin.pre[i]))
            rep.check(f"fwd{i} vs fp64 (act)", cand.act[i + 1], twin.act[i + 1], lip * zdev + f_rnd + 1e-37)

    # loss gradient
    Ln = L[n]
    yh_c, yh_t = cand.act[n], twin.act[n]
    if spec.loss == "mse":
        Yv = np.asarray(Y, np.float64).reshape(B, Ln)
        scale = 2.0 / (B * Ln)
        own = scale * (yh_c - Yv)
        rnd = 8 * EPS * scale * (np.abs(yh_c) + np.abs(Yv))
        if local:
            rep.check("loss grad local", cand.delta[n - 1], own, rnd)
        rep.check("loss grad vs fp64", cand.delta[n - 1], twin.delta[n - 1], scale * np.abs(yh_c - yh_t) + rnd)
    else:
        lab = np.asarray(Y).reshape(B)
        z = yh_c - yh_c.max(axis=1, keepdims=True)
        p = np.exp(z)
        p /= p.sum(axis=1, keepdims=True)
        onehot = np.zeros((B, Ln))
        onehot[np.arange(B), lab] = 1.0
        own = (p - onehot) / B
        rnd = (4 * Ln + 16) * EPS / B * np.ones((B, Ln))
        if local:
            rep.check("loss grad local", cand.delta[n - 1], own, rnd)
        dz = np.abs(yh_c - yh_t).max(axis=1, keepdims=True)
        rep.check("loss grad vs fp64", cand.delta[n - 1], twin.delta[n - 1], dz / B + rnd)

    # backward: delta_{i-1} = (delta_i W_i^T) * f'(pre_{i-1}) (K = c terms)
    for i in range(n - 1, 0, -1):
        c = L[i + 1]
        D_c, D_t = cand.delta[i], twin.delta[i]
        P_c = D_c @ W[i].T
        P_t = D_t @ W[i].T
        rnd = 2 * c * EPS * (np.abs(D_c) @ aW[i].T)
        pdev = np.abs(D_c - D_t) @ aW[i].T + rnd
        if spec.activation in RELU_LIKE:
            f_c = (cand.act[i] > 0).astype(np.float64)
            f_t = (twin.act[i] > 0).astype(np.float64)
            f_rnd = 0.0
        else:
            pre_c = cand.pre[i - 1]
            if pre_c is None:  # derivative from the output (sigmoid/tanh) or recomputed pre
                pre_c = cand.act[i - 1] @ W[i - 1] + bvec[i - 1]
            f_c = act_derivative(orc, spec, pre_c, cand.act[i])
            f_t = act_derivative(orc, spec, twin.pre[i - 1], twin.act[i])
            f_rnd = 32 * EPS  # the candidate's fp32 evaluation of f' (absolute; terms of f' are O(1))
        if local:
            rep.check(f"dx{i} local", cand.delta[i - 1], P_c * f_c,
                      rnd * (np.abs(f_c) + f_rnd) + np.abs(P_c) * f_rnd + 8 * EPS * np.abs(P_c * f_c) + 1e-37)
        bound = pdev * (np.abs(f_c) + f_rnd) + np.abs(P_t) * (np.abs(f_c - f_t) + f_rnd) \
            + 8 * EPS * np.abs(P_t * f_c) + 1e-37
        rep.check(f"dx{i} vs fp64", cand.delta[i - 1], twin.delta[i - 1], bound)

    # dW_i = act_i^T delta_i and db_i = sum_b delta_i (K = B terms)
    for i in range(n):
        A_c, A_t = cand.act[i], twin.act[i]
        D_c, D_t = cand.delta[i], twin.delta[i]
        rnd = 2 * B * EPS * (np.abs(A_c).T @ np.abs(D_c))
        if local:
            rep.check(f"dw{i} local", cand.dw[i], A_c.T @ D_c, rnd + 1e-37)
        bound = np.abs(A_c - A_t).T @ np.abs(D_c) + np.abs(A_t).T @ np.abs(D_c - D_t) + rnd + 1e-37
        rep.check(f"dw{i} vs fp64", cand.dw[i], twin.dw[i], bound)
        rnd_b = 2 * B * EPS * np.abs(D_c).sum(axis=0)
        if local:
            rep.check(f"db{i} local", cand.db[i], D_c.sum(axis=0), rnd_b + 1e-37)
        rep.check(f"db{i} vs fp64", cand.db[i], twin.db[i], np.abs(D_c - D_t).sum(axis=0) + rnd_b + 1e-37)
    return rep


def expected_update(orc, spec, lr, t_next, W0, b0, state0, dw, db):
    """The oracle's fp32 optimizer applied to the given gradients from the
    starting parameters and state: (W list, b list, state) -- what the
    candidate's fused update must equal bit for bit.  `t_next` is the step
    counter after the step (Adam's bias correction uses it)."""
    F = C.POINTER(C.c_float)

    def p(a):
        return a.ctypes.data_as(F)

    n = spec.n_layers
    W = [np.array(w, np.float32, copy=True).ravel() for w in W0]
    bb = [np.array(b, np.float32, copy=True).ravel() for b in b0]
    st = np.array(state0, np.float32, copy=True)
    g_w = [np.ascontiguousarray(np.asarray(g, np.float32).ravel()) for g in dw]
    g_b = [np.ascontiguousarray(np.asarray(g, np.float32).ravel()) for g in db]
    off = 0
    adam = spec.optimizer in ("adam", "adamw")
    if adam:
        bc1 = orc.lib.volta_oracle_bias_correction(spec.beta1, t_next)
        bc2 = orc.lib.volta_oracle_bias_correction(spec.beta2, t_next)
    for i in range(n):
        nw, nb = W[i].size, bb[i].size
        if adam:
            mw, mb = st[off:off + nw], st[off + nw:off + nw + nb]
            vw, vb = st[off + nw + nb:off + 2 * nw + nb], st[off + 2 * nw + nb:off + 2 * (nw + nb)]
            mw, mb, vw, vb = (np.ascontiguousarray(x) for x in (mw, mb, vw, vb))
            wd = spec.to_c().weight_decay if spec.optimizer == "adamw" else 0.0
            orc.lib.volta_oracle_adam(p(W[i]), p(mw), p(vw), p(g_w[i]), nw, spec.beta1, spec.beta2, bc1, bc2, lr,
                                      spec.eps, wd)
            orc.lib.volta_oracle_adam(p(bb[i]), p(mb), p(vb), p(g_b[i]), nb, spec.beta1, spec.beta2, bc1, bc2, lr,
                                      spec.eps, 0.0)
            st[off:off + nw], st[off + nw:off + nw + nb] = mw, mb
            st[off + nw + nb:off + 2 * nw + nb], st[off + 2 * nw + nb:off + 2 * (nw + nb)] = vw, vb
            off += 2 * (nw + nb)
        elif spec.optimizer == "adagrad":
            gw, gb = (np.ascontiguousarray(x) for x in (st[off:off + nw], st[off + nw:off + nw + nb]))
            orc.lib.volta_oracle_adagrad(p(W[i]), p(gw), p(g_w[i]), nw, lr, spec.eps)
            orc.lib.volta_oracle_adagrad(p(bb[i]), p(gb), p(g_b[i]), nb, lr, spec.eps)
            st[off:off + nw], st[off + nw:off + nw + nb] = gw, gb
            off += nw + nb
        else:
            raise ValueError("expected_update covers the adaptive optimizers")
    return W, bb, st


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32).ravel()
    b = np.ascontiguousarray(b, np.float32).ravel()
    return a.shape == b.shape and bool(np.array_equal(a.view(np.uint32), b.view(np.uint32)))


# ---------------------------------------------------------------------------
# Steps with the codegen extras (LayerNorm, dropout, gradient clipping,
# softmax hidden rows; mlp_train_rust_codegen.rs:727-788, :829-955).
#
# The step order there: phase 1 for i = n-1 .. 0 runs, on a hidden layer,
# LayerNorm backward (dgamma/dbeta as batch sums of the upstream gradient g
# and of g * xhat, xhat recomputed from the layer's stored output as
# (y - beta) / (gamma + 1e-12), then gamma/beta -= lr * grad), the dropout
# mask and f'; then db_i = sum_b delta_i; then delta_{i-1} = delta_i W_i^T.
# The clip scales every delta by s = clip / ||delta|| when the norm exceeds
# clip; phase 2 forms dW_i = act_i^T delta_i from the scaled deltas.  So db
# comes from the unscaled deltas and dW from the scaled ones.
#
# Checks on the candidate's own operands (bounds as above): every forward
# product, the loss gradient, dW_i (2 B eps), db_i over the unscaled deltas
# (delta / s), dgamma/dbeta as batch sums of g = delta_{i+1,unscaled}
# W_{i+1}^T (and of g * xhat), and s against clip / ||delta||.  Against the
# fp64 twin: every forward product, dW_i, db_i, dgamma and dbeta by the
# triangle bounds on the measured operand deviations; the dropout masks
# bit for bit; and the hidden activations and deltas, whose LayerNorm /
# softmax row arithmetic has no closed elementwise bound here, by their
# distance from the twin measured against the fp32 oracle's own distance
# from it for the same step (norm within 4x plus 16 eps of the twin's norm,
# largest element within 8x plus 16 eps of the largest).
# ---------------------------------------------------------------------------

class ExtBuffers(StepBuffers):
    """StepBuffers plus the extras' buffers: dgamma/dbeta and gamma/beta
    (after the step) of each hidden layer with LayerNorm, the dropout masks
    and the clip scale (1.0 without clipping).  `delta` holds the deltas as
    the step left them (scaled by the clip)."""

    def __init__(self, base: StepBuffers, dg, dbe, gamma, beta, mask, scale):
        super().__init__(base.act, base.delta, base.pre, base.dw, base.db)
        self.dg, self.dbe, self.gamma, self.beta, self.mask, self.scale = dg, dbe, gamma, beta, mask, scale


def _ext_parts(get, spec, B):
    from volta_amd.abi import BUF_CLIP_SCALE, BUF_DROPOUT_MASK, BUF_LN_BETA, BUF_LN_DBETA, BUF_LN_DGAMMA, \
        BUF_LN_GAMMA
    nh, L = spec.n_layers - 1, spec.sizes
    ln = bool(spec.layernorm)
    dg = [get(BUF_LN_DGAMMA, i, (L[i + 1],)) for i in range(nh)] if ln else []
    dbe = [get(BUF_LN_DBETA, i, (L[i + 1],)) for i in range(nh)] if ln else []
    gam = [get(BUF_LN_GAMMA, i, (L[i + 1],)) for i in range(nh)] if ln else []
    bet = [get(BUF_LN_BETA, i, (L[i + 1],)) for i in range(nh)] if ln else []
    mask = [get(BUF_DROPOUT_MASK, i, (B, L[i + 1])) for i in range(nh)] if spec.dropout_p > 0 else []
    scale = float(get(BUF_CLIP_SCALE, 0, (1,))[0]) if spec.clip_grad > 0 else 1.0
    return dg, dbe, gam, bet, mask, scale


def read_candidate_ext(t, spec, B) -> ExtBuffers:
    """read_candidate plus the extras' buffers, through
    volta_train_debug_buffer (the HIP library, or the fp32 oracle)."""
    base = read_candidate(t, spec, B)

    def get(kind, i, shape):
        return t.debug_buffer(kind, i).astype(np.float64).reshape(shape)
    return ExtBuffers(base, *_ext_parts(get, spec, B))


def read_twin_ext(orc, t, spec, B) -> ExtBuffers:
    """read_twin plus the extras' buffers, unrounded."""
    base = read_twin(orc, t, spec, B)
    fn = orc.lib.volta_oracle_debug_buffer_f64

    def get(kind, i, shape):
        out = np.zeros(int(np.prod(shape)), np.float64)
        if fn(t.h, kind, i, out.ctypes.data_as(_D)) != out.size:
            raise RuntimeError(f"fp64 twin has no buffer {kind} of layer {i}")
        return out.reshape(shape)
    return ExtBuffers(base, *_ext_parts(get, spec, B))


def _norm(x):
    return float(np.sqrt(np.sum(np.square(np.asarray(x, np.float64)))))


def check_against_yardstick(rep, name, got, want, yard):
    """Distance of `got` from the twin's `want`, against the fp32 oracle's
    (`yard`) distance from it on the same step: norm within 4x the oracle's
    plus 16 eps of the twin's norm, largest element within 8x the oracle's
    largest plus 16 eps of the twin's largest."""
    got, want, yard = (np.asarray(x, np.float64) for x in (got, want, yard))
    e_got, e_yard = got - want, yard - want
    n_bound = 4.0 * _norm(e_yard) + 16 * EPS * _norm(want) + 1e-37
    m_bound = 8.0 * float(np.max(np.abs(e_yard), initial=0.0)) + 16 * EPS * float(np.max(np.abs(want), initial=0.0)) \
        + 1e-37
    n_got, m_got = _norm(e_got), float(np.max(np.abs(e_got), initial=0.0))
    ratio = max(n_got / n_bound, m_got / m_bound)
    bad = int(n_got > n_bound) + int(m_got > m_bound)
    rep.rows.append((name, ratio, bad, 2))
    if bad:
        rep.failures.append(f"{rep.label} {name}: distance from fp64 {n_got:.3e} (norm) / {m_got:.3e} (max) "
                            f"against the fp32 oracle's {_norm(e_yard):.3e} / "
                            f"{float(np.max(np.abs(e_yard), initial=0.0)):.3e}")


def clip_sum_terms(spec, B):
    """Sequential terms per thread in the clip's sum of squares (the library
    cuts the deltas into 256 chunks of 256 threads, then two fixed trees)."""
    total = B * sum(spec.sizes[1:])
    chunk = -(-total // 256)
    return -(-chunk // 256)


def check_step_ext(orc, spec, B, X, Y, W0, b0, g0, be0, cand: ExtBuffers, twin: ExtBuffers, yard: ExtBuffers,
                   label, clip_terms=None) -> Report:
    """All checks of one extras step.  W0/b0/g0/be0: the parameters and
    LayerNorm gamma/beta the step started from; yard: the fp32 oracle's
    buffers of the same step (the yardstick of the row-operation checks);
    clip_terms: the longest run of sequential additions in the candidate's
    sum of squares for the clip (default: the HIP library's)."""
    n, L = spec.n_layers, spec.sizes
    rep = Report(label)
    W = [np.asarray(w, np.float64).reshape(L[i], L[i + 1]) for i, w in enumerate(W0)]
    bvec = [np.asarray(b, np.float64) for b in b0]
    aW = [np.abs(w) for w in W]
    ln = bool(spec.layernorm)

    rep.check("act0 (input)", cand.act[0], np.asarray(X, np.float64).reshape(B, L[0]), np.zeros((B, L[0])))
    for i in range(n):
        r = L[i]
        A_c, A_t = cand.act[i], twin.act[i]
        rnd = 2 * (r + 1) * EPS * (np.abs(A_c) @ aW[i] + np.abs(bvec[i]))
        zdev = np.abs(A_c - A_t) @ aW[i] + rnd
        z_own = A_c @ W[i] + bvec[i]
        if i == n - 1:
            rep.check(f"fwd{i} local (output)", cand.act[n], z_own, rnd)
            rep.check(f"fwd{i} vs fp64 (output)", cand.act[n], twin.act[n], zdev)
        elif cand.pre[i] is not None:
            rep.check(f"fwd{i} local (pre)", cand.pre[i], z_own, rnd)
            rep.check(f"fwd{i} vs fp64 (pre)", cand.pre[i], twin.pre[i], zdev)
            check_against_yardstick(rep, f"fwd{i} vs fp64 (act, row ops)", cand.act[i + 1], twin.act[i + 1],
                                    yard.act[i + 1])
        else:
            # no row operation and no stored pre-activation (ReLU, sigmoid,
            # tanh derive f' from the output): act = f(z) from the GEMM
            # epilogue, within f's Lipschitz constant of the operand bound
            lip = LIPSCHITZ.get(spec.activation, 1.0)
            f_rnd = 16 * EPS * (np.abs(twin.act[i + 1]) + np.abs(twin.pre[i]))
            rep.check(f"fwd{i} vs fp64 (act)", cand.act[i + 1], twin.act[i + 1], lip * zdev + f_rnd + 1e-37)
    for i, (mc, mt) in enumerate(zip(cand.mask, twin.mask)):
        rep.check(f"dropout mask {i}", mc, mt, np.zeros_like(mt))

    # the clip scale and the unscaled deltas (delta / s; the division adds
    # one rounding of the product delta * s)
    s_c, s_t = cand.scale, twin.scale
    Du_c = [d / s_c for d in cand.delta]
    Du_t = [d / s_t for d in twin.delta]
    Du_y = [d / yard.scale for d in yard.delta]
    if spec.clip_grad > 0:
        gsq = sum(float(np.sum(d * d)) for d in Du_c)
        own = float(np.float32(spec.clip_grad)) / np.sqrt(gsq) if np.sqrt(gsq) > np.float32(spec.clip_grad) else 1.0
        m = clip_sum_terms(spec, B) if clip_terms is None else clip_terms
        rep.check("clip scale local", np.array([s_c]), np.array([own]), np.array([own * (m + 24) * EPS]))

    # loss gradient (unscaled)
    Ln = L[n]
    yh_c, yh_t = cand.act[n], twin.act[n]
    if spec.loss == "mse":
        Yv = np.asarray(Y, np.float64).reshape(B, Ln)
        scale = 2.0 / (B * Ln)
        rnd = 10 * EPS * scale * (np.abs(yh_c) + np.abs(Yv))
        rep.check("loss grad local", Du_c[n - 1], scale * (yh_c - Yv), rnd)
        rep.check("loss grad vs fp64", Du_c[n - 1], Du_t[n - 1], scale * np.abs(yh_c - yh_t) + rnd)
    else:
        lab = np.asarray(Y).reshape(B)
        z = yh_c - yh_c.max(axis=1, keepdims=True)
        p = np.exp(z)
        p /= p.sum(axis=1, keepdims=True)
        onehot = np.zeros((B, Ln))
        onehot[np.arange(B), lab] = 1.0
        rnd = (4 * Ln + 18) * EPS / B * np.ones((B, Ln))
        rep.check("loss grad local", Du_c[n - 1], (p - onehot) / B, rnd)
        dz = np.abs(yh_c - yh_t).max(axis=1, keepdims=True)
        rep.check("loss grad vs fp64", Du_c[n - 1], Du_t[n - 1], dz / B + rnd)

    for i in range(n - 1, 0, -1):
        check_against_yardstick(rep, f"delta{i - 1} vs fp64", Du_c[i - 1], Du_t[i - 1], Du_y[i - 1])

    # LayerNorm parameter gradients of hidden layer i: g = delta_{i+1} W_{i+1}^T
    # (the upstream gradient, before LayerNorm's backward rewrote it)
    if ln:
        for i in range(n - 1):
            c2 = L[i + 2]
            G_c = Du_c[i + 1] @ W[i + 1].T
            G_t = Du_t[i + 1] @ W[i + 1].T
            # fp32 summation of c2 terms, plus the delta / s reconstruction
            G_rnd = (2 * c2 + 1) * EPS * (np.abs(Du_c[i + 1]) @ aW[i + 1].T)
            gam = np.asarray(g0[i], np.float64)
            bet = np.asarray(be0[i], np.float64)
            den = gam + float(np.float32(1e-12))
            xh_c = (cand.act[i + 1] - bet) / den
            xh_t = (twin.act[i + 1] - bet) / den
            xh_rnd = 3 * EPS * np.abs(xh_c) + EPS * (np.abs(cand.act[i + 1]) + np.abs(bet)) / np.abs(den)
            rnd_b = (G_rnd + 2 * B * EPS * np.abs(G_c)).sum(axis=0)
            rep.check(f"dbeta{i} local", cand.dbe[i], G_c.sum(axis=0), rnd_b + 1e-37)
            rep.check(f"dbeta{i} vs fp64", cand.dbe[i], twin.dbe[i],
                      np.abs(G_c - G_t).sum(axis=0) + rnd_b + 1e-37)
            P_c = G_c * xh_c
            rnd_g = (G_rnd * np.abs(xh_c) + np.abs(G_c) * xh_rnd + (2 * B + 2) * EPS * np.abs(P_c)).sum(axis=0)
            rep.check(f"dgamma{i} local", cand.dg[i], P_c.sum(axis=0), rnd_g + 1e-37)
            rep.check(f"dgamma{i} vs fp64", cand.dg[i], twin.dg[i],
                      (np.abs(G_c - G_t) * np.abs(xh_c) + np.abs(G_t) * np.abs(xh_c - xh_t)).sum(axis=0)
                      + rnd_g + 1e-37)

    # dW_i from the scaled deltas, db_i from the unscaled ones
    for i in range(n):
        A_c, A_t = cand.act[i], twin.act[i]
        D_c, D_t = cand.delta[i], twin.delta[i]
        rnd = 2 * B * EPS * (np.abs(A_c).T @ np.abs(D_c))
        rep.check(f"dw{i} local", cand.dw[i], A_c.T @ D_c, rnd + 1e-37)
        rep.check(f"dw{i} vs fp64", cand.dw[i], twin.dw[i],
                  np.abs(A_c - A_t).T @ np.abs(D_c) + np.abs(A_t).T @ np.abs(D_c - D_t) + rnd + 1e-37)
        rnd_b = (2 * B + 2) * EPS * np.abs(Du_c[i]).sum(axis=0)
        rep.check(f"db{i} local", cand.db[i], Du_c[i].sum(axis=0), rnd_b + 1e-37)
        rep.check(f"db{i} vs fp64", cand.db[i], twin.db[i], np.abs(Du_c[i] - Du_t[i]).sum(axis=0) + rnd_b + 1e-37)
    return rep


def expected_update_ext(orc, spec, lr, t_next, W0, b0, state0, dw, db, g0, be0, dg, dbe):
    """expected_update plus LayerNorm's SGD step of gamma/beta
    (gamma -= lr * dgamma, :884-885) written into the state's tail
    ([gamma_i | beta_i] per hidden layer after the optimizer's moments)."""
    n, L = spec.n_layers, spec.sizes
    per = sum(L[i] * L[i + 1] + L[i + 1] for i in range(n))
    k = {"adam": 2, "adamw": 2, "adagrad": 1}[spec.optimizer] * per
    st0 = np.asarray(state0, np.float32)
    W, bb, head = expected_update(orc, spec, lr, t_next, W0, b0, st0[:k], dw, db)
    tail = []
    lr32 = np.float32(lr)
    for i in range(len(g0)):
        g = np.asarray(g0[i], np.float32) - lr32 * np.asarray(dg[i], np.float32)
        b = np.asarray(be0[i], np.float32) - lr32 * np.asarray(dbe[i], np.float32)
        tail += [g.astype(np.float32), b.astype(np.float32)]
    st = np.concatenate([head] + tail).astype(np.float32) if tail else head
    return W, bb, st
