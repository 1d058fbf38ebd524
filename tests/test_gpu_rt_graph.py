"""GPU: graph execution of the HIP backend (volta_rt_execute_value /
execute_terminal, include/volta_backend.h) against the oracle's
node-by-node interpreter on the same graphs and values.

  * every value of a chain (bound input, product, bias sum, activation,
    softmax, Output alias) equals the oracle's within the fp32 tolerance
    (rel 1e-4 / abs 1e-5), and each layer's bias sum is within the fp32
    summation bound K u |A||B| + u(|AB| + |b|) of the float64 product of the
    HIP layer's own input (teacher-forced, so an error in one layer cannot
    hide behind the tolerance of the whole chain);
  * the activations equal the oracle's activation of the HIP bias sum: ReLU
    bit for bit, sigmoid and GELU within 4 ulps;
  * the 16-byte and the element-wise code paths (misaligned bindings) agree
    with the oracle; repeated runs are bit-identical;
  * at C5's shape (4096 rows, 1024-4096-4096-1024-10) the first 64 rows
    against the oracle's run on those rows (rows are independent).
"""
import sys

import numpy as np
import pytest

from tests.oracle_lib import load_oracle
from tests.test_rt_graph_oracle import mlp_values, model_graph
from volta_amd import DeviceArray, load_hip
from volta_amd.backend import BackendError, Graph, GraphLibrary, build_execution_plan

pytestmark = pytest.mark.gpu
F32 = np.float32
U = 2.0 ** -24


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


class Bound:
    """Values of a graph on the device (one allocation per name, optionally
    4 bytes past a 16-byte boundary) and on the host."""

    def __init__(self, vals, misalign=False):
        self.host = {k: np.ascontiguousarray(v, F32) for k, v in vals.items()}
        self.dev = {}
        self.addr = {}
        for k, v in self.host.items():
            flat = v.ravel()
            if misalign:
                flat = np.concatenate([np.zeros(1, F32), flat])
            d = DeviceArray(flat)
            self.dev[k] = d
            self.addr[k] = d.ptr + (4 if misalign else 0)


def hip_value(g, plan, bound, target, cap=None):
    lib = GraphLibrary(load_hip().lib)
    cap = cap or 1 << 22
    out = DeviceArray(np.zeros(cap, F32))
    try:
        r, c = lib.execute(g, plan, target, bound.addr, out.ptr, cap)
        return out.numpy()[: r * c].reshape(r, c)
    finally:
        out.free()


def oracle_value(g, plan, bound, target):
    lib = GraphLibrary(load_oracle().lib)
    cap = 1 << 24
    out = np.zeros(cap, F32)
    r, c = lib.execute(g, plan, target, {k: v.ctypes.data for k, v in bound.host.items()}, out.ctypes.data, cap)
    return out[: r * c].reshape(r, c).copy()


def assert_close(got, want, label, rtol=1e-4, atol=1e-5):
    assert got.shape == want.shape, (label, got.shape, want.shape)
    err = np.abs(got.astype(np.float64) - want)
    bad = err > atol + rtol * np.abs(want)
    assert not bad.any(), f"{label}: {int(bad.sum())} elements out of tolerance, max abs err {err.max():.3e}"


def chain_ids(g):
    """ValueIds of the chain with their op, in order."""
    return [(i, op) for i, (op, args, name, a, b) in enumerate(g.nodes) if op not in ("parameter",)]


CASES = [([32, 64, 48, 8], "relu", 64), ([17, 40, 23], "sigmoid", 7), ([64, 128, 128, 10], "softmax", 300),
         ([512, 1024, 1024, 512, 256, 1], "relu", 64), ([33, 20, 20, 5], "tanh", 1), ([256, 512, 256], "relu", 1000)]


@pytest.mark.parametrize("layers,activation,rows", CASES,
                         ids=[f"{'-'.join(map(str, l))}_{a}_r{r}" for l, a, r in CASES])
def test_every_value_matches_oracle(layers, activation, rows):
    say(f"graph {layers} {activation} rows={rows}")
    g = model_graph(layers, activation, rows)
    plan = build_execution_plan(g)
    b = Bound(mlp_values(layers, rows, 7))
    for vid, op in chain_ids(g):
        got = hip_value(g, plan, b, vid)
        want = oracle_value(g, plan, b, vid)
        if op == "input":
            np.testing.assert_array_equal(got, want)
        else:
            assert_close(got, want, f"value {vid} ({op})")
    # execute_terminal: the last node's value (no Output node in this graph)
    np.testing.assert_array_equal(hip_value(g, plan, b, None), hip_value(g, plan, b, g.last_value_id()))


@pytest.mark.parametrize("layers,activation,rows", [([48, 96, 64, 12], "relu", 64), ([48, 96, 64, 12], "sigmoid", 5),
                                                    ([512, 1024, 1024, 512, 256, 1], "relu", 64)])
def test_layers_teacher_forced(layers, activation, rows):
    """Each bias sum against the float64 product of the HIP layer's own input,
    each activation against the oracle's activation of the HIP bias sum."""
    say(f"teacher-forced layers {layers} {activation} rows={rows}")
    g = model_graph(layers, activation, rows)
    plan = build_execution_plan(g)
    vals = mlp_values(layers, rows, 11)
    b = Bound(vals)
    prev = vals["input"].astype(np.float64)
    ids = chain_ids(g)
    adds = [vid for vid, op in ids if op == "add"]
    acts = {vid: op for vid, op in ids if op in ("relu", "sigmoid")}
    for li, (fi, fo) in enumerate(zip(layers[:-1], layers[1:])):
        W = vals[f"weight_{fi}_{fo}"].astype(np.float64)
        bias = vals[f"bias_{fo}"].astype(np.float64)
        pre = hip_value(g, plan, b, adds[li]).astype(np.float64)
        exact = prev @ W + bias
        bound = 1.01 * (fi * U * (np.abs(prev) @ np.abs(W)) + U * (np.abs(prev @ W) + np.abs(bias))) + 1e-30
        err = np.abs(pre - exact)
        assert (err <= bound).all(), f"layer {li}: bias sum off by {float((err / bound).max()):.2f}x its bound"
        act_id = adds[li] + 1 if (adds[li] + 1) in acts else None
        if act_id is None:
            prev = pre
            continue
        y = hip_value(g, plan, b, act_id)
        one = Graph()
        x = one.add_op("input", name="x")
        one.add_op(acts[act_id], x)
        one.bind_input_shape("x", list(pre.shape))
        ref = oracle_value(one, build_execution_plan(one), Bound({"x": pre.astype(F32)}), None)
        if acts[act_id] == "relu":
            np.testing.assert_array_equal(y, ref)
        else:
            ulp = np.spacing(np.abs(ref).astype(F32)).astype(np.float64)
            assert (np.abs(y.astype(np.float64) - ref) <= 4 * ulp).all(), f"layer {li} {acts[act_id]}"
        prev = y.astype(np.float64)


def test_gemm_form_gelu_and_output_aliases():
    """The Gemm form with a [c] bias, a GELU, a bias-less MatMul layer, and
    Output nodes: every value matches the oracle; execute_terminal returns
    the last Output's value."""
    say("gemm form")
    g = Graph()
    x = g.add_op("input", name="x")
    w1, b1, w2, w3, b3 = (g.add_op("parameter", name=n) for n in ("w1", "b1", "w2", "w3", "b3"))
    h1 = g.add_op("gelu", g.add_op("gemm", x, w1, b1))
    o1 = g.add_op("output", h1)
    h2 = g.add_op("relu", g.add_op("matmul", h1, w2))
    h3 = g.add_op("gemm", h2, w3, b3, beta=0.0)  # beta = 0: no bias
    g.add_op("output", h3)
    g.add_op("output", o1)  # the last Output names h1
    rows = 37
    shapes = {"x": [rows, 24], "w1": [24, 40], "b1": [40], "w2": [40, 36], "w3": [36, 8], "b3": [1, 8]}
    for n, s in shapes.items():
        g.bind_input_shape(n, s)
    rng = np.random.default_rng(5)
    vals = {n: rng.uniform(-1, 1, s).astype(F32) for n, s in shapes.items()}
    plan = build_execution_plan(g)
    b = Bound(vals)
    for vid, op in chain_ids(g):
        assert_close(hip_value(g, plan, b, vid), oracle_value(g, plan, b, vid), f"value {vid} ({op})")
    np.testing.assert_array_equal(hip_value(g, plan, b, None), hip_value(g, plan, b, h1))


@pytest.mark.parametrize("rows", [64, 5])
def test_misaligned_bindings_take_the_elementwise_path(rows):
    layers = [32, 64, 16]
    say(f"misaligned bindings rows={rows}")
    g = model_graph(layers, "relu", rows)
    plan = build_execution_plan(g)
    vals = mlp_values(layers, rows, 2)
    aligned = hip_value(g, plan, Bound(vals), None)
    off = hip_value(g, plan, Bound(vals, misalign=True), None)
    want = oracle_value(g, plan, Bound(vals), None)
    assert_close(off, want, "misaligned")
    assert_close(aligned, want, "aligned")


def test_big_tile_layer_into_unaligned_output():
    """A 4096-row graph whose last layer runs on the 256x256 tile with its
    bias epilogue, written straight into the caller's output: an output 4
    bytes off a 16-byte boundary (the epilogue's 4-byte path) holds the same
    bits as an aligned one."""
    layers, rows = [1024, 4096, 4096], 4096
    say("big-tile layer into an unaligned output")
    g = model_graph(layers, "relu", rows)
    plan = build_execution_plan(g)
    b = Bound(mlp_values(layers, rows, 13))
    lib = GraphLibrary(load_hip().lib)
    n = rows * layers[-1]
    outs = []
    for off in (0, 1):
        out = DeviceArray(np.zeros(n + 1, F32))
        try:
            r, c = lib.execute(g, plan, None, b.addr, out.ptr + 4 * off, n)
            assert (r, c) == (rows, layers[-1])
            outs.append(out.numpy()[off:off + n].copy())
        finally:
            out.free()
    assert np.isfinite(outs[0]).all() and (outs[0] > 0).any()
    np.testing.assert_array_equal(outs[1], outs[0])


def test_repeated_runs_bit_identical_and_cache_reused():
    layers = [128, 256, 256, 10]
    g = model_graph(layers, "softmax", 96)
    plan = build_execution_plan(g)
    b = Bound(mlp_values(layers, 96, 4))
    lib = GraphLibrary(load_hip().lib)
    first = hip_value(g, plan, b, None)
    n = lib.compile_count()
    for _ in range(3):
        np.testing.assert_array_equal(hip_value(g, plan, b, None), first)
    assert lib.compile_count() == n
    np.testing.assert_allclose(first.sum(axis=1), 1.0, rtol=1e-5)


def test_execute_errors():
    layers = [8, 16, 4]
    g = model_graph(layers, "relu", 4)
    plan = build_execution_plan(g)
    b = Bound(mlp_values(layers, 4, 0))
    with pytest.raises(BackendError, match="the output holds 15 floats"):
        hip_value(g, plan, b, None, cap=15)
    with pytest.raises(BackendError, match="not computed by this graph"):
        hip_value(g, plan, b, 999)
    addr = dict(b.addr)
    addr["bias_16"] = 0
    lib = GraphLibrary(load_hip().lib)
    out = DeviceArray(np.zeros(64, F32))
    with pytest.raises(BackendError, match="is NULL"):
        lib.execute(g, plan, None, addr, out.ptr, 64)
    out.free()


def test_c5_shape_rows_against_oracle():
    """1024-4096-4096-1024-10 over 4096 rows (the 256x256 tile path), softmax
    at the end; the first 64 rows against the oracle on those rows."""
    layers = [1024, 4096, 4096, 1024, 10]
    rows = 4096
    say("C5-shaped graph, 4096 rows")
    vals = mlp_values(layers, rows, 9)
    g = model_graph(layers, "softmax", rows)
    plan = build_execution_plan(g)
    got = hip_value(g, plan, Bound(vals), None)
    assert got.shape == (rows, 10) and np.isfinite(got).all()
    sub = dict(vals)
    sub["input"] = vals["input"][:64]
    gs = model_graph(layers, "softmax", 64)
    want = oracle_value(gs, build_execution_plan(gs), Bound(sub), None)
    assert_close(got[:64], want, "C5 rows 0-63")


@pytest.mark.parametrize("layers,activation,rows", [([512, 1024, 1024, 512, 256, 1], "relu", 64),
                                                    ([64, 128, 128, 10], "softmax", 300),
                                                    ([1024, 256, 128, 8], "relu", 64)],
                         ids=["c2_relu_r64", "softmax_r300", "splitk_r64"])
def test_captured_replays_match_direct_launches(layers, activation, rows):
    """With VOLTA_RT_GRAPH=1 a call whose bindings and output repeat a
    recent call's runs as a replay of its launch sequence captured into a
    hipGraph.  Every replay equals, bit for bit, the same call launched
    layer by layer (the default), with direct launches, other values' calls
    and host synchronizations between the replays; a replay reads the
    bindings' current contents (new input values in the same buffer give
    the new values' result); more pointer sets than the program keeps
    graphs for still give the right values."""
    import os

    say(f"captured graph replays {layers} {activation} rows={rows}")
    lib = load_hip()
    gl = GraphLibrary(lib.lib)
    g = model_graph(layers, activation, rows)
    plan = build_execution_plan(g)
    vals = mlp_values(layers, rows, 21)
    b = Bound(vals)
    ncols = layers[-1]
    cap = rows * ncols
    out = DeviceArray(np.zeros(cap, F32))
    mid = DeviceArray(np.zeros(rows * layers[1], F32))
    bias0 = [i for i, op in chain_ids(g) if op == "add"][0]  # layer 0's bias sum [rows x L1]
    term = gl.prepare(g, plan, None, b.addr, out.ptr, cap)
    value1 = gl.prepare(g, plan, bias0, b.addr, mid.ptr, rows * layers[1])

    def direct(fn):
        old = os.environ.pop("VOLTA_RT_GRAPH", None)
        try:
            fn()
        finally:
            if old is not None:
                os.environ["VOLTA_RT_GRAPH"] = old

    direct(term)
    want = out.numpy().copy()
    direct(value1)
    want_mid = mid.numpy().copy()
    os.environ["VOLTA_RT_GRAPH"] = "1"
    r0 = lib.lib.volta_hip_rt_graph_replays()
    for k in range(4):
        term()
        np.testing.assert_array_equal(out.numpy(), want, err_msg=f"replay {k}")
        value1()  # another value of the program: its own sequence
        np.testing.assert_array_equal(mid.numpy(), want_mid, err_msg=f"value replay {k}")
        direct(term)
        np.testing.assert_array_equal(out.numpy(), want, err_msg=f"direct launch after replay {k}")
    assert lib.lib.volta_hip_rt_graph_replays() - r0 >= 6, "the repeated calls did not run as graph replays"
    # new input values in the same buffer
    x2 = np.random.default_rng(5).standard_normal((rows, layers[0])).astype(F32)
    assert lib.lib.volta_hip_copy(b.addr["input"], x2.ctypes.data, x2.nbytes, 1) == 0
    term()
    got2 = out.numpy().copy()
    direct(term)
    np.testing.assert_array_equal(got2, out.numpy())
    b2 = dict(vals)
    b2["input"] = x2
    assert_close(got2.reshape(rows, ncols), oracle_value(g, plan, Bound(b2), None), "replay on new input")
    # more output buffers than captured graphs kept per program
    outs = [DeviceArray(np.zeros(cap, F32)) for _ in range(10)]
    for rnd in range(2):
        for o in outs:
            c = gl.prepare(g, plan, None, b.addr, o.ptr, cap)
            c()
            c()
            np.testing.assert_array_equal(o.numpy(), got2, err_msg=f"eviction round {rnd}")
    os.environ.pop("VOLTA_RT_GRAPH", None)
    for d in outs + [out, mid]:
        d.free()
