"""Graph execution on the CPU: the oracle's interpreter (oracle/rt_graph.cpp)
pinned against the reference's own expected values and a float64 torch
forward, and the HIP library's compile step (lowering + plan cache,
include/volta_backend.h), which is host work and runs without a GPU."""
import ctypes as C
import os

import numpy as np
import pytest

from tests.oracle_lib import load_oracle
from volta_amd import HIP_LIB
from volta_amd.backend import (BackendError, ExecutionPlan, Graph, GraphLibrary, build_execution_plan,
                               lower_model_to_graph)

F32 = np.float32


def oracle_lib():
    return GraphLibrary(load_oracle().lib)


def run_oracle(graph, values, target=None, plan=None):
    """execute_value (target) / execute_terminal (None) on host arrays."""
    plan = plan or build_execution_plan(graph)
    arrs = {k: np.ascontiguousarray(v, F32) for k, v in values.items()}
    cap = 1 << 16
    out = np.zeros(cap, F32)
    r, c = oracle_lib().execute(graph, plan, target, {k: a.ctypes.data for k, a in arrs.items()},
                                out.ctypes.data, cap)
    return out[: r * c].reshape(r, c).copy()


def const_graph(shape, name="x"):
    g = Graph()
    x = g.add_op("input", name=name)
    g.bind_input_shape(name, shape)
    return g, x


# ---------------------------------------------------------------------------
# the reference's own expected values
def test_matmul_reference_values():
    """interpreter.rs:1880-1901 / tensor.rs:518-524: [[1,2],[3,4]] @ [[5,6],[7,8]]."""
    g, a = const_graph([2, 2], "a")
    b = g.add_op("input", name="b")
    g.bind_input_shape("b", [2, 2])
    g.add_op("matmul", a, b)
    out = run_oracle(g, {"a": [[1, 2], [3, 4]], "b": [[5, 6], [7, 8]]})
    np.testing.assert_array_equal(out, [[19, 22], [43, 50]])


def test_relu_reference_values():
    """interpreter.rs:1905-1928: [-2, -0.5, 1, 3.5] -> [0, 0, 1, 3.5]."""
    g, x = const_graph([4])
    g.add_op("relu", x)
    np.testing.assert_array_equal(run_oracle(g, {"x": [-2.0, -0.5, 1.0, 3.5]}), [[0, 0, 1, 3.5]])


def test_softmax_reference_values():
    """interpreter.rs:1931-1955: softmax([1, 2, 3]) sums to one; each entry is
    exp(k - 3) / sum, within fp32 rounding of the closed form."""
    g, x = const_graph([3])
    g.add_op("softmax", x)
    out = run_oracle(g, {"x": [1.0, 2.0, 3.0]})
    assert abs(float(out.sum()) - 1.0) < 1e-5
    e = np.exp(np.array([1.0, 2.0, 3.0]) - 3.0)
    np.testing.assert_allclose(out[0], e / e.sum(), rtol=3e-7)


@pytest.mark.parametrize("a_shape,a,b_shape,b,want_shape,want", [
    # tensor.rs:579-585 add_broadcast_extends_rank
    ([2, 3], [1, 2, 3, 4, 5, 6], [3], [10, 20, 30], (2, 3), [11, 22, 33, 14, 25, 36]),
    # tensor.rs:588-600 add_broadcast_two_sided
    ([3, 1], [1, 2, 3], [1, 4], [10, 20, 30, 40], (3, 4),
     [11, 21, 31, 41, 12, 22, 32, 42, 13, 23, 33, 43]),
    # tensor.rs:602-608 add_broadcast_scalar
    ([2, 2], [1, 2, 3, 4], [1], [5], (2, 2), [6, 7, 8, 9]),
])
def test_add_broadcast_reference_values(a_shape, a, b_shape, b, want_shape, want):
    g, x = const_graph(a_shape, "a")
    y = g.add_op("input", name="b")
    g.bind_input_shape("b", b_shape)
    g.add_op("add", x, y)
    out = run_oracle(g, {"a": a, "b": b})
    assert out.shape == want_shape
    np.testing.assert_array_equal(out.ravel(), want)


def test_gemm_vector_bias_reference_values():
    """tensor.rs:611-618 gemm_accepts_vector_bias_via_broadcast."""
    g, a = const_graph([2, 2], "a")
    b = g.add_op("input", name="b")
    bias = g.add_op("input", name="bias")
    g.bind_input_shape("b", [2, 3])
    g.bind_input_shape("bias", [3])
    g.add_op("gemm", a, b, bias, alpha=1.0, beta=1.0)
    out = run_oracle(g, {"a": [[1, 2], [3, 4]], "b": [[5, 6, 7], [8, 9, 10]], "bias": [1, 2, 3]})
    np.testing.assert_array_equal(out.ravel(), [22, 26, 30, 48, 56, 64])


def test_gemm_alpha_beta_scaling():
    """Tensor::gemm (tensor.rs:481-503): alpha * (a @ b) + beta * bias, and
    beta = 0 drops the bias."""
    g, a = const_graph([2, 2], "a")
    b = g.add_op("input", name="b")
    bias = g.add_op("input", name="bias")
    g.bind_input_shape("b", [2, 2])
    g.bind_input_shape("bias", [1, 2])
    g.add_op("gemm", a, b, bias, alpha=2.0, beta=0.5)
    vals = {"a": [[1, 2], [3, 4]], "b": [[5, 6], [7, 8]], "bias": [[2, 4]]}
    np.testing.assert_array_equal(run_oracle(g, vals), [[39, 46], [87, 102]])
    g.nodes[-1] = ("gemm", (a, b, bias), None, 1.0, 0.0)
    np.testing.assert_array_equal(run_oracle(g, vals), [[19, 22], [43, 50]])


def test_activations_closed_forms():
    """Sigmoid (both branches), tanh-GELU and ReLU against their closed forms
    in float64, within a few fp32 ulps; sigmoid(0) = 0.5 and gelu(0) = 0
    exactly; sigmoid(-x) = 1 - sigmoid(x) to rounding."""
    x = np.linspace(-12, 12, 97).astype(F32)
    for op, f in (("sigmoid", lambda v: 1 / (1 + np.exp(-v))),
                  ("gelu", lambda v: 0.5 * v * (1 + np.tanh(np.sqrt(2 / np.pi) * (v + 0.044715 * v ** 3)))),
                  ("relu", lambda v: np.maximum(v, 0))):
        g, xi = const_graph([1, x.size])
        g.add_op(op, xi)
        got = run_oracle(g, {"x": x[None, :]})[0].astype(np.float64)
        want = f(x.astype(np.float64))
        np.testing.assert_allclose(got, want, rtol=4e-7, atol=1e-7, err_msg=op)
    g, xi = const_graph([1, 3])
    g.add_op("sigmoid", xi)
    s = run_oracle(g, {"x": [[0.0, 3.0, -3.0]]})[0]
    assert s[0] == 0.5 and abs(float(s[1]) + float(s[2]) - 1.0) < 1e-7
    g, xi = const_graph([1, 1])
    g.add_op("gelu", xi)
    assert run_oracle(g, {"x": [[0.0]]})[0, 0] == 0.0


def mlp_values(layers, rows, seed):
    rng = np.random.default_rng(seed)
    vals = {"input": rng.standard_normal((rows, layers[0])).astype(F32)}
    for fi, fo in zip(layers[:-1], layers[1:]):
        vals[f"weight_{fi}_{fo}"] = rng.uniform(-1, 1, (fi, fo)).astype(F32) * F32(np.sqrt(6.0 / fi))
        vals[f"bias_{fo}"] = rng.uniform(-0.5, 0.5, (1, fo)).astype(F32)
    return vals


def model_graph(layers, activation, rows, final=True):
    """The inference graph the reference's executor builds (executor.rs:827-857)."""
    g = Graph()
    x = g.add_op("input", name="input")
    lower_model_to_graph(g, layers, activation, x, final)
    g.bind_input_shape("input", [rows, layers[0]])
    for fi, fo in zip(layers[:-1], layers[1:]):
        g.bind_parameter_shape(f"weight_{fi}_{fo}", [fi, fo])
        g.bind_parameter_shape(f"bias_{fo}", [1, fo])
    return g


def torch_forward(layers, activation, vals, final=True):
    import torch

    h = torch.tensor(vals["input"], dtype=torch.float64)
    for i, (fi, fo) in enumerate(zip(layers[:-1], layers[1:])):
        h = h @ torch.tensor(vals[f"weight_{fi}_{fo}"], dtype=torch.float64) + \
            torch.tensor(vals[f"bias_{fo}"], dtype=torch.float64)
        if i < len(layers) - 2:
            if activation == "relu":
                h = torch.relu(h)
            elif activation == "sigmoid":
                h = torch.sigmoid(h)
        elif final and activation == "softmax":
            h = torch.softmax(h, dim=1)
    return h.numpy()


@pytest.mark.parametrize("layers,activation,rows", [
    ([6, 10, 7, 3], "relu", 5), ([12, 16, 4], "sigmoid", 9), ([8, 8, 8, 5], "softmax", 4),
    ([5, 9, 2], "tanh", 3)])
def test_model_graph_matches_torch_fp64(layers, activation, rows):
    """The whole graph lower_model_to_graph builds, against torch in float64
    (independent matmul, activations and softmax); [8, 8, 8] shares the
    parameters weight_8_8 / bias_8 between two layers, as the reference's
    naming makes it."""
    vals = mlp_values(layers, rows, 3)
    g = model_graph(layers, activation, rows)
    got = run_oracle(g, vals)
    want = torch_forward(layers, activation, vals)
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-6)


def test_oracle_rejects_missing_binding_and_off_values():
    g = model_graph([4, 3, 2], "relu", 2)
    vals = mlp_values([4, 3, 2], 2, 0)
    del vals["bias_2"]
    with pytest.raises(BackendError):
        run_oracle(g, vals)
    with pytest.raises(BackendError, match="not computed"):
        run_oracle(model_graph([4, 3, 2], "relu", 2), mlp_values([4, 3, 2], 2, 0), target=999)


# ---------------------------------------------------------------------------
# the HIP library's compile step (host only)
needs_hip = pytest.mark.skipif(not os.path.exists(HIP_LIB), reason="libvolta_hip.so not built")


def hip_graphs():
    return GraphLibrary(C.CDLL(HIP_LIB))


@needs_hip
@pytest.mark.parametrize("activation", ["relu", "sigmoid", "softmax", "tanh"])
def test_hip_compile_accepts_model_graphs(activation):
    g = model_graph([16, 32, 24, 4], activation, 8)
    info = hip_graphs().compile(g, build_execution_plan(g))
    assert info["schedule_len"] == len(g.nodes) and info["fingerprint"] != 0


@needs_hip
def test_hip_compile_accepts_gemm_form():
    """The Gemm form of an MLP (train_api.rs:316-345)."""
    g = Graph()
    x = g.add_op("input", name="x")
    w1, b1 = g.add_op("parameter", name="w1"), g.add_op("parameter", name="b1")
    w2, b2 = g.add_op("parameter", name="w2"), g.add_op("parameter", name="b2")
    h = g.add_op("relu", g.add_op("gemm", x, w1, b1))
    g.add_op("output", g.add_op("gemm", h, w2, b2))
    for n, s in (("x", [4, 3]), ("w1", [3, 5]), ("b1", [1, 5]), ("w2", [5, 2]), ("b2", [2])):
        g.bind_input_shape(n, s)
    hip_graphs().compile(g, build_execution_plan(g))


def _rejects(g, match):
    with pytest.raises(BackendError, match=match):
        hip_graphs().compile(g, build_execution_plan(g))


@needs_hip
def test_hip_compile_rejections():
    # an op outside the subset (the MSE tail of a loss graph, lowering.rs:143-153)
    g = model_graph([4, 3, 2], "relu", 2)
    y = g.add_op("input", name="y")
    g.bind_input_shape("y", [2, 2])
    g.add_op("other", g.last_value_id(), y)
    _rejects(g, "not lowered")
    # shape mismatch, with the CUDA executor's wording (cuda/executor.rs:243-250)
    g = model_graph([4, 3, 2], "relu", 2)
    g.bind_parameter_shape("weight_3_2", [5, 2])
    _rejects(g, r"Shape mismatch in MatMul: lhs \[2, 3\] rhs \[5, 2\]")
    # a bias that is not [1, c]
    g = model_graph([4, 3, 2], "relu", 2)
    g.bind_parameter_shape("bias_3", [2, 3])
    _rejects(g, "the bias must be a bound")
    # a value consumed off the chain
    g = Graph()
    x = g.add_op("input", name="x")
    w = g.add_op("parameter", name="w")
    m = g.add_op("matmul", x, w)
    g.add_op("relu", m)
    g.add_op("sigmoid", m)
    g.bind_input_shape("x", [2, 4])
    g.bind_parameter_shape("w", [4, 4])
    _rejects(g, "activation is lowered only")
    # Gemm alpha other than 1
    g = Graph()
    x, w = g.add_op("input", name="x"), g.add_op("parameter", name="w")
    g.add_op("gemm", x, w, None, alpha=2.0)
    g.bind_input_shape("x", [2, 4])
    g.bind_parameter_shape("w", [4, 4])
    _rejects(g, "alpha other than 1")
    # a product of the softmax
    g = model_graph([4, 3], "softmax", 2)
    sm = g.last_value_id()
    w2 = g.add_op("parameter", name="w2")
    g.bind_parameter_shape("w2", [3, 3])
    g.add_op("matmul", sm, w2)
    _rejects(g, "Softmax output")


@needs_hip
def test_hip_plan_cache_reuses_compiled_program():
    """plan_cache.rs:66-96 and the CountingCompileBackend test
    (train.rs:1296-1316): the same key compiles once; clear_plan_cache, a new
    determinism level or new shapes compile again; the same fingerprints over
    different contents are compiled again instead of reusing the entry."""
    lib = hip_graphs()
    lib.clear_plan_cache()
    g = model_graph([16, 32, 4], "relu", 8)
    plan = build_execution_plan(g)
    n0 = lib.compile_count()
    first = lib.compile(g, plan)
    second = lib.compile(g, plan)
    assert first == second and lib.compile_count() == n0 + 1
    lib.compile(g, plan, determinism=1)
    assert lib.compile_count() == n0 + 2
    lib.clear_plan_cache()
    assert lib.compile(g, plan)["fingerprint"] == first["fingerprint"] and lib.compile_count() == n0 + 3
    g2 = model_graph([16, 32, 4], "relu", 16)
    assert lib.compile(g2, build_execution_plan(g2))["fingerprint"] != first["fingerprint"]
    assert lib.compile_count() == n0 + 4
    # a colliding key: other contents under plan's fingerprints
    g3 = model_graph([16, 32, 4], "sigmoid", 8)
    forged = ExecutionPlan(g3)
    forged.graph_fingerprint, forged.shape_signature_hash = plan.graph_fingerprint, plan.shape_signature_hash
    third = lib.compile(g3, forged)
    assert third["fingerprint"] != first["fingerprint"] and lib.compile_count() == n0 + 5
    plan_peak = ExecutionPlan(g, peak_bytes=4096)
    assert lib.compile(g, plan_peak)["peak_bytes"] == 4096
    with pytest.raises(BackendError, match="determinism"):
        lib.compile(g, plan, determinism=3)
