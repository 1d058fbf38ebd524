"""The allocation-free inference entry point (volta_train_infer_device_noalloc)
against volta_train_infer, through the C ABI: device input and output, the
forward's split-K partial planes in the library's static scratch.  Same
plans and kernels, so the outputs are bit-identical; two calls in a row, the
second with fewer rows, so the second reads scratch the first has left."""
import os
import sys

import numpy as np
import pytest

from volta_amd import DeviceArray, data, load_hip
from volta_amd.abi import MlpSpec, Trainer

pytestmark = pytest.mark.gpu

CASES = {
    # B=1024 (the forward runs 1024 rows at a time; on a 256-CU MI355X): at
    # 1024 and 976 rows fwd0 (N=1024, K=2048) runs its two K slices as K
    # groups of one workgroup (no scratch), fwd1 (N=512, K=1024) splits K in
    # 4 and the output layer (N=10, K=512) in 8, both through the scratch;
    # at 700 rows fwd0 splits in 2 as well.  test_splitk_case_reaches_scratch
    # asserts through the planner that each row count splits some layer.
    "splitk_b1024": (MlpSpec([2048, 1024, 512, 10], "relu", "sgd", "ce"), 1024, (2000, 700)),
    # B=64: small-M tiles, no split (the scratch is not touched); LayerNorm
    "smallm_ln_b64": (MlpSpec([512, 1024, 256, 1], "gelu", "adam", layernorm=True), 64, (130, 50)),
}


def _chunk_rows(rows, B):
    return [min(B, rows - r0) for r0 in range(0, rows, B)]


def test_splitk_case_reaches_scratch():
    """Every row count of the split-K case runs at least one forward layer
    with K split over workgroups (partial planes in the scratch), so the
    bit-equality below covers the scratch path whatever the planner picks."""
    from tests.test_planner import NN, plan

    spec, B, row_counts = CASES["splitk_b1024"]
    for rows in row_counts:
        for m in _chunk_rows(rows, B):
            splits = [plan(NN, m, c, r)[1] for r, c in spec.shapes()]
            assert max(splits) > 1, f"rows={rows}: no forward layer splits K at {m} rows ({splits})"


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("name", sorted(CASES))
def test_noalloc_infer_matches_infer(name):
    spec, B, row_counts = CASES[name]
    lib = load_hip()
    ws, bs = data.he_uniform(21, spec.sizes)
    t = Trainer(lib, spec, B)
    t.set_all_params(ws, bs)
    Ln = spec.sizes[-1]
    rng = np.random.default_rng(5)
    for rows in row_counts:
        say(f"noalloc {name}: rows={rows} B={B}")
        X = rng.standard_normal((rows, spec.sizes[0])).astype(np.float32)
        want = t.infer(X)
        dX = DeviceArray(X, lib)
        dO = DeviceArray(np.full((rows, Ln), np.nan, np.float32), lib)
        rc = lib.lib.volta_train_infer_device_noalloc(t.h, dX.ptr, rows, dO.ptr)
        assert rc == 0, lib.last_error()
        assert t.sync() == 0
        got = dO.numpy()
        np.testing.assert_array_equal(got, want)
        assert t.status() == 0
        dX.free()
        dO.free()
    t.close()


def test_noalloc_rejects_workspace_beyond_scratch():
    """With the split-K planner asked for 8 workgroups per CU and 128x128
    tiles from 2^20 outputs, a 1024x1024 product with K=4096 splits K 32
    ways (asserted through the planner): 32 x 1025 x 1024 floats of partial
    planes, above the 64 MiB scratch.  The call is refused on the host with
    a message naming both sizes; nothing is launched."""
    from tests.test_planner import NN, plan
    lib = load_hip()
    spec = MlpSpec([4096, 1024, 10], "relu", "sgd", "ce")
    env = {"VOLTA_SPLITK_WGS_PER_CU": "8", "VOLTA_TILE128_MIN_MN": str(1 << 20)}
    tile, splits = plan(NN, 1024, 1024, 4096, env=env)[:2]
    assert tile == 1 and splits == 32, (tile, splits)  # 128x128 tiles, K in 32 slices
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        t = Trainer(lib, spec, 1024)
        dX = DeviceArray(np.zeros((1024, 4096), np.float32), lib)
        dO = DeviceArray(np.zeros((1024, 10), np.float32), lib)
        rc = lib.lib.volta_train_infer_device_noalloc(t.h, dX.ptr, 1024, dO.ptr)
        msg = lib.last_error()
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    assert rc == -1
    assert "split-K workspace" in msg and str(16 << 22) in msg, msg
    t.clear_status()
    assert t.sync() == 0
    dX.free()
    dO.free()
    t.close()
