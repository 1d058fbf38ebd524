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
    # B=1024: fwd0 (1024x1024, K=2048) splits K in 4 on 128x128 tiles, fwd1
    # (1024x512, K=1024) in 2 on 64x64 tiles: both use the scratch
    "splitk_b1024": (MlpSpec([2048, 1024, 512, 10], "relu", "sgd", "ce"), 1024, (2000, 700)),
    # B=64: small-M tiles, no split (the scratch is not touched); LayerNorm
    "smallm_ln_b64": (MlpSpec([512, 1024, 256, 1], "gelu", "adam", layernorm=True), 64, (130, 50)),
}


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
    tiles from 2^20 outputs, a 1024x1024 product with K=4096 splits K 16
    ways: 16 x 1025 x 1024 floats of partial planes, above the 64 MiB
    scratch.  The call is refused on the host with a message naming both
    sizes; nothing is launched."""
    lib = load_hip()
    spec = MlpSpec([4096, 1024, 10], "relu", "sgd", "ce")
    env = {"VOLTA_SPLITK_WGS_PER_CU": "8", "VOLTA_TILE128_MIN_MN": str(1 << 20)}
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
