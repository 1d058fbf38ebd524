"""bench.py's host logic on the CPU: the algorithmic work model against the
hot-path survey's own per-config figures, the roofline arithmetic, the
choice of the dominant launch, and the split of a profiler's dispatch list
into whole steps."""
import math

import pytest

import bench

# (GFLOP, MB) per step, as the survey tabulates them for every BASELINE config
MODEL_STEP_FIGURES = {
    "c1": (0.185, 15.0), "c2": (0.789, 93.6), "c3": (2.282, 258.0), "c4_128": (1.577, 64.4),
    "c4_256": (3.155, 77.4), "c4_1024": (12.618, 155.3), "c5": (584.4, 2115),
}


@pytest.mark.parametrize("name", sorted(MODEL_STEP_FIGURES))
def test_step_model_matches_survey(name):
    spec, B, _ = bench.WORKLOADS[name]
    fl, by = bench.survey_step_cost(spec, B)
    gf, mb = MODEL_STEP_FIGURES[name]
    assert round(fl / 1e9, 3 if gf < 100 else 1) == gf
    assert round(by / 1e6, 1 if mb < 1000 else 0) == mb
    assert bench.gemm_flops(spec, B) == pytest.approx(fl, rel=1e-12)


def test_launch_labels_sum_to_the_step():
    """Every launch label of the C2 step (grouped dW, merged output launch)
    adds up to the whole-step model: nothing counted twice or dropped."""
    spec, B, _ = bench.WORKLOADS["c2"]
    labels = ["fwd0", "fwd1", "fwd2", "fwd3", "fwd4+loss+dx4", "dx3", "dx2", "dx1",
              "dw4+db+opt|dw3+db+opt|dw2+db+opt|dw1+db+opt|dw0+db+opt"]
    tot = [bench.survey_cost(spec, B, l) for l in labels]
    fl, by = bench.survey_step_cost(spec, B)
    assert sum(f for f, _ in tot) == pytest.approx(fl)
    assert sum(b for _, b in tot) == pytest.approx(by)
    # a split-K reduce carries nothing of its own
    assert bench.survey_cost(spec, B, "fwd1.splitk_reduce") == (0.0, 0.0)


def test_dw_term_by_hand():
    """dW_1 + db_1 + Adam of C2's 1024x1024 layer: 4(B r + B c + r c) +
    4(B c + c) + 4*7*(r c + c)."""
    spec, B, _ = bench.WORKLOADS["c2"]
    r = c = 1024
    want = 4 * (B * r + B * c + r * c) + 4 * (B * c + c) + 4 * 7 * (r * c + c)
    assert bench.survey_cost(spec, B, "dw1+db+opt") == (2.0 * B * r * c, float(want))


def test_roofline_bound_and_fraction():
    hbm = {"kernel": "x", "survey_flops": 1e6, "survey_bytes": 8e6, "bytes": 6e6, "ms": 0.002}
    r = bench.roofline_of(hbm)
    assert r["bound"] == "hbm" and r["achieved"] == pytest.approx(4000.0) and r["frac"] == pytest.approx(0.5)
    mf = {"kernel": "y", "survey_flops": 157.3e9, "survey_bytes": 1e6, "bytes": 1e6, "ms": 2.0}
    r = bench.roofline_of(mf)
    assert r["bound"] == "mfma" and r["frac"] == pytest.approx(0.5)
    assert bench.RIDGE == pytest.approx(157.3e12 / 8e12)


def test_dominant_launch_is_the_longest_measured():
    rows = [{"kernel": "a", "ms": 0.003}, {"kernel": "b", "ms": 0.011}, {"kernel": "c", "ms": 0.005}]
    assert max(rows, key=bench.dominance)["kernel"] == "b"


def test_per_launch_splits_whole_steps():
    """A primary workload of 3 launches and a secondary of 2 (its first a
    large-tile kernel), each run for whole steps after a warm-up fragment:
    values are grouped per step position from the end of each region."""
    def row(i, name, v):
        return {"Dispatch_Id": str(i), "Kernel_Name": f"void volta::{name}(args)", "Grid_Size_X": "256",
                "Workgroup_Size_X": "64", "Grid_Size_Y": "1", "v": v}

    seq = [("gemm_smallm<1>", 9.0)]  # a leftover fragment before the whole steps
    for s in range(3):
        seq += [("gemm_smallm<1>", 1.0 + s), ("out_layer_dx_kernel<1>", 2.0), ("dw_group_kernel<1>", 3.0)]
    for s in range(2):
        seq += [("gemm_big<true>", 10.0 + s), ("splitk_reduce<1>", 1.5)]
    rows = [row(i, n, v) for i, (n, v) in enumerate(seq)]
    labels = {"c2": ["fwd0", "fwd1+loss", "dw"], "c5": ["fwd0", "fwd0.splitk_reduce"]}
    out = bench._per_launch(rows, labels, lambda r: r["v"])
    assert [v for _, _, v in out["c2"]] == [[1.0, 2.0, 3.0], [2.0, 2.0, 2.0], [3.0, 3.0, 3.0]]
    assert [v for _, _, v in out["c5"]] == [[10.0, 11.0], [1.5, 1.5]]
    assert out["c5"][0][1] == 4  # workgroups from the grid


def test_gpu_count_other_than_one_is_refused(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU only" in capsys.readouterr().err
    assert math.isfinite(bench.PEAK_HBM_GBS)
