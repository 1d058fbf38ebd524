#!/usr/bin/env python3
"""Benchmark of the compile-train MLP step on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2] [--secondary c5]

Headline workload ("c2"): MLP 512-1024-1024-512-256-1,
ReLU hidden, linear output, MSE, Adam (lr 1e-3, b1 0.9, b2 0.999, eps 1e-8),
fp32, B=64, X,Y ~ N(0,1), He-uniform weights, zero biases, all from seed 42.
The same resident batch is used every step (inputs in HBM before timing), as
Volta's synthetic dataset is a single batch.  One "step" = forward, loss,
backward and optimizer update = the step's fixed launch sequence, enqueued
directly (the library's default; the graph_replay leg times the same
sequence replayed from its captured hipGraph).  The process sets no HIP or
HSA environment unless asked (--graph-dispatch nodes, --hsa-completion
polling): the figures are what a caller of the library gets.

Secondary workload (configs[4], "c5"): the wide classifier at B=4096, the
fp32-MFMA-bound case, reported in the same JSON line under "secondary".

The JSON line also carries:
  roofline      the dominant kernel of the headline step: algorithmic bytes or
                flops per launch / its average duration, timed with HIP events
                on the handle's stream (kernel-by-kernel replay of the step);
  cpu_baseline  the CPU oracle (C++ restatement of Volta's compile-train step,
                OpenMP GEMMs) on this host's cores, on a bounded sample;
  runtime_optimizer  the runtime optimizer (Backend::apply_gradients path,
                include/volta_backend.h) over C5's parameter tensors, Adam;
  graph_execution    the runtime's inference graph of the C5 and C2 models
                through Backend::execute_terminal (include/volta_backend.h);
  extras_path   the codegen extras' launch structure on the C2 topology.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

from volta_amd import data, load_hip  # noqa: E402
from volta_amd.abi import MlpSpec, Trainer  # noqa: E402

METRIC = "ms/train-step (samples/s) MLP at B=64 and B=4096; % fp32 MFMA peak"
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
RIDGE = PEAK_FP32_MFMA_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)  # flop/byte

WORKLOADS = {
    "c1": (MlpSpec([256, 512, 512, 256, 1], "relu", "sgd"), 64, 0.01),
    "c2": (MlpSpec([512, 1024, 1024, 512, 256, 1], "relu", "adam"), 64, 1e-3),
    "c3": (MlpSpec([512, 2048, 2048, 512, 1], "gelu", "adamw"), 64, 1e-3),
    "c4_128": (MlpSpec([512, 1024, 1024, 512, 256, 1], "silu", "sgd"), 128, 0.01),
    "c4_256": (MlpSpec([512, 1024, 1024, 512, 256, 1], "silu", "sgd"), 256, 0.01),
    "c4_1024": (MlpSpec([512, 1024, 1024, 512, 256, 1], "silu", "sgd"), 1024, 0.01),
    "c5": (MlpSpec([1024, 4096, 4096, 1024, 10], "relu", "adagrad", "ce", eps=1e-10), 4096, 1e-2),
    # the codegen extras on the headline topology, as the reference's own
    # benchmark scripts set them (examples/bench_layernorm.vt,
    # bench_dropout.vt: SGD, lr 0.01, B=64), and all three together
    "x_layernorm": (MlpSpec([512, 1024, 1024, 512, 256, 1], "relu", "sgd", layernorm=True), 64, 0.01),
    "x_dropout": (MlpSpec([512, 1024, 1024, 512, 256, 1], "relu", "sgd", dropout_p=0.2), 64, 0.01),
    "x_all": (MlpSpec([512, 1024, 1024, 512, 256, 1], "relu", "adam", layernorm=True, dropout_p=0.2,
                      clip_grad=1.0), 64, 1e-3),
}
EXTRAS_WORKLOADS = ("x_layernorm", "x_dropout", "x_all")

# Reference's own published CPU figure for the headline topology with Adam
# (docs/BENCHMARKS.md:87; 6-core x86, MKL; different input pattern).
PUBLISHED_CPU = {"c2": {"ms_per_step": 4.259, "source": "docs/BENCHMARKS.md:87",
                        "hardware": "Windows 11, 6-core x86-64 CPU, MKL"}}


def _env_on(name: str) -> bool:
    """The library's reading of a switch variable: set, non-empty, not '0'."""
    v = os.environ.get(name, "")
    return bool(v) and not v.startswith("0")


def gemm_flops(spec: MlpSpec, B: int) -> float:
    """2B*sumW (fwd) + 2B*sumW (dW) + 2B*(sumW - L0*L1) (dX, none for layer 0)."""
    sw = sum(r * c for r, c in spec.shapes())
    l0l1 = spec.sizes[0] * spec.sizes[1]
    return 2.0 * B * sw * 2 + 2.0 * B * (sw - l0l1)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def launches(lib, t):
    """The step's launch sequence: label and algorithmic flops/bytes of each
    launch (volta_hip_profile_step, one kernel-by-kernel replay)."""
    fn = lib.lib.volta_hip_profile_step
    fn.restype = C.c_int32
    fn.argtypes = [C.c_void_p, C.c_int32, C.c_char_p, C.c_int32]
    buf = C.create_string_buffer(1 << 16)
    n = fn(t.h, 1, buf, len(buf))
    if n <= 0:
        raise RuntimeError("volta_hip_profile_step failed: " + lib.last_error())
    rows = []
    for line in buf.value.decode().strip().splitlines():
        label, ms, fl, by = line.split("\t")
        rows.append({"kernel": label, "flops": float(fl), "bytes": float(by)})
    return rows


def profile(lib, t, step_ms, spec, B):
    """Per-launch duration inside whole steps (time_in_step for every launch);
    about 0.4 s of steps per launch, 3..50 repetitions.  Each row carries the
    launch's fused-kernel flops/bytes from the library and the survey-model
    flops/bytes (survey_cost)."""
    rows = launches(lib, t)
    for r in rows:
        r["survey_flops"], r["survey_bytes"] = survey_cost(spec, B, r["kernel"])
    reps = int(max(3, min(50, 200.0 / max(step_ms, 1e-3))))
    for i, r in enumerate(rows):
        ms, bracket, marker, label = time_in_step(lib, t, i, reps)
        if label != r["kernel"]:
            raise RuntimeError(f"launch order mismatch: {label} vs {r['kernel']}")
        r["ms"] = ms
        r["bracket_ms"] = round(bracket, 5)
        r["marker_ms"] = round(marker, 5)
    return rows


def time_in_step(lib, t, index, reps=50):
    """Duration of launch `index` inside whole steps: HIP events on the
    library's stream around that launch only (the other launches run back to
    back), minus the same two events recorded back to back at that position
    (the markers' own cost).  Returns (ms, bracket_ms, marker_ms, label)."""
    avg = (C.c_float * 2)()
    lab = C.create_string_buffer(128)
    if lib.lib.volta_hip_time_kernel(t.h, index, reps, avg, lab, len(lab)) != 0:
        raise RuntimeError("volta_hip_time_kernel failed: " + lib.last_error())
    return max(avg[0] - avg[1], 0.0), float(avg[0]), float(avg[1]), lab.value.decode()


OPT_STATE_STREAMS = {"sgd": 3, "adagrad": 5, "adam": 7, "adamw": 7}


def survey_cost(spec: MlpSpec, B: int, label: str):
    """Algorithmic (flops, bytes) of one launch by the unfused-kernel model of
    the hot-path survey, from the launch's label (parts joined by '|' and
    '+'): per layer i (r = L[i], c = L[i+1]) fwd 4(B r + r c + B c (2 if
    hidden else 1)), dW 4(B r + B c + r c), dX (i > 0) 4(B c + r c + 2 B r),
    db 4(B c + c), optimizer 4 s (r c + c) with s = 3 (SGD), 5 (Adagrad), 7
    (Adam/AdamW); flops 2 B r c per product; loss terms and the split-K
    reduce launches carry none (the product's launch carries its bytes)."""
    import re

    if label.endswith(".splitk_reduce"):
        return 0.0, 0.0
    n = spec.n_layers
    s_opt = OPT_STATE_STREAMS[spec.optimizer]
    flops = nbytes = 0.0
    for half in label.split("|"):
        parts = half.split("+")
        for part in parts:
            m = re.fullmatch(r"(fwd|dx|dw)(\d+)", part)
            if not m:
                continue
            kind, i = m.group(1), int(m.group(2))
            r, c = spec.sizes[i], spec.sizes[i + 1]
            flops += 2.0 * B * r * c
            if kind == "fwd":
                nbytes += 4.0 * (B * r + r * c + B * c * (2 if i < n - 1 else 1))
            elif kind == "dx":
                nbytes += 4.0 * (B * c + r * c + 2 * B * r)
            else:
                nbytes += 4.0 * (B * r + B * c + r * c)
                if "db" in parts:
                    nbytes += 4.0 * (B * c + c)
                if "opt" in parts:
                    nbytes += 4.0 * s_opt * (r * c + c)
    return flops, nbytes


def survey_step_cost(spec: MlpSpec, B: int):
    """(flops, bytes) of the whole step by the same model."""
    n = spec.n_layers
    labels = [f"fwd{i}" for i in range(n)] + [f"dx{i}" for i in range(1, n)]
    labels += [f"dw{i}+db+opt" for i in range(n)]
    tot = [survey_cost(spec, B, lab) for lab in labels]
    return sum(f for f, _ in tot), sum(b for _, b in tot)


def roofline_of(row):
    """Roofline fraction of one launch from its survey-model flops and bytes
    and its measured in-step duration; the launch's own fused-kernel byte
    count (what it must move once fused) is kept beside it."""
    fl, by = row["survey_flops"], row["survey_bytes"]
    ai = fl / by if by > 0 else math.inf
    sec = row["ms"] * 1e-3
    base = {"kernel": row["kernel"], "traffic": None, "avg_ms": round(row["ms"], 5),
            "algorithmic_flops": fl, "algorithmic_bytes": by, "fused_model_bytes": row["bytes"],
            "model": "hot-path survey unfused-kernel bytes (fwd, dW, dX, db, optimizer 4 s P)"}
    if ai > RIDGE:
        ach = fl / sec / 1e12
        return {**base, "bound": "mfma", "achieved": round(ach, 3), "peak": PEAK_FP32_MFMA_TFLOPS,
                "unit": "TFLOP/s", "frac": round(ach / PEAK_FP32_MFMA_TFLOPS, 4)}
    ach = by / sec / 1e9
    return {**base, "bound": "hbm", "achieved": round(ach, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(ach / PEAK_HBM_GBS, 4)}


def dominance(row):
    """The dominant launch of a step: the longest measured in-step duration."""
    return row["ms"]


PROFILES = os.path.join(ROOT, "profiles")


def committed_trace_us(workload, label):
    """Traced average duration (us) of launch `label` in the committed
    rocprofv3 kernel-trace summary profiles/kernel_trace_<workload>.txt, or
    None."""
    path = os.path.join(PROFILES, f"kernel_trace_{workload}.txt")
    try:
        lines = open(path).read().splitlines()
    except OSError:
        return None
    for line in lines:
        f = line.split()
        if len(f) >= 4 and not line.startswith("#") and f[3] == label:
            try:
                return float(f[0])
            except ValueError:
                continue
    return None


def committed_mfma(workload, label):
    """The committed MFMA counter figures of launch `label`
    (profiles/mfma_counters.txt): {"counted_flops", "algorithmic_flops",
    "busy_frac"}, or None."""
    try:
        lines = open(os.path.join(PROFILES, "mfma_counters.txt")).read().splitlines()
    except OSError:
        return None
    for line in lines:
        f = line.split("\t")
        if len(f) >= 5 and not line.startswith("#") and f[0] == workload and f[1] == label:
            return {"counted_flops": float(f[2]), "algorithmic_flops": float(f[3]), "busy_frac": float(f[4])}
    return None


def add_committed_fractions(workload, rf):
    """Beside the roofline's in-step fraction: the fraction on the launch's
    own fused bytes (hbm-bound launches), on the traced average of the
    committed kernel trace, and from the committed MFMA counters (mfma-bound
    launches: the MFMA flops the hardware counted over the in-step time, and
    the fraction of cycles the MFMA pipes were busy)."""
    sec = rf["avg_ms"] * 1e-3
    if rf["bound"] == "hbm":
        rf["frac_fused_bytes"] = round(rf["fused_model_bytes"] / sec / 1e9 / PEAK_HBM_GBS, 4)
    t_us = committed_trace_us(workload, rf["kernel"])
    if t_us:
        work = rf["algorithmic_bytes"] / 1e9 / PEAK_HBM_GBS if rf["bound"] == "hbm" else \
            rf["algorithmic_flops"] / 1e12 / PEAK_FP32_MFMA_TFLOPS
        rf["trace_avg_ms"] = round(t_us * 1e-3, 5)
        rf["frac_trace"] = round(work / (t_us * 1e-6), 4)
        rf["trace_source"] = f"profiles/kernel_trace_{workload}.txt"
    if rf["bound"] == "mfma":
        m = committed_mfma(workload, rf["kernel"])
        if m:
            rf["mfma_counted_flops"] = m["counted_flops"]
            rf["frac_mfma_counters"] = round(m["counted_flops"] / sec / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4)
            rf["mfma_busy_frac"] = m["busy_frac"]
            rf["mfma_source"] = "profiles/mfma_counters.txt"
    return rf


def run_gpu(name, steps, warmup, want_profile=True, count_launches=False):
    spec, B, lr = WORKLOADS[name]
    lib = load_hip()
    ws, bs = data.he_uniform(42, spec.sizes)
    X, Y = data.batch(42, spec.sizes, B, spec.loss)
    t = Trainer(lib, spec, B)
    t.set_all_params(ws, bs)
    t.step(X, Y, lr)  # stages X/Y into the handle's resident buffers
    xp, yp = t.batch_buffers()
    for _ in range(warmup):
        if t.step_device(xp, yp, lr) != 0:
            raise RuntimeError(lib.last_error())
    t.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        t.step_device(xp, yp, lr)
    t.sync()
    t1 = time.perf_counter()
    loss = t.loss()
    status = t.status()
    if status != 0 or not math.isfinite(loss):
        raise RuntimeError(f"{name}: bad step status {status}, loss {loss}")
    ms = (t1 - t0) / steps * 1e3
    out = {"ms_per_step": ms, "samples_per_s": B / (ms * 1e-3), "loss_after": loss,
           "gemm_gflop_per_step": gemm_flops(spec, B) / 1e9}
    # The reference ABI hands over host buffers: the same steps through
    # volta_train_step(host X, Y) (staged via pinned memory, PCIe included).
    # Reported beside the resident-input rate, never as the value.
    hs = max(3, min(steps, int(steps * 0.25)))
    t.sync()
    h0 = time.perf_counter()
    for _ in range(hs):
        t.step(X, Y, lr)
    t.sync()
    out["host_staged_ms_per_step"] = round((time.perf_counter() - h0) / hs * 1e3, 5)
    out["mfma_frac_step"] = gemm_flops(spec, B) / (ms * 1e-3) / (PEAK_FP32_MFMA_TFLOPS * 1e12)
    extra = lib.lib.volta_hip_arena_bytes
    extra.restype = C.c_int64
    extra.argtypes = [C.c_void_p]
    out["arena_bytes"] = int(extra(t.h))
    if count_launches:
        out["launches"] = len(launches(lib, t))
    if want_profile:
        rows = profile(lib, t, ms, spec, B)
        out["kernels"] = rows
        out["roofline"] = add_committed_fractions(name, roofline_of(max(rows, key=dominance)))
        tr = measured_traffic(name, out["roofline"]["kernel"])
        if tr:
            out["roofline"]["traffic"] = tr["bytes"]
            out["roofline"]["traffic_detail"] = tr
        out["kernel_sum_ms"] = sum(r["ms"] for r in rows)
    t.close()
    return spec, B, lr, out


def run_rt_optimizer(name="c5", kind="adam", reps=20):
    """The runtime optimizer (volta_rt_apply_gradients, Backend::apply_gradients
    of the reference's runtime) over the parameter tensors of a workload:
    one multi-tensor launch per call; HBM-bound, 28 bytes per element for
    Adam (p, m, v read and written, g read)."""
    from volta_amd import DeviceArray
    from volta_amd.backend import RtOptimizer, config

    spec, _, _ = WORKLOADS[name]
    lib = load_hip()
    rng = np.random.default_rng(1)
    counts = []
    for r, c in spec.shapes():
        counts += [r * c, c]
    params = [DeviceArray(rng.standard_normal(n).astype(np.float32), lib) for n in counts]
    grads = [DeviceArray((rng.standard_normal(n) * 0.01).astype(np.float32), lib) for n in counts]
    opt = RtOptimizer(lib.lib, counts)
    cfg = config(kind, 1e-3)
    pp, gp = [d.ptr for d in params], [d.ptr for d in grads]
    opt.apply(cfg, pp, gp)  # state allocation, warm-up
    t0 = time.perf_counter()
    for _ in range(reps):
        opt.apply(cfg, pp, gp)
    dt = (time.perf_counter() - t0) / reps
    n = sum(counts)
    nbytes = {"sgd": 12, "adagrad": 20, "adam": 28, "adamw": 28}[kind] * n
    out = {"workload": name, "optimizer": kind, "tensors": len(counts), "elements": n,
           "ms_per_call": round(dt * 1e3, 4), "algorithmic_bytes": nbytes,
           "achieved_GBs": round(nbytes / dt / 1e9, 1), "frac_hbm": round(nbytes / dt / 1e9 / PEAK_HBM_GBS, 4),
           "note": "synchronous call: one multi-tensor launch plus a descriptor upload and a stream synchronize"}
    opt.close()
    for d in params + grads:
        d.free()
    return out


def run_rt_graph(name="c5", rows=4096, reps=20):
    """Graph execution (volta_rt_execute_terminal, Backend::execute_terminal
    of the reference's runtime) of the inference graph the reference's
    executor builds for a workload's model (lower_model_to_graph,
    executor.rs:827-857) over `rows` resident input rows: one GEMM launch per
    layer (bias + activation in the epilogue) and a synchronize per call."""
    from volta_amd import DeviceArray
    from volta_amd.backend import Graph, GraphLibrary, build_execution_plan, lower_model_to_graph

    spec, _, _ = WORKLOADS[name]
    lib = load_hip()
    g = Graph()
    x = g.add_op("input", name="input")
    lower_model_to_graph(g, spec.sizes, spec.activation, x, True)
    g.bind_input_shape("input", [rows, spec.sizes[0]])
    rng = np.random.default_rng(3)
    vals = {"input": rng.standard_normal((rows, spec.sizes[0])).astype(np.float32)}
    for r, c in spec.shapes():
        g.bind_parameter_shape(f"weight_{r}_{c}", [r, c])
        g.bind_parameter_shape(f"bias_{c}", [1, c])
        vals[f"weight_{r}_{c}"] = (rng.uniform(-1, 1, (r, c)) * np.sqrt(6.0 / r)).astype(np.float32)
        vals[f"bias_{c}"] = np.zeros((1, c), np.float32)
    plan = build_execution_plan(g)
    dev = {k: DeviceArray(v, lib) for k, v in vals.items()}
    cap = rows * spec.sizes[-1]
    out = DeviceArray(np.zeros(cap, np.float32), lib)
    gl = GraphLibrary(lib.lib)
    addr = {k: d.ptr for k, d in dev.items()}
    call = gl.prepare(g, plan, None, addr, out.ptr, cap)

    def per_call(fn, n):
        fn()
        fn()  # compile + device state; the second call with the same pointers captures the graph
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        return (time.perf_counter() - t0) / n

    dt = per_call(call, reps)
    os.environ["VOLTA_RT_GRAPH"] = "1"
    try:
        dt_graph = per_call(call, reps)
    finally:
        os.environ.pop("VOLTA_RT_GRAPH", None)
    dt_tables = per_call(lambda: gl.execute(g, plan, None, addr, out.ptr, cap), reps)
    flops = sum(2.0 * rows * r * c for r, c in spec.shapes())
    res = {"workload": name, "rows": rows, "layers": list(spec.sizes), "activation": spec.activation,
           "ms_per_call": round(dt * 1e3, 4), "samples_per_s": round(rows / dt, 1),
           "tflops": round(flops / dt / 1e12, 2), "frac_mfma": round(flops / dt / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
           "ms_per_call_graph_replay": round(dt_graph * 1e3, 4),
           "ms_per_call_tables_rebuilt_in_python": round(dt_tables * 1e3, 4),
           "note": "synchronous execute_terminal with the caller's tables built once (plan-cache lookup, one "
                   "launch per layer, stream synchronize); beside it the same call replaying the launch "
                   "sequence captured as a hipGraph (VOLTA_RT_GRAPH=1) and with the tables rebuilt in Python "
                   "each call"}
    for d in list(dev.values()) + [out]:
        d.free()
    return res


def run_default_runtime_leg(name, steps, warmup):
    """The headline workload timed in a child process that runs with HIP's
    default graph dispatch (recorded packets) and the HSA runtime's default
    completion waits (interrupts): what a caller of the library that sets no
    environment gets, resident and host-staged.  Started before this
    process's first HIP call."""
    import subprocess

    env = dict(os.environ)
    env.pop("DEBUG_CLR_GRAPH_PACKET_CAPTURE", None)
    env.pop("HSA_ENABLE_INTERRUPT", None)
    cmd = [sys.executable, os.path.abspath(__file__), "--config", name, "--secondary", "none", "--no-cpu",
           "--no-profile", "--configs", "none", "--no-default-runtime-leg", "--graph-dispatch", "packets",
           "--hsa-completion", "interrupts", "--steps", str(steps), "--warmup", str(warmup)]
    r = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=600)
    if r.returncode != 0:
        raise RuntimeError(f"default-runtime leg failed ({r.returncode}): {r.stderr[-2000:]}")
    j = json.loads([ln for ln in r.stdout.splitlines() if ln.startswith("{")][-1])
    return {"workload": name, "ms_per_step": j["ms_per_step"], "samples_per_s": j["value"],
            "host_staged_ms_per_step": j["host_staged_ms_per_step"], "graph_dispatch": "packets (HIP default)",
            "hsa_completion": "interrupts (HSA default)", "steps": steps,
            "note": "child process with neither DEBUG_CLR_GRAPH_PACKET_CAPTURE nor HSA_ENABLE_INTERRUPT set"}


CPU_REF_SO = os.path.join(ROOT, "oracle", "_ref", "libvolta_cpu_ref.so")


def host_cpu():
    """This host's CPU: model name, logical CPUs, physical cores (lscpu-style
    count of distinct (package, core) pairs in /proc/cpuinfo)."""
    model, cores, phys, cur = "unknown", set(), None, {}
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name":
                model = v
            elif k in ("physical id", "core id"):
                cur[k] = v
            elif not k and cur:
                cores.add((cur.get("physical id"), cur.get("core id")))
                cur = {}
        if cur:
            cores.add((cur.get("physical id"), cur.get("core id")))
        phys = len(cores) or None
    except OSError:
        pass
    return {"model": model, "logical_cpus": os.cpu_count(), "physical_cores": phys,
            "affinity_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None}


def _cpu_leg(lib, name, threads, warmup, runs, steps_per_run):
    """Time one CPU library on workload `name` at `threads` OpenMP threads:
    `warmup` untimed steps, then `runs` runs of `steps_per_run` steps; the
    per-step time of each run, and their median (the reference's protocol,
    docs/BENCHMARKS.md:11-24: 10 warm-up steps, 7 runs of 50 steps, median)."""
    spec, B, lr = WORKLOADS[name]
    lib.lib.volta_oracle_set_threads(threads)
    ws, bs = data.he_uniform(42, spec.sizes)
    X, Y = data.batch(42, spec.sizes, B, spec.loss)
    t = Trainer(lib, spec, B)
    t.set_all_params(ws, bs)
    for _ in range(warmup):
        t.step(X, Y, lr)
    per = []
    for _ in range(runs):
        t0 = time.perf_counter()
        for _ in range(steps_per_run):
            t.step(X, Y, lr)
        per.append((time.perf_counter() - t0) / steps_per_run)
    t.close()
    med = float(np.median(per))
    return {"value": round(B / med, 2), "unit": "samples/s", "ms_per_step": round(med * 1e3, 3),
            "cores": threads, "runs_ms": [round(x * 1e3, 3) for x in per]}


def run_cpu(name, threads_all, full_protocol=True):
    """CPU baseline legs on this host, rank 0 only.  Leg "port": the oracle
    (oracle/liboracle_volta.so, the C++ restatement of Volta's compile-train
    step: ascending-k OpenMP GEMMs, Adam over 8192-element chunks in parallel
    as the reference's Rayon loop) at all threads and at 6 threads (the
    reference's published machine).  Leg "port+ref_gemm": the same step with
    every fp32 GEMM done by the reference's own C GEMM (gemm_shim.c, compiled
    from its source into oracle/_ref/; single-threaded, the reference's build
    without an OpenMP runtime) -- only where that build is present.  Protocol:
    10 warm-up steps, 7 x 50 steps, median; a bounded sample for workloads
    whose steps take seconds (stated in `sample`).  Returns (primary, legs)."""
    from tests.oracle_lib import load_oracle
    from volta_amd.abi import TrainLibrary

    spec, B, lr = WORKLOADS[name]
    proto = (10, 7, 50) if full_protocol else (1, 3, 1)
    what = ("10 warm-up steps, 7 runs x 50 steps, median run" if full_protocol else
            "bounded sample: 1 warm-up step, 3 runs x 1 step, median run")
    legs = []
    orc = load_oracle()
    for th in sorted({threads_all, 6}, reverse=True) if full_protocol else [threads_all]:
        r = _cpu_leg(orc, name, th, *proto)
        r.update(kind="port", sample=f"workload {name} (B={B}), {what}; oracle/liboracle_volta.so "
                                     f"(C++ restatement of Volta compile-train), {th} threads")
        legs.append(r)
        log(f"cpu baseline leg: {r}")
    if full_protocol and os.path.exists(CPU_REF_SO):
        from tests.oracle_lib import ORACLE_EXTRA

        ref = TrainLibrary(CPU_REF_SO, extra=ORACLE_EXTRA)
        r = _cpu_leg(ref, name, threads_all, 2, 7, 5)
        r.update(kind="port+ref_gemm",
                 sample=f"workload {name} (B={B}), bounded sample: 2 warm-up steps, 7 runs x 5 steps, median run; "
                        f"oracle/_ref/libvolta_cpu_ref.so: the restatement's step "
                        f"with the reference's own gemm_shim.c GEMMs (single-threaded), "
                        f"{threads_all} threads elsewhere")
        legs.append(r)
        log(f"cpu baseline leg: {r}")
    primary = dict(legs[0])
    primary.pop("runs_ms", None)
    return primary, legs


def calibration_copy(mib, reps=10):
    """A copy kernel over a known byte count, for scaling FETCH_SIZE and
    WRITE_SIZE: each dispatch reads and writes exactly mib MiB."""
    lib = load_hip()
    n = mib << 20
    f = lib.lib
    src, dst = f.volta_hip_device_alloc(n), f.volta_hip_device_alloc(n)
    if not src or not dst:
        raise RuntimeError("device allocation failed")
    try:
        if f.volta_hip_calibration_copy(dst, src, n, reps) != 0:
            raise RuntimeError("calibration copy failed")
    finally:
        f.volta_hip_device_free(src)
        f.volta_hip_device_free(dst)
    log(f"calibration copy: {reps} dispatches of {mib} MiB read + {mib} MiB written")
    return 0


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.txt")


def measured_traffic(workload, label):
    """HBM bytes per launch of `label` from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy calibration), or None."""
    try:
        lines = open(TRAFFIC_FILE).read().splitlines()
    except OSError:
        return None
    for line in lines:
        if line.startswith("#") or not line.strip():
            continue
        f = line.split("\t")
        if len(f) >= 4 and f[0] == workload and f[1] == label:
            return {"bytes": float(f[2]) + float(f[3]), "fetch": float(f[2]), "write": float(f[3]),
                    "source": "profiles/hbm_traffic.txt"}
    return None


def _bench_labels(bench_json):
    """Launch labels per workload, in launch order, from a bench JSON line."""
    for line in open(bench_json):
        if line.startswith("{"):
            b = json.loads(line)
    labels = {b["config"]["workload"]: [k["kernel"] for k in b["kernels"]]}
    if b.get("secondary"):
        labels[b["secondary"]["workload"]] = [k["kernel"] for k in b["secondary"]["kernels"]]
    return b, labels


def _per_launch(rows, labels, value):
    """Split a profiler's dispatch rows (one bench process: primary workload,
    then secondary) into whole steps and map each step position to its launch
    label.  Returns {workload: [(kernel, workgroups, [values...]) per launch]}
    over every whole step of that workload."""
    import re

    seq = []
    for r in sorted(rows, key=lambda r: int(r["Dispatch_Id"])):
        if "__amd_rocclr" in r["Kernel_Name"] or "::rt_" in r["Kernel_Name"]:
            continue  # runtime copies/fills; the runtime optimizer's own measurement
        nm = re.sub(r"\(.*", "", r["Kernel_Name"].replace("volta::", "").replace("void ", ""))
        v = value(r)
        if nm.startswith("loss_finish_kernel") and seq:  # second kernel of the output-layer launch
            seq[-1][2] += v
            continue
        if "Grid_Size" in r:  # counter collection: total threads
            wg = int(r["Grid_Size"]) // int(r["Workgroup_Size"])
        else:  # kernel trace: per dimension
            wg = int(r["Grid_Size_X"]) // int(r["Workgroup_Size_X"]) * int(r["Grid_Size_Y"])
        seq.append([nm, wg, v])
    order = list(labels)
    regions = [seq]
    if len(order) > 1:  # the secondary's first launch is a large-tile kernel (B=4096)
        i2 = next(i for i, x in enumerate(seq) if "gemm_big" in x[0] or "128, 128" in x[0])
        regions = [seq[:i2], seq[i2:]]
    out = {}
    for wl, reg in zip(order, regions):
        n = len(labels[wl])
        reg = reg[len(reg) - (len(reg) // n) * n:]
        steps = [reg[k * n:(k + 1) * n] for k in range(len(reg) // n)]
        out[wl] = [(steps[-1][p][0], steps[-1][p][1], [s[p][2] for s in steps]) for p in range(n)]
    return out


def traffic_table(pmc_dir, bench_json):
    """Text table of HBM bytes per launch from four rocprofv3 --pmc passes
    (FETCH_SIZE and WRITE_SIZE over `--calibration-copy 256` into
    pmc_dir/cal_<COUNTER>/ and over `--no-cpu --no-profile` into
    pmc_dir/bench_<COUNTER>/), each counter scaled by what it reads for the
    copy's known 256 MiB; launches are named from a bench JSON line of the
    same build (same launch order); averages over the last 10 steps."""
    import csv

    cal = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        rows = [r for r in csv.DictReader(open(f"{pmc_dir}/cal_{c}/cal_counter_collection.csv"))
                if "calibration_copy" in r["Kernel_Name"]]
        cal[c] = 256 * 1024 / (sum(float(r["Counter_Value"]) for r in rows) / len(rows))
    _, labels = _bench_labels(bench_json)
    per = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        rows = list(csv.DictReader(open(f"{pmc_dir}/bench_{c}/bench_counter_collection.csv")))
        for wl, lst in _per_launch(rows, labels, lambda r, c=c: float(r["Counter_Value"]) * 1024 * cal[c]).items():
            per[(wl, c)] = [(k, w, sum(v[-10:]) / len(v[-10:])) for k, w, v in lst]
    out = [f"# calibration (plain copy, 256 MiB read and written per dispatch): "
           f"FETCH_SIZE x{cal['FETCH_SIZE']:.3f}, WRITE_SIZE x{cal['WRITE_SIZE']:.3f}",
           "# workload\tlaunch\tfetch_bytes\twrite_bytes\tkernel (workgroups)"]
    for wl in labels:
        for p, lab in enumerate(labels[wl]):
            f, w = per[(wl, "FETCH_SIZE")][p], per[(wl, "WRITE_SIZE")][p]
            out.append(f"{wl}\t{lab}\t{f[2]:.0f}\t{w[2]:.0f}\t{f[0]} ({f[1]})")
    print("\n".join(out))
    return 0


MI355X_XCDS = 8  # GRBM_GUI_ACTIVE as rocprofv3 reports it: summed over the 8 XCDs
MI355X_CUS = 256


def mfma_table(pmc_csv, bench_json):
    """Text table of MFMA work per launch from one rocprofv3 --pmc pass with
    SQ_INSTS_VALU_MFMA_MOPS_F32, SQ_VALU_MFMA_BUSY_CYCLES and GRBM_GUI_ACTIVE
    over `--no-cpu --no-profile` (launches named from a bench JSON line of
    the same build), averaged over the last 10 steps of each workload:
      counted_flops  SQ_INSTS_VALU_MFMA_MOPS_F32 x 512 (the counter counts
                     fp32 MFMA work in units of 512 flops)
      algorithmic    the hot-path survey's 2 B r c per product of the launch
      busy_frac      SQ_VALU_MFMA_BUSY_CYCLES / (4 SIMDs x 256 CUs x
                     GRBM_GUI_ACTIVE / 8): the share of the launch's active
                     cycles the MFMA pipes were busy, at the clock the chip ran
                     (busy cycles per SIMD; the GUI counter summed over the 8
                     XCDs)."""
    import csv

    b, labels = _bench_labels(bench_json)
    res = {b["config"]["workload"]: b}
    if b.get("secondary"):
        res[b["secondary"]["workload"]] = b["secondary"]
    rows = list(csv.DictReader(open(pmc_csv)))
    per = {}
    for c in ("SQ_INSTS_VALU_MFMA_MOPS_F32", "SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE"):
        rc = [r for r in rows if r["Counter_Name"] == c]
        for wl, lst in _per_launch(rc, labels, lambda r: float(r["Counter_Value"])).items():
            per[(wl, c)] = [(k, w, sum(v[-10:]) / len(v[-10:])) for k, w, v in lst]
    out = ["# workload\tlaunch\tcounted_flops\talgorithmic_flops\tbusy_frac\tgui_active_per_xcd\tkernel (workgroups)"]
    for wl in labels:
        alg = {k["kernel"]: k.get("survey_flops", 0.0) for k in res[wl]["kernels"]}
        for p, lab in enumerate(labels[wl]):
            mops = per[(wl, "SQ_INSTS_VALU_MFMA_MOPS_F32")][p]
            busy = per[(wl, "SQ_VALU_MFMA_BUSY_CYCLES")][p][2]
            gui = per[(wl, "GRBM_GUI_ACTIVE")][p][2] / MI355X_XCDS
            frac = busy / (4 * MI355X_CUS * gui) if gui > 0 else 0.0
            out.append(f"{wl}\t{lab}\t{mops[2] * 512:.0f}\t{alg.get(lab, 0.0):.0f}\t{frac:.4f}\t{gui:.0f}\t"
                       f"{mops[0]} ({mops[1]})")
    print("\n".join(out))
    return 0


def trace_summary(trace_csv, bench_json):
    """Per-launch kernel durations from a rocprofv3 --kernel-trace of one
    bench run, averaged over every whole step the run executed, beside the
    in-step figure of the same launch from `bench_json` (a plain run of the
    same build: the profiler itself slows the B=64 launches)."""
    import csv

    b, labels = _bench_labels(bench_json)
    rows = [r for r in csv.DictReader(open(trace_csv)) if r["Kind"] == "KERNEL_DISPATCH"]
    per = _per_launch(rows, labels, lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    res = {b["config"]["workload"]: b}
    if b.get("secondary"):
        res[b["secondary"]["workload"]] = b["secondary"]
    out = []
    for wl in labels:
        r = res[wl]
        bench_ms = {k["kernel"]: k["ms"] for k in r["kernels"]}
        lst = per[wl]
        tot = sum(sum(v) / len(v) for _, _, v in lst)
        rf = roofline_of(max(r["kernels"], key=dominance))
        trace_of = {lab: sum(v) / len(v) for (_, _, v), lab in zip(lst, labels[wl])}
        t_us = trace_of[rf["kernel"]]
        t_frac = (rf["algorithmic_bytes"] / (t_us * 1e-6) / 1e9 / PEAK_HBM_GBS if rf["bound"] == "hbm"
                  else rf["algorithmic_flops"] / (t_us * 1e-6) / 1e12 / PEAK_FP32_MFMA_TFLOPS)
        mode = b["config"].get("step_launch", "graph replay")
        out += [f"## workload {wl}: step {r['ms_per_step'] * 1000:.1f} us (plain bench run, {mode}); "
                f"sum of traced kernel durations per step {tot:.1f} us over {len(lst[0][2])} steps",
                f"## roofline launch {rf['kernel']} (longest in-step launch): plain run {rf['avg_ms'] * 1000:.2f} us "
                f"-> {rf['achieved']} {rf['unit']} = {rf['frac'] * 100:.1f}% of {rf['peak']}; traced average "
                f"{t_us:.2f} us -> {t_frac * 100:.1f}%",
                f"{'avg_us':>9} {'min_us':>9} {'bench_us':>9}  launch  [kernel (workgroups)]"]
        for (k, w, v), lab in zip(lst, labels[wl]):
            out.append(f"{sum(v) / len(v):9.2f} {min(v):9.2f} {bench_ms[lab] * 1000:9.2f}  {lab}  [{k} ({w})]")
        out.append("")
    print("\n".join(out))
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 2000 C2 steps = 0.12 s timed after 12 ms of warm-up: shorter runs of the
    # B=64 step (tens of microseconds each) read the GPU still ramping up
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--config", default="c2", choices=sorted(WORKLOADS))
    ap.add_argument("--secondary", default="c5", help="second workload in the same line, or 'none'")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-profile", action="store_true", help="skip the per-kernel profile")
    ap.add_argument("--no-extra-legs", action="store_true",
                    help="skip the runtime optimizer, graph execution and extras-path measurements (profiler runs "
                         "whose dispatches are split into the two workloads' steps)")
    ap.add_argument("--cpu-threads", type=int, default=int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
                    or len(os.sched_getaffinity(0)), help="threads of the CPU baseline's all-cores leg")
    ap.add_argument("--graph-dispatch", choices=("nodes", "packets"), default="packets",
                    help="how HIP replays graphs in this process (the step runs as direct launches unless "
                         "VOLTA_GRAPH=1; the graph-replay leg and graph execution replay graphs): 'packets' "
                         "leaves HIP's default (recorded kernel packets); 'nodes' sets "
                         "DEBUG_CLR_GRAPH_PACKET_CAPTURE=0 before the first HIP call (nodes dispatched in order "
                         "as stream launches)")
    ap.add_argument("--hsa-completion", choices=("polling", "interrupts"), default="interrupts",
                    help="how this process's HSA runtime waits for GPU completion signals: 'interrupts' leaves "
                         "the runtime's default; 'polling' sets HSA_ENABLE_INTERRUPT=0 before the first HIP call "
                         "(the waiting thread spins)")
    ap.add_argument("--calibration-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB 10 times (scales rocprofv3 HBM counters)")
    ap.add_argument("--traffic-table", nargs=2, metavar=("PMC_DIR", "BENCH_JSON"),
                    help="only print HBM bytes per launch from rocprofv3 counter passes (no GPU)")
    ap.add_argument("--trace-summary", nargs=2, metavar=("TRACE_CSV", "BENCH_JSON"),
                    help="only print per-launch durations from a rocprofv3 kernel trace of a bench run (no GPU)")
    ap.add_argument("--mfma-table", nargs=2, metavar=("PMC_CSV", "BENCH_JSON"),
                    help="only print MFMA flops and busy cycles per launch from a rocprofv3 --pmc run (no GPU)")
    ap.add_argument("--configs", default="c1,c3,c4_128,c4_256,c4_1024",
                    help="other BASELINE.json configurations reported briefly in the line ('none': skip)")
    ap.add_argument("--default-runtime-leg", action=argparse.BooleanOptionalAction, default=False,
                    help="also time the headline in a child process with HIP's default graph dispatch and "
                         "completion waits (what a caller that sets no environment gets), for runs that set "
                         "--graph-dispatch nodes or --hsa-completion polling")
    ap.add_argument("--graph-replay-leg", action=argparse.BooleanOptionalAction, default=True,
                    help="also time the headline with its launch sequence replayed from a captured hipGraph "
                         "(VOLTA_GRAPH=1) instead of enqueued directly")
    a = ap.parse_args(argv)
    if a.traffic_table:
        return traffic_table(*a.traffic_table)
    if a.trace_summary:
        return trace_summary(*a.trace_summary)
    if a.mfma_table:
        return mfma_table(*a.mfma_table)
    if a.calibration_copy:
        return calibration_copy(a.calibration_copy)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the step would shard by data parallelism over B, with one all-reduce of the flat "
              "[dW; db] buffer before the optimizer).", file=sys.stderr)
        return 2

    # The host's choices of HIP's graph replay mode and of how the HSA runtime
    # waits for completion signals; both are read once, at the first HIP
    # call, so they are set before the library is loaded.  By default the
    # bench sets neither (what a caller of the library gets); they matter
    # for graph replays (with node dispatch the host takes part in each
    # replay and polling shortens its wake-ups), not for the step's direct
    # launches.
    if a.graph_dispatch == "nodes":
        os.environ["DEBUG_CLR_GRAPH_PACKET_CAPTURE"] = "0"
    else:
        os.environ.pop("DEBUG_CLR_GRAPH_PACKET_CAPTURE", None)
    if a.hsa_completion == "polling":
        os.environ["HSA_ENABLE_INTERRUPT"] = "0"
    else:
        os.environ.pop("HSA_ENABLE_INTERRUPT", None)
    # The CPU legs run first, before this process's first HIP call: once the
    # HSA runtime has started with polled completion signals, its event
    # thread spins on a host core and an all-cores OpenMP step slows many
    # times over (C2 4.4 -> 160-180 ms on 16 threads).
    cpu_primary = cpu_secondary = None
    if not a.no_cpu:
        cpu_primary = run_cpu(a.config, a.cpu_threads)
        if a.secondary and a.secondary != "none":
            cpu_secondary, _ = run_cpu(a.secondary, a.cpu_threads, full_protocol=False)
    default_leg = None
    if a.default_runtime_leg:
        default_leg = run_default_runtime_leg(a.config, a.steps, a.warmup)
        log(f"default runtime leg: {default_leg}")
    spec, B, lr, res = run_gpu(a.config, a.steps, a.warmup, want_profile=not a.no_profile)
    log(f"{a.config}: {res['ms_per_step']:.4f} ms/step, {res['samples_per_s']:.0f} samples/s")
    line = {
        "metric": METRIC,
        "value": round(res["samples_per_s"], 2),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(res["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: X,Y ~ N(0,1) (splitmix64 + Box-Muller, seed 42), He-uniform weights, zero biases; "
                "one resident batch reused every step",
        "config": {"workload": a.config, "layers": list(spec.sizes), "activation": spec.activation,
                   "loss": spec.loss, "optimizer": spec.optimizer, "lr": lr, "batch": B,
                   "parallelism": "single GPU",
                   "step_launch": "graph replay (VOLTA_GRAPH=1)" if _env_on("VOLTA_GRAPH") and not
                   _env_on("VOLTA_NO_GRAPH") else "direct launches (the library's default)",
                   "graph_dispatch": a.graph_dispatch, "hsa_completion": a.hsa_completion},
        "mfma_frac_step": round(res["mfma_frac_step"], 5),
        "gemm_gflop_per_step": round(res["gemm_gflop_per_step"], 4),
        "loss_after": res["loss_after"],
        "arena_bytes": res["arena_bytes"],
        "host_staged_ms_per_step": res["host_staged_ms_per_step"],
    }
    if "roofline" in res:
        line["roofline"] = res["roofline"]
        line["kernel_sum_ms"] = round(res["kernel_sum_ms"], 5)
        line["kernels"] = [{k: (round(v, 5) if isinstance(v, float) else v) for k, v in r.items()}
                           for r in res["kernels"]]
    if a.config in PUBLISHED_CPU:
        line["reference_published_cpu"] = PUBLISHED_CPU[a.config]
    if cpu_primary:
        line["cpu_baseline"], line["cpu_baseline_legs"] = cpu_primary
        line["cpu_host"] = host_cpu()
    if a.secondary and a.secondary != "none":
        s_steps = max(5, a.steps // 20)
        s_spec, s_B, s_lr, s_res = run_gpu(a.secondary, s_steps, max(2, a.warmup // 10),
                                           want_profile=not a.no_profile)
        log(f"{a.secondary}: {s_res['ms_per_step']:.4f} ms/step, {s_res['samples_per_s']:.0f} samples/s, "
            f"MFMA frac {s_res['mfma_frac_step']:.3f}")
        sec = {"workload": a.secondary, "layers": list(s_spec.sizes), "activation": s_spec.activation,
               "loss": s_spec.loss, "optimizer": s_spec.optimizer, "lr": s_lr, "batch": s_B, "steps": s_steps,
               "ms_per_step": round(s_res["ms_per_step"], 5), "samples_per_s": round(s_res["samples_per_s"], 2),
               "mfma_frac_step": round(s_res["mfma_frac_step"], 5),
               "gemm_gflop_per_step": round(s_res["gemm_gflop_per_step"], 3),
               "host_staged_ms_per_step": s_res["host_staged_ms_per_step"]}
        if "roofline" in s_res:
            sec["roofline"] = s_res["roofline"]
            sec["kernels"] = [{k: (round(v, 5) if isinstance(v, float) else v) for k, v in r.items()}
                              for r in s_res["kernels"]]
        if cpu_secondary:
            sec["cpu_baseline"] = cpu_secondary
        line["secondary"] = sec
    if default_leg:
        line["default_runtime"] = default_leg
    if a.graph_replay_leg and not _env_on("VOLTA_GRAPH") and not _env_on("VOLTA_NO_GRAPH"):
        # the same step replayed from its captured hipGraph (VOLTA_GRAPH is
        # read when a handle is created)
        os.environ["VOLTA_GRAPH"] = "1"
        try:
            _, _, _, g_res = run_gpu(a.config, a.steps, a.warmup, want_profile=False)
        finally:
            os.environ.pop("VOLTA_GRAPH", None)
        line["graph_replay"] = {"workload": a.config, "ms_per_step": round(g_res["ms_per_step"], 5),
                                "samples_per_s": round(g_res["samples_per_s"], 2),
                                "host_staged_ms_per_step": g_res["host_staged_ms_per_step"],
                                "note": "the same launch sequence captured once as a hipGraph and replayed "
                                        "(VOLTA_GRAPH=1), graph dispatch as config.graph_dispatch"}
        log(f"graph replay: {line['graph_replay']}")
    if a.configs and a.configs != "none":
        # the other BASELINE.json configurations: step time and launch count
        line["configs"] = []
        for c in a.configs.split(","):
            c_spec, c_B, c_lr, c_res = run_gpu(c, max(100, a.steps // 2), max(20, a.warmup // 2),
                                               want_profile=False, count_launches=True)
            row = {"workload": c, "layers": list(c_spec.sizes), "activation": c_spec.activation,
                   "loss": c_spec.loss, "optimizer": c_spec.optimizer, "batch": c_B,
                   "ms_per_step": round(c_res["ms_per_step"], 5), "samples_per_s": round(c_res["samples_per_s"], 2),
                   "mfma_frac_step": round(c_res["mfma_frac_step"], 5), "launches": c_res["launches"],
                   "host_staged_ms_per_step": c_res["host_staged_ms_per_step"]}
            line["configs"].append(row)
            log(f"{c}: {row['ms_per_step']:.4f} ms/step, {row['launches']} launches")
    if not a.no_profile and not a.no_extra_legs:
        line["runtime_optimizer"] = run_rt_optimizer()
        log(f"runtime optimizer: {line['runtime_optimizer']}")
        line["graph_execution"] = [run_rt_graph("c5", 4096), run_rt_graph("c2", 64)]
        log(f"graph execution: {line['graph_execution']}")
        # the extras launch structure (not paired; 3-4 more launches per
        # hidden layer), on the headline topology
        line["extras_path"] = []
        for x in EXTRAS_WORKLOADS:
            x_spec, x_B, x_lr, x_res = run_gpu(x, max(50, a.steps // 4), max(10, a.warmup // 4))
            row = {"workload": x, "layernorm": bool(x_spec.layernorm), "dropout_p": x_spec.dropout_p,
                   "clip_grad": x_spec.clip_grad, "optimizer": x_spec.optimizer, "batch": x_B,
                   "ms_per_step": round(x_res["ms_per_step"], 5),
                   "samples_per_s": round(x_res["samples_per_s"], 2), "launches": len(x_res["kernels"]),
                   "kernel_sum_ms": round(x_res["kernel_sum_ms"], 5),
                   "slowest": max(({"kernel": r["kernel"], "ms": round(r["ms"], 5)} for r in x_res["kernels"]),
                                  key=lambda r: r["ms"])}
            line["extras_path"].append(row)
            log(f"{x}: {row['ms_per_step']:.4f} ms/step, {row['launches']} launches")
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
