"""Build libvolta_hip.so (hand-written HIP for gfx950) in-tree with hipcc.

    python -m volta_amd.build            # compile + link
    python -m volta_amd.build --check    # print the command lines only

Flags:
  --offload-arch=gfx950                  CDNA4 code objects only
  -ffp-contract=off                      keep a*b+c as two roundings, like the reference
  -fhip-fp32-correctly-rounded-divide-sqrt  IEEE '/' and sqrtf in the elementwise math
  -Xclang -target-feature -Xclang -packed-fp32-ops  no packed fp32 VALU ops
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libvolta_hip.so")

SOURCES = ["gemm.hip", "skinny.hip", "step_kernels.hip", "extras.hip", "runtime.hip", "test_hooks.hip", "rt_optimizer.hip",
           "rt_graph.hip", "rt_lower.cpp", "spec.cpp", "vt_frontend.cpp"]
HEADERS = ["gemm.h", "skinny.h", "step_kernels.h", "extras.h", "device_common.h", "recorder.h", "spec.h",
           "narrow_dw.h", "out_head.h", "vt_frontend.h", "rt_lower.h"]
CLI = os.path.join(PKG, "volta-hip")
CLI_SOURCES = ["volta_hip_cli.cpp", "vt_frontend.cpp", "spec.cpp"]
CXX = os.environ.get("CXX", "g++")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("VOLTA_OFFLOAD_ARCH", "gfx950")

COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-ffp-contract=off",
]
DEVICE = [
    f"--offload-arch={ARCH}",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def compile_cmd(src: str) -> list:
    path = os.path.join(CSRC, src)
    obj = os.path.join(BUILD, src + ".o")
    cmd = [HIPCC] + COMMON + ["-I", os.path.join(ROOT, "include")]
    if src.endswith(".hip"):
        cmd += DEVICE + ["-x", "hip"]
    return cmd + ["-c", path, "-o", obj]


def link_cmd() -> list:
    objs = [os.path.join(BUILD, s + ".o") for s in SOURCES]
    return [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", LIB + ".tmp"] + objs


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    cmds = [compile_cmd(s) for s in SOURCES]

    def run(cmd):
        r = subprocess.run(cmd, capture_output=True, text=True)
        err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
        return cmd, r.returncode, err

    with cf.ThreadPoolExecutor(max_workers=min(len(cmds), 8)) as ex:
        for cmd, rc, err in ex.map(run, cmds):
            if verbose:
                print(" ".join(cmd))
            if rc != 0:
                raise RuntimeError(f"hipcc failed ({rc}): {' '.join(cmd)}\n{err}")
            if err.strip() and verbose:
                print(err)
    cmd = link_cmd()
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stderr}")
    shutil.move(LIB + ".tmp", LIB)
    # the command line (host code only; finds libvolta_hip.so beside itself)
    cmd = [CXX, "-O2", "-std=c++17", "-Wall", "-I", os.path.join(ROOT, "include"), "-o", CLI + ".tmp"] + \
        [os.path.join(CSRC, s) for s in CLI_SOURCES]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"CLI build failed: {' '.join(cmd)}\n{r.stderr}")
    shutil.move(CLI + ".tmp", CLI)
    return LIB


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--check", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args(argv)
    if a.check:
        for s in SOURCES:
            print(" ".join(compile_cmd(s)))
        print(" ".join(link_cmd()))
        return 0
    print(build(verbose=a.verbose))
    return 0


if __name__ == "__main__":
    sys.exit(main())
