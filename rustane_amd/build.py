"""Builds librustane_hip.so (gfx950) in-tree with hipcc.

Every HIP translation unit is compiled for gfx950 only, with packed-fp32
VALU ops disabled, and linked into rustane_amd/librustane_hip.so.  The GEMM
test harness (rh_gemm_harness.cpp, used only by the tests) is linked with the
GEMM objects into rustane_amd/librustane_gemm_harness.so.  Object files go to
rustane_amd/_build/.  Run as `python -m rustane_amd.build`.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "librustane_hip.so")
HARNESS = os.path.join(HERE, "librustane_gemm_harness.so")
HARNESS_SOURCES = ["rh_gemm_harness.cpp"]
HARNESS_DEPS = ["rh_gemm.hip", "rh_rowops.hip"]  # objects of SOURCES it links

SOURCES = ["rh_gemm.hip", "rh_attn.hip", "rh_attn_bwd.hip", "rh_gemv.hip", "rh_rowops.hip", "rh_trainops.hip", "rh_optim.hip",
           "rh_runtime.cpp", "rh_train.cpp", "rh_data.cpp", "rh_sched.cpp", "rh_noalloc.cpp"]
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
]


# Per-file extras.  Attention rescales its MFMA accumulators with VALU ops
# every key block; with accumulators in AGPRs each rescale costs two copies
# per register, so its MFMAs take the VGPR form (the GEMMs keep AGPRs: their
# accumulators exceed the 256 architectural VGPRs).
FILE_FLAGS = {"rh_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"],
              "rh_attn_bwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"]}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *CFLAGS, *FILE_FLAGS.get(src, []), "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{out}")
    if out.strip():
        sys.stderr.write(out + "\n")
    return obj


def _link(out: str, objs: list) -> None:
    tmp = out + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout)
    shutil.move(tmp, out)


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = SOURCES + HARNESS_SOURCES
    with cf.ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 4)) as ex:
        objs = dict(zip(srcs, ex.map(_compile, srcs)))
    _link(LIB, [objs[s] for s in SOURCES])
    _link(HARNESS, [objs[s] for s in HARNESS_SOURCES + HARNESS_DEPS])
    if verbose:
        print(f"built {LIB} and {HARNESS}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
