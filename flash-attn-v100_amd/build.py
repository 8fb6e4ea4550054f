"""Build the gfx950 kernel library ``flash_attention_v100/libfa_gfx950.so``.

Compiles every translation unit in ``csrc/`` with hipcc for gfx950 (in
parallel), then links one shared library exporting the C ABI of
``include/fa_abi.h``.  Runs on a machine without a GPU (hipcc cross-compiles).

    python flash-attn-v100_amd/build.py [-j N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
OBJDIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "flash_attention_v100", "libfa_gfx950.so")
ARCH = "gfx950"

SOURCES = ["fa_abi.cpp", "fa_misc.hip", "fa_fwd_fit.hip"] + [
    f"fa_{pas}_{mode}{dt}.hip"
    for pas in ("bwd", "fwd")  # the backward units take longest: start them first
    for mode, dts in (("d256_", ("bf16", "f16")), ("", ("bf16", "f16", "f32")), ("bias_", ("bf16", "f16", "f32")),
                      ("bias32_", ("bf16", "f16")))
    for dt in dts
]

# units whose MFMA accumulators may live in AGPRs (the head-dim-256 backward:
# its dK / dV and dQ kernels need more than 256 registers a lane; with the
# accumulators forced into VGPR form the compiler crashes on them)
AGPR_FORM_SOURCES = ("fa_bwd_d256_bf16.hip", "fa_bwd_d256_f16.hip")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def common_flags():
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-fPIC",
        "-std=c++17",
        "-I", INCLUDE,
        "-I", CSRC,
        # keep the compiler from emitting packed-fp32 VALU ops (v_pk_*_f32)
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # keep MFMA accumulators in VGPR form: without it the register allocator
        # parks the dK/dV accumulators in AGPRs and copies them every iteration
        "-mllvm", "-amdgpu-mfma-vgpr-form=true",
        # no implicit contraction: every fused multiply-add is an explicit
        # __builtin_fmaf in the source.  With contraction on, the compiler may
        # fuse a product with its fp32 -> fp16 conversion (v_fma_mixlo_f16, one
        # rounding instead of two) in some instantiations and not in others, so
        # paths meant to be bit-identical (stored vs regenerated dropout mask)
        # could differ by an ulp
        "-ffp-contract=off",
        "-Wall",
        "-Wno-unused-command-line-argument",
    ]


def flags_for(src: str):
    f = common_flags()
    if src in AGPR_FORM_SOURCES:
        i = f.index("-amdgpu-mfma-vgpr-form=true")
        del f[i - 1:i + 1]
    return f


def _compile(src: str) -> str:
    obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc()] + flags_for(src) + ["-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    # hipcc's host pass warns that it does not know the packed-fp32 feature: drop that noise
    noise = ("packed-fp32-ops", "is not a recognized feature")
    msgs = [ln for ln in r.stderr.splitlines() if not any(n in ln for n in noise)]
    if msgs:
        sys.stderr.write("\n".join(msgs) + "\n")
    return obj


def build(jobs: int | None = None, verbose: bool = True) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    jobs = jobs or min(len(SOURCES), max(1, os.cpu_count() or 1))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    a = ap.parse_args()
    build(a.j)
