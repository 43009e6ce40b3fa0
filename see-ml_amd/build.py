"""Builds the gfx950 backend library in-tree: see-ml_amd/lib/libseeml_hip.so.

Every source under csrc/ is compiled by hipcc for gfx950 only, in parallel,
then linked into one shared library whose exported surface is exactly
include/seeml_hip.h. Flags:
  -ffp-contract=off            expressions round where written (CPU bit parity
                               for the pointwise/optimizer kernels)
  -packed-fp32-ops disabled    no v_pk_*_f32 generation (unreliable on the
                               target pool)
  correctly-rounded / and sqrtf (explicit; clang's HIP default) so AdamW and
                               the norm statistics reproduce the CPU's bits
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIB_DIR, "libseeml_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    "-O3", "-fPIC", "-std=c++20", "-ffp-contract=off",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]
DEVICE = [
    f"--offload-arch={ARCH}",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".cc")))


def compile_one(src: str) -> str:
    path = os.path.join(CSRC, src)
    obj = os.path.join(OBJ, src + ".o")
    cmd = [HIPCC] + COMMON
    if src.endswith(".hip"):
        cmd += DEVICE + ["-x", "hip"]
    cmd += ["-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    # hipcc's host pass warns that it does not know the device-only feature.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    warn = "\n".join(l for l in r.stderr.splitlines() if l.strip() and noise not in l)
    if warn:
        print(f"[build] {src}:\n{warn}", file=sys.stderr)
    return obj


def build(jobs: int | None = None) -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
