"""Launches one backend GEMM (a bench workload's dominant kernel) and a
plain copy of known size, for hardware-counter runs under rocprofv3:

  python3 tests/perf/kernel_probe.py --layout NN --m 8192 --n 5504 --k 2048 \\
      --cfg 128x64x32/w4x1 --reps 3 --copy-mib 1024

With --dual it launches the LoRA backward's dual skinny pass instead: the
stream x [m, k] read once for dt = x b^T and db = t^T x, both of rank n
(the stream scaled as loaded, as the engine's folded Scale does).

With --step CFG it runs one eager train step of a BASELINE config (every
instruction dispatched on its own, batch 0), for per-dispatch counters of
all of a step's kernels:

  python3 tests/perf/kernel_probe.py --step c4

Each dispatch's FETCH_SIZE / WRITE_SIZE (KiB) is read from the profiler's
counter file; the copy's counters against its known 2 x copy-mib MiB of
traffic calibrate the GEMM's. Inputs are seeded normals in device memory.
A profiling harness beside the tests: the product never imports it.
"""
from __future__ import annotations

import argparse
import ctypes as C
import os
import sys

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "..", "see-ml_amd"))

LAYOUTS = {"NN": 0, "NT": 1, "TN": 2}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--step", default=None, help="one eager train step of this config")
    ap.add_argument("--layout", default="NN", choices=sorted(LAYOUTS))
    ap.add_argument("--m", type=int, default=0)
    ap.add_argument("--n", type=int, default=0)
    ap.add_argument("--k", type=int, default=0)
    ap.add_argument("--cfg", default="skinny", help="tile config name, e.g. 128x64x32/w4x1")
    ap.add_argument("--dual", action="store_true",
                    help="the dual skinny pass over x [m, k] at rank n (no --cfg)")
    ap.add_argument("--splits", type=int, default=1)
    ap.add_argument("--tail-cfg", default=None,
                    help="column split: tile config of columns [n-split, n) (two launches)")
    ap.add_argument("--n-split", type=int, default=0)
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--copy-mib", type=int, default=1024)
    a = ap.parse_args(argv)
    if a.step:
        from seeml_amd import DeviceUpdateEngine, configs, planner
        w = configs.make(a.step)
        plan = planner.compile_update(w.model, w.cfg, teacher=w.teacher)
        e = DeviceUpdateEngine(plan.blob, use_graph=False)
        x, y = configs.batch(w, 0)
        print(f"kernel_probe: {a.step} eager step, loss {e.train_step(x, y)}", flush=True)
        e.close()
        return
    if min(a.m, a.n, a.k) <= 0:
        sys.exit("kernel_probe: --m, --n and --k are required (or --step)")

    import torch
    from seeml_amd import _lib

    L = _lib.lib()
    names = {}
    for i in range(L.seeml_hip_gemm_config_count()):
        names[L.seeml_hip_gemm_config_name(i).decode()] = i
    if a.cfg not in names:
        sys.exit(f"kernel_probe: unknown tile config {a.cfg!r}; have {sorted(names)}")
    cfg = names[a.cfg]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(7)
    M, N, K = a.m, a.n, a.k
    A = torch.randn(M * K, device=dev, generator=g)
    B = torch.randn(K * N, device=dev, generator=g)
    Cm = torch.empty(M * N, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    if a.tail_cfg is not None and a.tail_cfg not in names:
        sys.exit(f"kernel_probe: unknown tile config {a.tail_cfg!r}; have {sorted(names)}")
    for _ in range(a.reps if not a.dual else 0):
        if a.tail_cfg is not None:
            rc = L.seeml_hip_gemm_forced_split(LAYOUTS[a.layout], A.data_ptr(), B.data_ptr(),
                                               Cm.data_ptr(), M, N, K, cfg, names[a.tail_cfg],
                                               a.n_split, None, None, s)
        else:
            rc = L.seeml_hip_gemm_forced(LAYOUTS[a.layout], A.data_ptr(), B.data_ptr(), Cm.data_ptr(),
                                         M, N, K, cfg, a.splits, s)
        if rc != 0:
            sys.exit(f"kernel_probe: {_lib.kernel_error()}")
    if a.dual:
        b = torch.randn(N * K, device=dev, generator=g)
        t = torch.randn(M * N, device=dev, generator=g)
        dt = torch.empty(M * N, device=dev)
        db = torch.empty(N * K, device=dev)
        for _ in range(a.reps):
            rc = L.seeml_hip_gemm_skinny_dual(A.data_ptr(), M, K, b.data_ptr(), N, dt.data_ptr(),
                                              t.data_ptr(), N, db.data_ptr(), 3, 1, 0.5, s)
            if rc != 0:
                sys.exit(f"kernel_probe: {_lib.kernel_error()}")
    n = a.copy_mib * (1 << 20) // 4
    x = torch.randn(n, device=dev, generator=g)
    y = torch.empty(n, device=dev)
    for _ in range(a.reps):
        rc = L.seeml_hip_copy(x.data_ptr(), y.data_ptr(), n, s)
        if rc != 0:
            sys.exit(f"kernel_probe: {_lib.kernel_error()}")
    torch.cuda.synchronize()
    tail = f" | {a.tail_cfg} @ {a.n_split}" if a.tail_cfg is not None else ""
    what = f"dual x {M}x{K} rank {N}" if a.dual else f"{a.layout} {M}x{N}x{K} {a.cfg}{tail}"
    print(f"kernel_probe: {what} x{a.reps}, copy {a.copy_mib} MiB x{a.reps}", flush=True)


if __name__ == "__main__":
    main()
