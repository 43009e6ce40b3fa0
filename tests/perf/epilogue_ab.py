"""Times the 256x128 GEMM tile with its plain, fused-AddEW and LoRA
epilogues on the C4 projection shapes, in one process, so that the fused
forms are compared with the plain form on the same box and clock:

  python3 tests/perf/epilogue_ab.py [--cold] [NAME=path/to/libseeml_hip.so ...]

With no library arguments it times this tree's library; with several it
interleaves them launch by launch (an A/B of two builds). Each case is
timed with HIP events around single launches (--cold: after a 1 GiB copy
that evicts the operands from the caches, as in the train step, where the
addend was written several kernels earlier) or around 10 back-to-back
launches (warm), 5 rounds, median. The fused AddEW stores only its sum
(C null: the engine's form when nothing else reads the product); the LoRA
epilogue is rank 16, scaled. A profiling harness beside the tests: the
product never imports it.
"""
from __future__ import annotations

import argparse
import ctypes as C
import os
import statistics
import sys

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "..", "see-ml_amd"))

SHAPES = [(0, 8192, 2048, 2048), (1, 8192, 2048, 2048), (1, 8192, 2048, 5504), (0, 8192, 5504, 2048)]


def bind(path):
    P, U = C.c_void_p, C.c_uint64
    L = C.CDLL(path)
    L.seeml_hip_gemm_forced_split.argtypes = [C.c_int, P, P, P, U, U, U, C.c_int, C.c_int, U, P, P, P]
    L.seeml_hip_gemm_forced_lora.argtypes = [C.c_int, P, P, P, U, U, U, C.c_int, C.c_int, U, P, P,
                                             U, C.c_int, C.c_float, C.c_int, P]
    L.seeml_hip_copy.argtypes = [P, P, U, P]
    L.seeml_hip_kernel_error.restype = C.c_char_p
    return L


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--cold", action="store_true", help="evict the operands before each launch")
    ap.add_argument("--rounds", type=int, default=5)
    ap.add_argument("libs", nargs="*", help="NAME=path of a library build (default: this tree's)")
    a = ap.parse_args(argv)
    import torch
    from seeml_amd import _lib

    libs = [(x.split("=", 1)[0], bind(x.split("=", 1)[1])) for x in a.libs] or [("tree", bind(_lib.LIB_PATH))]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(3)
    cfg = 2  # 256x128x32/w4x2
    cases = []
    for lay, M, N, K in SHAPES:
        ops = dict(A=torch.randn(M, K, device=dev, generator=g),
                   B=torch.randn(K * N, device=dev, generator=g),
                   C=torch.empty(M, N, device=dev), Y=torch.randn(M, N, device=dev, generator=g),
                   O=torch.empty(M, N, device=dev), T=torch.randn(M, 16, device=dev, generator=g),
                   BL=torch.randn(16, N, device=dev, generator=g))
        nm = f"{'NN' if lay == 0 else 'NT'} {M}x{N}x{K}"

        def plain(L, s, lay=lay, M=M, N=N, K=K, o=ops):
            return L.seeml_hip_gemm_forced_split(lay, o["A"].data_ptr(), o["B"].data_ptr(), o["C"].data_ptr(),
                                                 M, N, K, cfg, cfg, 0, None, None, s)

        def addew(L, s, lay=lay, M=M, N=N, K=K, o=ops):
            return L.seeml_hip_gemm_forced_split(lay, o["A"].data_ptr(), o["B"].data_ptr(), None, M, N, K,
                                                 cfg, cfg, 0, o["Y"].data_ptr(), o["O"].data_ptr(), s)

        def lora(L, s, lay=lay, M=M, N=N, K=K, o=ops):
            return L.seeml_hip_gemm_forced_lora(lay, o["A"].data_ptr(), o["B"].data_ptr(), o["O"].data_ptr(),
                                                M, N, K, cfg, cfg, 0, o["T"].data_ptr(), o["BL"].data_ptr(),
                                                16, 1, 0.5, 1, s)

        cases += [(nm, "plain", plain), (nm, "+AddEW", addew), (nm, "+LoRA", lora)]
    flush_n = (1 << 30) // 4
    fx, fy = torch.empty(flush_n, device=dev), torch.empty(flush_n, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    res = {}
    for rnd in range(a.rounds):
        for nm, kind, fn in cases:
            for ln, L in libs:
                reps = 1 if a.cold else 10
                if fn(L, s) != 0:
                    sys.exit(f"epilogue_ab: {ln} {nm} {kind}: {L.seeml_hip_kernel_error()}")
                ts = []
                for _ in range(3 if a.cold else 1):
                    if a.cold:
                        L.seeml_hip_copy(fx.data_ptr(), fy.data_ptr(), flush_n, s)
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    for _ in range(reps):
                        fn(L, s)
                    e1.record()
                    e1.synchronize()
                    ts.append(e0.elapsed_time(e1) / reps * 1e3)
                res.setdefault((ln, nm, kind), []).append(statistics.median(ts))
        print(f"epilogue_ab: round {rnd + 1}/{a.rounds}", flush=True)
    print(f"epilogue_ab: {'cold' if a.cold else 'warm'} operands, tile 256x128x32/w4x2, median us per launch")
    head = "".join(f" {ln:>10s} {'vs plain':>9s}" for ln, _ in libs)
    print(f"{'shape':22s} {'epilogue':8s}{head}")
    for nm, kind, _ in cases:
        row = ""
        for ln, _ in libs:
            v = statistics.median(res[(ln, nm, kind)])
            base = statistics.median(res[(ln, nm, "plain")])
            row += f" {v:10.1f} {100.0 * (v / base - 1.0):+8.1f}%"
        print(f"{nm:22s} {kind:8s}{row}", flush=True)


if __name__ == "__main__":
    main()
