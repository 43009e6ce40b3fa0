"""CPU baseline timing — TEST AND MEASUREMENT INFRASTRUCTURE ONLY.

Times the reference's own executor kernels (oracle/_ref, compiled from the
reference sources) on this host, the way BASELINE's CPU plan and the
reference's bench (tool/seeml_bench.cc:288-333) measure a step:

* whole steps (configs whose CPU step is short): 4 warm-up steps, then
  `repeats` pairs of runs of `lo` and `hi` steps; per-step time = the slope
  (t_hi - t_lo) / (hi - lo), the median over the repeats;
* kernel model (C4/C5, where one CPU step is tens of TFLOP): every distinct
  (opcode, dims, flags) group of the train program is timed once on a
  bounded sample of its work — rows of a GEMM's output or of a row kernel,
  elements of a pointwise kernel, one (batch, head) of attention — median of
  3 after a warm-up, scaled to the full instruction, times its multiplicity.
  Every kernel's work is linear in the sampled extent (rows of C are the
  reference's GEMM parallel unit; attention's (batch, head) units are
  independent), so the sum is the step's kernel time.

Only bench.py's cpu_baseline leg and tests import this module."""
from __future__ import annotations

import os
import statistics
import time

import numpy as np

import oracle

_GEMMS = {"GemmNN", "GemmNT", "GemmTN", "GemmAccNN", "GemmNNQ8", "GemmNTQ8"}


def host_cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _hi(w):
    return int(w) >> 32


def _lo(w):
    return int(w) & 0xFFFFFFFF


def _f32(w):
    return float(np.array([int(w) & 0xFFFFFFFF], np.uint32).view(np.float32)[0])


_POOL = None


def _rnd(n, seed=0):
    """Read-only operand values: a view into one shared pool of uniform
    draws in [-1, 1) (kernel cost does not depend on the values; drawing
    each operand afresh took longer than timing the kernels)."""
    global _POOL
    n = max(int(n), 1)
    if _POOL is None or _POOL.size < n + 4096:
        size = max(n + 4096, 1 << 26)
        _POOL = (np.random.default_rng(11).random(size, dtype=np.float32) * 2 - 1)
    off = (seed * 997) % 4096
    return _POOL[off:off + n]


def _sampled_call(lib, name, ins, threads, rows_cap=None):
    """(call, scale): one call of the reference kernel on a bounded sample
    of the instruction's work, and the factor to its full work."""
    o, i = ins["out"], ins["inp"]
    rows_cap = rows_cap or (1024 if threads > 1 else 64)
    elem_cap = (1 << 22) if threads > 1 else (1 << 19)
    if name in _GEMMS:
        M, N, K = (int(x) for x in o)
        # ~4 GFLOP per sample on the pool (256..1024 output rows); 16 rows
        # on one thread, where a row costs the same at any sample size
        m = min(M, max(256, min(1024, int(4e9 / (2 * N * K)))) if threads > 1 else 8)
        A, C = _rnd(m * K, 1), np.zeros(m * N, np.float32)
        if name in ("GemmNNQ8", "GemmNTQ8"):
            B = np.random.default_rng(2).integers(-127, 128, K * N).astype(np.int8)
        else:
            B = _rnd(K * N, 2)
        act = (ins["flags"] >> 1) & 3
        bias = _rnd(N, 3) if ins["flags"] & 1 else None
        call = {
            "GemmNN": lambda: lib.gemm_nn(A, B, C, m, N, K, bias, act),
            "GemmNT": lambda: lib.gemm_nt(A, B, C, m, N, K),
            "GemmTN": lambda: lib.gemm_tn(A, B, C, m, N, K),
            "GemmAccNN": lambda: lib.gemm_acc_nn(A, B, C, m, N, K, 0.5),
            "GemmNNQ8": lambda: lib.gemm_nn_q8(A, B, C, m, N, K, 0.01, act),
            "GemmNTQ8": lambda: lib.gemm_nt_q8(A, B, C, m, N, K, 0.01),
        }[name]
        return call, M / m
    if name in ("AddEW", "MulEW", "Scale", "ReluFwd", "GeluFwd", "SiluFwd", "ReluBwd", "GeluBwd",
                "SiluBwd", "Fill", "Copy", "MseFwd", "MseBwd", "ClipNorm"):
        n = int(o[0])
        k = min(n, elem_cap)
        x, y, z = _rnd(k, 1), _rnd(k, 2), np.zeros(k, np.float32)
        seed = np.ones(1, np.float32)
        call = {
            "AddEW": lambda: lib.add_ew(x, y, z, k), "MulEW": lambda: lib.mul_ew(x, y, z, k),
            "Scale": lambda: lib.scale(x, z, 2.0, k), "ReluFwd": lambda: lib.relu_fwd(x, z, k),
            "GeluFwd": lambda: lib.gelu_fwd(x, z, k), "SiluFwd": lambda: lib.silu_fwd(x, z, k),
            "ReluBwd": lambda: lib.relu_bwd(x, y, z, k), "GeluBwd": lambda: lib.gelu_bwd(x, y, z, k),
            "SiluBwd": lambda: lib.silu_bwd(x, y, z, k), "Fill": lambda: lib.fill(z, 1.0, k),
            "Copy": lambda: lib.copy(x, z, k), "MseFwd": lambda: lib.mse_fwd(x, y, z, k),
            "MseBwd": lambda: lib.mse_bwd(x, y, seed, z, k),
            "ClipNorm": lambda: lib.clip_norm(z, k, 1.0),  # z is a private buffer
        }[name]
        return call, n / k
    if name in ("AddBias", "ReduceRows"):
        R, Cc = int(o[0]), int(o[1])
        r = min(R, rows_cap * 4)
        x, b, z = _rnd(r * Cc, 1), _rnd(Cc, 2), np.zeros(max(r * Cc, Cc), np.float32)
        call = (lambda: lib.add_bias(x, b, z, r, Cc)) if name == "AddBias" else \
            (lambda: lib.reduce_rows(x, z, r, Cc))
        return call, R / r
    if name in ("RmsNormFwd", "RmsNormBwd", "LayerNormFwd", "LayerNormBwd", "SoftmaxRowsBwd",
                "SoftmaxXEntFwd", "SoftmaxXEntBwd", "KLDistillFwd", "KLDistillBwd"):
        if name in ("RmsNormFwd", "LayerNormFwd", "SoftmaxRowsBwd"):
            R, Cc = _hi(o[0]), _lo(o[0])
        elif name == "RmsNormBwd":
            R, Cc = _hi(o[1]), _lo(o[1])
        elif name == "LayerNormBwd":
            R, Cc = _hi(o[2]), _lo(o[2])
        elif name in ("KLDistillFwd",):
            R, Cc = _hi(o[1]), _lo(o[1])
        elif name == "KLDistillBwd":
            R, Cc = _hi(o[0]), _lo(o[0])
        else:
            R, Cc = int(o[0]), int(o[1])
        r = min(R, rows_cap)
        x, y, z, g = _rnd(r * Cc, 1), _rnd(r * Cc, 2), np.zeros(r * Cc, np.float32), _rnd(Cc, 3)
        stat, stat2 = np.ones(r, np.float32), np.zeros(r, np.float32)
        lab = np.random.default_rng(4).integers(0, Cc, r).astype(np.int32)
        one = np.ones(1, np.float32)
        pt = np.zeros(r * Cc, np.float32)
        ax, ay = np.abs(x), np.abs(y)
        T = 2.0
        call = {
            "RmsNormFwd": lambda: lib.rms_norm_fwd(x, g, z, stat, r, Cc),
            "RmsNormBwd": lambda: lib.rms_norm_bwd(x, y, g, stat, z, r, Cc),
            "LayerNormFwd": lambda: lib.layer_norm_fwd(x, g, g, z, stat2, stat, r, Cc),
            "LayerNormBwd": lambda: lib.layer_norm_bwd(x, y, g, stat2, stat, z, r, Cc),
            "SoftmaxRowsBwd": lambda: lib.softmax_rows_bwd(x, y, z, r, Cc),
            "SoftmaxXEntFwd": lambda: lib.softmax_xent_fwd(x, lab, one, z, r, Cc),
            "SoftmaxXEntBwd": lambda: lib.softmax_xent_bwd(ax, lab, one, z, r, Cc),
            "KLDistillFwd": lambda: lib.kl_distill_fwd(x, y, one, z, pt, r, Cc, T),
            "KLDistillBwd": lambda: lib.kl_distill_bwd(ax, ay, one, z, r, Cc, T),
        }[name]
        return call, R / r
    if name in ("RopeFwd", "RopeBwd"):
        B, S, H, d = _hi(o[0]), _lo(o[0]), _hi(o[1]), _lo(o[1])
        b = min(B, max(1, -(-elem_cap // (S * H * d))))  # whole sequences, >= elem_cap
        x, z = _rnd(b * S * H * d, 1), np.zeros(b * S * H * d, np.float32)
        fn = lib.rope_fwd if name == "RopeFwd" else lib.rope_bwd
        return (lambda: fn(x, z, b, S, H, d, _f32(o[2]))), B / b
    if name in ("AttnFwd", "AttnDP", "AttnDV", "AttnDQ", "AttnDK"):
        bs, hd = (o[1], o[2]) if name == "AttnFwd" else (o[0], o[1])
        B, S, H, d = _hi(bs), _lo(bs), _hi(hd), _lo(hd)
        # One sequence, as many heads as threads (the reference spreads its
        # (batch, head, row) units over the pool); a single thread takes one
        # head at S/4 (causal work ~ S^2) to keep the sample bounded.
        h = min(H, threads)
        s = S if threads > 1 else max(64, S // 4)
        q, k, v = (_rnd(s * h * d, j) for j in (1, 2, 3))
        tri = np.tril(np.abs(_rnd(s * s, 4)).reshape(s, s))
        p = np.ascontiguousarray(np.broadcast_to(tri, (h, s, s))).ravel()
        out_t, out_p = np.zeros(s * h * d, np.float32), np.zeros(h * s * s, np.float32)
        call = {
            "AttnFwd": lambda: lib.attn_fwd(q, k, v, out_t, out_p, 1, s, h, d),
            "AttnDP": lambda: lib.attn_dp(q, v, out_p, 1, s, h, d),
            "AttnDV": lambda: lib.attn_dv(p, q, out_t, 1, s, h, d),
            "AttnDQ": lambda: lib.attn_dq(p, k, out_t, 1, s, h, d),
            "AttnDK": lambda: lib.attn_dk(p, q, out_t, 1, s, h, d),
        }[name]
        return call, float(B * H / h) * (S / s) ** 2
    if name == "EmbedFwd":
        T, V, D = int(o[0]), _hi(o[1]), _lo(o[1])
        t = min(T, rows_cap * 4)
        tok = np.random.default_rng(5).integers(0, V, t).astype(np.int32)
        table, z = _rnd(V * D, 1), np.zeros(t * D, np.float32)
        return (lambda: lib.embed_fwd(tok, table, z, t, D)), T / t
    if name in ("AdamWStep", "SgdStep"):
        n = int(o[0])
        p_, g_, m_, v_ = _rnd(n, 1).copy(), _rnd(n, 2), np.zeros(n, np.float32), np.zeros(n, np.float32)
        if name == "AdamWStep":
            return (lambda: lib.adamw_step(p_, g_, m_, v_, n, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1)), 1.0
        return (lambda: lib.sgd_step(p_, g_, n, 1e-3, 0.01)), 1.0
    return None, 0.0  # Nop


def _time(call, reps=3, long_s=0.05):
    """Median of `reps` timed calls after a warm-up call; a call longer than
    `long_s` is timed once (its timing noise is already small)."""
    call()  # warm-up (pool, caches)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        call()
        ts.append(time.perf_counter() - t0)
        if ts[0] > long_s:
            break
    return statistics.median(ts)


def kernel_model(lib, train, threads, rows_cap=None):
    """Per-step CPU time (ms) of a train program from per-group samples:
    {ms_per_step, gemm_ms, gemm_flops, groups}."""
    from seeml_amd import planner
    lib.set_threads(threads)
    groups = {}
    for ins in train:
        key = (ins["opcode"], ins["flags"], tuple(int(x) for x in ins["out"]))
        groups.setdefault(key, [ins, 0])[1] += 1
    total = gemm = 0.0
    flops = 0
    for (op, _, _), (ins, count) in groups.items():
        name = planner.OP_NAME[op]
        call, scale = _sampled_call(lib, name, ins, threads, rows_cap)
        if call is None:
            continue
        t = _time(call) * scale * count
        total += t
        if name in _GEMMS:
            gemm += t
            flops += 2 * int(ins["out"][0]) * int(ins["out"][1]) * int(ins["out"][2]) * count
    return dict(ms_per_step=total * 1e3, gemm_ms=gemm * 1e3, gemm_flops=flops, groups=len(groups))


def slope_steps(plan, lib, w, threads, lo, hi, repeats=3, warm=4):
    """The reference bench's step timing (seeml_bench.cc:288-310): per-step
    ms = median over `repeats` of (t(hi steps) - t(lo steps)) / (hi - lo)."""
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                    "tests"))
    from helpers import HostPlanRunner
    from seeml_amd import configs
    lib.set_threads(threads)
    r = HostPlanRunner(plan, lib)
    batches = [configs.batch(w, s) for s in range(2)]

    def run(n):
        t0 = time.perf_counter()
        for s in range(n):
            r.train_step(*batches[s % 2])
        return time.perf_counter() - t0

    run(warm)
    slopes = []
    for _ in range(repeats):
        t_lo, t_hi = run(lo), run(hi)
        slopes.append((t_hi - t_lo) / (hi - lo))
    return statistics.median(slopes) * 1e3


# whole-step slope (lo, hi) per config whose CPU step is short enough
STEP_SLOPE = {"c1": (20, 80), "c2": (2, 6), "c2dx": (2, 6), "c3": (2, 6)}


def measure(w, plan, cores):
    """The cpu_baseline object for bench.py: `cores` threads (this host's
    CPU share) and one thread; whole-step slope where STEP_SLOPE lists the
    config, the kernel model otherwise and for every one-thread figure."""
    lib = oracle.ref()
    tokens = w.cfg.batch
    out = {}
    model_cores = kernel_model(lib, plan.train, cores)
    if w.name in STEP_SLOPE:
        lo, hi = STEP_SLOPE[w.name]
        ms = slope_steps(plan, lib, w, cores, lo, hi)
        method = (f"reference kernels (oracle/_ref) on {cores} threads: 4 warm-up steps, "
                  f"median of 3 steps-{lo}/{hi} slopes (tool/seeml_bench.cc:288-310); "
                  f"kernel model {model_cores['ms_per_step']:.1f} ms/step for comparison")
        out["kernel_model_ms_per_step"] = round(model_cores["ms_per_step"], 3)
    else:
        ms = model_cores["ms_per_step"]
        method = (f"reference kernels (oracle/_ref) on {cores} threads, kernel model: each of "
                  f"{model_cores['groups']} distinct (opcode, dims, flags) groups timed on a "
                  f"bounded sample of its work (GEMMs 256-1024 output rows, ~4 GFLOP; row "
                  f"kernels 1024 rows; pointwise 4M elements; attention one sequence with "
                  f"{cores} heads), median of 3 after a warm-up (one timed call "
                  f"beyond 50 ms), scaled to the instruction, x multiplicity")
    one = kernel_model(lib, plan.train, 1)
    lib.set_threads(cores)
    out.update(
        value=tokens / (ms * 1e-3), unit="tokens/s", cores=cores, kind="reference",
        ms_per_step=round(ms, 3),
        gemm_gflops=round(model_cores["gemm_flops"] / (model_cores["gemm_ms"] * 1e-3) / 1e9, 1)
        if model_cores["gemm_ms"] else None,
        one_thread=dict(value=tokens / (one["ms_per_step"] * 1e-3), ms_per_step=round(
            one["ms_per_step"], 3), gemm_gflops=round(
            one["gemm_flops"] / (one["gemm_ms"] * 1e-3) / 1e9, 1) if one["gemm_ms"] else None),
        cpu_model=host_cpu_model(),
        sample=method + "; one thread: the kernel model (GEMMs 8 output rows, row kernels 64 "
                        "rows, pointwise 512K elements, attention one head at S/4)")
    return out
