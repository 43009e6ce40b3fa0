"""Algorithmic work per plan instruction: FLOPs and compulsory HBM bytes.

Bytes count each operand the reference kernel must read or write once, at
4 B per f32/i32 element (1 B per int8 weight) — the traffic floor, not what
a kernel happens to move — except where the engine has proven part of an
operand's contents (a causal SoftmaxRowsBwd: the masked half of P and dP is
exact +0), where they count only what must still be read. FLOPs count 2 per multiply-add of the
contractions (causal attention counts only the j <= i half the kernels
compute). These are the numbers `roofline.achieved` and the MFMA-utilisation
/ HBM-throughput figures divide by measured kernel time.

Classes: "mfma" for GEMM-family contractions with min(M, N, K) >= 64 (dense,
compute-bound on the matrix cores); "hbm" for skinny LoRA GEMMs (a dim = r)
and every non-contraction kernel; "attn" for the attention contractions,
judged by min(compute, bandwidth); "fused" for an instruction executed inside
another's launch (no time, no bytes of its own).
"""
from __future__ import annotations

from .planner import OP_NAME

GEMMS = {"GemmNN", "GemmNT", "GemmTN", "GemmAccNN", "GemmNNQ8", "GemmNTQ8"}
ATTN = {"AttnFwd", "AttnDP", "AttnDV", "AttnDQ", "AttnDK"}


def _hi(w):
    return w >> 32


def _lo(w):
    return w & 0xFFFFFFFF


def work(ins: dict, variant: str = "") -> dict:
    """{'op', 'flops', 'bytes', 'cls', 'shape'} for one decoded instruction.

    `variant` is the engine's kernel choice for it (seeml_hip_gemm_choice):
    a causal SoftmaxRowsBwd reads only the float4s of P and dP that hold
    j <= i, so its bytes are those reads plus the dS write (only those
    float4s with "no zero tail"; AttnFwd/AttnDP with "no zero tail" store
    each 32-row block's P/dP only up to its diagonal tile, and "P unused"
    none of it); a GEMM with
    the following AddEW in its epilogue ("+AddEW") also reads the addend and
    writes the sum. A fused launch (skinny chain, pointwise run) reports the
    bytes it moves ("B=<n>") on its first instruction; the instructions
    executed inside another's launch ("in ...") are class "fused"."""
    name = OP_NAME.get(ins["opcode"], str(ins["opcode"]))
    if variant.startswith("in "):
        return dict(op=name, flops=0, bytes=0, cls="fused", shape=())
    o = ins["out"]
    flops, nbytes, cls, shape = 0, 0, "hbm", ()
    if name in GEMMS:
        M, N, K = o
        bw = 1 if name in ("GemmNNQ8", "GemmNTQ8") else 4
        flops = 2 * M * N * K
        nbytes = 4 * M * K + bw * K * N + 4 * M * N
        if name == "GemmAccNN":
            nbytes += 4 * M * N
        if ins["flags"] & 1:
            nbytes += 4 * N
        if variant.endswith("+AddEW"):
            nbytes += 8 * M * N
        cls = "mfma" if min(M, N, K) >= 64 else "hbm"
        shape = (M, N, K)
    elif name in ATTN or name in ("RopeFwd", "RopeBwd"):
        bs, hd = (o[1], o[2]) if name == "AttnFwd" else (o[0], o[1])
        B, S, H, d = _hi(bs), _lo(bs), _hi(hd), _lo(hd)
        TD, P = B * S * H * d, B * H * S * S
        half = B * H * d * S * (S + 1)  # 2 flops x S(S+1)/2 causal pairs x d
        shape = (B, S, H, d)
        # P-shaped stores without the zero tail: each 32-row block up to its
        # diagonal tile.
        nblk = (S + 31) // 32
        P_head = B * H * sum(32 * min(S, 32 * (w + 1)) for w in range(nblk)) if S else 0
        P_st = P if "no zero tail" not in variant else min(P, P_head)
        if name in ("RopeFwd", "RopeBwd"):
            nbytes = 8 * TD
        elif name == "AttnFwd":
            P_st = 0 if variant == "P unused" else P_st
            flops, nbytes, cls = 2 * half, 4 * (4 * TD + P_st), "attn"
        elif name == "AttnDP":
            flops, nbytes, cls = half, 4 * (2 * TD + P_st), "attn"
        else:  # DV / DQ / DK: read P-shaped + one activation, write one
            flops, nbytes, cls = half, 4 * (2 * TD + P), "attn"
    elif name in ("AddEW", "MulEW", "ReluBwd", "GeluBwd", "SiluBwd"):
        nbytes, shape = 12 * o[0], (o[0],)
    elif name in ("Scale", "ReluFwd", "GeluFwd", "SiluFwd", "Copy"):
        nbytes, shape = 8 * o[0], (o[0],)
    elif name == "Fill":
        nbytes, shape = 4 * o[0], (o[0],)
    elif name == "AddBias":
        nbytes, shape = 8 * o[0] * o[1] + 4 * o[1], (o[0], o[1])
    elif name == "ReduceRows":
        nbytes, shape = 4 * o[0] * o[1] + 4 * o[1], (o[0], o[1])
    elif name == "RmsNormFwd":
        r, c = _hi(o[0]), _lo(o[0])
        nbytes, shape = 8 * r * c + 4 * c + 4 * r, (r, c)
    elif name == "RmsNormBwd":
        r, c = _hi(o[1]), _lo(o[1])
        nbytes, shape = 12 * r * c + 4 * c + 4 * r, (r, c)
    elif name == "LayerNormFwd":
        r, c = _hi(o[0]), _lo(o[0])
        nbytes, shape = 8 * r * c + 8 * c + 8 * r, (r, c)
    elif name == "LayerNormBwd":
        r, c = _hi(o[2]), _lo(o[2])
        nbytes, shape = 12 * r * c + 4 * c + 8 * r, (r, c)
    elif name == "SoftmaxRowsBwd":
        r, c = _hi(o[0]), _lo(o[0])
        nbytes, shape = 12 * r * c, (r, c)
        if variant.startswith("causal") and c and r % c == 0:
            read = sum(4 * (i // 4 + 1) for i in range(c)) * (r // c)
            nbytes = 8 * read + 4 * (read if "no zero tail" in variant else r * c)
    elif name == "EmbedFwd":
        T, D = o[0], _lo(o[1])
        nbytes, shape = 4 * T + 8 * T * D, (T, D)
    elif name in ("SoftmaxXEntFwd", "SoftmaxXEntBwd"):
        N, C = o[0], o[1]
        nbytes, shape = 8 * N * C + 4 * N + 4, (N, C)
    elif name == "MseFwd":
        nbytes, shape = 8 * o[0] + 4, (o[0],)
    elif name == "MseBwd":
        nbytes, shape = 12 * o[0] + 4, (o[0],)
    elif name == "AdamWStep":
        nbytes, shape = 28 * o[0], (o[0],)
    elif name == "SgdStep":
        nbytes, shape = 12 * o[0], (o[0],)
    elif name == "ClipNorm":
        nbytes, shape = 12 * o[0], (o[0],)
    elif name in ("KLDistillFwd",):
        N, C = _hi(o[1]), _lo(o[1])
        nbytes, shape = 16 * N * C + 4, (N, C)
    elif name in ("KLDistillBwd",):
        N, C = _hi(o[0]), _lo(o[0])
        nbytes, shape = 12 * N * C + 4, (N, C)
    if " B=" in variant:
        nbytes = int(variant.rsplit(" B=", 1)[1])
    return dict(op=name, flops=flops, bytes=nbytes, cls=cls, shape=shape)


def summarize(program: list, ms: list, peak_tflops: float = 157.3, peak_gbps: float = 8000.0,
              variants: list = None, launches: list = None):
    """Aggregate per-instruction timings into the BASELINE metric's parts.

    `launches[i]`, when given and not None, is the engine's (flops, bytes)
    for the fused launch row i carries (seeml_hip_launch_work): a colsum
    group's one pass over its shared operand, an operand copy (bytes, no
    FLOPs), a dual pass, a LoRA run or a GEMM with its fused AddEW. It
    replaces the lone instruction's work, so no operand is counted once per
    member of a launch that reads it once."""
    variants = variants or [""] * len(program)
    launches = launches or [None] * len(program)
    rows = []
    for ins, t, v, lw in zip(program, ms, variants, launches):
        r = dict(work(ins, v), ms=t)
        if lw is not None and r["cls"] != "fused":
            r["flops"], r["bytes"] = int(lw[0]), int(lw[1])
            if r["flops"] == 0:
                r["cls"] = "hbm"
        rows.append(r)
    dense = [r for r in rows if r["cls"] == "mfma"]
    gem_all = [r for r in rows if r["op"] in GEMMS]
    # every HBM-bound kernel, the skinny LoRA GEMMs (a dim = the rank)
    # included; and the north star's narrower set, the elementwise, norm,
    # RoPE, loss, embed and optimizer kernels
    hbm = [r for r in rows if r["cls"] == "hbm"]
    elementwise = [r for r in hbm if r["op"] not in GEMMS]

    def util(rs):
        t = sum(r["ms"] for r in rs) * 1e-3
        f = sum(r["flops"] for r in rs)
        return (f / t / 1e12 / peak_tflops) if t > 0 else None

    def gbps(rs):
        t = sum(r["ms"] for r in rs) * 1e-3
        b = sum(r["bytes"] for r in rs)
        return (b / t / 1e9) if t > 0 else None

    by_op = {}
    for r in rows:
        k = r["op"]
        a = by_op.setdefault(k, dict(count=0, ms=0.0, flops=0, bytes=0))
        a["count"] += 1
        a["ms"] += r["ms"]
        a["flops"] += r["flops"]
        a["bytes"] += r["bytes"]
    total_ms = sum(r["ms"] for r in rows)
    return dict(
        rows=rows, by_op=by_op, total_ms=total_ms,
        gemm_dense_mfma_util=util(dense), gemm_all_mfma_util=util(gem_all),
        hbm_kernels_gbps=gbps(hbm),
        hbm_kernels_frac=(gbps(hbm) / peak_gbps) if gbps(hbm) else None,
        hbm_elementwise_gbps=gbps(elementwise),
        hbm_skinny_gemm_gbps=gbps([r for r in hbm if r["op"] in GEMMS]),
    )
