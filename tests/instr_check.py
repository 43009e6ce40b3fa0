"""Per-instruction parity at full size: one instruction of a plan, checked
against the oracle on the inputs the device actually held.

The engine replays a program instruction by instruction
(seeml_hip_run_range). Before a checked instruction runs, its operands are
read from the arena (and rodata); after it runs, its outputs. The oracle
then recomputes the outputs from those same inputs — for GEMMs on 64
sampled output rows (each output row's k order does not depend on the other
rows, so the oracle's rows are its full product's rows; 16 for a further fused variant of an already checked group), for attention on
one (batch, head), for row kernels on sampled rows, for everything else on
whole tensors. Operand layouts follow the lowering
(compiler/backend/trainer/instruction_lowering.cc:55-340, restated in
seeml_amd.planner.lower). TEST INFRASTRUCTURE ONLY.

Bars: bit-exact for the per-element kernels whose expressions round as the
reference's (AddEW, MulEW, Scale, AddBias, ReLU, Fill, Copy, Embed,
SoftmaxXEntBwd, MseBwd, SGD, AdamW); normwise max rel err <= TOL_STEP for
reductions and device libm (GEMM, attention, norms, softmax, RoPE,
GELU/SiLU)."""
import numpy as np

from helpers import TOL_STEP, rel_err
from seeml_amd import planner

OPN = planner.OP_NAME
RO = planner.RODATA_BIT


def hi(w):
    return int(w) >> 32


def lo(w):
    return int(w) & 0xFFFFFFFF


def fbits(w):
    return float(np.array([int(w) & 0xFFFFFFFF], np.uint32).view(np.float32)[0])


def group_key(ins):
    """(opcode name, flags, dims, B-in-rodata): one check per group."""
    return (OPN[ins["opcode"]], ins["flags"], tuple(int(x) for x in ins["out"]),
            int(ins["inp"][1]) >> 63 if ins["inp"][1] != planner.NULL_REF else 0)


CHECKED = {"GemmNN", "GemmNT", "GemmTN", "GemmAccNN", "GemmNNQ8", "GemmNTQ8", "AddEW", "MulEW",
           "AddBias", "Scale", "ReluFwd", "ReluBwd", "GeluFwd", "GeluBwd", "SiluFwd", "SiluBwd",
           "RmsNormFwd", "RmsNormBwd", "LayerNormFwd", "LayerNormBwd", "RopeFwd", "RopeBwd",
           "AttnFwd", "AttnDP", "AttnDV", "SoftmaxRowsBwd", "AttnDQ", "AttnDK", "EmbedFwd",
           "SoftmaxXEntFwd", "SoftmaxXEntBwd", "MseFwd", "MseBwd", "Fill", "AdamWStep"}

GEMMS = {"GemmNN", "GemmNT", "GemmTN", "GemmAccNN", "GemmNNQ8", "GemmNTQ8"}


class Checker:
    def __init__(self, engine, header, orc, seed=5, sample_rows=64):
        self.e, self.h, self.orc = engine, header, orc
        self.rng = np.random.default_rng(seed)
        self.rows = sample_rows
        self.step = 1
        self.peak = None  # max|want| of the latest GEMM check

    def rd(self, ref, count, dtype=np.float32):
        if dtype == np.float32:
            return self.e.read(ref, count)
        nb = count * np.dtype(dtype).itemsize
        raw = self.e.read(ref, (nb + 3) // 4)
        return raw.view(np.uint8)[:nb].view(dtype).copy()

    def pblock(self, ref, B, H, S):
        """The checked (b, h) = (B - 1, H // 2) block [S, S] of a
        [B*H*S, S] probability-shaped tensor."""
        b, h = B - 1, H // 2
        return self.e.read(int(ref) + 4 * (b * H + h) * S * S, S * S).reshape(S, S)

    # -- operands read before the instruction runs -------------------------
    def before(self, ins):
        op, i, o = OPN[ins["opcode"]], ins["inp"], ins["out"]
        r = self.rd
        if op in ("GemmNN", "GemmNT", "GemmTN", "GemmAccNN", "GemmNNQ8", "GemmNTQ8"):
            M, N, K = (int(x) for x in o)
            b8 = op in ("GemmNNQ8", "GemmNTQ8")
            d = {"A": r(i[0], M * K), "B": r(i[1], K * N, np.int8 if b8 else np.float32)}
            if op == "GemmAccNN":
                d["C0"] = r(i[2], M * N)
            if op == "GemmNN" and ins["flags"] & 1:
                d["bias"] = r(i[3], N)
            return d
        if op in ("AddEW", "MulEW"):
            n = int(o[0])
            return {"x": r(i[0], n), "y": r(i[1], n)}
        if op == "AddBias":
            R, Cc = int(o[0]), int(o[1])
            return {"x": r(i[0], R * Cc), "b": r(i[1], Cc)}
        if op in ("Scale", "ReluFwd", "GeluFwd", "SiluFwd"):
            return {"x": r(i[0], int(o[0]))}
        if op in ("ReluBwd", "GeluBwd", "SiluBwd"):
            n = int(o[0])
            return {"dy": r(i[0], n), "x": r(i[1], n)}
        if op == "RmsNormFwd":
            R, Cc = hi(o[0]), lo(o[0])
            return {"x": r(i[0], R * Cc), "g": r(i[1], Cc)}
        if op == "RmsNormBwd":
            R, Cc = hi(o[1]), lo(o[1])
            return {"dy": r(i[0], R * Cc), "x": r(i[1], R * Cc), "g": r(i[2], Cc),
                    "rstd": r(o[0], R)}
        if op == "LayerNormFwd":
            R, Cc = hi(o[0]), lo(o[0])
            return {"x": r(i[0], R * Cc), "g": r(i[1], Cc), "b": r(i[2], Cc)}
        if op == "LayerNormBwd":
            R, Cc = hi(o[2]), lo(o[2])
            return {"dy": r(i[0], R * Cc), "x": r(i[1], R * Cc), "g": r(i[2], Cc),
                    "mean": r(o[0], R), "rstd": r(o[1], R)}
        if op in ("RopeFwd", "RopeBwd"):
            n = hi(o[0]) * lo(o[0]) * hi(o[1]) * lo(o[1])
            return {"x": r(i[0], n)}
        if op in ("AttnFwd", "AttnDP", "AttnDV", "AttnDQ", "AttnDK"):
            bs, hd = (o[1], o[2]) if op == "AttnFwd" else (o[0], o[1])
            B, S, H, d = hi(bs), lo(bs), hi(hd), lo(hd)
            T = B * S * H * d
            if op == "AttnFwd":
                return {"q": r(i[0], T), "k": r(i[1], T), "v": r(i[2], T)}
            if op == "AttnDP":
                return {"dout": r(i[0], T), "v": r(i[1], T)}
            if op == "AttnDV":
                return {"p": self.pblock(i[0], B, H, S), "dout": r(i[1], T)}
            return {"ds": self.pblock(i[0], B, H, S), "kq": r(i[1], T)}
        if op == "SoftmaxRowsBwd":
            R, Cc = hi(o[0]), lo(o[0])
            rows = np.sort(self.rng.choice(R, min(R, self.rows), replace=False))
            return {"rows": rows,
                    "p": np.stack([r(int(i[0]) + 4 * int(k) * Cc, Cc) for k in rows]),
                    "dp": np.stack([r(int(i[1]) + 4 * int(k) * Cc, Cc) for k in rows])}
        if op == "EmbedFwd":
            T, V, D = int(o[0]), hi(o[1]), lo(o[1])
            return {"tok": r(i[0], T, np.int32), "table": r(i[1], V * D)}
        if op == "SoftmaxXEntFwd":
            N, Cc = int(o[0]), int(o[1])
            return {"logits": r(i[0], N * Cc), "labels": r(i[1], N, np.int32)}
        if op == "SoftmaxXEntBwd":
            N, Cc = int(o[0]), int(o[1])
            return {"p": r(i[0], N * Cc), "labels": r(i[1], N, np.int32), "seed": r(i[2], 1)}
        if op in ("MseFwd", "MseBwd"):
            n = int(o[0])
            d = {"pred": r(i[0], n), "target": r(i[1], n)}
            if op == "MseBwd":
                d["seed"] = r(i[2], 1)
            return d
        if op == "Fill":
            return {}
        if op == "AdamWStep":
            n = int(o[0])
            return {"p": r(i[0], n), "g": r(i[1], n), "m": r(i[2], n), "v": r(i[3], n)}
        raise KeyError(op)

    # -- the check after it ran --------------------------------------------
    def check(self, ins, d):
        op, i, o = OPN[ins["opcode"]], ins["inp"], ins["out"]
        orc, r, f32 = self.orc, self.rd, np.float32

        def exact(got, want, what=""):
            assert np.array_equal(np.asarray(got, f32).view(np.uint32),
                                  np.asarray(want, f32).view(np.uint32)), (op, what)

        def close(got, want, what=""):
            err = rel_err(got, want)
            assert err <= TOL_STEP, (op, what, err)

        if op in ("GemmNN", "GemmNT", "GemmTN", "GemmAccNN", "GemmNNQ8", "GemmNTQ8"):
            M, N, K = (int(x) for x in o)
            rows = np.sort(self.rng.choice(M, min(M, self.rows), replace=False))
            m = len(rows)
            A = d["A"].reshape((K, M) if op == "GemmTN" else (M, K))
            Asub = np.ascontiguousarray(A[:, rows] if op == "GemmTN" else A[rows])
            want = np.zeros(m * N, f32)
            act = (ins["flags"] >> 1) & 3
            if op == "GemmNN":
                orc.gemm_nn(Asub, d["B"], want, m, N, K, d.get("bias"), act)
            elif op == "GemmNT":
                orc.gemm_nt(Asub, d["B"], want, m, N, K)
            elif op == "GemmTN":
                orc.gemm_tn(Asub, d["B"], want, m, N, K)
            elif op == "GemmAccNN":
                want[:] = d["C0"].reshape(M, N)[rows].ravel()
                orc.gemm_acc_nn(Asub, d["B"], want, m, N, K, fbits(i[3]))
            elif op == "GemmNNQ8":
                orc.gemm_nn_q8(Asub, d["B"], want, m, N, K, fbits(i[3]), act)
            else:
                orc.gemm_nt_q8(Asub, d["B"], want, m, N, K, fbits(i[3]))
            got = r(i[2], M * N).reshape(M, N)[rows].ravel()
            close(got, want, f"{M}x{N}x{K}")
            self.peak = float(np.max(np.abs(want))) if want.size else 0.0
            return
        if op in ("AddEW", "MulEW"):
            n = int(o[0])
            want = np.zeros(n, f32)
            getattr(orc, "add_ew" if op == "AddEW" else "mul_ew")(d["x"], d["y"], want, n)
            exact(r(i[2], n), want)
            return
        if op == "AddBias":
            R, Cc = int(o[0]), int(o[1])
            want = np.zeros(R * Cc, f32)
            orc.add_bias(d["x"], d["b"], want, R, Cc)
            exact(r(i[2], R * Cc), want)
            return
        if op == "Scale":
            n = int(o[0])
            want = np.zeros(n, f32)
            orc.scale(d["x"], want, fbits(i[2]), n)
            exact(r(i[1], n), want)
            return
        if op in ("ReluFwd", "GeluFwd", "SiluFwd"):
            n = int(o[0])
            want = np.zeros(n, f32)
            getattr(orc, {"ReluFwd": "relu_fwd", "GeluFwd": "gelu_fwd", "SiluFwd": "silu_fwd"}[op])(
                d["x"], want, n)
            (exact if op == "ReluFwd" else close)(r(i[1], n), want)
            return
        if op in ("ReluBwd", "GeluBwd", "SiluBwd"):
            n = int(o[0])
            want = np.zeros(n, f32)
            getattr(orc, {"ReluBwd": "relu_bwd", "GeluBwd": "gelu_bwd", "SiluBwd": "silu_bwd"}[op])(
                d["dy"], d["x"], want, n)
            (exact if op == "ReluBwd" else close)(r(i[2], n), want)
            return
        if op == "RmsNormFwd":
            R, Cc = hi(o[0]), lo(o[0])
            y, rs = np.zeros(R * Cc, f32), np.zeros(R, f32)
            orc.rms_norm_fwd(d["x"], d["g"], y, rs, R, Cc)
            close(r(i[2], R * Cc), y, "y")
            close(r(i[3], R), rs, "rstd")
            return
        if op == "RmsNormBwd":
            R, Cc = hi(o[1]), lo(o[1])
            dx = np.zeros(R * Cc, f32)
            orc.rms_norm_bwd(d["dy"], d["x"], d["g"], d["rstd"], dx, R, Cc)
            close(r(i[3], R * Cc), dx)
            return
        if op == "LayerNormFwd":
            R, Cc = hi(o[0]), lo(o[0])
            y, mu, rs = np.zeros(R * Cc, f32), np.zeros(R, f32), np.zeros(R, f32)
            orc.layer_norm_fwd(d["x"], d["g"], d["b"], y, mu, rs, R, Cc)
            close(r(i[3], R * Cc), y, "y")
            close(r(o[1], R), mu, "mean")
            close(r(o[2], R), rs, "rstd")
            return
        if op == "LayerNormBwd":
            R, Cc = hi(o[2]), lo(o[2])
            dx = np.zeros(R * Cc, f32)
            orc.layer_norm_bwd(d["dy"], d["x"], d["g"], d["mean"], d["rstd"], dx, R, Cc)
            close(r(i[3], R * Cc), dx)
            return
        if op in ("RopeFwd", "RopeBwd"):
            B, S, H, dd = hi(o[0]), lo(o[0]), hi(o[1]), lo(o[1])
            n = B * S * H * dd
            want = np.zeros(n, f32)
            getattr(orc, "rope_fwd" if op == "RopeFwd" else "rope_bwd")(
                d["x"], want, B, S, H, dd, fbits(o[2]))
            close(r(i[1], n), want)
            return
        if op in ("AttnFwd", "AttnDP", "AttnDV", "AttnDQ", "AttnDK"):
            bs, hd = (o[1], o[2]) if op == "AttnFwd" else (o[0], o[1])
            B, S, H, dd = hi(bs), lo(bs), hi(hd), lo(hd)
            b, h = B - 1, H // 2
            lower = np.tril(np.ones((S, S), bool))

            def act_slice(t):   # [B*S, H*d] -> the (b, h) block [S, d]
                return np.ascontiguousarray(t.reshape(B, S, H, dd)[b, :, h, :]).ravel()

            def p_slice(blk):   # the (b, h) block [S, S], zeros above the diagonal
                blk = blk.copy()
                blk[~lower] = 0.0
                return np.ascontiguousarray(blk).ravel()

            T = B * S * H * dd
            if op == "AttnFwd":
                out, pr = np.zeros(S * dd, f32), np.zeros(S * S, f32)
                orc.attn_fwd(act_slice(d["q"]), act_slice(d["k"]), act_slice(d["v"]), out, pr,
                             1, S, 1, dd)
                close(act_slice(r(i[3], T)), out, "O")
                gp = self.pblock(o[0], B, H, S)
                close(gp[lower], pr.reshape(S, S)[lower], "P")
                return
            if op == "AttnDP":
                out = np.zeros(S * S, f32)
                orc.attn_dp(act_slice(d["dout"]), act_slice(d["v"]), out, 1, S, 1, dd)
                gp = self.pblock(i[2], B, H, S)
                close(gp[lower], out.reshape(S, S)[lower])
                return
            out = np.zeros(S * dd, f32)
            if op == "AttnDV":
                orc.attn_dv(p_slice(d["p"]), act_slice(d["dout"]), out, 1, S, 1, dd)
            elif op == "AttnDQ":
                orc.attn_dq(p_slice(d["ds"]), act_slice(d["kq"]), out, 1, S, 1, dd)
            else:
                orc.attn_dk(p_slice(d["ds"]), act_slice(d["kq"]), out, 1, S, 1, dd)
            close(act_slice(r(i[2], T)), out)
            return
        if op == "SoftmaxRowsBwd":
            R, Cc = hi(o[0]), lo(o[0])
            rows = d["rows"]
            keep = np.arange(Cc)[None, :] <= (rows % Cc)[:, None]  # causal rows (S = Cc)
            p, dp = d["p"].copy(), d["dp"].copy()
            p[~keep], dp[~keep] = 0.0, 0.0
            want = np.zeros(len(rows) * Cc, f32)
            orc.softmax_rows_bwd(np.ascontiguousarray(p).ravel(), np.ascontiguousarray(dp).ravel(),
                                 want, len(rows), Cc)
            got = np.stack([r(int(i[2]) + 4 * int(k) * Cc, Cc) for k in rows])
            close(got[keep], want.reshape(len(rows), Cc)[keep])
            return
        if op == "EmbedFwd":
            T, V, D = int(o[0]), hi(o[1]), lo(o[1])
            want = np.zeros(T * D, f32)
            orc.embed_fwd(d["tok"], d["table"], want, T, D)
            exact(r(i[2], T * D), want)
            return
        if op == "SoftmaxXEntFwd":
            N, Cc = int(o[0]), int(o[1])
            loss, probs = np.zeros(1, f32), np.zeros(N * Cc, f32)
            orc.softmax_xent_fwd(d["logits"], d["labels"], loss, probs, N, Cc)
            close(r(i[2], 1), loss, "loss")
            rows = np.sort(self.rng.choice(N, min(N, self.rows), replace=False))
            close(r(i[3], N * Cc).reshape(N, Cc)[rows], probs.reshape(N, Cc)[rows], "probs")
            return
        if op == "SoftmaxXEntBwd":
            N, Cc = int(o[0]), int(o[1])
            want = np.zeros(N * Cc, f32)
            orc.softmax_xent_bwd(d["p"], d["labels"], d["seed"], want, N, Cc)
            exact(r(i[3], N * Cc), want)
            return
        if op == "MseFwd":
            loss = np.zeros(1, f32)
            orc.mse_fwd(d["pred"], d["target"], loss, int(o[0]))
            close(r(i[2], 1), loss)
            return
        if op == "MseBwd":
            n = int(o[0])
            want = np.zeros(n, f32)
            orc.mse_bwd(d["pred"], d["target"], d["seed"], want, n)
            exact(r(i[3], n), want)
            return
        if op == "Fill":
            n = int(o[0])
            exact(r(i[0], n), np.full(n, fbits(i[1]), f32))
            return
        if op == "AdamWStep":
            n = int(o[0])
            h = self.h
            p, g, m, v = (d[k].copy() for k in ("p", "g", "m", "v"))
            lr = orc.effective_lr(h["lr"], h["lr_schedule"], h["warmup_steps"], h["default_steps"],
                                  h["min_lr_factor"], self.step)
            orc.adamw_step(p, g, m, v, n, lr, h["beta1"], h["beta2"], h["eps"], h["weight_decay"],
                           self.step)
            exact(r(i[0], n), p, "p")
            exact(r(i[2], n), m, "m")
            exact(r(i[3], n), v, "v")
            return
        raise KeyError(op)


def replay_and_check(engine, plan, orc, program_words, x, y, step=1, skip=(), variants=None,
                     progress=None):
    """Stages (x, y), sets step_, replays the train program instruction by
    instruction and checks the first instance of every (opcode, shape)
    group against the oracle on 64 sampled rows. `variants(j)`, when given,
    names how the fused graph runs instruction j (the engine's gemm_choice:
    tile, split, epilogue chain, dual pass, rowdot/colsum group member);
    then the first instance of every (group, variant) pair is checked too,
    on 16 rows when its group was already checked. Returns {checked key:
    max|oracle output| for GEMMs, None otherwise}."""
    from seeml_amd import PROGRAM_TRAIN
    ck = Checker(engine, plan.header, orc)
    ck.step = step
    engine.stage(x, y)
    engine.set_step(step)
    seen, groups, done = {}, set(), 0
    for j, ins in enumerate(program_words):
        key = group_key(ins)
        name = key[0]
        if name not in CHECKED or name in skip:
            continue
        if variants is not None:
            key = key + (variants(j),)
        if key in seen:
            continue
        ck.rows = 16 if key[:4] in groups else 64
        groups.add(key[:4])
        engine.run_range(PROGRAM_TRAIN, done, j)
        d = ck.before(ins)
        engine.run_range(PROGRAM_TRAIN, j, j + 1)
        ck.peak = None
        ck.check(ins, d)
        seen[key] = ck.peak if name in GEMMS else None
        if progress is not None:
            progress(j, key)
        done = j + 1
    engine.run_range(PROGRAM_TRAIN, done, len(program_words))
    return seen
