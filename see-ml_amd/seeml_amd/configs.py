"""The BASELINE workload configurations as model descriptions + compiler
configs, plus seeded synthetic batches of the right shape.

C1 MLP update, C2 single large LoRA linear, C3 small / C4 mid / C5 large
LoRA decoders. Decoder layers follow the reference's decoder-stack builder
(test/support/models.cc:235-322: RmsNorm, q/k/v MatMuls, RoPE on q and k,
causal Attention, o MatMul, residual Add, RmsNorm, SiLU-gated MLP, residual
Add) fed by an Embedding gather (models.cc:324-345); C5 swaps in LayerNorm
and a GELU MLP with biases. Weight names follow the same convention
("l{i}.wq" ...), which is what the LoRA target filters match against.

Synthetic choices the BASELINE text leaves open are recorded here: norm
gains 1, norm/bias offsets 0, decoder weights ~N(0, 0.02), MLP weights
~N(0, 1/fan_in); token ids Zipf(1.1) over the vocab as records of S+1 ids,
labels the shifted view (runtime/feeder/dataset.cc:290-313); root seed 7.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from .planner import LoraSpec, Model, SmfOp, Tensor, UpdateConfig


@dataclass
class Workload:
    name: str
    model: Model
    cfg: UpdateConfig
    teacher: Model | None = None  # distillation losses
    vocab: int = 0            # token models
    classes: int = 0          # xent width
    seq: int = 0
    out_dim: int = 0          # MSE target width
    in_dim: int = 0           # feature width
    description: str = ""


def mlp_model(d_in=256, hidden=512, d_out=256) -> Model:
    s1, s2 = 1.0 / math.sqrt(d_in), 1.0 / math.sqrt(hidden)
    return Model("x", "logits", 0, [
        Tensor("x", (-1, d_in), const=False),
        Tensor("w1", (d_in, hidden), std=s1), Tensor("b1", (hidden,), std=s1),
        Tensor("w2", (hidden, d_out), std=s2), Tensor("b2", (d_out,), std=s2),
    ], [
        SmfOp("MatMul", ["x", "w1"], "h1"), SmfOp("AddBias", ["h1", "b1"], "h1b"),
        SmfOp("Relu", ["h1b"], "a1"),
        SmfOp("MatMul", ["a1", "w2"], "h2"), SmfOp("AddBias", ["h2", "b2"], "logits"),
    ])


def mlp3_model(d_in, h1, h2, d_out, acts=("relu", "gelu", None), biases=(True, True, True)) -> Model:
    """A three-layer MLP: each layer MatMul, optional AddBias, optional
    activation (Relu/Gelu/Silu); weights ~N(0, 1/fan_in)."""
    dims = [(d_in, h1), (h1, h2), (h2, d_out)]
    T = [Tensor("x", (-1, d_in), const=False)]
    ops = []
    prev = "x"
    for i, ((k, n), act, bias) in enumerate(zip(dims, acts, biases), start=1):
        sd = 1.0 / math.sqrt(k)
        T.append(Tensor(f"w{i}", (k, n), std=sd))
        out = "logits" if i == 3 and not bias and act is None else f"h{i}"
        ops.append(SmfOp("MatMul", [prev, f"w{i}"], out))
        prev = out
        if bias:
            T.append(Tensor(f"b{i}", (n,), std=sd))
            out = "logits" if i == 3 and act is None else f"h{i}b"
            ops.append(SmfOp("AddBias", [prev, f"b{i}"], out))
            prev = out
        if act is not None:
            out = "logits" if i == 3 else f"a{i}"
            ops.append(SmfOp(act.capitalize(), [prev], out))
            prev = out
    return Model("x", "logits", 0, T, ops)


def linear_model(d=4096) -> Model:
    return Model("x", "y", 0, [
        Tensor("x", (-1, d), const=False), Tensor("w", (d, d), std=1.0 / math.sqrt(d)),
    ], [SmfOp("MatMul", ["x", "w"], "y")])


def decoder_model(vocab, dim, layers, heads, ffn, seq, norm="rms", mlp="swiglu") -> Model:
    T = [Tensor("x", (-1,), const=False), Tensor("emb", (vocab, dim))]
    ops = [SmfOp("Embedding", ["x", "emb"], "e")]
    prev = "e"

    def norm_op(src, tag, out):
        if norm == "rms":
            T.append(Tensor(tag, (dim,), init="ones"))
            ops.append(SmfOp("RmsNorm", [src, tag], out))
        else:
            T.append(Tensor(tag, (dim,), init="ones"))
            T.append(Tensor(tag + "b", (dim,), init="zeros"))
            ops.append(SmfOp("LayerNorm", [src, tag, tag + "b"], out))

    for i in range(layers):
        p = f"l{i}."
        norm_op(prev, p + "g1", p + "n1")
        for w in ("q", "k", "v"):
            T.append(Tensor(p + "w" + w, (dim, dim)))
            ops.append(SmfOp("MatMul", [p + "n1", p + "w" + w], p + w))
        ops.append(SmfOp("Rope", [p + "q"], p + "qr", heads))
        ops.append(SmfOp("Rope", [p + "k"], p + "kr", heads))
        ops.append(SmfOp("Attention", [p + "qr", p + "kr", p + "v"], p + "a", heads))
        T.append(Tensor(p + "wo", (dim, dim)))
        ops.append(SmfOp("MatMul", [p + "a", p + "wo"], p + "o"))
        ops.append(SmfOp("Add", [prev, p + "o"], p + "x1"))
        norm_op(p + "x1", p + "g2", p + "n2")
        if mlp == "swiglu":
            T += [Tensor(p + "wg", (dim, ffn)), Tensor(p + "wu", (dim, ffn)),
                  Tensor(p + "wd", (ffn, dim))]
            ops += [SmfOp("MatMul", [p + "n2", p + "wg"], p + "gt"),
                    SmfOp("MatMul", [p + "n2", p + "wu"], p + "u"),
                    SmfOp("Silu", [p + "gt"], p + "s"),
                    SmfOp("Mul", [p + "s", p + "u"], p + "mg"),
                    SmfOp("MatMul", [p + "mg", p + "wd"], p + "dn")]
            down = p + "dn"
        else:  # gelu MLP with biases
            T += [Tensor(p + "wu", (dim, ffn)), Tensor(p + "bu", (ffn,), init="zeros"),
                  Tensor(p + "wd", (ffn, dim)), Tensor(p + "bd", (dim,), init="zeros")]
            ops += [SmfOp("MatMul", [p + "n2", p + "wu"], p + "h"),
                    SmfOp("AddBias", [p + "h", p + "bu"], p + "hb"),
                    SmfOp("Gelu", [p + "hb"], p + "ha"),
                    SmfOp("MatMul", [p + "ha", p + "wd"], p + "dn"),
                    SmfOp("AddBias", [p + "dn", p + "bd"], p + "dnb")]
            down = p + "dnb"
        ops.append(SmfOp("Add", [p + "x1", down], p + "x2"))
        prev = p + "x2"
    norm_op(prev, "gf", "nf")
    T.append(Tensor("wh", (dim, vocab)))
    ops.append(SmfOp("MatMul", ["nf", "wh"], "logits"))
    return Model("x", "logits", seq, T, ops)


def make(name: str) -> Workload:
    """Full-size BASELINE configs: c1..c5. Reduced parity variants: c2s,
    c3s, c4s, c5s keep each config's op structure at CPU-checkable size;
    c3m, c4m do too with head widths 64 and 128 (the fused attention
    kernels' shapes); c4mr is c4m at LoRA rank 128. c2dx (c2sdx reduced) is C2 with the input's dX, the
    interior-layer stream BASELINE's C2 text describes."""
    if name == "c1":
        return Workload("c1", mlp_model(), UpdateConfig(
            batch=32, loss="xent", lora=LoraSpec(rank=8, alpha=16.0, seed=7), lr=1e-3,
            weight_decay=0.01, default_steps=1000), classes=256, in_dim=256,
            description="MLP 256->512->256 + bias/ReLU, xent over 256, LoRA r8 a16, batch 32")
    # Plans carrying the ABI's remaining instruction kinds, compiled the way
    # the reference compiler emits them (source/plan/config.h:56-81):
    #   f1  fused GEMM epilogues (bias+ReLU, GELU alone), per-tensor ClipNorm,
    #       AdamW under the warmup + cosine LR schedule
    #   f2  fused bias+SiLU and bias-only epilogues, SGD with ClipNorm
    #   q1  int8 frozen weights (GemmNNQ8 with a fused SiLU, GemmNNQ8,
    #       GemmNTQ8 for the input gradient)
    #   k1  KL distillation against a frozen teacher (KLDistillFwd/Bwd)
    #   k2  (1-w)*xent + w*KL, with an int8 teacher and student
    abi = {
        "f1": dict(acts=("relu", "gelu", None), biases=(True, False, True), targets=("w3",),
                   cfg=dict(clip_norm=0.05, lr=1e-2, lr_schedule=1, warmup_steps=3,
                            default_steps=12, min_lr_factor=0.1)),
        "f2": dict(acts=("silu", None, None), biases=(True, True, True), targets=("w3",),
                   cfg=dict(optimizer="sgd", clip_norm=0.05, lr=5e-2)),
        "q1": dict(acts=("silu", "gelu", None), biases=(False, True, True), targets=("w2", "w3"),
                   cfg=dict(quantize_base=True)),
        "k1": dict(acts=("relu", "gelu", None), biases=(True, True, True), targets=(),
                   cfg=dict(loss="kl", temperature=2.0), teacher=True),
        "k2": dict(acts=("gelu", "silu", None), biases=(True, False, True), targets=(),
                   cfg=dict(loss="xent_kl", distill_weight=0.3, temperature=1.5,
                            quantize_base=True), teacher=True),
    }
    if name in abi:
        a = abi[name]
        d_in, h1, h2, d_out, b = 128, 256, 192, 96, 64
        model = mlp3_model(d_in, h1, h2, d_out, a["acts"], a["biases"])
        teacher = mlp3_model(d_in, h1, h2, d_out, ("gelu", "relu", None), (True, True, True)) \
            if a.get("teacher") else None
        cfg = UpdateConfig(batch=b, lora=LoraSpec(rank=8, alpha=16.0, seed=7, targets=a["targets"]),
                           **{"loss": "xent", "default_steps": 100, **a["cfg"]})
        return Workload(name, model, cfg, teacher=teacher, classes=d_out, in_dim=d_in,
                        description=f"MLP {d_in}->{h1}->{h2}->{d_out} {a['acts']} {a['cfg']}")
    if name in ("c2", "c2s", "c2dx", "c2sdx"):
        d, b = (4096, 8192) if name in ("c2", "c2dx") else (512, 1024)
        r = 16
        dx = name.endswith("dx")
        return Workload(name, linear_model(d), UpdateConfig(
            batch=b, loss="mse", lora=LoraSpec(rank=r, alpha=32.0, seed=7), lr=1e-3,
            input_grad=dx),
            out_dim=d, in_dim=d,
            description=f"LoRA linear X[{b},{d}] W[{d},{d}] r{r} a32, MSE" +
                        (", with dX (BASELINE's forward, dX, dA, dB)" if dx else ""))
    dec = {
        # name: vocab, dim, layers, heads, ffn, seq, batch_seqs, rank, targets, lr, norm, mlp
        "c3": (8192, 512, 4, 8, 1376, 256, 16, 8, ("wq", "wv"), 1e-3, "rms", "swiglu"),
        "c4": (32000, 2048, 16, 16, 5504, 1024, 8, 16, ("wq", "wk", "wv", "wo"), 1e-4, "rms", "swiglu"),
        "c5": (32000, 4096, 8, 32, 16384, 2048, 4, 64, (), 1e-3, "layer", "gelu"),
        "c3s": (512, 64, 2, 4, 96, 32, 4, 8, ("wq", "wv"), 1e-3, "rms", "swiglu"),
        "c4s": (1000, 128, 2, 4, 256, 64, 2, 16, ("wq", "wk", "wv", "wo"), 1e-4, "rms", "swiglu"),
        "c5s": (1000, 128, 2, 4, 512, 64, 2, 16, (), 1e-3, "layer", "gelu"),
        # C5's rank 64 on every MatMul (the head included), reduced
        "c5s64": (1000, 128, 2, 4, 512, 64, 2, 64, (), 1e-3, "layer", "gelu"),
        # rank 64 at widths where the backward's dt = (s du) B^T and
        # dB = t^T (s du) are rowdot / colsum shapes on tile plans: the Scale
        # folds into their loads
        "c5m64": (1000, 256, 2, 4, 512, 128, 2, 64, (), 1e-3, "layer", "gelu"),
        # odd widths (200 tokens, an MLP of 520): partial tiles in both
        # dimensions for the fused epilogues
        "c5o64": (1000, 256, 1, 4, 520, 100, 2, 64, (), 1e-3, "layer", "gelu"),
        # head widths 64 and 128: the fused attention kernels' shapes
        "c3m": (512, 128, 2, 2, 192, 64, 4, 8, ("wq", "wv"), 1e-3, "rms", "swiglu"),
        "c4m": (1000, 256, 2, 2, 512, 128, 2, 16, ("wq", "wk", "wv", "wo"), 1e-4, "rms", "swiglu"),
        # c4m at S = 48: row widths and positions that are not powers of two
        "c4m48": (1000, 256, 2, 2, 512, 48, 2, 16, ("wq", "wk", "wv", "wo"), 1e-4, "rms", "swiglu"),
        # c4m over a 2048-token vocabulary: the loss forward and backward run
        # as one pass over the logits (rows of at least 2048 classes)
        "c4mv": (2048, 256, 2, 2, 512, 128, 2, 16, ("wq", "wk", "wv", "wo"), 1e-4, "rms", "swiglu"),
        # c4m at rank 128: the LoRA up-projections are dense tile GEMMs
        # (rank > 64) with the Scale and the residual AddEW in their epilogue
        "c4mr": (1000, 256, 2, 2, 512, 128, 2, 128, ("wq", "wk", "wv", "wo"), 1e-4, "rms", "swiglu"),
    }
    if name not in dec:
        raise KeyError(name)
    V, D, L, H, F, S, Bs, r, tg, lr, norm, mlp = dec[name]
    model = decoder_model(V, D, L, H, F, S, norm=norm, mlp=mlp)
    cfg = UpdateConfig(batch=Bs * S, loss="xent", lora=LoraSpec(rank=r, alpha=16.0, seed=7,
                                                               targets=tg),
                       lr=lr, token_input=True)
    return Workload(name, model, cfg, vocab=V, classes=V, seq=S,
                    description=f"decoder V{V} D{D} L{L} H{H} F{F} S{S} B{Bs} LoRA r{r} "
                                f"{'/'.join(tg) or 'all'} {norm}/{mlp}")


def zipf_tokens(rng: np.random.Generator, vocab: int, n: int, s: float = 1.1) -> np.ndarray:
    """Token ids with P(k) proportional to (k+1)^-s over [0, vocab)."""
    p = (np.arange(1, vocab + 1, dtype=np.float64)) ** (-s)
    cdf = np.cumsum(p)
    cdf /= cdf[-1]
    return np.searchsorted(cdf, rng.random(n), side="right").clip(0, vocab - 1).astype(np.int32)


def batch(w: Workload, step: int = 0, seed: int = 7):
    """One seeded synthetic batch (input, labels) as numpy arrays."""
    rng = np.random.default_rng([seed, step])
    b = w.cfg.batch
    if w.cfg.token_input:
        seqs = b // w.seq
        recs = zipf_tokens(rng, w.vocab, seqs * (w.seq + 1)).reshape(seqs, w.seq + 1)
        # Token record r -> inputs tokens[0..S), labels tokens[1..S] (dataset.cc:290-313)
        return (np.ascontiguousarray(recs[:, :-1]).reshape(-1),
                np.ascontiguousarray(recs[:, 1:]).reshape(-1))
    x = rng.standard_normal((b, w.in_dim), dtype=np.float32)
    if w.cfg.loss == "mse":
        y = rng.standard_normal((b, w.out_dim), dtype=np.float32)
    elif w.cfg.loss == "kl":
        return x.reshape(-1), None  # no label slot: the teacher is the target
    else:
        y = rng.integers(0, w.classes, b).astype(np.int32)
    return x.reshape(-1), y.reshape(-1)
