"""Plan builder: produces SeeML .seeu plans (train / merge / eval programs,
rodata, persistent image, emit table) for LoRA update steps.

The reference's update compiler produces these plans, but it cannot be built
in this toolchain (it needs <expected>); this module restates its pipeline
so the backend can be fed the same instruction sequences and binder-decided
arena offsets. Each stage cites the reference code it follows:

  forward SIR from a model description   compiler/frontend/parser/parser.cc:12-253,
                                         value_resolver.cc:26-47 (lazy weight decls)
  loss graft                             compiler/driver/update_compiler.cc:132-199
  LoRA graft                             compiler/analysis/algebra/lora_grafter.cc:24-180
  primal snapshot -> eval program        update_compiler.cc:236-238
  reverse-mode autodiff (pruned)         compiler/analysis/calculus/autodiff.cc:15-444
  AdamW synthesis (sorted by param id)   compiler/analysis/calculus/optimizer.cc:12-57
  merge program                          compiler/analysis/algebra/merge_builder.cc:12-68
  arena binding + liveness first-fit     compiler/backend/trainer/arena_binder.cc:25-185
  merge binding above the high-water     update_compiler.cc:345-369
  lowering to 64-byte instructions       compiler/backend/trainer/instruction_lowering.cc:18-350
  counter-based randn init image         update_compiler.cc:415-442
  plan assembly + PlanSelfHash seal      update_compiler.cc:458-536

Epilogue fusion never fires for these models (every GEMM output feeds a
LoRA add or a backward op) and DCE removes nothing from a minimally built
program, so neither pass is restated. The plan hash is computed by the
backend library's PlanSelfHash (the same function its loader verifies with).
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass, field

import numpy as np

# ---------------------------------------------------------------- ABI -------

RODATA_BIT = 1 << 63
NULL_REF = (1 << 64) - 1
ALIGN = 64
HEADER_SIZE = 280
PLAN_HASH_OFFSET = 216

OP = dict(
    Nop=0, GemmNN=1, GemmNT=2, GemmTN=3, GemmAccNN=4, AddEW=5, AddBias=6, ReluFwd=7, ReluBwd=8,
    Scale=9, ReduceRows=10, SoftmaxXEntFwd=11, SoftmaxXEntBwd=12, MseFwd=13, MseBwd=14,
    KLDistillFwd=15, KLDistillBwd=16, SgdStep=17, AdamWStep=18, Fill=19, Copy=20, MulEW=21,
    GeluFwd=22, GeluBwd=23, SiluFwd=24, SiluBwd=25, LayerNormFwd=26, LayerNormBwd=27,
    ClipNorm=28, GemmNNQ8=29, GemmNTQ8=30, RmsNormFwd=31, RmsNormBwd=32, RopeFwd=33,
    RopeBwd=34, AttnFwd=35, AttnDP=36, AttnDV=37, SoftmaxRowsBwd=38, AttnDQ=39, AttnDK=40,
    EmbedFwd=41,
)
OP_NAME = {v: k for k, v in OP.items()}

INSTR = struct.Struct("<HHI4Q3Q")
assert INSTR.size == 64

HEADER_FIELDS = [
    ("magic", "I"), ("version", "I"), ("arena_size", "Q"), ("persistent_size", "Q"),
    ("input_ref", "Q"), ("input_floats", "Q"), ("label_ref", "Q"), ("label_bytes", "Q"),
    ("label_kind", "I"), ("optimizer_kind", "I"), ("loss_ref", "Q"),
    ("train_instr_offset", "Q"), ("train_instr_count", "Q"), ("merge_instr_offset", "Q"),
    ("merge_instr_count", "Q"), ("rodata_offset", "Q"), ("rodata_size", "Q"),
    ("persist_init_offset", "Q"), ("persist_init_size", "Q"), ("emit_table_offset", "Q"),
    ("emit_count", "Q"), ("lr", "f"), ("beta1", "f"), ("beta2", "f"), ("eps", "f"),
    ("weight_decay", "f"), ("pad2", "I"), ("batch", "Q"), ("default_steps", "Q"),
    ("eval_instr_offset", "Q"), ("eval_instr_count", "Q"), ("source_model_hash", "Q"),
    ("plan_hash", "Q"), ("lr_schedule", "I"), ("pad3", "I"), ("warmup_steps", "Q"),
    ("min_lr_factor", "f"), ("clip_norm", "f"), ("input_kind", "I"), ("pad4", "I"),
    ("seq_len", "Q"), ("reserved0", "Q"), ("reserved1", "Q"),
]
HEADER = struct.Struct("<" + "".join(f for _, f in HEADER_FIELDS))
assert HEADER.size == HEADER_SIZE


def align_up(v: int) -> int:
    return (v + ALIGN - 1) & ~(ALIGN - 1)


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def pack32(hi: int, lo: int) -> int:
    if not (0 <= hi <= 0xFFFFFFFF and 0 <= lo <= 0xFFFFFFFF):
        raise ValueError(f"dimension pair ({hi}, {lo}) exceeds the 32-bit ISA dim fields")
    return (hi << 32) | lo


def decode_header(blob: bytes) -> dict:
    return dict(zip([n for n, _ in HEADER_FIELDS], HEADER.unpack_from(blob, 0)))


def decode_program(blob: bytes, offset: int, count: int) -> list:
    out = []
    for i in range(count):
        op, flags, pad, a, b, c, d, o0, o1, o2 = INSTR.unpack_from(blob, offset + 64 * i)
        out.append(dict(opcode=op, flags=flags, pad=pad, inp=[a, b, c, d], out=[o0, o1, o2]))
    return out


# ---------------------------------------------------------------- SIR --------

class Value:
    __slots__ = ("id", "shape", "dtype", "op")

    def __init__(self, vid, shape, dtype="f32", op=None):
        self.id = vid
        self.shape = tuple(int(s) for s in shape)
        self.dtype = dtype
        self.op = op

    @property
    def volume(self) -> int:
        v = 1
        for s in self.shape:
            v *= s
        return v

    @property
    def nbytes(self) -> int:
        return self.volume * 4  # f32 and i32 are both 4 bytes

    def __repr__(self):
        return f"%{self.id}{list(self.shape)}"


class Op:
    __slots__ = ("mn", "operands", "results", "attrs")

    def __init__(self, mn, operands=(), attrs=None):
        self.mn = mn
        self.operands = list(operands)
        self.results = []
        self.attrs = dict(attrs or {})

    def add_result(self, vid, shape, dtype="f32") -> Value:
        v = Value(vid, shape, dtype, self)
        self.results.append(v)
        return v


class Block:
    def __init__(self):
        self.ops: list[Op] = []
        self.args: list[Value] = []

    def add_argument(self, shape, dtype) -> Value:
        v = Value(f"arg{len(self.args)}", shape, dtype)
        self.args.append(v)
        return v

    def append(self, mn, operands=(), attrs=None) -> Op:
        op = Op(mn, operands, attrs)
        self.ops.append(op)
        return op

    def insert_after(self, anchor: Op, new_ops: list) -> None:
        i = self.ops.index(anchor)
        self.ops[i + 1:i + 1] = new_ops

    def users(self, v: Value) -> list:
        return [op for op in self.ops if any(o is v for o in op.operands)]


# ------------------------------------------------------- model description ---

@dataclass
class Tensor:
    name: str
    dims: tuple
    const: bool = True
    init: str = "normal"   # normal | ones | zeros
    std: float = 0.02


@dataclass
class SmfOp:
    kind: str           # MatMul AddBias Relu Gelu Silu Mul LayerNorm Add RmsNorm Rope Attention Embedding
    inputs: list
    output: str
    attr0: int = 0      # heads for Rope / Attention


@dataclass
class Model:
    input_name: str
    output_name: str
    seq_len: int
    tensors: list
    ops: list

    def tensor(self, name):
        for t in self.tensors:
            if t.name == name:
                return t
        return None


def build_forward(block: Block, model: Model, inp: Value, weights: dict, prefix: str = "") -> Value:
    """BuildForward (parser.cc:12-253): one SIR op per model op in order; a
    constant tensor is declared (sc_mem.weight) at its first use
    (value_resolver.cc:26-47). `prefix` names a second graph sharing the
    input (the distillation teacher, "t::", update_compiler.cc:118): every
    value and weight id it declares carries it."""
    env = {model.input_name: inp}

    def resolve(name):
        if name in env:
            return env[name]
        t = model.tensor(name)
        if t is None or not t.const:
            raise ValueError(f"'{name}' is not a constant tensor in the model")
        op = block.append("sc_mem.weight")
        v = op.add_result(prefix + name, t.dims)
        weights[prefix + name] = (v, t)
        env[name] = v
        return v

    for o in model.ops:
        ins = [resolve(n) for n in o.inputs]
        k = o.kind
        if k == "MatMul":
            op = block.append("sc_high.matmul", ins)
            env[o.output] = op.add_result(prefix + o.output, (ins[0].shape[0], ins[1].shape[1]))
        elif k == "AddBias":
            op = block.append("sc_high.add_bias", ins)
            env[o.output] = op.add_result(prefix + o.output, ins[0].shape)
        elif k in ("Relu", "Gelu", "Silu"):
            op = block.append("sc_high." + k.lower(), ins)
            env[o.output] = op.add_result(prefix + o.output, ins[0].shape)
        elif k == "Mul":
            op = block.append("sc_high.mul", ins)
            env[o.output] = op.add_result(prefix + o.output, ins[0].shape)
        elif k == "Embedding":
            op = block.append("sc_high.embedding", ins)
            env[o.output] = op.add_result(prefix + o.output, (ins[0].shape[0], ins[1].shape[1]))
        elif k == "Add":
            op = block.append("sc_high.add", ins)
            env[o.output] = op.add_result(prefix + o.output, ins[0].shape)
        elif k == "RmsNorm":
            op = block.append("sc_high.rms_norm", ins)
            env[o.output] = op.add_result(prefix + o.output, ins[0].shape)
            op.add_result(prefix + o.output + ".rstd", (ins[0].shape[0],))
        elif k == "Rope":
            op = block.append("sc_high.rope", ins, {"heads": o.attr0, "seq": model.seq_len})
            env[o.output] = op.add_result(prefix + o.output, ins[0].shape)
        elif k == "Attention":
            rows = ins[0].shape[0]
            op = block.append("sc_high.attention", ins, {"heads": o.attr0, "seq": model.seq_len})
            env[o.output] = op.add_result(prefix + o.output, ins[0].shape)
            op.add_result(prefix + o.output + ".probs", (rows * o.attr0, model.seq_len))
        elif k == "LayerNorm":
            rows = ins[0].shape[0]
            op = block.append("sc_high.layer_norm", ins)
            env[o.output] = op.add_result(prefix + o.output, ins[0].shape)
            op.add_result(prefix + o.output + ".mean", (rows,))
            op.add_result(prefix + o.output + ".rstd", (rows,))
        else:
            raise ValueError(f"unknown model op kind {k}")
    return env[model.output_name]


# ------------------------------------------------------------ LoRA graft ----

@dataclass
class LoraSpec:
    rank: int = 8
    alpha: float = 16.0
    seed: int = 42
    targets: tuple = ()   # substring filters; empty = every eligible MatMul


@dataclass
class Adapter:
    weight: Value
    A: Value
    B: Value
    scale: float
    id_base: str


def graft_lora(block: Block, spec: LoraSpec) -> list:
    """LoraGrafter::Run (lora_grafter.cc:24-180)."""
    targets = []
    for op in block.ops:
        if op.mn != "sc_high.matmul" or len(op.operands) != 2:
            continue
        w = op.operands[1]
        if w.op is None or w.op.mn != "sc_mem.weight":
            continue
        # the student graph only (lora_grafter.cc:16-18,38)
        if w.id.startswith("t::") or op.results[0].id.startswith("t::"):
            continue
        if any(u.mn != "sc_high.matmul" or len(u.operands) != 2 or u.operands[1] is not w
               or u.operands[0] is w for u in block.users(w)):
            continue
        if spec.targets and not any(f in w.id for f in spec.targets):
            continue
        targets.append(op)
    if not targets:
        raise ValueError("LoraGrafter: no eligible MatMul targets found")
    adapters, by_weight, sites = [], {}, {}
    scale = np.float32(spec.alpha) / np.float32(spec.rank)
    for idx_t, target in enumerate(targets):
        x, w, c = target.operands[0], target.operands[1], target.results[0]
        n, k, m, r = x.shape[0], w.shape[0], w.shape[1], spec.rank
        consumers = block.users(c)
        base = w.id
        site = sites.get(base, 0)
        sites[base] = site + 1
        if site > 0:
            base += f"@{site}"
        new_ops = []
        if id(w) not in by_weight:
            a_op = Op("sc_mem.param", attrs={"trainable": 1, "init": "randn",
                                             "std": float(np.float32(1.0) / np.sqrt(np.float32(k))),
                                             "seed": spec.seed + len(adapters)})
            A = a_op.add_result(base + ".lora_A", (k, r))
            b_op = Op("sc_mem.param", attrs={"trainable": 1, "init": "zeros"})
            B = b_op.add_result(base + ".lora_B", (r, m))
            new_ops += [a_op, b_op]
        else:
            ad = adapters[by_weight[id(w)]]
            A, B = ad.A, ad.B
        t_op = Op("sc_high.matmul", [x, A])
        t = t_op.add_result(base + ".lora_t", (n, r))
        u_op = Op("sc_high.matmul", [t, B])
        u = u_op.add_result(base + ".lora_u", (n, m))
        s_op = Op("sc_high.scale", [u], {"alpha": float(scale)})
        s = s_op.add_result(base + ".lora_s", (n, m))
        add_op = Op("sc_high.add", [c, s])
        cp = add_op.add_result(base + ".lora_out", (n, m))
        new_ops += [t_op, u_op, s_op, add_op]
        block.insert_after(target, new_ops)
        for cons in consumers:
            cons.operands = [cp if o is c else o for o in cons.operands]
        if id(w) not in by_weight:
            by_weight[id(w)] = len(adapters)
            adapters.append(Adapter(w, A, B, float(scale), base))
    return adapters


# -------------------------------------------------------------- autodiff ----

def autodiff(block: Block, loss: Value, trainables: list, extra: tuple = ()) -> dict:
    """TrainableAutodiff::Run (autodiff.cc:362-444) with the VJP rules of
    autodiff.cc:66-358, emission order included. `extra` values are treated
    as needing a gradient too (their gradients are returned with the
    trainables'); the reference prunes them (autodiff.cc:76-82)."""
    needs = set(id(p) for p in trainables) | set(id(v) for v in extra)
    for op in block.ops:
        if any(id(o) in needs for o in op.operands):
            for r in op.results:
                needs.add(id(r))
    if id(loss) not in needs:
        raise ValueError("loss does not depend on any trainable parameter")
    adj = {}
    counter = [0]

    def N(v):
        return id(v) in needs

    def fresh():
        c = counter[0]
        counter[0] += 1
        return c

    def accumulate(primal, grad):
        if not N(primal):
            return
        if id(primal) not in adj:
            adj[id(primal)] = grad
            return
        s = block.append("sc_high.add", [adj[id(primal)], grad])
        adj[id(primal)] = s.add_result(f"{primal.id}.grad_acc{fresh()}", grad.shape)

    def emit1(mn, operands, like, attrs=None):
        op = block.append(mn, operands, attrs)
        return op.add_result(f"{like.id}.d{fresh()}", like.shape)

    fill = block.append("sc_low.fill", [], {"value": 1.0})
    adj[id(loss)] = fill.add_result(loss.id + ".seed", loss.shape)
    primal = list(block.ops)
    for op in reversed(primal):
        if op.mn.startswith("sc_mem."):
            continue
        if not op.results or id(op.results[0]) not in adj:
            continue
        if not any(N(o) for o in op.operands):
            continue
        mn, g = op.mn, adj[id(op.results[0])]
        if mn == "sc_high.matmul":
            x, w = op.operands
            if N(x):
                accumulate(x, emit1("sc_low.matmul_nt", [g, w], x))
            if N(w):
                accumulate(w, emit1("sc_low.matmul_tn", [x, g], w))
        elif mn == "sc_high.add":
            accumulate(op.operands[0], g)
            accumulate(op.operands[1], g)
        elif mn == "sc_high.add_bias":
            accumulate(op.operands[0], g)
            b = op.operands[1]
            if N(b):
                accumulate(b, emit1("sc_low.reduce_rows", [g], b))
        elif mn in ("sc_high.relu", "sc_high.gelu", "sc_high.silu"):
            x = op.operands[0]
            accumulate(x, emit1("sc_low." + mn.split(".")[1] + "_grad", [g, x], x))
        elif mn == "sc_high.mul":
            x, y = op.operands
            if N(x):
                accumulate(x, emit1("sc_low.mul", [g, y], x))
            if N(y):
                accumulate(y, emit1("sc_low.mul", [g, x], y))
        elif mn == "sc_high.layer_norm":
            x, gamma, beta = op.operands
            if N(gamma) or N(beta):
                raise ValueError("trainable LayerNorm affine params are unsupported")
            if N(x):
                accumulate(x, emit1("sc_low.layer_norm_grad",
                                    [g, x, gamma, op.results[1], op.results[2]], x))
        elif mn == "sc_high.rms_norm":
            x, gamma = op.operands
            if N(gamma):
                raise ValueError("trainable RMSNorm gamma is unsupported")
            if N(x):
                accumulate(x, emit1("sc_low.rms_norm_grad", [g, x, gamma, op.results[1]], x))
        elif mn == "sc_high.rope":
            x = op.operands[0]
            if N(x):
                attrs = {"heads": op.attrs["heads"], "seq": op.attrs["seq"]}
                if "base" in op.attrs:
                    attrs["base"] = op.attrs["base"]
                accumulate(x, emit1("sc_low.rope_grad", [g], x, attrs))
        elif mn == "sc_high.attention":
            q, k, v = op.operands
            probs = op.results[1]
            geo = {"heads": op.attrs["heads"], "seq": op.attrs["seq"]}
            if N(v):
                accumulate(v, emit1("sc_low.attn_dv", [probs, g], v, geo))
            if N(q) or N(k):
                dp = emit1("sc_low.attn_dp", [g, v], probs, geo)
                ds = emit1("sc_low.softmax_rows_grad", [probs, dp], probs, geo)
                if N(q):
                    accumulate(q, emit1("sc_low.attn_dq", [ds, k], q, geo))
                if N(k):
                    accumulate(k, emit1("sc_low.attn_dk", [ds, q], k, geo))
        elif mn == "sc_high.scale":
            x = op.operands[0]
            accumulate(x, emit1("sc_low.scale", [g], x, {"alpha": op.attrs["alpha"]}))
        elif mn == "sc_high.softmax_xent":
            logits, labels = op.operands
            if N(logits):
                accumulate(logits, emit1("sc_low.softmax_xent_grad", [op.results[1], labels, g],
                                         logits))
        elif mn == "sc_high.mse":
            pred, target = op.operands
            if N(target):
                raise ValueError("d/dtarget unsupported")
            if N(pred):
                accumulate(pred, emit1("sc_low.mse_grad", [pred, target, g], pred))
        elif mn == "sc_high.kl_distill":
            # dstudent = seed * (p_s - p_t) / (N * T); the teacher is frozen
            # (autodiff.cc:331-353)
            s_logits, t_logits = op.operands
            if N(t_logits):
                raise ValueError("d/dteacher unsupported")
            if N(s_logits):
                accumulate(s_logits, emit1("sc_low.kl_grad", [op.results[1], op.results[2], g],
                                           s_logits, {"temperature": op.attrs["temperature"]}))
        else:
            raise ValueError(f"no VJP rule for '{mn}'")
    grads = {}
    for p in list(trainables) + list(extra):
        if id(p) not in adj:
            raise ValueError(f"no gradient reached '{p.id}'")
        grads[id(p)] = adj[id(p)]
    return grads


def synthesize_optimizer(block: Block, trainables: list, grads: dict, kind: str = "adamw",
                         clip_norm: float = 0.0) -> None:
    """OptimizerSynthesizer::Run (compiler/analysis/calculus/optimizer.cc:
    12-57): params in ascending id order; per parameter an optional
    per-tensor ClipNorm of its gradient, then the SGD step, or AdamW's
    zero-init m/v state and the fused step."""
    for p in sorted(trainables, key=lambda v: v.id.encode()):
        g = grads[id(p)]
        if clip_norm > 0.0:
            block.append("sc_low.clip_norm", [g], {"max_norm": float(np.float32(clip_norm))})
        if kind == "sgd":
            block.append("sc_low.sgd_step", [p, g])
            continue
        m = block.append("sc_mem.param", [], {"trainable": 0, "init": "zeros"}).add_result(
            p.id + ".adam_m", p.shape)
        v = block.append("sc_mem.param", [], {"trainable": 0, "init": "zeros"}).add_result(
            p.id + ".adam_v", p.shape)
        block.append("sc_low.adamw_step", [p, g, m, v])


# ------------------------------------------------- quantization + fusion ---

_WEIGHT_SWEEP_GRAIN = 65536  # kWeightSweepGrain (reviewer/quantization.h:26)


def quant_scale(values: np.ndarray):
    """SelectQuantizedWeights' per-tensor scale (reviewer/quantization.cc:
    29-52): max|w| / 127 in f32 (1 for an all-zero tensor), or None when the
    scale is not a normal float (such a tensor stays f32)."""
    max_abs = np.float32(np.max(np.abs(values))) if values.size else np.float32(0.0)
    scale = np.float32(max_abs / np.float32(127.0)) if max_abs > 0 else np.float32(1.0)
    if not np.isfinite(scale) or scale < np.finfo(np.float32).tiny:
        return None
    return scale


def quantize_int8(values: np.ndarray, scale) -> np.ndarray:
    """The binder's int8 pack (arena_binder.cc:135-160): clamp(round(w /
    scale), -127, 127), with the quotient rounded to f32 and std::round's
    halves away from zero."""
    q = (values.astype(np.float32) / np.float32(scale)).astype(np.float64)
    r = np.sign(q) * np.floor(np.abs(q) + 0.5)
    return np.clip(r, -127.0, 127.0).astype(np.int8)


def select_quantized(block: Block) -> list:
    """The weights SelectQuantizedWeights considers (quantization.cc:13-28):
    every frozen weight whose every reader is a forward or input-gradient
    GEMM taking it as the right operand only."""
    out = []
    for op in block.ops:
        if op.mn != "sc_mem.weight":
            continue
        v = op.results[0]
        users = block.users(v)
        if all(u.mn in ("sc_high.matmul", "sc_low.matmul_nt") and len(u.operands) == 2
               and u.operands[1] is v and u.operands[0] is not v for u in users):
            out.append(v)
    return out


_EPILOGUE_ACT = {"sc_high.relu": "relu", "sc_high.gelu": "gelu", "sc_high.silu": "silu"}


def _uses(block: Block, v: Value) -> int:
    return sum(1 for op in block.ops for o in op.operands if o is v)


def _replace_uses(block: Block, old: Value, new: Value) -> None:
    for op in block.ops:
        op.operands = [new if o is old else o for o in op.operands]


def fuse_epilogues(block: Block, quantized: set, protected: set) -> list:
    """GemmEpilogueFuser::Run (algebra/epilogue_fuser.cc:36-118): a forward
    GEMM whose only reader is an AddBias (and that one's only reader an
    activation), or an activation, absorbs them into its epilogue; the
    orphaned ops are returned for the DCE sweep. A bias declared after the
    GEMM moves before it; a bias never rides a quantized GEMM."""
    fused_away = []
    for gemm in list(block.ops):
        if gemm.mn != "sc_high.matmul" or len(gemm.operands) != 2 or len(gemm.results) != 1:
            continue
        c = gemm.results[0]
        if _uses(block, c) != 1 or id(c) in protected:
            continue
        user = next(op for op in block.ops if any(o is c for o in op.operands))
        if (user.mn == "sc_high.add_bias" and len(user.operands) == 2 and user.operands[0] is c
                and len(user.results) == 1 and id(gemm.operands[1]) not in quantized):
            y, bias = user.results[0], user.operands[1]
            bdef = bias.op
            if bdef is not None and block.ops.index(bdef) > block.ops.index(gemm):
                if not bdef.mn.startswith("sc_mem."):
                    continue
                block.ops.remove(bdef)
                block.ops.insert(block.ops.index(gemm), bdef)
            act = None
            if _uses(block, y) == 1:
                act = next(op for op in block.ops if any(o is y for o in op.operands))
            name = (_EPILOGUE_ACT.get(act.mn) if act is not None and len(act.operands) == 1
                    and len(act.results) == 1 else None)
            if name and id(y) not in protected and id(act.results[0]) not in protected:
                gemm.operands.append(bias)
                gemm.attrs["epilogue_act"] = name
                _replace_uses(block, act.results[0], c)
                fused_away += [user, act]
            elif id(y) not in protected:
                gemm.operands.append(bias)
                _replace_uses(block, y, c)
                fused_away.append(user)
        elif (user.mn in _EPILOGUE_ACT and len(user.operands) == 1 and len(user.results) == 1
              and id(user.results[0]) not in protected):
            gemm.attrs["epilogue_act"] = _EPILOGUE_ACT[user.mn]
            _replace_uses(block, user.results[0], c)
            fused_away.append(user)
    return fused_away


_EFFECTFUL = ("sc_low.clip_norm", "sc_low.sgd_step", "sc_low.adamw_step", "sc_low.gemm_acc")


def dead_code_elimination(block: Block, roots: set) -> int:
    """DeadCodeElimination::Run (updater/dce.cc:23-45): a backward sweep
    removing every op whose results nothing reads and no root names;
    storage declarations and in-place updates are kept."""
    removed = 0
    for op in reversed(list(block.ops)):
        if op.mn.startswith("sc_mem.") or op.mn in _EFFECTFUL:
            continue
        if any(_uses(block, r) or id(r) in roots for r in op.results):
            continue
        block.ops.remove(op)
        removed += 1
    return removed


def build_merge(adapters: list):
    """MergeBuilder::Run (merge_builder.cc:12-68)."""
    mb = Block()
    aliases, outputs = {}, []
    for i, ad in enumerate(adapters):
        a = mb.append("sc_mem.param").add_result(ad.A.id + ".merge_a", ad.A.shape)
        aliases[id(a)] = ad.A
        b = mb.append("sc_mem.param").add_result(ad.B.id + ".merge_b", ad.B.shape)
        aliases[id(b)] = ad.B
        delta = mb.append("sc_low.fill", [], {"value": 0.0}).add_result(
            ad.id_base + ".delta", ad.weight.shape)
        mb.append("sc_low.gemm_acc", [a, b, delta], {"alpha": ad.scale})
        outputs.append((delta, i))
    return mb, aliases, outputs


# ---------------------------------------------------------- arena binding ---

def linear_scan(block: Block, base: int, bound: dict, pinned: set, refs: dict) -> int:
    """LinearScanTransients (arena_binder.cc:25-100): births/deaths by op
    tick, stable sort by birth, first-fit over live blocks sorted by start."""
    birth, death, order = {}, {}, []
    tick = 0
    for op in block.ops:
        if not op.mn.startswith("sc_mem."):
            for r in op.results:
                if id(r) in bound:
                    continue
                birth[id(r)] = tick
                death[id(r)] = tick
                order.append(r)
        for o in op.operands:
            if id(o) in death:
                death[id(o)] = tick
        tick += 1
    INF = float("inf")
    intervals = [(v, birth[id(v)], INF if id(v) in pinned else death[id(v)], align_up(v.nbytes))
                 for v in order]
    intervals.sort(key=lambda iv: iv[1])  # Python's sort is stable
    active = []  # (start, end, free_after), sorted by start
    high = base
    for v, start, end, nbytes in intervals:
        active = [a for a in active if not (a[2] != INF and a[2] < start)]
        off = base
        for a in active:
            if off + nbytes <= a[0]:
                break
            off = max(off, a[1])
        refs[id(v)] = off
        blk = (off, off + nbytes, end)
        # insert at the upper bound of equal starts
        pos = len(active)
        for i, a in enumerate(active):
            if a[0] > off:
                pos = i
                break
        active.insert(pos, blk)
        high = max(high, off + nbytes)
    return high


# --------------------------------------------------------------- lowering ---

_ACT_CODE = {"relu": 1, "gelu": 2, "silu": 3}  # EpilogueAct (instruction.h:124)


def lower(ops: list, ref, quant: dict | None = None) -> list:
    """LowerOps (instruction_lowering.cc:18-350): one 64-byte word per op.
    `quant` maps a quantized weight's value id to its dequant scale: GEMMs
    reading it as B take the q8 opcodes with the scale in in[3]."""
    quant = quant or {}
    words = []
    for op in ops:
        mn = op.mn
        if mn.startswith("sc_mem."):
            continue
        ins = dict(opcode=0, flags=0, inp=[NULL_REF] * 4, out=[0, 0, 0])
        i, o = ins["inp"], ins["out"]
        R = op.results

        def geo():
            act = op.operands[0] if mn in ("sc_high.attention", "sc_low.attn_dp") else R[0]
            heads, seq = op.attrs["heads"], op.attrs["seq"]
            rows, width = act.shape
            if heads <= 0 or seq <= 0 or rows % seq or width % heads:
                raise ValueError(f"malformed sequence geometry on '{mn}'")
            return pack32(rows // seq, seq), pack32(heads, width // heads)

        if mn in ("sc_high.matmul", "sc_low.matmul_nt", "sc_low.matmul_tn"):
            a = op.operands[0]
            scale = quant.get(id(op.operands[1])) if mn != "sc_low.matmul_tn" else None
            if scale is None:
                ins["opcode"] = {"sc_high.matmul": OP["GemmNN"], "sc_low.matmul_nt": OP["GemmNT"],
                                 "sc_low.matmul_tn": OP["GemmTN"]}[mn]
            else:
                ins["opcode"] = OP["GemmNNQ8"] if mn == "sc_high.matmul" else OP["GemmNTQ8"]
                i[3] = f32_bits(scale)
            i[0], i[1], i[2] = ref(a), ref(op.operands[1]), ref(R[0])
            o[0], o[1] = R[0].shape
            o[2] = a.shape[0] if mn == "sc_low.matmul_tn" else a.shape[1]
            # fused epilogue (plan v5): a third operand is the bias, riding
            # in[3]; "epilogue_act" sets the activation bits
            # (instruction_lowering.cc:79-103)
            bias = mn == "sc_high.matmul" and len(op.operands) == 3
            if bias and scale is not None:
                raise ValueError(f"fused bias on a quantized GEMM ('{R[0].id}')")
            if bias:
                i[3] = ref(op.operands[2])
            act = _ACT_CODE.get(op.attrs.get("epilogue_act"), 0)
            ins["flags"] = (1 if bias else 0) | (act << 1)
        elif mn == "sc_low.gemm_acc":
            a, b = op.operands[0], op.operands[1]
            ins["opcode"] = OP["GemmAccNN"]
            i[0], i[1], i[2] = ref(a), ref(b), ref(op.operands[2])
            i[3] = f32_bits(op.attrs.get("alpha", 1.0))
            o[0], o[1], o[2] = a.shape[0], b.shape[1], a.shape[1]
        elif mn == "sc_high.add":
            ins["opcode"] = OP["AddEW"]
            i[0], i[1], i[2] = ref(op.operands[0]), ref(op.operands[1]), ref(R[0])
            o[0] = R[0].volume
        elif mn == "sc_high.add_bias":
            ins["opcode"] = OP["AddBias"]
            i[0], i[1], i[2] = ref(op.operands[0]), ref(op.operands[1]), ref(R[0])
            o[0], o[1] = R[0].shape
        elif mn in ("sc_high.relu", "sc_high.gelu", "sc_high.silu"):
            ins["opcode"] = OP[{"relu": "ReluFwd", "gelu": "GeluFwd", "silu": "SiluFwd"}[mn[8:]]]
            i[0], i[1] = ref(op.operands[0]), ref(R[0])
            o[0] = R[0].volume
        elif mn in ("sc_low.relu_grad", "sc_low.gelu_grad", "sc_low.silu_grad"):
            ins["opcode"] = OP[{"relu_grad": "ReluBwd", "gelu_grad": "GeluBwd",
                                "silu_grad": "SiluBwd"}[mn[7:]]]
            i[0], i[1], i[2] = ref(op.operands[0]), ref(op.operands[1]), ref(R[0])
            o[0] = R[0].volume
        elif mn in ("sc_high.mul", "sc_low.mul"):
            ins["opcode"] = OP["MulEW"]
            i[0], i[1], i[2] = ref(op.operands[0]), ref(op.operands[1]), ref(R[0])
            o[0] = R[0].volume
        elif mn == "sc_high.layer_norm":
            ins["opcode"] = OP["LayerNormFwd"]
            i[0], i[1], i[2], i[3] = ref(op.operands[0]), ref(op.operands[1]), ref(op.operands[2]), ref(R[0])
            o[0] = pack32(*R[0].shape)
            o[1], o[2] = ref(R[1]), ref(R[2])
        elif mn == "sc_low.layer_norm_grad":
            ins["opcode"] = OP["LayerNormBwd"]
            i[0], i[1], i[2], i[3] = ref(op.operands[0]), ref(op.operands[1]), ref(op.operands[2]), ref(R[0])
            o[0], o[1] = ref(op.operands[3]), ref(op.operands[4])
            o[2] = pack32(*R[0].shape)
        elif mn == "sc_high.embedding":
            table = op.operands[1]
            ins["opcode"] = OP["EmbedFwd"]
            i[0], i[1], i[2] = ref(op.operands[0]), ref(table), ref(R[0])
            o[0] = R[0].shape[0]
            o[1] = pack32(*table.shape)
        elif mn == "sc_high.rms_norm":
            ins["opcode"] = OP["RmsNormFwd"]
            i[0], i[1], i[2], i[3] = ref(op.operands[0]), ref(op.operands[1]), ref(R[0]), ref(R[1])
            o[0] = pack32(*R[0].shape)
        elif mn == "sc_low.rms_norm_grad":
            ins["opcode"] = OP["RmsNormBwd"]
            i[0], i[1], i[2], i[3] = ref(op.operands[0]), ref(op.operands[1]), ref(op.operands[2]), ref(R[0])
            o[0] = ref(op.operands[3])
            o[1] = pack32(*R[0].shape)
        elif mn in ("sc_high.rope", "sc_low.rope_grad"):
            bs, hd = geo()
            ins["opcode"] = OP["RopeFwd"] if mn == "sc_high.rope" else OP["RopeBwd"]
            i[0], i[1] = ref(op.operands[0]), ref(R[0])
            o[0], o[1], o[2] = bs, hd, f32_bits(op.attrs.get("base", 10000.0))
        elif mn == "sc_high.attention":
            bs, hd = geo()
            ins["opcode"] = OP["AttnFwd"]
            i[0], i[1], i[2], i[3] = ref(op.operands[0]), ref(op.operands[1]), ref(op.operands[2]), ref(R[0])
            o[0], o[1], o[2] = ref(R[1]), bs, hd
        elif mn in ("sc_low.attn_dp", "sc_low.attn_dv", "sc_low.attn_dq", "sc_low.attn_dk"):
            bs, hd = geo()
            ins["opcode"] = OP[{"attn_dp": "AttnDP", "attn_dv": "AttnDV", "attn_dq": "AttnDQ",
                                "attn_dk": "AttnDK"}[mn[7:]]]
            i[0], i[1], i[2] = ref(op.operands[0]), ref(op.operands[1]), ref(R[0])
            o[0], o[1] = bs, hd
        elif mn == "sc_low.softmax_rows_grad":
            ins["opcode"] = OP["SoftmaxRowsBwd"]
            i[0], i[1], i[2] = ref(op.operands[0]), ref(op.operands[1]), ref(R[0])
            o[0] = pack32(*R[0].shape)
        elif mn in ("sc_high.scale", "sc_low.scale"):
            ins["opcode"] = OP["Scale"]
            i[0], i[1] = ref(op.operands[0]), ref(R[0])
            i[2] = f32_bits(op.attrs.get("alpha", 1.0))
            o[0] = R[0].volume
        elif mn == "sc_low.reduce_rows":
            ins["opcode"] = OP["ReduceRows"]
            i[0], i[1] = ref(op.operands[0]), ref(R[0])
            o[0], o[1] = op.operands[0].shape
        elif mn == "sc_high.softmax_xent":
            ins["opcode"] = OP["SoftmaxXEntFwd"]
            i[0], i[1], i[2], i[3] = ref(op.operands[0]), ref(op.operands[1]), ref(R[0]), ref(R[1])
            o[0], o[1] = op.operands[0].shape
        elif mn == "sc_low.softmax_xent_grad":
            ins["opcode"] = OP["SoftmaxXEntBwd"]
            i[0], i[1], i[2], i[3] = ref(op.operands[0]), ref(op.operands[1]), ref(op.operands[2]), ref(R[0])
            o[0], o[1] = R[0].shape
        elif mn == "sc_high.mse":
            ins["opcode"] = OP["MseFwd"]
            i[0], i[1], i[2] = ref(op.operands[0]), ref(op.operands[1]), ref(R[0])
            o[0] = op.operands[0].volume
        elif mn == "sc_low.mse_grad":
            ins["opcode"] = OP["MseBwd"]
            i[0], i[1], i[2], i[3] = ref(op.operands[0]), ref(op.operands[1]), ref(op.operands[2]), ref(R[0])
            o[0] = R[0].volume
        elif mn == "sc_high.kl_distill":
            s_logits = op.operands[0]
            ins["opcode"] = OP["KLDistillFwd"]
            i[0], i[1], i[2], i[3] = ref(s_logits), ref(op.operands[1]), ref(R[0]), ref(R[1])
            o[0], o[1] = ref(R[2]), pack32(*s_logits.shape)
            o[2] = f32_bits(op.attrs.get("temperature", 1.0))
        elif mn == "sc_low.kl_grad":
            ins["opcode"] = OP["KLDistillBwd"]
            for j in range(3):
                i[j] = ref(op.operands[j])
            i[3] = ref(R[0])
            o[0], o[1] = pack32(*R[0].shape), f32_bits(op.attrs.get("temperature", 1.0))
        elif mn == "sc_low.clip_norm":
            ins["opcode"] = OP["ClipNorm"]
            i[0], i[1] = ref(op.operands[0]), f32_bits(op.attrs.get("max_norm", 0.0))
            o[0] = op.operands[0].volume
        elif mn == "sc_low.sgd_step":
            ins["opcode"] = OP["SgdStep"]
            i[0], i[1] = ref(op.operands[0]), ref(op.operands[1])
            o[0] = op.operands[0].volume
        elif mn == "sc_low.adamw_step":
            ins["opcode"] = OP["AdamWStep"]
            for j in range(4):
                i[j] = ref(op.operands[j])
            o[0] = op.operands[0].volume
        elif mn == "sc_low.fill":
            ins["opcode"] = OP["Fill"]
            i[0] = ref(R[0])
            i[1] = f32_bits(op.attrs.get("value", 0.0))
            o[0] = R[0].volume
        else:
            raise ValueError(f"cannot lower '{mn}'")
        words.append(ins)
    return words


def encode(words: list) -> bytes:
    return b"".join(INSTR.pack(w["opcode"], w["flags"], 0, *w["inp"], *w["out"]) for w in words)


# ---------------------------------------------------------- init image ----

_GOLD = 0x9E3779B97F4A7C15
_MASK = (1 << 64) - 1


def counter_randn(seed: int, count: int) -> np.ndarray:
    """The compiler's counter-based randn (update_compiler.cc:415-442):
    element j mixes splitmix64 draws at counter seed + golden*(2j+1),
    then Box-Muller in double, rounded to f32."""
    j = np.arange(count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        s = np.uint64(seed & _MASK) + np.uint64(_GOLD) * (np.uint64(2) * j + np.uint64(1))

        def nxt(state):
            state = state + np.uint64(_GOLD)
            z = state
            z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
            z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
            return state, z ^ (z >> np.uint64(31))

        s, a = nxt(s)
        s, b = nxt(s)
    u1 = ((a >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
    u2 = (b >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    return (np.sqrt(-2.0 * np.log(u1)) * np.cos(6.283185307179586476925286766559 * u2)).astype(np.float32)


# ---------------------------------------------------------- the compiler ----

@dataclass
class UpdateConfig:
    batch: int
    loss: str = "xent"            # xent | mse
    lora: LoraSpec = field(default_factory=LoraSpec)
    lr: float = 1e-3
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    weight_decay: float = 0.01
    default_steps: int = 1000
    lr_schedule: int = 0
    warmup_steps: int = 0
    min_lr_factor: float = 0.0
    token_input: bool = False
    weight_seed: int = 7
    # Benchmark variant: also compute the input's gradient dX, as for an
    # interior layer (the compiler prunes it for the input layer,
    # autodiff.cc:76-82). dX is pinned like the loss, so it keeps a slot.
    input_grad: bool = False
    # source/plan/config.h:25-81: optimizer kind and per-tensor gradient
    # clipping, distillation (loss "kl" or "xent_kl" against a teacher
    # model), int8 frozen weights, GEMM epilogue fusion.
    optimizer: str = "adamw"      # adamw | sgd
    clip_norm: float = 0.0
    temperature: float = 2.0
    distill_weight: float = 0.5
    quantize_base: bool = False
    fuse_epilogues: bool = True
    # source/plan/config.h:74-76: when false the train program is forward
    # + backward only (no parameter mutation), the build the reference's
    # finite-difference gradient checks use (update_compiler.cc:253).
    emit_optimizer: bool = True


@dataclass
class CompiledPlan:
    blob: bytearray  # the .seeu bytes (mutable buffer, never resized)
    header: dict
    train: list
    merge: list
    eval: list
    params: list          # [(id, param_ref, grad_ref, count)]
    weights: dict         # name -> rodata offset
    adapters: list        # [(id_base, A_ref, B_ref, (K, M), scale)]


_WEIGHT_CHUNK = 1 << 24


def _fill_weights(out: np.ndarray, t: Tensor, seed: int, index: int, pool) -> list:
    """Writes tensor `t`'s synthetic values into `out` (f32 view). Chunk c of
    tensor `index` draws from its own stream SeedSequence([seed, index, c]),
    so the values depend only on (seed, tensor, position) — never on how
    many threads fill them."""
    if t.init == "ones":
        out[:] = 1.0
        return []
    if t.init == "zeros":
        out[:] = 0.0
        return []
    std = np.float32(t.std)

    def fill(c):
        sl = out[c * _WEIGHT_CHUNK:(c + 1) * _WEIGHT_CHUNK]
        g = np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, index, c])))
        g.standard_normal(out=sl, dtype=np.float32)
        sl *= std

    n_chunks = (out.size + _WEIGHT_CHUNK - 1) // _WEIGHT_CHUNK
    return [pool.submit(fill, c) for c in range(n_chunks)]


def _fill_now(out: np.ndarray, t: Tensor, seed: int, index: int) -> None:
    """_fill_weights run synchronously (the same values, chunk by chunk)."""
    class _Now:
        def submit(self, fn, *a):
            fn(*a)
            return None
    _fill_weights(out, t, seed, index, _Now())


def compile_update(model: Model, cfg: UpdateConfig, hash_fn=None, materialize: bool = True,
                   teacher: Model | None = None) -> CompiledPlan:
    """UpdateCompiler::CompileImpl restated (update_compiler.cc:43-602)."""
    wants_teacher = cfg.loss in ("kl", "xent_kl")
    if wants_teacher and teacher is None:
        raise ValueError("the selected loss requires a teacher model")
    block = Block()
    batch = cfg.batch
    if cfg.token_input:
        if model.seq_len == 0 or batch % model.seq_len:
            raise ValueError("the compiled batch must be a whole number of sequences")
        inp = block.add_argument((batch,), "i32")
    else:
        in_dim = model.tensor(model.input_name).dims[-1]
        inp = block.add_argument((batch, in_dim), "f32")
    weights = {}
    out = build_forward(block, model, inp, weights)
    out_dim = out.shape[1]
    t_out = None
    if wants_teacher:
        t_out = build_forward(block, teacher, inp, weights, prefix="t::")
        if t_out.shape[1] != out_dim:
            raise ValueError("teacher output dimensionality mismatch")
    # --- loss graft (update_compiler.cc:132-199)
    labels, label_kind, label_bytes = None, 0, 0

    def make_xent():
        lab = block.add_argument((batch,), "i32")
        op = block.append("sc_high.softmax_xent", [out, lab])
        l = op.add_result("loss.xent", ())
        op.add_result("loss.xent_probs", (batch, out_dim))
        return lab, l

    def make_kl():
        op = block.append("sc_high.kl_distill", [out, t_out],
                          {"temperature": float(np.float32(cfg.temperature))})
        l = op.add_result("loss.kl", ())
        op.add_result("loss.kl_ps", (batch, out_dim))
        op.add_result("loss.kl_pt", (batch, out_dim))
        return l

    if cfg.loss == "xent":
        labels, loss = make_xent()
        label_kind, label_bytes = 1, batch * 4
    elif cfg.loss == "mse":
        labels = block.add_argument((batch, out_dim), "f32")
        label_kind, label_bytes = 2, batch * out_dim * 4
        op = block.append("sc_high.mse", [out, labels])
        loss = op.add_result("loss.mse", ())
    elif cfg.loss == "kl":
        loss = make_kl()
    elif cfg.loss == "xent_kl":
        labels, xent = make_xent()
        label_kind, label_bytes = 1, batch * 4
        kl = make_kl()
        w = np.float32(cfg.distill_weight)
        wx = block.append("sc_high.scale", [xent], {"alpha": float(np.float32(1.0) - w)}).add_result(
            "loss.xent_w", ())
        wk = block.append("sc_high.scale", [kl], {"alpha": float(w)}).add_result("loss.kl_w", ())
        loss = block.append("sc_high.add", [wx, wk]).add_result("loss.total", ())
    else:
        raise ValueError(cfg.loss)
    adapters = graft_lora(block, cfg.lora)
    trainables = [v for ad in adapters for v in (ad.A, ad.B)]
    primal_ops = list(block.ops)
    if cfg.input_grad and cfg.token_input:
        raise ValueError("input_grad needs a float input")
    grads = autodiff(block, loss, trainables, (inp,) if cfg.input_grad else ())
    if cfg.emit_optimizer:
        synthesize_optimizer(block, trainables, grads, cfg.optimizer, cfg.clip_norm)
    merge_block, aliases, merge_outputs = build_merge(adapters)

    # --- frozen-weight quantization (update_compiler.cc:272-285): the
    # selected weights' values are drawn here, because the scale the q8
    # GEMMs carry is their max |w| / 127.
    weight_index = {name: k for k, name in enumerate(weights)}
    quant, packed = {}, {}
    if cfg.quantize_base:
        for v in select_quantized(block):
            vals = np.empty(v.volume, np.float32)
            _fill_now(vals, weights[v.id][1], cfg.weight_seed, weight_index[v.id])
            sc = quant_scale(vals)
            if sc is not None:
                quant[id(v)] = sc
                packed[v.id] = quantize_int8(vals, sc)
    # --- epilogue fusion, then the DCE sweep (update_compiler.cc:287-336)
    protected = {id(loss)} | {id(g) for g in grads.values()}
    if cfg.fuse_epilogues:
        fused_away = fuse_epilogues(block, set(quant), protected)
        if fused_away:
            dead = {id(op) for op in fused_away}
            primal_ops = [op for op in primal_ops if id(op) not in dead]
    roots = set(protected) | {id(r) for op in primal_ops for r in op.results}
    dead_code_elimination(block, roots)

    # --- segmented arena binding (arena_binder.cc:102-185)
    refs = {}
    cursor = 0
    params = []
    for op in block.ops:
        if op.mn == "sc_mem.param":
            v = op.results[0]
            refs[id(v)] = cursor
            params.append((v, cursor, op.attrs))
            cursor += align_up(v.nbytes)
    persistent_size = cursor
    for a in block.args:
        refs[id(a)] = cursor
        cursor += align_up(a.nbytes)
    io_end = cursor
    rodata_offsets = {}
    rodata_size = 0
    for op in block.ops:
        if op.mn == "sc_mem.weight":
            v = op.results[0]
            off = align_up(rodata_size)
            rodata_offsets[v.id] = off
            refs[id(v)] = off | RODATA_BIT
            # a quantized weight packs as int8: one byte per element
            rodata_size = off + (v.volume if v.id in packed else v.nbytes)
    pinned = {id(loss)} | {id(g) for g in grads.values()}
    arena = linear_scan(block, align_up(io_end), refs, pinned, refs)
    merge_refs = {mid: refs[id(orig)] for mid, orig in aliases.items()}
    merge_high = linear_scan(merge_block, align_up(arena), merge_refs,
                             {id(d) for d, _ in merge_outputs}, merge_refs)
    arena = max(arena, merge_high)

    def ref_train(v):
        return refs[id(v)]

    def ref_merge(v):
        return merge_refs[id(v)]

    train_words = lower(block.ops, ref_train, quant)
    eval_words = lower(primal_ops, ref_train, quant)
    merge_words = lower(merge_block.ops, ref_merge)

    # --- persistent image (update_compiler.cc:415-442)
    persist = np.zeros(persistent_size // 4, np.float32)
    for v, off, attrs in params:
        if attrs.get("init") == "randn":
            persist[off // 4: off // 4 + v.volume] = (
                counter_randn(attrs["seed"], v.volume) * np.float32(attrs["std"]))

    # --- rodata layout (values are written straight into the blob below)
    smf_offsets, smf_cursor = {}, 0
    for name, (v, t) in weights.items():
        if name.startswith("t::"):
            continue  # the teacher's weights live in its own model file
        smf_offsets[name] = smf_cursor
        smf_cursor = align_up(smf_cursor + v.nbytes)

    # --- emit table: delta arena range -> (synthetic) source-file range
    emit = []
    for delta, ai in merge_outputs:
        w = adapters[ai].weight
        emit.append((smf_offsets[w.id], w.nbytes, merge_refs[id(delta)]))

    # --- plan assembly (update_compiler.cc:458-536)
    h = dict((n, 0) for n, _ in HEADER_FIELDS)
    h.update(magic=0x55454553, version=7, arena_size=align_up(arena),
             persistent_size=persistent_size, input_ref=refs[id(inp)],
             input_floats=batch if cfg.token_input else batch * inp.shape[1],
             label_ref=refs[id(labels)] if labels is not None else NULL_REF,
             label_bytes=label_bytes, label_kind=label_kind,
             optimizer_kind=0 if cfg.optimizer == "sgd" else 1, clip_norm=cfg.clip_norm,
             loss_ref=refs[id(loss)], lr=cfg.lr, beta1=cfg.beta1,
             beta2=cfg.beta2, eps=cfg.eps, weight_decay=cfg.weight_decay, batch=batch,
             default_steps=cfg.default_steps, lr_schedule=cfg.lr_schedule,
             warmup_steps=cfg.warmup_steps, min_lr_factor=cfg.min_lr_factor,
             input_kind=1 if cfg.token_input else 0,
             seq_len=model.seq_len if cfg.token_input else 0)
    off = align_up(HEADER_SIZE)
    h["train_instr_offset"], h["train_instr_count"] = off, len(train_words)
    off += 64 * len(train_words)
    h["merge_instr_offset"], h["merge_instr_count"] = off, len(merge_words)
    off += 64 * len(merge_words)
    h["eval_instr_offset"], h["eval_instr_count"] = off, len(eval_words)
    off += 64 * len(eval_words)
    off = align_up(off)
    h["rodata_offset"], h["rodata_size"] = off, rodata_size
    off = align_up(off + rodata_size)
    h["persist_init_offset"], h["persist_init_size"] = off, persistent_size
    off = align_up(off + persistent_size)
    h["emit_table_offset"], h["emit_count"] = off, len(emit)
    off += 24 * len(emit)

    plan_info = dict(
        train=train_words, merge=merge_words, eval=eval_words,
        params=[(p.id, refs[id(p)], refs[id(grads[id(p)])], p.volume) for p in trainables],
        weights=rodata_offsets,
        adapters=[(ad.id_base, refs[id(ad.A)], refs[id(ad.B)], ad.weight.shape, ad.scale)
                  for ad in adapters])
    if not materialize:
        return CompiledPlan(b"", h, **plan_info)

    blob = bytearray(off)
    view = np.frombuffer(blob, np.uint8)
    view[h["train_instr_offset"]:h["train_instr_offset"] + 64 * len(train_words)] = \
        np.frombuffer(encode(train_words), np.uint8)
    view[h["merge_instr_offset"]:h["merge_instr_offset"] + 64 * len(merge_words)] = \
        np.frombuffer(encode(merge_words), np.uint8)
    view[h["eval_instr_offset"]:h["eval_instr_offset"] + 64 * len(eval_words)] = \
        np.frombuffer(encode(eval_words), np.uint8)
    # Frozen weights, generated in place by seeded per-chunk streams (no
    # separate multi-GB staging copy).
    import concurrent.futures as cf
    import os
    with cf.ThreadPoolExecutor(max(1, min(16, os.cpu_count() or 1))) as pool:
        futs = []
        for index, (name, (v, t)) in enumerate(weights.items()):
            off0 = h["rodata_offset"] + rodata_offsets[name]
            if name in packed:
                view[off0:off0 + v.volume] = packed[name].view(np.uint8)
                continue
            futs += _fill_weights(view[off0:off0 + v.nbytes].view(np.float32), t,
                                  cfg.weight_seed, index, pool)
        for f in futs:
            f.result()
    p0 = h["persist_init_offset"]
    view[p0:p0 + persistent_size] = persist.view(np.uint8)
    for i, (a, b, c) in enumerate(emit):
        struct.pack_into("<3Q", blob, h["emit_table_offset"] + 24 * i, a, b, c)
    del view
    h["plan_hash"] = 0
    HEADER.pack_into(blob, 0, *[h[n] for n, _ in HEADER_FIELDS])
    if hash_fn is None:
        from . import _lib
        import ctypes
        buf = (ctypes.c_uint8 * len(blob)).from_buffer(blob)
        h["plan_hash"] = _lib.lib().seeml_hip_plan_self_hash(buf, len(blob), PLAN_HASH_OFFSET)
        del buf
    else:
        h["plan_hash"] = hash_fn(bytes(blob), PLAN_HASH_OFFSET)
    struct.pack_into("<Q", blob, PLAN_HASH_OFFSET, h["plan_hash"])
    return CompiledPlan(blob, h, **plan_info)
