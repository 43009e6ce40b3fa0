"""CPU tests of the plan boundary: the ABI layout, the compiler restatement's
instruction census, PlanSelfHash against the reference's own hash, the
load-time checks, the C-ABI's exported surface, and the oracle dispatcher
pinned bit-for-bit against the reference kernels driven the same way."""
import collections
import re
import struct

import numpy as np
import pytest

from helpers import (HostPlanRunner, NULL, compile_workload, verify_plan)
from seeml_amd import _lib, configs, planner


def test_abi_sizes_and_offsets():
    assert planner.INSTR.size == 64
    assert planner.HEADER.size == 280
    names = [n for n, _ in planner.HEADER_FIELDS]
    off = 0
    offsets = {}
    for n, f in planner.HEADER_FIELDS:
        offsets[n] = off
        off += struct.calcsize("<" + f)
    assert offsets["plan_hash"] == planner.PLAN_HASH_OFFSET == 216
    assert offsets["lr"] == 152 and offsets["seq_len"] == 256
    assert names[0] == "magic" and off == 280


# Survey Appendix A census (derived from the reference pipeline).
CENSUS = {
    "c1": (32, {"GemmNN": 6, "GemmNT": 4, "GemmTN": 4, "Scale": 4, "AddEW": 3, "AddBias": 2,
                "ReluFwd": 1, "ReluBwd": 1, "SoftmaxXEntFwd": 1, "SoftmaxXEntBwd": 1, "Fill": 1,
                "AdamWStep": 4}),
    "c2": (14, {"GemmNN": 3, "GemmNT": 1, "GemmTN": 2, "Scale": 2, "AddEW": 1, "MseFwd": 1,
                "MseBwd": 1, "Fill": 1, "AdamWStep": 2}),
    "c3": (251, {"GemmNN": 45, "GemmNT": 40, "GemmTN": 16, "AddEW": 39, "Scale": 16, "MulEW": 12,
                 "RmsNormFwd": 9, "RmsNormBwd": 8, "RopeFwd": 8, "RopeBwd": 7, "SiluFwd": 4,
                 "SiluBwd": 4, "AttnFwd": 4, "AttnDP": 4, "AttnDV": 4, "SoftmaxRowsBwd": 4,
                 "AttnDQ": 4, "AttnDK": 3, "EmbedFwd": 1, "SoftmaxXEntFwd": 1,
                 "SoftmaxXEntBwd": 1, "Fill": 1, "AdamWStep": 16}),
    "c4": (1403, {"GemmNN": 241, "GemmNT": 235, "GemmTN": 128, "AddEW": 234, "Scale": 128,
                  "MulEW": 48, "RmsNormFwd": 33, "RmsNormBwd": 32, "RopeFwd": 32, "RopeBwd": 32,
                  "AdamWStep": 128}),
    "c5": (871, {"GemmNN": 147, "GemmNT": 141, "GemmTN": 98, "AddEW": 140, "Scale": 98,
                 "AddBias": 16, "LayerNormFwd": 17, "LayerNormBwd": 16, "GeluFwd": 8,
                 "GeluBwd": 8, "RopeFwd": 16, "RopeBwd": 16, "AdamWStep": 98}),
}


@pytest.mark.parametrize("name", sorted(CENSUS))
def test_instruction_census_matches_reference_pipeline(name):
    w = configs.make(name)
    p = planner.compile_update(w.model, w.cfg, materialize=False)
    total, per_op = CENSUS[name]
    assert len(p.train) == total
    cnt = collections.Counter(planner.OP_NAME[i["opcode"]] for i in p.train)
    for op, n in per_op.items():
        assert cnt[op] == n, (op, cnt[op], n)


def test_c2_gemm_shapes_match_appendix():
    w = configs.make("c2")
    p = planner.compile_update(w.model, w.cfg, materialize=False)
    gemms = [(planner.OP_NAME[i["opcode"]], tuple(i["out"])) for i in p.train
             if i["opcode"] in (1, 2, 3)]
    assert gemms == [("GemmNN", (8192, 4096, 4096)), ("GemmNN", (8192, 16, 4096)),
                     ("GemmNN", (8192, 4096, 16)), ("GemmNT", (8192, 16, 4096)),
                     ("GemmTN", (16, 4096, 8192)), ("GemmTN", (4096, 16, 8192))]


def test_c2_dx_stream_adds_the_interior_layer_gradient():
    """C2 with the input's dX (BASELINE's "forward, dX, dA, dB"): the pruned
    stream plus GemmNT 8192x4096x16 (dX through the LoRA branch), GemmNT
    8192x4096x4096 (dX through W) and their AddEW: 17 instructions."""
    w = configs.make("c2dx")
    p = planner.compile_update(w.model, w.cfg, materialize=False)
    base = planner.compile_update(configs.make("c2").model, configs.make("c2").cfg,
                                  materialize=False)
    assert len(base.train) == 14 and len(p.train) == 17
    extra = collections.Counter((planner.OP_NAME[i["opcode"]], tuple(i["out"])) for i in p.train)
    extra.subtract((planner.OP_NAME[i["opcode"]], tuple(i["out"])) for i in base.train)
    assert +extra == collections.Counter({("GemmNT", (8192, 4096, 16)): 1,
                                          ("GemmNT", (8192, 4096, 4096)): 1,
                                          ("AddEW", (8192 * 4096, 0, 0)): 1})


def test_plan_hash_matches_reference(ref):
    for n in (0, 1, 7, 64, (1 << 20) - 1, 1 << 20, (1 << 20) * 3 + 5, 300 * (1 << 20) + 3):
        blob = np.random.default_rng(n).integers(0, 256, n).astype(np.uint8)
        ours = _lib.lib().seeml_hip_plan_self_hash(blob.ctypes.data, n, 216)
        assert ours == ref.plan_self_hash(blob, n, 216), n
        assert (_lib.lib().seeml_hip_content_hash64(blob.ctypes.data, n)
                == ref.content_hash64(blob, n)), n


@pytest.mark.parametrize("name", ["c1", "c2s", "c2sdx", "c3s", "c4s", "c5s", "c3m", "c4m", "c4mr"])
def test_compiled_plans_verify_and_corruption_is_caught(name):
    w, p = compile_workload(name)
    assert verify_plan(p.blob) == (0, "")
    bad = bytearray(p.blob)
    bad[len(bad) // 2] ^= 0x10
    rc, msg = verify_plan(bytes(bad))
    assert rc == 1 and msg.startswith("UpdateEngine: plan hash mismatch")


def reseal(blob: bytearray):
    struct.pack_into("<Q", blob, 216, 0)
    buf = np.frombuffer(bytes(blob), np.uint8)
    h = _lib.lib().seeml_hip_plan_self_hash(buf.ctypes.data, len(blob), 216)
    struct.pack_into("<Q", blob, 216, h)
    return bytes(blob)


def test_loader_contracts_reject_malformed_headers():
    w, p = compile_workload("c1")
    h = p.header

    def patched(field, value):
        b = bytearray(p.blob)
        fields = dict(h)
        fields[field] = value
        fields["plan_hash"] = 0
        planner.HEADER.pack_into(b, 0, *[fields[n] for n, _ in planner.HEADER_FIELDS])
        return reseal(b)

    assert verify_plan(patched("version", 3))[1].startswith("UpdateEngine: unsupported plan version 3")
    assert verify_plan(patched("version", 8))[1].startswith("UpdateEngine: unsupported plan version 8")
    assert "batch size is zero" in verify_plan(patched("batch", 0))[1]
    assert "persistent segment exceeds arena" in verify_plan(
        patched("persistent_size", h["arena_size"] + 64))[1]
    assert "loss slot out of bounds" in verify_plan(patched("loss_ref", h["arena_size"]))[1]
    assert "input slot out of bounds" in verify_plan(patched("input_ref", 2))[1]
    assert "section out of bounds" in verify_plan(patched("rodata_size", 1 << 40))[1]
    assert verify_plan(patched("magic", 0))[1] == "UpdateEngine: bad plan magic"
    rc, msg = verify_plan(b"\0" * 100)
    assert msg == "UpdateEngine: plan smaller than its header"


def test_softmax_labels_must_be_the_label_slot():
    w, p = compile_workload("c1")
    b = bytearray(p.blob)
    h = p.header
    for i in range(h["train_instr_count"]):
        off = h["train_instr_offset"] + 64 * i
        if struct.unpack_from("<H", b, off)[0] == 11:  # SoftmaxXEntFwd: move the labels ref
            struct.pack_into("<Q", b, off + 8 + 8, h["input_ref"])
    rc, msg = verify_plan(reseal(b))
    assert msg in ("UpdateEngine: softmax labels are not the plan's staged label slot",
                   "PlanValidator: instruction operands alias a written range (opcode 11)")


def test_library_exports_every_declared_symbol():
    declared = set(_lib.parse_header())
    lib = _lib.lib()
    for name in declared:
        assert hasattr(lib, name), name
    text = open(_lib.HEADER).read()
    assert len(declared) == len(set(re.findall(r"\b(seeml_hip_\w+)\s*\(", text)))


@pytest.mark.parametrize("name,steps", [("c1", 3), ("c3s", 2), ("c5s", 2), ("c2s", 2), ("c2sdx", 2),
                                        ("c4m", 1), ("f1", 14), ("f2", 3), ("q1", 3), ("k1", 2),
                                        ("k2", 2)])
def test_oracle_dispatch_bitwise_equals_reference_dispatch(orc, ref, name, steps):
    """orc_execute (the C restatement) and ref_execute (the reference's own
    kernels) run the same compiled plan for several steps: every arena byte
    agrees, which pins the oracle's dispatcher and kernels end to end."""
    w, p = compile_workload(name)
    a, b = HostPlanRunner(p, orc), HostPlanRunner(p, ref)
    for s in range(steps):
        x, y = configs.batch(w, s)
        la, lb = a.train_step(x, y), b.train_step(x, y)
        assert np.float32(la).view(np.uint32) == np.float32(lb).view(np.uint32)
    assert np.array_equal(a.arena.view(np.uint32), b.arena.view(np.uint32))
    a.run(1)
    b.run(1)
    assert np.array_equal(a.arena.view(np.uint32), b.arena.view(np.uint32))


def test_oracle_training_reduces_loss_c1(orc):
    w, p = compile_workload("c1")
    r = HostPlanRunner(p, orc)
    x, y = configs.batch(w, 0)
    losses = [r.train_step(x, y) for _ in range(30)]
    assert losses[-1] < losses[0] * 0.9


def test_lora_init_matches_counter_randn_statistics():
    a = planner.counter_randn(7, 200000)
    assert abs(float(a.mean())) < 0.01 and abs(float(a.std()) - 1.0) < 0.01
    # element j depends only on (seed, j): a prefix is stable
    assert np.array_equal(planner.counter_randn(7, 100), a[:100])


# ---- plans carrying the ABI's remaining instruction kinds -----------------

def _kinds(p):
    out = collections.Counter()
    for prog in (p.train, p.eval, p.merge):
        for ins in prog:
            out[(planner.OP_NAME[ins["opcode"]], ins["flags"])] += 1
    return out


def test_abi_workloads_carry_every_remaining_instruction_kind():
    """The compiler restatement emits what the reference compiler emits for
    these configs (source/plan/config.h:56-81): fused GEMM epilogues with
    every bias/activation combination the fuser forms (epilogue_fuser.cc:
    55-112; flags per instruction.h:106-134), q8 GEMMs with the scale in
    in[3] and an activation-only epilogue, ClipNorm before each optimizer
    step, SGD, the KL-distillation pair, and the LR schedule header."""
    seen = collections.Counter()
    for n in ("f1", "f2", "q1", "k1", "k2"):
        w, p = compile_workload(n)
        assert verify_plan(bytes(p.blob)) == (0, ""), n
        seen.update(_kinds(p))
    for flags in (1, 3, 4, 5, 7):   # bias; bias+relu; gelu; bias+gelu; bias+silu
        assert seen[("GemmNN", flags)] > 0, flags
    assert seen[("GemmNNQ8", 6)] > 0 and seen[("GemmNNQ8", 0)] > 0 and seen[("GemmNTQ8", 0)] > 0
    for op in ("ClipNorm", "SgdStep", "KLDistillFwd", "KLDistillBwd"):
        assert seen[(op, 0)] > 0, op
    w, p = compile_workload("f1")
    assert (p.header["lr_schedule"], p.header["warmup_steps"], p.header["default_steps"]) == (1, 3, 12)
    # ClipNorm precedes each parameter's optimizer step (optimizer.cc:24-30)
    names = [planner.OP_NAME[i["opcode"]] for i in p.train]
    steps = [k for k, nm in enumerate(names) if nm == "AdamWStep"]
    assert all(names[k - 1] == "ClipNorm" for k in steps)
    w, p = compile_workload("f2")
    assert p.header["optimizer_kind"] == 0
    w, p = compile_workload("k1")
    assert p.header["label_kind"] == 0 and p.header["label_ref"] == NULL


def test_fused_epilogue_plans_equal_the_unfused_plan_bitwise(orc):
    """Fusion changes memory traffic, never bits (instruction.h:106-112): the
    same model compiled with and without fuse_epilogues trains to the same
    loss and adapter bits on the oracle."""
    for n in ("f1", "f2"):
        w = configs.make(n)
        fused = planner.compile_update(w.model, w.cfg)
        cfg = planner.UpdateConfig(**{**w.cfg.__dict__, "fuse_epilogues": False})
        plain = planner.compile_update(w.model, cfg)
        assert len(fused.train) < len(plain.train)
        a, b = HostPlanRunner(fused, orc), HostPlanRunner(plain, orc)
        for s in range(4):
            x, y = configs.batch(w, s)
            la, lb = a.train_step(x, y), b.train_step(x, y)
            assert np.float32(la).view(np.uint32) == np.float32(lb).view(np.uint32)
        n_p = fused.header["persistent_size"] // 4
        assert np.array_equal(a.read(0, n_p).view(np.uint32), b.read(0, n_p).view(np.uint32))


def test_int8_pack_known_answers():
    """The binder's per-tensor symmetric pack (arena_binder.cc:135-160) and
    the quantizer's scale (reviewer/quantization.cc:29-52): halves round
    away from zero (std::round), values clamp to [-127, 127], an all-zero
    tensor takes scale 1, and a subnormal scale deselects the tensor."""
    vals = np.array([0.0, 1.27, -1.27, 0.005, -0.005, 0.015, 0.6349999, 2.0], np.float32)
    sc = planner.quant_scale(vals)
    assert sc == np.float32(np.float32(2.0) / np.float32(127.0))
    q = planner.quantize_int8(vals, np.float32(0.01))
    assert list(q) == [0, 127, -127, 1, -1, 2, 63, 127]
    assert planner.quant_scale(np.zeros(5, np.float32)) == np.float32(1.0)
    assert planner.quant_scale(np.full(3, 1e-37, np.float32)) is None
    # a q8 plan's int8 rodata dequantizes back within half a step
    w, p = compile_workload("q1")
    INV = {v: k for k, v in planner.OP.items()}
    q8 = [i for i in p.train if INV[i["opcode"]] == "GemmNNQ8"]
    assert q8 and all(np.array([i["inp"][3]], np.uint64).astype(np.uint32).view(np.float32)[0] > 0
                      for i in q8)


@pytest.mark.parametrize("lr,warmup,horizon,floor", [(0.1, 10, 100, 0.1), (1e-2, 3, 12, 0.1),
                                                     (1e-3, 0, 50, 0.0), (5e-4, 20, 10, 0.25)])
def test_backend_effective_lr_equals_the_oracle(orc, lr, warmup, horizon, floor):
    """seeml_hip_effective_lr (the scalar the engine uploads each step) reads
    the schedule from a plan header and equals the oracle's restatement of
    UpdateEngine::EffectiveLr (update_engine.cc:515-534) bit for bit at every
    step, with the reference's boundary behaviour (update_engine_test.cc:
    811-841): the warmup ramp, exactly lr at the warmup boundary, monotone
    cosine decay, the floor at the horizon and beyond."""
    import ctypes as C
    h = dict((n, 0) for n, _ in planner.HEADER_FIELDS)
    h.update(lr=lr, lr_schedule=1, warmup_steps=warmup, default_steps=horizon,
             min_lr_factor=floor)
    raw = planner.HEADER.pack(*[h[n] for n, _ in planner.HEADER_FIELDS])
    buf = (C.c_uint8 * len(raw)).from_buffer_copy(raw)
    L = _lib.lib()
    got = np.array([L.seeml_hip_effective_lr(buf, s) for s in range(1, 3 * horizon + 30)],
                   np.float32)
    want = np.array([orc.effective_lr(lr, 1, warmup, horizon, floor, s)
                     for s in range(1, 3 * horizon + 30)], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    base, fl = np.float32(lr), np.float32(lr) * np.float32(floor)
    if warmup:
        assert got[0] == np.float32(base * np.float32(1) / np.float32(warmup))
        assert got[warmup - 1] == base
    if horizon > warmup:
        decay = got[warmup:horizon - 1]
        assert np.all(np.diff(decay) <= 0) and np.all(decay < base) and np.all(decay > fl)
        assert got[horizon - 1] == fl
    assert np.all(got[max(horizon, warmup):] == fl)
    h["lr_schedule"] = 0
    raw0 = planner.HEADER.pack(*[h[n] for n, _ in planner.HEADER_FIELDS])
    buf0 = (C.c_uint8 * len(raw0)).from_buffer_copy(raw0)
    assert L.seeml_hip_effective_lr(buf0, 7) == np.float32(lr)


def test_summarize_takes_a_fused_launchs_work_over_its_instructions():
    """workmodel.summarize with the engine's launch work: a colsum group of
    three over one x [K, M] — two operand copies and the group's launch —
    counts x once (not once per member) and credits the members' FLOPs to
    the launch, none to the copies."""
    from seeml_amd import workmodel
    M, N, K = 2048, 16, 8192
    ins = dict(opcode=planner.OP["GemmTN"], flags=0, inp=(0, 0, 0, 0), out=(M, N, K))
    prog = [ins, ins, ins]
    lone = workmodel.work(ins)
    x_bytes, small, out = 4 * K * M, 4 * K * N, 4 * M * N
    assert lone["bytes"] == x_bytes + small + out and lone["flops"] == 2 * M * N * K
    group = (3 * lone["flops"], x_bytes + 3 * (small + out))
    launches = [(0.0, 2.0 * small), (0.0, 2.0 * small), group]
    s = workmodel.summarize(prog, [0.01, 0.01, 0.05], variants=["", "", ""], launches=launches)
    total_bytes = sum(r["bytes"] for r in s["rows"])
    assert total_bytes == 4 * small + x_bytes + 3 * (small + out)
    assert sum(r["flops"] for r in s["rows"]) == 3 * lone["flops"]
    assert [r["flops"] for r in s["rows"][:2]] == [0, 0]
    assert s["hbm_skinny_gemm_gbps"] == pytest.approx(total_bytes / 0.07e-3 / 1e9)
    naive = workmodel.summarize(prog, [0.01, 0.01, 0.05], variants=["", "", ""])
    assert naive["hbm_skinny_gemm_gbps"] > 2 * s["hbm_skinny_gemm_gbps"]
