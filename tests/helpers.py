"""Shared test helpers: instruction encoding, the oracle-side plan runner,
and the parity tolerance used across the GPU tests."""
import ctypes as C
import os
import struct
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "see-ml_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

from seeml_amd import _lib, configs, planner  # noqa: E402

NULL = planner.NULL_REF
RO = planner.RODATA_BIT

# Parity bar: fp32 results within max rel err
# 1e-4 per step and 1e-3 after 100 steps, where rel err is normwise:
# max|gpu - ref| / max|ref| over the tensor.
TOL_STEP = 1e-4
TOL_100 = 1e-3


def rel_err(got, want) -> float:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(float(np.max(np.abs(want))) if want.size else 0.0, 1e-30)
    return float(np.max(np.abs(got - want))) / scale if want.size else 0.0


def instr(opcode, inp=(NULL, NULL, NULL, NULL), out=(0, 0, 0), flags=0) -> bytes:
    inp = list(inp) + [NULL] * (4 - len(inp))
    out = list(out) + [0] * (3 - len(out))
    return planner.INSTR.pack(opcode, flags, 0, *inp, *out)


def validate(ins: bytes, arena: int, rodata: int, version: int = 7):
    err = C.create_string_buffer(512)
    buf = (C.c_uint8 * 64).from_buffer_copy(ins)
    rc = _lib.lib().seeml_hip_validate_instruction(buf, arena, rodata, version, err, 512)
    return rc, err.value.decode()


def verify_plan(blob: bytes):
    err = C.create_string_buffer(1024)
    buf = (C.c_uint8 * len(blob)).from_buffer_copy(blob)
    rc = _lib.lib().seeml_hip_verify_plan(buf, len(blob), err, 1024)
    return rc, err.value.decode()


def compile_workload(name: str, hash_fn=None):
    w = configs.make(name)
    return w, planner.compile_update(w.model, w.cfg, hash_fn=hash_fn, teacher=w.teacher)


def append_train_instructions(plan, words: list, extra_arena: int = 0):
    """A copy of compiled `plan` with the 64-byte instruction words `words`
    appended to its train program and the arena grown by `extra_arena`
    bytes (room for their outputs), re-sealed. Returns (blob, header)."""
    h = dict(plan.header)
    n = len(words)
    old = bytes(plan.blob)
    t_end = h["train_instr_offset"] + 64 * h["train_instr_count"]
    blob = bytearray(old[:t_end] + b"".join(words) + old[t_end:])
    for k in ("merge_instr_offset", "eval_instr_offset", "rodata_offset", "persist_init_offset",
              "emit_table_offset"):
        h[k] += 64 * n
    h["train_instr_count"] += n
    h["arena_size"] = planner.align_up(h["arena_size"] + extra_arena)
    h["plan_hash"] = 0
    planner.HEADER.pack_into(blob, 0, *[h[k] for k, _ in planner.HEADER_FIELDS])
    buf = (C.c_uint8 * len(blob)).from_buffer(blob)
    h["plan_hash"] = _lib.lib().seeml_hip_plan_self_hash(buf, len(blob), planner.PLAN_HASH_OFFSET)
    del buf
    struct.pack_into("<Q", blob, planner.PLAN_HASH_OFFSET, h["plan_hash"])
    return blob, h


class PlanView:
    """The fields HostPlanRunner reads from a compiled plan, for a raw blob."""

    def __init__(self, blob, header):
        self.blob, self.header = blob, header


class HostPlanRunner:
    """Runs a compiled plan on the CPU through an oracle library's execute
    (orc_execute / ref_execute): the host-side counterpart of the device
    engine, used as the parity reference. TEST INFRASTRUCTURE ONLY."""

    def __init__(self, plan, lib):
        self.plan = plan
        self.lib = lib
        h = plan.header
        self.h = h
        self.arena = np.zeros(planner.align_up(h["arena_size"]) // 4 + 16, np.float32)
        blob = np.frombuffer(plan.blob, np.uint8)
        p0, ps = h["persist_init_offset"], h["persist_init_size"]
        self.arena.view(np.uint8)[:ps] = blob[p0:p0 + ps]
        r0, rs = h["rodata_offset"], h["rodata_size"]
        self.rodata = np.zeros(max(rs, 64) // 4 + 16, np.float32)
        self.rodata.view(np.uint8)[:rs] = blob[r0:r0 + rs]
        self.programs = {}
        for k, (off, cnt) in enumerate(((h["train_instr_offset"], h["train_instr_count"]),
                                        (h["merge_instr_offset"], h["merge_instr_count"]),
                                        (h["eval_instr_offset"], h["eval_instr_count"]))):
            self.programs[k] = (np.frombuffer(plan.blob[off:off + 64 * cnt], np.uint8).copy(), cnt)
        self.step = 0

    def stage(self, x, y):
        h = self.h
        a8 = self.arena.view(np.uint8)
        xb = np.ascontiguousarray(x).view(np.uint8)
        a8[h["input_ref"]:h["input_ref"] + xb.size] = xb
        if h["label_kind"] and y is not None:
            yb = np.ascontiguousarray(y).view(np.uint8)
            a8[h["label_ref"]:h["label_ref"] + yb.size] = yb

    def run(self, program=0, lr=None):
        h = self.h
        prog, cnt = self.programs[program]
        step = self.step if self.step else 1
        if lr is None:
            import oracle
            lr = oracle.oracle().effective_lr(h["lr"], h["lr_schedule"], h["warmup_steps"],
                                              h["default_steps"], h["min_lr_factor"], step)
        self.lib.execute(prog, cnt, self.arena, self.rodata, lr, h["beta1"], h["beta2"],
                         h["eps"], h["weight_decay"], step)

    def loss(self):
        return float(self.arena.view(np.uint8)[self.h["loss_ref"]:self.h["loss_ref"] + 4]
                     .view(np.float32)[0])

    def train_step(self, x, y):
        self.step += 1
        self.stage(x, y)
        self.run(0)
        return self.loss()

    def write(self, ref, data):
        b = np.ascontiguousarray(data).view(np.uint8)
        self.arena.view(np.uint8)[ref:ref + b.size] = b

    def read(self, ref, count, dtype=np.float32):
        a8 = self.arena.view(np.uint8)
        nb = count * np.dtype(dtype).itemsize
        return a8[ref:ref + nb].view(dtype).copy()
