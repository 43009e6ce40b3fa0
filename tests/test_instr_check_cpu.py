"""The full-size per-instruction checker (instr_check.py), pinned on the
CPU: driven through a stand-in engine that executes instructions with the
oracle itself, it must accept every checked group of the reduced plans
(oracle against oracle), and a perturbed output must make it fail. This
pins its operand decoding before it judges the device."""
import numpy as np
import pytest

from helpers import HostPlanRunner, compile_workload
from instr_check import CHECKED, OPN, replay_and_check
from seeml_amd import configs


class OracleEngine:
    """The engine calls replay_and_check makes, served by HostPlanRunner."""

    def __init__(self, plan, orc, corrupt=None):
        self.r = HostPlanRunner(plan, orc)
        self.h = plan.header
        self.corrupt = corrupt  # opcode name whose output gets one ulp

    def read(self, ref, count):
        if int(ref) >> 63:
            off = int(ref) & ~(1 << 63)
            return self.r.rodata.view(np.uint8)[off:off + 4 * count].view(np.float32).copy()
        return self.r.read(ref, count)

    def write(self, ref, data):
        a8 = self.r.arena.view(np.uint8)
        b = np.ascontiguousarray(data).view(np.uint8)
        a8[ref:ref + b.size] = b

    def stage(self, x, y):
        self.r.stage(x, y)

    def set_step(self, s):
        self.r.step = s

    def run_range(self, program, begin, end):
        prog, _ = self.r.programs[program]
        h = self.h
        import oracle
        lr = oracle.oracle().effective_lr(h["lr"], h["lr_schedule"], h["warmup_steps"],
                                          h["default_steps"], h["min_lr_factor"], self.r.step)
        if end > begin:
            self.r.lib.execute(np.ascontiguousarray(prog[64 * begin:64 * end]), end - begin,
                               self.r.arena, self.r.rodata, lr, h["beta1"], h["beta2"], h["eps"],
                               h["weight_decay"], self.r.step)
        if self.corrupt and end == begin + 1:
            ins = self.r.plan.train[begin]
            if OPN[ins["opcode"]] == self.corrupt:
                out = int(ins["inp"][2])
                v = self.r.read(out, 1)
                self.write(out, np.nextafter(v, np.float32(np.inf)) * np.float32(1.5))

    def loss(self):
        return self.r.loss()


@pytest.mark.parametrize("name", ["c1", "c2sdx", "c3m", "c4m", "c5s", "f1", "q1", "k2"])
def test_checker_accepts_the_oracle(orc, name):
    w, p = compile_workload(name)
    e = OracleEngine(p, orc)
    x, y = configs.batch(w, 0)
    seen = replay_and_check(e, p, orc, p.train, x, y, step=1)
    assert {k[0] for k in seen} == {OPN[i["opcode"]] for i in p.train} & CHECKED


@pytest.mark.parametrize("op", ["GemmNN", "GemmTN", "AddEW", "RmsNormFwd"])
def test_checker_rejects_a_wrong_output(orc, op):
    w, p = compile_workload("c4m")
    e = OracleEngine(p, orc, corrupt=op)
    x, y = configs.batch(w, 0)
    with pytest.raises(AssertionError):
        replay_and_check(e, p, orc, p.train, x, y, step=1)
