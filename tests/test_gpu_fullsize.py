"""The BASELINE configs at their own size on the GPU.

C3 (vocab 8192, d_model 512, 4 layers, S = 256, 16 sequences, LoRA r8 on
q/v) runs two whole steps against the reference's own executor kernels
(oracle/_ref, ParallelFor on the host's cores): losses and the trained
state within the north star's per-step bar.

C2 (with and without the input's dX), C4 and C5 are too large for a CPU
step, so each is checked the way the bench runs it and then instruction by
instruction:
  1. the plan is opened and autotuned exactly as bench.py does, and two
     steps run through the fused hipGraph (LoRA runs, GEMM epilogue chains,
     pointwise runs, Scale folds, dual passes, rowdot and colsum groups,
     causal tails, column splits);
  2. the persistent state after step 1 is put back and step 2 is replayed
     eagerly, one instruction at a time; the first instruction of every
     (opcode, shape) group, and of every fused variant the graph runs it
     as (the engine's gemm_choice), is checked against the oracle on the
     inputs the device held (instr_check.py);
  3. the replay's loss and trained state equal the graph's step 2 bit for
     bit.
Step 2, not step 1: the plan's initial image has LoRA B = 0, so at step 1
the LoRA up-projection t*B, dt = du*B^T, dA = X^T*dt and the dt*A^T input
gradient are exactly zero and a check of them would compare zeros. After
one AdamW step B is nonzero (as the reference's own gradient checks nudge
B off zero, test/system/update_system_test.cc:141-151); the test asserts
that every checked GEMM's oracle output has a nonzero entry. So every
kernel variant the bench times is checked on live data: the eager replay
runs the same autotuned tile plans, and the graph differs from it only by
fusions that must give the same bits."""
import os

import numpy as np
import pytest

from helpers import TOL_STEP, HostPlanRunner, compile_workload, rel_err
from instr_check import CHECKED, OPN, replay_and_check
from seeml_amd import configs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _host_threads() -> int:
    # the GPU box's CPU share is 16 cores per GPU, whatever os.cpu_count says
    return max(1, min(16, os.cpu_count() or 1))


def test_c3_full_size_parity_vs_reference_kernels(torch_gpu, ref):
    from seeml_amd import DeviceUpdateEngine
    ref.set_threads(_host_threads())
    w, p = compile_workload("c3")
    e = DeviceUpdateEngine(p.blob)
    r = HostPlanRunner(p, ref)
    for s in range(2):
        x, y = configs.batch(w, s)
        lg, lr = e.train_step(x, y), r.train_step(x, y)
        assert abs(lg - lr) <= TOL_STEP * abs(lr), (s, lg, lr)
    n = p.header["persistent_size"] // 4
    assert rel_err(e.read(0, n), r.read(0, n)) <= TOL_STEP
    e.close()


@pytest.mark.parametrize("name", ["c2", "c2dx", "c4", "c5"])
def test_full_size_graph_step_equals_the_checked_eager_replay(torch_gpu, orc, name):
    from seeml_amd import PROGRAM_TRAIN, DeviceUpdateEngine
    w, p = compile_workload(name)
    n = p.header["persistent_size"] // 4
    e = DeviceUpdateEngine(p.blob)
    e.autotune(16)  # as bench.py
    x0, y0 = configs.batch(w, 0)
    x1, y1 = configs.batch(w, 1)
    assert np.isfinite(e.train_step(x0, y0))
    state1 = e.read(0, n)
    loss_graph = e.train_step(x1, y1)
    state_graph = e.read(0, n)
    assert np.isfinite(loss_graph)
    bs = [(pid, ref, cnt) for pid, ref, _, cnt in p.params if pid.endswith(".lora_B")]
    assert bs
    for pid, ref, cnt in bs:
        assert np.any(e.read(ref, cnt) != 0), pid  # step 2 runs with B != 0
    e.write(0, state1)
    checked = replay_and_check(e, p, orc, p.train, x1, y1, step=2,
                               variants=lambda j: e.gemm_choice(PROGRAM_TRAIN, j),
                               progress=lambda j, key: print(f"  checked #{j} {key}", flush=True))
    loss_eager = e.loss()
    assert np.float32(loss_eager).view(np.uint32) == np.float32(loss_graph).view(np.uint32)
    assert np.array_equal(e.read(0, n).view(np.uint32), state_graph.view(np.uint32))
    in_plan = {OPN[i["opcode"]] for i in p.train} & CHECKED
    assert {k[0] for k in checked} == in_plan
    zero = [k for k, peak in checked.items() if peak is not None and not peak > 0]
    assert not zero, zero
    print(f"{name}: {len(checked)} (group, variant) checks, "
          f"{sum(v is not None for v in checked.values())} GEMM")
    e.close()
