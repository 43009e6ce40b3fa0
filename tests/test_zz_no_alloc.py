"""seeml_hip_gemm_tn_noalloc: GemmTN for callers that cannot allocate.

It runs seeml_hip_gemm_tn's plan and kernels with its scratch in a fixed
per-GPU device array (SEEML_HIP_NOALLOC_SCRATCH_BYTES) instead of the
library's growable workspace, so its output must equal seeml_hip_gemm_tn's
bit for bit — on consecutive calls that reuse the array (the second with a
smaller input) — and the oracle's to the GEMM tolerance. A shape whose plan
needs more scratch than the array holds is rejected before any launch."""
import ctypes as C

import numpy as np
import pytest

from helpers import TOL_STEP, rel_err
from seeml_amd import _lib

f32 = np.float32
SCRATCH = 16 << 20

# Oversized: an unbatched 960x960 TN over K = 8192 plans 8 split-K slices
# on 128x128 tiles, 8 * 960 * 960 * 4 = 29.5 MB of partials.
OVERSIZED = (960, 960, 8192)


def test_noalloc_rejects_a_shape_beyond_its_scratch():
    """Host only: the size check runs before any HIP call (the pointers are
    never dereferenced)."""
    L = _lib.lib()
    M, N, K = OVERSIZED
    rc = L.seeml_hip_gemm_tn_noalloc(0x100000, 0x200000, 0x300000, M, N, K, None)
    assert rc == 1
    msg = L.seeml_hip_kernel_error().decode()
    assert msg.startswith("UpdateEngine: GemmTN(no-alloc): this shape needs 29491200 bytes"), msg
    assert str(SCRATCH) in msg


@pytest.mark.gpu
def test_noalloc_gemm_tn_equals_the_allocating_entry_point(orc):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L = _lib.lib()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    # LoRA gradient shapes (skinny colsum: k-group partials in the scratch)
    # and dense TN shapes with split-K partials; each pair runs the larger
    # input first, then a smaller one over the same scratch.
    cases = [(2048, 16, 8192), (512, 16, 1024),
             (64, 4096, 8192), (16, 520, 1000),
             (256, 192, 4096), (200, 136, 520)]
    for i, (M, N, K) in enumerate(cases):
        print(f"noalloc GemmTN case {i}: M={M} N={N} K={K}", flush=True)
        rng = np.random.default_rng(100 + i)
        A = rng.standard_normal(K * M).astype(f32)
        B = rng.standard_normal(K * N).astype(f32)
        tA, tB = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
        got = torch.full((M * N,), float("nan"), device=dev)
        want = torch.full((M * N,), float("nan"), device=dev)
        assert L.seeml_hip_gemm_tn_noalloc(tA.data_ptr(), tB.data_ptr(), got.data_ptr(),
                                           M, N, K, stream) == 0, L.seeml_hip_kernel_error()
        assert L.seeml_hip_gemm_tn(tA.data_ptr(), tB.data_ptr(), want.data_ptr(),
                                   M, N, K, stream) == 0, L.seeml_hip_kernel_error()
        torch.cuda.synchronize()
        g, w = got.cpu().numpy(), want.cpu().numpy()
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), (M, N, K)
        ref = np.zeros(M * N, f32)
        orc.gemm_tn(A, B, ref, M, N, K)
        assert rel_err(g, ref) <= TOL_STEP, (M, N, K)
    # the oversized shape is rejected on the GPU too, before any launch
    M, N, K = OVERSIZED
    a = torch.zeros(K * M, device=dev)
    b = torch.zeros(K * N, device=dev)
    c = torch.full((M * N,), 7.0, device=dev)
    assert L.seeml_hip_gemm_tn_noalloc(a.data_ptr(), b.data_ptr(), c.data_ptr(), M, N, K,
                                       stream) == 1
    torch.cuda.synchronize()
    assert bool((c == 7.0).all())


_CHILD = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
from seeml_amd import _lib
L = _lib.lib()
dev = torch.device("cuda:0")
s = torch.cuda.current_stream().cuda_stream

def call(M, N, K):
    a = torch.randn(K * M, device=dev)
    b = torch.randn(K * N, device=dev)
    c = torch.empty(M * N, device=dev)
    torch.cuda.synchronize()
    return a, b, c

# warm-up through the no-alloc entry point only: code objects loaded, the
# scratch symbol looked up, on a skinny colsum and a split-K tile shape
for M, N, K in ((64, 16, 512), (192, 136, 1024)):
    a, b, c = call(M, N, K)
    assert L.seeml_hip_gemm_tn_noalloc(a.data_ptr(), b.data_ptr(), c.data_ptr(), M, N, K, s) == 0
torch.cuda.synchronize()
# a split-K shape whose partials (8 slices of 512 x 512) fill half the scratch
M, N, K = 512, 512, 1024
a, b, c = call(M, N, K)
free0 = torch.cuda.mem_get_info()[0]
for _ in range(3):
    assert L.seeml_hip_gemm_tn_noalloc(a.data_ptr(), b.data_ptr(), c.data_ptr(), M, N, K, s) == 0, \
        L.seeml_hip_kernel_error()
torch.cuda.synchronize()
free1 = torch.cuda.mem_get_info()[0]
print(f"noalloc child: free device memory {free0} -> {free1}", flush=True)
assert free1 == free0, (free0, free1)
# the allocating entry point, by contrast, grows its workspace here
assert L.seeml_hip_gemm_tn(a.data_ptr(), b.data_ptr(), c.data_ptr(), M, N, K, s) == 0
torch.cuda.synchronize()
free2 = torch.cuda.mem_get_info()[0]
print(f"noalloc child: after the allocating entry point {free2}", flush=True)
assert free2 < free1, (free1, free2)
print("noalloc child ok", flush=True)
"""


@pytest.mark.gpu
def test_noalloc_allocates_no_device_memory():
    """The entry point's promise itself, in a fresh process (no library
    workspace yet, so any allocation on its path would show): free device
    memory is unchanged across three calls whose plan needs megabytes of
    split-K partials, while the allocating entry point's first call with
    the same shape takes memory. A child process, not an exec."""
    import os
    import subprocess
    import sys
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "see-ml_amd")
    r = subprocess.run([sys.executable, "-c", _CHILD, pkg], capture_output=True, text=True,
                       timeout=240)
    print(r.stdout, r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "noalloc child ok" in r.stdout
