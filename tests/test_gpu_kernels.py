"""GPU parity of every standalone kernel entry point (C-ABI, device
pointers) against the C oracle on the same seeded inputs.

Bars: bit-exact for the pointwise, optimizer, gather, label-indexed and
column-reduction kernels (their per-element expressions round exactly as the
reference's); normwise max rel err <= 1e-4 (TOL_STEP) for everything that
reorders an fp32 reduction (GEMM/MFMA, softmax sums) or calls the device
libm (exp/tanh/sin/cos). Every kernel is also re-run to show run-to-run
bitwise determinism."""
import math

import numpy as np
import pytest

from helpers import TOL_STEP, rel_err

pytestmark = pytest.mark.gpu

f32 = np.float32


@pytest.fixture(scope="module")
def env():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from seeml_amd import _lib
    L = _lib.lib()
    dev = torch.device("cuda:0")

    class Env:
        pass

    e = Env()
    e.torch, e.L, e.dev = torch, L, dev
    e.T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    e.H = lambda t: t.detach().cpu().numpy()
    e.s = lambda: torch.cuda.current_stream().cuda_stream

    def call(name, *args):
        rc = getattr(L, name)(*[a.data_ptr() if hasattr(a, "data_ptr") else a for a in args],
                              e.s())
        torch.cuda.synchronize()
        assert rc == 0, f"{name}: {L.seeml_hip_kernel_error().decode()}"

    e.call = call
    return e


def rnd(n, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(n) * scale).astype(f32)


def same_bits(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


GEMM_SHAPES = [
    (1, 1, 1), (3, 5, 7), (33, 47, 131), (128, 128, 128), (257, 129, 64), (64, 16, 256),
    (512, 16, 1024), (16, 512, 1024), (1024, 512, 16), (300, 200, 9), (8, 8, 4096),
]


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_gemm_family(env, orc, M, N, K):
    A, B, Bt, At, bias = rnd(M * K, 1), rnd(K * N, 2), rnd(N * K, 3), rnd(K * M, 4), rnd(N, 5)
    for act in range(4):
        want = np.zeros(M * N, f32)
        orc.gemm_nn(A, B, want, M, N, K, bias, act)
        out = env.T(np.full(M * N, np.nan, f32))
        env.call("seeml_hip_gemm_nn", env.T(A), env.T(B), out, M, N, K, env.T(bias), act)
        assert rel_err(env.H(out), want) <= TOL_STEP, ("nn", act)
    want = np.zeros(M * N, f32)
    orc.gemm_nt(A, Bt, want, M, N, K)
    out = env.T(np.full(M * N, np.nan, f32))
    env.call("seeml_hip_gemm_nt", env.T(A), env.T(Bt), out, M, N, K)
    assert rel_err(env.H(out), want) <= TOL_STEP
    want = np.zeros(M * N, f32)
    orc.gemm_tn(At, B, want, M, N, K)
    out = env.T(np.full(M * N, np.nan, f32))
    env.call("seeml_hip_gemm_tn", env.T(At), env.T(B), out, M, N, K)
    got1 = env.H(out)
    assert rel_err(got1, want) <= TOL_STEP
    env.call("seeml_hip_gemm_tn", env.T(At), env.T(B), out, M, N, K)
    assert same_bits(env.H(out), got1), "run-to-run bits differ"


@pytest.mark.parametrize("layout", [0, 1, 2])
def test_gemm_every_tile_config_and_split(env, orc, layout):
    M, N, K = 200, 136, 520
    A = rnd(M * K, 11)
    B = rnd(K * N, 12)
    want = np.zeros(M * N, f32)
    if layout == 0:
        orc.gemm_nn(A, B, want, M, N, K, None, 0)
    elif layout == 1:
        orc.gemm_nt(A, B, want, M, N, K)
    else:
        orc.gemm_tn(A, B, want, M, N, K)
    ncfg = env.L.seeml_hip_gemm_config_count()
    for cfg in range(ncfg):
        for splits in (1, 3):
            out = env.T(np.full(M * N, np.nan, f32))
            env.call("seeml_hip_gemm_forced", layout, env.T(A), env.T(B), out, M, N, K, cfg, splits)
            assert rel_err(env.H(out), want) <= TOL_STEP, (cfg, splits)


@pytest.mark.parametrize("layout,M,N,K", [(1, 512, 64, 512), (1, 300, 64, 292), (1, 256, 48, 1024),
                                           (2, 64, 512, 512), (2, 48, 260, 300), (2, 64, 136, 1024)])
def test_gemm_scaled_loads_are_bitwise_the_scale_then_the_gemm(env, orc, layout, M, N, K):
    """A Scale folded into a tile GEMM's streamed operand (the rank-64 LoRA
    backward's dt = (s du) B^T, NT with A scaled, and dB = t^T (s du), TN with
    B scaled) equals, bit for bit, the Scale into a buffer and then the GEMM
    on the same plan: every scaled tile config, split-K or not, a K with a
    partial last stage, and a negative factor."""
    A, B = rnd(M * K, 81), rnd(K * N, 82)
    scale = f32(-0.37)
    sa = layout == 1  # NT: A is the stream; TN: B
    x = A if sa else B
    xs = env.T(np.full(x.size, np.nan, f32))
    env.call("seeml_hip_scale", env.T(x), xs, scale, x.size)
    assert same_bits(env.H(xs), (scale * x).astype(f32))
    a_dev, b_dev = env.T(A), env.T(B)
    ran = 0
    for cfg in (4, 5, 8, 9, 10, 11):
        for splits in (1, 4):
            want = env.T(np.full(M * N, np.nan, f32))
            env.call("seeml_hip_gemm_forced", layout, xs if sa else a_dev, b_dev if sa else xs, want,
                     M, N, K, cfg, splits)
            got = env.T(np.full(M * N, np.nan, f32))
            env.call("seeml_hip_gemm_forced_scaled", layout, a_dev, b_dev, got, M, N, K, cfg, splits,
                     scale)
            assert same_bits(env.H(got), env.H(want)), (cfg, splits)
            ran += 1
    assert ran == 12
    # and the product is the oracle's on the scaled operand
    ref = np.zeros(M * N, f32)
    if layout == 1:
        orc.gemm_nt((scale * A).astype(f32), B, ref, M, N, K)
    else:
        orc.gemm_tn(A, (scale * B).astype(f32), ref, M, N, K)
    assert rel_err(env.H(got), ref) <= TOL_STEP


@pytest.mark.parametrize("M,N,K", [(200, 136, 520), (256, 192, 128), (130, 68, 96)])
def test_gemm_nn_equals_nt_on_the_transposed_operand_bitwise(env, M, N, K):
    """The engine runs a GemmNN on a frozen weight as GemmNT on a transposed
    copy: every tile config and split gives the same bits both ways (the
    per-output k order does not depend on the operand layout)."""
    A = rnd(M * K, 21)
    B = rnd(K * N, 22)
    Bt = np.ascontiguousarray(B.reshape(K, N).T).ravel()
    ncfg = env.L.seeml_hip_gemm_config_count()
    for cfg in range(ncfg):
        for splits in (1, 3):
            nn = env.T(np.full(M * N, np.nan, f32))
            nt = env.T(np.full(M * N, np.nan, f32))
            env.call("seeml_hip_gemm_forced", 0, env.T(A), env.T(B), nn, M, N, K, cfg, splits)
            env.call("seeml_hip_gemm_forced", 1, env.T(A), env.T(Bt), nt, M, N, K, cfg, splits)
            assert same_bits(env.H(nn), env.H(nt)), (cfg, splits)


# LoRA-shaped GEMMs: the heuristic takes the skinny kernels for rowdot (N <=
# 64 with A k-contiguous) and colsum (TN with min(M, N) <= 64) up to rank 16,
# the tile kernels with split-K for wider ranks, and the tile kernels for
# rank-K outer products (K <= 64); the skinny kernels stay reachable as a
# forced config. The same shapes forced onto a generic tile config give the
# reference for run-to-run and path-to-path agreement.
SKINNY = [
    (0, 1000, 520, 16), (0, 256, 2048, 64), (0, 300, 132, 8), (0, 129, 68, 4), (1, 1000, 520, 16),
    (1, 200, 256, 64), (0, 1000, 16, 2048), (0, 130, 64, 1024), (0, 77, 8, 260), (1, 300, 40, 512),
    (1, 1000, 16, 2048), (2, 520, 16, 1000), (2, 16, 520, 1000), (2, 64, 1024, 300),
    (2, 1024, 64, 2048), (2, 8, 132, 256), (2, 2048, 16, 4096),
]


def heuristic_splits(M, N, K):
    """The untuned plan's split-K count for a batch-1 GEMM (PlanGemmWith,
    csrc/k_gemm.hip): its tile (128x32 for N <= 32, 32x128 for M <= 32,
    else 128x128 or, when that leaves few tiles or an extent <= 64, 64x64);
    fewer than 512 tiles and K >= 256 split K so the slices cover the chip
    twice, each at least 128 deep."""
    cdiv = lambda a, b: -(-a // b)
    if N <= 32 < M:
        mt = (128, 32)
    elif M <= 32 < N:
        mt = (32, 128)
    else:
        big, mid = cdiv(M, 128) * cdiv(N, 128), cdiv(M, 64) * cdiv(N, 64)
        mt = (128, 128) if big >= 512 else ((64, 64) if (mid >= 256 or M <= 64 or N <= 64) else (128, 128))
    tiles = cdiv(M, mt[0]) * cdiv(N, mt[1])
    if tiles >= 512 or K < 256:
        return 1
    return max(1, min(cdiv(512, tiles), K // 128, 64))


@pytest.mark.parametrize("layout,M,N,K", SKINNY)
def test_gemm_skinny(env, orc, layout, M, N, K):
    A = rnd(M * K, 31)
    B = rnd(K * N, 32)
    want = np.zeros(M * N, f32)
    fn = ("seeml_hip_gemm_nn", "seeml_hip_gemm_nt", "seeml_hip_gemm_tn")[layout]
    if layout == 0:
        orc.gemm_nn(A, B, want, M, N, K, None, 0)
    elif layout == 1:
        orc.gemm_nt(A, B, want, M, N, K)
    else:
        orc.gemm_tn(A, B, want, M, N, K)
    out = env.T(np.full(M * N, np.nan, f32))
    args = (env.T(A), env.T(B), out, M, N, K) + ((None, 0) if layout == 0 else ())
    env.call(fn, *args)
    got = env.H(out)
    assert rel_err(got, want) <= TOL_STEP
    env.call(fn, *args)
    assert same_bits(env.H(out), got), "run-to-run bits differ"
    skinny = env.L.seeml_hip_gemm_config_count() - 1
    assert env.L.seeml_hip_gemm_config_name(skinny).decode() == "skinny"
    forced = env.T(np.full(M * N, np.nan, f32))
    env.call("seeml_hip_gemm_forced", layout, env.T(A), env.T(B), forced, M, N, K, skinny, 1)
    assert rel_err(env.H(forced), want) <= TOL_STEP
    generic = env.T(np.full(M * N, np.nan, f32))
    env.call("seeml_hip_gemm_forced", layout, env.T(A), env.T(B), generic, M, N, K, 0, 1)
    outer = layout != 2 and K <= 64
    wide = not outer and (min(M, N) if layout == 2 else N) > 16
    if outer:   # heuristic = a tile kernel at one slice: any tile config's bits
        assert same_bits(env.H(generic), got)
    elif wide:  # heuristic = the tile kernels at the rule's split count
        tiled = env.T(np.full(M * N, np.nan, f32))
        env.call("seeml_hip_gemm_forced", layout, env.T(A), env.T(B), tiled, M, N, K, 0,
                 heuristic_splits(M, N, K))
        assert same_bits(env.H(tiled), got)
        assert rel_err(env.H(forced), got) <= TOL_STEP
    else:       # heuristic = the skinny kernel
        assert same_bits(env.H(forced), got)
        assert rel_err(env.H(generic), got) <= TOL_STEP


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("cfg", [0, 1, 2, 3, 4, 5, 8, 9])
def test_gemm_group_members_are_bitwise_their_own_launches(env, orc, layout, cfg):
    """Two to four GEMMs of different (ragged) shapes as one tile-group
    launch, plain and fused-AddEW members mixed: each member's output has
    the bits of its own launch on the same tile config (the AddEW's sum
    those of the GEMM then AddEW) and matches the oracle's GEMM."""
    import ctypes
    shapes = [(256, 192, 96), (200, 136, 64), (384, 128, 160), (72, 264, 32)]
    for n in (2, 3, 4):
        A, B, C, adds, outs, want, fused = [], [], [], [], [], [], []
        for j, (M, N, K) in enumerate(shapes[:n]):
            a = rnd(M * K, 300 + 10 * j + n)
            b = rnd(K * N, 301 + 10 * j + n)
            w = np.zeros(M * N, f32)
            if layout == 0:
                orc.gemm_nn(a, b, w, M, N, K, None, 0)
            else:
                orc.gemm_nt(a, b, w, M, N, K)
            fz = j % 2 == 1
            A.append(env.T(a))
            B.append(env.T(b))
            C.append(env.T(np.full(M * N, np.nan, f32)))
            adds.append(env.T(rnd(M * N, 302 + 10 * j + n)) if fz else None)
            outs.append(env.T(np.full(M * N, np.nan, f32)) if fz else None)
            want.append(w)
            fused.append(fz)
        ptrs = lambda ts: (ctypes.c_void_p * n)(*[t.data_ptr() if t is not None else None for t in ts])
        dims = (ctypes.c_uint64 * (3 * n))(*[v for sh in shapes[:n] for v in sh])
        pa, pb, pc, pad, po = ptrs(A), ptrs(B), ptrs(C), ptrs(adds), ptrs(outs)
        env.call("seeml_hip_gemm_group", layout, cfg, n, ctypes.addressof(pa), ctypes.addressof(pb),
                 ctypes.addressof(pc), ctypes.addressof(dims), ctypes.addressof(pad), ctypes.addressof(po))
        for j, (M, N, K) in enumerate(shapes[:n]):
            lone = env.T(np.full(M * N, np.nan, f32))
            env.call("seeml_hip_gemm_forced", layout, A[j], B[j], lone, M, N, K, cfg, 1)
            if fused[j]:
                lone_sum = env.T(np.full(M * N, np.nan, f32))
                env.call("seeml_hip_add_ew", adds[j], lone, lone_sum, M * N)
                assert same_bits(env.H(outs[j]), env.H(lone_sum)), (n, j)
                assert np.all(np.isnan(env.H(C[j]))), (n, j)  # C is not stored
            else:
                got = env.H(C[j])
                assert same_bits(got, env.H(lone)), (n, j)
                assert rel_err(got, want[j]) <= TOL_STEP, (n, j)


@pytest.mark.parametrize("T,D,r_rd,r_cs,scaled", [
    (8192, 2048, 16, 16, 1), (4096, 512, 8, 8, 0), (300, 260, 5, 16, 1), (257, 1028, 16, 3, 0),
    (256, 256, 1, 1, 1)])
def test_skinny_dual_pass(env, orc, T, D, r_rd, r_cs, scaled):
    """dt = x b^T and db = t^T x in one pass over x (the LoRA backward pair):
    each output against the oracle's GEMM on the stream as the Scale would
    have stored it, and bit-equal whether computed alone or with the other
    (the engine's eager and fused forms). Ragged T and D, ranks below 16."""
    alpha = f32(0.37)
    x, b, t = rnd(T * D, 71), rnd(r_rd * D, 72), rnd(T * r_cs, 73)
    xs = (alpha * x).astype(f32) if scaled else x
    want_dt, want_db = np.zeros(T * r_rd, f32), np.zeros(r_cs * D, f32)
    orc.gemm_nt(xs, b, want_dt, T, r_rd, D)
    orc.gemm_tn(t, xs, want_db, r_cs, D, T)
    outs = {}
    for which in (3, 1, 2):
        dt = env.T(np.full(T * r_rd, np.nan, f32))
        db = env.T(np.full(r_cs * D, np.nan, f32))
        env.call("seeml_hip_gemm_skinny_dual", env.T(x), T, D, env.T(b), r_rd, dt, env.T(t), r_cs, db,
                 which, scaled, alpha)
        outs[which] = (env.H(dt), env.H(db))
    dt3, db3 = outs[3]
    assert rel_err(dt3, want_dt) <= TOL_STEP and rel_err(db3, want_db) <= TOL_STEP
    assert same_bits(outs[1][0], dt3) and same_bits(outs[2][1], db3)
    assert np.all(np.isnan(outs[1][1])) and np.all(np.isnan(outs[2][0]))  # the other is untouched


@pytest.mark.parametrize("kind,T,D,r,n", [
    (0, 8192, 2048, 16, 3), (0, 1000, 520, 8, 2), (0, 300, 256, 16, 4), (0, 4096, 1028, 5, 3),
    (1, 8192, 2048, 16, 3), (1, 1000, 520, 8, 2), (1, 257, 256, 16, 4), (1, 4100, 1028, 5, 3)])
def test_skinny_groups_are_bitwise_their_members(env, orc, kind, T, D, r, n):
    """The q/k/v LoRA GEMMs over one layer input as one pass over x: the
    rowdot group (t_j = x a_j, the down-projections) and the colsum group
    (dA_j = x^T dt_j). Each member's output has the bits of its own skinny
    GEMM and matches the oracle's GEMM; ragged T and D, ranks below 16, and
    2 to 4 members."""
    import ctypes
    skinny = env.L.seeml_hip_gemm_config_count() - 1
    x = rnd(T * D, 81)
    k_small = D if kind == 0 else T
    rows = T if kind == 0 else D
    a = [rnd(k_small * r, 82 + j) for j in range(n)]
    xd, ad = env.T(x), [env.T(v) for v in a]
    outs = [env.T(np.full(rows * r, np.nan, f32)) for _ in range(n)]
    ap = (ctypes.c_void_p * n)(*[t.data_ptr() for t in ad])
    op = (ctypes.c_void_p * n)(*[t.data_ptr() for t in outs])
    env.call("seeml_hip_gemm_skinny_group", kind, xd, T, D, ctypes.addressof(ap), r, ctypes.addressof(op), n)
    for j in range(n):
        lone = env.T(np.full(rows * r, np.nan, f32))
        want = np.zeros(rows * r, f32)
        if kind == 0:
            env.call("seeml_hip_gemm_forced", 0, xd, ad[j], lone, T, r, D, skinny, 1)
            orc.gemm_nn(x, a[j], want, T, r, D, None, 0)
        else:
            env.call("seeml_hip_gemm_forced", 2, xd, ad[j], lone, D, r, T, skinny, 1)
            orc.gemm_tn(x, a[j], want, D, r, T)
        got = env.H(outs[j])
        assert same_bits(got, env.H(lone)), j
        assert rel_err(got, want) <= TOL_STEP, j


@pytest.mark.parametrize("layout,M,N,K,tail,n_split", [
    (1, 512, 1000, 256, 0, 768), (0, 300, 520, 128, 4, 384), (2, 256, 640, 96, 0, 512),
    (1, 256, 5504, 64, 4, 5120), (1, 512, 5504, 96, 5, 5120), (0, 300, 1000, 128, 5, 768)])
def test_gemm_column_split_is_bitwise_one_launch(env, layout, M, N, K, tail, n_split):
    """A column-split plan (256x128 tiles on [0, n_split), smaller tiles on
    the rest) gives every output the same k order as one launch: bit-equal
    C, and bit-equal fused-AddEW output through the offset column views."""
    A, B, Y = rnd(M * K, 61), rnd(K * N, 62), rnd(M * N, 63)
    whole, split = (env.T(np.full(M * N, np.nan, f32)) for _ in range(2))
    env.call("seeml_hip_gemm_forced_split", layout, env.T(A), env.T(B), whole, M, N, K, 2, 0, 0, None, None)
    env.call("seeml_hip_gemm_forced_split", layout, env.T(A), env.T(B), split, M, N, K, 2, tail, n_split,
             None, None)
    assert same_bits(env.H(split), env.H(whole))
    a = A.reshape((K, M) if layout == 2 else (M, K)).astype(np.float64)
    b = B.reshape((N, K) if layout == 1 else (K, N)).astype(np.float64)
    want = (a.T if layout == 2 else a) @ (b.T if layout == 1 else b)
    assert rel_err(env.H(whole), want.reshape(-1).astype(f32)) <= TOL_STEP
    outs = []
    for ns, tl in ((0, 0), (n_split, tail)):
        c, o = env.T(np.full(M * N, np.nan, f32)), env.T(np.full(M * N, np.nan, f32))
        env.call("seeml_hip_gemm_forced_split", layout, env.T(A), env.T(B), c, M, N, K, 2, tl, ns,
                 env.T(Y), o)
        outs.append((env.H(c), env.H(o)))
    assert same_bits(outs[0][0], env.H(whole)) and same_bits(outs[1][0], env.H(whole))
    assert same_bits(outs[1][1], outs[0][1])
    assert same_bits(outs[0][1], (Y + env.H(whole)).astype(f32))
    # C null: the engine's form, C not stored and the same sums.
    for ns, tl in ((0, 0), (n_split, tail)):
        o = env.T(np.full(M * N, np.nan, f32))
        env.call("seeml_hip_gemm_forced_split", layout, env.T(A), env.T(B), None, M, N, K, 2, tl, ns,
                 env.T(Y), o)
        assert same_bits(env.H(o), outs[0][1]), ns


@pytest.mark.parametrize("layout,M,N,K,r,cfg,tail,n_split", [
    (1, 512, 384, 256, 16, 2, 0, 0), (0, 300, 200, 96, 16, 2, 0, 0),
    (1, 256, 512, 128, 16, 0, 0, 0), (1, 260, 130, 64, 8, 0, 0, 0),
    (1, 512, 1000, 128, 16, 2, 0, 768), (1, 300, 520, 128, 8, 2, 0, 384)])
def test_gemm_lora_epilogue_is_bitwise_the_unfused_chain(env, layout, M, N, K, r, cfg, tail, n_split):
    """The base GEMM with the LoRA up-projection, Scale and AddEW in its
    epilogue equals, bit for bit, the base GEMM, the up-projection as a tile
    GEMM (one slice), the Scale and the AddEW run one by one — also as a
    column split, whose right launch reads the offset columns of B and of
    the up-projection's bl."""
    A, B = rnd(M * K, 71), rnd(K * N, 72)
    t, bl = rnd(M * r, 73), rnd(r * N, 74)
    scale = f32(0.37)
    y = env.T(np.full(M * N, np.nan, f32))
    env.call("seeml_hip_gemm_forced", layout, env.T(A), env.T(B), y, M, N, K, cfg, 1)
    u = env.T(np.full(M * N, np.nan, f32))
    env.call("seeml_hip_gemm_forced", 0, env.T(t), env.T(bl), u, M, N, r, 5, 1)
    yh, uh = env.H(y), env.H(u)
    for scaled, y_first in ((1, 1), (1, 0), (0, 1)):
        s = (scale * uh).astype(f32) if scaled else uh
        want = (yh + s) if y_first else (s + yh)
        out = env.T(np.full(M * N, np.nan, f32))
        env.call("seeml_hip_gemm_forced_lora", layout, env.T(A), env.T(B), out, M, N, K, cfg,
                 tail, n_split, env.T(t), env.T(bl), r, scaled, scale, y_first)
        assert same_bits(env.H(out), want.astype(f32)), (scaled, y_first)


def test_gemm_skinny_epilogue(env, orc):
    """GemmNN's fused bias/act epilogue at a LoRA outer-product shape
    (K = 16: the heuristic's tile kernel)."""
    M, N, K = 600, 264, 16
    A, B, bias = rnd(M * K, 41), rnd(K * N, 42), rnd(N, 43)
    for act in range(4):
        want = np.zeros(M * N, f32)
        orc.gemm_nn(A, B, want, M, N, K, bias, act)
        out = env.T(np.full(M * N, np.nan, f32))
        env.call("seeml_hip_gemm_nn", env.T(A), env.T(B), out, M, N, K, env.T(bias), act)
        assert rel_err(env.H(out), want) <= TOL_STEP, act


def test_gemm_acc_and_q8(env, orc):
    M, N, K = 70, 90, 110
    A, B, C0 = rnd(M * K, 21), rnd(K * N, 22), rnd(M * N, 23)
    want = C0.copy()
    orc.gemm_acc_nn(A, B, want, M, N, K, 0.37)
    out = env.T(C0)
    env.call("seeml_hip_gemm_acc_nn", env.T(A), env.T(B), out, M, N, K, f32(0.37))
    assert rel_err(env.H(out), want) <= TOL_STEP
    q = np.random.default_rng(24).integers(-127, 128, K * N).astype(np.int8)
    for act in (0, 3):
        want = np.zeros(M * N, f32)
        orc.gemm_nn_q8(A, q, want, M, N, K, 0.013, act)
        out = env.T(np.zeros(M * N, f32))
        env.call("seeml_hip_gemm_nn_q8", env.T(A), env.T(q), out, M, N, K, f32(0.013), act)
        assert rel_err(env.H(out), want) <= TOL_STEP
    want = np.zeros(M * N, f32)
    orc.gemm_nt_q8(A, q, want, M, N, K, 0.013)
    out = env.T(np.zeros(M * N, f32))
    env.call("seeml_hip_gemm_nt_q8", env.T(A), env.T(q), out, M, N, K, f32(0.013))
    assert rel_err(env.H(out), want) <= TOL_STEP


def test_pointwise_bit_exact(env, orc):
    n = 301 * 333 + 7  # >= rows*cols of the broadcast cases below
    x, y, dy = rnd(n, 30, 3), rnd(n, 31, 3), rnd(n, 32)
    for name in ("add_ew", "mul_ew"):
        want = np.zeros(n, f32)
        getattr(orc, name)(x, y, want, n)
        out = env.T(np.zeros(n, f32))
        env.call("seeml_hip_" + name, env.T(x), env.T(y), out, n)
        assert same_bits(env.H(out), want), name
    want = np.zeros(n, f32)
    orc.scale(x, want, 1.7, n)
    out = env.T(np.zeros(n, f32))
    env.call("seeml_hip_scale", env.T(x), out, f32(1.7), n)
    assert same_bits(env.H(out), want)
    want = np.zeros(n, f32)
    orc.relu_fwd(x, want, n)
    out = env.T(np.zeros(n, f32))
    env.call("seeml_hip_relu_fwd", env.T(x), out, n)
    assert same_bits(env.H(out), want)
    want = np.zeros(n, f32)
    orc.relu_bwd(dy, x, want, n)
    out = env.T(np.zeros(n, f32))
    env.call("seeml_hip_relu_bwd", env.T(dy), env.T(x), out, n)
    assert same_bits(env.H(out), want)
    rows, cols = 301, 333
    xb, b = x[:rows * cols].copy(), y[:cols].copy()
    want = np.zeros(rows * cols, f32)
    orc.add_bias(xb, b, want, rows, cols)
    out = env.T(np.zeros(rows * cols, f32))
    env.call("seeml_hip_add_bias", env.T(xb), env.T(b), out, rows, cols)
    assert same_bits(env.H(out), want)
    want = np.zeros(cols, f32)
    orc.reduce_rows(xb, want, rows, cols)
    out = env.T(np.zeros(cols, f32))
    env.call("seeml_hip_reduce_rows", env.T(xb), out, rows, cols)
    assert same_bits(env.H(out), want)
    out = env.T(np.zeros(n, f32))
    env.call("seeml_hip_fill", out, f32(-2.5), n)
    assert np.all(env.H(out) == -2.5)
    out2 = env.T(np.zeros(n, f32))
    env.call("seeml_hip_copy", env.T(x), out2, n)
    assert same_bits(env.H(out2), x)
    # unaligned (scalar path) views
    out = env.T(np.zeros(n + 1, f32))
    xt = env.T(np.concatenate([[0], x]).astype(f32))
    yt = env.T(np.concatenate([[0], y]).astype(f32))
    env.call("seeml_hip_add_ew", xt[1:], yt[1:], out[1:], n)
    want = np.zeros(n, f32)
    orc.add_ew(x, y, want, n)
    assert same_bits(env.H(out)[1:], want)


def test_activations(env, orc):
    n = 65_537
    x, dy = rnd(n, 40, 4), rnd(n, 41)
    x[:4] = [1e30, -1e30, 0.0, -0.0]
    for fwd, bwd in (("gelu_fwd", "gelu_bwd"), ("silu_fwd", "silu_bwd")):
        want = np.zeros(n, f32)
        getattr(orc, fwd)(x, want, n)
        out = env.T(np.zeros(n, f32))
        env.call("seeml_hip_" + fwd, env.T(x), out, n)
        assert np.array_equal(np.isfinite(env.H(out)), np.isfinite(want))
        assert rel_err(np.nan_to_num(env.H(out)), np.nan_to_num(want)) <= 1e-6, fwd
        want = np.zeros(n, f32)
        getattr(orc, bwd)(dy, x, want, n)
        out = env.T(np.zeros(n, f32))
        env.call("seeml_hip_" + bwd, env.T(dy), env.T(x), out, n)
        assert rel_err(env.H(out), want) <= 1e-6, bwd
    # GELU saturation golden (kernels_test.cc:772-781)
    out = env.T(np.zeros(2, f32))
    env.call("seeml_hip_gelu_bwd", env.T(np.array([2, 2], f32)), env.T(np.array([1e30, -1e30], f32)),
             out, 2)
    assert env.H(out).tolist() == [2.0, 0.0]


def test_embed_gather(env, orc):
    V, D, T = 97, 40, 500
    table = rnd(V * D, 50)
    tok = np.random.default_rng(51).integers(0, V, T).astype(np.int32)
    want = np.zeros(T * D, f32)
    orc.embed_fwd(tok, table, want, T, D)
    out = env.T(np.zeros(T * D, f32))
    env.call("seeml_hip_embed_fwd", env.T(tok), env.T(table), out, T, D, V)
    assert same_bits(env.H(out), want)
    # an id outside the vocab (excluded by the feeder contract) yields NaNs,
    # never an out-of-bounds read
    bad = tok.copy()
    bad[3] = V + 5
    out = env.T(np.zeros(T * D, f32))
    env.call("seeml_hip_embed_fwd", env.T(bad), env.T(table), out, T, D, V)
    h = env.H(out).reshape(T, D)
    assert np.all(np.isnan(h[3])) and same_bits(h[4:], want.reshape(T, D)[4:])


# cols % 4 == 0 up to 8192 (16-byte rows): the register-resident row forms
# (64 threads x 4 or 8 float4s, 256 threads x 4 or 8); otherwise the strided
# two-pass rows.
@pytest.mark.parametrize("rows,cols", [(257, 300), (64, 2048), (3, 5000), (33, 1024), (7, 4096),
                                       (9, 8192), (5, 8196), (6, 1030)])
def test_norms(env, orc, rows, cols):
    n = rows * cols
    x, dy, g, b = rnd(n, 60, 2), rnd(n, 61), rnd(cols, 62), rnd(cols, 63)
    y, mean, rstd = np.zeros(n, f32), np.zeros(rows, f32), np.zeros(rows, f32)
    orc.layer_norm_fwd(x, g, b, y, mean, rstd, rows, cols)
    ty, tm, tr = env.T(np.zeros(n, f32)), env.T(np.zeros(rows, f32)), env.T(np.zeros(rows, f32))
    env.call("seeml_hip_layer_norm_fwd", env.T(x), env.T(g), env.T(b), ty, tm, tr, rows, cols)
    assert rel_err(env.H(ty), y) <= 1e-6 and rel_err(env.H(tm), mean) <= 1e-6
    assert rel_err(env.H(tr), rstd) <= 1e-6
    dx = np.zeros(n, f32)
    orc.layer_norm_bwd(dy, x, g, mean, rstd, dx, rows, cols)
    tdx = env.T(np.zeros(n, f32))
    env.call("seeml_hip_layer_norm_bwd", env.T(dy), env.T(x), env.T(g), env.T(mean), env.T(rstd),
             tdx, rows, cols)
    assert rel_err(env.H(tdx), dx) <= 1e-5
    y, rstd = np.zeros(n, f32), np.zeros(rows, f32)
    orc.rms_norm_fwd(x, g, y, rstd, rows, cols)
    ty, tr = env.T(np.zeros(n, f32)), env.T(np.zeros(rows, f32))
    env.call("seeml_hip_rms_norm_fwd", env.T(x), env.T(g), ty, tr, rows, cols)
    assert rel_err(env.H(ty), y) <= 1e-6 and rel_err(env.H(tr), rstd) <= 1e-6
    dx = np.zeros(n, f32)
    orc.rms_norm_bwd(dy, x, g, rstd, dx, rows, cols)
    tdx = env.T(np.zeros(n, f32))
    env.call("seeml_hip_rms_norm_bwd", env.T(dy), env.T(x), env.T(g), env.T(rstd), tdx, rows, cols)
    assert rel_err(env.H(tdx), dx) <= 1e-5


# d % 4 == 0 and d/2 <= 256: the row-streaming float4 form with a per-row
# angle table (256/(d/2) rows per workgroup); otherwise the per-pair form.
@pytest.mark.parametrize("B,S,H,d", [(2, 300, 3, 64), (2, 17, 3, 6), (1, 3, 1, 2052),
                                     (2, 65, 4, 128), (1, 5, 2, 512), (1, 7, 2, 1024),
                                     (3, 11, 1, 4)])
def test_rope(env, orc, B, S, H, d):
    n = B * S * H * d
    x = rnd(n, 70)
    for name, base in (("rope_fwd", 10000.0), ("rope_bwd", 500.0)):
        want = np.zeros(n, f32)
        getattr(orc, name)(x, want, B, S, H, d, base)
        out = env.T(np.zeros(n, f32))
        env.call("seeml_hip_" + name, env.T(x), out, B, S, H, d, f32(base))
        assert rel_err(env.H(out), want) <= TOL_STEP, name
        # position 0 passes through bit-for-bit
        h = env.H(out).reshape(B, S, H * d)
        assert same_bits(h[:, 0], x.reshape(B, S, H * d)[:, 0])


# AttnFwd with d in {64, 128} and S % 4 == 0 runs the fused two-pass kernel
# (partial query blocks and key tiles included); other shapes run scores ->
# row softmax -> PV on the GEMM engine.
@pytest.mark.parametrize("B,S,H,d", [(2, 33, 3, 8), (1, 130, 2, 64), (2, 256, 2, 128), (1, 1, 2, 3),
                                     (1, 300, 2, 64), (2, 4, 1, 128), (1, 1024, 2, 128),
                                     (3, 160, 2, 64), (1, 132, 1, 128)])
def test_attention_family(env, orc, B, S, H, d):
    n, pn = B * S * H * d, B * H * S * S
    q, k, v, w = rnd(n, 80), rnd(n, 81), rnd(n, 82), rnd(n, 83)
    o, p = np.zeros(n, f32), np.zeros(pn, f32)
    orc.attn_fwd(q, k, v, o, p, B, S, H, d)
    to, tp = env.T(np.zeros(n, f32)), env.T(np.full(pn, np.nan, f32))
    tq, tk, tv, tw = env.T(q), env.T(k), env.T(v), env.T(w)
    env.call("seeml_hip_attn_fwd", tq, tk, tv, to, tp, B, S, H, d)
    hp = env.H(tp)
    assert rel_err(hp, p) <= TOL_STEP and rel_err(env.H(to), o) <= TOL_STEP
    pm = hp.reshape(B * H, S, S)
    for i in range(S):
        assert np.all(pm[:, i, i + 1:] == 0.0)  # masked entries exactly 0
    dp = np.zeros(pn, f32)
    orc.attn_dp(w, v, dp, B, S, H, d)
    tdp = env.T(np.full(pn, np.nan, f32))
    env.call("seeml_hip_attn_dp", tw, tv, tdp, B, S, H, d)
    assert rel_err(env.H(tdp), dp) <= TOL_STEP
    dv = np.zeros(n, f32)
    orc.attn_dv(p, w, dv, B, S, H, d)
    tdv = env.T(np.zeros(n, f32))
    env.call("seeml_hip_attn_dv", env.T(p), tw, tdv, B, S, H, d)
    assert rel_err(env.H(tdv), dv) <= TOL_STEP
    ds = np.zeros(pn, f32)
    orc.softmax_rows_bwd(p, dp, ds, B * H * S, S)
    tds = env.T(np.zeros(pn, f32))
    env.call("seeml_hip_softmax_rows_bwd", env.T(p), env.T(dp), tds, B * H * S, S)
    assert rel_err(env.H(tds), ds) <= 1e-6
    dq = np.zeros(n, f32)
    orc.attn_dq(ds, k, dq, B, S, H, d)
    tdq = env.T(np.zeros(n, f32))
    env.call("seeml_hip_attn_dq", env.T(ds), tk, tdq, B, S, H, d)
    assert rel_err(env.H(tdq), dq) <= TOL_STEP
    dk = np.zeros(n, f32)
    orc.attn_dk(ds, q, dk, B, S, H, d)
    tdk = env.T(np.zeros(n, f32))
    env.call("seeml_hip_attn_dk", env.T(ds), tq, tdk, B, S, H, d)
    assert rel_err(env.H(tdk), dk) <= TOL_STEP
    if S == 1:  # S = 1: P is exactly 1 and O copies V (kernels_test.cc:795-805)
        assert np.all(hp == 1.0) and same_bits(env.H(to), v)


def test_softmax_rows_bwd_widths(env, orc):
    """Register-resident rows (cols % 4 == 0 up to 8192) and the strided
    fallback, against the oracle, with masked-causal-like zero tails."""
    rng = np.random.default_rng(95)
    for rows, cols in ((37, 256), (65, 1024), (9, 2048), (5, 4096), (3, 8192), (4, 8200),
                       (6, 1030)):
        p = rng.random(rows * cols).astype(f32)
        p.reshape(rows, cols)[:, cols // 2:] = 0.0
        dp = rnd(rows * cols, 96)
        want = np.zeros(rows * cols, f32)
        orc.softmax_rows_bwd(p, dp, want, rows, cols)
        out = env.T(np.full(rows * cols, np.nan, f32))
        env.call("seeml_hip_softmax_rows_bwd", env.T(p), env.T(dp), out, rows, cols)
        got = env.H(out)
        assert rel_err(got, want) <= 1e-6, (rows, cols)
        assert np.all(got.reshape(rows, cols)[:, cols // 2:] == 0.0)


# C < 2048: a wave per row; C % 4 == 0 up to 32768: the register-resident row
# (256/512/1024 threads); otherwise the three-pass block per row.
@pytest.mark.parametrize("N,C", [(32, 256), (100, 8192), (17, 32000), (3, 1), (5, 12000),
                                 (4, 2050), (3, 40000)])
def test_softmax_xent(env, orc, N, C):
    logits = rnd(N * C, 90, 3)
    labels = np.random.default_rng(91).integers(0, C, N).astype(np.int32)
    loss, probs = np.zeros(1, f32), np.zeros(N * C, f32)
    orc.softmax_xent_fwd(logits, labels, loss, probs, N, C)
    tl, tp = env.T(np.zeros(1, f32)), env.T(np.zeros(N * C, f32))
    env.call("seeml_hip_softmax_xent_fwd", env.T(logits), env.T(labels), tl, tp, N, C)
    # vs the CPU reference (sequential f32 exp-sum) and vs float64 (the
    # device's fixed-tree sum is the more accurate of the two)
    assert rel_err(env.H(tp), probs) <= TOL_STEP
    assert abs(env.H(tl)[0] - loss[0]) <= 1e-5 * max(1.0, abs(loss[0]))
    z = logits.reshape(N, C).astype(np.float64)
    z = np.exp(z - z.max(axis=1, keepdims=True))
    z /= z.sum(axis=1, keepdims=True)
    assert rel_err(env.H(tp).reshape(N, C), z) <= 1e-5
    seed = np.array([1.0], f32)
    want = np.zeros(N * C, f32)
    orc.softmax_xent_bwd(probs, labels, seed, want, N, C)
    out = env.T(np.zeros(N * C, f32))
    env.call("seeml_hip_softmax_xent_bwd", env.T(probs), env.T(labels), env.T(seed), out, N, C)
    assert same_bits(env.H(out), want)


def test_xent_nan_propagates_and_single_class_exact(env):
    logits = np.full(6, 0.5, f32)
    logits[4] = np.nan
    tl = env.T(np.zeros(1, f32))
    env.call("seeml_hip_softmax_xent_fwd", env.T(logits), env.T(np.array([0, 2], np.int32)), tl,
             env.T(np.zeros(6, f32)), 2, 3)
    assert np.isnan(env.H(tl)[0])
    tl, tp = env.T(np.full(1, -1, f32)), env.T(np.zeros(3, f32))
    env.call("seeml_hip_softmax_xent_fwd", env.T(np.array([2, -5, 100], f32)),
             env.T(np.zeros(3, np.int32)), tl, tp, 3, 1)
    assert env.H(tl)[0] == 0.0 and env.H(tp).tolist() == [1, 1, 1]


def test_gemm_propagates_non_finites_like_ieee(env):
    # inf/NaN inputs must reach C as IEEE arithmetic says (the engine's
    # finite-loss guard depends on it); compared with float64 numpy.
    M, N, K = 40, 70, 33
    A, B = rnd(M * K, 120), rnd(K * N, 121)
    A[5] = np.inf
    A[K * 7 + 3] = np.nan
    B[K * 0 + 9] = -np.inf
    want = A.reshape(M, K).astype(np.float64) @ B.reshape(K, N).astype(np.float64)
    out = env.T(np.zeros(M * N, f32))
    env.call("seeml_hip_gemm_nn", env.T(A), env.T(B), out, M, N, K, None, 0)
    got = env.H(out).reshape(M, N)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isposinf(got), np.isposinf(want))
    assert np.array_equal(np.isneginf(got), np.isneginf(want))


def test_mse_and_kl(env, orc):
    n = 256 * 32768 + 4097
    pred, tgt = rnd(n, 100), rnd(n, 101)
    loss = np.zeros(1, f32)
    orc.mse_fwd(pred, tgt, loss, n)
    tl = env.T(np.zeros(1, f32))
    tpred, ttgt = env.T(pred), env.T(tgt)
    env.call("seeml_hip_mse_fwd", tpred, ttgt, tl, n)
    assert abs(env.H(tl)[0] - loss[0]) <= 1e-6 * abs(loss[0])
    seed = np.array([0.75], f32)
    want = np.zeros(n, f32)
    orc.mse_bwd(pred, tgt, seed, want, n)
    out = env.T(np.zeros(n, f32))
    env.call("seeml_hip_mse_bwd", tpred, ttgt, env.T(seed), out, n)
    assert same_bits(env.H(out), want)
    N, C = 300, 70
    s, t = rnd(N * C, 102, 4), rnd(N * C, 103, 4)
    loss, ps, pt = np.zeros(1, f32), np.zeros(N * C, f32), np.zeros(N * C, f32)
    orc.kl_distill_fwd(s, t, loss, ps, pt, N, C, 2.0)
    tl, tps, tpt = env.T(np.zeros(1, f32)), env.T(np.zeros(N * C, f32)), env.T(np.zeros(N * C, f32))
    env.call("seeml_hip_kl_distill_fwd", env.T(s), env.T(t), tl, tps, tpt, N, C, f32(2.0))
    assert rel_err(env.H(tps), ps) <= 1e-5 and rel_err(env.H(tpt), pt) <= 1e-5
    assert abs(env.H(tl)[0] - loss[0]) <= 1e-4 * abs(loss[0])
    want = np.zeros(N * C, f32)
    orc.kl_distill_bwd(ps, pt, np.ones(1, f32), want, N, C, 2.0)
    out = env.T(np.zeros(N * C, f32))
    env.call("seeml_hip_kl_distill_bwd", env.T(ps), env.T(pt), env.T(np.ones(1, f32)), out, N, C,
             f32(2.0))
    assert same_bits(env.H(out), want)


def test_optimizers_bit_exact(env, orc):
    n = 300_007
    g = rnd(n, 110, 0.1)
    p0, m0, v0 = rnd(n, 111), rnd(n, 112, 0.01), np.abs(rnd(n, 113, 0.001))
    p, m, v = p0.copy(), m0.copy(), v0.copy()
    tp, tm, tv, tg = env.T(p0), env.T(m0), env.T(v0), env.T(g)
    for step in (1, 2, 3, 17, 1000):
        orc.adamw_step(p, g, m, v, n, 1e-3, 0.9, 0.999, 1e-8, 0.01, step)
        env.call("seeml_hip_adamw_step", tp, tg, tm, tv, n, f32(1e-3), f32(0.9), f32(0.999),
                 f32(1e-8), f32(0.01), step)
        assert same_bits(env.H(tp), p) and same_bits(env.H(tm), m) and same_bits(env.H(tv), v), step
    p = p0.copy()
    orc.sgd_step(p, g, n, 1e-3, 0.01)
    tp = env.T(p0)
    env.call("seeml_hip_sgd_step", tp, tg, n, f32(1e-3), f32(0.01))
    assert same_bits(env.H(tp), p)
    for cap in (0.5, 1e9, 0.0):
        gg = g.copy()
        orc.clip_norm(gg, n, cap)
        tgg = env.T(g)
        env.call("seeml_hip_clip_norm", tgg, n, f32(cap))
        assert rel_err(env.H(tgg), gg) <= 1e-6
