"""Pins the C oracle BIT-FOR-BIT against oracle/_ref — the reference's own
executor sources (runtime/executor/*.cc + parallel_for.cc) compiled in place.
Shapes are chosen so every chunked reduction spans many ParallelFor chunks
(the partial-sum grouping is part of the bits) and K crosses several 64-wide
GEMM K tiles with a ragged remainder."""
import numpy as np
import pytest

f32 = np.float32


def rnd(n, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(n) * scale).astype(f32)


def bits(a):
    return a.view(np.uint32) if a.dtype == f32 else a


def same(a, b):
    return np.array_equal(bits(a), bits(b))


def run_both(orc, ref, name, make_args, out_idx):
    a1 = make_args()
    a2 = make_args()
    getattr(orc, name)(*a1)
    getattr(ref, name)(*a2)
    for i in out_idx:
        assert same(a1[i], a2[i]), f"{name}: output {i} differs from reference bits"


@pytest.fixture(scope="module", autouse=True)
def threads(ref):
    ref.set_threads(8)  # multi-threaded reference: bits must not depend on it
    yield


@pytest.mark.parametrize("M,N,K", [(33, 47, 131), (64, 16, 256), (5, 300, 7)])
def test_gemm_family_bitwise(orc, ref, M, N, K):
    A, B, Bt, At = rnd(M * K, 1), rnd(K * N, 2), rnd(N * K, 3), rnd(K * M, 4)
    bias = rnd(N, 5)
    for act in range(4):
        run_both(orc, ref, "gemm_nn", lambda: [A, B, np.zeros(M * N, f32), M, N, K, bias, act], [2])
    run_both(orc, ref, "gemm_nn", lambda: [A, B, np.zeros(M * N, f32), M, N, K, None, 0], [2])
    run_both(orc, ref, "gemm_nt", lambda: [A, Bt, np.zeros(M * N, f32), M, N, K], [2])
    run_both(orc, ref, "gemm_tn", lambda: [At, B, np.zeros(M * N, f32), M, N, K], [2])
    C0 = rnd(M * N, 6)
    run_both(orc, ref, "gemm_acc_nn", lambda: [A, B, C0.copy(), M, N, K, 0.37], [2])
    q = np.random.default_rng(7).integers(-127, 128, K * N).astype(np.int8)
    run_both(orc, ref, "gemm_nn_q8", lambda: [A, q, np.zeros(M * N, f32), M, N, K, 0.013, 3], [2])
    run_both(orc, ref, "gemm_nt_q8", lambda: [A, q, np.zeros(M * N, f32), M, N, K, 0.013], [2])


def test_elementwise_family_bitwise(orc, ref):
    n = 301 * 333 + 7
    x, y, dy = rnd(n, 10, 3), rnd(n, 11, 3), rnd(n, 12)
    for name in ("add_ew", "mul_ew"):
        run_both(orc, ref, name, lambda: [x, y, np.zeros(n, f32), n], [2])
    for name in ("relu_fwd", "gelu_fwd", "silu_fwd"):
        run_both(orc, ref, name, lambda: [x, np.zeros(n, f32), n], [1])
    for name in ("relu_bwd", "gelu_bwd", "silu_bwd"):
        run_both(orc, ref, name, lambda: [dy, x, np.zeros(n, f32), n], [2])
    run_both(orc, ref, "scale", lambda: [x, np.zeros(n, f32), 1.7, n], [1])
    rows, cols = 301, 333
    run_both(orc, ref, "add_bias", lambda: [x[:rows * cols].copy(), y[:cols].copy(),
                                            np.zeros(rows * cols, f32), rows, cols], [2])
    run_both(orc, ref, "reduce_rows", lambda: [x[:rows * cols].copy(), np.zeros(cols, f32),
                                               rows, cols], [1])
    V, D, T = 97, 40, 500
    table = rnd(V * D, 13)
    tok = np.random.default_rng(14).integers(0, V, T).astype(np.int32)
    run_both(orc, ref, "embed_fwd", lambda: [tok, table, np.zeros(T * D, f32), T, D], [2])


def test_norm_family_bitwise(orc, ref):
    rows, cols = 257, 300
    n = rows * cols
    x, dy, g, b = rnd(n, 20, 2), rnd(n, 21), rnd(cols, 22), rnd(cols, 23)

    def ln():
        return [x, g, b, np.zeros(n, f32), np.zeros(rows, f32), np.zeros(rows, f32), rows, cols]
    run_both(orc, ref, "layer_norm_fwd", ln, [3, 4, 5])
    a = ln()
    orc.layer_norm_fwd(*a)
    run_both(orc, ref, "layer_norm_bwd",
             lambda: [dy, x, g, a[4], a[5], np.zeros(n, f32), rows, cols], [5])
    run_both(orc, ref, "rms_norm_fwd",
             lambda: [x, g, np.zeros(n, f32), np.zeros(rows, f32), rows, cols], [2, 3])
    r = [x, g, np.zeros(n, f32), np.zeros(rows, f32), rows, cols]
    orc.rms_norm_fwd(*r)
    run_both(orc, ref, "rms_norm_bwd",
             lambda: [dy, x, g, r[3], np.zeros(n, f32), rows, cols], [4])


def test_attention_family_bitwise(orc, ref):
    B, S, H, d = 2, 33, 3, 8
    n, pn = B * S * H * d, B * H * S * S
    q, k, v, w = rnd(n, 30), rnd(n, 31), rnd(n, 32), rnd(n, 33)
    run_both(orc, ref, "rope_fwd", lambda: [q, np.zeros(n, f32), B, S, H, d, 10000.0], [1])
    run_both(orc, ref, "rope_bwd", lambda: [w, np.zeros(n, f32), B, S, H, d, 500.0], [1])
    run_both(orc, ref, "attn_fwd", lambda: [q, k, v, np.zeros(n, f32), np.zeros(pn, f32),
                                            B, S, H, d], [3, 4])
    o, p = np.zeros(n, f32), np.zeros(pn, f32)
    orc.attn_fwd(q, k, v, o, p, B, S, H, d)
    run_both(orc, ref, "attn_dp", lambda: [w, v, np.zeros(pn, f32), B, S, H, d], [2])
    run_both(orc, ref, "attn_dv", lambda: [p, w, np.zeros(n, f32), B, S, H, d], [2])
    dp = np.zeros(pn, f32)
    orc.attn_dp(w, v, dp, B, S, H, d)
    run_both(orc, ref, "softmax_rows_bwd", lambda: [p, dp, np.zeros(pn, f32), B * H * S, S], [2])
    ds = np.zeros(pn, f32)
    orc.softmax_rows_bwd(p, dp, ds, B * H * S, S)
    run_both(orc, ref, "attn_dq", lambda: [ds, k, np.zeros(n, f32), B, S, H, d], [2])
    run_both(orc, ref, "attn_dk", lambda: [ds, q, np.zeros(n, f32), B, S, H, d], [2])


def test_loss_family_bitwise(orc, ref):
    N, C = 1500, 70  # RowGrain(70, 4096) = 58 rows/chunk -> 26 chunks
    logits, t_logits = rnd(N * C, 40, 4), rnd(N * C, 41, 4)
    labels = np.random.default_rng(42).integers(0, C, N).astype(np.int32)
    run_both(orc, ref, "softmax_xent_fwd",
             lambda: [logits, labels, np.zeros(1, f32), np.zeros(N * C, f32), N, C], [2, 3])
    probs = np.zeros(N * C, f32)
    orc.softmax_xent_fwd(logits, labels, np.zeros(1, f32), probs, N, C)
    seed = np.array([1.0], f32)
    run_both(orc, ref, "softmax_xent_bwd",
             lambda: [probs, labels, seed, np.zeros(N * C, f32), N, C], [3])
    n = 256 * 32768 + 4097  # MSE: 256 chunks at the cap
    pred, tgt = rnd(n, 43), rnd(n, 44)
    run_both(orc, ref, "mse_fwd", lambda: [pred, tgt, np.zeros(1, f32), n], [2])
    run_both(orc, ref, "mse_bwd", lambda: [pred, tgt, np.array([0.75], f32), np.zeros(n, f32), n], [3])
    run_both(orc, ref, "kl_distill_fwd",
             lambda: [logits, t_logits, np.zeros(1, f32), np.zeros(N * C, f32),
                      np.zeros(N * C, f32), N, C, 2.0], [2, 3, 4])
    ps, pt = np.zeros(N * C, f32), np.zeros(N * C, f32)
    orc.kl_distill_fwd(logits, t_logits, np.zeros(1, f32), ps, pt, N, C, 2.0)
    run_both(orc, ref, "kl_distill_bwd", lambda: [ps, pt, seed, np.zeros(N * C, f32), N, C, 2.0], [3])


def test_optimizer_family_bitwise(orc, ref):
    n = 300007
    g = rnd(n, 50, 0.1)
    run_both(orc, ref, "clip_norm", lambda: [g.copy(), n, 0.5], [0])
    p0, m0, v0 = rnd(n, 51), rnd(n, 52, 0.01), np.abs(rnd(n, 53, 0.001))
    run_both(orc, ref, "sgd_step", lambda: [p0.copy(), g, n, 1e-3, 0.01], [0])
    for step in (1, 2, 17, 1000):
        run_both(orc, ref, "adamw_step",
                 lambda: [p0.copy(), g, m0.copy(), v0.copy(), n, 1e-3, 0.9, 0.999,
                          1e-8, 0.01, step], [0, 2, 3])


def test_plan_hash_reference_available(ref):
    blob = np.random.default_rng(60).integers(0, 256, 3_000_001).astype(np.uint8)
    h1 = ref.plan_self_hash(blob, blob.size, 240)
    blob2 = blob.copy()
    blob2[240:248] = 0
    assert h1 == ref.plan_self_hash(blob2, blob2.size, 240)
    assert h1 != ref.content_hash64(blob, blob.size)
