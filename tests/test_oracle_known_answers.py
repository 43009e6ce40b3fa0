"""Pins the C oracle with the reference's own closed-form / known-answer cases
(test/runtime/executor/kernels_test.cc) and with what the mathematics fixes
(finite differences, adjoint identities, brute-force naive references in
float64). None of these retype the oracle's formula: each is an independent
statement a plausible mistake (dropped term, wrong sign, transposed operand,
off-by-one position) would violate."""
import math

import numpy as np
import pytest

f32 = np.float32


def rnd(n, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(n) * scale).astype(f32)


# --- GEMM (kernels_test.cc:26-138) -----------------------------------------

def test_gemm_nn_hand_product(orc):
    a = np.array([1, 2, 3, 4, 5, 6], f32)
    b = np.array([7, 8, 9, 10, 11, 12], f32)
    c = np.full(4, -1, f32)
    orc.gemm_nn(a, b, c, 2, 2, 3, None, 0)
    assert c.tolist() == [58, 64, 139, 154]


@pytest.mark.parametrize("M,N,K", [(3, 4, 5), (17, 9, 70), (1, 1, 1)])
def test_gemm_layouts_match_float64_brute_force(orc, M, N, K):
    a = rnd(M * K, 1).reshape(M, K)
    b = rnd(K * N, 2).reshape(K, N)
    want = a.astype(np.float64) @ b.astype(np.float64)
    c = np.zeros((M, N), f32)
    orc.gemm_nn(a, b, c, M, N, K, None, 0)
    np.testing.assert_allclose(c, want, rtol=1e-5, atol=1e-5)
    bt = np.ascontiguousarray(b.T)
    orc.gemm_nt(a, bt, c, M, N, K)
    np.testing.assert_allclose(c, want, rtol=1e-5, atol=1e-5)
    at = np.ascontiguousarray(a.T)
    orc.gemm_tn(at, b, c, M, N, K)
    np.testing.assert_allclose(c, want, rtol=1e-5, atol=1e-5)


def test_gemm_acc_closed_form(orc):
    a = np.array([1, 0, 0, 1], f32)
    b = np.array([5, 6, 7, 8], f32)
    c = np.array([100, 200, 300, 400], f32)
    orc.gemm_acc_nn(a, b, c, 2, 2, 2, 0.5)
    assert c.tolist() == [102.5, 203.0, 303.5, 404.0]


@pytest.mark.parametrize("act", [0, 1, 2, 3])
def test_gemm_epilogue_bitwise_equals_unfused(orc, act):
    M, N, K = 5, 7, 6
    a, b, bias = rnd(M * K, 11), rnd(K * N, 12), rnd(N, 13)
    fused = np.zeros(M * N, f32)
    orc.gemm_nn(a, b, fused, M, N, K, bias, act)
    plain = np.zeros(M * N, f32)
    orc.gemm_nn(a, b, plain, M, N, K, None, 0)
    biased = np.zeros(M * N, f32)
    orc.add_bias(plain, bias, biased, M, N)
    out = biased.copy()
    if act == 1:
        orc.relu_fwd(biased, out, M * N)
    elif act == 2:
        orc.gelu_fwd(biased, out, M * N)
    elif act == 3:
        orc.silu_fwd(biased, out, M * N)
    assert np.array_equal(fused.view(np.uint32), out.view(np.uint32))


def test_gemm_q8_matches_dequantized(orc):
    M, N, K = 4, 6, 9
    a = rnd(M * K, 3)
    q = np.random.default_rng(4).integers(-127, 128, K * N).astype(np.int8)
    c = np.zeros(M * N, f32)
    orc.gemm_nn_q8(a, q, c, M, N, K, 0.01, 0)
    want = a.reshape(M, K).astype(np.float64) @ (0.01 * q.reshape(K, N).astype(np.float64))
    np.testing.assert_allclose(c.reshape(M, N), want, rtol=1e-5, atol=1e-5)
    qt = np.ascontiguousarray(q.reshape(K, N).T)
    orc.gemm_nt_q8(a, qt, c, M, N, K, 0.01)
    np.testing.assert_allclose(c.reshape(M, N), want, rtol=1e-5, atol=1e-5)


# --- Elementwise (kernels_test.cc:142-200) ---------------------------------

def test_elementwise_closed_forms(orc):
    x = np.array([1, 2, 3], f32)
    y = np.array([10, 20, 30], f32)
    out = np.zeros(3, f32)
    orc.add_ew(x, y, out, 3)
    assert out.tolist() == [11, 22, 33]
    orc.mul_ew(x, y, out, 3)
    assert out.tolist() == [10, 40, 90]
    orc.scale(np.array([1, -2, 4], f32), out, 2.5, 3)
    assert out.tolist() == [2.5, -5, 10]
    xb = np.array([1, 2, 3, 4, 5, 6], f32)
    ob = np.zeros(6, f32)
    orc.add_bias(xb, np.array([10, 20, 30], f32), ob, 2, 3)
    assert ob.tolist() == [11, 22, 33, 14, 25, 36]
    db = np.full(3, -99, f32)
    orc.reduce_rows(np.array([1, 2, 3, 10, 20, 30], f32), db, 2, 3)
    assert db.tolist() == [11, 22, 33]
    r = np.zeros(5, f32)
    orc.relu_fwd(np.array([-2, -0.5, 0, 0.5, 2], f32), r, 5)
    assert r.tolist() == [0, 0, 0, 0.5, 2]
    dx = np.zeros(4, f32)
    orc.relu_bwd(np.ones(4, f32), np.array([-1, 0, 0.5, 3], f32), dx, 4)
    assert dx.tolist() == [0, 0, 1, 1]


def test_gelu_silu_backward_match_finite_differences(orc):
    x = np.array([-5, -2, -0.5, -1e-3, 0, 1e-3, 0.5, 2, 5], f32)
    n = x.size
    eps = 1e-3
    for fwd, bwd in ((orc.gelu_fwd, orc.gelu_bwd), (orc.silu_fwd, orc.silu_bwd)):
        dx = np.zeros(n, f32)
        bwd(np.ones(n, f32), x, dx, n)
        for i in range(n):
            xp, xm = x.copy(), x.copy()
            xp[i] += f32(eps)
            xm[i] -= f32(eps)
            fp, fm = np.zeros(n, f32), np.zeros(n, f32)
            fwd(xp, fp, n)
            fwd(xm, fm, n)
            assert abs(dx[i] - (fp[i] - fm[i]) / (2 * eps)) < 2e-3


def test_gelu_matches_tanh_formula_in_float64(orc):
    x = rnd(257, 5, 3.0)
    out = np.zeros_like(x)
    orc.gelu_fwd(x, out, x.size)
    xd = x.astype(np.float64)
    want = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd ** 3)))
    np.testing.assert_allclose(out, want, rtol=1e-5, atol=1e-6)


def test_gelu_backward_saturation_golden(orc):
    dx = np.zeros(2, f32)
    orc.gelu_bwd(np.array([2, 2], f32), np.array([1e30, -1e30], f32), dx, 2)
    assert dx.tolist() == [2.0, 0.0]


def test_embed_gather_golden(orc):
    table = np.array([0, 1, 2, 10, 11, 12, 20, 21, 22, 30, 31, 32], f32)
    tokens = np.array([2, 0, 3, 0], np.int32)
    out = np.full(12, -1, f32)
    orc.embed_fwd(tokens, table, out, 4, 3)
    assert out.tolist() == [20, 21, 22, 0, 1, 2, 30, 31, 32, 0, 1, 2]


def test_fill_copy(orc):
    d = np.zeros(5, f32)
    orc.fill(d, 3.5, 5)
    assert d.tolist() == [3.5] * 5
    e = np.zeros(5, f32)
    orc.copy(d, e, 5)
    assert e.tolist() == [3.5] * 5


# --- Losses (kernels_test.cc:204-265, 689-713) ------------------------------

def test_softmax_xent_uniform_gives_log_c(orc):
    N, C = 2, 4
    probs = np.zeros(N * C, f32)
    loss = np.zeros(1, f32)
    orc.softmax_xent_fwd(np.zeros(N * C, f32), np.array([0, 3], np.int32), loss, probs, N, C)
    assert abs(loss[0] - math.log(4)) < 1e-6
    np.testing.assert_allclose(probs, 0.25, atol=1e-6)


def test_softmax_xent_shift_invariant(orc):
    la, lb = np.zeros(1, f32), np.zeros(1, f32)
    p = np.zeros(3, f32)
    lab = np.array([2], np.int32)
    orc.softmax_xent_fwd(np.array([1, 2, 3], f32), lab, la, p, 1, 3)
    orc.softmax_xent_fwd(np.array([101, 102, 103], f32), lab, lb, p, 1, 3)
    assert abs(la[0] - lb[0]) < 1e-6 and la[0] > 0


def test_softmax_xent_backward_closed_form(orc):
    probs = np.array([0.2, 0.3, 0.5, 0.1, 0.8, 0.1], f32)
    d = np.zeros(6, f32)
    orc.softmax_xent_bwd(probs, np.array([2, 1], np.int32), np.array([2.0], f32), d, 2, 3)
    np.testing.assert_allclose(d, [0.2, 0.3, -0.5, 0.1, -0.2, 0.1], atol=1e-6)


def test_softmax_xent_matches_float64_reference(orc):
    N, C = 37, 53
    logits = rnd(N * C, 9, 3.0)
    labels = np.random.default_rng(10).integers(0, C, N).astype(np.int32)
    loss = np.zeros(1, f32)
    probs = np.zeros(N * C, f32)
    orc.softmax_xent_fwd(logits, labels, loss, probs, N, C)
    z = logits.reshape(N, C).astype(np.float64)
    z -= z.max(axis=1, keepdims=True)
    p = np.exp(z) / np.exp(z).sum(axis=1, keepdims=True)
    np.testing.assert_allclose(probs.reshape(N, C), p, rtol=1e-5, atol=1e-7)
    want = -np.mean(np.log(p[np.arange(N), labels]))
    assert abs(loss[0] - want) < 1e-5


def test_single_class_softmax_is_exact(orc):
    loss = np.full(1, -1, f32)
    probs = np.zeros(3, f32)
    orc.softmax_xent_fwd(np.array([2, -5, 100], f32), np.zeros(3, np.int32), loss, probs, 3, 1)
    assert loss[0] == 0.0 and probs.tolist() == [1, 1, 1]


def test_nan_logit_propagates(orc):
    logits = np.full(6, 0.5, f32)
    logits[4] = np.nan
    loss = np.zeros(1, f32)
    orc.softmax_xent_fwd(logits, np.array([0, 2], np.int32), loss, np.zeros(6, f32), 2, 3)
    assert np.isnan(loss[0])


def test_mse_closed_forms(orc):
    loss = np.zeros(1, f32)
    orc.mse_fwd(np.array([1, 2], f32), np.zeros(2, f32), loss, 2)
    assert loss[0] == 2.5
    d = np.zeros(2, f32)
    orc.mse_bwd(np.array([1, 2], f32), np.zeros(2, f32), np.array([2], f32), d, 2)
    assert d.tolist() == [2.0, 4.0]


def test_kl_identical_logits_zero(orc):
    logits = np.array([1, 2, 3, -1, 0, 1], f32)
    ps, pt = np.zeros(6, f32), np.zeros(6, f32)
    loss = np.full(1, -1, f32)
    orc.kl_distill_fwd(logits, logits, loss, ps, pt, 2, 3, 2.0)
    assert abs(loss[0]) < 1e-6
    d = np.zeros(6, f32)
    orc.kl_distill_bwd(ps, pt, np.ones(1, f32), d, 2, 3, 2.0)
    assert np.abs(d).max() < 1e-7


# --- Optimizers (kernels_test.cc:321-366, 715-723) ---------------------------

def test_sgd_closed_form(orc):
    p = np.array([1.0, -2.0], f32)
    orc.sgd_step(p, np.array([0.5, 0.5], f32), 2, 0.1, 0.2)
    np.testing.assert_allclose(p, [1 - 0.1 * (0.5 + 0.2), -2 - 0.1 * (0.5 - 0.4)], atol=1e-6)


def test_adamw_first_step_closed_form(orc):
    lr, b1, b2, eps, wd, g0, p0 = 0.01, 0.9, 0.999, 1e-8, 0.1, 0.4, 2.0
    p, m, v = np.array([p0], f32), np.zeros(1, f32), np.zeros(1, f32)
    orc.adamw_step(p, np.array([g0], f32), m, v, 1, lr, b1, b2, eps, wd, 1)
    # evaluated in float32, as the reference test evaluates it
    F = np.float32
    assert abs(m[0] - (F(1) - F(b1)) * F(g0)) < 1e-7
    assert abs(v[0] - (F(1) - F(b2)) * F(g0) * F(g0)) < 1e-9
    assert abs(p[0] - (p0 - lr * (g0 / (abs(g0) + eps) + wd * p0))) < 1e-6


def test_adamw_two_steps_track_float64(orc):
    lr, b1, b2, eps, wd = 0.05, 0.9, 0.99, 1e-8, 0.01
    p, m, v = np.array([1.5], f32), np.zeros(1, f32), np.zeros(1, f32)
    rp, rm, rv = 1.5, 0.0, 0.0
    for step, gf in ((1, 0.3), (2, -0.2)):
        orc.adamw_step(p, np.array([gf], f32), m, v, 1, lr, b1, b2, eps, wd, step)
        gd = float(f32(gf))
        rm = b1 * rm + (1 - b1) * gd
        rv = b2 * rv + (1 - b2) * gd * gd
        mh, vh = rm / (1 - b1 ** step), rv / (1 - b2 ** step)
        rp -= lr * (mh / (math.sqrt(vh) + eps) + wd * rp)
    assert abs(p[0] - rp) < 1e-5


def test_clip_norm_edges(orc):
    g = np.zeros(3, f32)
    orc.clip_norm(g, 3, 1.0)
    assert g.tolist() == [0, 0, 0]
    h = np.array([3, -4], f32)
    orc.clip_norm(h, 2, 0.0)
    assert h.tolist() == [0, 0]
    k = np.array([3, -4], f32)
    orc.clip_norm(k, 2, 1.0)
    np.testing.assert_allclose(k, [0.6, -0.8], atol=1e-7)


# --- Norms (kernels_test.cc:532-575, 725-735) --------------------------------

def test_rms_norm_naive_and_fd(orc):
    rows, cols = 3, 5
    x, g = rnd(rows * cols, 60), rnd(cols, 61)
    y, rstd = np.zeros(rows * cols, f32), np.zeros(rows, f32)
    orc.rms_norm_fwd(x, g, y, rstd, rows, cols)
    xd = x.reshape(rows, cols).astype(np.float64)
    rs = 1 / np.sqrt((xd ** 2).mean(axis=1) + 1e-5)
    np.testing.assert_allclose(rstd, rs, rtol=1e-5)
    np.testing.assert_allclose(y.reshape(rows, cols), xd * rs[:, None] * g, rtol=1e-5, atol=1e-5)
    # backward vs central differences of L = <dy, y>
    rows, cols = 2, 4
    n = rows * cols
    x, g, dy = rnd(n, 62), rnd(cols, 63), rnd(n, 64)
    y, rstd, dx = np.zeros(n, f32), np.zeros(rows, f32), np.zeros(n, f32)
    orc.rms_norm_fwd(x, g, y, rstd, rows, cols)
    orc.rms_norm_bwd(dy, x, g, rstd, dx, rows, cols)
    eps = 1e-3
    for i in range(n):
        xp, xm = x.copy(), x.copy()
        xp[i] += f32(eps)
        xm[i] -= f32(eps)
        yp, ym, t = np.zeros(n, f32), np.zeros(n, f32), np.zeros(rows, f32)
        orc.rms_norm_fwd(xp, g, yp, t, rows, cols)
        orc.rms_norm_fwd(xm, g, ym, t, rows, cols)
        fd = (np.dot(dy.astype(np.float64), yp) - np.dot(dy.astype(np.float64), ym)) / (2 * eps)
        assert abs(dx[i] - fd) < 2e-3


def test_layer_norm_zero_variance_and_fd(orc):
    x = np.full(4, 7.25, f32)
    beta = np.array([0.5, -1, 3, 0], f32)
    y, mean, rstd = np.zeros(4, f32), np.zeros(1, f32), np.zeros(1, f32)
    orc.layer_norm_fwd(x, np.full(4, 2, f32), beta, y, mean, rstd, 1, 4)
    assert np.array_equal(y, beta)
    rows, cols = 2, 5
    n = rows * cols
    x, g, b, dy = rnd(n, 65), rnd(cols, 66), rnd(cols, 67), rnd(n, 68)
    y, mean, rstd, dx = np.zeros(n, f32), np.zeros(rows, f32), np.zeros(rows, f32), np.zeros(n, f32)
    orc.layer_norm_fwd(x, g, b, y, mean, rstd, rows, cols)
    xd = x.reshape(rows, cols).astype(np.float64)
    mu = xd.mean(axis=1, keepdims=True)
    want = (xd - mu) / np.sqrt(((xd - mu) ** 2).mean(axis=1, keepdims=True) + 1e-5) * g + b
    np.testing.assert_allclose(y.reshape(rows, cols), want, rtol=1e-5, atol=1e-5)
    orc.layer_norm_bwd(dy, x, g, mean, rstd, dx, rows, cols)
    eps = 1e-3
    for i in range(n):
        xp, xm = x.copy(), x.copy()
        xp[i] += f32(eps)
        xm[i] -= f32(eps)
        yp, ym = np.zeros(n, f32), np.zeros(n, f32)
        t1, t2 = np.zeros(rows, f32), np.zeros(rows, f32)
        orc.layer_norm_fwd(xp, g, b, yp, t1, t2, rows, cols)
        orc.layer_norm_fwd(xm, g, b, ym, t1, t2, rows, cols)
        fd = (np.dot(dy.astype(np.float64), yp) - np.dot(dy.astype(np.float64), ym)) / (2 * eps)
        assert abs(dx[i] - fd) < 3e-3


# --- RoPE / attention (kernels_test.cc:577-687, 795-838) ----------------------

def test_rope_adjoint_and_position_zero(orc):
    B, S, H, d = 2, 3, 2, 4
    n = B * S * H * d
    x, y = rnd(n, 70), rnd(n, 71)
    rx, rty = np.zeros(n, f32), np.zeros(n, f32)
    orc.rope_fwd(x, rx, B, S, H, d, 10000.0)
    orc.rope_bwd(y, rty, B, S, H, d, 10000.0)
    assert abs(np.dot(rx.astype(np.float64), y) - np.dot(x.astype(np.float64), rty)) < 1e-4
    for b in range(B):
        s0 = slice(b * S * H * d, b * S * H * d + H * d)
        assert np.array_equal(rx[s0], x[s0])


def test_rope_golden_convention(orc):
    B, S, H, d = 1, 2, 1, 4
    x = rnd(B * S * H * d, 72)
    y = np.zeros_like(x)
    orc.rope_fwd(x, y, B, S, H, d, 10000.0)
    r1 = H * d
    xd = x.astype(np.float64)
    assert abs(y[r1] - (xd[r1] * math.cos(1) - xd[r1 + 1] * math.sin(1))) < 1e-5
    assert abs(y[r1 + 1] - (xd[r1] * math.sin(1) + xd[r1 + 1] * math.cos(1))) < 1e-5
    t1 = 0.01
    assert abs(y[r1 + 2] - (xd[r1 + 2] * math.cos(t1) - xd[r1 + 3] * math.sin(t1))) < 1e-5
    assert abs(y[r1 + 3] - (xd[r1 + 2] * math.sin(t1) + xd[r1 + 3] * math.cos(t1))) < 1e-5


def naive_attention(q, k, v, B, S, H, d):
    D = H * d
    q4 = q.reshape(B, S, H, d).astype(np.float64)
    k4 = k.reshape(B, S, H, d).astype(np.float64)
    v4 = v.reshape(B, S, H, d).astype(np.float64)
    sc = np.einsum("bihc,bjhc->bhij", q4, k4) / math.sqrt(d)
    mask = np.tril(np.ones((S, S), bool))
    sc = np.where(mask, sc, -np.inf)
    sc -= sc.max(axis=-1, keepdims=True)
    e = np.exp(sc)
    p = e / e.sum(axis=-1, keepdims=True)
    o = np.einsum("bhij,bjhc->bihc", p, v4).reshape(B * S, D)
    return o, p.reshape(B * H * S, S)


def test_attention_forward_naive_and_causal(orc):
    B, S, H, d = 2, 5, 2, 3
    n = B * S * H * d
    q, k, v = rnd(n, 80), rnd(n, 81), rnd(n, 82)
    o, p = np.zeros(n, f32), np.zeros(B * H * S * S, f32)
    orc.attn_fwd(q, k, v, o, p, B, S, H, d)
    wo, wp = naive_attention(q, k, v, B, S, H, d)
    np.testing.assert_allclose(p.reshape(-1, S), wp, atol=1e-6)
    np.testing.assert_allclose(o.reshape(B * S, H * d), wo, atol=1e-5)
    pm = p.reshape(B * H, S, S)
    for i in range(S):
        assert np.all(pm[:, i, i + 1:] == 0.0)


def test_attention_backward_matches_finite_differences(orc):
    B, S, H, d = 1, 3, 2, 2
    n = B * S * H * d
    pn = B * H * S * S
    q, k, v, w = rnd(n, 90), rnd(n, 91), rnd(n, 92), rnd(n, 93)
    o, p = np.zeros(n, f32), np.zeros(pn, f32)
    orc.attn_fwd(q, k, v, o, p, B, S, H, d)
    dp, ds = np.zeros(pn, f32), np.zeros(pn, f32)
    dq, dk, dv = np.zeros(n, f32), np.zeros(n, f32), np.zeros(n, f32)
    orc.attn_dp(w, v, dp, B, S, H, d)
    orc.attn_dv(p, w, dv, B, S, H, d)
    orc.softmax_rows_bwd(p, dp, ds, B * H * S, S)
    orc.attn_dq(ds, k, dq, B, S, H, d)
    orc.attn_dk(ds, q, dk, B, S, H, d)

    def loss(qq, kk, vv):
        oo, pp = np.zeros(n, f32), np.zeros(pn, f32)
        orc.attn_fwd(qq, kk, vv, oo, pp, B, S, H, d)
        return float(np.dot(w.astype(np.float64), oo))

    eps = 1e-3
    for which, base, g in ((0, q, dq), (1, k, dk), (2, v, dv)):
        for i in range(n):
            bp, bm = base.copy(), base.copy()
            bp[i] += f32(eps)
            bm[i] -= f32(eps)
            args_p = [q, k, v]
            args_m = [q, k, v]
            args_p[which] = bp
            args_m[which] = bm
            fd = (loss(*args_p) - loss(*args_m)) / (2 * eps)
            assert abs(g[i] - fd) < 2e-3


def test_attention_single_token_is_identity_over_v(orc):
    B, S, H, d = 2, 1, 2, 3
    n = B * S * H * d
    q, k, v = rnd(n, 130), rnd(n, 131), rnd(n, 132)
    o, p = np.zeros(n, f32), np.zeros(B * H, f32)
    orc.attn_fwd(q, k, v, o, p, B, S, H, d)
    assert p.tolist() == [1.0] * (B * H)
    assert np.array_equal(o, v)


# --- Engine pieces ----------------------------------------------------------------

def test_chunk_geometry(orc):
    assert orc.chunk_grain(1000, 32768) == 32768
    assert orc.chunk_count(1000, 32768) == 1
    assert orc.chunk_count(0, 5) == 0
    assert orc.chunk_grain(256 * 100 + 1, 1) == 101
    assert orc.chunk_count(33554432, 32768) == 256


def test_effective_lr_schedule_boundaries(orc):
    # constant schedule
    assert orc.effective_lr(1e-3, 0, 10, 100, 0.1, 5) == np.float32(1e-3)
    # warmup is linear and reaches lr at warmup_steps
    assert abs(orc.effective_lr(1.0, 1, 10, 100, 0.1, 5) - 0.5) < 1e-7
    assert abs(orc.effective_lr(1.0, 1, 10, 100, 0.1, 10) - 1.0) < 1e-7
    # cosine mid-horizon is halfway between lr and floor; past horizon = floor
    assert abs(orc.effective_lr(1.0, 1, 10, 110, 0.1, 60) - 0.55) < 1e-6
    assert abs(orc.effective_lr(1.0, 1, 10, 110, 0.1, 500) - 0.1) < 1e-7
