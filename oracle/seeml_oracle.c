/*
 * seeml_oracle.c — TEST INFRASTRUCTURE ONLY (see seeml_oracle.h).
 *
 * CPU restatement of the reference executor, built with -ffp-contract=off
 * so every float expression rounds exactly where the reference's does.
 * Chunked reductions reproduce ParallelFor's shape-only chunk geometry
 * (source/parallel/parallel_for.h:55-67): chunks run serially here, which
 * is bit-identical to any thread count by the reference's own design.
 *
 * Parity status per function (pinning evidence lives in tests/):
 *   every kernel: bit-exact against oracle/_ref (the reference's own
 *   executor sources compiled in place) on seeded random inputs, plus the
 *   reference's closed-form / known-answer cases (kernels_test.cc).
 *   orc_execute: pinned by per-opcode dispatch tests against the
 *   individual kernels and by whole-plan runs against oracle/_ref's
 *   kernels driven through the same decode.
 */
#include "seeml_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define ORC_MAX_CHUNKS 256
#define ORC_GRAIN_CHEAP 32768
#define ORC_GRAIN_MATH 4096
#define ORC_TILE_K 64

/* parallel_for.h:55-67 */
size_t orc_chunk_grain(size_t n, size_t grain) {
  if (grain == 0) grain = 1;
  const size_t cap = (n + ORC_MAX_CHUNKS - 1) / ORC_MAX_CHUNKS;
  return grain < cap ? cap : grain;
}

size_t orc_chunk_count(size_t n, size_t grain) {
  if (n == 0) return 0;
  const size_t g = orc_chunk_grain(n, grain);
  return (n + g - 1) / g;
}

/* kernel_policy.h:34-36 */
static size_t row_grain(size_t per_row, size_t budget) {
  return per_row == 0 ? budget : (budget / per_row > 0 ? budget / per_row : 1);
}

/* kernel_policy.h:47-67 — the shared activation expressions. */
static const float kGeluC = 0.7978845608028654f;
static const float kGeluA = 0.044715f;
static float sigmoid_expr(float x) { return 1.0f / (1.0f + expf(-x)); }
static float relu_expr(float x) { return x > 0.0f ? x : 0.0f; }
static float gelu_expr(float x) {
  const float t = tanhf(kGeluC * (x + kGeluA * x * x * x));
  return 0.5f * x * (1.0f + t);
}
static float silu_expr(float x) { return x * sigmoid_expr(x); }
static float act_expr(int act, float v) {
  switch (act) {
    case 1: return relu_expr(v);
    case 2: return gelu_expr(v);
    case 3: return silu_expr(v);
    default: return v;
  }
}

/* ---- GEMM family (gemm.cc) ------------------------------------------------ */

/* BlockedNN (gemm.cc:55-93): per C element, k advances in 4-wide groups
 * inside 64-wide K tiles, c += ((a0 b0 + a1 b1) + a2 b2) + a3 b3 with each a
 * pre-multiplied by alpha; a K tile's remainder is added one k at a time.
 * The N tile only changes traversal order, never the per-element sequence,
 * so it is omitted here. */
static void blocked_nn_f32(const float* A, const float* B, float* C, size_t M,
                           size_t N, size_t K, float alpha, size_t a_stride,
                           int a_transposed) {
  for (size_t k0 = 0; k0 < K; k0 += ORC_TILE_K) {
    const size_t k1 = k0 + ORC_TILE_K < K ? k0 + ORC_TILE_K : K;
    for (size_t m = 0; m < M; ++m) {
      float* c_row = C + m * N;
      size_t k = k0;
#define A_AT(kk) (a_transposed ? A[(kk) * a_stride + m] : A[m * a_stride + (kk)])
      for (; k + 4 <= k1; k += 4) {
        const float a0 = alpha * A_AT(k + 0);
        const float a1 = alpha * A_AT(k + 1);
        const float a2 = alpha * A_AT(k + 2);
        const float a3 = alpha * A_AT(k + 3);
        const float* b0 = B + (k + 0) * N;
        const float* b1 = B + (k + 1) * N;
        const float* b2 = B + (k + 2) * N;
        const float* b3 = B + (k + 3) * N;
        for (size_t n = 0; n < N; ++n)
          c_row[n] += a0 * b0[n] + a1 * b1[n] + a2 * b2[n] + a3 * b3[n];
      }
      for (; k < k1; ++k) {
        const float a = alpha * A_AT(k);
        const float* b_row = B + k * N;
        for (size_t n = 0; n < N; ++n) c_row[n] += a * b_row[n];
      }
#undef A_AT
    }
  }
}

static void blocked_nn_q8(const float* A, const int8_t* B, float* C, size_t M,
                          size_t N, size_t K, float alpha) {
  for (size_t k0 = 0; k0 < K; k0 += ORC_TILE_K) {
    const size_t k1 = k0 + ORC_TILE_K < K ? k0 + ORC_TILE_K : K;
    for (size_t m = 0; m < M; ++m) {
      float* c_row = C + m * N;
      size_t k = k0;
      for (; k + 4 <= k1; k += 4) {
        const float a0 = alpha * A[m * K + k + 0];
        const float a1 = alpha * A[m * K + k + 1];
        const float a2 = alpha * A[m * K + k + 2];
        const float a3 = alpha * A[m * K + k + 3];
        const int8_t* b0 = B + (k + 0) * N;
        const int8_t* b1 = B + (k + 1) * N;
        const int8_t* b2 = B + (k + 2) * N;
        const int8_t* b3 = B + (k + 3) * N;
        for (size_t n = 0; n < N; ++n)
          c_row[n] += a0 * (float)b0[n] + a1 * (float)b1[n] +
                      a2 * (float)b2[n] + a3 * (float)b3[n];
      }
      for (; k < k1; ++k) {
        const float a = alpha * A[m * K + k];
        const int8_t* b_row = B + k * N;
        for (size_t n = 0; n < N; ++n) c_row[n] += a * (float)b_row[n];
      }
    }
  }
}

/* EpilogueRows (gemm.cc:145-169): c = act(bias ? c + bias[n] : c). */
static void epilogue_rows(float* C, const float* bias, size_t M, size_t N,
                          int act) {
  if (act == 0 && !bias) return;
  for (size_t m = 0; m < M; ++m)
    for (size_t n = 0; n < N; ++n) {
      const float v = bias ? C[m * N + n] + bias[n] : C[m * N + n];
      C[m * N + n] = act_expr(act, v);
    }
}

/* gemm.cc:173-182 */
void orc_gemm_nn(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K, const float* bias, int act) {
  memset(C, 0, M * N * sizeof(float));
  blocked_nn_f32(A, B, C, M, N, K, 1.0f, K, 0);
  epilogue_rows(C, bias, M, N, act);
}

/* BlockedNT (gemm.cc:99-136): one sequential f32 accumulator per output,
 * then alpha * acc. */
void orc_gemm_nt(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K) {
  for (size_t m = 0; m < M; ++m)
    for (size_t n = 0; n < N; ++n) {
      float acc = 0.0f;
      for (size_t k = 0; k < K; ++k) acc += A[m * K + k] * B[n * K + k];
      C[m * N + n] = 1.0f * acc;
    }
}

/* gemm.cc:192-200 */
void orc_gemm_tn(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K) {
  memset(C, 0, M * N * sizeof(float));
  blocked_nn_f32(A, B, C, M, N, K, 1.0f, M, 1);
}

/* gemm.cc:202-209 */
void orc_gemm_acc_nn(const float* A, const float* B, float* C, size_t M,
                     size_t N, size_t K, float alpha) {
  blocked_nn_f32(A, B, C, M, N, K, alpha, K, 0);
}

/* gemm.cc:211-220 */
void orc_gemm_nn_q8(const float* A, const int8_t* B, float* C, size_t M,
                    size_t N, size_t K, float scale, int act) {
  memset(C, 0, M * N * sizeof(float));
  blocked_nn_q8(A, B, C, M, N, K, scale);
  epilogue_rows(C, NULL, M, N, act);
}

/* gemm.cc:222-228 */
void orc_gemm_nt_q8(const float* A, const int8_t* B, float* C, size_t M,
                    size_t N, size_t K, float scale) {
  for (size_t m = 0; m < M; ++m)
    for (size_t n = 0; n < N; ++n) {
      float acc = 0.0f;
      for (size_t k = 0; k < K; ++k) acc += A[m * K + k] * (float)B[n * K + k];
      C[m * N + n] = scale * acc;
    }
}

/* ---- Elementwise (elementwise.cc, activation.cc) ------------------------- */

void orc_add_ew(const float* x, const float* y, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = x[i] + y[i]; /* elementwise.cc:16-20 */
}
void orc_mul_ew(const float* x, const float* y, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = x[i] * y[i]; /* elementwise.cc:22-26 */
}
void orc_add_bias(const float* x, const float* b, float* out, size_t rows,
                  size_t cols) { /* elementwise.cc:28-36 */
  for (size_t r = 0; r < rows; ++r)
    for (size_t c = 0; c < cols; ++c) out[r * cols + c] = x[r * cols + c] + b[c];
}
void orc_scale(const float* x, float* out, float alpha, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = alpha * x[i]; /* elementwise.cc:38-42 */
}
void orc_reduce_rows(const float* dy, float* db, size_t rows, size_t cols) {
  /* elementwise.cc:55-67: column-owned, rows in order. */
  for (size_t c = 0; c < cols; ++c) db[c] = 0.0f;
  for (size_t r = 0; r < rows; ++r)
    for (size_t c = 0; c < cols; ++c) db[c] += dy[r * cols + c];
}
void orc_relu_fwd(const float* x, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = relu_expr(x[i]); /* activation.cc:22-26 */
}
void orc_relu_bwd(const float* dy, const float* x, float* dx, size_t n) {
  for (size_t i = 0; i < n; ++i) dx[i] = x[i] > 0.0f ? dy[i] : 0.0f; /* :28-32 */
}
void orc_gelu_fwd(const float* x, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = gelu_expr(x[i]); /* activation.cc:34-38 */
}
void orc_gelu_bwd(const float* dy, const float* x, float* dx, size_t n) {
  /* activation.cc:40-60, including the saturation guard. */
  for (size_t i = 0; i < n; ++i) {
    const float v = x[i];
    const float u = kGeluC * (v + kGeluA * v * v * v);
    const float t = tanhf(u);
    const float one_minus_t2 = 1.0f - t * t;
    const float tail =
        one_minus_t2 == 0.0f
            ? 0.0f
            : 0.5f * v * one_minus_t2 * (kGeluC * (1.0f + 3.0f * kGeluA * v * v));
    dx[i] = dy[i] * (0.5f * (1.0f + t) + tail);
  }
}
void orc_silu_fwd(const float* x, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = silu_expr(x[i]); /* activation.cc:62-66 */
}
void orc_silu_bwd(const float* dy, const float* x, float* dx, size_t n) {
  for (size_t i = 0; i < n; ++i) { /* activation.cc:68-75 */
    const float s = sigmoid_expr(x[i]);
    dx[i] = dy[i] * (s * (1.0f + x[i] * (1.0f - s)));
  }
}
void orc_embed_fwd(const int32_t* tokens, const float* table, float* out,
                   size_t rows, size_t dim) { /* elementwise.cc:44-53 */
  for (size_t r = 0; r < rows; ++r)
    memcpy(out + r * dim, table + (size_t)tokens[r] * dim, dim * sizeof(float));
}
void orc_fill(float* dst, float value, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = value; /* elementwise.cc:72-74 */
}
void orc_copy(const float* src, float* dst, size_t n) {
  memcpy(dst, src, n * sizeof(float)); /* elementwise.cc:76-78 */
}

/* ---- Normalization (normalization.cc) ------------------------------------- */

void orc_layer_norm_fwd(const float* x, const float* gamma, const float* beta,
                        float* y, float* mean, float* rstd, size_t rows,
                        size_t cols) { /* normalization.cc:17-42 */
  const float kEps = 1e-5f;
  for (size_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    double sum = 0.0;
    for (size_t c = 0; c < cols; ++c) sum += xr[c];
    const float mu = (float)(sum / (double)cols);
    double var = 0.0;
    for (size_t c = 0; c < cols; ++c) {
      const double d = (double)xr[c] - mu;
      var += d * d;
    }
    const float rs = 1.0f / sqrtf((float)(var / (double)cols) + kEps);
    mean[r] = mu;
    rstd[r] = rs;
    float* yr = y + r * cols;
    for (size_t c = 0; c < cols; ++c) yr[c] = (xr[c] - mu) * rs * gamma[c] + beta[c];
  }
}

void orc_layer_norm_bwd(const float* dy, const float* x, const float* gamma,
                        const float* mean, const float* rstd, float* dx,
                        size_t rows, size_t cols) { /* normalization.cc:44-73 */
  const float inv_d = 1.0f / (float)cols;
  for (size_t r = 0; r < rows; ++r) {
    const float* dyr = dy + r * cols;
    const float* xr = x + r * cols;
    float* dxr = dx + r * cols;
    const float mu = mean[r], rs = rstd[r];
    double sum_g = 0.0, sum_gx = 0.0;
    for (size_t c = 0; c < cols; ++c) {
      const float xhat = (xr[c] - mu) * rs;
      const float g = dyr[c] * gamma[c];
      sum_g += g;
      sum_gx += (double)g * xhat;
    }
    const float mg = (float)sum_g * inv_d;
    const float mgx = (float)sum_gx * inv_d;
    for (size_t c = 0; c < cols; ++c) {
      const float xhat = (xr[c] - mu) * rs;
      const float g = dyr[c] * gamma[c];
      dxr[c] = rs * (g - mg - xhat * mgx);
    }
  }
}

void orc_rms_norm_fwd(const float* x, const float* gamma, float* y,
                      float* rstd, size_t rows, size_t cols) { /* :75-92 */
  const float kEps = 1e-5f;
  for (size_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    double ss = 0.0;
    for (size_t c = 0; c < cols; ++c) ss += (double)xr[c] * xr[c];
    const float rs = 1.0f / sqrtf((float)(ss / (double)cols) + kEps);
    rstd[r] = rs;
    float* yr = y + r * cols;
    for (size_t c = 0; c < cols; ++c) yr[c] = xr[c] * rs * gamma[c];
  }
}

void orc_rms_norm_bwd(const float* dy, const float* x, const float* gamma,
                      const float* rstd, float* dx, size_t rows,
                      size_t cols) { /* normalization.cc:94-113 */
  const float inv_d = 1.0f / (float)cols;
  for (size_t r = 0; r < rows; ++r) {
    const float* dyr = dy + r * cols;
    const float* xr = x + r * cols;
    float* dxr = dx + r * cols;
    const float rs = rstd[r];
    double sum_gx = 0.0;
    for (size_t c = 0; c < cols; ++c)
      sum_gx += (double)(dyr[c] * gamma[c]) * xr[c];
    const float mgx = (float)sum_gx * inv_d;
    for (size_t c = 0; c < cols; ++c)
      dxr[c] = rs * (dyr[c] * gamma[c] - xr[c] * rs * rs * mgx);
  }
}

/* ---- Transformer family (attention.cc) ------------------------------------ */

void orc_rope_fwd(const float* x, float* y, size_t B, size_t S, size_t H,
                  size_t d, float base) { /* attention.cc:39-66 */
  const size_t D = H * d;
  const float step = powf(base, -2.0f / (float)d);
  for (size_t u = 0; u < B * S * H; ++u) {
    const size_t s = (u / H) % S;
    const float* xr = x + (u / H) * D + (u % H) * d;
    float* yr = y + (u / H) * D + (u % H) * d;
    float freq = 1.0f;
    for (size_t c = 0; c + 1 < d; c += 2) {
      const float theta = (float)s * freq;
      const float cs = cosf(theta), sn = sinf(theta);
      const float a = xr[c], b2 = xr[c + 1];
      yr[c] = a * cs - b2 * sn;
      yr[c + 1] = a * sn + b2 * cs;
      freq *= step;
    }
  }
}

void orc_rope_bwd(const float* dy, float* dx, size_t B, size_t S, size_t H,
                  size_t d, float base) { /* attention.cc:68-92 */
  const size_t D = H * d;
  const float step = powf(base, -2.0f / (float)d);
  for (size_t u = 0; u < B * S * H; ++u) {
    const size_t s = (u / H) % S;
    const float* gr = dy + (u / H) * D + (u % H) * d;
    float* dr = dx + (u / H) * D + (u % H) * d;
    float freq = 1.0f;
    for (size_t c = 0; c + 1 < d; c += 2) {
      const float theta = (float)s * freq;
      const float cs = cosf(theta), sn = sinf(theta);
      const float a = gr[c], b2 = gr[c + 1];
      dr[c] = a * cs + b2 * sn;
      dr[c + 1] = -a * sn + b2 * cs;
      freq *= step;
    }
  }
}

/* attention.cc:94-136 */
void orc_attn_fwd(const float* q, const float* k, const float* v, float* o,
                  float* probs, size_t B, size_t S, size_t H, size_t d) {
  const size_t D = H * d;
  const float inv_sqrt_d = 1.0f / sqrtf((float)d);
  for (size_t u = 0; u < B * H * S; ++u) {
    const size_t b = u / (H * S), h = (u / S) % H, i = u % S;
    const float* qi = q + (b * S + i) * D + h * d;
    float* prow = probs + u * S;
    float row_max = -INFINITY;
    for (size_t j = 0; j <= i; ++j) {
      const float* kj = k + (b * S + j) * D + h * d;
      double dot = 0.0;
      for (size_t c = 0; c < d; ++c) dot += (double)qi[c] * kj[c];
      const float s = (float)dot * inv_sqrt_d;
      prow[j] = s;
      if (s > row_max) row_max = s;
    }
    double denom = 0.0;
    for (size_t j = 0; j <= i; ++j) {
      const float e = expf(prow[j] - row_max);
      prow[j] = e;
      denom += e;
    }
    const float inv_denom = 1.0f / (float)denom;
    for (size_t j = 0; j <= i; ++j) prow[j] *= inv_denom;
    for (size_t j = i + 1; j < S; ++j) prow[j] = 0.0f;
    float* oi = o + (b * S + i) * D + h * d;
    for (size_t c = 0; c < d; ++c) oi[c] = 0.0f;
    for (size_t j = 0; j <= i; ++j) {
      const float p = prow[j];
      const float* vj = v + (b * S + j) * D + h * d;
      for (size_t c = 0; c < d; ++c) oi[c] += p * vj[c];
    }
  }
}

/* attention.cc:138-163 */
void orc_attn_dp(const float* dout, const float* v, float* dp, size_t B,
                 size_t S, size_t H, size_t d) {
  const size_t D = H * d;
  for (size_t u = 0; u < B * H * S; ++u) {
    const size_t b = u / (H * S), h = (u / S) % H, i = u % S;
    const float* doi = dout + (b * S + i) * D + h * d;
    float* dprow = dp + u * S;
    for (size_t j = 0; j <= i; ++j) {
      const float* vj = v + (b * S + j) * D + h * d;
      double dot = 0.0;
      for (size_t c = 0; c < d; ++c) dot += (double)doi[c] * vj[c];
      dprow[j] = (float)dot;
    }
    for (size_t j = i + 1; j < S; ++j) dprow[j] = 0.0f;
  }
}

/* attention.cc:165-183 */
void orc_attn_dv(const float* probs, const float* dout, float* dv, size_t B,
                 size_t S, size_t H, size_t d) {
  const size_t D = H * d;
  for (size_t u = 0; u < B * H * S; ++u) {
    const size_t b = u / (H * S), h = (u / S) % H, j = u % S;
    float* dvj = dv + (b * S + j) * D + h * d;
    for (size_t c = 0; c < d; ++c) dvj[c] = 0.0f;
    for (size_t i = j; i < S; ++i) {
      const float p = probs[((b * H + h) * S + i) * S + j];
      const float* doi = dout + (b * S + i) * D + h * d;
      for (size_t c = 0; c < d; ++c) dvj[c] += p * doi[c];
    }
  }
}

/* attention.cc:185-201 */
void orc_softmax_rows_bwd(const float* probs, const float* dp, float* ds,
                          size_t rows, size_t cols) {
  for (size_t r = 0; r < rows; ++r) {
    const float* pr = probs + r * cols;
    const float* dpr = dp + r * cols;
    float* dsr = ds + r * cols;
    double dot = 0.0;
    for (size_t c = 0; c < cols; ++c) dot += (double)dpr[c] * pr[c];
    const float sum = (float)dot;
    for (size_t c = 0; c < cols; ++c) dsr[c] = pr[c] * (dpr[c] - sum);
  }
}

/* attention.cc:203-222 */
void orc_attn_dq(const float* ds, const float* k, float* dq, size_t B,
                 size_t S, size_t H, size_t d) {
  const size_t D = H * d;
  const float inv_sqrt_d = 1.0f / sqrtf((float)d);
  for (size_t u = 0; u < B * H * S; ++u) {
    const size_t b = u / (H * S), h = (u / S) % H, i = u % S;
    const float* dsrow = ds + u * S;
    float* dqi = dq + (b * S + i) * D + h * d;
    for (size_t c = 0; c < d; ++c) dqi[c] = 0.0f;
    for (size_t j = 0; j <= i; ++j) {
      const float g = dsrow[j] * inv_sqrt_d;
      const float* kj = k + (b * S + j) * D + h * d;
      for (size_t c = 0; c < d; ++c) dqi[c] += g * kj[c];
    }
  }
}

/* attention.cc:224-242 */
void orc_attn_dk(const float* ds, const float* q, float* dk, size_t B,
                 size_t S, size_t H, size_t d) {
  const size_t D = H * d;
  const float inv_sqrt_d = 1.0f / sqrtf((float)d);
  for (size_t u = 0; u < B * H * S; ++u) {
    const size_t b = u / (H * S), h = (u / S) % H, j = u % S;
    float* dkj = dk + (b * S + j) * D + h * d;
    for (size_t c = 0; c < d; ++c) dkj[c] = 0.0f;
    for (size_t i = j; i < S; ++i) {
      const float g = ds[((b * H + h) * S + i) * S + j] * inv_sqrt_d;
      const float* qi = q + (b * S + i) * D + h * d;
      for (size_t c = 0; c < d; ++c) dkj[c] += g * qi[c];
    }
  }
}

/* ---- Losses (loss.cc) ------------------------------------------------------ */

/* RowSoftmax (loss.cc:21-32) */
static void row_softmax(const float* logits, float* probs, size_t C,
                        float inv_T) {
  float max_v = logits[0] * inv_T;
  for (size_t c = 1; c < C; ++c) max_v = fmaxf(max_v, logits[c] * inv_T);
  float sum = 0.0f;
  for (size_t c = 0; c < C; ++c) {
    probs[c] = expf(logits[c] * inv_T - max_v);
    sum += probs[c];
  }
  const float inv_sum = 1.0f / sum;
  for (size_t c = 0; c < C; ++c) probs[c] *= inv_sum;
}

/* loss.cc:36-59: one double partial per ParallelFor chunk, chunk order. */
void orc_softmax_xent_fwd(const float* logits, const int32_t* labels,
                          float* loss, float* probs, size_t N, size_t C) {
  const size_t grain = row_grain(C, ORC_GRAIN_MATH);
  const size_t g = orc_chunk_grain(N, grain);
  const size_t chunks = orc_chunk_count(N, grain);
  double partials[ORC_MAX_CHUNKS] = {0};
  for (size_t ch = 0; ch < chunks; ++ch) {
    const size_t r0 = ch * g, r1 = r0 + g < N ? r0 + g : N;
    double total = 0.0;
    for (size_t n = r0; n < r1; ++n) {
      row_softmax(logits + n * C, probs + n * C, C, 1.0f);
      const float p = probs[n * C + (size_t)labels[n]];
      const double safe = isnan(p) ? (double)p : (double)fmaxf(p, 1e-12f);
      total -= log(safe);
    }
    partials[ch] = total;
  }
  double total = 0.0;
  for (size_t ch = 0; ch < chunks; ++ch) total += partials[ch];
  *loss = (float)(total / (double)N);
}

/* loss.cc:61-72 */
void orc_softmax_xent_bwd(const float* probs, const int32_t* labels,
                          const float* seed, float* dlogits, size_t N,
                          size_t C) {
  const float scale = *seed / (float)N;
  for (size_t n = 0; n < N; ++n) {
    for (size_t c = 0; c < C; ++c) dlogits[n * C + c] = scale * probs[n * C + c];
    dlogits[n * C + (size_t)labels[n]] -= scale;
  }
}

/* loss.cc:74-89 */
void orc_mse_fwd(const float* pred, const float* target, float* loss,
                 size_t n) {
  const size_t g = orc_chunk_grain(n, ORC_GRAIN_CHEAP);
  const size_t chunks = orc_chunk_count(n, ORC_GRAIN_CHEAP);
  double partials[ORC_MAX_CHUNKS] = {0};
  for (size_t ch = 0; ch < chunks; ++ch) {
    const size_t b = ch * g, e = b + g < n ? b + g : n;
    double total = 0.0;
    for (size_t i = b; i < e; ++i) {
      const double d = (double)pred[i] - target[i];
      total += d * d;
    }
    partials[ch] = total;
  }
  double total = 0.0;
  for (size_t ch = 0; ch < chunks; ++ch) total += partials[ch];
  *loss = (float)(total / (double)n);
}

/* loss.cc:91-97 */
void orc_mse_bwd(const float* pred, const float* target, const float* seed,
                 float* dpred, size_t n) {
  const float scale = 2.0f * *seed / (float)n;
  for (size_t i = 0; i < n; ++i) dpred[i] = scale * (pred[i] - target[i]);
}

/* loss.cc:99-132 */
void orc_kl_distill_fwd(const float* s_logits, const float* t_logits,
                        float* loss, float* p_s, float* p_t, size_t N,
                        size_t C, float T) {
  const float inv_T = 1.0f / T;
  const size_t grain = row_grain(C, ORC_GRAIN_MATH);
  const size_t g = orc_chunk_grain(N, grain);
  const size_t chunks = orc_chunk_count(N, grain);
  double partials[ORC_MAX_CHUNKS] = {0};
  for (size_t ch = 0; ch < chunks; ++ch) {
    const size_t r0 = ch * g, r1 = r0 + g < N ? r0 + g : N;
    double total = 0.0;
    for (size_t n = r0; n < r1; ++n) {
      row_softmax(s_logits + n * C, p_s + n * C, C, inv_T);
      row_softmax(t_logits + n * C, p_t + n * C, C, inv_T);
      for (size_t c = 0; c < C; ++c) {
        const float pt = p_t[n * C + c];
        if (pt <= 0.0f) continue;
        const float ps_raw = p_s[n * C + c];
        const double ps =
            isnan(ps_raw) ? (double)ps_raw : (double)fmaxf(ps_raw, 1e-12f);
        total += (double)pt * (log((double)pt) - log(ps));
      }
    }
    partials[ch] = total;
  }
  double total = 0.0;
  for (size_t ch = 0; ch < chunks; ++ch) total += partials[ch];
  *loss = (float)(total / (double)N);
}

/* loss.cc:134-140 */
void orc_kl_distill_bwd(const float* p_s, const float* p_t, const float* seed,
                        float* dlogits, size_t N, size_t C, float T) {
  const float scale = *seed / ((float)N * T);
  for (size_t i = 0; i < N * C; ++i) dlogits[i] = scale * (p_s[i] - p_t[i]);
}

/* ---- Optimizers (optimizer.cc) ---------------------------------------------- */

/* optimizer.cc:17-35 */
void orc_clip_norm(float* g, size_t n, float max_norm) {
  const size_t gr = orc_chunk_grain(n, ORC_GRAIN_CHEAP);
  const size_t chunks = orc_chunk_count(n, ORC_GRAIN_CHEAP);
  double partials[ORC_MAX_CHUNKS] = {0};
  for (size_t ch = 0; ch < chunks; ++ch) {
    const size_t b = ch * gr, e = b + gr < n ? b + gr : n;
    double sq = 0.0;
    for (size_t i = b; i < e; ++i) sq += (double)g[i] * (double)g[i];
    partials[ch] = sq;
  }
  double sq = 0.0;
  for (size_t ch = 0; ch < chunks; ++ch) sq += partials[ch];
  const double norm = sqrt(sq);
  if (norm <= (double)max_norm || norm == 0.0) return;
  const float s = (float)((double)max_norm / norm);
  for (size_t i = 0; i < n; ++i) g[i] *= s;
}

/* optimizer.cc:37-42 */
void orc_sgd_step(float* p, const float* g, size_t n, float lr, float wd) {
  for (size_t i = 0; i < n; ++i) p[i] -= lr * (g[i] + wd * p[i]);
}

/* optimizer.cc:44-69 */
void orc_adamw_step(float* p, const float* g, float* m, float* v, size_t n,
                    float lr, float beta1, float beta2, float eps, float wd,
                    uint64_t step) {
  const float inv_bc1 = 1.0f / (1.0f - powf(beta1, (float)step));
  const float inv_bc2 = 1.0f / (1.0f - powf(beta2, (float)step));
  const float om_b1 = 1.0f - beta1;
  const float om_b2 = 1.0f - beta2;
  for (size_t i = 0; i < n; ++i) {
    const float gi = g[i];
    const float mi = beta1 * m[i] + om_b1 * gi;
    const float vi = beta2 * v[i] + om_b2 * gi * gi;
    m[i] = mi;
    v[i] = vi;
    const float m_hat = mi * inv_bc1;
    const float v_hat = vi * inv_bc2;
    p[i] -= lr * (m_hat / (sqrtf(v_hat) + eps) + wd * p[i]);
  }
}

/* ---- Compiler pieces (compiler/driver/update_compiler.cc) --------------------- */

/* update_compiler.cc:415-436: element j of a "randn" adapter tensor mixes two
 * splitmix64 draws from the counter seed + golden * (2j + 1) and feeds
 * Box-Muller in double, with the C library's log, sqrt and cos, rounded to
 * f32 (the tensor's std is applied by the caller). */
void orc_counter_randn(uint64_t seed, uint64_t count, float* out) {
  const uint64_t golden = 0x9E3779B97F4A7C15ULL;
  for (uint64_t j = 0; j < count; ++j) {
    uint64_t s = seed + golden * (2 * j + 1);
    uint64_t d[2];
    for (int k = 0; k < 2; ++k) {
      uint64_t z = (s += golden);
      z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
      z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
      d[k] = z ^ (z >> 31);
    }
    const double u1 = ((double)(d[0] >> 11) + 1.0) * 0x1.0p-53;
    const double u2 = (double)(d[1] >> 11) * 0x1.0p-53;
    const double two_pi = 6.283185307179586476925286766559;
    out[j] = (float)(sqrt(-2.0 * log(u1)) * cos(two_pi * u2));
  }
}

/* ---- Engine pieces (update_engine.cc) ----------------------------------------- */

/* update_engine.cc:515-534 */
float orc_effective_lr(float lr, uint32_t schedule, uint64_t warmup_steps,
                       uint64_t default_steps, float min_lr_factor,
                       uint64_t step) {
  const float base = lr;
  if (schedule != 1) return base;
  if (warmup_steps > 0 && step <= warmup_steps)
    return base * (float)step / (float)warmup_steps;
  const uint64_t horizon =
      default_steps > warmup_steps ? default_steps - warmup_steps : 0;
  const float floor_v = base * min_lr_factor;
  if (horizon == 0 || step - warmup_steps >= horizon) return floor_v;
  const float t = (float)(step - warmup_steps) / (float)horizon;
  const float kPi = 3.14159265358979323846f;
  return floor_v + (base - floor_v) * 0.5f * (1.0f + cosf(kPi * t));
}

#pragma pack(push, 1)
typedef struct {
  uint16_t opcode;
  uint16_t flags;
  uint32_t pad;
  uint64_t in[4];
  uint64_t out[3];
} OrcInstr;
#pragma pack(pop)

static float bits_f32(uint64_t bits) {
  uint32_t u = (uint32_t)bits;
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

#define RODATA_BIT (1ULL << 63)
#define LO32(w) ((size_t)((w) & 0xFFFFFFFFu))
#define HI32(w) ((size_t)((w) >> 32))

/* update_engine.cc:306-509: decode each word into raw pointers and call the
 * kernel. ReadPtr = base + RefOffset(ref) in arena or rodata (:39-55). */
void orc_execute(const void* program, size_t count, uint8_t* arena,
                 const uint8_t* rodata, float lr, float beta1, float beta2,
                 float eps, float weight_decay, uint64_t step) {
  const OrcInstr* prog = (const OrcInstr*)program;
#define RP(ref) ((const float*)(((ref) & RODATA_BIT) ? rodata + ((ref) & ~RODATA_BIT) : arena + (ref)))
#define RQ8(ref) ((const int8_t*)(rodata + ((ref) & ~RODATA_BIT)))
#define WP(ref) ((float*)(arena + ((ref) & ~RODATA_BIT)))
#define IP(ref) ((const int32_t*)RP(ref))
  for (size_t idx = 0; idx < count; ++idx) {
    OrcInstr ins;
    memcpy(&ins, prog + idx, sizeof ins);
    const int act = (ins.flags >> 1) & 3;
    switch (ins.opcode) {
      case 0: break;
      case 1:
        orc_gemm_nn(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), ins.out[0],
                    ins.out[1], ins.out[2], (ins.flags & 1) ? RP(ins.in[3]) : NULL,
                    act);
        break;
      case 2:
        orc_gemm_nt(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), ins.out[0],
                    ins.out[1], ins.out[2]);
        break;
      case 3:
        orc_gemm_tn(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), ins.out[0],
                    ins.out[1], ins.out[2]);
        break;
      case 4:
        orc_gemm_acc_nn(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]),
                        ins.out[0], ins.out[1], ins.out[2], bits_f32(ins.in[3]));
        break;
      case 5: orc_add_ew(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), ins.out[0]); break;
      case 6:
        orc_add_bias(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), ins.out[0],
                     ins.out[1]);
        break;
      case 7: orc_relu_fwd(RP(ins.in[0]), WP(ins.in[1]), ins.out[0]); break;
      case 8: orc_relu_bwd(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), ins.out[0]); break;
      case 9: orc_scale(RP(ins.in[0]), WP(ins.in[1]), bits_f32(ins.in[2]), ins.out[0]); break;
      case 10: orc_reduce_rows(RP(ins.in[0]), WP(ins.in[1]), ins.out[0], ins.out[1]); break;
      case 11:
        orc_softmax_xent_fwd(RP(ins.in[0]), IP(ins.in[1]), WP(ins.in[2]),
                             WP(ins.in[3]), ins.out[0], ins.out[1]);
        break;
      case 12:
        orc_softmax_xent_bwd(RP(ins.in[0]), IP(ins.in[1]), RP(ins.in[2]),
                             WP(ins.in[3]), ins.out[0], ins.out[1]);
        break;
      case 13: orc_mse_fwd(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), ins.out[0]); break;
      case 14:
        orc_mse_bwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), WP(ins.in[3]),
                    ins.out[0]);
        break;
      case 15:
        orc_kl_distill_fwd(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]),
                           WP(ins.in[3]), WP(ins.out[0]), HI32(ins.out[1]),
                           LO32(ins.out[1]), bits_f32(ins.out[2]));
        break;
      case 16:
        orc_kl_distill_bwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]),
                           WP(ins.in[3]), HI32(ins.out[0]), LO32(ins.out[0]),
                           bits_f32(ins.out[1]));
        break;
      case 17: orc_sgd_step(WP(ins.in[0]), RP(ins.in[1]), ins.out[0], lr, weight_decay); break;
      case 18:
        orc_adamw_step(WP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), WP(ins.in[3]),
                       ins.out[0], lr, beta1, beta2, eps, weight_decay, step);
        break;
      case 19: orc_fill(WP(ins.in[0]), bits_f32(ins.in[1]), ins.out[0]); break;
      case 20: orc_copy(RP(ins.in[0]), WP(ins.in[1]), ins.out[0]); break;
      case 21: orc_mul_ew(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), ins.out[0]); break;
      case 22: orc_gelu_fwd(RP(ins.in[0]), WP(ins.in[1]), ins.out[0]); break;
      case 23: orc_gelu_bwd(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), ins.out[0]); break;
      case 24: orc_silu_fwd(RP(ins.in[0]), WP(ins.in[1]), ins.out[0]); break;
      case 25: orc_silu_bwd(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), ins.out[0]); break;
      case 26:
        orc_layer_norm_fwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]),
                           WP(ins.in[3]), WP(ins.out[1]), WP(ins.out[2]),
                           HI32(ins.out[0]), LO32(ins.out[0]));
        break;
      case 27:
        orc_layer_norm_bwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]),
                           RP(ins.out[0]), RP(ins.out[1]), WP(ins.in[3]),
                           HI32(ins.out[2]), LO32(ins.out[2]));
        break;
      case 28: orc_clip_norm(WP(ins.in[0]), ins.out[0], bits_f32(ins.in[1])); break;
      case 29:
        orc_gemm_nn_q8(RP(ins.in[0]), RQ8(ins.in[1]), WP(ins.in[2]), ins.out[0],
                       ins.out[1], ins.out[2], bits_f32(ins.in[3]), act);
        break;
      case 30:
        orc_gemm_nt_q8(RP(ins.in[0]), RQ8(ins.in[1]), WP(ins.in[2]), ins.out[0],
                       ins.out[1], ins.out[2], bits_f32(ins.in[3]));
        break;
      case 31:
        orc_rms_norm_fwd(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]),
                         WP(ins.in[3]), HI32(ins.out[0]), LO32(ins.out[0]));
        break;
      case 32:
        orc_rms_norm_bwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]),
                         RP(ins.out[0]), WP(ins.in[3]), HI32(ins.out[1]),
                         LO32(ins.out[1]));
        break;
      case 33:
        orc_rope_fwd(RP(ins.in[0]), WP(ins.in[1]), HI32(ins.out[0]), LO32(ins.out[0]),
                     HI32(ins.out[1]), LO32(ins.out[1]), bits_f32(ins.out[2]));
        break;
      case 34:
        orc_rope_bwd(RP(ins.in[0]), WP(ins.in[1]), HI32(ins.out[0]), LO32(ins.out[0]),
                     HI32(ins.out[1]), LO32(ins.out[1]), bits_f32(ins.out[2]));
        break;
      case 35:
        orc_attn_fwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), WP(ins.in[3]),
                     WP(ins.out[0]), HI32(ins.out[1]), LO32(ins.out[1]),
                     HI32(ins.out[2]), LO32(ins.out[2]));
        break;
      case 36:
        orc_attn_dp(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), HI32(ins.out[0]),
                    LO32(ins.out[0]), HI32(ins.out[1]), LO32(ins.out[1]));
        break;
      case 37:
        orc_attn_dv(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), HI32(ins.out[0]),
                    LO32(ins.out[0]), HI32(ins.out[1]), LO32(ins.out[1]));
        break;
      case 38:
        orc_softmax_rows_bwd(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]),
                             HI32(ins.out[0]), LO32(ins.out[0]));
        break;
      case 39:
        orc_attn_dq(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), HI32(ins.out[0]),
                    LO32(ins.out[0]), HI32(ins.out[1]), LO32(ins.out[1]));
        break;
      case 40:
        orc_attn_dk(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), HI32(ins.out[0]),
                    LO32(ins.out[0]), HI32(ins.out[1]), LO32(ins.out[1]));
        break;
      case 41:
        orc_embed_fwd(IP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), ins.out[0],
                      LO32(ins.out[1]));
        break;
      default: break;
    }
  }
#undef RP
#undef RQ8
#undef WP
#undef IP
}
