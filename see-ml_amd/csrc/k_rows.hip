// k_rows.hip — row-reduction kernels for gfx950: norms, softmaxes, losses.
//
// Reference semantics: runtime/executor/normalization.cc, loss.cc:21-59,
// 74-89, 99-132, optimizer.cc:17-35, attention.cc:94-136 (softmax part) and
// :185-201. Accumulator types follow the reference: the norm statistics,
// loss totals, clip norm, attention denominator and softmax-backward rowsum
// accumulate in double; the loss-side softmax max/sum in f32.
//
// Layout & mapping: one row per TPR threads (TPR = 64, one wavefront, for
// rows up to ~2K; TPR = 256, one workgroup, for wider rows), elements of a
// row strided by TPR so every pass is a coalesced sweep. Reductions are the
// fixed trees of device_common.h; cross-row totals (losses, norms) go
// through a per-row (or per-block) double workspace summed by one
// workgroup in index order — deterministic, no atomics.
#include "device_common.h"
#include "kernels.h"

#include <initializer_list>

namespace seeml_hip {

namespace {

constexpr int kBlock = 256;

template <int TPR>
__device__ __forceinline__ double row_sum_d(double v, double* scratch) {
  if constexpr (TPR == kWave) return wave_sum(v);
  else return block_sum<double, kBlock>(v, scratch);
}
template <int TPR>
__device__ __forceinline__ float row_sum_f(float v, float* scratch) {
  if constexpr (TPR == kWave) return wave_sum(v);
  else return block_sum<float, kBlock>(v, scratch);
}
template <int TPR>
__device__ __forceinline__ float row_max_f(float v, float* scratch) {
  if constexpr (TPR == kWave) return wave_max(v);
  else return block_max<kBlock>(v, scratch);
}

// Sum of n doubles in index-strided order, one workgroup; out = total/div.
__global__ __launch_bounds__(kBlock) void finish_mean_kernel(const double* __restrict__ terms,
                                                             size_t n, double div,
                                                             float* __restrict__ out) {
  __shared__ double scratch[kBlock / kWave];
  double acc = 0.0;
  for (size_t i = threadIdx.x; i < n; i += kBlock) acc += terms[i];
  const double total = block_sum<double, kBlock>(acc, scratch);
  if (threadIdx.x == 0) *out = static_cast<float>(total / div);
}

// ---- MSE / ClipNorm partials ------------------------------------------------

size_t PartialBlocks(size_t n) {
  size_t g = (n + 16383) / 16384;
  if (g < 1) g = 1;
  if (g > 2048) g = 2048;
  return g;
}

// Block b owns the contiguous range [b*chunk, (b+1)*chunk): a shape-only
// decomposition, like ParallelFor's. Each thread sums its elements in index
// order (DIFF: (a - b)^2, else a^2, in double); the block's threads are
// then reduced in a fixed tree. VEC (16-byte operands, chunk % 4 == 0):
// the thread's elements are whole float4 runs, four runs of each operand in
// flight per step, and only the last block can have a scalar tail.
template <bool VEC, bool DIFF>
__global__ __launch_bounds__(kBlock) void sq_diff_partials(const float* __restrict__ a,
                                                           const float* __restrict__ b,
                                                           size_t n, size_t chunk,
                                                           double* __restrict__ out) {
  __shared__ double scratch[kBlock / kWave];
  const size_t begin = static_cast<size_t>(blockIdx.x) * chunk;
  const size_t end = begin + chunk < n ? begin + chunk : n;
  auto term = [&](float x, float y) {
    const double d = DIFF ? static_cast<double>(x) - static_cast<double>(y) : static_cast<double>(x);
    return d * d;
  };
  double acc = 0.0;
  size_t tail = begin + threadIdx.x;
  if constexpr (VEC) {
    const float4* a4 = reinterpret_cast<const float4*>(a);
    const float4* b4 = reinterpret_cast<const float4*>(b);
    const size_t v1 = end / 4;
    size_t i = begin / 4 + threadIdx.x;
    for (; i + 3 * kBlock < v1; i += 4 * kBlock) {
      float4 x[4], y[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        x[u] = a4[i + u * kBlock];
        if constexpr (DIFF) y[u] = b4[i + u * kBlock];
        else y[u] = x[u];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        acc += term(x[u].x, y[u].x);
        acc += term(x[u].y, y[u].y);
        acc += term(x[u].z, y[u].z);
        acc += term(x[u].w, y[u].w);
      }
    }
    for (; i < v1; i += kBlock) {
      const float4 x = a4[i];
      const float4 y = DIFF ? b4[i] : x;
      acc += term(x.x, y.x);
      acc += term(x.y, y.y);
      acc += term(x.z, y.z);
      acc += term(x.w, y.w);
    }
    tail = 4 * v1 + threadIdx.x;
  }
  for (size_t k = tail; k < end; k += kBlock) acc += term(a[k], DIFF ? b[k] : 0.0f);
  const double t = block_sum<double, kBlock>(acc, scratch);
  if (threadIdx.x == 0) out[blockIdx.x] = t;
}

// The partials' geometry: at most PartialBlocks(n) blocks; with VEC the
// chunk is rounded up to whole float4s (fewer blocks, never more).
struct PartialGeo {
  size_t blocks, chunk;
  bool vec;
};

PartialGeo MakePartialGeo(size_t n, const float* a, const float* b) {
  const size_t g = PartialBlocks(n);
  size_t chunk = (n + g - 1) / g;
  const bool vec = aligned16(a) && (!b || aligned16(b));
  if (vec) chunk = (chunk + 3) / 4 * 4;
  return {(n + chunk - 1) / chunk, chunk, vec};
}

void LaunchSqPartials(const PartialGeo& pg, const float* a, const float* b, size_t n,
                      double* partials, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(pg.blocks));
  if (pg.vec && b)
    hipLaunchKernelGGL((sq_diff_partials<true, true>), grid, dim3(kBlock), 0, stream, a, b, n, pg.chunk, partials);
  else if (pg.vec)
    hipLaunchKernelGGL((sq_diff_partials<true, false>), grid, dim3(kBlock), 0, stream, a, b, n, pg.chunk, partials);
  else if (b)
    hipLaunchKernelGGL((sq_diff_partials<false, true>), grid, dim3(kBlock), 0, stream, a, b, n, pg.chunk, partials);
  else
    hipLaunchKernelGGL((sq_diff_partials<false, false>), grid, dim3(kBlock), 0, stream, a, b, n, pg.chunk, partials);
}

// ClipNorm decision + scale on device (optimizer.cc:28-34): sum the
// partials, norm = sqrt(total) in double, scale only if norm > max_norm.
__global__ __launch_bounds__(kBlock) void clip_apply_kernel(float* __restrict__ g, size_t n,
                                                            const double* __restrict__ partials,
                                                            size_t np, float max_norm) {
  __shared__ double scratch[kBlock / kWave];
  double acc = 0.0;
  for (size_t i = threadIdx.x; i < np; i += kBlock) acc += partials[i];
  const double sq = block_sum<double, kBlock>(acc, scratch);
  const double norm = sqrt(sq);
  if (norm <= static_cast<double>(max_norm) || norm == 0.0) return;
  const float s = static_cast<float>(static_cast<double>(max_norm) / norm);
  const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
    g[i] *= s;
}

// ---- softmax cross-entropy forward -------------------------------------------

// One row per TPR threads: f32 max, f32 exp-sum, probs = e * (1/sum); the
// row's -log(max(p_label, 1e-12)) term in double goes to terms[row]. NaN in
// the row propagates (fmax scrubs NaN from the max, but exp(NaN) does not).
template <int TPR>
__global__ __launch_bounds__(kBlock) void xent_fwd_rows(const float* __restrict__ logits,
                                                        const int32_t* __restrict__ labels,
                                                        float* __restrict__ probs, size_t N,
                                                        size_t C, double* __restrict__ terms) {
  __shared__ float fscratch[kBlock / kWave];
  constexpr int kRows = kBlock / TPR;
  const int t = threadIdx.x % TPR;
  const size_t n = static_cast<size_t>(blockIdx.x) * kRows + threadIdx.x / TPR;
  if (n >= N) return;  // block-uniform when TPR == kBlock
  const float* x = logits + n * C;
  float* p = probs + n * C;
  float mx = x[0];
  for (size_t c = t; c < C; c += TPR) mx = fmaxf(mx, x[c]);
  mx = row_max_f<TPR>(mx, fscratch);
  float s = 0.0f;
  for (size_t c = t; c < C; c += TPR) {
    const float e = expf(x[c] - mx);
    p[c] = e;
    s += e;
  }
  const float sum = row_sum_f<TPR>(s, fscratch);
  const float inv = 1.0f / sum;
  for (size_t c = t; c < C; c += TPR) p[c] = p[c] * inv;
  if (t == 0) {
    const int32_t lab = labels[n];
    double term;
    if (lab < 0 || static_cast<size_t>(lab) >= C) {
      term = __builtin_nan("");  // outside the feeder contract: poison the loss
    } else {
      const float pl = expf(x[lab] - mx) * inv;  // same expression as p[lab]
      const double safe = isnan(pl) ? static_cast<double>(pl)
                                    : static_cast<double>(fmaxf(pl, 1e-12f));
      term = -log(safe);
    }
    terms[n] = term;
  }
}

// Register-resident form for 16-byte aligned rows with C % 4 == 0 and
// C <= NT * 4 * kXentVec: one workgroup per row holds the row in registers
// (thread t owns float4s t, t + NT, ...), so logits are read once and probs
// written once. Same expressions as xent_fwd_rows: f32 max, f32 exp-sum
// (per-thread partials in index order, then the fixed block tree), probs =
// e * (1/sum), the label term from the same expression as p[label].
constexpr int kXentVec = 8;

// BWD: the backward in the same pass (SoftmaxXEntFwdBwd): with the row's
// probabilities still in registers, dl = scale * p, and at the label
// scale * p - scale, scale = seed / N (the backward kernel's expressions on
// the same p values); probs stored only when store_p; block 0 also writes
// the seed to its slot, as the Fill between the two would. dl may be the
// logits themselves (the plans compute it in place): a row's workgroup has
// consumed all of the row's loads before its first barrier, and the label's
// logit is taken from the registers of the thread holding it, so no load
// can follow a store of the row.
template <int NT, bool BWD = false>
__global__ __launch_bounds__(NT) void xent_fwd_rows_reg(const float* logits,
                                                        const int32_t* __restrict__ labels,
                                                        float* probs, size_t N,
                                                        size_t C, double* __restrict__ terms,
                                                        int nt, float* dl = nullptr,
                                                        float seed = 0.0f, float* seed_slot = nullptr,
                                                        int store_p = 1) {
  __shared__ float fscratch[NT / kWave];
  const size_t n = blockIdx.x;
  const int nv = static_cast<int>(C / 4);
  const int t = threadIdx.x;
  // Every load first, unconditionally from float4s clamped into the row, so
  // they are in flight together (loaded under a per-position test and used
  // at once, each was followed by a full wait); then the max in the same
  // order as before. Thread 0 also fetches the label's logit up front.
  float4 v[kXentVec];
#pragma unroll
  for (int i = 0; i < kXentVec; ++i)
    v[i] = ld4(logits + n * C + 4 * static_cast<size_t>(min(t + i * NT, nv - 1)), nt);
  int32_t lab = 0;
  float xl = 0.0f;
  bool own = false;  // BWD: this thread holds the label's logit in v
  if constexpr (BWD) {
    lab = labels[n];
    if (lab >= 0 && static_cast<size_t>(lab) < C) {
#pragma unroll
      for (int i = 0; i < kXentVec; ++i)
        if (t + i * NT == lab / 4) {
          own = true;
          const int e = lab % 4;
          xl = e == 0 ? v[i].x : e == 1 ? v[i].y : e == 2 ? v[i].z : v[i].w;
        }
    }
  } else if (t == 0) {
    lab = labels[n];
    if (lab >= 0 && static_cast<size_t>(lab) < C) xl = logits[n * C + lab];
  }
  float mx = logits[n * C];
#pragma unroll
  for (int i = 0; i < kXentVec; ++i)
    if (t + i * NT < nv) mx = fmaxf(fmaxf(fmaxf(fmaxf(mx, v[i].x), v[i].y), v[i].z), v[i].w);
  mx = block_max<NT>(mx, fscratch);
  float sacc = 0.0f;
#pragma unroll
  for (int i = 0; i < kXentVec; ++i) {
    const int j = t + i * NT;
    if (j < nv) {
      v[i].x = expf(v[i].x - mx);
      v[i].y = expf(v[i].y - mx);
      v[i].z = expf(v[i].z - mx);
      v[i].w = expf(v[i].w - mx);
      sacc += v[i].x;
      sacc += v[i].y;
      sacc += v[i].z;
      sacc += v[i].w;
    }
  }
  const float sum = block_sum<float, NT>(sacc, fscratch);
  const float inv = 1.0f / sum;
  if constexpr (BWD) {
    if (n == 0 && t == 0) *seed_slot = seed;
    const float scale = seed / static_cast<float>(N);
    const size_t lc = lab >= 0 ? static_cast<size_t>(lab) : ~size_t{0};
#pragma unroll
    for (int i = 0; i < kXentVec; ++i) {
      const int j = t + i * NT;
      if (j < nv) {
        const float4 pv = make_float4(v[i].x * inv, v[i].y * inv, v[i].z * inv, v[i].w * inv);
        if (store_p) st4(probs + n * C + 4 * static_cast<size_t>(j), pv, nt);
        float4 o = make_float4(scale * pv.x, scale * pv.y, scale * pv.z, scale * pv.w);
        if (lc / 4 == static_cast<size_t>(j)) {
          if (lc % 4 == 0) o.x -= scale;
          else if (lc % 4 == 1) o.y -= scale;
          else if (lc % 4 == 2) o.z -= scale;
          else o.w -= scale;
        }
        st4(dl + n * C + 4 * static_cast<size_t>(j), o, nt);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < kXentVec; ++i) {
      const int j = t + i * NT;
      if (j < nv)
        st4(probs + n * C + 4 * static_cast<size_t>(j),
            make_float4(v[i].x * inv, v[i].y * inv, v[i].z * inv, v[i].w * inv), nt);
    }
  }
  const bool in_range = lab >= 0 && static_cast<size_t>(lab) < C;
  if (BWD ? (own || (t == 0 && !in_range)) : t == 0) {
    double term;
    if (!in_range) {
      term = __builtin_nan("");  // outside the feeder contract: poison the loss
    } else {
      const float pl = expf(xl - mx) * inv;  // same expression as p[lab]
      const double safe = isnan(pl) ? static_cast<double>(pl)
                                    : static_cast<double>(fmaxf(pl, 1e-12f));
      term = -log(safe);
    }
    terms[n] = term;
  }
}

// ---- KL distillation forward ----------------------------------------------------

template <int TPR>
__device__ void row_softmax_T(const float* __restrict__ x, float* __restrict__ p, size_t C,
                              float inv_T, int t, float* scratch) {
  float mx = x[0] * inv_T;
  for (size_t c = t; c < C; c += TPR) mx = fmaxf(mx, x[c] * inv_T);
  mx = row_max_f<TPR>(mx, scratch);
  float s = 0.0f;
  for (size_t c = t; c < C; c += TPR) {
    const float e = expf(x[c] * inv_T - mx);
    p[c] = e;
    s += e;
  }
  const float inv = 1.0f / row_sum_f<TPR>(s, scratch);
  for (size_t c = t; c < C; c += TPR) p[c] = p[c] * inv;
}

template <int TPR>
__global__ __launch_bounds__(kBlock) void kl_fwd_rows(const float* __restrict__ s_logits,
                                                      const float* __restrict__ t_logits,
                                                      float* __restrict__ ps,
                                                      float* __restrict__ pt, size_t N, size_t C,
                                                      float inv_T, double* __restrict__ terms) {
  __shared__ float fscratch[kBlock / kWave];
  __shared__ double dscratch[kBlock / kWave];
  constexpr int kRows = kBlock / TPR;
  const int t = threadIdx.x % TPR;
  const size_t n = static_cast<size_t>(blockIdx.x) * kRows + threadIdx.x / TPR;
  if (n >= N) return;
  float* prs = ps + n * C;
  float* prt = pt + n * C;
  row_softmax_T<TPR>(s_logits + n * C, prs, C, inv_T, t, fscratch);
  row_softmax_T<TPR>(t_logits + n * C, prt, C, inv_T, t, fscratch);
  double acc = 0.0;
  for (size_t c = t; c < C; c += TPR) {
    const float q = prt[c];
    if (q <= 0.0f) continue;
    const float raw = prs[c];
    const double s = isnan(raw) ? static_cast<double>(raw) : static_cast<double>(fmaxf(raw, 1e-12f));
    acc += static_cast<double>(q) * (log(static_cast<double>(q)) - log(s));
  }
  const double total = row_sum_d<TPR>(acc, dscratch);
  if (t == 0) terms[n] = total;
}

// ---- norms ---------------------------------------------------------------------

template <int TPR>
__global__ __launch_bounds__(kBlock) void layer_norm_fwd_rows(
    const float* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ beta,
    float* __restrict__ y, float* __restrict__ mean, float* __restrict__ rstd, size_t rows,
    size_t cols) {
  __shared__ double dscratch[kBlock / kWave];
  constexpr int kRows = kBlock / TPR;
  const int t = threadIdx.x % TPR;
  const size_t r = static_cast<size_t>(blockIdx.x) * kRows + threadIdx.x / TPR;
  if (r >= rows) return;
  const float* xr = x + r * cols;
  double s = 0.0;
  for (size_t c = t; c < cols; c += TPR) s += static_cast<double>(xr[c]);
  const double sum = row_sum_d<TPR>(s, dscratch);
  const float mu = static_cast<float>(sum / static_cast<double>(cols));
  double v = 0.0;
  for (size_t c = t; c < cols; c += TPR) {
    const double d = static_cast<double>(xr[c]) - static_cast<double>(mu);
    v += d * d;
  }
  const double var = row_sum_d<TPR>(v, dscratch);
  const float rs =
      1.0f / sqrtf(static_cast<float>(var / static_cast<double>(cols)) + 1e-5f);
  if (t == 0) {
    mean[r] = mu;
    rstd[r] = rs;
  }
  float* yr = y + r * cols;
  for (size_t c = t; c < cols; c += TPR) yr[c] = (xr[c] - mu) * rs * gamma[c] + beta[c];
}

template <int TPR>
__global__ __launch_bounds__(kBlock) void layer_norm_bwd_rows(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ mean, const float* __restrict__ rstd, float* __restrict__ dx,
    size_t rows, size_t cols) {
  __shared__ double dscratch[kBlock / kWave];
  constexpr int kRows = kBlock / TPR;
  const int t = threadIdx.x % TPR;
  const size_t r = static_cast<size_t>(blockIdx.x) * kRows + threadIdx.x / TPR;
  if (r >= rows) return;
  const float inv_d = 1.0f / static_cast<float>(cols);
  const float* dyr = dy + r * cols;
  const float* xr = x + r * cols;
  const float mu = mean[r], rs = rstd[r];
  double sg = 0.0, sgx = 0.0;
  for (size_t c = t; c < cols; c += TPR) {
    const float xhat = (xr[c] - mu) * rs;
    const float g = dyr[c] * gamma[c];
    sg += static_cast<double>(g);
    sgx += static_cast<double>(g) * static_cast<double>(xhat);
  }
  const double sum_g = row_sum_d<TPR>(sg, dscratch);
  const double sum_gx = row_sum_d<TPR>(sgx, dscratch);
  const float mg = static_cast<float>(sum_g) * inv_d;
  const float mgx = static_cast<float>(sum_gx) * inv_d;
  float* dxr = dx + r * cols;
  for (size_t c = t; c < cols; c += TPR) {
    const float xhat = (xr[c] - mu) * rs;
    const float g = dyr[c] * gamma[c];
    dxr[c] = rs * (g - mg - xhat * mgx);
  }
}

template <int TPR>
__global__ __launch_bounds__(kBlock) void rms_norm_fwd_rows(const float* __restrict__ x,
                                                            const float* __restrict__ gamma,
                                                            float* __restrict__ y,
                                                            float* __restrict__ rstd, size_t rows,
                                                            size_t cols) {
  __shared__ double dscratch[kBlock / kWave];
  constexpr int kRows = kBlock / TPR;
  const int t = threadIdx.x % TPR;
  const size_t r = static_cast<size_t>(blockIdx.x) * kRows + threadIdx.x / TPR;
  if (r >= rows) return;
  const float* xr = x + r * cols;
  double s = 0.0;
  for (size_t c = t; c < cols; c += TPR) s += static_cast<double>(xr[c]) * static_cast<double>(xr[c]);
  const double ss = row_sum_d<TPR>(s, dscratch);
  const float rs =
      1.0f / sqrtf(static_cast<float>(ss / static_cast<double>(cols)) + 1e-5f);
  if (t == 0) rstd[r] = rs;
  float* yr = y + r * cols;
  for (size_t c = t; c < cols; c += TPR) yr[c] = xr[c] * rs * gamma[c];
}

template <int TPR>
__global__ __launch_bounds__(kBlock) void rms_norm_bwd_rows(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ rstd, float* __restrict__ dx, size_t rows, size_t cols) {
  __shared__ double dscratch[kBlock / kWave];
  constexpr int kRows = kBlock / TPR;
  const int t = threadIdx.x % TPR;
  const size_t r = static_cast<size_t>(blockIdx.x) * kRows + threadIdx.x / TPR;
  if (r >= rows) return;
  const float inv_d = 1.0f / static_cast<float>(cols);
  const float* dyr = dy + r * cols;
  const float* xr = x + r * cols;
  const float rs = rstd[r];
  double s = 0.0;
  for (size_t c = t; c < cols; c += TPR)
    s += static_cast<double>(dyr[c] * gamma[c]) * static_cast<double>(xr[c]);
  const float mgx = static_cast<float>(row_sum_d<TPR>(s, dscratch)) * inv_d;
  float* dxr = dx + r * cols;
  for (size_t c = t; c < cols; c += TPR)
    dxr[c] = rs * (dyr[c] * gamma[c] - xr[c] * rs * rs * mgx);
}

// dS = P * (dP - rowsum(dP * P)), rowsum in double (attention.cc:185-201).
template <int TPR>
__global__ __launch_bounds__(kBlock) void softmax_rows_bwd_kernel(
    const float* __restrict__ p, const float* __restrict__ dp, float* __restrict__ ds,
    size_t rows, size_t cols) {
  __shared__ double dscratch[kBlock / kWave];
  constexpr int kRows = kBlock / TPR;
  const int t = threadIdx.x % TPR;
  const size_t r = static_cast<size_t>(blockIdx.x) * kRows + threadIdx.x / TPR;
  if (r >= rows) return;
  const float* pr = p + r * cols;
  const float* dpr = dp + r * cols;
  double s = 0.0;
  for (size_t c = t; c < cols; c += TPR)
    s += static_cast<double>(dpr[c]) * static_cast<double>(pr[c]);
  const float sum = static_cast<float>(row_sum_d<TPR>(s, dscratch));
  float* dsr = ds + r * cols;
  for (size_t c = t; c < cols; c += TPR) dsr[c] = pr[c] * (dpr[c] - sum);
}

// ---- register-resident rows -------------------------------------------------
//
// For 16-byte aligned rows with cols % 4 == 0 and cols <= TPR * 4 * V: TPR
// threads own one row, thread t holding float4s t, t + TPR, ... (V of them,
// zero past the row's end), so each input row is read from HBM once and each
// output row written once, all as 16-byte accesses. A row reduction's
// per-thread partial runs over the thread's own elements in ascending order
// (zero padding adds exact zeros), then the fixed wave/block tree: the same
// bits on every run. Expressions per element are the strided kernels' above.

template <int TPR, int V>
__device__ __forceinline__ void load_row(const float* __restrict__ row, int nv, int t,
                                         float4 (&v)[V], bool nt) {
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = t + i * TPR;
    v[i] = j < nv ? ld4(row + 4 * j, nt) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
}

template <int TPR, int V>
__device__ __forceinline__ void store_row(float* __restrict__ row, int nv, int t,
                                          const float4 (&v)[V], bool nt) {
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = t + i * TPR;
    if (j < nv) st4(row + 4 * j, v[i], nt);
  }
}

// A per-column parameter (gamma, beta) at this thread's row positions,
// loaded with the row: unconditionally, from indices clamped into the
// vector, so the loads issue back to back and their latency overlaps the
// row's (under a per-position test each load was followed by a full wait).
// Positions past the row are never used.
template <int TPR, int V>
__device__ __forceinline__ void load_param(const float* __restrict__ p, int nv, int t,
                                           float4 (&v)[V]) {
  const float4* p4 = reinterpret_cast<const float4*>(p);
#pragma unroll
  for (int i = 0; i < V; ++i) v[i] = p4[min(t + i * TPR, nv - 1)];
}

// Row index and lane of this thread; false past the last row (uniform per
// row group, and per block when TPR == kBlock).
template <int TPR>
__device__ __forceinline__ bool row_of(size_t rows, size_t* r, int* t) {
  *t = static_cast<int>(threadIdx.x % TPR);
  *r = static_cast<size_t>(blockIdx.x) * (kBlock / TPR) + threadIdx.x / TPR;
  return *r < rows;
}

__device__ __forceinline__ double sq4(float4 a) {
  double s = static_cast<double>(a.x) * static_cast<double>(a.x);
  s += static_cast<double>(a.y) * static_cast<double>(a.y);
  s += static_cast<double>(a.z) * static_cast<double>(a.z);
  s += static_cast<double>(a.w) * static_cast<double>(a.w);
  return s;
}

// y of one register-resident RmsNormFwd row (normalization.cc:75-95): xv
// holds x on entry and y on return; returns rstd.
template <int TPR, int V>
__device__ __forceinline__ float rms_fwd_math(float4 (&xv)[V], const float4 (&gm)[V], int nv,
                                              int t, int cols, double* dscratch) {
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < V; ++i) s += sq4(xv[i]);
  const double ss = row_sum_d<TPR>(s, dscratch);
  const float rs = 1.0f / sqrtf(static_cast<float>(ss / static_cast<double>(cols)) + 1e-5f);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = t + i * TPR;
    if (j < nv) {
      const float4 g = gm[i];
      xv[i] = make_float4(xv[i].x * rs * g.x, xv[i].y * rs * g.y, xv[i].z * rs * g.z,
                          xv[i].w * rs * g.w);
    }
  }
  return rs;
}

template <int TPR, int V>
__global__ __launch_bounds__(kBlock) void rms_norm_fwd_reg(const float* __restrict__ x,
                                                           const float* __restrict__ gamma,
                                                           float* __restrict__ y,
                                                           float* __restrict__ rstd, size_t rows,
                                                           int cols, int nt) {
  __shared__ double dscratch[kBlock / kWave];
  size_t r;
  int t;
  if (!row_of<TPR>(rows, &r, &t)) return;
  const int nv = cols / 4;
  float4 gm[V], xv[V];
  load_param<TPR, V>(gamma, nv, t, gm);
  load_row<TPR, V>(x + r * cols, nv, t, xv, nt);
  const float rs = rms_fwd_math<TPR, V>(xv, gm, nv, t, cols, dscratch);
  if (t == 0) rstd[r] = rs;
  store_row<TPR, V>(y + r * cols, nv, t, xv, nt);
}

// The preceding AddEW's sum x = a + b, formed from the two rows as the AddEW
// forms it (its operand order), and stored when a later reader needs it.
template <int TPR, int V>
__device__ __forceinline__ void load_sum(const float* a, const float* b, float* sum, int nv, int t,
                                         int nt, int store_sum, float4 (&xv)[V]) {
  float4 bv[V];
  load_row<TPR, V>(a, nv, t, xv, nt);
  load_row<TPR, V>(b, nv, t, bv, nt);
#pragma unroll
  for (int i = 0; i < V; ++i)
    xv[i] = make_float4(xv[i].x + bv[i].x, xv[i].y + bv[i].y, xv[i].z + bv[i].z, xv[i].w + bv[i].w);
  if (store_sum) store_row<TPR, V>(sum, nv, t, xv, nt);
}

// RmsNormFwd of the preceding AddEW's output, that AddEW in its prologue. The
// row operands (a, b, sum, y) may be the same range as one another: every
// thread reads its float4 positions of a row before it writes any, and
// writes only those positions, so they carry no __restrict__.
template <int TPR, int V>
__global__ __launch_bounds__(kBlock) void rms_norm_fwd_add_reg(
    const float* a, const float* b, float* sum, const float* __restrict__ gamma, float* y,
    float* __restrict__ rstd, size_t rows, int cols, int nt, int store_sum) {
  __shared__ double dscratch[kBlock / kWave];
  size_t r;
  int t;
  if (!row_of<TPR>(rows, &r, &t)) return;
  const int nv = cols / 4;
  float4 gm[V], xv[V];
  load_param<TPR, V>(gamma, nv, t, gm);
  load_sum<TPR, V>(a + r * cols, b + r * cols, sum + r * cols, nv, t, nt, store_sum, xv);
  const float rs = rms_fwd_math<TPR, V>(xv, gm, nv, t, cols, dscratch);
  if (t == 0) rstd[r] = rs;
  store_row<TPR, V>(y + r * cols, nv, t, xv, nt);
}

// dx of one register-resident RmsNormBwd row (normalization.cc:97-113): gv
// holds dy on entry and dx on return.
template <int TPR, int V>
__device__ __forceinline__ void rms_bwd_math(float4 (&gv)[V], const float4 (&xv)[V],
                                             const float4 (&gm)[V], float rs, int nv, int t,
                                             int cols, double* dscratch) {
  const float inv_d = 1.0f / static_cast<float>(cols);
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = t + i * TPR;
    const float4 g = j < nv ? gm[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    gv[i] = make_float4(gv[i].x * g.x, gv[i].y * g.y, gv[i].z * g.z, gv[i].w * g.w);
    s += static_cast<double>(gv[i].x) * static_cast<double>(xv[i].x);
    s += static_cast<double>(gv[i].y) * static_cast<double>(xv[i].y);
    s += static_cast<double>(gv[i].z) * static_cast<double>(xv[i].z);
    s += static_cast<double>(gv[i].w) * static_cast<double>(xv[i].w);
  }
  const float mgx = static_cast<float>(row_sum_d<TPR>(s, dscratch)) * inv_d;
#pragma unroll
  for (int i = 0; i < V; ++i)
    gv[i] = make_float4(rs * (gv[i].x - xv[i].x * rs * rs * mgx),
                        rs * (gv[i].y - xv[i].y * rs * rs * mgx),
                        rs * (gv[i].z - xv[i].z * rs * rs * mgx),
                        rs * (gv[i].w - xv[i].w * rs * rs * mgx));
}

template <int TPR, int V>
__global__ __launch_bounds__(kBlock) void rms_norm_bwd_reg(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ rstd, float* __restrict__ dx, size_t rows, int cols, int nt) {
  __shared__ double dscratch[kBlock / kWave];
  size_t r;
  int t;
  if (!row_of<TPR>(rows, &r, &t)) return;
  const int nv = cols / 4;
  const float rs = rstd[r];  // issued with the row's loads
  float4 gm[V], gv[V], xv[V];
  load_param<TPR, V>(gamma, nv, t, gm);
  load_row<TPR, V>(dy + r * cols, nv, t, gv, nt);
  load_row<TPR, V>(x + r * cols, nv, t, xv, nt);
  rms_bwd_math<TPR, V>(gv, xv, gm, rs, nv, t, cols, dscratch);
  store_row<TPR, V>(dx + r * cols, nv, t, gv, nt);
}

// out = addend (+) dx for a following AddEW, in its operand order (IEEE
// addition: the AddEW's bits either way); dx is stored as well when live.
template <int TPR, int V>
__device__ __forceinline__ void store_with_addend(const float4 (&dxv)[V], float4 (&av)[V],
                                                  float* dx, float* out, int nv, int t, int nt,
                                                  int add_first, int store_dx) {
  if (store_dx) store_row<TPR, V>(dx, nv, t, dxv, nt);
#pragma unroll
  for (int i = 0; i < V; ++i)
    av[i] = add_first ? make_float4(av[i].x + dxv[i].x, av[i].y + dxv[i].y, av[i].z + dxv[i].z,
                                    av[i].w + dxv[i].w)
                      : make_float4(dxv[i].x + av[i].x, dxv[i].y + av[i].y, dxv[i].z + av[i].z,
                                    dxv[i].w + av[i].w);
  store_row<TPR, V>(out, nv, t, av, nt);
}

// RmsNormBwd with the AddEW that consumes its dx in the write-back. The row
// operands (dy, x, dx, addend, out) may be the same range as one another:
// every thread reads its float4 positions of a row before it writes any,
// and writes only those positions, so they carry no __restrict__.
template <int TPR, int V>
__global__ __launch_bounds__(kBlock) void rms_norm_bwd_add_reg(
    const float* dy, const float* x, const float* __restrict__ gamma,
    const float* __restrict__ rstd, float* dx, const float* addend, float* out, size_t rows,
    int cols, int nt, int add_first, int store_dx) {
  __shared__ double dscratch[kBlock / kWave];
  size_t r;
  int t;
  if (!row_of<TPR>(rows, &r, &t)) return;
  const int nv = cols / 4;
  const float rs = rstd[r];
  float4 gm[V], gv[V], xv[V], av[V];
  load_param<TPR, V>(gamma, nv, t, gm);
  load_row<TPR, V>(dy + r * cols, nv, t, gv, nt);
  load_row<TPR, V>(x + r * cols, nv, t, xv, nt);
  load_row<TPR, V>(addend + r * cols, nv, t, av, nt);
  rms_bwd_math<TPR, V>(gv, xv, gm, rs, nv, t, cols, dscratch);
  store_with_addend<TPR, V>(gv, av, dx + r * cols, out + r * cols, nv, t, nt, add_first, store_dx);
}

// y of one register-resident LayerNormFwd row (normalization.cc:17-43): xv
// holds x on entry and y on return; returns (mean, rstd).
template <int TPR, int V>
__device__ __forceinline__ float2 ln_fwd_math(float4 (&xv)[V], const float4 (&gm)[V],
                                              const float4 (&bm)[V], int nv, int t, int cols,
                                              double* dscratch) {
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    s += static_cast<double>(xv[i].x);
    s += static_cast<double>(xv[i].y);
    s += static_cast<double>(xv[i].z);
    s += static_cast<double>(xv[i].w);
  }
  const double sum = row_sum_d<TPR>(s, dscratch);
  const float mu = static_cast<float>(sum / static_cast<double>(cols));
  const double dmu = static_cast<double>(mu);
  double v = 0.0;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    if (t + i * TPR < nv) {
      const double d0 = static_cast<double>(xv[i].x) - dmu, d1 = static_cast<double>(xv[i].y) - dmu;
      const double d2 = static_cast<double>(xv[i].z) - dmu, d3 = static_cast<double>(xv[i].w) - dmu;
      v += d0 * d0;
      v += d1 * d1;
      v += d2 * d2;
      v += d3 * d3;
    }
  }
  const double var = row_sum_d<TPR>(v, dscratch);
  const float rs = 1.0f / sqrtf(static_cast<float>(var / static_cast<double>(cols)) + 1e-5f);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = t + i * TPR;
    if (j < nv) {
      const float4 g = gm[i], b = bm[i];
      xv[i] = make_float4((xv[i].x - mu) * rs * g.x + b.x, (xv[i].y - mu) * rs * g.y + b.y,
                          (xv[i].z - mu) * rs * g.z + b.z, (xv[i].w - mu) * rs * g.w + b.w);
    }
  }
  return make_float2(mu, rs);
}

template <int TPR, int V>
__global__ __launch_bounds__(kBlock) void layer_norm_fwd_reg(
    const float* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ beta,
    float* __restrict__ y, float* __restrict__ mean, float* __restrict__ rstd, size_t rows,
    int cols, int nt) {
  __shared__ double dscratch[kBlock / kWave];
  size_t r;
  int t;
  if (!row_of<TPR>(rows, &r, &t)) return;
  const int nv = cols / 4;
  float4 gm[V], bm[V], xv[V];
  load_param<TPR, V>(gamma, nv, t, gm);
  load_param<TPR, V>(beta, nv, t, bm);
  load_row<TPR, V>(x + r * cols, nv, t, xv, nt);
  const float2 st = ln_fwd_math<TPR, V>(xv, gm, bm, nv, t, cols, dscratch);
  if (t == 0) {
    mean[r] = st.x;
    rstd[r] = st.y;
  }
  store_row<TPR, V>(y + r * cols, nv, t, xv, nt);
}

// LayerNormFwd of the preceding AddEW's output, that AddEW in its prologue
// (as rms_norm_fwd_add_reg).
template <int TPR, int V>
__global__ __launch_bounds__(kBlock) void layer_norm_fwd_add_reg(
    const float* a, const float* b, float* sum, const float* __restrict__ gamma,
    const float* __restrict__ beta, float* y, float* __restrict__ mean, float* __restrict__ rstd,
    size_t rows, int cols, int nt, int store_sum) {
  __shared__ double dscratch[kBlock / kWave];
  size_t r;
  int t;
  if (!row_of<TPR>(rows, &r, &t)) return;
  const int nv = cols / 4;
  float4 gm[V], bm[V], xv[V];
  load_param<TPR, V>(gamma, nv, t, gm);
  load_param<TPR, V>(beta, nv, t, bm);
  load_sum<TPR, V>(a + r * cols, b + r * cols, sum + r * cols, nv, t, nt, store_sum, xv);
  const float2 st = ln_fwd_math<TPR, V>(xv, gm, bm, nv, t, cols, dscratch);
  if (t == 0) {
    mean[r] = st.x;
    rstd[r] = st.y;
  }
  store_row<TPR, V>(y + r * cols, nv, t, xv, nt);
}

// dx of one register-resident LayerNormBwd row (normalization.cc:45-73): gv
// holds dy on entry and dx on return; xv is overwritten with x-hat.
template <int TPR, int V>
__device__ __forceinline__ void ln_bwd_math(float4 (&gv)[V], float4 (&xv)[V],
                                            const float4 (&gm)[V], float mu, float rs, int nv,
                                            int t, int cols, double* dscratch) {
  const float inv_d = 1.0f / static_cast<float>(cols);
  double sg = 0.0, sgx = 0.0;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int j = t + i * TPR;
    if (j < nv) {
      const float4 g = gm[i];
      // xv becomes x-hat, gv becomes g = dy * gamma.
      xv[i] = make_float4((xv[i].x - mu) * rs, (xv[i].y - mu) * rs, (xv[i].z - mu) * rs,
                          (xv[i].w - mu) * rs);
      gv[i] = make_float4(gv[i].x * g.x, gv[i].y * g.y, gv[i].z * g.z, gv[i].w * g.w);
      sg += static_cast<double>(gv[i].x);
      sgx += static_cast<double>(gv[i].x) * static_cast<double>(xv[i].x);
      sg += static_cast<double>(gv[i].y);
      sgx += static_cast<double>(gv[i].y) * static_cast<double>(xv[i].y);
      sg += static_cast<double>(gv[i].z);
      sgx += static_cast<double>(gv[i].z) * static_cast<double>(xv[i].z);
      sg += static_cast<double>(gv[i].w);
      sgx += static_cast<double>(gv[i].w) * static_cast<double>(xv[i].w);
    }
  }
  const double sum_g = row_sum_d<TPR>(sg, dscratch);
  const double sum_gx = row_sum_d<TPR>(sgx, dscratch);
  const float mg = static_cast<float>(sum_g) * inv_d;
  const float mgx = static_cast<float>(sum_gx) * inv_d;
#pragma unroll
  for (int i = 0; i < V; ++i)
    gv[i] = make_float4(rs * (gv[i].x - mg - xv[i].x * mgx), rs * (gv[i].y - mg - xv[i].y * mgx),
                        rs * (gv[i].z - mg - xv[i].z * mgx), rs * (gv[i].w - mg - xv[i].w * mgx));
}

template <int TPR, int V>
__global__ __launch_bounds__(kBlock) void layer_norm_bwd_reg(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ mean, const float* __restrict__ rstd, float* __restrict__ dx,
    size_t rows, int cols, int nt) {
  __shared__ double dscratch[kBlock / kWave];
  size_t r;
  int t;
  if (!row_of<TPR>(rows, &r, &t)) return;
  const int nv = cols / 4;
  const float mu = mean[r], rs = rstd[r];
  float4 gm[V], gv[V], xv[V];
  load_param<TPR, V>(gamma, nv, t, gm);
  load_row<TPR, V>(dy + r * cols, nv, t, gv, nt);
  load_row<TPR, V>(x + r * cols, nv, t, xv, nt);
  ln_bwd_math<TPR, V>(gv, xv, gm, mu, rs, nv, t, cols, dscratch);
  store_row<TPR, V>(dx + r * cols, nv, t, gv, nt);
}

// LayerNormBwd with the AddEW that consumes its dx (as rms_norm_bwd_add_reg).
template <int TPR, int V>
__global__ __launch_bounds__(kBlock) void layer_norm_bwd_add_reg(
    const float* dy, const float* x, const float* __restrict__ gamma,
    const float* __restrict__ mean, const float* __restrict__ rstd, float* dx,
    const float* addend, float* out, size_t rows, int cols, int nt, int add_first, int store_dx) {
  __shared__ double dscratch[kBlock / kWave];
  size_t r;
  int t;
  if (!row_of<TPR>(rows, &r, &t)) return;
  const int nv = cols / 4;
  const float mu = mean[r], rs = rstd[r];
  float4 gm[V], gv[V], xv[V], av[V];
  load_param<TPR, V>(gamma, nv, t, gm);
  load_row<TPR, V>(dy + r * cols, nv, t, gv, nt);
  load_row<TPR, V>(x + r * cols, nv, t, xv, nt);
  load_row<TPR, V>(addend + r * cols, nv, t, av, nt);
  ln_bwd_math<TPR, V>(gv, xv, gm, mu, rs, nv, t, cols, dscratch);
  store_with_addend<TPR, V>(gv, av, dx + r * cols, out + r * cols, nv, t, nt, add_first, store_dx);
}

// causal_s > 0: row r is query i = r % causal_s and the entries j > i of P
// and dP are known exact +0 (see SoftmaxRowsBwd); only the float4s holding
// j <= i are read, the rest of the row is written as (+0) * (0 - sum).
template <int TPR, int V>
__global__ __launch_bounds__(kBlock) void softmax_rows_bwd_reg(const float* __restrict__ p,
                                                               const float* __restrict__ dp,
                                                               float* __restrict__ ds,
                                                               size_t rows, int cols, int nt,
                                                               int causal_s, int tail) {
  __shared__ double dscratch[kBlock / kWave];
  size_t r;
  int t;
  if (!row_of<TPR>(rows, &r, &t)) return;
  const int nv = cols / 4;
  // Float4s that hold any j <= i (the rest are known zeros when causal).
  const int nread = causal_s > 0 ? static_cast<int>(r % causal_s) / 4 + 1 : nv;
  float4 pv[V], dv[V];
  load_row<TPR, V>(p + r * cols, nread, t, pv, nt);
  load_row<TPR, V>(dp + r * cols, nread, t, dv, nt);
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    s += static_cast<double>(dv[i].x) * static_cast<double>(pv[i].x);
    s += static_cast<double>(dv[i].y) * static_cast<double>(pv[i].y);
    s += static_cast<double>(dv[i].z) * static_cast<double>(pv[i].z);
    s += static_cast<double>(dv[i].w) * static_cast<double>(pv[i].w);
  }
  const float sum = static_cast<float>(row_sum_d<TPR>(s, dscratch));
#pragma unroll
  for (int i = 0; i < V; ++i)
    dv[i] = make_float4(pv[i].x * (dv[i].x - sum), pv[i].y * (dv[i].y - sum),
                        pv[i].z * (dv[i].z - sum), pv[i].w * (dv[i].w - sum));
  // Unread float4s were zero-filled, so their entries already equal
  // (+0) * (0 - sum), the value the full read would give. Without `tail`
  // only the float4s read are stored (the caller's readers never look
  // past them).
  store_row<TPR, V>(ds + r * cols, tail ? nv : nread, t, dv, nt);
}

// Causal row softmax in place (attention.cc:106-125): row u = (b, h, i) holds
// raw scaled scores for j <= i and exact zeros beyond (written by the score
// GEMM). f32 max over the prefix, e = exp(s - max), denominator in double,
// p = e * (1/(float)denom); masked entries are left at exact 0.
__global__ __launch_bounds__(kBlock) void attn_softmax_rows_kernel(float* __restrict__ p,
                                                                   size_t rows, size_t S) {
  const int t = threadIdx.x % kWave;
  const size_t u = static_cast<size_t>(blockIdx.x) * (kBlock / kWave) + threadIdx.x / kWave;
  if (u >= rows) return;
  const size_t i = u % S;
  float* pr = p + u * S;
  float mx = -__builtin_inff();
  for (size_t j = t; j <= i; j += kWave) {
    const float s = pr[j];
    if (s > mx) mx = s;
  }
  mx = wave_max(mx);
  double den = 0.0;
  for (size_t j = t; j <= i; j += kWave) {
    const float e = expf(pr[j] - mx);
    pr[j] = e;
    den += static_cast<double>(e);
  }
  den = wave_sum(den);
  const float inv = 1.0f / static_cast<float>(den);
  for (size_t j = t; j <= i; j += kWave) pr[j] = pr[j] * inv;
}

// Argmax hit count: a wavefront per row. Each lane keeps the first index
// of its strided maximum (NaN skipped, strict '>'); lanes merge by larger
// value, then lower index, which equals the sequential strict-'>' scan
// whenever column 0 is not NaN.
constexpr uint32_t kNoIndex = 0xFFFFFFFFu;

__global__ __launch_bounds__(kBlock) void argmax_correct_kernel(const float* __restrict__ probs,
                                                                const int32_t* __restrict__ labels,
                                                                uint64_t rows, uint32_t cols,
                                                                uint32_t* __restrict__ partials) {
  __shared__ uint32_t hits[kBlock / kWave];
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const uint64_t r = static_cast<uint64_t>(blockIdx.x) * (kBlock / kWave) + w;
  uint32_t hit = 0;
  if (r < rows) {
    const float* row = probs + r * cols;
    float best = 0.0f;
    uint32_t bi = kNoIndex;
    for (uint32_t c = lane; c < cols; c += kWave) {
      const float v = row[c];
      if (v == v && (bi == kNoIndex || v > best)) {
        best = v;
        bi = c;
      }
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
      const float ob = __shfl_xor(best, off, kWave);
      const uint32_t oi = static_cast<uint32_t>(__shfl_xor(static_cast<int>(bi), off, kWave));
      if (oi != kNoIndex && (bi == kNoIndex || ob > best || (ob == best && oi < bi))) {
        best = ob;
        bi = oi;
      }
    }
    const float first = row[0];
    const uint32_t arg = first != first ? 0u : bi;
    const int32_t lab = labels[r];
    hit = (lab >= 0 && static_cast<uint32_t>(lab) == arg) ? 1u : 0u;
  }
  if (lane == 0) hits[w] = hit;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t s = 0;
    for (int i = 0; i < kBlock / kWave; ++i) s += hits[i];
    partials[blockIdx.x] = s;
  }
}

__global__ __launch_bounds__(kBlock) void sum_u32_kernel(const uint32_t* __restrict__ partials,
                                                         uint64_t n, uint64_t* __restrict__ total) {
  __shared__ uint64_t scratch[kBlock / kWave];
  uint64_t acc = 0;
  for (uint64_t i = threadIdx.x; i < n; i += kBlock) acc += partials[i];
  const uint64_t t = block_sum<uint64_t, kBlock>(acc, scratch);
  if (threadIdx.x == 0) *total = t;
}

inline unsigned RowsGrid(size_t rows, int tpr) {
  const size_t per = kBlock / tpr;
  return static_cast<unsigned>((rows + per - 1) / per);
}

}  // namespace

size_t MseFwdWorkspace(size_t n) { return PartialBlocks(n) * sizeof(double); }

Status MseFwd(const float* pred, const float* target, float* loss, size_t n, const Ctx& c) {
  if (n == 0) return Status::Fail(kUnitEngine, "MseFwd: empty input");
  const PartialGeo pg = MakePartialGeo(n, pred, target);
  if (c.ws_bytes < pg.blocks * sizeof(double))
    return Status::Fail(kUnitEngine, "MseFwd: workspace too small");
  double* partials = static_cast<double*>(c.ws);
  LaunchSqPartials(pg, pred, target, n, partials, c.stream);
  hipLaunchKernelGGL(finish_mean_kernel, dim3(1), dim3(kBlock), 0, c.stream, partials, pg.blocks,
                     static_cast<double>(n), loss);
  return LaunchStatus("MseFwd");
}

size_t ClipNormWorkspace(size_t n) { return PartialBlocks(n) * sizeof(double); }

Status ClipNorm(float* g, size_t n, float max_norm, const Ctx& c) {
  if (n == 0) return Status::Ok();
  const PartialGeo pg = MakePartialGeo(n, g, nullptr);
  if (c.ws_bytes < pg.blocks * sizeof(double))
    return Status::Fail(kUnitEngine, "ClipNorm: workspace too small");
  double* partials = static_cast<double*>(c.ws);
  LaunchSqPartials(pg, g, nullptr, n, partials, c.stream);
  hipLaunchKernelGGL(clip_apply_kernel, dim3(grid_for(n, kBlock, 4096)), dim3(kBlock), 0,
                     c.stream, g, n, partials, pg.blocks, max_norm);
  return LaunchStatus("ClipNorm");
}

size_t SoftmaxXEntFwdWorkspace(size_t N) { return N * sizeof(double); }

Status SoftmaxXEntFwd(const float* logits, const int32_t* labels, float* loss, float* probs,
                      size_t N, size_t C, const Ctx& c) {
  if (N == 0 || C == 0) return Status::Fail(kUnitEngine, "SoftmaxXEntFwd: empty input");
  if (c.ws_bytes < N * sizeof(double))
    return Status::Fail(kUnitEngine, "SoftmaxXEntFwd: workspace too small");
  double* terms = static_cast<double*>(c.ws);
  const bool reg = C >= 2048 && C % 4 == 0 && aligned16(logits) && aligned16(probs) &&
                   N <= 0x7FFFFFFF;
  const int nt = StreamPolicy(8 * N * C) ? 1 : 0;
  if (reg && C <= static_cast<size_t>(256 * 4 * kXentVec))
    hipLaunchKernelGGL(xent_fwd_rows_reg<256>, dim3(static_cast<unsigned>(N)), dim3(256), 0,
                       c.stream, logits, labels, probs, N, C, terms, nt);
  else if (reg && C <= static_cast<size_t>(512 * 4 * kXentVec))
    hipLaunchKernelGGL(xent_fwd_rows_reg<512>, dim3(static_cast<unsigned>(N)), dim3(512), 0,
                       c.stream, logits, labels, probs, N, C, terms, nt);
  else if (reg && C <= static_cast<size_t>(1024 * 4 * kXentVec))
    hipLaunchKernelGGL(xent_fwd_rows_reg<1024>, dim3(static_cast<unsigned>(N)), dim3(1024), 0,
                       c.stream, logits, labels, probs, N, C, terms, nt);
  else if (C >= 2048)
    hipLaunchKernelGGL(xent_fwd_rows<kBlock>, dim3(RowsGrid(N, kBlock)), dim3(kBlock), 0,
                       c.stream, logits, labels, probs, N, C, terms);
  else
    hipLaunchKernelGGL(xent_fwd_rows<kWave>, dim3(RowsGrid(N, kWave)), dim3(kBlock), 0, c.stream,
                       logits, labels, probs, N, C, terms);
  hipLaunchKernelGGL(finish_mean_kernel, dim3(1), dim3(kBlock), 0, c.stream, terms, N,
                     static_cast<double>(N), loss);
  return LaunchStatus("SoftmaxXEntFwd");
}

bool XEntFwdBwdFits(const float* logits, const float* probs, const float* dl, size_t N, size_t C) {
  return C >= 2048 && C % 4 == 0 && C <= static_cast<size_t>(1024 * 4 * kXentVec) && aligned16(logits) &&
         (!probs || aligned16(probs)) && aligned16(dl) && N > 0 && N <= 0x7FFFFFFF;
}

Status SoftmaxXEntFwdBwd(const float* logits, const int32_t* labels, float* loss, float* probs,
                         float seed, float* seed_slot, float* dl, size_t N, size_t C, const Ctx& c) {
  if (!XEntFwdBwdFits(logits, probs, dl, N, C) || !seed_slot)
    return Status::Fail(kUnitEngine, "SoftmaxXEntFwdBwd: shape or alignment outside the one-pass form");
  if (c.ws_bytes < N * sizeof(double))
    return Status::Fail(kUnitEngine, "SoftmaxXEntFwdBwd: workspace too small");
  double* terms = static_cast<double*>(c.ws);
  const int nt = StreamPolicy(8 * N * C) ? 1 : 0;
  const int sp = probs ? 1 : 0;
  if (C <= static_cast<size_t>(256 * 4 * kXentVec))
    hipLaunchKernelGGL((xent_fwd_rows_reg<256, true>), dim3(static_cast<unsigned>(N)), dim3(256), 0,
                       c.stream, logits, labels, probs, N, C, terms, nt, dl, seed, seed_slot, sp);
  else if (C <= static_cast<size_t>(512 * 4 * kXentVec))
    hipLaunchKernelGGL((xent_fwd_rows_reg<512, true>), dim3(static_cast<unsigned>(N)), dim3(512), 0,
                       c.stream, logits, labels, probs, N, C, terms, nt, dl, seed, seed_slot, sp);
  else
    hipLaunchKernelGGL((xent_fwd_rows_reg<1024, true>), dim3(static_cast<unsigned>(N)), dim3(1024), 0,
                       c.stream, logits, labels, probs, N, C, terms, nt, dl, seed, seed_slot, sp);
  hipLaunchKernelGGL(finish_mean_kernel, dim3(1), dim3(kBlock), 0, c.stream, terms, N,
                     static_cast<double>(N), loss);
  return LaunchStatus("SoftmaxXEntFwdBwd");
}

size_t KLDistillFwdWorkspace(size_t N) { return N * sizeof(double); }

Status KLDistillFwd(const float* s, const float* t, float* loss, float* p_s, float* p_t, size_t N,
                    size_t C, float T, const Ctx& c) {
  if (N == 0 || C == 0) return Status::Fail(kUnitEngine, "KLDistillFwd: empty input");
  if (c.ws_bytes < N * sizeof(double))
    return Status::Fail(kUnitEngine, "KLDistillFwd: workspace too small");
  double* terms = static_cast<double*>(c.ws);
  const float inv_T = 1.0f / T;
  if (C >= 2048)
    hipLaunchKernelGGL(kl_fwd_rows<kBlock>, dim3(RowsGrid(N, kBlock)), dim3(kBlock), 0, c.stream,
                       s, t, p_s, p_t, N, C, inv_T, terms);
  else
    hipLaunchKernelGGL(kl_fwd_rows<kWave>, dim3(RowsGrid(N, kWave)), dim3(kBlock), 0, c.stream, s,
                       t, p_s, p_t, N, C, inv_T, terms);
  hipLaunchKernelGGL(finish_mean_kernel, dim3(1), dim3(kBlock), 0, c.stream, terms, N,
                     static_cast<double>(N), loss);
  return LaunchStatus("KLDistillFwd");
}

#define ROWS_DISPATCH(kernel, rows, cols, ...)                                                 \
  do {                                                                                         \
    if ((cols) >= 1024)                                                                        \
      hipLaunchKernelGGL(kernel<kBlock>, dim3(RowsGrid(rows, kBlock)), dim3(kBlock), 0,        \
                         c.stream, __VA_ARGS__);                                               \
    else                                                                                       \
      hipLaunchKernelGGL(kernel<kWave>, dim3(RowsGrid(rows, kWave)), dim3(kBlock), 0,          \
                         c.stream, __VA_ARGS__);                                               \
  } while (0)

// Register-resident shape for rows of `cols` floats: case 0..3 = (64, 4),
// (64, 8), (256, 4), (256, 8) threads per row x float4s per thread; -1 when
// the row is too wide, not a whole number of float4s, or not 16-byte aligned.
static int RegCase(size_t cols, std::initializer_list<const void*> rows_base) {
  if (cols == 0 || cols % 4 != 0 || cols > 8192) return -1;
  for (const void* p : rows_base)
    if (p && !aligned16(p)) return -1;
  if (cols <= 1024) return 0;
  if (cols <= 2048) return 1;
  if (cols <= 4096) return 2;
  return 3;
}

#define REG_DISPATCH(kernel, rcase, rows, ...)                                                  \
  do {                                                                                         \
    switch (rcase) {                                                                           \
      case 0:                                                                                  \
        hipLaunchKernelGGL((kernel<kWave, 4>), dim3(RowsGrid(rows, kWave)), dim3(kBlock), 0,   \
                           c.stream, __VA_ARGS__);                                             \
        break;                                                                                 \
      case 1:                                                                                  \
        hipLaunchKernelGGL((kernel<kWave, 8>), dim3(RowsGrid(rows, kWave)), dim3(kBlock), 0,   \
                           c.stream, __VA_ARGS__);                                             \
        break;                                                                                 \
      case 2:                                                                                  \
        hipLaunchKernelGGL((kernel<kBlock, 4>), dim3(RowsGrid(rows, kBlock)), dim3(kBlock), 0, \
                           c.stream, __VA_ARGS__);                                             \
        break;                                                                                 \
      default:                                                                                 \
        hipLaunchKernelGGL((kernel<kBlock, 8>), dim3(RowsGrid(rows, kBlock)), dim3(kBlock), 0, \
                           c.stream, __VA_ARGS__);                                             \
        break;                                                                                 \
    }                                                                                          \
  } while (0)

Status LayerNormFwd(const float* x, const float* gamma, const float* beta, float* y, float* mean,
                    float* rstd, size_t rows, size_t cols, const Ctx& c, const RowPreAdd* pre) {
  if (rows == 0 || cols == 0) return Status::Ok();
  if (pre) {
    const int rc = RegCase(cols, {pre->a, pre->b, pre->sum, gamma, beta, y});
    if (rc < 0) return Status::Fail(kUnitEngine, "AddEW+LayerNormFwd: rows not register-resident");
    REG_DISPATCH(layer_norm_fwd_add_reg, rc, rows, pre->a, pre->b, pre->sum, gamma, beta, y, mean,
                 rstd, rows, static_cast<int>(cols),
                 StreamPolicy((pre->store_sum ? 16 : 12) * rows * cols) ? 1 : 0,
                 pre->store_sum ? 1 : 0);
    return LaunchStatus("AddEW+LayerNormFwd");
  }
  const int rc = RegCase(cols, {x, gamma, beta, y});
  if (rc >= 0)
    REG_DISPATCH(layer_norm_fwd_reg, rc, rows, x, gamma, beta, y, mean, rstd, rows,
                 static_cast<int>(cols), StreamPolicy(8 * rows * cols) ? 1 : 0);
  else
    ROWS_DISPATCH(layer_norm_fwd_rows, rows, cols, x, gamma, beta, y, mean, rstd, rows, cols);
  return LaunchStatus("LayerNormFwd");
}

bool RowAddendForm(size_t cols, std::initializer_list<const void*> rows_base) {
  return RegCase(cols, rows_base) >= 0;
}

Status LayerNormBwd(const float* dy, const float* x, const float* gamma, const float* mean,
                    const float* rstd, float* dx, size_t rows, size_t cols, const Ctx& c,
                    const RowAddend* add) {
  if (rows == 0 || cols == 0) return Status::Ok();
  if (add) {
    const int rc = RegCase(cols, {dy, x, gamma, dx, add->addend, add->out});
    if (rc < 0) return Status::Fail(kUnitEngine, "LayerNormBwd+AddEW: rows not register-resident");
    REG_DISPATCH(layer_norm_bwd_add_reg, rc, rows, dy, x, gamma, mean, rstd, dx, add->addend,
                 add->out, rows, static_cast<int>(cols),
                 StreamPolicy((add->store_dx ? 20 : 16) * rows * cols) ? 1 : 0,
                 add->add_first ? 1 : 0, add->store_dx ? 1 : 0);
    return LaunchStatus("LayerNormBwd+AddEW");
  }
  const int rc = RegCase(cols, {dy, x, gamma, dx});
  if (rc >= 0)
    REG_DISPATCH(layer_norm_bwd_reg, rc, rows, dy, x, gamma, mean, rstd, dx, rows,
                 static_cast<int>(cols), StreamPolicy(12 * rows * cols) ? 1 : 0);
  else
    ROWS_DISPATCH(layer_norm_bwd_rows, rows, cols, dy, x, gamma, mean, rstd, dx, rows, cols);
  return LaunchStatus("LayerNormBwd");
}

Status RmsNormFwd(const float* x, const float* gamma, float* y, float* rstd, size_t rows,
                  size_t cols, const Ctx& c, const RowPreAdd* pre) {
  if (rows == 0 || cols == 0) return Status::Ok();
  if (pre) {
    const int rc = RegCase(cols, {pre->a, pre->b, pre->sum, gamma, y});
    if (rc < 0) return Status::Fail(kUnitEngine, "AddEW+RmsNormFwd: rows not register-resident");
    REG_DISPATCH(rms_norm_fwd_add_reg, rc, rows, pre->a, pre->b, pre->sum, gamma, y, rstd, rows,
                 static_cast<int>(cols), StreamPolicy((pre->store_sum ? 16 : 12) * rows * cols) ? 1 : 0,
                 pre->store_sum ? 1 : 0);
    return LaunchStatus("AddEW+RmsNormFwd");
  }
  const int rc = RegCase(cols, {x, gamma, y});
  if (rc >= 0)
    REG_DISPATCH(rms_norm_fwd_reg, rc, rows, x, gamma, y, rstd, rows, static_cast<int>(cols),
                 StreamPolicy(8 * rows * cols) ? 1 : 0);
  else
    ROWS_DISPATCH(rms_norm_fwd_rows, rows, cols, x, gamma, y, rstd, rows, cols);
  return LaunchStatus("RmsNormFwd");
}

Status RmsNormBwd(const float* dy, const float* x, const float* gamma, const float* rstd,
                  float* dx, size_t rows, size_t cols, const Ctx& c, const RowAddend* add) {
  if (rows == 0 || cols == 0) return Status::Ok();
  if (add) {
    const int rc = RegCase(cols, {dy, x, gamma, dx, add->addend, add->out});
    if (rc < 0) return Status::Fail(kUnitEngine, "RmsNormBwd+AddEW: rows not register-resident");
    REG_DISPATCH(rms_norm_bwd_add_reg, rc, rows, dy, x, gamma, rstd, dx, add->addend, add->out,
                 rows, static_cast<int>(cols),
                 StreamPolicy((add->store_dx ? 20 : 16) * rows * cols) ? 1 : 0,
                 add->add_first ? 1 : 0, add->store_dx ? 1 : 0);
    return LaunchStatus("RmsNormBwd+AddEW");
  }
  const int rc = RegCase(cols, {dy, x, gamma, dx});
  if (rc >= 0)
    REG_DISPATCH(rms_norm_bwd_reg, rc, rows, dy, x, gamma, rstd, dx, rows,
                 static_cast<int>(cols), StreamPolicy(12 * rows * cols) ? 1 : 0);
  else
    ROWS_DISPATCH(rms_norm_bwd_rows, rows, cols, dy, x, gamma, rstd, dx, rows, cols);
  return LaunchStatus("RmsNormBwd");
}

bool SoftmaxRowsBwdCausalForm(const float* probs, const float* dp, const float* ds, size_t cols) {
  return RegCase(cols, {probs, dp, ds}) >= 0;
}

Status SoftmaxRowsBwd(const float* probs, const float* dp, float* ds, size_t rows, size_t cols,
                      const Ctx& c, size_t causal_s, bool tail) {
  if (rows == 0 || cols == 0) return Status::Ok();
  const int rc = RegCase(cols, {probs, dp, ds});
  if (causal_s != 0 && (causal_s != cols || rows % causal_s != 0))
    return Status::Fail(kUnitEngine, "SoftmaxRowsBwd: causal geometry does not match the rows");
  if (rc >= 0) {
    // Traffic: the causal form reads about half of P and dP.
    const size_t traffic = causal_s ? 8 * rows * cols : 12 * rows * cols;
    REG_DISPATCH(softmax_rows_bwd_reg, rc, rows, probs, dp, ds, rows, static_cast<int>(cols),
                 StreamPolicy(traffic) ? 1 : 0, static_cast<int>(causal_s),
                 causal_s == 0 || tail ? 1 : 0);
  } else {
    ROWS_DISPATCH(softmax_rows_bwd_kernel, rows, cols, probs, dp, ds, rows, cols);
  }
  return LaunchStatus("SoftmaxRowsBwd");
}

Status AttnSoftmaxRows(float* p, size_t rows, size_t S, const Ctx& c) {
  if (rows == 0 || S == 0) return Status::Ok();
  hipLaunchKernelGGL(attn_softmax_rows_kernel, dim3(RowsGrid(rows, kWave)), dim3(kBlock), 0,
                     c.stream, p, rows, S);
  return LaunchStatus("AttnFwd(softmax)");
}

size_t ArgmaxPartials(uint64_t rows) { return (rows + kBlock / kWave - 1) / (kBlock / kWave); }

Status ArgmaxCorrect(const float* probs, const int32_t* labels, uint64_t rows, uint64_t cols,
                     uint32_t* partials, uint64_t* total, const Ctx& c) {
  if (cols == 0 || cols >= kNoIndex) return Status::Fail(kUnitEngine, "argmax: bad class count");
  const size_t blocks = ArgmaxPartials(rows);
  if (blocks > 0x7FFFFFFF) return Status::Fail(kUnitEngine, "argmax: too many rows");
  if (blocks)
    hipLaunchKernelGGL(argmax_correct_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0,
                       c.stream, probs, labels, rows, static_cast<uint32_t>(cols), partials);
  hipLaunchKernelGGL(sum_u32_kernel, dim3(1), dim3(kBlock), 0, c.stream, partials,
                     static_cast<uint64_t>(blocks), total);
  return LaunchStatus("argmax");
}

}  // namespace seeml_hip
