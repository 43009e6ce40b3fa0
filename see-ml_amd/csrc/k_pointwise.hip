// k_pointwise.hip — bandwidth-bound elementwise kernels for gfx950.
//
// Reference semantics: runtime/executor/elementwise.cc, activation.cc,
// optimizer.cc:37-69, loss.cc:61-72,91-97,134-140, attention.cc:39-92.
// Layout: flat f32 arrays in the device arena. Each kernel is a grid-stride
// loop over float4 vectors (when every pointer is 16-byte aligned) plus a
// scalar tail, so HBM traffic is fully coalesced 16-byte accesses; the grid
// is capped so one launch keeps every CU busy without oversubscribing.
//
// Bits: with -ffp-contract=off the per-element expressions below round
// exactly where the reference's do, so AddEW/MulEW/Scale/AddBias/ReLU/
// AdamW/SGD/Fill/Copy/Embed/loss-backward results are bit-identical to the
// CPU executor; GELU/SiLU/RoPE go through device expf/tanhf/sinf/cosf and
// match to within a few ulp.
#include "device_common.h"
#include "kernels.h"

#include <math.h>

#include <algorithm>
#include <cmath>

namespace seeml_hip {

namespace {

constexpr int kBlock = 256;
constexpr size_t kGridCap = 8192;

struct AddF { __device__ float operator()(float a, float b) const { return a + b; } };
struct MulF { __device__ float operator()(float a, float b) const { return a * b; } };
struct ScaleF {
  float alpha;
  __device__ float operator()(float x) const { return alpha * x; }
};
struct ReluF { __device__ float operator()(float x) const { return dev_relu(x); } };
struct ReluBwdF { __device__ float operator()(float dy, float x) const { return x > 0.0f ? dy : 0.0f; } };
struct GeluF { __device__ float operator()(float x) const { return dev_gelu(x); } };
struct SiluF { __device__ float operator()(float x) const { return dev_silu(x); } };
struct GeluBwdF {
  __device__ float operator()(float dy, float v) const {
    const float kC = 0.7978845608028654f, kA = 0.044715f;
    const float u = kC * (v + kA * v * v * v);
    const float t = tanhf(u);
    const float one_minus_t2 = 1.0f - t * t;
    // Saturated tanh: the sech^2 factor is an exact zero while u' may
    // overflow; drop the dead term (activation.cc:47-56).
    const float tail = one_minus_t2 == 0.0f
                           ? 0.0f
                           : 0.5f * v * one_minus_t2 * (kC * (1.0f + 3.0f * kA * v * v));
    return dy * (0.5f * (1.0f + t) + tail);
  }
};
struct SiluBwdF {
  __device__ float operator()(float dy, float x) const {
    const float s = dev_sigmoid(x);
    return dy * (s * (1.0f + x * (1.0f - s)));
  }
};
struct FillF {
  float v;
  __device__ float operator()(float) const { return v; }
};
struct CopyF { __device__ float operator()(float x) const { return x; } };

// Each thread handles Unroll(NT) float4s per iteration, all loads issued
// before any store. NT (streams larger than the memory-side cache) selects
// the streaming cache policy and a 4-deep unroll; cache-resident streams run
// one float4 per iteration with the default policy, which measured faster.
constexpr int Unroll(bool nt) { return nt ? 4 : 1; }
constexpr size_t kStreamGridCap = 16384;

template <class F, bool NT>
__global__ __launch_bounds__(kBlock) void ew_unary(const float* __restrict__ x,
                                                   float* __restrict__ out, size_t n, size_t nv,
                                                   F f) {
  constexpr int kUnroll = Unroll(NT);
  const size_t stride = static_cast<size_t>(gridDim.x) * kBlock * kUnroll;
  for (size_t base = static_cast<size_t>(blockIdx.x) * kBlock * kUnroll + threadIdx.x; base < nv;
       base += stride) {
    float4 a[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const size_t i = base + static_cast<size_t>(u) * kBlock;
      if (i < nv) a[u] = ld4(x + 4 * i, NT);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const size_t i = base + static_cast<size_t>(u) * kBlock;
      if (i < nv) st4(out + 4 * i, make_float4(f(a[u].x), f(a[u].y), f(a[u].z), f(a[u].w)), NT);
    }
  }
  const size_t gid = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  const size_t tstride = static_cast<size_t>(gridDim.x) * kBlock;
  for (size_t i = nv * 4 + gid; i < n; i += tstride) out[i] = f(x[i]);
}

template <class F, bool NT>
__global__ __launch_bounds__(kBlock) void ew_binary(const float* __restrict__ x,
                                                    const float* __restrict__ y,
                                                    float* __restrict__ out, size_t n, size_t nv,
                                                    F f) {
  constexpr int kUnroll = Unroll(NT);
  const size_t stride = static_cast<size_t>(gridDim.x) * kBlock * kUnroll;
  for (size_t base = static_cast<size_t>(blockIdx.x) * kBlock * kUnroll + threadIdx.x; base < nv;
       base += stride) {
    float4 a[kUnroll], b[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const size_t i = base + static_cast<size_t>(u) * kBlock;
      if (i < nv) {
        a[u] = ld4(x + 4 * i, NT);
        b[u] = ld4(y + 4 * i, NT);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const size_t i = base + static_cast<size_t>(u) * kBlock;
      if (i < nv)
        st4(out + 4 * i,
            make_float4(f(a[u].x, b[u].x), f(a[u].y, b[u].y), f(a[u].z, b[u].z),
                        f(a[u].w, b[u].w)),
            NT);
    }
  }
  const size_t gid = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  const size_t tstride = static_cast<size_t>(gridDim.x) * kBlock;
  for (size_t i = nv * 4 + gid; i < n; i += tstride) out[i] = f(x[i], y[i]);
}

// ---- pointwise runs (kernels.h PointwiseRun) ------------------------------
struct PwProg {
  int nin, nops;
  PwOp op[kPwOps];
  int a[kPwOps], b[kPwOps];
};
// The programs compiled, one kernel each: the wirings of the instruction
// runs the compiler emits (LoRA scaling, SwiGLU, residual-gradient sums).
constexpr PwProg kPwProgs[] = {
    // SwiGLU forward: s = silu(g); h = s * u
    {2, 2, {PwOp::kSilu, PwOp::kMul}, {0, 4}, {0, 1}},
    // SwiGLU backward: ds = dh * u; du = dh * s; dg = silu'(ds, g)
    {4, 3, {PwOp::kMul, PwOp::kMul, PwOp::kSiluBwd}, {0, 0, 4}, {1, 2, 3}},
    // a gradient sum, then its LoRA-scaled copy
    {2, 2, {PwOp::kAdd, PwOp::kScale}, {0, 4}, {1, 4}},
    // a gradient sum through an activation's backward, then scaled
    {3, 3, {PwOp::kAdd, PwOp::kReluBwd, PwOp::kScale}, {0, 4, 5}, {1, 2, 5}},
    {3, 3, {PwOp::kAdd, PwOp::kGeluBwd, PwOp::kScale}, {0, 4, 5}, {1, 2, 5}},
    // LoRA branch scaled and added (when no skinny GEMM chain absorbed it)
    {2, 2, {PwOp::kScale, PwOp::kAdd}, {0, 1}, {0, 4}},
    // SwiGLU backward over (dh, u, g): du = dh * silu(g) from g, whose
    // SiluFwd output s it would otherwise read (same function, same bits)
    {3, 3, {PwOp::kMul, PwOp::kMulSilu, PwOp::kSiluBwd}, {0, 0, 4}, {1, 2, 2}},
};
static_assert(kPwProgs[kPwSwiGluBwd].op[2] == PwOp::kSiluBwd &&
                  kPwProgs[kPwSwiGluBwdRecompute].op[1] == PwOp::kMulSilu,
              "the SwiGLU backward programs' indices");
constexpr int kNumPwProgs = sizeof(kPwProgs) / sizeof(kPwProgs[0]);

template <PwOp OP>
__device__ __forceinline__ float PwApply(float a, float b, float alpha) {
  if constexpr (OP == PwOp::kAdd) return AddF()(a, b);
  else if constexpr (OP == PwOp::kMul) return MulF()(a, b);
  else if constexpr (OP == PwOp::kScale) return ScaleF{alpha}(a);
  else if constexpr (OP == PwOp::kRelu) return ReluF()(a);
  else if constexpr (OP == PwOp::kReluBwd) return ReluBwdF()(a, b);
  else if constexpr (OP == PwOp::kGelu) return GeluF()(a);
  else if constexpr (OP == PwOp::kGeluBwd) return GeluBwdF()(a, b);
  else if constexpr (OP == PwOp::kSilu) return SiluF()(a);
  else if constexpr (OP == PwOp::kSiluBwd) return SiluBwdF()(a, b);
  else if constexpr (OP == PwOp::kMulSilu) return MulF()(a, SiluF()(b));
  else return a;  // kCopy
}

// Steps J.. of program P on one set of slot values (plain floats: arrays of
// the float4 struct type are placed in scratch memory).
template <int P, int J>
__device__ __forceinline__ void PwSteps(float (&v)[kPwIn + kPwOps][4], const PointwiseRun& r) {
  constexpr PwProg prog = kPwProgs[P];
  if constexpr (J < prog.nops) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      v[kPwIn + J][e] = PwApply<prog.op[J]>(v[prog.a[J]][e], v[prog.b[J]][e], r.alpha[J]);
    PwSteps<P, J + 1>(v, r);
  }
}

template <int P, bool NT>
__global__ __launch_bounds__(kBlock) void pw_run_kernel(PointwiseRun r, size_t nv) {
  constexpr PwProg prog = kPwProgs[P];
  constexpr int kUnroll = Unroll(NT);
  const size_t stride = static_cast<size_t>(gridDim.x) * kBlock * kUnroll;
  for (size_t base = static_cast<size_t>(blockIdx.x) * kBlock * kUnroll + threadIdx.x; base < nv;
       base += stride) {
    float v[kUnroll][kPwIn + kPwOps][4];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const size_t i = base + static_cast<size_t>(u) * kBlock;
#pragma unroll
      for (int k = 0; k < prog.nin; ++k) {
        float4 q = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (i < nv) q = ld4(r.in[k] + 4 * i, NT);
        v[u][k][0] = q.x; v[u][k][1] = q.y; v[u][k][2] = q.z; v[u][k][3] = q.w;
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const size_t i = base + static_cast<size_t>(u) * kBlock;
      if (i >= nv) continue;
      PwSteps<P, 0>(v[u], r);
#pragma unroll
      for (int j = 0; j < prog.nops; ++j)
        if (r.out[j])
          st4(r.out[j] + 4 * i,
              make_float4(v[u][kPwIn + j][0], v[u][kPwIn + j][1], v[u][kPwIn + j][2],
                          v[u][kPwIn + j][3]),
              NT);
    }
  }
  const size_t gid = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  const size_t tstride = static_cast<size_t>(gridDim.x) * kBlock;
  for (size_t i = nv * 4 + gid; i < r.n; i += tstride) {
    float v[kPwIn + kPwOps][4] = {};
#pragma unroll
    for (int k = 0; k < prog.nin; ++k) v[k][0] = r.in[k][i];
    PwSteps<P, 0>(v, r);
#pragma unroll
    for (int j = 0; j < prog.nops; ++j)
      if (r.out[j]) r.out[j][i] = v[kPwIn + j][0];
  }
}

template <int P>
void LaunchPw(const PointwiseRun& r, size_t nv, bool nt, dim3 grid, hipStream_t s) {
  if (nt) hipLaunchKernelGGL((pw_run_kernel<P, true>), grid, dim3(kBlock), 0, s, r, nv);
  else hipLaunchKernelGGL((pw_run_kernel<P, false>), grid, dim3(kBlock), 0, s, r, nv);
}

// Fill writes only: a separate kernel so no read of uninitialised memory.
__global__ __launch_bounds__(kBlock) void fill_kernel(float* __restrict__ out, size_t n, size_t nv,
                                                      float v) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
  const size_t gid = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  float4* o4 = reinterpret_cast<float4*>(out);
  for (size_t i = gid; i < nv; i += stride) o4[i] = make_float4(v, v, v, v);
  for (size_t i = nv * 4 + gid; i < n; i += stride) out[i] = v;
}

template <class F>
Status Unary(const float* x, float* out, size_t n, F f, const Ctx& c, const char* what) {
  if (n == 0) return Status::Ok();
  const size_t nv = (aligned16(x) && aligned16(out)) ? n / 4 : 0;
  const bool nt = StreamPolicy(8 * n);
  const size_t work = nv ? (nv + Unroll(nt) - 1) / Unroll(nt) : n;
  const dim3 grid(grid_for(work, kBlock, nt ? kStreamGridCap : kGridCap));
  if (nt)
    hipLaunchKernelGGL((ew_unary<F, true>), grid, dim3(kBlock), 0, c.stream, x, out, n, nv, f);
  else
    hipLaunchKernelGGL((ew_unary<F, false>), grid, dim3(kBlock), 0, c.stream, x, out, n, nv, f);
  return LaunchStatus(what);
}

template <class F>
Status Binary(const float* x, const float* y, float* out, size_t n, F f, const Ctx& c,
              const char* what) {
  if (n == 0) return Status::Ok();
  const size_t nv = (aligned16(x) && aligned16(y) && aligned16(out)) ? n / 4 : 0;
  const bool nt = StreamPolicy(12 * n);
  const size_t work = nv ? (nv + Unroll(nt) - 1) / Unroll(nt) : n;
  const dim3 grid(grid_for(work, kBlock, nt ? kStreamGridCap : kGridCap));
  if (nt)
    hipLaunchKernelGGL((ew_binary<F, true>), grid, dim3(kBlock), 0, c.stream, x, y, out, n, nv, f);
  else
    hipLaunchKernelGGL((ew_binary<F, false>), grid, dim3(kBlock), 0, c.stream, x, y, out, n, nv,
                       f);
  return LaunchStatus(what);
}

// out[r, c] = x[r, c] + b[c]  (elementwise.cc:28-36)
__global__ __launch_bounds__(kBlock) void add_bias_kernel(const float* __restrict__ x,
                                                          const float* __restrict__ b,
                                                          float* __restrict__ out, size_t n,
                                                          size_t cols, int vec) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
  const size_t gid = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (vec) {
    const size_t nv = n / 4, cv = cols / 4;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const float4* b4 = reinterpret_cast<const float4*>(b);
    float4* o4 = reinterpret_cast<float4*>(out);
    for (size_t i = gid; i < nv; i += stride) {
      const float4 a = x4[i], bb = b4[i % cv];
      o4[i] = make_float4(a.x + bb.x, a.y + bb.y, a.z + bb.z, a.w + bb.w);
    }
  } else {
    for (size_t i = gid; i < n; i += stride) out[i] = x[i] + b[i % cols];
  }
}

// Row gather out[t, :] = table[tokens[t], :] (elementwise.cc:44-53). A token
// outside [0, vocab) — which the feeder contract excludes — yields a NaN row
// instead of an out-of-bounds read, so the step's finite-loss guard trips.
__global__ __launch_bounds__(kBlock) void embed_kernel(const int32_t* __restrict__ tokens,
                                                       const float* __restrict__ table,
                                                       float* __restrict__ out, size_t rows,
                                                       size_t dim, size_t vocab, int vec) {
  const int lane = threadIdx.x % kWave;
  const size_t row0 = (static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x) / kWave;
  const size_t rstride = static_cast<size_t>(gridDim.x) * (kBlock / kWave);
  for (size_t r = row0; r < rows; r += rstride) {
    const int32_t t = tokens[r];
    float* dst = out + r * dim;
    if (t < 0 || static_cast<size_t>(t) >= vocab) {
      for (size_t c = lane; c < dim; c += kWave) dst[c] = __builtin_nanf("");
      continue;
    }
    const float* src = table + static_cast<size_t>(t) * dim;
    if (vec) {
      const float4* s4 = reinterpret_cast<const float4*>(src);
      float4* d4 = reinterpret_cast<float4*>(dst);
      for (size_t c = lane; c < dim / 4; c += kWave) d4[c] = s4[c];
    } else {
      for (size_t c = lane; c < dim; c += kWave) dst[c] = src[c];
    }
  }
}

// db[c] = sum_r dy[r, c], rows in order per column (elementwise.cc:55-67):
// one thread owns a column, so the f32 sum order — and the bits — are the
// reference's.
__global__ __launch_bounds__(kBlock) void reduce_rows_kernel(const float* __restrict__ dy,
                                                             float* __restrict__ db, size_t rows,
                                                             size_t cols) {
  const size_t c = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (c >= cols) return;
  float acc = 0.0f;
  for (size_t r = 0; r < rows; ++r) acc += dy[r * cols + c];
  db[c] = acc;
}

// dlogits = (seed/N) * probs, minus seed/N at the label (loss.cc:61-72).
// Row-structured: blockIdx.y strides over rows, so no per-element index
// division; 16-byte rows (C % 4 == 0, aligned) stream as float4.
__global__ __launch_bounds__(kBlock) void xent_bwd_kernel(const float* __restrict__ probs,
                                                          const int32_t* __restrict__ labels,
                                                          const float* __restrict__ seed,
                                                          float* __restrict__ dl, size_t N,
                                                          size_t C, int vec, int nt) {
  const float scale = *seed / static_cast<float>(N);
  const size_t cstride = static_cast<size_t>(gridDim.x) * kBlock;
  const size_t c0 = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  for (size_t n = blockIdx.y; n < N; n += gridDim.y) {
    const int32_t lab = labels[n];
    const size_t lc = lab >= 0 ? static_cast<size_t>(lab) : ~size_t{0};
    if (vec) {
      for (size_t j = c0; j < C / 4; j += cstride) {
        const float4 p = ld4(probs + n * C + 4 * j, nt);
        float4 o = make_float4(scale * p.x, scale * p.y, scale * p.z, scale * p.w);
        if (lc / 4 == j) {
          if (lc % 4 == 0) o.x -= scale;
          else if (lc % 4 == 1) o.y -= scale;
          else if (lc % 4 == 2) o.z -= scale;
          else o.w -= scale;
        }
        st4(dl + n * C + 4 * j, o, nt);
      }
    } else {
      const float* pr = probs + n * C;
      float* dr = dl + n * C;
      for (size_t cc = c0; cc < C; cc += cstride) {
        float v = scale * pr[cc];
        if (lc == cc) v -= scale;
        dr[cc] = v;
      }
    }
  }
}

// dpred = (2*seed/n) * (pred - target)  (loss.cc:91-97)
__global__ __launch_bounds__(kBlock) void mse_bwd_kernel(const float* __restrict__ pred,
                                                         const float* __restrict__ target,
                                                         const float* __restrict__ seed,
                                                         float* __restrict__ dp, size_t n,
                                                         size_t nv) {
  const float scale = 2.0f * *seed / static_cast<float>(n);
  const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
  const size_t gid = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  const float4* p4 = reinterpret_cast<const float4*>(pred);
  const float4* t4 = reinterpret_cast<const float4*>(target);
  float4* d4 = reinterpret_cast<float4*>(dp);
  for (size_t i = gid; i < nv; i += stride) {
    const float4 a = p4[i], b = t4[i];
    d4[i] = make_float4(scale * (a.x - b.x), scale * (a.y - b.y), scale * (a.z - b.z),
                        scale * (a.w - b.w));
  }
  for (size_t i = nv * 4 + gid; i < n; i += stride) dp[i] = scale * (pred[i] - target[i]);
}

// dlogits = seed/(N*T) * (p_s - p_t)  (loss.cc:134-140)
__global__ __launch_bounds__(kBlock) void kl_bwd_kernel(const float* __restrict__ ps,
                                                        const float* __restrict__ pt,
                                                        const float* __restrict__ seed,
                                                        float* __restrict__ dl, size_t total,
                                                        size_t N, float T) {
  const float scale = *seed / (static_cast<float>(N) * T);
  const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < total; i += stride)
    dl[i] = scale * (ps[i] - pt[i]);
}

// p -= lr * (g + wd * p)  (optimizer.cc:37-42), lr = this step's EffectiveLr.
__global__ __launch_bounds__(kBlock) void sgd_kernel(float* __restrict__ p,
                                                     const float* __restrict__ g, size_t n,
                                                     const StepScalars* __restrict__ s) {
  const float lr = s->lr, wd = s->weight_decay;
  const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
    p[i] -= lr * (g[i] + wd * p[i]);
}

// AdamW with host-hoisted bias corrections (optimizer.cc:44-69).
__device__ __forceinline__ void adamw_elem(float& p, float g, float& m, float& v, float lr,
                                           float b1, float b2, float omb1, float omb2,
                                           float ibc1, float ibc2, float eps, float wd) {
  const float mi = b1 * m + omb1 * g;
  const float vi = b2 * v + omb2 * g * g;
  m = mi;
  v = vi;
  const float m_hat = mi * ibc1;
  const float v_hat = vi * ibc2;
  // HIP device '/' and sqrtf are IEEE correctly rounded (clang's default
  // -fhip-fp32-correctly-rounded-divide-sqrt), matching the CPU's bits.
  p -= lr * (m_hat / (sqrtf(v_hat) + eps) + wd * p);
}

__global__ __launch_bounds__(kBlock) void adamw_kernel(float* __restrict__ p,
                                                       const float* __restrict__ g,
                                                       float* __restrict__ m,
                                                       float* __restrict__ v, size_t n, size_t nv,
                                                       const StepScalars* __restrict__ s) {
  const float lr = s->lr, b1 = s->beta1, b2 = s->beta2, omb1 = s->om_b1, omb2 = s->om_b2;
  const float ibc1 = s->inv_bc1, ibc2 = s->inv_bc2, eps = s->eps, wd = s->weight_decay;
  const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
  const size_t gid = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  float4* p4 = reinterpret_cast<float4*>(p);
  const float4* g4 = reinterpret_cast<const float4*>(g);
  float4* m4 = reinterpret_cast<float4*>(m);
  float4* v4 = reinterpret_cast<float4*>(v);
  for (size_t i = gid; i < nv; i += stride) {
    float4 pp = p4[i], mm = m4[i], vv = v4[i];
    const float4 gg = g4[i];
    adamw_elem(pp.x, gg.x, mm.x, vv.x, lr, b1, b2, omb1, omb2, ibc1, ibc2, eps, wd);
    adamw_elem(pp.y, gg.y, mm.y, vv.y, lr, b1, b2, omb1, omb2, ibc1, ibc2, eps, wd);
    adamw_elem(pp.z, gg.z, mm.z, vv.z, lr, b1, b2, omb1, omb2, ibc1, ibc2, eps, wd);
    adamw_elem(pp.w, gg.w, mm.w, vv.w, lr, b1, b2, omb1, omb2, ibc1, ibc2, eps, wd);
    p4[i] = pp;
    m4[i] = mm;
    v4[i] = vv;
  }
  for (size_t i = nv * 4 + gid; i < n; i += stride) {
    float pp = p[i], mm = m[i], vv = v[i];
    adamw_elem(pp, g[i], mm, vv, lr, b1, b2, omb1, omb2, ibc1, ibc2, eps, wd);
    p[i] = pp;
    m[i] = mm;
    v[i] = vv;
  }
}

// Multi-tensor AdamW: workgroup b owns elements [lb*kAdamWChunk,
// (lb+1)*kAdamWChunk) of the segment whose first_block <= b (binary search),
// lb = b - first_block.
constexpr uint64_t kAdamWChunk = 4096;

__global__ __launch_bounds__(kBlock) void adamw_multi_kernel(const AdamWSegment* __restrict__ segs,
                                                             uint32_t nseg,
                                                             const StepScalars* __restrict__ s) {
  uint32_t lo = 0, hi = nseg - 1;
  const uint64_t b = blockIdx.x;
  while (lo < hi) {
    const uint32_t mid = (lo + hi + 1) / 2;
    if (segs[mid].first_block <= b) lo = mid;
    else hi = mid - 1;
  }
  const AdamWSegment sg = segs[lo];
  const uint64_t begin = (b - sg.first_block) * kAdamWChunk;
  const uint64_t end = begin + kAdamWChunk < sg.n ? begin + kAdamWChunk : sg.n;
  const float lr = s->lr, b1 = s->beta1, b2 = s->beta2, omb1 = s->om_b1, omb2 = s->om_b2;
  const float ibc1 = s->inv_bc1, ibc2 = s->inv_bc2, eps = s->eps, wd = s->weight_decay;
  uint64_t i = begin + threadIdx.x * 4;
  const bool vec = aligned16(sg.p) && aligned16(sg.g) && aligned16(sg.m) && aligned16(sg.v);
  if (vec) {
    for (; i + 3 < end; i += kBlock * 4) {
      float4 p = *reinterpret_cast<float4*>(sg.p + i);
      const float4 g = *reinterpret_cast<const float4*>(sg.g + i);
      float4 m = *reinterpret_cast<float4*>(sg.m + i);
      float4 v = *reinterpret_cast<float4*>(sg.v + i);
      adamw_elem(p.x, g.x, m.x, v.x, lr, b1, b2, omb1, omb2, ibc1, ibc2, eps, wd);
      adamw_elem(p.y, g.y, m.y, v.y, lr, b1, b2, omb1, omb2, ibc1, ibc2, eps, wd);
      adamw_elem(p.z, g.z, m.z, v.z, lr, b1, b2, omb1, omb2, ibc1, ibc2, eps, wd);
      adamw_elem(p.w, g.w, m.w, v.w, lr, b1, b2, omb1, omb2, ibc1, ibc2, eps, wd);
      *reinterpret_cast<float4*>(sg.p + i) = p;
      *reinterpret_cast<float4*>(sg.m + i) = m;
      *reinterpret_cast<float4*>(sg.v + i) = v;
    }
  }
  // Element form: the unaligned case, and a segment's last partial vector.
  for (uint64_t e = vec ? i : begin + threadIdx.x * 4; e < end; e += kBlock * 4)
    for (uint64_t k = e; k < e + 4 && k < end; ++k)
      adamw_elem(sg.p[k], sg.g[k], sg.m[k], sg.v[k], lr, b1, b2, omb1, omb2, ibc1, ibc2, eps, wd);
}

// RoPE on interleaved pairs (attention.cc:39-92). theta = s * freq_c with
// freq_c = step^c built by the reference's recurrence freq *= step (c
// multiplications in float, so freq_c has the CPU's bits); cos/sin are the
// device's accurate cosf/sinf. Rows are [B*S] x [H*d]; s = row % S.
//
// Fast form (d % 4 == 0, d/2 <= kRopeTable, 16-byte aligned rows): the
// angle depends on (position, pair) only, not on the head, so a workgroup
// owning R consecutive rows first evaluates cos/sin of their R * d/2 angles
// once into LDS (the same float expressions, so the same bits), then
// streams the rows' H heads as float4 = 2 pairs.
constexpr int kRopeTable = 256;

template <int DIR>
__global__ __launch_bounds__(kBlock) void rope_rows_kernel(const float* __restrict__ x,
                                                           float* __restrict__ y, uint32_t rows,
                                                           uint32_t S, uint32_t width,
                                                           uint32_t d, uint32_t rpb, float step,
                                                           int nt) {
  __shared__ float2 cs[kRopeTable];
  const uint32_t half_d = d / 2;
  const uint32_t row0 = blockIdx.x * rpb;
  const uint32_t nrow = rows - row0 < rpb ? rows - row0 : rpb;
  for (uint32_t e = threadIdx.x; e < nrow * half_d; e += kBlock) {
    const uint32_t c = e % half_d, r = e / half_d;
    float f = 1.0f;
    for (uint32_t i = 0; i < c; ++i) f *= step;
    const float theta = static_cast<float>((row0 + r) % S) * f;
    cs[e] = make_float2(cosf(theta), sinf(theta));
  }
  __syncthreads();
  const uint32_t nv = width / 4;
  for (uint32_t r = 0; r < nrow; ++r) {
    const float4* xr = reinterpret_cast<const float4*>(x + static_cast<size_t>(row0 + r) * width);
    float4* yr = reinterpret_cast<float4*>(y + static_cast<size_t>(row0 + r) * width);
    const float2* tr = cs + r * half_d;
    for (uint32_t j = threadIdx.x; j < nv; j += kBlock) {
      const uint32_t c2 = ((4 * j) % d) / 2;
      const float4 v = ld4(reinterpret_cast<const float*>(xr + j), nt);
      const float2 a = tr[c2], b = tr[c2 + 1];
      const float c0 = a.x, s0 = a.y, c1 = b.x, s1 = b.y;
      float4 o;
      if constexpr (DIR > 0) {
        o.x = v.x * c0 - v.y * s0;
        o.y = v.x * s0 + v.y * c0;
        o.z = v.z * c1 - v.w * s1;
        o.w = v.z * s1 + v.w * c1;
      } else {
        o.x = v.x * c0 + v.y * s0;
        o.y = -v.x * s0 + v.y * c0;
        o.z = v.z * c1 + v.w * s1;
        o.w = -v.z * s1 + v.w * c1;
      }
      st4(reinterpret_cast<float*>(yr + j), o, nt);
    }
  }
}

// The angle table: one thread per (position, pair), the same expressions as
// rope_rows_kernel's LDS table.
__global__ __launch_bounds__(kBlock) void rope_angle_table_kernel(float* __restrict__ table,
                                                                  uint32_t S, uint32_t half_d,
                                                                  float step) {
  const uint32_t e = blockIdx.x * kBlock + threadIdx.x;
  if (e >= S * half_d) return;
  const uint32_t c = e % half_d, sp = e / half_d;
  float f = 1.0f;
  for (uint32_t i = 0; i < c; ++i) f *= step;
  const float theta = static_cast<float>(sp) * f;
  table[2 * e] = cosf(theta);
  table[2 * e + 1] = sinf(theta);
}

// RoPE through the angle table: each float4 of x is two pairs of one
// position; its cos/sin are one float4 of the (cache-resident) table. POW2:
// the row width (in float4s), S and d are powers of two, and the element's
// row, column and position come from shifts and masks (nv_shift = log2 of
// the row width) rather than three integer divisions per float4.
// PAIR: a second tensor of the same geometry (x2 -> y2) in the same
// launch, as the instruction after the first would run it. Each thread
// loads both tensors' float4s before it stores either, and stores y before
// y2, so the two may share ranges as long as every pair of ranges is
// identical or disjoint and x2 is not y (the host's conditions).
template <int DIR, bool NT, bool POW2, bool PAIR = false>
__global__ __launch_bounds__(kBlock) void rope_table_kernel(const float* x, float* y,
                                                            const float* __restrict__ table,
                                                            uint32_t nv_row, uint32_t total4,
                                                            uint32_t S, uint32_t d,
                                                            uint32_t nv_shift, const float* x2,
                                                            float* y2) {
  constexpr int kU = Unroll(NT);
  const uint32_t stride = gridDim.x * kBlock * kU;
  for (uint32_t base = blockIdx.x * kBlock * kU + threadIdx.x; base < total4; base += stride) {
    float4 v[kU], t[kU], v2[PAIR ? kU : 1];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const uint32_t i = base + u * kBlock;
      if (i >= total4) continue;
      uint32_t pos, c2;  // c2 even: the float4 below is aligned
      if constexpr (POW2) {
        const uint32_t row = i >> nv_shift, col4 = i & (nv_row - 1);
        c2 = ((4 * col4) & (d - 1)) >> 1;
        pos = row & (S - 1);
      } else {
        const uint32_t row = i / nv_row, col4 = i - row * nv_row;
        c2 = ((4 * col4) % d) / 2;
        pos = row % S;
      }
      v[u] = ld4(x + 4 * static_cast<size_t>(i), NT);
      if constexpr (PAIR) v2[u] = ld4(x2 + 4 * static_cast<size_t>(i), NT);
      t[u] = *reinterpret_cast<const float4*>(table + 2 * (pos * (d / 2) + c2));
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const uint32_t i = base + u * kBlock;
      if (i >= total4) continue;
      const float c0 = t[u].x, s0 = t[u].y, c1 = t[u].z, s1 = t[u].w;
      auto rot = [&](const float4 w) {
        float4 o;
        if constexpr (DIR > 0) {
          o.x = w.x * c0 - w.y * s0;
          o.y = w.x * s0 + w.y * c0;
          o.z = w.z * c1 - w.w * s1;
          o.w = w.z * s1 + w.w * c1;
        } else {
          o.x = w.x * c0 + w.y * s0;
          o.y = -w.x * s0 + w.y * c0;
          o.z = w.z * c1 + w.w * s1;
          o.w = -w.z * s1 + w.w * c1;
        }
        return o;
      };
      st4(y + 4 * static_cast<size_t>(i), rot(v[u]), NT);
      if constexpr (PAIR) st4(y2 + 4 * static_cast<size_t>(i), rot(v2[u]), NT);
    }
  }
}

// General form: one thread per pair.
__global__ __launch_bounds__(kBlock) void rope_kernel(const float* __restrict__ x,
                                                      float* __restrict__ y, size_t pairs,
                                                      size_t S, size_t H, size_t half_d,
                                                      float step, int dir) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
  for (size_t p = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; p < pairs; p += stride) {
    const size_t c2 = p % half_d;
    const size_t u = p / half_d;  // (row, head) unit
    const size_t s = (u / H) % S;
    float freq = 1.0f;
    for (size_t i = 0; i < c2; ++i) freq *= step;
    const float theta = static_cast<float>(s) * freq;
    const float cs = cosf(theta), sn = sinf(theta);
    const float a = x[2 * p], b2 = x[2 * p + 1];
    if (dir > 0) {
      y[2 * p] = a * cs - b2 * sn;
      y[2 * p + 1] = a * sn + b2 * cs;
    } else {
      y[2 * p] = a * cs + b2 * sn;
      y[2 * p + 1] = -a * sn + b2 * cs;
    }
  }
}

Status Rope(const float* x, float* y, size_t B, size_t S, size_t H, size_t d, float base,
            int dir, const Ctx& c, const char* what) {
  if (d % 2 != 0) return Status::Fail(kUnitEngine, std::string(what) + ": odd head width");
  const size_t pairs = B * S * H * (d / 2);
  if (pairs == 0) return Status::Ok();
  // step = base^(-2/d) evaluated on the host with the reference's powf.
  const float step = ::powf(base, -2.0f / static_cast<float>(d));
  const size_t rows = B * S, width = H * d;
  const bool fast = d % 4 == 0 && d / 2 <= static_cast<size_t>(kRopeTable) && aligned16(x) &&
                    aligned16(y) && rows <= 0xFFFFFFFFu && width <= 0xFFFFFFFFu && S > 0;
  if (fast) {
    const uint32_t rpb = static_cast<uint32_t>(kRopeTable / (d / 2));
    const int nt = StreamPolicy(8 * rows * width) ? 1 : 0;
    const unsigned grid = static_cast<unsigned>((rows + rpb - 1) / rpb);
    if (dir > 0)
      hipLaunchKernelGGL(rope_rows_kernel<1>, dim3(grid), dim3(kBlock), 0, c.stream, x, y,
                         static_cast<uint32_t>(rows), static_cast<uint32_t>(S),
                         static_cast<uint32_t>(width), static_cast<uint32_t>(d), rpb, step, nt);
    else
      hipLaunchKernelGGL(rope_rows_kernel<-1>, dim3(grid), dim3(kBlock), 0, c.stream, x, y,
                         static_cast<uint32_t>(rows), static_cast<uint32_t>(S),
                         static_cast<uint32_t>(width), static_cast<uint32_t>(d), rpb, step, nt);
  } else {
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(pairs, kBlock, kGridCap)), dim3(kBlock), 0,
                       c.stream, x, y, pairs, S, H, d / 2, step, dir);
  }
  return LaunchStatus(what);
}

}  // namespace

int PwProgramOf(int nin, const PwStep* steps, int nops) {
  for (int p = 0; p < kNumPwProgs; ++p) {
    const PwProg& g = kPwProgs[p];
    if (g.nin != nin || g.nops != nops) continue;
    bool same = true;
    for (int j = 0; j < nops; ++j)
      same = same && g.op[j] == steps[j].op && g.a[j] == steps[j].a && g.b[j] == steps[j].b;
    if (same) return p;
  }
  return -1;
}

Status LaunchPointwiseRun(const PointwiseRun& r, const Ctx& c) {
  if (r.program < 0 || r.program >= kNumPwProgs)
    return Status::Fail(kUnitEngine, "pointwise run: no compiled program");
  const PwProg& g = kPwProgs[r.program];
  bool aligned = true;
  int nout = 0;
  for (int k = 0; k < g.nin; ++k) aligned = aligned && aligned16(r.in[k]);
  for (int j = 0; j < g.nops; ++j)
    if (r.out[j]) aligned = aligned && aligned16(r.out[j]), ++nout;
  if (r.n == 0 || nout == 0) return Status::Ok();
  const size_t nv = aligned ? r.n / 4 : 0;
  const bool nt = StreamPolicy(4 * r.n * static_cast<size_t>(g.nin + nout));
  const size_t work = nv ? (nv + Unroll(nt) - 1) / Unroll(nt) : r.n;
  const dim3 grid(grid_for(work, kBlock, nt ? kStreamGridCap : kGridCap));
  switch (r.program) {
    case 0: LaunchPw<0>(r, nv, nt, grid, c.stream); break;
    case 1: LaunchPw<1>(r, nv, nt, grid, c.stream); break;
    case 2: LaunchPw<2>(r, nv, nt, grid, c.stream); break;
    case 3: LaunchPw<3>(r, nv, nt, grid, c.stream); break;
    case 4: LaunchPw<4>(r, nv, nt, grid, c.stream); break;
    case 5: LaunchPw<5>(r, nv, nt, grid, c.stream); break;
    default: LaunchPw<6>(r, nv, nt, grid, c.stream); break;
  }
  static_assert(kNumPwProgs == 7, "one launch case per program");
  return LaunchStatus("pointwise run");
}

Status AddEW(const float* x, const float* y, float* out, size_t n, const Ctx& c) {
  return Binary(x, y, out, n, AddF{}, c, "AddEW");
}
Status MulEW(const float* x, const float* y, float* out, size_t n, const Ctx& c) {
  return Binary(x, y, out, n, MulF{}, c, "MulEW");
}
Status Scale(const float* x, float* out, float alpha, size_t n, const Ctx& c) {
  return Unary(x, out, n, ScaleF{alpha}, c, "Scale");
}
Status ReluFwd(const float* x, float* out, size_t n, const Ctx& c) {
  return Unary(x, out, n, ReluF{}, c, "ReluFwd");
}
Status ReluBwd(const float* dy, const float* x, float* dx, size_t n, const Ctx& c) {
  return Binary(dy, x, dx, n, ReluBwdF{}, c, "ReluBwd");
}
Status GeluFwd(const float* x, float* out, size_t n, const Ctx& c) {
  return Unary(x, out, n, GeluF{}, c, "GeluFwd");
}
Status GeluBwd(const float* dy, const float* x, float* dx, size_t n, const Ctx& c) {
  return Binary(dy, x, dx, n, GeluBwdF{}, c, "GeluBwd");
}
Status SiluFwd(const float* x, float* out, size_t n, const Ctx& c) {
  return Unary(x, out, n, SiluF{}, c, "SiluFwd");
}
Status SiluBwd(const float* dy, const float* x, float* dx, size_t n, const Ctx& c) {
  return Binary(dy, x, dx, n, SiluBwdF{}, c, "SiluBwd");
}
Status Copy(const float* src, float* dst, size_t n, const Ctx& c) {
  return Unary(src, dst, n, CopyF{}, c, "Copy");
}

// 32x32 tiles through LDS (padded a column against bank conflicts): reads
// and writes are both row-contiguous 128-byte runs.
constexpr int kTr = 32;
__global__ __launch_bounds__(256) void transpose_kernel(const float* __restrict__ src,
                                                        float* __restrict__ dst, int64_t rows,
                                                        int64_t cols) {
  __shared__ float tile[kTr][kTr + 1];
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * kTr, c0 = static_cast<int64_t>(blockIdx.x) * kTr;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8 threads
  for (int k = ty; k < kTr; k += 8) {
    const int64_t r = r0 + k, c = c0 + tx;
    if (r < rows && c < cols) tile[k][tx] = src[r * cols + c];
  }
  __syncthreads();
  for (int k = ty; k < kTr; k += 8) {
    const int64_t c = c0 + k, r = r0 + tx;
    if (r < rows && c < cols) dst[c * rows + r] = tile[tx][k];
  }
}

Status Transpose(const float* src, float* dst, int64_t rows, int64_t cols, const Ctx& c) {
  if (rows <= 0 || cols <= 0) return Status::Ok();
  const int64_t gx = (cols + kTr - 1) / kTr, gy = (rows + kTr - 1) / kTr;
  if (gx > 0x7FFFFFFF || gy > 65535) return Status::Fail(kUnitEngine, "Transpose: grid exceeds launch limits");
  hipLaunchKernelGGL(transpose_kernel, dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gy)),
                     dim3(256), 0, c.stream, src, dst, rows, cols);
  return LaunchStatus("Transpose");
}

Status Fill(float* dst, float value, size_t n, const Ctx& c) {
  if (n == 0) return Status::Ok();
  const size_t nv = aligned16(dst) ? n / 4 : 0;
  hipLaunchKernelGGL(fill_kernel, dim3(grid_for(nv ? nv : n, kBlock, kGridCap)), dim3(kBlock), 0,
                     c.stream, dst, n, nv, value);
  return LaunchStatus("Fill");
}

Status AddBias(const float* x, const float* b, float* out, size_t rows, size_t cols,
               const Ctx& c) {
  const size_t n = rows * cols;
  if (n == 0) return Status::Ok();
  const int vec = (cols % 4 == 0 && aligned16(x) && aligned16(b) && aligned16(out)) ? 1 : 0;
  hipLaunchKernelGGL(add_bias_kernel, dim3(grid_for(vec ? n / 4 : n, kBlock, kGridCap)),
                     dim3(kBlock), 0, c.stream, x, b, out, n, cols, vec);
  return LaunchStatus("AddBias");
}

Status EmbedFwd(const int32_t* tokens, const float* table, float* out, size_t rows, size_t dim,
                size_t vocab, const Ctx& c) {
  if (rows == 0 || dim == 0) return Status::Ok();
  const int vec = (dim % 4 == 0 && aligned16(table) && aligned16(out)) ? 1 : 0;
  const size_t waves = rows;
  hipLaunchKernelGGL(embed_kernel, dim3(grid_for(waves * kWave, kBlock, kGridCap)), dim3(kBlock),
                     0, c.stream, tokens, table, out, rows, dim, vocab, vec);
  return LaunchStatus("EmbedFwd");
}

Status ReduceRows(const float* dy, float* db, size_t rows, size_t cols, const Ctx& c) {
  if (cols == 0) return Status::Ok();
  hipLaunchKernelGGL(reduce_rows_kernel, dim3((cols + kBlock - 1) / kBlock), dim3(kBlock), 0,
                     c.stream, dy, db, rows, cols);
  return LaunchStatus("ReduceRows");
}

Status SoftmaxXEntBwd(const float* probs, const int32_t* labels, const float* seed,
                      float* dlogits, size_t N, size_t C, const Ctx& c) {
  if (N == 0 || C == 0) return Status::Ok();
  const bool vec = C % 4 == 0 && aligned16(probs) && aligned16(dlogits);
  const size_t per_row = vec ? C / 4 : C;
  // Columns: enough blocks to cover a row in ~4 passes; rows: up to 65535
  // per grid row, striding beyond.
  const unsigned gx = std::max(1u, grid_for((per_row + 3) / 4, kBlock, 64));
  const unsigned gy = static_cast<unsigned>(std::min<size_t>(N, 65535));
  hipLaunchKernelGGL(xent_bwd_kernel, dim3(gx, gy), dim3(kBlock), 0, c.stream, probs, labels,
                     seed, dlogits, N, C, vec ? 1 : 0, StreamPolicy(8 * N * C) ? 1 : 0);
  return LaunchStatus("SoftmaxXEntBwd");
}

Status MseBwd(const float* pred, const float* target, const float* seed, float* dpred, size_t n,
              const Ctx& c) {
  if (n == 0) return Status::Ok();
  const size_t nv = (aligned16(pred) && aligned16(target) && aligned16(dpred)) ? n / 4 : 0;
  hipLaunchKernelGGL(mse_bwd_kernel, dim3(grid_for(nv ? nv : n, kBlock, kGridCap)), dim3(kBlock),
                     0, c.stream, pred, target, seed, dpred, n, nv);
  return LaunchStatus("MseBwd");
}

Status KLDistillBwd(const float* p_s, const float* p_t, const float* seed, float* dlogits,
                    size_t N, size_t C, float T, const Ctx& c) {
  if (N * C == 0) return Status::Ok();
  hipLaunchKernelGGL(kl_bwd_kernel, dim3(grid_for(N * C, kBlock, kGridCap)), dim3(kBlock), 0,
                     c.stream, p_s, p_t, seed, dlogits, N * C, N, T);
  return LaunchStatus("KLDistillBwd");
}

Status SgdStep(float* p, const float* g, size_t n, const Ctx& c) {
  if (n == 0) return Status::Ok();
  if (!c.scalars) return Status::Fail(kUnitEngine, "SgdStep: no step scalars bound");
  hipLaunchKernelGGL(sgd_kernel, dim3(grid_for(n, kBlock, kGridCap)), dim3(kBlock), 0, c.stream,
                     p, g, n, c.scalars);
  return LaunchStatus("SgdStep");
}

uint64_t AdamWMultiPlan(AdamWSegment* segs, size_t nseg) {
  uint64_t blocks = 0;
  for (size_t i = 0; i < nseg; ++i) {
    segs[i].first_block = blocks;
    blocks += (segs[i].n + kAdamWChunk - 1) / kAdamWChunk;
  }
  return blocks;
}

Status AdamWMulti(const AdamWSegment* segs, size_t nseg, uint64_t blocks, const Ctx& c) {
  if (nseg == 0 || blocks == 0) return Status::Ok();
  if (!c.scalars) return Status::Fail(kUnitEngine, "AdamWStep: no step scalars bound");
  if (blocks > 0x7FFFFFFFu || nseg > 0xFFFFFFFFu)
    return Status::Fail(kUnitEngine, "AdamWStep: fused launch too large");
  hipLaunchKernelGGL(adamw_multi_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0,
                     c.stream, segs, static_cast<uint32_t>(nseg), c.scalars);
  return LaunchStatus("AdamWStep(fused)");
}

Status AdamWStep(float* p, const float* g, float* m, float* v, size_t n, const Ctx& c) {
  if (n == 0) return Status::Ok();
  if (!c.scalars) return Status::Fail(kUnitEngine, "AdamWStep: no step scalars bound");
  const size_t nv =
      (aligned16(p) && aligned16(g) && aligned16(m) && aligned16(v)) ? n / 4 : 0;
  hipLaunchKernelGGL(adamw_kernel, dim3(grid_for(nv ? nv : n, kBlock, kGridCap)), dim3(kBlock),
                     0, c.stream, p, g, m, v, n, nv, c.scalars);
  return LaunchStatus("AdamWStep");
}

size_t RopeTableFloats(size_t S, size_t d) { return S * d; }

Status RopeTable(float* table, size_t S, size_t d, float base, const Ctx& c) {
  if (d % 2 != 0 || S * (d / 2) > 0xFFFFFFFFu) return Status::Fail(kUnitEngine, "RopeTable: bad shape");
  if (S == 0 || d == 0) return Status::Ok();
  const float step = ::powf(base, -2.0f / static_cast<float>(d));  // as Rope
  const size_t n = S * (d / 2);
  hipLaunchKernelGGL(rope_angle_table_kernel, dim3(static_cast<unsigned>((n + kBlock - 1) / kBlock)),
                     dim3(kBlock), 0, c.stream, table, static_cast<uint32_t>(S),
                     static_cast<uint32_t>(d / 2), step);
  return LaunchStatus("RopeTable");
}

Status RopeWithTable(const float* x, float* y, size_t B, size_t S, size_t H, size_t d,
                     const float* table, int dir, const Ctx& c, const float* x2, float* y2) {
  const size_t rows = B * S, width = H * d;
  if (rows == 0 || width == 0) return Status::Ok();
  const bool pair = x2 != nullptr;
  if (d % 4 != 0 || S == 0 || !aligned16(x) || !aligned16(y) || !aligned16(table) ||
      (pair && (!y2 || !aligned16(x2) || !aligned16(y2) || x2 == y)) ||
      rows * width / 4 > 0xFFFFFFFFu || S * d > 0xFFFFFFFFu)
    return Status::Fail(kUnitEngine, "Rope: the table form needs d % 4 == 0 and aligned operands");
  const uint32_t total4 = static_cast<uint32_t>(rows * width / 4);
  const bool nt = StreamPolicy((pair ? 16 : 8) * rows * width);
  const size_t work = (total4 + Unroll(nt) - 1) / Unroll(nt);
  const dim3 grid(grid_for(work, kBlock, nt ? kStreamGridCap : kGridCap));
  const uint32_t nv_row = static_cast<uint32_t>(width / 4), S32 = static_cast<uint32_t>(S),
                 d32 = static_cast<uint32_t>(d);
  auto pow2 = [](uint32_t v) { return v != 0 && (v & (v - 1)) == 0; };
  const bool p2 = pow2(nv_row) && pow2(S32) && pow2(d32);
  uint32_t shift = 0;
  while (p2 && (1u << shift) < nv_row) ++shift;
#define SEEML_ROPE1(D, N, P, Q)                                                                 \
  hipLaunchKernelGGL((rope_table_kernel<D, N, P, Q>), grid, dim3(kBlock), 0, c.stream, x, y, table, \
                     nv_row, total4, S32, d32, shift, x2, y2)
#define SEEML_ROPE(D, N, P) \
  do { if (pair) SEEML_ROPE1(D, N, P, true); else SEEML_ROPE1(D, N, P, false); } while (0)
  if (dir > 0) {
    if (p2) { if (nt) SEEML_ROPE(1, true, true); else SEEML_ROPE(1, false, true); }
    else { if (nt) SEEML_ROPE(1, true, false); else SEEML_ROPE(1, false, false); }
  } else {
    if (p2) { if (nt) SEEML_ROPE(-1, true, true); else SEEML_ROPE(-1, false, true); }
    else { if (nt) SEEML_ROPE(-1, true, false); else SEEML_ROPE(-1, false, false); }
  }
#undef SEEML_ROPE
#undef SEEML_ROPE1
  return LaunchStatus(dir > 0 ? "RopeFwd" : "RopeBwd");
}

Status RopeFwd(const float* x, float* y, size_t B, size_t S, size_t H, size_t d, float base,
               const Ctx& c) {
  return Rope(x, y, B, S, H, d, base, +1, c, "RopeFwd");
}
Status RopeBwd(const float* dy, float* dx, size_t B, size_t S, size_t H, size_t d, float base,
               const Ctx& c) {
  return Rope(dy, dx, B, S, H, d, base, -1, c, "RopeBwd");
}

// One launch before a step: the step's scalars (kernel arguments, so no
// host buffer has to outlive the launch) and up to two device-resident
// batch copies into the arena slots. Copies run in 4-byte words (every slot
// holds f32 or i32 elements), 16-byte vectors where both ends allow.
struct StageCopy {
  const uint32_t* src;
  uint32_t* dst;
  size_t words;
};

__global__ __launch_bounds__(kBlock) void stage_step_kernel(StepScalars s, StepScalars* __restrict__ dst,
                                                            StageCopy a, StageCopy b) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
  const size_t gid = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (dst && gid == 0) *dst = s;
  const StageCopy cs[2] = {a, b};
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const StageCopy& c = cs[k];
    if (!c.words) continue;
    const bool vec = aligned16(c.src) && aligned16(c.dst);
    const size_t nv = vec ? c.words / 4 : 0;
    const uint4* s4 = reinterpret_cast<const uint4*>(c.src);
    uint4* d4 = reinterpret_cast<uint4*>(c.dst);
    for (size_t i = gid; i < nv; i += stride) d4[i] = s4[i];
    for (size_t i = nv * 4 + gid; i < c.words; i += stride) c.dst[i] = c.src[i];
  }
}

Status StageStep(const StepScalars* s, StepScalars* dst, const void* in_src, void* in_dst,
                 size_t in_bytes, const void* lab_src, void* lab_dst, size_t lab_bytes,
                 hipStream_t stream) {
  if (in_bytes % 4 != 0 || lab_bytes % 4 != 0)
    return Status::Fail(kUnitEngine, "StageStep: slot sizes must be whole 4-byte elements");
  const StageCopy a{static_cast<const uint32_t*>(in_src), static_cast<uint32_t*>(in_dst),
                    in_src ? in_bytes / 4 : 0};
  const StageCopy b{static_cast<const uint32_t*>(lab_src), static_cast<uint32_t*>(lab_dst),
                    lab_src ? lab_bytes / 4 : 0};
  if (!s && !a.words && !b.words) return Status::Ok();
  const size_t work = std::max<size_t>(std::max(a.words, b.words) / 4, 1);
  hipLaunchKernelGGL(stage_step_kernel, dim3(grid_for(work, kBlock, kGridCap)), dim3(kBlock), 0, stream,
                     s ? *s : StepScalars{}, s ? dst : nullptr, a, b);
  return LaunchStatus("StageStep");
}

// The loss scalar into host memory the device writes directly (a mapped
// pinned allocation): the host reads it after the stream's synchronisation,
// with no device-to-host copy launch.
__global__ void post_loss_kernel(const float* __restrict__ src, float* dst) {
  if (threadIdx.x == 0) {
    *dst = *src;
    __threadfence_system();
  }
}

Status PostLoss(const float* src, float* host_dst, hipStream_t stream) {
  hipLaunchKernelGGL(post_loss_kernel, dim3(1), dim3(64), 0, stream, src, host_dst);
  return LaunchStatus("PostLoss");
}

// The device's constant-rate wall clock, read by one lane: a graph node
// before a launch stores it (slot[0]); one after adds the elapsed ticks to
// slot[1] and counts the interval in slot[2], so repeated replays
// accumulate with no host read between them (one stream: the nodes of one
// slot never run concurrently).
__global__ void wall_stamp_kernel(uint64_t* slot, int close) {
  if (threadIdx.x == 0) {
    const uint64_t now = wall_clock64();
    if (close) {
      slot[1] += now - slot[0];
      slot[2] += 1;
    } else {
      slot[0] = now;
    }
  }
}

Status WallStamp(uint64_t* slot, bool close, hipStream_t stream) {
  hipLaunchKernelGGL(wall_stamp_kernel, dim3(1), dim3(64), 0, stream, slot, close ? 1 : 0);
  return LaunchStatus("WallStamp");
}

StepScalars MakeStepScalars(const PlanHeader& h, uint64_t step) {
  StepScalars s{};
  s.lr = EffectiveLr(h, step);
  // optimizer.cc:52-58: float pow, hoisted reciprocal bias corrections.
  s.inv_bc1 = 1.0f / (1.0f - ::powf(h.beta1, static_cast<float>(step)));
  s.inv_bc2 = 1.0f / (1.0f - ::powf(h.beta2, static_cast<float>(step)));
  s.beta1 = h.beta1;
  s.beta2 = h.beta2;
  s.om_b1 = 1.0f - h.beta1;
  s.om_b2 = 1.0f - h.beta2;
  s.eps = h.eps;
  s.weight_decay = h.weight_decay;
  return s;
}

Status LaunchStatus(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return Status::Ok();
  return Status::Fail(kUnitEngine, std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace seeml_hip
