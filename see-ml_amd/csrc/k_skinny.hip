// k_skinny.hip — the LoRA-shaped GEMMs: one dimension is the adapter rank r
// (8..64), the others are a token count and a model width. They are bound
// by streaming the one large operand (reads) or the large output (writes)
// through HBM, not by the matrix cores, so each has its own kernel shaped
// for full-width 16-byte traffic. Serves GemmNN / GemmNT / GemmTN of
// runtime/executor/gemm.cc:173-200 at these shapes (the LoRA graft's
// t = x A, u = t B and their VJPs, compiler/.../lora_grafter.cc:130-159).
//
//   outer   K <= 64 (u = t B, dx = dt A^T): C[M,N] written once. Computed
//           transposed, C^T = B^T A^T, with v_mfma_f32_16x16x4_f32, so the
//           four lanes of a row hold 16 consecutive outputs and C is stored
//           as 64-byte row runs.
//   rowdot  N <= 64, A k-contiguous (t = x A, dt = du B^T): the [M, K]
//           operand is read once. 16 rows per workgroup with
//           v_mfma_f32_16x16x4_f32 (lane quarter q supplies k = 16g + 4q + j,
//           one float4 per group); the eight wavefronts take consecutive
//           slices of K, prefetching one batch ahead, and their partial tiles
//           are summed in wavefront order through LDS.
//   colsum  TN with min(M, N) <= 64 (dA = x^T dt, dB = t^T du): the large
//           [K, W] operand is read once, row by row, as float4 runs (MFMA c4
//           of v_mfma_f32_16x16x4_f32 takes component c4 of the lane's four
//           columns). A workgroup owns 64 columns and a k-group; its four
//           wavefronts are summed in order through LDS into one partial per
//           k-group, and a second kernel sums the k-group partials in group
//           order and applies the epilogue.
//
// Every reduction has a fixed order: results are bit-identical run to run.
#include "device_common.h"
#include "kernels.h"

#include <algorithm>

namespace seeml_hip {

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

struct SkArgs {
  const float* A;
  const float* B;
  float* C;
  float* ws;
  int64_t M, N, K, lda, ldb, ldc;
  float alpha;
  int accumulate;
  const float* bias;
  int act;
  int b_kc;
  // colsum
  int64_t W, R;        // large and small output extents
  int big_is_m;        // the large operand is A (W = M) or B (W = N)
  int groups;          // k-groups (partials)
  int64_t k_per_group;
  // outer: chained Scale / AddEW epilogue (SkinnyChain)
  int chain;
  float chain_alpha;
  float* S;
  const float* Y;
  float* Yout;
  int write_u;
  int y_first;
  // rowdot / colsum: the streamed operand is scaled as loaded (GemmDesc::
  // stream_scale), each element fl(stream_scale * x) as the folded Scale
  // would have stored it.
  int scale_stream;
  float stream_scale;
  // rowdot group: block nb of the output reads its own B operand Bm[nb] and
  // writes its own C, Cm[nb]; each is N <= 16 columns wide (same ldb, ldc).
  const float* Bm[4];
  float* Cm[4];
};

// v * scale where `keep`, else +0.0, with no branch: the mask is an AND of
// the bits (a select of a float4 can be lowered to per-lane branches).
__device__ __forceinline__ float4 Keep4(float4 v, bool keep, float scale) {
  const unsigned m = 0u - static_cast<unsigned>(keep);
  return make_float4(__uint_as_float(__float_as_uint(scale * v.x) & m),
                     __uint_as_float(__float_as_uint(scale * v.y) & m),
                     __uint_as_float(__float_as_uint(scale * v.z) & m),
                     __uint_as_float(__float_as_uint(scale * v.w) & m));
}

__device__ __forceinline__ float4 ScaleLoaded(const SkArgs& p, float4 v) {
  if (!p.scale_stream) return v;
  return make_float4(p.stream_scale * v.x, p.stream_scale * v.y, p.stream_scale * v.z,
                     p.stream_scale * v.w);
}

__device__ __forceinline__ float Epilogue(const SkArgs& p, int64_t m, int64_t n, float acc) {
  float val = p.alpha * acc;
  if (p.accumulate) val = p.C[m * p.ldc + n] + val;
  if (p.bias) val = val + p.bias[n];
  return dev_act(p.act, val);
}

// ---- outer (small K) ----------------------------------------------------------
//
// C^T blocks of 16 n x 16 m with v_mfma_f32_16x16x4_f32: lane (q, c) supplies
// A[m + c][16g + 4q + j] (one float4 per k group) and B(16g + 4q + j, n + c)
// for MFMA j, and holds C[m + c][n + 4q .. 4q + 3] — the four lanes of a row
// cover 64 contiguous bytes, so every store instruction writes 16 rows x 64 B
// (32-byte runs measured ~30% slower on this write-bound shape). A wavefront
// owns kOuterRB row blocks of 16 (their A fragments stay in registers) and
// walks 16-column steps, each B fragment serving all its row blocks. A
// workgroup is 4 wavefronts side by side in n: 16 * kOuterRB rows x
// 4 * kOuterWN columns.

constexpr int kOuterRB = 4;     // row blocks of 16 per wavefront
constexpr int kOuterWN = 128;   // columns per wavefront
constexpr int kOuterRows = 16 * kOuterRB;
constexpr int kOuterN = 4 * kOuterWN;

constexpr int kOuterSteps = kOuterWN / 16;  // 16-column steps per wavefront
// Loads issued ahead of their step: every B fragment at kernel entry when K
// fits one k group (8 float4 per lane), else two steps ahead; the chain's y
// operand two steps ahead. The step loop is unrolled, so each step's values
// are distinct registers and the loads stay in flight across steps (with one
// step ahead, the per-step latency of these small loads set the pace).
template <int KG>
constexpr int OuterBAhead() { return KG == 1 ? kOuterSteps : 2; }
constexpr int kOuterYAhead = 2;

template <int KG>  // k groups of 16: ceil(K / 16)
__device__ __forceinline__ void OuterLoadB(const SkArgs& p, int64_t n, int q, float (&bf)[KG][4]) {
#pragma unroll
  for (int g = 0; g < KG; ++g) {
    const int64_t k0 = 16 * g + 4 * q;
    if (p.b_kc) {
      const float4 v = k0 < p.K ? *reinterpret_cast<const float4*>(p.B + n * p.ldb + k0)
                                : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      bf[g][0] = v.x; bf[g][1] = v.y; bf[g][2] = v.z; bf[g][3] = v.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[g][j] = k0 + j < p.K ? p.B[(k0 + j) * p.ldb + n] : 0.0f;
    }
  }
}

// PLAIN: the GEMM epilogue is the identity (alpha == 1, no accumulate, bias or
// activation: 1 * x == x exactly), so accumulators are stored as they are.
template <int KG, bool CHAIN, bool PLAIN>
__global__ __launch_bounds__(kThreads) void skinny_outer(SkArgs p) {
  constexpr int kBA = OuterBAhead<KG>();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int q = lane >> 4, c = lane & 15;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * kOuterRows;
  const int64_t n0 = static_cast<int64_t>(blockIdx.y) * kOuterN + w * kOuterWN;
  if (n0 >= p.N) return;
  float af[kOuterRB][KG][4];
#pragma unroll
  for (int rb = 0; rb < kOuterRB; ++rb) {
    const int64_t m = std::min<int64_t>(m0 + 16 * rb + c, p.M - 1);
#pragma unroll
    for (int g = 0; g < KG; ++g) {
      const int64_t k0 = 16 * g + 4 * q;
      const float4 v = k0 < p.K ? *reinterpret_cast<const float4*>(p.A + m * p.lda + k0)
                                : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      af[rb][g][0] = v.x; af[rb][g][1] = v.y; af[rb][g][2] = v.z; af[rb][g][3] = v.w;
    }
  }
  // Per step: B fragments and (chain) the AddEW operand y. Columns past N
  // read column N-1, rows past M read row 0; neither is stored.
  float bf[kOuterSteps][KG][4];
  float yv[kOuterSteps][kOuterRB][4];
  auto load_b = [&](int st) {
    OuterLoadB<KG>(p, std::min<int64_t>(n0 + 16 * st + c, p.N - 1), q, bf[st]);
  };
  auto load_y = [&](int st) {
#pragma unroll
    for (int rb = 0; rb < kOuterRB; ++rb) {
      const int64_t mo = m0 + 16 * rb + c, n = n0 + 16 * st + 4 * q;
      const bool in = mo < p.M && n < p.N;
      const float4 v = *reinterpret_cast<const float4*>(p.Y + (in ? mo * p.N + n : 0));
      yv[st][rb][0] = v.x; yv[st][rb][1] = v.y; yv[st][rb][2] = v.z; yv[st][rb][3] = v.w;
    }
  };
#pragma unroll
  for (int st = 0; st < kBA && st < kOuterSteps; ++st) load_b(st);
  if constexpr (CHAIN)
#pragma unroll
    for (int st = 0; st < kOuterYAhead && st < kOuterSteps; ++st) load_y(st);
#pragma unroll
  for (int st = 0; st < kOuterSteps; ++st) {
    const int64_t nb = n0 + 16 * st;
    if (nb >= p.N) break;
    if (st + kBA < kOuterSteps) load_b(st + kBA);
    if constexpr (CHAIN)
      if (st + kOuterYAhead < kOuterSteps) load_y(st + kOuterYAhead);
    floatx4 acc[kOuterRB];
#pragma unroll
    for (int rb = 0; rb < kOuterRB; ++rb) acc[rb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < KG; ++g)
#pragma unroll
      for (int rb = 0; rb < kOuterRB; ++rb)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(bf[st][g][j], af[rb][g][j], acc[rb], 0, 0, 0);
    const int64_t n = nb + 4 * q;
    if (n < p.N) {
#pragma unroll
      for (int rb = 0; rb < kOuterRB; ++rb) {
        const int64_t mo = m0 + 16 * rb + c;
        if (mo >= p.M) continue;
        const float4 u =
            PLAIN ? make_float4(acc[rb][0], acc[rb][1], acc[rb][2], acc[rb][3])
                  : make_float4(Epilogue(p, mo, n + 0, acc[rb][0]), Epilogue(p, mo, n + 1, acc[rb][1]),
                                Epilogue(p, mo, n + 2, acc[rb][2]), Epilogue(p, mo, n + 3, acc[rb][3]));
        if (p.write_u) *reinterpret_cast<float4*>(p.C + mo * p.ldc + n) = u;
        if constexpr (CHAIN) {
          // The Scale and AddEW element expressions, in plan order.
          const int64_t at = mo * p.N + n;
          float4 v = u;
          if (p.chain == 1) {
            v = make_float4(p.chain_alpha * u.x, p.chain_alpha * u.y, p.chain_alpha * u.z,
                            p.chain_alpha * u.w);
            if (p.S) *reinterpret_cast<float4*>(p.S + at) = v;
          }
          const float* y = yv[st][rb];
          *reinterpret_cast<float4*>(p.Yout + at) =
              p.y_first ? make_float4(y[0] + v.x, y[1] + v.y, y[2] + v.z, y[3] + v.w)
                        : make_float4(v.x + y[0], v.y + y[1], v.z + y[2], v.w + y[3]);
        }
      }
    }
  }
}

// ---- rowdot (small N, A k-contiguous) -----------------------------------------

constexpr int kRowdotM = 16;
constexpr int kRowdotWaves = 8;   // wavefronts per workgroup, each a slice of K
// k groups per batch (the next batch is in flight), fewer for wider N to stay
// within the register file.
constexpr int RowdotUnroll(int nb) { return nb == 1 ? 4 : (nb == 2 ? 2 : 1); }

template <int NB>  // ceil(N / 16)
__global__ __launch_bounds__(64 * kRowdotWaves) void skinny_rowdot(SkArgs p) {
  constexpr int kRowdotUnroll = RowdotUnroll(NB);
  __shared__ floatx4 red[kRowdotWaves][NB][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int q = lane >> 4, c = lane & 15;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * kRowdotM;
  const int64_t m = std::min<int64_t>(m0 + c, p.M - 1);
  const int64_t ngroups = (p.K + 15) / 16;
  const int64_t per = (ngroups + kRowdotWaves - 1) / kRowdotWaves;
  const int64_t gb = w * per, ge = std::min<int64_t>(gb + per, ngroups);
  const float* arow = p.A + m * p.lda;
  int64_t ncol[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) ncol[nb] = std::min<int64_t>(16 * nb + c, p.N - 1);
  floatx4 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  auto load = [&](int64_t g, float4& a, float4 (&b)[NB]) {
    const int64_t k0 = 16 * g + 4 * q;
    const bool in = g < ge && k0 < p.K;  // K % 4 == 0: a float4 is wholly in or out
    a = in ? ScaleLoaded(p, *reinterpret_cast<const float4*>(arow + k0))
           : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if (p.b_kc) {
        b[nb] = in ? *reinterpret_cast<const float4*>(p.B + ncol[nb] * p.ldb + k0)
                   : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      } else {
        b[nb].x = in ? p.B[(k0 + 0) * p.ldb + ncol[nb]] : 0.0f;
        b[nb].y = in ? p.B[(k0 + 1) * p.ldb + ncol[nb]] : 0.0f;
        b[nb].z = in ? p.B[(k0 + 2) * p.ldb + ncol[nb]] : 0.0f;
        b[nb].w = in ? p.B[(k0 + 3) * p.ldb + ncol[nb]] : 0.0f;
      }
    }
  };
  float4 a[kRowdotUnroll], b[kRowdotUnroll][NB];
  float4 an[kRowdotUnroll], bn[kRowdotUnroll][NB];
#pragma unroll
  for (int u = 0; u < kRowdotUnroll; ++u) load(gb + u, a[u], b[u]);
  for (int64_t g = gb; g < ge; g += kRowdotUnroll) {
    if (g + kRowdotUnroll < ge)
#pragma unroll
      for (int u = 0; u < kRowdotUnroll; ++u) load(g + kRowdotUnroll + u, an[u], bn[u]);
#pragma unroll
    for (int u = 0; u < kRowdotUnroll; ++u)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].x, b[u][nb].x, acc[nb], 0, 0, 0);
        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].y, b[u][nb].y, acc[nb], 0, 0, 0);
        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].z, b[u][nb].z, acc[nb], 0, 0, 0);
        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].w, b[u][nb].w, acc[nb], 0, 0, 0);
      }
#pragma unroll
    for (int u = 0; u < kRowdotUnroll; ++u) {
      a[u] = an[u];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) b[u][nb] = bn[u][nb];
    }
  }
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) red[w][nb][lane] = acc[nb];
  __syncthreads();
  if (w != 0) return;
  // Lane (q, c) element i: C[m0 + 4q + i][16 nb + c]; wavefront partials in order.
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    floatx4 s = red[0][nb][lane];
#pragma unroll
    for (int ww = 1; ww < kRowdotWaves; ++ww) s += red[ww][nb][lane];
    const int64_t n = 16 * nb + c;
    if (n >= p.N) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t mo = m0 + 4 * q + i;
      if (mo < p.M) p.C[mo * p.ldc + n] = Epilogue(p, mo, n, s[i]);
    }
  }
}

// ---- rowdot group -------------------------------------------------------------
//
// NB rowdots over the same A (the LoRA down-projections of one layer input:
// t_nb = x A_nb), A read once. The layout and the per-output k order are the
// lone rowdot's (lane (q, c), wavefront K slices summed in order), so each
// member's output has the bits of its own launch; a workgroup takes RB
// blocks of 16 rows, so each of its B fragments serves RB row blocks.
template <int NB, int RB, int U>
__global__ __launch_bounds__(64 * kRowdotWaves) void skinny_rowdot_group(SkArgs p) {
  __shared__ floatx4 red[kRowdotWaves][RB][NB][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int q = lane >> 4, c = lane & 15;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * (16 * RB);
  const int64_t ngroups = (p.K + 15) / 16;
  const int64_t per = (ngroups + kRowdotWaves - 1) / kRowdotWaves;
  const int64_t gb = w * per, ge = std::min<int64_t>(gb + per, ngroups);
  const float* arow[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
    arow[rb] = p.A + std::min<int64_t>(m0 + 16 * rb + c, p.M - 1) * p.lda;
  const int64_t ncol = std::min<int64_t>(c, p.N - 1);
  floatx4 acc[RB][NB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[rb][nb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  auto load = [&](int64_t g, float4 (&a)[RB], float4 (&b)[NB]) {
    const int64_t k0 = 16 * g + 4 * q;
    const bool in = g < ge && k0 < p.K;  // K % 4 == 0: a float4 is wholly in or out
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      a[rb] = in ? *reinterpret_cast<const float4*>(arow[rb] + k0) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const float* B = p.Bm[nb];
      if (p.b_kc) {
        b[nb] = in ? *reinterpret_cast<const float4*>(B + ncol * p.ldb + k0)
                   : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      } else {
        b[nb].x = in ? B[(k0 + 0) * p.ldb + ncol] : 0.0f;
        b[nb].y = in ? B[(k0 + 1) * p.ldb + ncol] : 0.0f;
        b[nb].z = in ? B[(k0 + 2) * p.ldb + ncol] : 0.0f;
        b[nb].w = in ? B[(k0 + 3) * p.ldb + ncol] : 0.0f;
      }
    }
  };
  float4 a[U][RB], b[U][NB], an[U][RB], bn[U][NB];
#pragma unroll
  for (int u = 0; u < U; ++u) load(gb + u, a[u], b[u]);
  for (int64_t g = gb; g < ge; g += U) {
    if (g + U < ge)
#pragma unroll
      for (int u = 0; u < U; ++u) load(g + U + u, an[u], bn[u]);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          acc[rb][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u][rb].x, b[u][nb].x, acc[rb][nb], 0, 0, 0);
          acc[rb][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u][rb].y, b[u][nb].y, acc[rb][nb], 0, 0, 0);
          acc[rb][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u][rb].z, b[u][nb].z, acc[rb][nb], 0, 0, 0);
          acc[rb][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u][rb].w, b[u][nb].w, acc[rb][nb], 0, 0, 0);
        }
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) a[u][rb] = an[u][rb];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) b[u][nb] = bn[u][nb];
    }
  }
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) red[w][rb][nb][lane] = acc[rb][nb];
  __syncthreads();
  if (w != 0) return;
  // Lane (q, c) element i: row m0 + 16 rb + 4q + i, column c of member nb;
  // wavefront partials in order.
  if (c >= p.N) return;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      floatx4 s = red[0][rb][nb][lane];
#pragma unroll
      for (int ww = 1; ww < kRowdotWaves; ++ww) s += red[ww][rb][nb][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t mo = m0 + 16 * rb + 4 * q + i;
        if (mo < p.M) p.Cm[nb][mo * p.ldc + c] = s[i];
      }
    }
}

// ---- colsum (TN, small M or N) --------------------------------------------------
//
// P[w][n'] = sum_k X[k][w] Y[k][n'] with v_mfma_f32_16x16x4_f32: lane (q, c)
// loads the float4 X[k0 + q][w0 + 4c .. 4c + 3] (4 rows x 256 contiguous
// bytes per instruction) and Y[k0 + q][16 nb + c]; MFMA c4 takes component c4,
// so its row i is column w0 + 4i + c4. A wavefront owns 64 columns and a run
// of k quads (the next batch in flight); the workgroup's four wavefronts are
// summed in order through LDS into one partial per k-group.

constexpr int kColW = 64;  // columns w per workgroup

template <int NBN>  // ceil(R / 16)
__global__ __launch_bounds__(kThreads) void skinny_colsum(SkArgs p) {
  __shared__ floatx4 red[4][NBN][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int q = lane >> 4, c = lane & 15;
  const int64_t w0 = static_cast<int64_t>(blockIdx.x) * kColW;
  const int g = static_cast<int>(blockIdx.y);
  const float* X = p.big_is_m ? p.A : p.B;  // X[k][w]
  const float* Y = p.big_is_m ? p.B : p.A;  // Y[k][n']
  const int64_t ldx = p.big_is_m ? p.lda : p.ldb;
  const int64_t ldy = p.big_is_m ? p.ldb : p.lda;
  const int64_t kb0 = static_cast<int64_t>(g) * p.k_per_group;
  const int64_t ke0 = std::min<int64_t>(p.K, kb0 + p.k_per_group);
  const int64_t span = ke0 > kb0 ? ke0 - kb0 : 0;
  const int64_t sub = ((span + 15) / 16) * 4;  // k per wavefront, whole quads
  const int64_t kb = kb0 + w * sub, ke = std::min<int64_t>(ke0, kb + sub);
  const int64_t wl = w0 + 4 * c;
  const bool w_ok = wl < p.W;  // W % 4 == 0: the float4 is wholly in or out
  floatx4 acc[4][NBN];
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
    for (int nb = 0; nb < NBN; ++nb) acc[c4][nb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int U = 4;  // k quads per batch; the next batch is in flight
  auto load = [&](int64_t k4, float4 (&x)[U], float (&y)[U][NBN]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k = k4 + 4 * u + q;
      const bool kin = k < ke;
      x[u] = kin && w_ok ? ScaleLoaded(p, *reinterpret_cast<const float4*>(X + k * ldx + wl))
                         : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) {
        const int64_t n = 16 * nb + c;
        y[u][nb] = kin && n < p.R ? Y[k * ldy + n] : 0.0f;
      }
    }
  };
  float4 x[U], xn[U];
  float y[U][NBN], yn[U][NBN];
  load(kb, x, y);
  for (int64_t k4 = kb; k4 < ke; k4 += 4 * U) {
    if (k4 + 4 * U < ke) load(k4 + 4 * U, xn, yn);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) {
        acc[0][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[u].x, y[u][nb], acc[0][nb], 0, 0, 0);
        acc[1][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[u].y, y[u][nb], acc[1][nb], 0, 0, 0);
        acc[2][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[u].z, y[u][nb], acc[2][nb], 0, 0, 0);
        acc[3][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[u].w, y[u][nb], acc[3][nb], 0, 0, 0);
      }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      x[u] = xn[u];
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) y[u][nb] = yn[u][nb];
    }
  }
  // Wavefront partials summed in order 0 + 1 + 2 + 3 through LDS.
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4) {
    __syncthreads();
    if (w != 0)
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) red[w][nb][lane] = acc[c4][nb];
    __syncthreads();
    if (w == 0)
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) {
        acc[c4][nb] += red[1][nb][lane];
        acc[c4][nb] += red[2][nb][lane];
        acc[c4][nb] += red[3][nb][lane];
      }
  }
  if (w != 0) return;
  // Element i of acc[c4][nb] at lane (q, c): w = w0 + 4*(4q + i) + c4, n' = 16 nb + c.
  // Partial layout: ws[g][w][n'].
  float* part = p.ws + static_cast<int64_t>(g) * p.W * p.R;
#pragma unroll
  for (int nb = 0; nb < NBN; ++nb) {
    const int64_t n = 16 * nb + c;
    if (n >= p.R) continue;
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t wi = w0 + 4 * (4 * q + i) + c4;
        if (wi < p.W) part[wi * p.R + n] = acc[c4][nb][i];
      }
  }
}

// Sums the k-group partials in group order and writes C with the epilogue.
// Thread t owns outputs 4t .. 4t + 3 of the [W, R] partial layout (R % 4 == 0
// here, so they share one w); the group loads are issued four at a time.
__global__ __launch_bounds__(kThreads) void skinny_colsum_finish(SkArgs p) {
  const int64_t total = p.W * p.R, nq = total / 4;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; t < nq; t += stride) {
    float4 s = *reinterpret_cast<const float4*>(p.ws + 4 * t);
    int g = 1;
    for (; g + 3 < p.groups; g += 4) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        v[u] = *reinterpret_cast<const float4*>(p.ws + static_cast<int64_t>(g + u) * total + 4 * t);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        s.x += v[u].x;
        s.y += v[u].y;
        s.z += v[u].z;
        s.w += v[u].w;
      }
    }
    for (; g < p.groups; ++g) {
      const float4 v = *reinterpret_cast<const float4*>(p.ws + static_cast<int64_t>(g) * total + 4 * t);
      s.x += v.x;
      s.y += v.y;
      s.z += v.z;
      s.w += v.w;
    }
    const float sv[4] = {s.x, s.y, s.z, s.w};
    const int64_t wi = (4 * t) / p.R, n0 = (4 * t) % p.R;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t m = p.big_is_m ? wi : n0 + e, nn = p.big_is_m ? n0 + e : wi;
      p.C[m * p.ldc + nn] = Epilogue(p, m, nn, sv[e]);
    }
  }
}

// Reference order of the group sum for R % 4 != 0: one output per thread.
__global__ __launch_bounds__(kThreads) void skinny_colsum_finish1(SkArgs p) {
  const int64_t total = p.W * p.R;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; idx < total;
       idx += stride) {
    float s = p.ws[idx];
    for (int g = 1; g < p.groups; ++g) s += p.ws[static_cast<int64_t>(g) * total + idx];
    const int64_t wi = idx / p.R, n = idx % p.R;
    const int64_t m = p.big_is_m ? wi : n, nn = p.big_is_m ? n : wi;
    p.C[m * p.ldc + nn] = Epilogue(p, m, nn, s);
  }
}

// ---- colsum group ---------------------------------------------------------------
//
// NB colsums over the same large operand X (the LoRA dA_j = x^T dt_j of one
// layer input), X read once: member nb's small operand is Bm[nb] (its rank
// <= 16 wide, ldy shared) and its output Cm[nb]. The k-groups, the
// wavefronts' k ranges, the quad order and the group-order sum of the
// partials are those of skinny_colsum and its finish, so every member's
// output has the bits of its own launch. Partial layout: ws[g][w][16 nb + n].

template <int NB>
__global__ __launch_bounds__(kThreads) void skinny_colsum_group(SkArgs p) {
  __shared__ floatx4 red[4][NB][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int q = lane >> 4, c = lane & 15;
  const int64_t w0 = static_cast<int64_t>(blockIdx.x) * kColW;
  const int g = static_cast<int>(blockIdx.y);
  const float* X = p.big_is_m ? p.A : p.B;  // X[k][w]
  const int64_t ldx = p.big_is_m ? p.lda : p.ldb;
  const int64_t ldy = p.big_is_m ? p.ldb : p.lda;
  const int64_t kb0 = static_cast<int64_t>(g) * p.k_per_group;
  const int64_t ke0 = std::min<int64_t>(p.K, kb0 + p.k_per_group);
  const int64_t span = ke0 > kb0 ? ke0 - kb0 : 0;
  const int64_t sub = ((span + 15) / 16) * 4;  // k per wavefront, whole quads
  const int64_t kb = kb0 + w * sub, ke = std::min<int64_t>(ke0, kb + sub);
  const int64_t wl = w0 + 4 * c;
  const bool w_ok = wl < p.W;
  const bool n_ok = c < p.R;
  floatx4 acc[4][NB];
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[c4][nb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int U = 4;  // k quads per batch; the next batch is in flight
  auto load = [&](int64_t k4, float4 (&x)[U], float (&y)[U][NB]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k = k4 + 4 * u + q;
      const bool kin = k < ke;
      x[u] = kin && w_ok ? *reinterpret_cast<const float4*>(X + k * ldx + wl)
                         : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) y[u][nb] = kin && n_ok ? p.Bm[nb][k * ldy + c] : 0.0f;
    }
  };
  float4 x[U], xn[U];
  float y[U][NB], yn[U][NB];
  load(kb, x, y);
  for (int64_t k4 = kb; k4 < ke; k4 += 4 * U) {
    if (k4 + 4 * U < ke) load(k4 + 4 * U, xn, yn);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        acc[0][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[u].x, y[u][nb], acc[0][nb], 0, 0, 0);
        acc[1][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[u].y, y[u][nb], acc[1][nb], 0, 0, 0);
        acc[2][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[u].z, y[u][nb], acc[2][nb], 0, 0, 0);
        acc[3][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[u].w, y[u][nb], acc[3][nb], 0, 0, 0);
      }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      x[u] = xn[u];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) y[u][nb] = yn[u][nb];
    }
  }
  // Wavefront partials summed in order 0 + 1 + 2 + 3 through LDS.
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4) {
    __syncthreads();
    if (w != 0)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) red[w][nb][lane] = acc[c4][nb];
    __syncthreads();
    if (w == 0)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        acc[c4][nb] += red[1][nb][lane];
        acc[c4][nb] += red[2][nb][lane];
        acc[c4][nb] += red[3][nb][lane];
      }
  }
  if (w != 0 || !n_ok) return;
  constexpr int RT = 16 * NB;  // partial row width
  float* part = p.ws + static_cast<int64_t>(g) * p.W * RT;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t wi = w0 + 4 * (4 * q + i) + c4;
        if (wi < p.W) part[wi * RT + 16 * nb + c] = acc[c4][nb][i];
      }
}

// The group's partials summed in group order, one output per thread
// (skinny_colsum_finish's order).
template <int NB>
__global__ __launch_bounds__(kThreads) void skinny_colsum_group_finish(SkArgs p) {
  constexpr int RT = 16 * NB;
  const int64_t total = p.W * RT;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; idx < total;
       idx += stride) {
    const int64_t wi = idx / RT;
    const int nb = static_cast<int>((idx % RT) / 16), n = static_cast<int>(idx % 16);
    if (n >= p.R) continue;
    float s = p.ws[idx];
    for (int g = 1; g < p.groups; ++g) s += p.ws[static_cast<int64_t>(g) * total + idx];
    const int64_t m = p.big_is_m ? wi : n, nn = p.big_is_m ? n : wi;
    p.Cm[nb][m * p.ldc + nn] = s;
  }
}

// ---- dual: rowdot and colsum over one stream ---------------------------------
//
// The LoRA backward streams du twice: dt = du B^T (rowdot) and dB = t^T du
// (colsum). This pass reads the [T, D] stream X once for both. A workgroup
// owns a tile of 128 rows x 256 columns; wavefront w owns its 64 columns
// over all 128 rows, eight strips of 16 rows (32 KB), and keeps six strips'
// loads in flight (each strip's registers are reloaded as soon as it is
// used), so nearly the whole stream is requested at entry:
//  * colsum: lane (q, c) holds X[row 4u + q][4c .. 4c + 3] of the strip's
//    quad u; MFMA c4 takes component c4 against the Y values of those rows
//    (staged in LDS once per workgroup), rows in order;
//  * rowdot: the wavefront writes the strip to its own LDS buffer and reads
//    it back transposed (lane (q, c): row c, columns 16g + 4q .. + 3), so
//    the MFMAs contract over its 64 columns with no workgroup barrier; the
//    four wavefronts' partials are summed in wavefront order at the end.
// Partials go to the workspace: one per 256-column block for each dt row,
// one per 128-row block for each dB column; skinny_dual_finish sums them in
// a fixed order (below) and applies each output's epilogue. Either output may be
// left out (the engine's one-instruction form); each output's summation
// order is the same either way, so the pair and its two single launches
// give the same bits.

constexpr int kDualRows = 128;  // rows per workgroup
constexpr int kDualCols = 256;  // columns per workgroup (4 wavefronts x 64)
constexpr int kDualR = 16;      // partial stride: outputs per row / column
constexpr int kDualStrip = 16;  // rows per strip (one rowdot MFMA block)
constexpr int kDualStrips = kDualRows / kDualStrip;
constexpr int kDualTs = 68;     // floats per row of a wavefront's transpose buffer
constexpr int kDualAhead = 6;   // strips of loads in flight per wavefront

struct DualArgs {
  const float* X;
  int64_t ldx, T, D;
  int scale_stream;
  float stream_scale;
  // rowdot: Crd(row, n) = epi(sum_d X[row][d] Bf[n * ldb + d]), n < r_rd
  int r_rd;
  const float* Bf;
  int64_t ldb;
  float* Crd;
  int64_t ldc_rd;
  float alpha_rd;
  int acc_rd;
  const float* bias_rd;
  int act_rd;
  // colsum: C at (w = d, n') = epi(sum_row X[row][d] Y[row][n']), n' < r_cs;
  // stored at C[w * ldc + n'] when big_is_m, else C[n' * ldc + w]
  int r_cs;
  const float* Y;
  int64_t ldy;
  float* Ccs;
  int64_t ldc_cs;
  int big_is_m;
  float alpha_cs;
  int acc_cs;
  const float* bias_cs;
  int act_cs;
  float* ws_rd;  // [ncb][T][16]
  float* ws_cs;  // [nrb][D][16]
  int64_t ncb, nrb;
};

__device__ __forceinline__ float DualEpi(float acc, float alpha, int accumulate, const float* C,
                                         int64_t at, const float* bias, int64_t col, int act) {
  float val = alpha * acc;
  if (accumulate) val = C[at] + val;
  if (bias) val = val + bias[col];
  return dev_act(act, val);
}

// One workgroup's tile. EDGE: the tile reaches past T or D, and each value
// is masked (and scaled) where used; inside, every loaded value is kept, so
// the masks are left out, and SCALED multiplies by the folded Scale's
// factor (the same float product).
template <bool RD, bool CS, bool EDGE, bool SCALED>
__device__ __forceinline__ void DualTile(const DualArgs& p, float* __restrict__ ty,
                                         float* __restrict__ tb, float* __restrict__ rdl) {
  constexpr int kPerThread = kDualRows * kDualR / kThreads;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int q = lane >> 4, c = lane & 15;
  // Column blocks vary fastest: neighbouring workgroups read whole rows.
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * kDualRows;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kDualCols;
  const int64_t wl = c0 + 64 * w + 4 * c;  // this lane's four colsum columns
  const bool w_ok = wl < p.D;               // D % 4 == 0: wholly in or out
  // Every load is unconditional, from an address clamped into its operand,
  // so they issue back to back; rows past T, columns past D and ranks past
  // the rank are zeroed (and the stream scaled) where the values are used.
  const int64_t wlc = w_ok ? wl : 0;
  float yv[CS ? kPerThread : 1];
  if constexpr (CS) {
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
      const int i = static_cast<int>(threadIdx.x) + k * kThreads;
      const int64_t row = min<int64_t>(r0 + (i >> 4), p.T - 1);
      yv[k] = p.Y[row * p.ldy + min(i & 15, p.r_cs - 1)];
    }
  }
  // Rowdot B fragments of the wavefront's columns: Bf(n = c, 64w + 16g + 4q + j).
  float4 bf[4];
  if constexpr (RD) {
    const int cb = min(c, p.r_rd - 1);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int64_t kc = min<int64_t>(c0 + 64 * w + 16 * g + 4 * q, p.D - 4);
      bf[g] = *reinterpret_cast<const float4*>(p.Bf + cb * p.ldb + kc);
    }
  }
  // The wavefront's stream, kDualAhead strips in flight: strip s, quad u
  // holds row 16s + 4u + q.
  float4 x[kDualStrips][4];
  auto load_strip = [&](int s) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t row = min<int64_t>(r0 + kDualStrip * s + 4 * u + q, p.T - 1);
      x[s][u] = *reinterpret_cast<const float4*>(p.X + row * p.ldx + wlc);
    }
  };
#pragma unroll
  for (int s = 0; s < kDualAhead; ++s) load_strip(s);
  if constexpr (RD) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const bool keep = static_cast<int>(c < p.r_rd) & static_cast<int>(c0 + 64 * w + 16 * g + 4 * q < p.D);
      bf[g] = Keep4(bf[g], keep, 1.0f);
    }
  }
  if constexpr (CS) {
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
      const int i = static_cast<int>(threadIdx.x) + k * kThreads;
      const bool keep = static_cast<int>(r0 + (i >> 4) < p.T) & static_cast<int>((i & 15) < p.r_cs);
      ty[i] = __uint_as_float(__float_as_uint(yv[k]) & (0u - static_cast<unsigned>(keep)));
    }
    __syncthreads();
  }
  floatx4 cs[4];
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4) cs[c4] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  float* buf = tb + w * kDualStrip * kDualTs;
  const float sc = p.scale_stream ? p.stream_scale : 1.0f;  // x * 1 is x, bit for bit
#pragma unroll
  for (int s = 0; s < kDualStrips; ++s) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if constexpr (EDGE) {
        const bool keep = static_cast<int>(r0 + kDualStrip * s + 4 * u + q < p.T) & static_cast<int>(w_ok);
        v[u] = Keep4(x[s][u], keep, sc);
      } else if constexpr (SCALED) {
        v[u] = make_float4(sc * x[s][u].x, sc * x[s][u].y, sc * x[s][u].z, sc * x[s][u].w);
      } else {
        v[u] = x[s][u];
      }
    }
    if (s + kDualAhead < kDualStrips) load_strip(s + kDualAhead);  // into the registers just freed
    if constexpr (CS) {
      // Row quads in order; MFMA c4 takes column component c4 (as skinny_colsum).
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float y = ty[(kDualStrip * s + 4 * u + q) * kDualR + c];
        cs[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(v[u].x, y, cs[0], 0, 0, 0);
        cs[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(v[u].y, y, cs[1], 0, 0, 0);
        cs[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(v[u].z, y, cs[2], 0, 0, 0);
        cs[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(v[u].w, y, cs[3], 0, 0, 0);
      }
    }
    if constexpr (RD) {
      // The strip through the wavefront's own buffer, read back by other
      // lanes as rows of the MFMA's A operand. A wavefront's LDS operations
      // execute in issue order, so no workgroup barrier is needed; the wave
      // barriers keep the compiler from moving the reads above the writes,
      // or the next strip's writes above these reads (different addresses
      // per lane, so alias analysis alone would allow either).
#pragma unroll
      for (int u = 0; u < 4; ++u)
        *reinterpret_cast<float4*>(&buf[(4 * u + q) * kDualTs + 4 * c]) = v[u];
      __builtin_amdgcn_wave_barrier();
      floatx4 rd = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 a = *reinterpret_cast<const float4*>(&buf[c * kDualTs + 16 * g + 4 * q]);
        rd = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, bf[g].x, rd, 0, 0, 0);
        rd = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, bf[g].y, rd, 0, 0, 0);
        rd = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, bf[g].z, rd, 0, 0, 0);
        rd = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, bf[g].w, rd, 0, 0, 0);
      }
      __builtin_amdgcn_wave_barrier();
      // Lane (q, c) element e: strip row 4q + e, n = c.
#pragma unroll
      for (int e = 0; e < 4; ++e)
        rdl[(w * kDualRows + kDualStrip * s + 4 * q + e) * kDualR + c] = rd[e];
    }
  }
  if constexpr (RD) {
    __syncthreads();
    // The tile's dt partial: the four wavefronts' column partials in order.
    float* part = p.ws_rd + (static_cast<int64_t>(blockIdx.x) * p.T) * kDualR;
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
      const int i = static_cast<int>(threadIdx.x) + k * kThreads;
      const int rr = i >> 4, n = i & 15;
      float sum = rdl[rr * kDualR + n] + rdl[(kDualRows + rr) * kDualR + n];
      sum = sum + rdl[(2 * kDualRows + rr) * kDualR + n];
      sum = sum + rdl[(3 * kDualRows + rr) * kDualR + n];
      const int64_t row = r0 + rr;
      if (row < p.T) part[row * kDualR + n] = sum;
    }
  }
  if constexpr (CS) {
    // Element e of cs[c4] at lane (q, c): column c0 + 64w + 4(4q + e) + c4, n' = c.
    float* part = p.ws_cs + (static_cast<int64_t>(blockIdx.y) * p.D) * kDualR;
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t col = c0 + 64 * w + 4 * (4 * q + e) + c4;
        if (col < p.D) part[col * kDualR + c] = cs[c4][e];
      }
  }
}

template <bool RD, bool CS>
__global__ __launch_bounds__(kThreads, 2) void skinny_dual(DualArgs p) {
  __shared__ __align__(16) float ty[CS ? kDualRows * kDualR : 4];       // Y rows of the tile
  __shared__ __align__(16) float tb[RD ? 4 * kDualStrip * kDualTs : 4];  // per-wavefront transpose
  __shared__ __align__(16) float rdl[RD ? 4 * kDualRows * kDualR : 4];   // per-wavefront dt partials
  const bool edge = (static_cast<int64_t>(blockIdx.y) + 1) * kDualRows > p.T ||
                    (static_cast<int64_t>(blockIdx.x) + 1) * kDualCols > p.D;
  if (edge)
    DualTile<RD, CS, true, true>(p, ty, tb, rdl);
  else if (p.scale_stream)
    DualTile<RD, CS, false, true>(p, ty, tb, rdl);
  else
    DualTile<RD, CS, false, false>(p, ty, tb, rdl);
}

// Sum of n partials src[0], src[stride], .. in index order, loaded 16 at a
// time so each batch's loads are in flight together.
__device__ __forceinline__ float SumPartials(const float* __restrict__ src, int64_t n, int64_t stride) {
  float s = src[0];
  for (int64_t b0 = 1; b0 < n; b0 += 16) {
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = b0 + u < n ? src[(b0 + u) * stride] : 0.0f;
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (b0 + u < n) s += v[u];
  }
  return s;
}

constexpr int kDualSubs = 8;                     // threads per dB output in the finish
constexpr int kDualOuts = kThreads / kDualSubs;  // dB outputs per finish workgroup

// Sums the partials and applies each output's epilogue. The first
// `rd_blocks` workgroups take the dt outputs, one thread each, its ncb
// partials in block order. The rest take kDualOuts dB outputs each, with
// kDualSubs threads per output: thread `sub` sums its run of consecutive
// row blocks in order (all its loads in flight at once), and the runs' sums
// are added in run order.
template <bool RD, bool CS>
__global__ __launch_bounds__(kThreads) void skinny_dual_finish(DualArgs p, int64_t rd_blocks) {
  if (RD && static_cast<int64_t>(blockIdx.x) < rd_blocks) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (idx >= p.T * p.r_rd) return;
    const int64_t row = idx / p.r_rd, n = idx % p.r_rd;
    const float s = SumPartials(p.ws_rd + row * kDualR + n, p.ncb, p.T * kDualR);
    const int64_t at = row * p.ldc_rd + n;
    p.Crd[at] = DualEpi(s, p.alpha_rd, p.acc_rd, p.Crd, at, p.bias_rd, n, p.act_rd);
    return;
  }
  if constexpr (CS) {
    __shared__ float runs[kDualSubs][kDualOuts];
    const int o = static_cast<int>(threadIdx.x) % kDualOuts;
    const int sub = static_cast<int>(threadIdx.x) / kDualOuts;
    const int64_t j = (static_cast<int64_t>(blockIdx.x) - (RD ? rd_blocks : 0)) * kDualOuts + o;
    const bool out_ok = j < p.D * p.r_cs;
    const int64_t jc = out_ok ? j : 0;
    const int64_t col = jc / p.r_cs, n = jc % p.r_cs;
    const int64_t per = (p.nrb + kDualSubs - 1) / kDualSubs;
    const int64_t b0 = sub * per, nb = min<int64_t>(p.nrb - b0, per);
    if (nb > 0)
      runs[sub][o] = SumPartials(p.ws_cs + (b0 * p.D + col) * kDualR + n, nb, p.D * kDualR);
    __syncthreads();
    if (sub == 0 && out_ok) {
      float s = runs[0][o];
      for (int k = 1; k < kDualSubs && k * per < p.nrb; ++k) s += runs[k][o];
      const int64_t m = p.big_is_m ? col : n, nn = p.big_is_m ? n : col;
      const int64_t at = m * p.ldc_cs + nn;
      p.Ccs[at] = DualEpi(s, p.alpha_cs, p.acc_cs, p.Ccs, at, p.bias_cs, nn, p.act_cs);
    }
  }
}

bool Vec4(const void* base, int64_t ld) { return aligned16(base) && ld % 4 == 0; }

int64_t ColsumGroups(int64_t W, int64_t K) {
  const int64_t wtiles = (W + kColW - 1) / kColW;
  const int64_t want = std::max<int64_t>(1, (512 + wtiles - 1) / wtiles);
  return std::max<int64_t>(1, std::min<int64_t>(want, std::min<int64_t>(K / 128, 64)));
}

}  // namespace

const void* SkinnyStream(const GemmDesc& d, int64_t* elems) {
  switch (SkinnyKindOf(d)) {
    case SkinnyKind::kRowDot:
      *elems = d.M * d.K;
      return d.A;
    case SkinnyKind::kColSum: {
      const bool big_is_m = d.N <= 64 && d.M >= 128;  // as LaunchSkinnyImpl
      *elems = d.K * (big_is_m ? d.M : d.N);
      return big_is_m ? d.A : d.B;
    }
    default:
      *elems = 0;
      return nullptr;
  }
}

SkinnyKind SkinnyKindOf(const GemmDesc& d) {
  if (d.batch != 1 || d.heads != 1 || d.causal != Causal::kNone || d.b_int8) return SkinnyKind::kNone;
  if (d.M <= 0 || d.N <= 0 || d.K <= 0) return SkinnyKind::kNone;
  if (d.M > (int64_t{1} << 40) || d.N > (int64_t{1} << 40)) return SkinnyKind::kNone;
  const float* A = static_cast<const float*>(d.A);
  const float* B = static_cast<const float*>(d.B);
  if (d.a_kc) {
    const bool b_ok = !d.b_kc || Vec4(B, d.ldb);
    if (!Vec4(A, d.lda) || d.K % 4 != 0 || !b_ok) return SkinnyKind::kNone;
    // small K: the output C is the stream
    if (d.K <= 64 && d.M >= 64 && d.N >= 64 && d.N % 4 == 0 && Vec4(d.C, d.ldc))
      return SkinnyKind::kOuter;
    // small N: A is the stream
    if (d.N <= 64 && d.K >= 256 && d.M >= 64) return SkinnyKind::kRowDot;
    return SkinnyKind::kNone;
  }
  if (!d.b_kc && d.K >= 256) {
    // TN: A(m,k) = A[k*lda + m], B(k,n) = B[k*ldb + n]
    if (d.N <= 64 && d.M >= 128 && d.M % 4 == 0 && Vec4(A, d.lda)) return SkinnyKind::kColSum;
    if (d.M <= 64 && d.N >= 128 && d.N % 4 == 0 && Vec4(B, d.ldb)) return SkinnyKind::kColSum;
  }
  return SkinnyKind::kNone;
}

const char* SkinnyKindName(SkinnyKind k) {
  switch (k) {
    case SkinnyKind::kOuter: return "skinny/outer";
    case SkinnyKind::kRowDot: return "skinny/rowdot";
    case SkinnyKind::kColSum: return "skinny/colsum";
    default: return "skinny/none";
  }
}

size_t SkinnyWorkspace(const GemmDesc& d) {
  if (SkinnyKindOf(d) != SkinnyKind::kColSum) return 0;
  const bool big_m = d.N <= 64 && d.M >= 128;
  const int64_t W = big_m ? d.M : d.N, R = big_m ? d.N : d.M;
  return static_cast<size_t>(ColsumGroups(W, d.K)) * W * R * sizeof(float);
}

bool SkinnyDualFits(const GemmDesc& rd, const GemmDesc& cs) {
  if (SkinnyKindOf(rd) != SkinnyKind::kRowDot || SkinnyKindOf(cs) != SkinnyKind::kColSum)
    return false;
  int64_t elems = 0;
  if (SkinnyStream(cs, &elems) != rd.A || elems != rd.M * rd.K) return false;
  const bool big_is_m = cs.N <= 64 && cs.M >= 128;
  const int64_t W = big_is_m ? cs.M : cs.N, R = big_is_m ? cs.N : cs.M;
  const int64_t ldx = big_is_m ? cs.lda : cs.ldb;
  if (cs.K != rd.M || W != rd.K || ldx != rd.lda) return false;
  if (rd.N > kDualR || R > kDualR) return false;
  // dt = du B^T: B's rows are the rank's (GemmNT, 16-byte aligned rows).
  if (!rd.b_kc || !Vec4(rd.B, rd.ldb)) return false;
  if (rd.scale_stream != cs.scale_stream || (rd.scale_stream && rd.stream_scale != cs.stream_scale))
    return false;
  const int64_t nrb = (rd.M + kDualRows - 1) / kDualRows, ncb = (rd.K + kDualCols - 1) / kDualCols;
  return ncb <= 0x7FFFFFFF && nrb <= 65535;
}

size_t SkinnyDualWorkspace(const GemmDesc& rd) {
  const int64_t nrb = (rd.M + kDualRows - 1) / kDualRows, ncb = (rd.K + kDualCols - 1) / kDualCols;
  return static_cast<size_t>(ncb * rd.M + nrb * rd.K) * kDualR * sizeof(float);
}

Status LaunchSkinnyDual(const GemmDesc& rd, const GemmDesc& cs, int which, const Ctx& ctx) {
  if (!SkinnyDualFits(rd, cs) || which < 1 || which > 3)
    return Status::Fail(kUnitEngine, "Gemm: the pair does not fit the dual skinny pass");
  const size_t need = SkinnyDualWorkspace(rd);
  if (ctx.ws_bytes < need || !aligned16(ctx.ws))
    return Status::Fail(kUnitEngine, "Gemm: workspace too small for the dual skinny pass");
  DualArgs a{};
  a.X = static_cast<const float*>(rd.A);
  a.ldx = rd.lda;
  a.T = rd.M;
  a.D = rd.K;
  a.scale_stream = rd.scale_stream ? 1 : 0;
  a.stream_scale = rd.stream_scale;
  a.r_rd = static_cast<int>(rd.N);
  a.Bf = static_cast<const float*>(rd.B);
  a.ldb = rd.ldb;
  a.Crd = rd.C;
  a.ldc_rd = rd.ldc;
  a.alpha_rd = rd.alpha;
  a.acc_rd = rd.accumulate ? 1 : 0;
  a.bias_rd = rd.bias;
  a.act_rd = rd.act;
  a.big_is_m = (cs.N <= 64 && cs.M >= 128) ? 1 : 0;
  a.r_cs = static_cast<int>(a.big_is_m ? cs.N : cs.M);
  a.Y = static_cast<const float*>(a.big_is_m ? cs.B : cs.A);
  a.ldy = a.big_is_m ? cs.ldb : cs.lda;
  a.Ccs = cs.C;
  a.ldc_cs = cs.ldc;
  a.alpha_cs = cs.alpha;
  a.acc_cs = cs.accumulate ? 1 : 0;
  a.bias_cs = cs.bias;
  a.act_cs = cs.act;
  a.nrb = (a.T + kDualRows - 1) / kDualRows;
  a.ncb = (a.D + kDualCols - 1) / kDualCols;
  a.ws_rd = static_cast<float*>(ctx.ws);
  a.ws_cs = a.ws_rd + a.ncb * a.T * kDualR;
  const dim3 grid(static_cast<unsigned>(a.ncb), static_cast<unsigned>(a.nrb));
  const int64_t rd_blocks = which & 1 ? (a.T * a.r_rd + kThreads - 1) / kThreads : 0;
  const int64_t cs_blocks = which & 2 ? (a.D * a.r_cs + kDualOuts - 1) / kDualOuts : 0;
  if (rd_blocks + cs_blocks > 0x7FFFFFFF)
    return Status::Fail(kUnitEngine, "Gemm: the dual skinny pass's outputs exceed one grid");
  const dim3 fgrid(static_cast<unsigned>(rd_blocks + cs_blocks));
  switch (which) {
    case 1:
      hipLaunchKernelGGL((skinny_dual<true, false>), grid, dim3(kThreads), 0, ctx.stream, a);
      if (Status s = LaunchStatus("Gemm(skinny dual)"); !s) return s;
      hipLaunchKernelGGL((skinny_dual_finish<true, false>), fgrid, dim3(kThreads), 0, ctx.stream, a, rd_blocks);
      break;
    case 2:
      hipLaunchKernelGGL((skinny_dual<false, true>), grid, dim3(kThreads), 0, ctx.stream, a);
      if (Status s = LaunchStatus("Gemm(skinny dual)"); !s) return s;
      hipLaunchKernelGGL((skinny_dual_finish<false, true>), fgrid, dim3(kThreads), 0, ctx.stream, a, rd_blocks);
      break;
    default:
      hipLaunchKernelGGL((skinny_dual<true, true>), grid, dim3(kThreads), 0, ctx.stream, a);
      if (Status s = LaunchStatus("Gemm(skinny dual)"); !s) return s;
      hipLaunchKernelGGL((skinny_dual_finish<true, true>), fgrid, dim3(kThreads), 0, ctx.stream, a, rd_blocks);
      break;
  }
  return LaunchStatus("Gemm(skinny dual finish)");
}

bool SkinnyColsumGroupFits(const GemmDesc* ds, int n) {
  if (n < 2 || n > 4) return false;
  const GemmDesc& d = ds[0];
  if (SkinnyKindOf(d) != SkinnyKind::kColSum) return false;
  const bool big_m = d.N <= 64 && d.M >= 128;
  for (int j = 0; j < n; ++j) {
    const GemmDesc& e = ds[j];
    const bool em = e.N <= 64 && e.M >= 128;
    if (SkinnyKindOf(e) != SkinnyKind::kColSum || em != big_m || e.M != d.M || e.N != d.N ||
        e.K != d.K || e.lda != d.lda || e.ldb != d.ldb || e.ldc != d.ldc ||
        e.alpha != 1.0f || e.accumulate || e.bias || e.act != 0 || e.scale_stream || !e.C)
      return false;
    // the large operand is shared; the rank-wide one is the member's own
    if (big_m ? (e.A != d.A || !e.B) : (e.B != d.B || !e.A)) return false;
    if ((big_m ? d.N : d.M) > 16) return false;
  }
  return true;
}

size_t SkinnyColsumGroupWorkspace(const GemmDesc* ds, int n) {
  const GemmDesc& d = ds[0];
  const bool big_m = d.N <= 64 && d.M >= 128;
  const int64_t W = big_m ? d.M : d.N;
  return static_cast<size_t>(ColsumGroups(W, d.K)) * W * 16 * n * sizeof(float);
}

Status LaunchSkinnyColsumGroup(const GemmDesc* ds, int n, const Ctx& ctx) {
  if (!SkinnyColsumGroupFits(ds, n))
    return Status::Fail(kUnitEngine, "Gemm: the colsums do not form a group");
  if (ctx.ws_bytes < SkinnyColsumGroupWorkspace(ds, n))
    return Status::Fail(kUnitEngine, "Gemm: workspace too small for the colsum group");
  const GemmDesc& d = ds[0];
  SkArgs a{};
  a.big_is_m = (d.N <= 64 && d.M >= 128) ? 1 : 0;
  a.A = static_cast<const float*>(d.A);
  a.B = static_cast<const float*>(d.B);
  a.M = d.M; a.N = d.N; a.K = d.K;
  a.lda = d.lda; a.ldb = d.ldb; a.ldc = d.ldc;
  a.alpha = 1.0f;
  a.ws = static_cast<float*>(ctx.ws);
  a.W = a.big_is_m ? d.M : d.N;
  a.R = a.big_is_m ? d.N : d.M;
  // The rank-wide operand of member j: B when the large one is A, else A.
  for (int j = 0; j < n; ++j) {
    a.Bm[j] = static_cast<const float*>(a.big_is_m ? ds[j].B : ds[j].A);
    a.Cm[j] = ds[j].C;
  }
  a.groups = static_cast<int>(ColsumGroups(a.W, d.K));
  a.k_per_group = (d.K + a.groups - 1) / a.groups;
  const int64_t gx = (a.W + kColW - 1) / kColW;
  if (gx > 0x7FFFFFFF) return Status::Fail(kUnitEngine, "Gemm: grid exceeds launch limits");
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(a.groups));
  const dim3 fgrid(grid_for(static_cast<size_t>(a.W * 16 * n), kThreads, 4096));
  switch (n) {
    case 2:
      hipLaunchKernelGGL(skinny_colsum_group<2>, grid, dim3(kThreads), 0, ctx.stream, a);
      if (Status s = LaunchStatus("Gemm(skinny colsum group)"); !s) return s;
      hipLaunchKernelGGL(skinny_colsum_group_finish<2>, fgrid, dim3(kThreads), 0, ctx.stream, a);
      break;
    case 3:
      hipLaunchKernelGGL(skinny_colsum_group<3>, grid, dim3(kThreads), 0, ctx.stream, a);
      if (Status s = LaunchStatus("Gemm(skinny colsum group)"); !s) return s;
      hipLaunchKernelGGL(skinny_colsum_group_finish<3>, fgrid, dim3(kThreads), 0, ctx.stream, a);
      break;
    default:
      hipLaunchKernelGGL(skinny_colsum_group<4>, grid, dim3(kThreads), 0, ctx.stream, a);
      if (Status s = LaunchStatus("Gemm(skinny colsum group)"); !s) return s;
      hipLaunchKernelGGL(skinny_colsum_group_finish<4>, fgrid, dim3(kThreads), 0, ctx.stream, a);
      break;
  }
  return LaunchStatus("Gemm(skinny colsum group finish)");
}

bool SkinnyRowdotGroupFits(const GemmDesc* ds, int n) {
  if (n < 2 || n > 4) return false;
  const GemmDesc& d = ds[0];
  for (int j = 0; j < n; ++j) {
    const GemmDesc& e = ds[j];
    if (SkinnyKindOf(e) != SkinnyKind::kRowDot || e.A != d.A || e.M != d.M || e.K != d.K ||
        e.lda != d.lda || e.N != d.N || e.N > 16 || e.ldb != d.ldb || e.ldc != d.ldc ||
        e.b_kc != d.b_kc || e.alpha != 1.0f || e.accumulate || e.bias || e.act != 0 ||
        e.scale_stream || !e.B || !e.C)
      return false;
  }
  return true;
}

Status LaunchSkinnyRowdotGroup(const GemmDesc* ds, int n, const Ctx& ctx) {
  if (!SkinnyRowdotGroupFits(ds, n))
    return Status::Fail(kUnitEngine, "Gemm: the rowdots do not form a group");
  const GemmDesc& d = ds[0];
  SkArgs a{};
  a.A = static_cast<const float*>(d.A);
  a.M = d.M; a.N = d.N; a.K = d.K;
  a.lda = d.lda; a.ldb = d.ldb; a.ldc = d.ldc;
  a.alpha = 1.0f;
  a.b_kc = d.b_kc ? 1 : 0;
  a.write_u = 1;
  for (int j = 0; j < n; ++j) {
    a.Bm[j] = static_cast<const float*>(ds[j].B);
    a.Cm[j] = ds[j].C;
  }
  // Two 16-row blocks per workgroup, two k groups per batch: in the C4 step
  // the q/k/v group took 12 us less per layer than the three rowdots; with
  // one row block it took as long as they did (each workgroup re-reads all
  // of the group's B operands from L2), and four k groups per batch spill.
  constexpr int kRB = 2, kU = 2;
  const int64_t gx = (d.M + 16 * kRB - 1) / (16 * kRB);
  if (gx > 0x7FFFFFFF) return Status::Fail(kUnitEngine, "Gemm: grid exceeds launch limits");
  const dim3 grid(static_cast<unsigned>(gx)), block(64 * kRowdotWaves);
  switch (n) {
    case 2: hipLaunchKernelGGL((skinny_rowdot_group<2, kRB, kU>), grid, block, 0, ctx.stream, a); break;
    case 3: hipLaunchKernelGGL((skinny_rowdot_group<3, kRB, kU>), grid, block, 0, ctx.stream, a); break;
    default: hipLaunchKernelGGL((skinny_rowdot_group<4, kRB, kU>), grid, block, 0, ctx.stream, a); break;
  }
  return LaunchStatus("Gemm(skinny rowdot group)");
}

namespace {
Status LaunchSkinnyImpl(const GemmDesc& d, const SkinnyChain* ch, const Ctx& ctx);
}

Status LaunchSkinny(const GemmDesc& d, const Ctx& ctx) { return LaunchSkinnyImpl(d, nullptr, ctx); }

Status LaunchSkinnyChain(const GemmDesc& d, const SkinnyChain& ch, const Ctx& ctx) {
  if (SkinnyKindOf(d) != SkinnyKind::kOuter || d.ldc != d.N || (ch.kind != 1 && ch.kind != 2) ||
      !ch.y || !ch.yout || !aligned16(ch.y) || !aligned16(ch.yout) ||
      (ch.s && !aligned16(ch.s)))
    return Status::Fail(kUnitEngine, "Gemm: chain does not fit the skinny outer kernel");
  return LaunchSkinnyImpl(d, &ch, ctx);
}

namespace {
Status LaunchSkinnyImpl(const GemmDesc& d, const SkinnyChain* ch, const Ctx& ctx) {
  const SkinnyKind kind = SkinnyKindOf(d);
  if (kind == SkinnyKind::kNone) return Status::Fail(kUnitEngine, "Gemm: shape is not skinny");
  SkArgs a{};
  a.write_u = 1;
  if (ch) {
    a.chain = ch->kind;
    a.chain_alpha = ch->alpha;
    a.S = ch->s;
    a.Y = ch->y;
    a.Yout = ch->yout;
    a.write_u = ch->write_u ? 1 : 0;
    a.y_first = ch->y_first ? 1 : 0;
  }
  a.scale_stream = d.scale_stream ? 1 : 0;
  a.stream_scale = d.stream_scale;
  if (d.scale_stream && kind != SkinnyKind::kRowDot && kind != SkinnyKind::kColSum)
    return Status::Fail(kUnitEngine, "Gemm: only the rowdot and colsum kernels scale their stream");
  a.A = static_cast<const float*>(d.A);
  a.B = static_cast<const float*>(d.B);
  a.C = d.C;
  a.ws = static_cast<float*>(ctx.ws);
  a.M = d.M; a.N = d.N; a.K = d.K;
  a.lda = d.lda; a.ldb = d.ldb; a.ldc = d.ldc;
  a.alpha = d.alpha;
  a.accumulate = d.accumulate ? 1 : 0;
  a.bias = d.bias;
  a.act = d.act;
  a.b_kc = d.b_kc ? 1 : 0;
  if (kind == SkinnyKind::kOuter) {
    const int64_t gx = (d.M + kOuterRows - 1) / kOuterRows, gy = (d.N + kOuterN - 1) / kOuterN;
    if (gx > 0x7FFFFFFF || gy > 65535) return Status::Fail(kUnitEngine, "Gemm: grid exceeds launch limits");
    const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
    const bool plain = d.alpha == 1.0f && !d.accumulate && !d.bias && d.act == 0;
#define SEEML_OUTER(KG_)                                                                      \
  if (ch && plain)                                                                            \
    hipLaunchKernelGGL((skinny_outer<KG_, true, true>), grid, dim3(kThreads), 0, ctx.stream, a);  \
  else if (ch)                                                                                \
    hipLaunchKernelGGL((skinny_outer<KG_, true, false>), grid, dim3(kThreads), 0, ctx.stream, a); \
  else if (plain)                                                                             \
    hipLaunchKernelGGL((skinny_outer<KG_, false, true>), grid, dim3(kThreads), 0, ctx.stream, a); \
  else                                                                                        \
    hipLaunchKernelGGL((skinny_outer<KG_, false, false>), grid, dim3(kThreads), 0, ctx.stream, a);
    switch ((d.K + 15) / 16) {
      case 1: SEEML_OUTER(1) break;
      case 2: SEEML_OUTER(2) break;
      default: SEEML_OUTER(4) break;
    }
#undef SEEML_OUTER
    return LaunchStatus("Gemm(skinny outer)");
  }
  if (kind == SkinnyKind::kRowDot) {
    const int64_t gx = (d.M + kRowdotM - 1) / kRowdotM;
    if (gx > 0x7FFFFFFF) return Status::Fail(kUnitEngine, "Gemm: grid exceeds launch limits");
    const dim3 grid(static_cast<unsigned>(gx)), block(64 * kRowdotWaves);
    switch ((d.N + 15) / 16) {
      case 1: hipLaunchKernelGGL(skinny_rowdot<1>, grid, block, 0, ctx.stream, a); break;
      case 2: hipLaunchKernelGGL(skinny_rowdot<2>, grid, block, 0, ctx.stream, a); break;
      default: hipLaunchKernelGGL(skinny_rowdot<4>, grid, block, 0, ctx.stream, a); break;
    }
    return LaunchStatus("Gemm(skinny rowdot)");
  }
  a.big_is_m = (d.N <= 64 && d.M >= 128) ? 1 : 0;
  a.W = a.big_is_m ? d.M : d.N;
  a.R = a.big_is_m ? d.N : d.M;
  a.groups = static_cast<int>(ColsumGroups(a.W, d.K));
  a.k_per_group = (d.K + a.groups - 1) / a.groups;
  const size_t need = static_cast<size_t>(a.groups) * a.W * a.R * sizeof(float);
  if (ctx.ws_bytes < need) return Status::Fail(kUnitEngine, "Gemm: workspace too small for skinny colsum");
  const int64_t gx = (a.W + kColW - 1) / kColW;
  if (gx > 0x7FFFFFFF) return Status::Fail(kUnitEngine, "Gemm: grid exceeds launch limits");
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(a.groups));
  switch ((a.R + 15) / 16) {
    case 1: hipLaunchKernelGGL(skinny_colsum<1>, grid, dim3(kThreads), 0, ctx.stream, a); break;
    case 2: hipLaunchKernelGGL(skinny_colsum<2>, grid, dim3(kThreads), 0, ctx.stream, a); break;
    default: hipLaunchKernelGGL(skinny_colsum<4>, grid, dim3(kThreads), 0, ctx.stream, a); break;
  }
  if (Status s = LaunchStatus("Gemm(skinny colsum)"); !s) return s;
  if (a.R % 4 == 0 && aligned16(ctx.ws))
    hipLaunchKernelGGL(skinny_colsum_finish, dim3(grid_for(static_cast<size_t>(a.W * a.R / 4), kThreads, 4096)),
                       dim3(kThreads), 0, ctx.stream, a);
  else
    hipLaunchKernelGGL(skinny_colsum_finish1, dim3(grid_for(static_cast<size_t>(a.W * a.R), kThreads, 4096)),
                       dim3(kThreads), 0, ctx.stream, a);
  return LaunchStatus("Gemm(skinny colsum finish)");
}

}  // namespace

}  // namespace seeml_hip
