// k_gemm.hip — fp32 MFMA GEMM engine for gfx950.
//
// Serves the reference's whole GEMM family (runtime/executor/gemm.cc:173-228:
// GemmNN + fused bias/act epilogue, GemmNT, GemmTN, GemmAccNN, the int8-B
// GemmNNQ8/NTQ8) and the attention contractions (attention.cc: QK^T, PV,
// dO V^T, P^T dO, dS K, dS^T Q), all as one kernel template:
//
//   C[z](m,n) = epilogue(alpha * sum_k A[z](m,k) B[z](k,n))
//
// with each operand either k-contiguous or row-contiguous in memory (so NT/TN
// read their operands in place, no transposes), a (b, h) batch decomposition
// with arbitrary element strides (attention heads live interleaved in
// [B*S, H*d] rows), and causal modes that skip whole tiles the causal mask
// zeroes.
//
// Mapping to CDNA4: 256 threads = 4 wavefronts of 64. Each wavefront owns a
// WM x WN sub-tile accumulated with v_mfma_f32_32x32x2_f32 (32x32 outputs,
// 16 accumulators per lane, K = 2 per instruction). A and B tiles of KT = 16
// are staged through LDS, double-buffered so the next tile's global loads
// are in flight while the matrix cores work on the current one. Global loads
// are 16-byte vectors along the contiguous dimension; LDS rows are padded to
// a stride = 36 (mod 64) words so the MFMA operand reads of the two
// half-wavefronts and the transposing stores land in distinct banks.
//
// Determinism: each output is owned by one lane of one workgroup and its k
// order is fixed by the tile loop; split-K writes per-slice partials that a
// second kernel sums in slice order. No atomics.
//
// Numerics: fp32 products, fp32 accumulation in the matrix core (full
// IEEE single precision, not a reduced-precision xf32 mode). The reference
// accumulates in a different order (4-wide k groups / sequential), so GEMM
// outputs agree to within fp32 reordering error, not bit-for-bit.
#include "device_common.h"
#include "kernels.h"

#include <algorithm>

namespace seeml_hip {

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int KT = 16;

struct GemmKArgs {
  const void* A;
  const void* B;
  float* C;
  float* ws;
  int64_t M, N, K, lda, ldb, ldc;
  int64_t heads, batch;
  int64_t a_sb, a_sh, b_sb, b_sh, c_sb, c_sh;
  float alpha;
  int accumulate;
  const float* bias;
  int act;
  int causal;
  int splits;
  int64_t k_per_split;
  int tiles_n;
  int a_vec, b_vec;
};

constexpr int LdsStride(int mt) { return mt + (((36 - mt) % 64) + 64) % 64; }

// Loads an MT x KT operand tile (outer index o = m for A / n for B) into
// registers; KC = k-contiguous in memory.
template <int MT, bool KC, typename T>
struct TileIO {
  static constexpr int kVecs = MT * KT / 4;
  static constexpr int kPer = (kVecs + kThreads - 1) / kThreads;
  float r[kPer][4];

  __device__ __forceinline__ void load(const T* __restrict__ X, int64_t ld, int64_t o0,
                                       int64_t oe, int64_t k0, int64_t ke, int vec) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int v = tid + i * kThreads;
      if (kVecs % kThreads != 0 && v >= kVecs) break;
      int o, k;
      if constexpr (KC) {
        o = v / (KT / 4);
        k = (v % (KT / 4)) * 4;
      } else {
        k = v / (MT / 4);
        o = (v % (MT / 4)) * 4;
      }
      const int64_t go = o0 + o, gk = k0 + k;
      if constexpr (sizeof(T) == 4) {
        if (vec) {
          const bool ok = KC ? (go < oe && gk < ke) : (gk < ke && go < oe);
          float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
          if (ok) {
            const T* src = KC ? X + go * ld + gk : X + gk * ld + go;
            q = *reinterpret_cast<const float4*>(src);
          }
          r[i][0] = q.x; r[i][1] = q.y; r[i][2] = q.z; r[i][3] = q.w;
          continue;
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t eo = KC ? go : go + e;
        const int64_t ek = KC ? gk + e : gk;
        float val = 0.0f;
        if (eo < oe && ek < ke) val = static_cast<float>(KC ? X[eo * ld + ek] : X[ek * ld + eo]);
        r[i][e] = val;
      }
    }
  }

  __device__ __forceinline__ void store(float* __restrict__ lds) const {
    constexpr int S = LdsStride(MT);
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int v = tid + i * kThreads;
      if (kVecs % kThreads != 0 && v >= kVecs) break;
      if constexpr (KC) {
        const int o = v / (KT / 4), k = (v % (KT / 4)) * 4;
#pragma unroll
        for (int e = 0; e < 4; ++e) lds[(k + e) * S + o] = r[i][e];
      } else {
        const int k = v / (MT / 4), o = (v % (MT / 4)) * 4;
        *reinterpret_cast<float4*>(lds + k * S + o) = make_float4(r[i][0], r[i][1], r[i][2], r[i][3]);
      }
    }
  }
};

template <int MT_M, int MT_N, int WAVES_M, int WAVES_N, bool A_KC, bool B_KC, bool B_I8>
__global__ __launch_bounds__(kThreads) void gemm_mfma_kernel(GemmKArgs p) {
  using BT = typename std::conditional<B_I8, int8_t, float>::type;
  constexpr int WM = MT_M / WAVES_M, WN = MT_N / WAVES_N;
  constexpr int BM = WM / 32, BN = WN / 32;
  static_assert(WAVES_M * WAVES_N == 4 && WM % 32 == 0 && WN % 32 == 0, "tile shape");
  constexpr int SA = LdsStride(MT_M), SB = LdsStride(MT_N);
  __shared__ float As[2][KT * SA];
  __shared__ float Bs[2][KT * SB];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 5, r = lane & 31;
  const int wm0 = (wave / WAVES_N) * WM, wn0 = (wave % WAVES_N) * WN;
  const int tm = blockIdx.x / p.tiles_n, tn = blockIdx.x % p.tiles_n;
  const int64_t m0 = static_cast<int64_t>(tm) * MT_M, n0 = static_cast<int64_t>(tn) * MT_N;
  const int64_t z = blockIdx.z, zb = z / p.heads, zh = z % p.heads;
  const int slice = blockIdx.y;

  const float* A = static_cast<const float*>(p.A) + zb * p.a_sb + zh * p.a_sh;
  const BT* B = static_cast<const BT*>(p.B) + zb * p.b_sb + zh * p.b_sh;
  float* C = p.C + zb * p.c_sb + zh * p.c_sh;

  // Causal lower-triangular output: a tile wholly above the diagonal is
  // exact zeros, with no reduction at all.
  if (p.causal == static_cast<int>(Causal::kLowerOut) && n0 > m0 + MT_M - 1) {
    for (int idx = threadIdx.x; idx < MT_M * MT_N; idx += kThreads) {
      const int64_t m = m0 + idx / MT_N, n = n0 + idx % MT_N;
      if (m < p.M && n < p.N) C[m * p.ldc + n] = 0.0f;
    }
    return;
  }

  int64_t kb = 0, ke = p.K;
  if (p.causal == static_cast<int>(Causal::kKLeM)) ke = std::min<int64_t>(p.K, m0 + MT_M);
  if (p.causal == static_cast<int>(Causal::kKGeM)) kb = std::min<int64_t>(p.K, m0);
  if (p.splits > 1) {
    kb = static_cast<int64_t>(slice) * p.k_per_split;
    ke = std::min<int64_t>(p.K, kb + p.k_per_split);
  }

  floatx16 acc[BM][BN];
#pragma unroll
  for (int i = 0; i < BM; ++i)
#pragma unroll
    for (int j = 0; j < BN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  TileIO<MT_M, A_KC, float> ta;
  TileIO<MT_N, B_KC, BT> tb;
  const int64_t ntiles = ke > kb ? (ke - kb + KT - 1) / KT : 0;
  if (ntiles > 0) {
    ta.load(A, p.lda, m0, p.M, kb, ke, p.a_vec);
    tb.load(B, p.ldb, n0, p.N, kb, ke, p.b_vec);
    ta.store(As[0]);
    tb.store(Bs[0]);
    __syncthreads();
    for (int64_t t = 0; t < ntiles; ++t) {
      const int cur = static_cast<int>(t & 1);
      const bool more = t + 1 < ntiles;
      if (more) {
        const int64_t k0 = kb + (t + 1) * KT;
        ta.load(A, p.lda, m0, p.M, k0, ke, p.a_vec);
        tb.load(B, p.ldb, n0, p.N, k0, ke, p.b_vec);
      }
      const float* as = As[cur];
      const float* bs = Bs[cur];
#pragma unroll
      for (int kk = 0; kk < KT; kk += 2) {
        float av[BM], bv[BN];
#pragma unroll
        for (int i = 0; i < BM; ++i) av[i] = as[(kk + g) * SA + wm0 + 32 * i + r];
#pragma unroll
        for (int j = 0; j < BN; ++j) bv[j] = bs[(kk + g) * SB + wn0 + 32 * j + r];
#pragma unroll
        for (int i = 0; i < BM; ++i)
#pragma unroll
          for (int j = 0; j < BN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
      }
      if (more) {
        ta.store(As[cur ^ 1]);
        tb.store(Bs[cur ^ 1]);
      }
      __syncthreads();
    }
  }

  // Write-back. Lane (g, r) of the 32x32 block holds rows 8*(v/4) + 4*g + v%4
  // of column r in accumulator element v.
#pragma unroll
  for (int i = 0; i < BM; ++i)
#pragma unroll
    for (int j = 0; j < BN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t m = m0 + wm0 + 32 * i + 8 * (v >> 2) + 4 * g + (v & 3);
        const int64_t n = n0 + wn0 + 32 * j + r;
        if (m >= p.M || n >= p.N) continue;
        float val = acc[i][j][v];
        if (p.splits > 1) {
          p.ws[(static_cast<int64_t>(slice) * p.M + m) * p.N + n] = val;
          continue;
        }
        val = p.alpha * val;
        if (p.accumulate) val = C[m * p.ldc + n] + val;
        if (p.bias) val = val + p.bias[n];
        val = dev_act(p.act, val);
        if (p.causal == static_cast<int>(Causal::kLowerOut) && n > m) val = 0.0f;
        C[m * p.ldc + n] = val;
      }
}

// Sums split-K partials in slice order and applies the epilogue (batch 1).
__global__ __launch_bounds__(kThreads) void splitk_reduce_kernel(GemmKArgs p) {
  const int64_t total = p.M * p.N;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; idx < total;
       idx += stride) {
    float val = p.ws[idx];
    for (int s = 1; s < p.splits; ++s) val += p.ws[static_cast<int64_t>(s) * total + idx];
    const int64_t m = idx / p.N, n = idx % p.N;
    val = p.alpha * val;
    if (p.accumulate) val = p.C[m * p.ldc + n] + val;
    if (p.bias) val = val + p.bias[n];
    val = dev_act(p.act, val);
    p.C[m * p.ldc + n] = val;
  }
}

// ---- tile configurations ----------------------------------------------------

struct CfgInfo {
  int mt_m, mt_n;
  const char* name;
};
constexpr CfgInfo kCfgs[] = {
    {128, 128, "128x128/w2x2"}, {64, 64, "64x64/w2x2"},    {128, 32, "128x32/w4x1"},
    {32, 128, "32x128/w1x4"},   {128, 64, "128x64/w2x2"},  {64, 128, "64x128/w2x2"},
};
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

template <bool A_KC, bool B_KC, bool B_I8>
void Launch(int cfg, dim3 grid, hipStream_t s, const GemmKArgs& a) {
  switch (cfg) {
    case 0: hipLaunchKernelGGL((gemm_mfma_kernel<128, 128, 2, 2, A_KC, B_KC, B_I8>), grid, dim3(kThreads), 0, s, a); break;
    case 1: hipLaunchKernelGGL((gemm_mfma_kernel<64, 64, 2, 2, A_KC, B_KC, B_I8>), grid, dim3(kThreads), 0, s, a); break;
    case 2: hipLaunchKernelGGL((gemm_mfma_kernel<128, 32, 4, 1, A_KC, B_KC, B_I8>), grid, dim3(kThreads), 0, s, a); break;
    case 3: hipLaunchKernelGGL((gemm_mfma_kernel<32, 128, 1, 4, A_KC, B_KC, B_I8>), grid, dim3(kThreads), 0, s, a); break;
    case 4: hipLaunchKernelGGL((gemm_mfma_kernel<128, 64, 2, 2, A_KC, B_KC, B_I8>), grid, dim3(kThreads), 0, s, a); break;
    default: hipLaunchKernelGGL((gemm_mfma_kernel<64, 128, 2, 2, A_KC, B_KC, B_I8>), grid, dim3(kThreads), 0, s, a); break;
  }
}

int64_t CeilDiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool VecOk(const void* base, int64_t ld, int64_t sb, int64_t sh, int64_t contiguous_extent) {
  return aligned16(base) && ld % 4 == 0 && sb % 4 == 0 && sh % 4 == 0 && contiguous_extent % 4 == 0;
}

}  // namespace

int GemmConfigCount() { return kNumCfgs; }
const char* GemmConfigName(int cfg) { return cfg >= 0 && cfg < kNumCfgs ? kCfgs[cfg].name : "?"; }

GemmPlan PlanGemmWith(const GemmDesc& d, int forced_cfg, int forced_splits) {
  GemmPlan plan;
  if (forced_cfg >= 0 && forced_cfg < kNumCfgs) {
    plan.cfg = forced_cfg;
  } else if (d.N <= 32 && d.M > 32) {
    plan.cfg = 2;
  } else if (d.M <= 32 && d.N > 32) {
    plan.cfg = 3;
  } else {
    const int64_t big = CeilDiv(d.M, 128) * CeilDiv(d.N, 128) * d.batch;
    const int64_t mid = CeilDiv(d.M, 64) * CeilDiv(d.N, 64) * d.batch;
    plan.cfg = big >= 512 ? 0 : (mid >= 256 || d.M <= 64 || d.N <= 64) ? 1 : 0;
  }
  const CfgInfo& c = kCfgs[plan.cfg];
  const int64_t tiles = CeilDiv(d.M, c.mt_m) * CeilDiv(d.N, c.mt_n) * d.batch;
  int splits = 1;
  const bool can_split = d.batch == 1 && d.causal == Causal::kNone;
  if (forced_splits >= 1) {
    splits = can_split ? forced_splits : 1;
  } else if (can_split && tiles < 512 && d.K >= 256) {
    // Enough workgroups to cover the chip twice, each slice >= 128 deep.
    const int64_t want = CeilDiv(512, tiles);
    const int64_t most = d.K / 128;
    splits = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(want, std::min<int64_t>(most, 64))));
  }
  plan.splits = splits;
  plan.ws_bytes = splits > 1 ? static_cast<size_t>(splits) * d.M * d.N * sizeof(float) : 0;
  return plan;
}

GemmPlan PlanGemm(const GemmDesc& d) { return PlanGemmWith(d, -1, -1); }

Status LaunchGemm(const GemmDesc& d, const GemmPlan& plan, const Ctx& ctx) {
  if (d.M <= 0 || d.N <= 0 || d.batch <= 0 || d.heads <= 0)
    return Status::Fail(kUnitEngine, "Gemm: empty shape");
  if (plan.cfg < 0 || plan.cfg >= kNumCfgs) return Status::Fail(kUnitEngine, "Gemm: bad tile config");
  const CfgInfo& c = kCfgs[plan.cfg];
  const int64_t tm = CeilDiv(d.M, c.mt_m), tn = CeilDiv(d.N, c.mt_n);
  if (tm * tn > 0x7FFFFFFF || d.batch > 65535 || plan.splits > 65535)
    return Status::Fail(kUnitEngine, "Gemm: grid exceeds launch limits");
  if (plan.splits > 1 && (d.batch != 1 || d.causal != Causal::kNone))
    return Status::Fail(kUnitEngine, "Gemm: split-K needs an unbatched, non-causal GEMM");
  if (plan.splits > 1 && ctx.ws_bytes < plan.ws_bytes)
    return Status::Fail(kUnitEngine, "Gemm: workspace too small for split-K");
  if (d.K <= 0 && d.causal == Causal::kNone && !d.accumulate) {
    // An empty reduction: C = epilogue(0). Still a valid launch: zero tiles.
  }

  GemmKArgs a{};
  a.A = d.A;
  a.B = d.B;
  a.C = d.C;
  a.ws = static_cast<float*>(ctx.ws);
  a.M = d.M; a.N = d.N; a.K = d.K;
  a.lda = d.lda; a.ldb = d.ldb; a.ldc = d.ldc;
  a.heads = d.heads; a.batch = d.batch;
  a.a_sb = d.a_sb; a.a_sh = d.a_sh; a.b_sb = d.b_sb; a.b_sh = d.b_sh;
  a.c_sb = d.c_sb; a.c_sh = d.c_sh;
  a.alpha = d.alpha;
  a.accumulate = d.accumulate ? 1 : 0;
  a.bias = d.bias;
  a.act = d.act;
  a.causal = static_cast<int>(d.causal);
  a.splits = plan.splits;
  a.k_per_split = plan.splits > 1 ? CeilDiv(CeilDiv(d.K, plan.splits), KT) * KT : d.K;
  a.tiles_n = static_cast<int>(tn);
  // Vector loads need 16-byte alignment of every batch base and a
  // contiguous extent that is a multiple of 4 (so a float4 is all-in or
  // all-out of bounds).
  a.a_vec = VecOk(d.A, d.lda, d.a_sb, d.a_sh, d.a_kc ? d.K : d.M) ? 1 : 0;
  a.b_vec = (!d.b_int8 && VecOk(d.B, d.ldb, d.b_sb, d.b_sh, d.b_kc ? d.K : d.N)) ? 1 : 0;

  const dim3 grid(static_cast<unsigned>(tm * tn), static_cast<unsigned>(plan.splits),
                  static_cast<unsigned>(d.batch));
  if (d.b_int8) {
    if (d.a_kc && !d.b_kc) Launch<true, false, true>(plan.cfg, grid, ctx.stream, a);
    else if (d.a_kc && d.b_kc) Launch<true, true, true>(plan.cfg, grid, ctx.stream, a);
    else return Status::Fail(kUnitEngine, "Gemm: unsupported int8 operand layout");
  } else if (d.a_kc && !d.b_kc) {
    Launch<true, false, false>(plan.cfg, grid, ctx.stream, a);
  } else if (d.a_kc && d.b_kc) {
    Launch<true, true, false>(plan.cfg, grid, ctx.stream, a);
  } else if (!d.a_kc && !d.b_kc) {
    Launch<false, false, false>(plan.cfg, grid, ctx.stream, a);
  } else {
    Launch<false, true, false>(plan.cfg, grid, ctx.stream, a);
  }
  if (Status s = LaunchStatus("Gemm"); !s) return s;
  if (plan.splits > 1) {
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(grid_for(static_cast<size_t>(d.M * d.N), kThreads, 8192)),
                       dim3(kThreads), 0, ctx.stream, a);
    return LaunchStatus("Gemm(split-K reduce)");
  }
  return Status::Ok();
}

GemmDesc GemmNNDesc(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K) {
  GemmDesc d;
  d.A = A; d.B = B; d.C = C; d.M = M; d.N = N; d.K = K;
  d.lda = K; d.ldb = N; d.ldc = N;
  d.a_kc = true; d.b_kc = false;
  return d;
}

GemmDesc GemmNTDesc(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K) {
  GemmDesc d;
  d.A = A; d.B = B; d.C = C; d.M = M; d.N = N; d.K = K;
  d.lda = K; d.ldb = K; d.ldc = N;
  d.a_kc = true; d.b_kc = true;
  return d;
}

GemmDesc GemmTNDesc(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K) {
  GemmDesc d;
  d.A = A; d.B = B; d.C = C; d.M = M; d.N = N; d.K = K;
  d.lda = M; d.ldb = N; d.ldc = N;
  d.a_kc = false; d.b_kc = false;
  return d;
}

}  // namespace seeml_hip
