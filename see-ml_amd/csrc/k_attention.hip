// k_attention.hip — causal attention forward/backward primitives on the
// MFMA GEMM engine.
//
// Reference: runtime/executor/attention.cc:94-242. Layouts are the ABI's:
// activations [B*S, H*d] with heads interleaved along the row, so head h of
// sequence b is a strided [S, d] view at offset b*S*H*d + h*d with row
// stride H*d; the probability cache P[B,H,S,S] is [B*H*S, S], batch (b, h)
// at offset (b*H + h)*S*S. Every primitive is a batched GEMM over the B*H
// (b, h) pairs; the causal mask becomes tile skipping:
//
//   AttnFwd  scores = QK^T/sqrt(d) -> P (lower-triangular output, exact 0
//            above), causal row softmax in place, O = P V (k <= row)
//   AttnDP   dP = dO V^T (lower-triangular output, exact 0 above)
//   AttnDV   dV = P^T dO (k >= row)
//   AttnDQ   dQ = (dS K)/sqrt(d) (k <= row)
//   AttnDK   dK = (dS^T Q)/sqrt(d) (k >= row)
//
// The masked P/dP entries the reference stores as exact zeros are stored
// as exact zeros here too (kernels_test.cc:625-629 depends on that bit).
#include "device_common.h"
#include "kernels.h"

#include <math.h>

#include <initializer_list>

namespace seeml_hip {

namespace {

struct Geo {
  int64_t B, S, H, d, D;
};

Geo MakeGeo(size_t B, size_t S, size_t H, size_t d) {
  return Geo{static_cast<int64_t>(B), static_cast<int64_t>(S), static_cast<int64_t>(H),
             static_cast<int64_t>(d), static_cast<int64_t>(H * d)};
}

// A per-head [S, d] activation operand.
void ActOperand(const Geo& g, int64_t* ld, int64_t* sb, int64_t* sh) {
  *ld = g.D;
  *sb = g.S * g.D;
  *sh = g.d;
}
// A per-head [S, S] probability operand.
void ProbOperand(const Geo& g, int64_t* ld, int64_t* sb, int64_t* sh) {
  *ld = g.S;
  *sb = g.H * g.S * g.S;
  *sh = g.S * g.S;
}

Status Run(const GemmDesc& d, const Ctx& c) {
  const GemmPlan plan = PlanGemm(d);
  return LaunchGemm(d, plan, c);
}

float InvSqrtD(int64_t d) { return 1.0f / ::sqrtf(static_cast<float>(d)); }

}  // namespace

namespace {

// ---- fused causal forward (d = 64 or 128) -----------------------------------
//
// One workgroup = 4 wavefronts = 128 queries of one (b, h); wavefront w owns
// queries q0 + 32w .. + 31, one per lane column. Scores are computed
// transposed, S^T = K Q^T, with v_mfma_f32_32x32x2_f32: the lane's Q row is
// the B operand held in registers for the whole kernel, K tiles of 32 keys
// are staged through LDS (double-buffered, shared by the 4 wavefronts).
// Accumulator element v of lane (h, r) is key 8*(v/4) + 4h + v%4 of the tile
// for query r, so each query's softmax statistics live in one lane pair
// (r, r + 32) and each lane stores its probabilities as four float4 runs of
// its query's P row.
//
// Pass 1 walks the causal key tiles for the row maximum m and the exp-sum l
// (online: l = l * exp(m_old - m_new) + sum exp(s - m_new)), in the base-2
// domain on the hardware exp2, and parks each tile's raw dot products in
// the lane's own slots of its P row. Pass 2 reads them back, forms
// p = exp(s - m) * (1/l) (exact 0 for j > i), writes P over them and
// accumulates O^T = V^T P^T with the probabilities straight from those
// registers as the B operand (MFMA t's k index is the lane's own
// accumulator element t). The row tail beyond the diagonal tile is written
// as exact zeros. QK^T is computed once: the second pass costs a write and
// a read of the causal half of P instead of a second score GEMM, and every
// value and its order of evaluation are those of recomputing it. P's range
// is the instruction's own output, so parking scores there disturbs no
// other value (with P unused, the scores are all it ever holds).
//
// Each pass loads the next key tile into registers at the top of an
// iteration, runs the tile's MFMAs and vector work, then stages the loaded
// tile into the other LDS buffer ahead of the iteration's one barrier (the
// order AttnDP uses). Measured on MI355X at C4's shape (B 8, S 1024, H 16,
// d 128): 0.356 ms per launch inside the train graph (96.5 TFLOP/s of
// causal QK^T + PV); the MFMAs alone, without the parked-score and P
// traffic, take 0.34 ms standalone.
//
// Heavy (late) query blocks are scheduled first, for causal load balance.
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kAttnQ = 128;  // queries per workgroup
constexpr int kAttnK = 32;   // keys per tile
constexpr int kAttnThreads = 256;

template <int D>
struct KvTile {
  static constexpr int kStride = D + 4;  // floats per LDS row
  static constexpr int kPer = kAttnK * D / 4 / kAttnThreads;
  // Plain floats (not float4 members), so the staged tile stays in VGPRs.
  float r[kPer][4];
  // Rows j0.. of a [S, ld] head view; rows past S are clamped onto row S-1
  // (their keys are masked for every valid query).
  __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld, int j0, int S) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int vi = static_cast<int>(threadIdx.x) + i * kAttnThreads;
      const int row = vi / (D / 4), c4 = vi % (D / 4);
      const int j = min(j0 + row, S - 1);
      const float4 q = *reinterpret_cast<const float4*>(base + static_cast<int64_t>(j) * ld + 4 * c4);
      r[i][0] = q.x;
      r[i][1] = q.y;
      r[i][2] = q.z;
      r[i][3] = q.w;
    }
  }
  __device__ __forceinline__ void store(float* __restrict__ lds) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int vi = static_cast<int>(threadIdx.x) + i * kAttnThreads;
      const int row = vi / (D / 4), c4 = vi % (D / 4);
      *reinterpret_cast<float4*>(lds + row * kStride + 4 * c4) =
          make_float4(r[i][0], r[i][1], r[i][2], r[i][3]);
    }
  }
};

// On a wavefront's diagonal key tile t, sets the entries of keys j > i (the
// lane's query) to `fill`; every earlier tile is wholly inside the causal
// half (and a key >= S can only fall in the diagonal tile of a valid query).
__device__ __forceinline__ void MaskDiagonal(floatx16& sc, int t, int i, int h, float fill) {
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int j = t * kAttnK + 8 * (e >> 2) + 4 * h + (e & 3);
    if (j > i) sc[e] = fill;
  }
}

// S^T tile (32 keys x 32 queries) from the LDS K tile and the lane's Q
// fragments: MFMA (g, jj) takes feature 8g + 4h + jj on both operands. Two
// accumulators (even/odd g) keep consecutive MFMAs independent. ORDER pins
// the issue order (below); the forward leaves it to the scheduler, which
// interleaves its parked-score traffic better (C4 step: AttnFwd 5.69 ->
// 5.90 ms per 16 launches with the order pinned, AttnDP 2.69 -> 2.67 ms).
template <int D, bool ORDER = false>
__device__ __forceinline__ floatx16 ScoreTile(const float* __restrict__ kt,
                                              const float4 (&qf)[D / 8], int h, int r) {
  floatx16 a0, a1;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    a0[e] = 0.0f;
    a1[e] = 0.0f;
  }
  const float* row = kt + r * KvTile<D>::kStride + 4 * h;
  // Fragment reads run one group ahead of the MFMAs that consume them.
  float4 kf[2];
  kf[0] = *reinterpret_cast<const float4*>(row);
#pragma unroll
  for (int g = 0; g < D / 8; ++g) {
    if (g + 1 < D / 8) kf[(g + 1) & 1] = *reinterpret_cast<const float4*>(row + 8 * (g + 1));
    const float4 f = kf[g & 1];
    floatx16& acc = (g & 1) ? a1 : a0;
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(f.x, qf[g].x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(f.y, qf[g].y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(f.z, qf[g].z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(f.w, qf[g].w, acc, 0, 0, 0);
  }
  // Issue order as written: read g + 1, then g's four MFMAs, so each read's
  // latency runs under them (left alone, the scheduler pairs the reads and
  // waits on each right after issuing it).
  if constexpr (ORDER) {
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
    for (int g = 0; g < D / 8; ++g) {
      if (g + 1 < D / 8) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    }
  }
  return a0 + a1;
}

// acc^T += tile^T P^T over one 32-key tile: for k index e (key kk = 8*(e/4)
// + 4h + e%4 of the tile) the B operand is the lane's p[e], and MFMA nb's A
// operand at lane (h, r) is tile[kk][NB*r + nb], i.e. MFMA nb's row i is
// feature NB*i + nb. The NB values of one e are contiguous, read as one
// 8- or 16-byte LDS access, one e ahead of the MFMAs that use them.
template <int D>
struct Frag {
  static constexpr int NB = D / 32;
  float v[NB];
};

template <int D>
__device__ __forceinline__ Frag<D> ReadFrag(const float* __restrict__ tile, int e, int h, int r) {
  constexpr int NB = D / 32;
  const float* p = tile + (8 * (e >> 2) + 4 * h + (e & 3)) * KvTile<D>::kStride + NB * r;
  Frag<D> f;
  if constexpr (NB == 4) {
    const float4 x = *reinterpret_cast<const float4*>(p);
    f.v[0] = x.x; f.v[1] = x.y; f.v[2] = x.z; f.v[3] = x.w;
  } else {
    const float2 x = *reinterpret_cast<const float2*>(p);
    f.v[0] = x.x; f.v[1] = x.y;
  }
  return f;
}

template <int D, bool ORDER = false, typename PV>
__device__ __forceinline__ void AccumulateTile(const float* __restrict__ tile, const PV& pv, int h,
                                               int r, floatx16 (&acc)[D / 32]) {
  constexpr int NB = D / 32;
  Frag<D> f[2];
  f[0] = ReadFrag<D>(tile, 0, h, r);
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    if (e + 1 < 16) f[(e + 1) & 1] = ReadFrag<D>(tile, e + 1, h, r);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      acc[nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(f[e & 1].v[nb], pv[e], acc[nb], 0, 0, 0);
  }
  // ORDER: issue order as written (read e + 1, then e's NB MFMAs), as in
  // ScoreTile (C4 step: AttnDQ 2.74 -> 2.64 ms, AttnDV 3.00 -> 2.84 ms and
  // AttnDK 2.91 -> 2.88 ms per 16 launches, with dK/dV's column loads).
  if constexpr (ORDER) {
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      if (e + 1 < 16) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, NB, 0);
    }
  }
}

// Writes acc (as laid out by AccumulateTile) to row `out` of a [*, H*d] head
// view: element e of acc[nb] at lane (h, r) is feature NB*i + nb with
// i = 8*(e/4) + 4h + e%4, so the NB blocks of one e form one vector store.
template <int D>
__device__ __forceinline__ void StoreRow(float* __restrict__ out, const floatx16 (&acc)[D / 32],
                                         int h) {
  constexpr int NB = D / 32;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int i = 8 * (e >> 2) + 4 * h + (e & 3);
    if constexpr (NB == 4)
      *reinterpret_cast<float4*>(out + 4 * i) = make_float4(acc[0][e], acc[1][e], acc[2][e], acc[3][e]);
    else
      *reinterpret_cast<float2*>(out + 2 * i) = make_float2(acc[0][e], acc[1][e]);
  }
}

// One wavefront's share of the forward: queries qw .. qw+31 of one (b, h),
// key tiles 0 .. tiles_w-1 (the last one its diagonal tile), inside a
// workgroup that stages tiles 0 .. tiles_wg-1. CHECKED: some of the
// wavefront's rows lie past S (the last query block of a ragged S); every
// other wavefront's P slots and parked scores need no per-lane test, since
// its keys j <= qw + 31 < S. Every iteration ends in one barrier whatever
// the wavefront computes, so the four wavefronts stay in step. STOREP
// (whether P is stored) is a compile-time choice: with a run-time one, the
// wait for the next tile's parked scores at the end of a pass-2 iteration
// also covered the P stores just issued (loads and stores share one
// counter), so every tile waited for its stores to complete (C4 step:
// 5.94 -> 5.70 ms per 16 forwards without that wait).
template <int D, bool CHECKED, bool STOREP>
__device__ __forceinline__ void AttnFwdWave(const float* __restrict__ qh, const float* __restrict__ kh,
                                            const float* __restrict__ vh, float* __restrict__ oh,
                                            float* __restrict__ ph, float* __restrict__ lds, int S,
                                            int64_t ld, int qw, int tiles_wg, int tiles_w, int h,
                                            int r, float c2, int pstore) {
  constexpr int NB = D / 32;
  constexpr int kBuf = kAttnK * KvTile<D>::kStride;
  const int i = qw + r;  // this lane's query
  const int ic = min(i, S - 1);
  const bool row_ok = !CHECKED || i < S;
  float* prow = ph + static_cast<int64_t>(ic) * S;
  // The lane's 16 slots of tile t in its P row (keys 8 q4 + 4h .. + 3).
  auto store_row = [&](const floatx16& p, int t) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int j = t * kAttnK + 8 * q4 + 4 * h;
      if (!CHECKED || (row_ok && j < S))
        *reinterpret_cast<float4*>(prow + j) =
            make_float4(p[4 * q4], p[4 * q4 + 1], p[4 * q4 + 2], p[4 * q4 + 3]);
    }
  };
  auto load_row = [&](int t) {
    floatx16 p;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int j = t * kAttnK + 8 * q4 + 4 * h;
      float4 x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (!CHECKED || (row_ok && j < S)) x = *reinterpret_cast<const float4*>(prow + j);
      p[4 * q4] = x.x;
      p[4 * q4 + 1] = x.y;
      p[4 * q4 + 2] = x.z;
      p[4 * q4 + 3] = x.w;
    }
    return p;
  };

  // ---- pass 1: scores parked in P, row maximum and exp-sum ----
  float m = -__builtin_inff(), l = 0.0f;
  auto stats = [&](floatx16 sc, int t, bool diag) {
#pragma unroll
    for (int e = 0; e < 16; ++e) sc[e] = sc[e] * c2;
    if (diag) MaskDiagonal(sc, t, i, h, -__builtin_inff());
    float tmax = -__builtin_inff();
#pragma unroll
    for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, sc[e]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float mn = fmaxf(m, tmax);
    const float alpha = m == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
    float ssum = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) ssum += __builtin_amdgcn_exp2f(sc[e] - mn);
    ssum += __shfl_xor(ssum, 32, 64);
    l = l * alpha + ssum;
    m = mn;
  };
  {
    float4 qf[D / 8];
#pragma unroll
    for (int g = 0; g < D / 8; ++g)
      qf[g] = *reinterpret_cast<const float4*>(qh + static_cast<int64_t>(ic) * ld + 8 * g + 4 * h);
    KvTile<D> ks;
    ks.load(kh, ld, 0, S);
    ks.store(lds);
    __syncthreads();
    for (int t = 0; t < tiles_wg; ++t) {
      if (t + 1 < tiles_wg) ks.load(kh, ld, (t + 1) * kAttnK, S);
      if (t < tiles_w) {
        const floatx16 sc = ScoreTile<D>(lds + (t & 1) * kBuf, qf, h, r);
        store_row(sc, t);
        stats(sc, t, t + 1 == tiles_w);
      }
      if (t + 1 < tiles_wg) ks.store(lds + ((t + 1) & 1) * kBuf);
      __syncthreads();
    }
  }

  // ---- pass 2: probabilities over the parked scores, P, O ----
  const float inv_l = 1.0f / l;
  floatx16 oacc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[nb][e] = 0.0f;
  constexpr bool store_p = STOREP;
  KvTile<D> vs;
  vs.load(vh, ld, 0, S);
  floatx16 sc;
#pragma unroll
  for (int e = 0; e < 16; ++e) sc[e] = 0.0f;
  if (tiles_w > 0) sc = load_row(0);
  vs.store(lds);
  __syncthreads();
  for (int t = 0; t < tiles_wg; ++t) {
    if (t + 1 < tiles_wg) vs.load(vh, ld, (t + 1) * kAttnK, S);
    if (t < tiles_w) {
      // The lane reads back exactly the slots it parked (program order).
      floatx16 sn;
      if (t + 1 < tiles_w) sn = load_row(t + 1);
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[e] = __builtin_amdgcn_exp2f(sc[e] * c2 - m) * inv_l;
      if (t + 1 == tiles_w) MaskDiagonal(sc, t, i, h, 0.0f);
      if (store_p) store_row(sc, t);
      AccumulateTile<D>(lds + (t & 1) * kBuf, sc, h, r, oacc);
      sc = sn;
    }
    if (t + 1 < tiles_wg) vs.store(lds + ((t + 1) & 1) * kBuf);
    __syncthreads();
  }

  if (row_ok) StoreRow<D>(oh + static_cast<int64_t>(i) * ld, oacc, h);
  // Causal tail: columns past this wavefront's diagonal tile are exact 0.
  if (!(pstore & kAttnStoreTail)) return;
  const int lane = 32 * h + r;
  const int zc = tiles_w * kAttnK;
  for (int rr = 0; rr < 32; ++rr) {
    const int row = qw + rr;
    if (row >= S) break;
    float* pz = ph + static_cast<int64_t>(row) * S;
    for (int c4 = zc / 4 + lane; c4 < S / 4; c4 += 64)
      *reinterpret_cast<float4*>(pz + 4 * c4) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
}

template <int D, bool STOREP>
__global__ __launch_bounds__(kAttnThreads, 2) void attn_fwd_fused(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ o, float* __restrict__ probs, int B, int S, int H, float inv_sqrt_d,
    int pstore) {
  // One double buffer of key tiles serves both passes: pass 1 stages K
  // there, pass 2 V (pass 1's last barrier orders its reads before pass 2's
  // first stores).
  __shared__ __align__(16) float lds[2 * kAttnK * KvTile<D>::kStride];
  const int lane = threadIdx.x & 63;
  // The wavefront index is uniform; saying so keeps every branch on the
  // tile counts scalar.
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int h = lane >> 5, r = lane & 31;
  const int BH = B * H;
  const int nqb = (S + kAttnQ - 1) / kAttnQ;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x) / BH;
  const int bh = static_cast<int>(blockIdx.x) % BH;
  const int b = bh / H, hh = bh % H;
  const int64_t ld = static_cast<int64_t>(H) * D;
  const int64_t head = static_cast<int64_t>(b) * S * ld + static_cast<int64_t>(hh) * D;
  float* ph = probs + static_cast<int64_t>(bh) * S * S;
  const int q0 = qb * kAttnQ;
  const int qw = q0 + 32 * w;  // first query of this wavefront
  const int tiles_wg = min((min(q0 + kAttnQ, S) - 1) / kAttnK + 1, (S + kAttnK - 1) / kAttnK);
  const int tiles_w = qw < S ? qw / kAttnK + 1 : 0;
  // Scores are kept in the base-2 domain: s2 = dot * (1/sqrt(d)) * log2(e),
  // so exp(s - max) is the hardware exp2 of s2 - max2.
  const float c2 = inv_sqrt_d * 1.44269504088896340736f;
  if (qw + 31 < S)
    AttnFwdWave<D, false, STOREP>(q + head, k + head, v + head, o + head, ph, lds, S, ld, qw,
                                  tiles_wg, tiles_w, h, r, c2, pstore);
  else
    AttnFwdWave<D, true, STOREP>(q + head, k + head, v + head, o + head, ph, lds, S, ld, qw,
                                 tiles_wg, tiles_w, h, r, c2, pstore);
}

// ---- fused causal backward primitives (d = 64 or 128) ----------------------
//
// Same workgroup shape and MFMA layout as the forward.
//
// attn_dp_fused: dP = dO V^T for j <= i, exact 0 above (attention.cc:138-163).
//   The score pass of the forward with dO as the register operand and V
//   tiles in LDS, storing the raw dots.
// attn_dq_fused: dQ(i) = sum_{j <= i} (dS(i, j) / sqrt(d)) K(j)
//   (attention.cc:203-222). Per wavefront 32 queries; dQ^T = K^T dS^T with K
//   tiles in LDS as the A operand and the lane's own dS row as the B
//   operand (element t of the lane's 16 is key 8*(t/4) + 4h + t%4, read as
//   four float4s), prefetched one tile ahead.
// attn_dkv_fused: dK(j) = sum_{i >= j} (dS(i, j) / sqrt(d)) Q(i) and
//   dV(j) = sum_{i >= j} P(i, j) dO(i) (attention.cc:165-183, 224-242). Per
//   wavefront 32 keys, one per lane column; the workgroup walks the query
//   tiles at and below its keys' diagonal, X (= Q or dO) tiles in LDS as the
//   A operand, the (i, j) column entries of dS / P as the B operand (for
//   each MFMA the 32 lanes of a half read 32 consecutive keys of one query
//   row). Early key blocks (the longest walks) are scheduled first.
// Entries outside the causal half are masked to exact zeros before use, as
// the reference's loops never visit them.

// One wavefront's dP rows (queries qw .. qw + 31). CHECKED as in the
// forward: only a wavefront with rows past S tests each store; the others
// store with no per-lane branch (C4 step: 2.73 -> 2.70 ms per 16 launches).
template <int D, bool CHECKED>
__device__ __forceinline__ void AttnDpWave(const float* __restrict__ dh, const float* __restrict__ vh,
                                           float* __restrict__ ph, float* __restrict__ vt, int S,
                                           int64_t ld, int qw, int tiles_wg, int tiles_w, int h,
                                           int r, int lane, int tail) {
  constexpr int kBuf = kAttnK * KvTile<D>::kStride;
  const int i = qw + r;
  const int ic = min(i, S - 1);
  float4 qf[D / 8];
#pragma unroll
  for (int g = 0; g < D / 8; ++g)
    qf[g] = *reinterpret_cast<const float4*>(dh + static_cast<int64_t>(ic) * ld + 8 * g + 4 * h);
  const bool row_ok = !CHECKED || i < S;
  float* prow = ph + static_cast<int64_t>(ic) * S;
  KvTile<D> vs;
  vs.load(vh, ld, 0, S);
  vs.store(vt);
  __syncthreads();
  for (int t = 0; t < tiles_wg; ++t) {
    if (t + 1 < tiles_wg) vs.load(vh, ld, (t + 1) * kAttnK, S);
    if (t < tiles_w) {
      floatx16 sc = ScoreTile<D, true>(vt + (t & 1) * kBuf, qf, h, r);
      if (t == tiles_w - 1) MaskDiagonal(sc, t, i, h, 0.0f);
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int j = t * kAttnK + 8 * q4 + 4 * h;
        if (!CHECKED || (row_ok && j < S))
          *reinterpret_cast<float4*>(prow + j) =
              make_float4(sc[4 * q4], sc[4 * q4 + 1], sc[4 * q4 + 2], sc[4 * q4 + 3]);
      }
    }
    if (t + 1 < tiles_wg) vs.store(vt + ((t + 1) & 1) * kBuf);
    __syncthreads();
  }
  if (!tail) return;
  const int zc = tiles_w * kAttnK;
  for (int rr = 0; rr < 32; ++rr) {
    const int row = qw + rr;
    if (row >= S) break;
    float* pz = ph + static_cast<int64_t>(row) * S;
    for (int c4 = zc / 4 + lane; c4 < S / 4; c4 += 64)
      *reinterpret_cast<float4*>(pz + 4 * c4) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
}

template <int D>
__global__ __launch_bounds__(kAttnThreads, 2) void attn_dp_fused(
    const float* __restrict__ dout, const float* __restrict__ v, float* __restrict__ dp, int B,
    int S, int H, int tail) {
  __shared__ __align__(16) float vt[2 * kAttnK * KvTile<D>::kStride];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);  // uniform
  const int h = lane >> 5, r = lane & 31;
  const int BH = B * H;
  const int nqb = (S + kAttnQ - 1) / kAttnQ;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x) / BH;
  const int bh = static_cast<int>(blockIdx.x) % BH;
  const int b = bh / H, hh = bh % H;
  const int64_t ld = static_cast<int64_t>(H) * D;
  const int64_t head = static_cast<int64_t>(b) * S * ld + static_cast<int64_t>(hh) * D;
  float* ph = dp + static_cast<int64_t>(bh) * S * S;
  const int q0 = qb * kAttnQ;
  const int qw = q0 + 32 * w;
  const int tiles_wg = min((min(q0 + kAttnQ, S) - 1) / kAttnK + 1, (S + kAttnK - 1) / kAttnK);
  const int tiles_w = qw < S ? qw / kAttnK + 1 : 0;
  if (qw + 31 < S)
    AttnDpWave<D, false>(dout + head, v + head, ph, vt, S, ld, qw, tiles_wg, tiles_w, h, r, lane,
                         tail);
  else
    AttnDpWave<D, true>(dout + head, v + head, ph, vt, S, ld, qw, tiles_wg, tiles_w, h, r, lane,
                        tail);
}

// The lane's 16 dS entries of key tile t for query i (masked j > i), scaled.
__device__ __forceinline__ void LoadRowTile(const float* __restrict__ row, int t, int i, int h,
                                            bool row_ok, float4 (&x)[4]) {
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    const int j = t * kAttnK + 8 * q4 + 4 * h;
    x[q4] = (row_ok && j <= i) ? *reinterpret_cast<const float4*>(row + j)
                               : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
}

template <int D>
__global__ __launch_bounds__(kAttnThreads, 2) void attn_dq_fused(
    const float* __restrict__ ds, const float* __restrict__ k, float* __restrict__ dq, int B,
    int S, int H, float inv_sqrt_d) {
  constexpr int TS = KvTile<D>::kStride;
  constexpr int NB = D / 32;
  __shared__ __align__(16) float kt[2][kAttnK * TS];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);  // uniform
  const int h = lane >> 5, r = lane & 31;
  const int BH = B * H;
  const int nqb = (S + kAttnQ - 1) / kAttnQ;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x) / BH;
  const int bh = static_cast<int>(blockIdx.x) % BH;
  const int b = bh / H, hh = bh % H;
  const int64_t ld = static_cast<int64_t>(H) * D;
  const int64_t head = static_cast<int64_t>(b) * S * ld + static_cast<int64_t>(hh) * D;
  const float* kh = k + head;
  float* oh = dq + head;
  const int q0 = qb * kAttnQ;
  const int qw = q0 + 32 * w;
  const int i = qw + r;
  const int ic = min(i, S - 1);
  const bool row_ok = i < S;
  const float* dsrow = ds + static_cast<int64_t>(bh) * S * S + static_cast<int64_t>(ic) * S;
  const int tiles_wg = min((min(q0 + kAttnQ, S) - 1) / kAttnK + 1, (S + kAttnK - 1) / kAttnK);
  const int tiles_w = qw < S ? qw / kAttnK + 1 : 0;
  floatx16 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[nb][e] = 0.0f;
  KvTile<D> ks;
  float4 x[4], xn[4];
  ks.load(kh, ld, 0, S);
  LoadRowTile(dsrow, 0, i, h, row_ok && 0 < tiles_w, x);
  ks.store(kt[0]);
  __syncthreads();
  for (int t = 0; t < tiles_wg; ++t) {
    if (t + 1 < tiles_wg) {
      ks.load(kh, ld, (t + 1) * kAttnK, S);
      LoadRowTile(dsrow, t + 1, i, h, row_ok && t + 1 < tiles_w, xn);
    }
    if (t < tiles_w) {
      float g[16];
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        g[4 * q4 + 0] = x[q4].x * inv_sqrt_d;
        g[4 * q4 + 1] = x[q4].y * inv_sqrt_d;
        g[4 * q4 + 2] = x[q4].z * inv_sqrt_d;
        g[4 * q4 + 3] = x[q4].w * inv_sqrt_d;
      }
      if (t == tiles_w - 1) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int j = t * kAttnK + 8 * (e >> 2) + 4 * h + (e & 3);
          if (j > i) g[e] = 0.0f;
        }
      }
      AccumulateTile<D, true>(kt[t & 1], g, h, r, acc);
    }
    if (t + 1 < tiles_wg) {
      ks.store(kt[(t + 1) & 1]);
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) x[q4] = xn[q4];
    }
    __syncthreads();
  }
  if (row_ok) StoreRow<D>(oh + static_cast<int64_t>(i) * ld, acc, h);
}

template <int D, bool SCALED>
__global__ __launch_bounds__(kAttnThreads, 2) void attn_dkv_fused(
    const float* __restrict__ pm, const float* __restrict__ x, float* __restrict__ out, int B,
    int S, int H, float scale) {
  constexpr int TS = KvTile<D>::kStride;
  constexpr int NB = D / 32;
  __shared__ __align__(16) float xt[2][kAttnK * TS];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);  // uniform
  const int h = lane >> 5, r = lane & 31;
  const int BH = B * H;
  const int kb = static_cast<int>(blockIdx.x) / BH;  // early key blocks first
  const int bh = static_cast<int>(blockIdx.x) % BH;
  const int b = bh / H, hh = bh % H;
  const int64_t ld = static_cast<int64_t>(H) * D;
  const int64_t head = static_cast<int64_t>(b) * S * ld + static_cast<int64_t>(hh) * D;
  const float* xh = x + head;
  float* oh = out + head;
  const float* ph = pm + static_cast<int64_t>(bh) * S * S;
  const int k0 = kb * kAttnQ;
  const int kw = k0 + 32 * w;  // first key of this wavefront
  const int j = kw + r;        // this lane's key
  const bool col_ok = j < S;
  const int ntiles = (S + kAttnK - 1) / kAttnK;
  const int t0 = k0 / kAttnK;       // the workgroup's first query tile
  const int tw = kw / kAttnK;       // this wavefront's first query tile
  floatx16 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[nb][e] = 0.0f;
  // Column entries (i = 32t + 8*(e/4) + 4h + e%4, j) of query tile t, loaded
  // unconditionally from rows clamped into the slab (32-bit offsets: S*S
  // fits), so the loads carry no branches; entries outside the causal half
  // (i < j, i >= S, j >= S) are zeroed where used, by an AND of the bits.
  const float* pcol = ph + min(j, S - 1);
  auto load_col = [&](int t, float (&g)[16]) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int ii = min(t * kAttnK + 8 * (e >> 2) + 4 * h + (e & 3), S - 1);
      g[e] = pcol[static_cast<uint32_t>(ii) * static_cast<uint32_t>(S)];
    }
  };
  // One query tile: the next tile's X rows and column entries are loaded
  // into the other register set (gn) while this tile's (gc) are used, so
  // no copy between them waits for the loads in flight. The loads and the
  // LDS store are unconditional (the last tile reloads itself into the idle
  // buffer), so every path through a tile leaves the same loads in flight
  // and the waits before the MFMAs count only the older set.
  KvTile<D> xs;
  auto tile = [&](int t, float (&gc)[16], float (&gn)[16]) {
    const int tn = min(t + 1, ntiles - 1);
    xs.load(xh, ld, tn * kAttnK, S);
    load_col(tn, gn);
    if (t >= tw && kw < S) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int ii = t * kAttnK + 8 * (e >> 2) + 4 * h + (e & 3);
        const unsigned keep = static_cast<unsigned>(col_ok) & static_cast<unsigned>(ii < S) &
                              static_cast<unsigned>(ii >= j);
        gc[e] = __uint_as_float(__float_as_uint(gc[e]) & (0u - keep));
        if constexpr (SCALED) gc[e] = gc[e] * scale;
      }
      AccumulateTile<D, true>(xt[(t - t0) & 1], gc, h, r, acc);
    }
    xs.store(xt[(t + 1 - t0) & 1]);
    __syncthreads();
  };
  float ga[16], gb[16];
  xs.load(xh, ld, t0 * kAttnK, S);
  load_col(t0, ga);
  xs.store(xt[0]);
  __syncthreads();
  for (int t = t0; t < ntiles; t += 2) {
    tile(t, ga, gb);
    if (t + 1 < ntiles) tile(t + 1, gb, ga);
  }
  if (col_ok) StoreRow<D>(oh + static_cast<int64_t>(j) * ld, acc, h);
}

// The fused kernels' shape gate: d in {64, 128}, S % 4 == 0 (16-byte P
// rows), S * S < 2^31 (32-bit offsets inside one (b, h) slab of P),
// 16-byte aligned operands, 32-bit grid indices.
bool FusedEligible(std::initializer_list<const float*> ptrs, size_t B, size_t S, size_t H,
                   size_t d) {
  if (d != 64 && d != 128) return false;
  if (S == 0 || S % 4 != 0 || S > 46340) return false;
  for (const float* p : ptrs)
    if (!aligned16(p)) return false;
  const size_t blocks = B * H * ((S + kAttnQ - 1) / kAttnQ);
  return B * H <= 0x7FFFFFFFu && S <= 0x7FFFFFFFu && blocks <= 0x7FFFFFFFu &&
         B * S * H * d < (size_t{1} << 62);
}

unsigned FusedBlocks(size_t B, size_t S, size_t H) {
  return static_cast<unsigned>(B * H * ((S + kAttnQ - 1) / kAttnQ));
}

}  // namespace

size_t AttnWorkspace(size_t, size_t, size_t, size_t) { return 0; }

bool AttnFusedPath(std::initializer_list<const float*> ptrs, size_t B, size_t S, size_t H,
                   size_t d) {
  return FusedEligible(ptrs, B, S, H, d);
}

Status AttnFwd(const float* q, const float* k, const float* v, float* o, float* probs, size_t B,
               size_t S, size_t H, size_t d, const Ctx& c, int pstore) {
  if (B * S * H * d == 0) return Status::Ok();
  if (FusedEligible({q, k, v, o, probs}, B, S, H, d)) {
    const unsigned blocks = FusedBlocks(B, S, H);
    const float inv = InvSqrtD(static_cast<int64_t>(d));
#define SEEML_FWD(DD, SP)                                                                  \
  hipLaunchKernelGGL((attn_fwd_fused<DD, SP>), dim3(blocks), dim3(kAttnThreads), 0, c.stream, q, \
                     k, v, o, probs, static_cast<int>(B), static_cast<int>(S),                    \
                     static_cast<int>(H), inv, pstore)
    const bool sp = (pstore & kAttnStoreP) != 0;
    if (d == 128) {
      if (sp) SEEML_FWD(128, true); else SEEML_FWD(128, false);
    } else {
      if (sp) SEEML_FWD(64, true); else SEEML_FWD(64, false);
    }
#undef SEEML_FWD
    return LaunchStatus("AttnFwd");
  }
  const Geo g = MakeGeo(B, S, H, d);
  // 1) raw scores s_ij = (q_i . k_j) * (1/sqrt(d)) for j <= i, exact 0 above.
  GemmDesc sc;
  sc.A = q; sc.B = k; sc.C = probs;
  sc.M = g.S; sc.N = g.S; sc.K = g.d;
  sc.a_kc = true; sc.b_kc = true;
  ActOperand(g, &sc.lda, &sc.a_sb, &sc.a_sh);
  ActOperand(g, &sc.ldb, &sc.b_sb, &sc.b_sh);
  ProbOperand(g, &sc.ldc, &sc.c_sb, &sc.c_sh);
  sc.batch = g.B * g.H; sc.heads = g.H;
  sc.alpha = InvSqrtD(g.d);
  sc.causal = Causal::kLowerOut;
  if (Status s = Run(sc, c); !s) return s;
  // 2) causal row softmax in place.
  if (Status s = AttnSoftmaxRows(probs, B * H * S, S, c); !s) return s;
  // 3) O = P V, reducing only j <= i.
  GemmDesc pv;
  pv.A = probs; pv.B = v; pv.C = o;
  pv.M = g.S; pv.N = g.d; pv.K = g.S;
  pv.a_kc = true; pv.b_kc = false;
  ProbOperand(g, &pv.lda, &pv.a_sb, &pv.a_sh);
  ActOperand(g, &pv.ldb, &pv.b_sb, &pv.b_sh);
  ActOperand(g, &pv.ldc, &pv.c_sb, &pv.c_sh);
  pv.batch = g.B * g.H; pv.heads = g.H;
  pv.causal = Causal::kKLeM;
  return Run(pv, c);
}

Status AttnDP(const float* dout, const float* v, float* dp, size_t B, size_t S, size_t H,
              size_t d, const Ctx& c, bool tail) {
  if (B * S * H * d == 0) return Status::Ok();
  if (FusedEligible({dout, v, dp}, B, S, H, d)) {
    const int iB = static_cast<int>(B), iS = static_cast<int>(S), iH = static_cast<int>(H);
    if (d == 128)
      hipLaunchKernelGGL(attn_dp_fused<128>, dim3(FusedBlocks(B, S, H)), dim3(kAttnThreads), 0,
                         c.stream, dout, v, dp, iB, iS, iH, tail ? 1 : 0);
    else
      hipLaunchKernelGGL(attn_dp_fused<64>, dim3(FusedBlocks(B, S, H)), dim3(kAttnThreads), 0,
                         c.stream, dout, v, dp, iB, iS, iH, tail ? 1 : 0);
    return LaunchStatus("AttnDP");
  }
  const Geo g = MakeGeo(B, S, H, d);
  GemmDesc x;
  x.A = dout; x.B = v; x.C = dp;
  x.M = g.S; x.N = g.S; x.K = g.d;
  x.a_kc = true; x.b_kc = true;
  ActOperand(g, &x.lda, &x.a_sb, &x.a_sh);
  ActOperand(g, &x.ldb, &x.b_sb, &x.b_sh);
  ProbOperand(g, &x.ldc, &x.c_sb, &x.c_sh);
  x.batch = g.B * g.H; x.heads = g.H;
  x.causal = Causal::kLowerOut;
  return Run(x, c);
}

Status AttnDV(const float* probs, const float* dout, float* dv, size_t B, size_t S, size_t H,
              size_t d, const Ctx& c) {
  if (B * S * H * d == 0) return Status::Ok();
  if (FusedEligible({probs, dout, dv}, B, S, H, d)) {
    const int iB = static_cast<int>(B), iS = static_cast<int>(S), iH = static_cast<int>(H);
    if (d == 128)
      hipLaunchKernelGGL((attn_dkv_fused<128, false>), dim3(FusedBlocks(B, S, H)),
                         dim3(kAttnThreads), 0, c.stream, probs, dout, dv, iB, iS, iH, 1.0f);
    else
      hipLaunchKernelGGL((attn_dkv_fused<64, false>), dim3(FusedBlocks(B, S, H)),
                         dim3(kAttnThreads), 0, c.stream, probs, dout, dv, iB, iS, iH, 1.0f);
    return LaunchStatus("AttnDV");
  }
  const Geo g = MakeGeo(B, S, H, d);
  GemmDesc x;  // dV(j, c) = sum_{i >= j} P(i, j) dO(i, c): A(m=j, k=i) = P[i][j]
  x.A = probs; x.B = dout; x.C = dv;
  x.M = g.S; x.N = g.d; x.K = g.S;
  x.a_kc = false; x.b_kc = false;
  ProbOperand(g, &x.lda, &x.a_sb, &x.a_sh);
  ActOperand(g, &x.ldb, &x.b_sb, &x.b_sh);
  ActOperand(g, &x.ldc, &x.c_sb, &x.c_sh);
  x.batch = g.B * g.H; x.heads = g.H;
  x.causal = Causal::kKGeM;
  return Run(x, c);
}

Status AttnDQ(const float* ds, const float* k, float* dq, size_t B, size_t S, size_t H, size_t d,
              const Ctx& c) {
  if (B * S * H * d == 0) return Status::Ok();
  if (FusedEligible({ds, k, dq}, B, S, H, d)) {
    const int iB = static_cast<int>(B), iS = static_cast<int>(S), iH = static_cast<int>(H);
    const float inv = InvSqrtD(static_cast<int64_t>(d));
    if (d == 128)
      hipLaunchKernelGGL(attn_dq_fused<128>, dim3(FusedBlocks(B, S, H)), dim3(kAttnThreads), 0,
                         c.stream, ds, k, dq, iB, iS, iH, inv);
    else
      hipLaunchKernelGGL(attn_dq_fused<64>, dim3(FusedBlocks(B, S, H)), dim3(kAttnThreads), 0,
                         c.stream, ds, k, dq, iB, iS, iH, inv);
    return LaunchStatus("AttnDQ");
  }
  const Geo g = MakeGeo(B, S, H, d);
  GemmDesc x;  // dQ(i, c) = sum_{j <= i} dS(i, j) K(j, c) / sqrt(d)
  x.A = ds; x.B = k; x.C = dq;
  x.M = g.S; x.N = g.d; x.K = g.S;
  x.a_kc = true; x.b_kc = false;
  ProbOperand(g, &x.lda, &x.a_sb, &x.a_sh);
  ActOperand(g, &x.ldb, &x.b_sb, &x.b_sh);
  ActOperand(g, &x.ldc, &x.c_sb, &x.c_sh);
  x.batch = g.B * g.H; x.heads = g.H;
  x.alpha = InvSqrtD(g.d);
  x.causal = Causal::kKLeM;
  return Run(x, c);
}

Status AttnDK(const float* ds, const float* q, float* dk, size_t B, size_t S, size_t H, size_t d,
              const Ctx& c) {
  if (B * S * H * d == 0) return Status::Ok();
  if (FusedEligible({ds, q, dk}, B, S, H, d)) {
    const int iB = static_cast<int>(B), iS = static_cast<int>(S), iH = static_cast<int>(H);
    const float inv = InvSqrtD(static_cast<int64_t>(d));
    if (d == 128)
      hipLaunchKernelGGL((attn_dkv_fused<128, true>), dim3(FusedBlocks(B, S, H)),
                         dim3(kAttnThreads), 0, c.stream, ds, q, dk, iB, iS, iH, inv);
    else
      hipLaunchKernelGGL((attn_dkv_fused<64, true>), dim3(FusedBlocks(B, S, H)),
                         dim3(kAttnThreads), 0, c.stream, ds, q, dk, iB, iS, iH, inv);
    return LaunchStatus("AttnDK");
  }
  const Geo g = MakeGeo(B, S, H, d);
  GemmDesc x;  // dK(j, c) = sum_{i >= j} dS(i, j) Q(i, c) / sqrt(d)
  x.A = ds; x.B = q; x.C = dk;
  x.M = g.S; x.N = g.d; x.K = g.S;
  x.a_kc = false; x.b_kc = false;
  ProbOperand(g, &x.lda, &x.a_sb, &x.a_sh);
  ActOperand(g, &x.ldb, &x.b_sb, &x.b_sh);
  ActOperand(g, &x.ldc, &x.c_sb, &x.c_sh);
  x.batch = g.B * g.H; x.heads = g.H;
  x.alpha = InvSqrtD(g.d);
  x.causal = Causal::kKGeM;
  return Run(x, c);
}

}  // namespace seeml_hip
