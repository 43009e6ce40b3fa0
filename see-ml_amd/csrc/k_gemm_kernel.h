// k_gemm_kernel.h — the fp32 MFMA GEMM kernel template for gfx950 (device code
// shared by the per-layout instantiation units k_gemm_{nn,nt,tn,q8}.hip; host
// planning and launch live in k_gemm.hip).
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
// Mapping to CDNA4: a workgroup of 4 or 8 wavefronts (64 lanes) owns an
// MT_M x MT_N output tile; each wavefront owns a WM x WN sub-tile accumulated
// with v_mfma_f32_32x32x2_f32 (32x32 outputs, 16 accumulators per lane, two
// k values per instruction, one per half-wavefront). Operand tiles
// (KT = 32 or 64 per config) are staged through LDS, double-buffered:
// the next stage's 16-byte global loads are in flight while the matrix cores
// consume the current one. The k loop carries no per-element address math:
// each lane's offsets from the stage origin are fixed at kernel entry (rows
// past the operand's end are clamped onto its last row — their products
// reach only outputs that are never stored), the origin advances by a
// uniform step, and only a final partial stage masks k.
//
// k assignment: a fragment group covers 8 k. Half-wavefront h of MFMA j
// (j = 0..3) supplies k = 8g + 4h + j, for A and B alike, so a k-contiguous
// operand kept in LDS as [o][k] rows is read with ONE 16-byte ds_read per
// lane per four MFMAs; an o-contiguous operand is kept as [k][o] rows and
// read as four 4-byte reads (consecutive lanes, consecutive addresses).
//
// Workgroup order: the 8 XCDs (each with its own L2) receive workgroups
// round-robin, so the linear workgroup id is remapped to give each XCD a
// contiguous run of tiles, walked in groups of 8 tile-rows so the tiles
// resident on one XCD share A row-panels and B column-panels in its L2.
//
// Determinism: each output is owned by one lane of one workgroup and its k
// order is fixed by the tile loop; split-K writes per-slice partials that a
// second kernel sums in slice order. No atomics.
//
// Numerics: fp32 products, fp32 accumulation in the matrix core (full
// IEEE single precision, not a reduced-precision xf32 mode). The reference
// accumulates in a different order (4-wide k groups / sequential), so GEMM
// outputs agree to within fp32 reordering error, not bit-for-bit.
#pragma once

#include "device_common.h"
#include "kernels.h"

#include <algorithm>
#include <type_traits>

namespace seeml_hip {
namespace gemm {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int KG = 8;           // k covered by one fragment group
constexpr int kXcds = 8;
constexpr int kGroupRows = 8;   // tile-rows walked together (L2 panel sharing)
constexpr int kSplitAlign = 64; // split-K slice depth: a multiple of every KT

// LDS row strides in floats. [o][k] rows of KT + 4: the 16-byte fragment
// reads of 8 consecutive lanes (8 rows, same k) cover the 32 banks once.
// [k][o] rows padded by 8: the half-wavefronts (k and k + 4) fall in
// disjoint bank halves.
constexpr int KcStride(int kt) { return kt + 4; }
constexpr int RcStride(int mt) { return mt + 8; }
template <int MT, int KT, bool KC>
constexpr int TileFloats() { return KC ? MT * KcStride(KT) : KT * RcStride(MT); }

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
  int tiles_m, tiles_n;
  const float* addend;  // fused AddEW (GemmDesc::addend): out = addend (+) c
  float* out;
  int addend_first;
  int write_c;
  float out_scale;  // GemmDesc::out_scaled: the AddEW consumes fl(out_scale * c)
  int out_scaled;
  int c_scaled;     // GemmDesc::c_gets_scaled: the C store is the scaled value
  int64_t ldo;      // row stride of addend and out
  // LoRA up-projection in the epilogue (GemmDesc::lora_t): with lora_t set,
  // out = c (+) fl(out_scale * u) where u = T B' over lora_r (T [M, lora_r]
  // row-major, B' [lora_r, N] row-major), the same MFMA k order as a tile
  // GEMM of u; addend unused. lora_y_first: c is the AddEW's first operand.
  const float* lora_t;
  const float* lora_b;
  int64_t lora_ldt, lora_ldb;
  int lora_r;
  int lora_y_first;
  // A Scale folded into the operand loads (GemmDesc::scale_stream, the
  // SCL instantiations): the scaled operand is read as fl(op_scale * x).
  float op_scale;
  // The AddBias (+ activation) after the fused AddEW (GemmDesc::post_bias,
  // the POST instantiations): h = o + pbias[n] to hout, act(h) to gout
  // (each when set), o to out only with write_out.
  const float* pbias;
  float* hout;
  float* gout;
  int pact;
  int write_out;
};

// The fused AddEW's sum o of value v and addend y, stored with what follows
// it (POST: the AddBias of bias value b, then the activation) at element
// offset `at` of the out / hout / gout arrays (one layout, row stride ldo).
template <bool POST>
__device__ __forceinline__ void FusedSum(const GemmKArgs& p, int64_t at, float y, float sv, float b) {
  const float o = p.addend_first ? y + sv : sv + y;
  if constexpr (!POST) {
    p.out[at] = o;
  } else {
    if (p.write_out) p.out[at] = o;
    const float h = o + b;
    if (p.hout) p.hout[at] = h;
    if (p.gout) p.gout[at] = dev_act(p.pact, h);
  }
}

// Tile configurations (the autotuner's arms).
struct CfgInfo {
  int mt_m, mt_n, kt, threads;
  const char* name;
};
inline constexpr CfgInfo kCfgs[] = {
    {128, 128, 32, 256, "128x128x32/w2x2"}, {128, 128, 32, 512, "128x128x32/w4x2"},
    {256, 128, 32, 512, "256x128x32/w4x2"}, {128, 256, 32, 512, "128x256x32/w2x4"},
    {128, 64, 32, 256, "128x64x32/w2x2"},   {64, 64, 32, 256, "64x64x32/w2x2"},
    {128, 32, 32, 256, "128x32x32/w4x1"},   {32, 128, 32, 256, "32x128x32/w1x4"},
    {64, 128, 32, 256, "64x128x32/w2x2"},   {128, 64, 32, 256, "128x64x32/w4x1"},
    {128, 128, 16, 256, "128x128x16/w2x2"}, {64, 128, 16, 256, "64x128x16/w2x2"},
};
inline constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);
inline constexpr int kCfgDefault = 0, kCfgSmall = 5, kCfgSkinnyN = 6, kCfgSkinnyM = 7;

// One operand's MT x KT stage (outer index o = m for A / n for B), held in
// registers between its global loads and its LDS store. KC = k-contiguous.
//
// VEC (16-byte aligned rows, contiguous extent a multiple of 4): 16-byte
// loads at per-lane offsets fixed for the whole k loop; the stage origin is
// uniform. A final partial stage (k beyond the reduction's end) zeroes its
// out-of-range vectors, reading the row start instead.
// !VEC (int8 B, odd shapes): element loads with an in-range mask applied at
// the LDS store. Both forms are branch-free per element, so a stage's loads
// are all in flight together and the first wait is at the LDS store.
//
// SC (VEC only): every loaded element in range is scaled, fl(sc * x), as a
// Scale instruction would have stored it; zeros past the reduction's end
// stay +0. A whole stage is scaled at its LDS store, where its loads are
// waited for anyway (scaled as loaded, each stage's loads would be waited
// for at once, a stage early: 2.5x slower on the rank-64 shapes); a final
// partial stage is scaled as loaded, under its in-range masks.
template <int MT, int KT, bool KC, typename T, int NT, bool VEC, bool SC = false>
struct Stage {
  static constexpr int kVecs = MT * KT / 4;
  static constexpr int kPer = kVecs / NT;
  static_assert(kVecs % NT == 0 && kPer * 4 <= 64, "stage shape");
  static_assert(!SC || VEC, "scaled loads need the vector form");
  float r[kPer][4];
  uint32_t off[kPer];  // VEC: element offset of vector i from the stage origin
  uint64_t ok;         // !VEC: bit 4i+e set when element e of vector i is in range
  float sc;            // SC: the factor
  bool pend;           // SC: loaded unscaled (a whole stage), scaled at the store

  __device__ __forceinline__ static void coords(int v, int& o, int& k) {
    if constexpr (KC) {
      o = v / (KT / 4);
      k = (v % (KT / 4)) * 4;
    } else {
      k = v / (MT / 4);
      o = (v % (MT / 4)) * 4;
    }
  }

  // o0: first row of the tile (a multiple of 4); oe: the operand's extent.
  __device__ __forceinline__ void init(int64_t ld, int64_t o0, int64_t oe) {
    if constexpr (VEC) {
      const int64_t last = oe - o0 - (KC ? 1 : 4);  // >= 0: the tile starts in range
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        int o, k;
        coords(static_cast<int>(threadIdx.x) + i * NT, o, k);
        const int64_t oc = std::min<int64_t>(o, last);
        off[i] = static_cast<uint32_t>(KC ? oc * ld + k : k * ld + oc);
      }
    }
  }

  // A whole stage in range (VEC): one 16-byte load per vector, no masks.
  __device__ __forceinline__ void load_full(const T* __restrict__ org) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const float4 q = *reinterpret_cast<const float4*>(org + off[i]);
      r[i][0] = q.x; r[i][1] = q.y; r[i][2] = q.z; r[i][3] = q.w;
    }
    if constexpr (SC) pend = true;
  }

  // Any stage: k beyond ke (and, for !VEC, rows beyond oe) read as zero.
  __device__ __forceinline__ void load(const T* __restrict__ X, int64_t ld, int64_t o0,
                                       int64_t oe, int64_t k0, int64_t ke) {
    if constexpr (VEC) {
      const T* org = X + (KC ? o0 * ld + k0 : k0 * ld + o0);
      const int64_t kvalid = ke - k0;
      if (kvalid >= KT) {
        load_full(org);
      } else {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
          int o, k;
          coords(static_cast<int>(threadIdx.x) + i * NT, o, k);
          const bool in = k < kvalid;  // a KC vector is wholly in or out (K % 4 == 0)
          const int64_t back = KC ? k : static_cast<int64_t>(k) * ld;
          float4 q = *reinterpret_cast<const float4*>(org + (off[i] - (in ? 0 : back)));
          if constexpr (SC) q = make_float4(sc * q.x, sc * q.y, sc * q.z, sc * q.w);
          if constexpr (SC) pend = false;
          r[i][0] = in ? q.x : 0.0f;
          r[i][1] = in ? q.y : 0.0f;
          r[i][2] = in ? q.z : 0.0f;
          r[i][3] = in ? q.w : 0.0f;
        }
      }
    } else {
      ok = 0;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        int o, k;
        coords(static_cast<int>(threadIdx.x) + i * NT, o, k);
        const int64_t go = o0 + o, gk = k0 + k;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t eo = KC ? go : go + e;
          const int64_t ek = KC ? gk + e : gk;
          const bool in = eo < oe && ek < ke;
          r[i][e] = static_cast<float>(X[in ? (KC ? eo * ld + ek : ek * ld + eo) : 0]);
          ok |= (in ? uint64_t{1} : uint64_t{0}) << (4 * i + e);
        }
      }
    }
  }

  __device__ __forceinline__ void store(float* __restrict__ lds) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      int o, k;
      coords(static_cast<int>(threadIdx.x) + i * NT, o, k);
      float* dst = KC ? lds + o * KcStride(KT) + k : lds + k * RcStride(MT) + o;
      float4 q;
      if constexpr (VEC) {
        q = make_float4(r[i][0], r[i][1], r[i][2], r[i][3]);
        if constexpr (SC)
          if (pend) q = make_float4(sc * q.x, sc * q.y, sc * q.z, sc * q.w);
      } else {
        q.x = (ok >> (4 * i + 0)) & 1 ? r[i][0] : 0.0f;
        q.y = (ok >> (4 * i + 1)) & 1 ? r[i][1] : 0.0f;
        q.z = (ok >> (4 * i + 2)) & 1 ? r[i][2] : 0.0f;
        q.w = (ok >> (4 * i + 3)) & 1 ? r[i][3] : 0.0f;
      }
      *reinterpret_cast<float4*>(dst) = q;
    }
  }
};

// The 4 k values (8g + 4h + j, j = 0..3) of NB 32-wide fragments at o = w0 + 32i + r.
template <int MT, int KT, bool KC, int NB>
__device__ __forceinline__ void ReadFrags(const float* __restrict__ lds, int w0, int g, int h,
                                          int r, float (&f)[NB][4]) {
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int o = w0 + 32 * i + r;
    if constexpr (KC) {
      const float4 q = *reinterpret_cast<const float4*>(lds + o * KcStride(KT) + g * KG + 4 * h);
      f[i][0] = q.x; f[i][1] = q.y; f[i][2] = q.z; f[i][3] = q.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) f[i][j] = lds[(g * KG + 4 * h + j) * RcStride(MT) + o];
    }
  }
}

// Linear workgroup id -> logical id such that XCD x (= lin % 8) holds the
// contiguous logical range of its share. A bijection on [0, total).
// Workgroup counts fit 32 bits (a grid holds at most 2^32 - 1 workgroups),
// and 32-bit divisions are a few instructions where 64-bit ones are a long
// scalar routine run by every workgroup before its first load.
__device__ __forceinline__ uint32_t XcdLogical(uint32_t lin, uint32_t total) {
  const uint32_t per = total / kXcds, rem = total % kXcds;
  const uint32_t x = lin % kXcds, idx = lin / kXcds;
  return x < rem ? x * (per + 1) + idx : rem * (per + 1) + (x - rem) * per + idx;
}

// One workgroup's work item: logical id L (after the XCD remap) decomposes
// into (tile, split slice, batch z) over `nslices` slices. FUSED and LORA
// compile those epilogues in; each applies to a work item whose arguments
// ask for it (p.out / p.lora_t set), any other takes the plain write-back.
// SCL: a Scale folded into the loads of A (1) or B (2), factor p.op_scale.
// POST (with FUSED): the AddBias (+ activation) after the fused AddEW.
template <int MT_M, int MT_N, int KT, int WAVES_M, int WAVES_N, bool A_KC, bool B_KC, bool B_I8,
          bool VEC, bool SCHED, bool FUSED, bool LORA, int SCL = 0, bool POST = false>
__device__ __forceinline__ void gemm_tile(const GemmKArgs& p, uint32_t L, uint32_t nslices) {
  static_assert(!POST || (FUSED && !LORA && !(MT_M == 256 && MT_N == 128)), "post-AddEW variants");
  using BT = typename std::conditional<B_I8, int8_t, float>::type;
  constexpr int NT = 64 * WAVES_M * WAVES_N;
  constexpr int WM = MT_M / WAVES_M, WN = MT_N / WAVES_N;
  constexpr int BM = WM / 32, BN = WN / 32;
  static_assert(WM % 32 == 0 && WN % 32 == 0 && KT % KG == 0 && kSplitAlign % KT == 0,
                "tile shape");
  constexpr int TA = TileFloats<MT_M, KT, A_KC>(), TB = TileFloats<MT_N, KT, B_KC>();
  __shared__ __align__(16) float smem[2 * (TA + TB)];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane >> 5, r = lane & 31;
  const int wm0 = (wave / WAVES_N) * WM, wn0 = (wave % WAVES_N) * WN;

  // Logical work item of this workgroup: (tile, split slice, batch z).
  const uint32_t tiles = static_cast<uint32_t>(p.tiles_m) * static_cast<uint32_t>(p.tiles_n);
  const uint32_t t_id = L % tiles;
  L /= tiles;
  const int slice = static_cast<int>(L % nslices);
  const uint32_t z = L / nslices;
  const uint32_t grp = t_id / (kGroupRows * static_cast<uint32_t>(p.tiles_n));
  const uint32_t first = grp * kGroupRows;
  const uint32_t gm = std::min<uint32_t>(kGroupRows, static_cast<uint32_t>(p.tiles_m) - first);
  const uint32_t in_grp = t_id - grp * kGroupRows * static_cast<uint32_t>(p.tiles_n);
  const int64_t tm = first + in_grp % gm, tn = in_grp / gm;
  const int64_t m0 = tm * MT_M, n0 = tn * MT_N;
  const uint32_t heads = static_cast<uint32_t>(p.heads);
  const int64_t zb = z / heads, zh = z % heads;

  const float* A = static_cast<const float*>(p.A) + zb * p.a_sb + zh * p.a_sh;
  const BT* B = static_cast<const BT*>(p.B) + zb * p.b_sb + zh * p.b_sh;
  float* C = p.C + zb * p.c_sb + zh * p.c_sh;

  // Causal lower-triangular output: a tile wholly above the diagonal is
  // exact zeros, with no reduction at all.
  if (p.causal == static_cast<int>(Causal::kLowerOut) && n0 > m0 + MT_M - 1) {
    for (int idx = threadIdx.x; idx < MT_M * MT_N; idx += NT) {
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

  constexpr bool kVecB = VEC && !B_I8;
  using StageA = Stage<MT_M, KT, A_KC, float, NT, VEC, SCL == 1>;
  using StageB = Stage<MT_N, KT, B_KC, BT, NT, kVecB, SCL == 2>;
  // Two register sets: stage s is loaded into set s % 2 two iterations
  // before it is computed, stored to LDS buffer s % 2 one iteration before.
  StageA sa0, sa1;
  StageB sb0, sb1;

  // One stage's contraction out of LDS: 4 MFMAs per fragment group per
  // (i, jj) block, the next group's fragments read while the current
  // group's MFMAs run.
  auto compute = [&](const float* __restrict__ as, const float* __restrict__ bs) {
    float fa[2][BM][4], fb[2][BN][4];
    ReadFrags<MT_M, KT, A_KC, BM>(as, wm0, 0, h, r, fa[0]);
    ReadFrags<MT_N, KT, B_KC, BN>(bs, wn0, 0, h, r, fb[0]);
#pragma unroll
    for (int g = 0; g < KT / KG; ++g) {
      const int c = g & 1;
      if (g + 1 < KT / KG) {
        ReadFrags<MT_M, KT, A_KC, BM>(as, wm0, g + 1, h, r, fa[c ^ 1]);
        ReadFrags<MT_N, KT, B_KC, BN>(bs, wn0, g + 1, h, r, fb[c ^ 1]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < BM; ++i)
#pragma unroll
          for (int jj = 0; jj < BN; ++jj)
            acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[c][i][j], fb[c][jj][j],
                                                               acc[i][jj], 0, 0, 0);
    }
  };
  auto a_buf = [&](int i) { return smem + i * TA; };
  auto b_buf = [&](int i) { return smem + 2 * TA + i * TB; };

  const int64_t span = ke > kb ? ke - kb : 0;
  const int64_t nfull = span / KT;
  const int64_t ntiles = (span + KT - 1) / KT;
  const int64_t a_step = A_KC ? KT : KT * p.lda;
  const int64_t b_step = B_KC ? KT : KT * p.ldb;
  const float* a_org = A + (A_KC ? m0 * p.lda + kb : kb * p.lda + m0);
  const BT* b_org = B + (B_KC ? n0 * p.ldb + kb : kb * p.ldb + n0);
  // Loads stage s into a register set (any stage: k beyond ke reads zero).
  auto load_any = [&](StageA& xa, StageB& xb, int64_t s) {
    xa.load(A, p.lda, m0, p.M, kb + s * KT, ke);
    xb.load(B, p.ldb, n0, p.N, kb + s * KT, ke);
  };
  // Loads stage s < nfull (wholly in range).
  auto load_full = [&](StageA& xa, StageB& xb, int64_t s) {
    if constexpr (VEC) xa.load_full(a_org + s * a_step);
    else xa.load(A, p.lda, m0, p.M, kb + s * KT, ke);
    if constexpr (kVecB) xb.load_full(b_org + s * b_step);
    else xb.load(B, p.ldb, n0, p.N, kb + s * KT, ke);
  };
  // Steady-state iteration on stage t (t + 2 < nfull): load stage t + 2 into
  // set `ld`, contract stage t, store stage t + 1 from set `st`. With VEC the
  // body is one basic block, scheduled as one interleave.
  auto steady = [&](StageA& lda_, StageB& ldb_, const StageA& sta, const StageB& stb,
                    int64_t t, int cur) {
    load_full(lda_, ldb_, t + 2);
    compute(a_buf(cur), b_buf(cur));
    sta.store(a_buf(cur ^ 1));
    stb.store(b_buf(cur ^ 1));
    if constexpr (SCHED) {
      // Per MFMA: one LDS fragment read for a later group; global loads
      // over the first half; the next stage's LDS writes over the second.
      constexpr int kMfma = (KT / KG) * 4 * BM * BN;
      constexpr int kVmem = StageA::kPer + StageB::kPer;
      constexpr int kDsw = kVmem;
      constexpr int kDsrGroup = (A_KC ? BM : 2 * BM) + (B_KC ? BN : 2 * BN);
      __builtin_amdgcn_sched_group_barrier(0x100, kDsrGroup, 0);
#pragma unroll
      for (int i = 0; i < kMfma; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        if (i % 2 == 0 && i / 2 < kVmem) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        if (i >= kMfma / 2 && (i - kMfma / 2) % 2 == 0 && (i - kMfma / 2) / 2 < kDsw)
          __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      }
    }
    __syncthreads();
  };

  // Early epilogue loads (kEarly: the 256x128 tile, one workgroup per CU,
  // whose epilogue has no other workgroup's k loop to hide under; 128x256
  // has no registers to spare for them in its NN group kernel): issued
  // ahead of the last stage's MFMAs, so that their latency runs under them,
  // into registers that take the dead k-loop staging registers' place. A
  // fused AddEW's addend on a whole tile, or a LoRA epilogue's T and B'
  // fragments, in one array `ep`: a work item takes at most one of them.
  // Each addend load's address is a wave-uniform tile base plus a 32-bit
  // byte offset (per-lane part + wave-uniform part), so loads in flight hold
  // no 64-bit addresses. The values summed and their order are those of the
  // loads after the k loop that the other tiles issue: the same bits.
  // Measured alone on 8192x2048x2048, 8192x2048x5504 and 8192x5504x2048:
  // the fused AddEW 0-6 us and the NT LoRA epilogue 30-86 us less per
  // launch than with the loads after the k loop; the plain form unchanged.
  constexpr bool kEarly = MT_M == 256 && MT_N == 128;
  constexpr int kLoraG = 2;  // LoRA k groups held at once: rank <= 16
  constexpr int kEp = std::max(BM * BN * 16, (BM + BN) * kLoraG * 4);
  const bool lora_epi = LORA && p.lora_t;
  const bool addend_early = kEarly && FUSED && !lora_epi && p.out && p.splits == 1 &&
                            m0 + MT_M <= p.M && n0 + MT_N <= p.N &&
                            MT_M * p.ldo * 4 < (int64_t{1} << 30);
  float ep[kEp];
  auto yv_at = [](int i, int j, int v) { return (i * BN + j) * 16 + v; };
  auto ta_at = [](int i, int g, int q) { return (i * kLoraG + g) * 4 + q; };
  auto tb_at = [](int j, int g, int q) { return BM * kLoraG * 4 + (j * kLoraG + g) * 4 + q; };
  auto load_early = [&]() {
    if constexpr (FUSED) {
      if (addend_early) {
        const char* y_base = reinterpret_cast<const char*>(p.addend + m0 * p.ldo + n0);
        const uint32_t y_lane = static_cast<uint32_t>(((wm0 + 4 * h) * p.ldo + wn0 + r) * 4);
#pragma unroll
        for (int i = 0; i < BM; ++i)
#pragma unroll
          for (int j = 0; j < BN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const uint32_t uoff = static_cast<uint32_t>(
                  ((32 * i + 8 * (v >> 2) + (v & 3)) * p.ldo + 32 * j) * 4);
              ep[yv_at(i, j, v)] = *reinterpret_cast<const float*>(y_base + (y_lane + uoff));
            }
      }
    }
    if constexpr (LORA) {
      if (lora_epi) {
        // Unconditional loads (a k group beyond the rank reads group 0 and
        // is zeroed), so that no branch splits the loads in flight.
        const int ng = p.lora_r / KG;  // 1 or 2
#pragma unroll
        for (int i = 0; i < BM; ++i) {
          const int64_t row = std::min<int64_t>(m0 + wm0 + 32 * i + r, p.M - 1);
#pragma unroll
          for (int g = 0; g < kLoraG; ++g) {
            const int k0 = (g < ng ? g : 0) * KG + 4 * h;
            const float4 q = *reinterpret_cast<const float4*>(p.lora_t + row * p.lora_ldt + k0);
            ep[ta_at(i, g, 0)] = g < ng ? q.x : 0.0f;
            ep[ta_at(i, g, 1)] = g < ng ? q.y : 0.0f;
            ep[ta_at(i, g, 2)] = g < ng ? q.z : 0.0f;
            ep[ta_at(i, g, 3)] = g < ng ? q.w : 0.0f;
          }
        }
#pragma unroll
        for (int j = 0; j < BN; ++j) {
          const int64_t col = std::min<int64_t>(n0 + wn0 + 32 * j + r, p.N - 1);
#pragma unroll
          for (int g = 0; g < kLoraG; ++g)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
              const int k = (g < ng ? g : 0) * KG + 4 * h + jj;
              const float x = p.lora_b[k * p.lora_ldb + col];
              ep[tb_at(j, g, jj)] = g < ng ? x : 0.0f;
            }
        }
      }
    }
  };

  int64_t t = 0;
  if (ntiles > 0) {
    sa0.init(p.lda, m0, p.M);
    sb0.init(p.ldb, n0, p.N);
    sa1.init(p.lda, m0, p.M);
    sb1.init(p.ldb, n0, p.N);
    if constexpr (SCL == 1) sa0.sc = sa1.sc = p.op_scale;
    if constexpr (SCL == 2) sb0.sc = sb1.sc = p.op_scale;
    load_any(sa0, sb0, 0);
    if (ntiles > 1) load_any(sa1, sb1, 1);
    sa0.store(a_buf(0));
    sb0.store(b_buf(0));
    __syncthreads();

    for (; t + 3 < nfull; t += 2) {
      steady(sa0, sb0, sa1, sb1, t, 0);
      steady(sa1, sb1, sa0, sb0, t + 1, 1);
    }
    // The remaining stages (fewer than four): masked loads where needed.
    if constexpr (!kEarly) {
      for (; t < ntiles; ++t) {
        const int cur = static_cast<int>(t & 1);
        if (t + 2 < ntiles) {
          if (cur) load_any(sa1, sb1, t + 2);
          else load_any(sa0, sb0, t + 2);
        }
        compute(a_buf(cur), b_buf(cur));
        if (t + 1 < ntiles) {
          if (cur) {
            sa0.store(a_buf(0));
            sb0.store(b_buf(0));
          } else {
            sa1.store(a_buf(1));
            sb1.store(b_buf(1));
          }
          __syncthreads();
        }
      }
    } else {
      for (; t + 1 < ntiles; ++t) {
        const int cur = static_cast<int>(t & 1);
        if (t + 2 < ntiles) {
          if (cur) load_any(sa1, sb1, t + 2);
          else load_any(sa0, sb0, t + 2);
        }
        compute(a_buf(cur), b_buf(cur));
        if (cur) {
          sa0.store(a_buf(0));
          sb0.store(b_buf(0));
        } else {
          sa1.store(a_buf(1));
          sb1.store(b_buf(1));
        }
        __syncthreads();
      }
    }
  }
  if constexpr (kEarly) {
    // The last stage, with the early epilogue loads in flight under its MFMAs
    // (one program point for the loads, whether or not there is a stage).
    // s_waitcnt vmcnt(0) (0x0F70: expcnt and lgkmcnt not waited on). No
    // k-loop load is pending here; stated, it keeps the compiler from
    // placing waits on the early loads inside the last stage's MFMAs.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    load_early();
    __builtin_amdgcn_sched_barrier(0);
    if (ntiles > 0) compute(a_buf(static_cast<int>(t & 1)), b_buf(static_cast<int>(t & 1)));
  }

  // A fused AddEW (GemmKArgs::out; FUSED instantiations, launched with one
  // slice and a plain epilogue). On a whole tile, each lane holds one base
  // pointer per array; element (i, j, v) sits a compile-time number of rows
  // and columns from it, so no per-element offsets stay live. The addends
  // are loaded first, all in flight together, then the sums are stored.
  // The value summed is the one the plain epilogue would store in C.
  if constexpr (LORA) if (p.lora_t) {
    // u = T B' block by block (k = 8g + 4h + j for MFMA j of group g, as in
    // the k loop above). Up to rank 16 every fragment of the wavefront's
    // blocks is loaded at once, before any MFMA, so their latencies overlap;
    // each block's outputs are stored right after its MFMAs (stores from one
    // base pointer per lane, with no per-element bounds, measured 5% slower:
    // the per-element form spreads them between the next block's MFMAs).
    float ta[BM][kLoraG][4], tb[BN][kLoraG][4];
    const int ng = p.lora_r / KG;
    if constexpr (kEarly) {  // loaded ahead of the last stage
#pragma unroll
      for (int i = 0; i < BM; ++i)
#pragma unroll
        for (int g = 0; g < kLoraG; ++g)
#pragma unroll
          for (int q = 0; q < 4; ++q) ta[i][g][q] = ep[ta_at(i, g, q)];
    } else {
#pragma unroll
      for (int i = 0; i < BM; ++i) {
        const int64_t row = std::min<int64_t>(m0 + wm0 + 32 * i + r, p.M - 1);
#pragma unroll
        for (int g = 0; g < kLoraG; ++g) {
          const int k0 = g * KG + 4 * h;
          float4 q = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          if (g < ng) q = *reinterpret_cast<const float4*>(p.lora_t + row * p.lora_ldt + k0);
          ta[i][g][0] = q.x; ta[i][g][1] = q.y; ta[i][g][2] = q.z; ta[i][g][3] = q.w;
        }
      }
    }
    if constexpr (kEarly) {
#pragma unroll
      for (int j = 0; j < BN; ++j)
#pragma unroll
        for (int g = 0; g < kLoraG; ++g)
#pragma unroll
          for (int q = 0; q < 4; ++q) tb[j][g][q] = ep[tb_at(j, g, q)];
    } else {
#pragma unroll
      for (int j = 0; j < BN; ++j) {
        const int64_t col = std::min<int64_t>(n0 + wn0 + 32 * j + r, p.N - 1);
#pragma unroll
        for (int g = 0; g < kLoraG; ++g)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj)
            tb[j][g][jj] = g < ng ? p.lora_b[(g * KG + 4 * h + jj) * p.lora_ldb + col] : 0.0f;
      }
    }
#pragma unroll
    for (int i = 0; i < BM; ++i)
#pragma unroll
      for (int j = 0; j < BN; ++j) {
        floatx16 u;
#pragma unroll
        for (int v = 0; v < 16; ++v) u[v] = 0.0f;
#pragma unroll
        for (int g = 0; g < kLoraG; ++g) {
          if (g >= ng) break;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj)
            u = __builtin_amdgcn_mfma_f32_32x32x2f32(ta[i][g][jj], tb[j][g][jj], u, 0, 0, 0);
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t m = m0 + wm0 + 32 * i + 8 * (v >> 2) + 4 * h + (v & 3);
          const int64_t n = n0 + wn0 + 32 * j + r;
          if (m >= p.M || n >= p.N) continue;
          const float val = dev_act(p.act, p.alpha * acc[i][j][v]);
          const float sv = p.out_scaled ? p.out_scale * u[v] : u[v];
          p.out[m * p.ldo + n] = p.lora_y_first ? val + sv : sv + val;
        }
      }
    return;
  }
  if constexpr (FUSED && kEarly) {
    if (addend_early) {
      const int64_t lm = m0 + wm0 + 4 * h, ln = n0 + wn0 + r;
      float* oa = p.out + lm * p.ldo + ln;
      float* ca = C + lm * p.ldc + ln;
#pragma unroll
      for (int i = 0; i < BM; ++i)
#pragma unroll
        for (int j = 0; j < BN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int64_t row = 32 * i + 8 * (v >> 2) + (v & 3);
            const float val = dev_act(p.act, p.alpha * acc[i][j][v]);
            const float sv = p.out_scaled ? p.out_scale * val : val;
            if (p.write_c) ca[row * p.ldc + 32 * j] = p.c_scaled ? sv : val;
            const float y = ep[yv_at(i, j, v)];
            oa[row * p.ldo + 32 * j] = p.addend_first ? y + sv : sv + y;
          }
      return;
    }
  }
  if constexpr (FUSED) {
    if (p.out && p.splits == 1 && m0 + MT_M <= p.M && n0 + MT_N <= p.N &&
        (!POST || MT_M * p.ldo * 4 < (int64_t{1} << 30))) {
      const int64_t lm = m0 + wm0 + 4 * h, ln = n0 + wn0 + r;
      const float* ya = p.addend + lm * p.ldo + ln;
      float* oa = p.out + lm * p.ldo + ln;
      float* ca = C + lm * p.ldc + ln;
      float yv[BM][BN][16];
      float pb[BN];  // POST: the AddBias values of the lane's columns
#pragma unroll
      for (int j = 0; j < BN; ++j) pb[j] = POST ? p.pbias[ln + 32 * j] : 0.0f;
      const int64_t tile0 = m0 * p.ldo + n0;
      char* post_o = POST ? reinterpret_cast<char*>(p.out + tile0) : nullptr;
      char* post_h = POST && p.hout ? reinterpret_cast<char*>(p.hout + tile0) : nullptr;
      char* post_g = POST && p.gout ? reinterpret_cast<char*>(p.gout + tile0) : nullptr;
      const uint32_t post_lane = static_cast<uint32_t>(((lm - m0) * p.ldo + (ln - n0)) * 4);
#pragma unroll
      for (int i = 0; i < BM; ++i)
#pragma unroll
        for (int j = 0; j < BN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            yv[i][j][v] = ya[(32 * i + 8 * (v >> 2) + (v & 3)) * p.ldo + 32 * j];
#pragma unroll
      for (int i = 0; i < BM; ++i)
#pragma unroll
        for (int j = 0; j < BN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int64_t row = 32 * i + 8 * (v >> 2) + (v & 3);
            const float val = dev_act(p.act, p.alpha * acc[i][j][v]);
            const float sv = p.out_scaled ? p.out_scale * val : val;
            if (p.write_c) ca[row * p.ldc + 32 * j] = p.c_scaled ? sv : val;
            const float y = yv[i][j][v];
            if constexpr (POST) {
              // 32-bit byte offsets from the tile's wave-uniform origin (the
              // tile's span is checked to fit): three output arrays with no
              // 64-bit address per element.
              const uint32_t at = post_lane + static_cast<uint32_t>((row * p.ldo + 32 * j) * 4);
              const float o = p.addend_first ? y + sv : sv + y;
              if (p.write_out) *reinterpret_cast<float*>(post_o + at) = o;
              const float hv = o + pb[j];
              if (p.hout) *reinterpret_cast<float*>(post_h + at) = hv;
              if (p.gout) *reinterpret_cast<float*>(post_g + at) = dev_act(p.pact, hv);
            } else {
              oa[row * p.ldo + 32 * j] = p.addend_first ? y + sv : sv + y;
            }
          }
      return;
    }
  }

  // A whole tile with the plain epilogue (one slice, no accumulate, bias,
  // activation or causal zeroing): one base pointer per lane, every element
  // a compile-time number of rows and columns from it, no per-element bounds
  // or epilogue branches. Stores what the general write-back below stores.
  // The 128x128x32/w2x2 tile keeps the general write-back: two of its
  // workgroups share a CU, the other's k loop hides this one's write-back,
  // and the back-to-back stores measured ~1% slower on it in the C4 step.
  constexpr bool kPlainFast =
      VEC && !(MT_M == 128 && MT_N == 128 && KT == 32 && WAVES_M == 2 && WAVES_N == 2);
  if constexpr (kPlainFast) {
    if (!p.out && p.splits == 1 && !p.accumulate && !p.bias && p.act == 0 &&
        p.causal != static_cast<int>(Causal::kLowerOut) && m0 + MT_M <= p.M &&
        n0 + MT_N <= p.N) {
      float* ca = C + (m0 + wm0 + 4 * h) * p.ldc + n0 + wn0 + r;
#pragma unroll
      for (int i = 0; i < BM; ++i)
#pragma unroll
        for (int j = 0; j < BN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            ca[(32 * i + 8 * (v >> 2) + (v & 3)) * p.ldc + 32 * j] = p.alpha * acc[i][j][v];
      return;
    }
  }

  // Write-back. Lane (h, r) of the 32x32 block holds rows 8*(v/4) + 4*h + v%4
  // of column r in accumulator element v.
#pragma unroll
  for (int i = 0; i < BM; ++i)
#pragma unroll
    for (int j = 0; j < BN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t m = m0 + wm0 + 32 * i + 8 * (v >> 2) + 4 * h + (v & 3);
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
        if (FUSED && p.out) {  // a partial tile
          const float sv = p.out_scaled ? p.out_scale * val : val;
          if (p.write_c) C[m * p.ldc + n] = p.c_scaled ? sv : val;
          const float y = p.addend[m * p.ldo + n];
          if constexpr (POST)
            FusedSum<true>(p, m * p.ldo + n, y, sv, p.pbias[n]);
          else
            p.out[m * p.ldo + n] = p.addend_first ? y + sv : sv + y;
        } else {
          C[m * p.ldc + n] = val;
        }
      }
}

template <int MT_M, int MT_N, int KT, int WAVES_M, int WAVES_N, bool A_KC, bool B_KC, bool B_I8,
          bool VEC, bool SCHED, bool FUSED, bool LORA = false, int SCL = 0, bool POST = false>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_mfma_kernel(GemmKArgs p) {
  const uint32_t tiles = static_cast<uint32_t>(p.tiles_m) * static_cast<uint32_t>(p.tiles_n);
  const uint32_t lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const uint32_t L = XcdLogical(lin, tiles * gridDim.y * gridDim.z);
  gemm_tile<MT_M, MT_N, KT, WAVES_M, WAVES_N, A_KC, B_KC, B_I8, VEC, SCHED, FUSED, LORA, SCL, POST>(
      p, L, gridDim.y);
}

// A GEMM group: up to kMaxGroup independent GEMMs of one tile config and
// operand layout in one launch (each unsplit and unbatched), member j
// owning logical work items [wg_end[j-1], wg_end[j]). The XCD remap runs
// over the whole launch, so each XCD walks a contiguous run of the members'
// tiles. Every output is computed by the same code, k order and epilogue as
// in the member's own launch: the same bits.
constexpr int kMaxGroup = kGemmGroupMax;
struct GemmGroupArgs {
  GemmKArgs m[kMaxGroup];
  uint32_t wg_end[kMaxGroup];
  uint32_t count;
};

template <int MT_M, int MT_N, int KT, int WAVES_M, int WAVES_N, bool A_KC, bool B_KC, bool LORA>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_group_kernel(GemmGroupArgs g) {
  const uint32_t total = g.wg_end[g.count - 1];
  uint32_t L = XcdLogical(blockIdx.x, total);
  uint32_t j = 0;
  while (j + 1 < g.count && L >= g.wg_end[j]) ++j;
  if (j > 0) L -= g.wg_end[j - 1];
  gemm_tile<MT_M, MT_N, KT, WAVES_M, WAVES_N, A_KC, B_KC, false, true, true, true, LORA>(g.m[j], L, 1);
}

// Launches config `cfg` of one operand-layout variant. The element-load
// form (!VEC) exists only for the small tile; the host plans it as such.
template <bool A_KC, bool B_KC, bool B_I8, bool VEC, bool SCHED = false, bool FUSED = false>
void LaunchVariant(int cfg, dim3 grid, hipStream_t s, const GemmKArgs& a) {
  const dim3 block(kCfgs[cfg].threads);
#define SEEML_GEMM_CASE(I, MM, NN, KK, WM_, WN_)                                                \
  case I:                                                                                     \
    hipLaunchKernelGGL((gemm_mfma_kernel<MM, NN, KK, WM_, WN_, A_KC, B_KC, B_I8, VEC, SCHED, FUSED>), grid, \
                       block, 0, s, a);                                                       \
    break;
  if constexpr (!VEC) {
    hipLaunchKernelGGL((gemm_mfma_kernel<64, 64, 32, 2, 2, A_KC, B_KC, B_I8, false, false, false>), grid,
                       dim3(kCfgs[kCfgSmall].threads), 0, s, a);
  } else {
    switch (cfg) {
      SEEML_GEMM_CASE(0, 128, 128, 32, 2, 2)
      SEEML_GEMM_CASE(1, 128, 128, 32, 4, 2)
      SEEML_GEMM_CASE(2, 256, 128, 32, 4, 2)
      SEEML_GEMM_CASE(3, 128, 256, 32, 2, 4)
      SEEML_GEMM_CASE(4, 128, 64, 32, 2, 2)
      SEEML_GEMM_CASE(5, 64, 64, 32, 2, 2)
      SEEML_GEMM_CASE(6, 128, 32, 32, 4, 1)
      SEEML_GEMM_CASE(7, 32, 128, 32, 1, 4)
      SEEML_GEMM_CASE(8, 64, 128, 32, 2, 2)
      SEEML_GEMM_CASE(9, 128, 64, 32, 4, 1)
      SEEML_GEMM_CASE(10, 128, 128, 16, 2, 2)
      default:
      SEEML_GEMM_CASE(11, 64, 128, 16, 2, 2)
    }
  }
#undef SEEML_GEMM_CASE
}

// The LoRA-epilogue instantiations (GemmKArgs::lora_t): the tiles the base
// projection GEMMs run on (the large tiles of the d_model >= 2048 decoders
// and the 128x64 / 64x64 / 64x128 tiles of the small ones). Returns false
// for any other config.
template <bool A_KC, bool B_KC>
bool LaunchLoraVariant(int cfg, dim3 grid, hipStream_t s, const GemmKArgs& a) {
#define SEEML_LORA_CASE(I, MM, NN, KK, WM_, WN_)                                                       \
  case I:                                                                                            \
    hipLaunchKernelGGL((gemm_mfma_kernel<MM, NN, KK, WM_, WN_, A_KC, B_KC, false, true, true, true, true>), \
                       grid, dim3(kCfgs[I].threads), 0, s, a);                                       \
    return true;
  switch (cfg) {
    SEEML_LORA_CASE(0, 128, 128, 32, 2, 2)
    SEEML_LORA_CASE(2, 256, 128, 32, 4, 2)
    SEEML_LORA_CASE(4, 128, 64, 32, 2, 2)
    SEEML_LORA_CASE(5, 64, 64, 32, 2, 2)
    SEEML_LORA_CASE(8, 64, 128, 32, 2, 2)
    SEEML_LORA_CASE(9, 128, 64, 32, 4, 1)
    default:
      return false;
  }
#undef SEEML_LORA_CASE
}

// Tile configs with a group kernel (gemm_group_kernel): the configs the
// heuristic and the autotuner pick for the decoders' projection GEMMs.
inline constexpr bool GroupCfg(int cfg) { return cfg <= 5 || cfg == 8 || cfg == 9; }

// LORA: some member takes the LoRA epilogue (its registers cost the plain
// members occupancy, so groups without one use the kernel without it).
template <bool B_KC, bool LORA>
bool LaunchGroupVariant(int cfg, dim3 grid, hipStream_t s, const GemmGroupArgs& g) {
#define SEEML_GROUP_CASE(I, MM, NN, KK, WM_, WN_)                                                 \
  case I:                                                                                       \
    hipLaunchKernelGGL((gemm_group_kernel<MM, NN, KK, WM_, WN_, true, B_KC, LORA>), grid,         \
                       dim3(kCfgs[I].threads), 0, s, g);                                         \
    return true;
  switch (cfg) {
    SEEML_GROUP_CASE(0, 128, 128, 32, 2, 2)
    SEEML_GROUP_CASE(2, 256, 128, 32, 4, 2)
    SEEML_GROUP_CASE(4, 128, 64, 32, 2, 2)
    SEEML_GROUP_CASE(5, 64, 64, 32, 2, 2)
    SEEML_GROUP_CASE(8, 64, 128, 32, 2, 2)
    SEEML_GROUP_CASE(1, 128, 128, 32, 4, 2)
    SEEML_GROUP_CASE(3, 128, 256, 32, 2, 4)
    SEEML_GROUP_CASE(9, 128, 64, 32, 4, 1)
    default:
      return false;
  }
#undef SEEML_GROUP_CASE
}

// Tile configs with scaled-load instantiations (LaunchScaledVariant): the
// small tiles the rank-64 LoRA backward's dt = s du B^T (NT, A scaled) and
// dB = t^T (s du) (TN, B scaled) run on.
inline constexpr bool ScaledCfg(int cfg) { return cfg == 4 || cfg == 5 || (cfg >= 8 && cfg <= 11); }

template <bool A_KC, bool B_KC, int SCL>
bool LaunchScaledVariant(int cfg, dim3 grid, hipStream_t s, const GemmKArgs& a) {
#define SEEML_SCALED_CASE(I, MM, NN, KK, WM_, WN_)                                                     \
  case I:                                                                                            \
    hipLaunchKernelGGL((gemm_mfma_kernel<MM, NN, KK, WM_, WN_, A_KC, B_KC, false, true, true, false, false, \
                                         SCL>),                                                      \
                       grid, dim3(kCfgs[I].threads), 0, s, a);                                       \
    return true;
  switch (cfg) {
    SEEML_SCALED_CASE(4, 128, 64, 32, 2, 2)
    SEEML_SCALED_CASE(5, 64, 64, 32, 2, 2)
    SEEML_SCALED_CASE(8, 64, 128, 32, 2, 2)
    SEEML_SCALED_CASE(9, 128, 64, 32, 4, 1)
    SEEML_SCALED_CASE(10, 128, 128, 16, 2, 2)
    SEEML_SCALED_CASE(11, 64, 128, 16, 2, 2)
    default:
      return false;
  }
#undef SEEML_SCALED_CASE
}

// The post-AddEW instantiations (GemmKArgs::pbias): the fused AddEW's GEMM
// with an AddBias (+ activation) after it, on the small tile configs (the
// rank-64 LoRA up-projections u = t B feeding the biased MLP layers).
template <bool A_KC, bool B_KC>
bool LaunchPostVariant(int cfg, dim3 grid, hipStream_t s, const GemmKArgs& a) {
#define SEEML_POST_CASE(I, MM, NN, KK, WM_, WN_)                                                      \
  case I:                                                                                            \
    hipLaunchKernelGGL((gemm_mfma_kernel<MM, NN, KK, WM_, WN_, A_KC, B_KC, false, true, true, true, false, \
                                         0, true>),                                                  \
                       grid, dim3(kCfgs[I].threads), 0, s, a);                                       \
    return true;
  switch (cfg) {
    SEEML_POST_CASE(4, 128, 64, 32, 2, 2)
    SEEML_POST_CASE(5, 64, 64, 32, 2, 2)
    SEEML_POST_CASE(8, 64, 128, 32, 2, 2)
    SEEML_POST_CASE(9, 128, 64, 32, 4, 1)
    SEEML_POST_CASE(10, 128, 128, 16, 2, 2)
    SEEML_POST_CASE(11, 64, 128, 16, 2, 2)
    default:
      return false;
  }
#undef SEEML_POST_CASE
}

// Per-layout entry points, one instantiation unit each (built in parallel).
void LaunchNN(int cfg, bool vec, dim3 grid, hipStream_t s, const GemmKArgs& a);
void LaunchNT(int cfg, bool vec, dim3 grid, hipStream_t s, const GemmKArgs& a);
void LaunchTN(int cfg, bool vec, dim3 grid, hipStream_t s, const GemmKArgs& a);
void LaunchQ8(int cfg, bool b_kc, dim3 grid, hipStream_t s, const GemmKArgs& a);
// Group launches (A k-contiguous, B row- or k-contiguous); false for a
// config without a group kernel.
bool LaunchGroupNN(int cfg, dim3 grid, hipStream_t s, const GemmGroupArgs& g);
bool LaunchGroupNT(int cfg, dim3 grid, hipStream_t s, const GemmGroupArgs& g);
// Scaled-load launches: NT with A scaled, TN with B scaled; false for a
// config without the instantiation.
bool LaunchScaledNT(int cfg, dim3 grid, hipStream_t s, const GemmKArgs& a);
bool LaunchScaledTN(int cfg, dim3 grid, hipStream_t s, const GemmKArgs& a);
// Post-AddEW launches (NN); false for a config without the instantiation.
bool LaunchPostNN(int cfg, dim3 grid, hipStream_t s, const GemmKArgs& a);

}  // namespace gemm
}  // namespace seeml_hip
