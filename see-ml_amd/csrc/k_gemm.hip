// k_gemm.hip — host side of the fp32 MFMA GEMM engine: tile planning,
// split-K, launch-shape checks and the split-K reduction kernel. The kernel
// template itself is in k_gemm_kernel.h (design notes there), instantiated
// per operand layout in k_gemm_{nn,nt,tn,q8}.hip.
//
// Serves runtime/executor/gemm.cc:173-228 (GemmNN + fused bias/act
// epilogue, GemmNT, GemmTN, GemmAccNN, GemmNNQ8/NTQ8) and the attention
// contractions of attention.cc.
#include <atomic>
#include "k_gemm_kernel.h"

namespace seeml_hip {

using gemm::CfgInfo;
using gemm::GemmKArgs;
using gemm::kCfgs;
using gemm::kNumCfgs;

namespace {

constexpr int kThreads = 256;

// Sums split-K partials in slice order and applies the epilogue, a fused
// AddEW included (batch 1).
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
    if (p.out) {
      const float sv = p.out_scaled ? p.out_scale * val : val;
      if (p.write_c) p.C[m * p.ldc + n] = p.c_scaled ? sv : val;
      const float y = p.addend[m * p.ldo + n];
      p.out[m * p.ldo + n] = p.addend_first ? y + sv : sv + y;
    } else {
      p.C[m * p.ldc + n] = val;
    }
  }
}

int64_t CeilDiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool VecOk(const void* base, int64_t ld, int64_t sb, int64_t sh, int64_t contiguous_extent) {
  return aligned16(base) && ld % 4 == 0 && sb % 4 == 0 && sh % 4 == 0 && contiguous_extent % 4 == 0;
}

}  // namespace

// Plan indices 0..kNumCfgs-1 are the MFMA tile configs; kNumCfgs selects the
// skinny (LoRA-shaped) kernels where the shape admits them.
int GemmSkinnyConfig() { return kNumCfgs; }
int GemmConfigCount() { return kNumCfgs + 1; }
const char* GemmConfigName(int cfg) {
  if (cfg == kNumCfgs) return "skinny";
  return cfg >= 0 && cfg < kNumCfgs ? kCfgs[cfg].name : "?";
}

// The heuristic takes the skinny kernels only for the shapes that stream a
// rank-wide operand through a reduction over the token rows (rowdot: N is
// the rank; colsum: a weight gradient), up to rank kSkinnyMaxRank. Wider
// ranks run on the tile kernels with split-K, which re-read the rank-wide
// operand far less (measured with the stream cold, rank 64: 8192x64x4096
// rowdot 110 -> 63 us, 64x4096x8192 colsum 85 -> 56 us; at rank 16 the two
// are within a few percent either way). A rank-K outer product (K <= 64)
// runs on the tile kernels: they time within 1% of the skinny outer kernel
// alone and their epilogue takes a following Scale + AddEW or a whole LoRA
// run. A forced skinny config still selects the outer kernel (tests).
constexpr int64_t kSkinnyMaxRank = 16;

GemmPlan PlanGemmWith(const GemmDesc& d, int forced_cfg, int forced_splits) {
  GemmPlan plan;
  const SkinnyKind kind = SkinnyKindOf(d);
  const int64_t rank = kind == SkinnyKind::kRowDot ? d.N : std::min(d.M, d.N);
  const bool skinny = forced_cfg == kNumCfgs
                          ? kind != SkinnyKind::kNone
                          : forced_cfg < 0 && (kind == SkinnyKind::kRowDot || kind == SkinnyKind::kColSum) &&
                                rank <= kSkinnyMaxRank;
  if (skinny) {
    plan.cfg = kNumCfgs;
    plan.splits = 1;
    plan.ws_bytes = SkinnyWorkspace(d);
    return plan;
  }
  if (forced_cfg >= 0 && forced_cfg < kNumCfgs) {
    plan.cfg = forced_cfg;
  } else if (d.N <= 32 && d.M > 32) {
    plan.cfg = gemm::kCfgSkinnyN;
  } else if (d.M <= 32 && d.N > 32) {
    plan.cfg = gemm::kCfgSkinnyM;
  } else {
    const int64_t big = CeilDiv(d.M, 128) * CeilDiv(d.N, 128) * d.batch;
    const int64_t mid = CeilDiv(d.M, 64) * CeilDiv(d.N, 64) * d.batch;
    plan.cfg = big >= 512 ? gemm::kCfgDefault
               : (mid >= 256 || d.M <= 64 || d.N <= 64) ? gemm::kCfgSmall : gemm::kCfgDefault;
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

namespace {
// Compute units of the current device (cached per device; engines on
// several host threads may ask at once, and all store the same value).
int DeviceCUs() {
  static std::atomic<int> cus[16] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess) {
      cus[dev].store(v, std::memory_order_relaxed);
      n = v;
    }
  }
  return n;
}
}  // namespace

GemmOrder GemmOrderOf(const GemmDesc& d) {
  const GemmPlan h = PlanGemmWith(d, -1, -1);
  GemmOrder o;
  o.skinny = h.cfg == kNumCfgs;
  o.splits = o.skinny ? 1 : h.splits;
  return o;
}

bool GemmPlanKeepsOrder(const GemmDesc& d, const GemmPlan& p) {
  const GemmOrder o = GemmOrderOf(d);
  if (o.skinny) return p.cfg == kNumCfgs;
  return p.cfg >= 0 && p.cfg < kNumCfgs && p.splits == o.splits && (p.n_split == 0 || p.splits == 1);
}

// The heuristic plan, and for large GEMMs whose 256x128 tiles leave a
// partial last round, the column split of at least two whole rounds with
// the remainder on 64x64 tiles (the autotuner's first arm). The split was
// 2-3% faster inside the C4 step on 8192x5504x2048 and 8192x32000x2048 with
// a 128x128 remainder; 64x64 tiles spread the remainder over every CU
// (8192x5504x2048: 1282 against 1319 us per pair, 128x64 1310).
GemmPlan PlanGemm(const GemmDesc& d) {
  const GemmPlan plan = PlanGemmWith(d, -1, -1);
  if (plan.cfg == kNumCfgs || plan.splits != 1) return plan;
  const GemmPlan sp = PlanGemmSplit(d, 2, gemm::kCfgSmall);
  const int64_t cus = DeviceCUs();
  if (sp.n_split > 0 && cus > 0 && CeilDiv(d.M, 256) * (sp.n_split / 128) >= 2 * cus) return sp;
  return plan;
}


// Only the 256x128 tile, whose 108 KB of LDS holds one workgroup per CU, so
// a round of the chip is exactly one tile per CU.
GemmPlan PlanGemmSplit(const GemmDesc& d, int cfg, int tail_cfg, int64_t n_split) {
  GemmPlan plan = PlanGemmWith(d, cfg, 1);
  if (d.batch != 1 || d.causal != Causal::kNone || d.b_int8 || cfg < 0 || cfg >= kNumCfgs ||
      tail_cfg < 0 || tail_cfg >= kNumCfgs || plan.splits != 1 || !GemmVecForm(d))
    return plan;
  if (n_split <= 0) {
    if (cfg != 2) return plan;
    const CfgInfo& c = kCfgs[cfg];
    const int64_t cus = DeviceCUs();
    const int64_t tm = CeilDiv(d.M, c.mt_m), bands = CeilDiv(d.N, c.mt_n);
    if (cus <= 0 || (tm * bands) % cus == 0) return plan;
    int64_t b = bands - 1;
    while (b > 0 && (tm * b) % cus != 0) --b;
    if (b == 0) return plan;
    n_split = b * c.mt_n;
  }
  if (n_split >= d.N || n_split % 4 != 0) return plan;
  plan.tail_cfg = tail_cfg;
  plan.n_split = n_split;
  return plan;
}

bool GemmVecForm(const GemmDesc& d) {
  return !d.b_int8 && VecOk(d.A, d.lda, d.a_sb, d.a_sh, d.a_kc ? d.K : d.M) &&
         VecOk(d.B, d.ldb, d.b_sb, d.b_sh, d.b_kc ? d.K : d.N) &&
         d.lda < (int64_t{1} << 23) && d.ldb < (int64_t{1} << 23);
}

// Validates a tile-kernel launch of d under plan (one column range, no
// skinny kernels) and fills its kernel arguments, grid, config and load form.
Status CheckEpilogue(const GemmDesc& d, const GemmPlan& plan) {
  if (d.lora_t && (!d.out || d.addend || d.lora_r <= 0 || d.lora_r % 8 != 0 || d.lora_r > 16 || !d.lora_b ||
                   !aligned16(d.lora_t) || d.lora_ldt % 4 != 0 || plan.splits != 1 ||
                   !GemmLoraCfgOk(plan.cfg, d.b_kc) || !d.a_kc || d.b_int8 || d.batch != 1 ||
                   d.causal != Causal::kNone || d.accumulate || d.bias || !GemmVecForm(d)))
    return Status::Fail(kUnitEngine, "Gemm: unsupported LoRA epilogue");
  if (d.post_bias && !GemmPostOk(d, plan))
    return Status::Fail(kUnitEngine, "Gemm: unsupported AddBias after the fused AddEW");
  if (!d.post_bias && (d.post_h || d.post_g || !d.write_out))
    return Status::Fail(kUnitEngine, "Gemm: post-AddEW outputs without the AddBias");
  if (d.out && !d.lora_t && (!d.addend || d.batch != 1 || d.ldc != (d.ldo ? d.ldo : d.N) || d.causal != Causal::kNone ||
                d.accumulate || d.bias))
    return Status::Fail(kUnitEngine,
                        "Gemm: a fused AddEW needs batch 1, ldc == N and a plain epilogue "
                        "(no accumulate, bias or causal mode)");
  return Status::Ok();
}

Status PrepareKArgs(const GemmDesc& d, const GemmPlan& plan, const Ctx& ctx, GemmKArgs* out,
                    dim3* grid, int* cfg_out, bool* vec_out) {
  if (Status s = CheckEpilogue(d, plan); !s) return s;
  if (d.b_int8 && !d.a_kc)
    return Status::Fail(kUnitEngine, "Gemm: unsupported int8 operand layout");
  if (!d.a_kc && d.b_kc)
    return Status::Fail(kUnitEngine, "Gemm: unsupported operand layout (A row-major in m, B k-contiguous)");

  // 16-byte vector loads need 16-byte alignment of every batch base and a
  // contiguous extent that is a multiple of 4 (a float4 is then wholly in or
  // out of range); per-lane offsets within a tile must fit 32 bits. Other
  // GEMMs (int8 B, odd shapes) take the element-load form of the small tile.
  const bool vec = GemmVecForm(d);
  if (d.out_scaled && (!d.out || !vec))
    return Status::Fail(kUnitEngine, "Gemm: a fused Scale + AddEW needs the 16-byte-load kernels");
  if (d.out && !vec && d.ldo && d.ldo != d.N)
    return Status::Fail(kUnitEngine, "Gemm: a column view's fused AddEW needs the 16-byte-load kernels");
  if (d.out && !vec) return Status::Fail(kUnitEngine, "Gemm: a fused AddEW needs the 16-byte-load kernels");
  const int cfg = vec ? plan.cfg : gemm::kCfgSmall;
  const CfgInfo& c = kCfgs[cfg];
  const int64_t tm = CeilDiv(d.M, c.mt_m), tn = CeilDiv(d.N, c.mt_n);
  // The kernel decomposes its linear workgroup id in 32 bits.
  if (tm * tn > 0x7FFFFFFF || d.batch > 65535 || plan.splits > 65535 ||
      tm * tn * c.threads > 0xFFFFFFFF || tm * tn * plan.splits * d.batch > 0xFFFFFFFF)
    return Status::Fail(kUnitEngine, "Gemm: grid exceeds launch limits");

  GemmKArgs& a = *out;
  a = GemmKArgs{};
  a.A = d.A;
  a.B = d.B;
  a.C = d.C;
  a.ws = static_cast<float*>(ctx.ws);
  a.M = d.M; a.N = d.N; a.K = d.K;
  a.lda = d.lda; a.ldb = d.ldb; a.ldc = d.ldc;
  a.heads = std::min(d.heads, d.batch);  // same (z / heads, z % heads) for z < batch; fits 32 bits
  a.batch = d.batch;
  a.a_sb = d.a_sb; a.a_sh = d.a_sh; a.b_sb = d.b_sb; a.b_sh = d.b_sh;
  a.c_sb = d.c_sb; a.c_sh = d.c_sh;
  a.alpha = d.alpha;
  a.accumulate = d.accumulate ? 1 : 0;
  a.bias = d.bias;
  a.act = d.act;
  a.causal = static_cast<int>(d.causal);
  a.splits = plan.splits;
  a.k_per_split = plan.splits > 1
                      ? CeilDiv(CeilDiv(d.K, plan.splits), gemm::kSplitAlign) * gemm::kSplitAlign
                      : d.K;
  a.tiles_m = static_cast<int>(tm);
  a.tiles_n = static_cast<int>(tn);
  a.addend = d.addend;
  a.out = d.out;
  a.addend_first = d.addend_first ? 1 : 0;
  a.write_c = d.write_c ? 1 : 0;
  a.out_scale = d.out_scale;
  a.out_scaled = d.out_scaled ? 1 : 0;
  a.c_scaled = d.c_gets_scaled ? 1 : 0;
  a.ldo = d.ldo ? d.ldo : d.N;
  a.lora_t = d.lora_t;
  a.lora_b = d.lora_b;
  a.lora_ldt = d.lora_ldt;
  a.lora_ldb = d.lora_ldb;
  a.lora_r = d.lora_r;
  a.lora_y_first = d.lora_y_first ? 1 : 0;
  a.op_scale = d.scale_stream ? d.stream_scale : 1.0f;
  a.pbias = d.post_bias;
  a.hout = d.post_h;
  a.gout = d.post_g;
  a.pact = d.post_act;
  a.write_out = d.write_out ? 1 : 0;

  *grid = dim3(static_cast<unsigned>(tm * tn), static_cast<unsigned>(plan.splits),
               static_cast<unsigned>(d.batch));
  *cfg_out = cfg;
  *vec_out = vec;
  return Status::Ok();
}

Status LaunchGemm(const GemmDesc& d, const GemmPlan& plan, const Ctx& ctx) {
  if (d.M <= 0 || d.N <= 0 || d.batch <= 0 || d.heads <= 0)
    return Status::Fail(kUnitEngine, "Gemm: empty shape");
  if (plan.n_split > 0) {
    if (plan.n_split >= d.N || plan.n_split % 4 != 0 || plan.splits != 1 || d.batch != 1 ||
        d.causal != Causal::kNone || d.b_int8 || plan.cfg < 0 || plan.cfg >= kNumCfgs ||
        plan.tail_cfg < 0 || plan.tail_cfg >= kNumCfgs)
      return Status::Fail(kUnitEngine, "Gemm: unsupported column split");
    // Two launches over column ranges of the same operands: C, B's columns,
    // bias and the fused AddEW's arrays are offset views with the full row
    // strides.
    const int64_t n1 = plan.n_split;
    GemmDesc left = d, right = d;
    left.N = n1;
    right.N = d.N - n1;
    const float* B = static_cast<const float*>(d.B);
    right.B = d.b_kc ? B + n1 * d.ldb : B + n1;
    right.C = d.C + n1;
    if (d.bias) right.bias = d.bias + n1;
    if (d.out) {
      left.ldo = right.ldo = d.ldo ? d.ldo : d.N;
      if (d.addend) right.addend = d.addend + n1;
      right.out = d.out + n1;
    }
    if (d.lora_t) right.lora_b = d.lora_b + n1;
    GemmPlan pl, pr;
    pl.cfg = plan.cfg;
    pr.cfg = plan.tail_cfg;
    if (Status s = LaunchGemm(left, pl, ctx); !s) return s;
    return LaunchGemm(right, pr, ctx);
  }
  if (d.scale_stream && plan.cfg != kNumCfgs && !GemmScaledOk(d, plan))
    return Status::Fail(kUnitEngine,
                        "Gemm: a scaled stream needs the skinny kernels or a scaled tile config");
  if (plan.cfg == kNumCfgs) {
    if (d.out) return Status::Fail(kUnitEngine, "Gemm: the skinny kernels take no fused AddEW");
    if (ctx.ws_bytes < SkinnyWorkspace(d))
      return Status::Fail(kUnitEngine, "Gemm: workspace too small for the skinny kernel");
    return LaunchSkinny(d, ctx);
  }
  if (plan.cfg < 0 || plan.cfg >= kNumCfgs) return Status::Fail(kUnitEngine, "Gemm: bad tile config");
  if (plan.splits > 1 && (d.batch != 1 || d.causal != Causal::kNone))
    return Status::Fail(kUnitEngine, "Gemm: split-K needs an unbatched, non-causal GEMM");
  if (plan.splits > 1 && ctx.ws_bytes < plan.ws_bytes)
    return Status::Fail(kUnitEngine, "Gemm: workspace too small for split-K");
  if (Status s = CheckEpilogue(d, plan); !s) return s;
  const bool vec_form = GemmVecForm(d);
  if (d.out && !d.lora_t && !vec_form && !d.out_scaled && !(d.ldo && d.ldo != d.N)) {
    // The element-load form has no fused epilogue: the GEMM stores C (always
    // safe: C's range is C's while the GEMM writes it), then the AddEW runs.
    GemmDesc plain = d;
    plain.addend = nullptr;
    plain.out = nullptr;
    if (Status s = LaunchGemm(plain, plan, ctx); !s) return s;
    return d.addend_first ? AddEW(d.addend, d.C, d.out, static_cast<size_t>(d.M * d.N), ctx)
                          : AddEW(d.C, d.addend, d.out, static_cast<size_t>(d.M * d.N), ctx);
  }
  GemmKArgs a;
  dim3 grid;
  int cfg = 0;
  bool vec = false;
  if (Status s = PrepareKArgs(d, plan, ctx, &a, &grid, &cfg, &vec); !s) return s;
  if (d.post_bias) {  // GemmPostOk: NN
    if (!gemm::LaunchPostNN(cfg, grid, ctx.stream, a))
      return Status::Fail(kUnitEngine, "Gemm: no post-AddEW kernel for this tile config");
  } else if (d.scale_stream) {  // GemmScaledOk: NT with A the stream, or TN with B
    const bool launched = d.a_kc ? gemm::LaunchScaledNT(cfg, grid, ctx.stream, a)
                                 : gemm::LaunchScaledTN(cfg, grid, ctx.stream, a);
    if (!launched) return Status::Fail(kUnitEngine, "Gemm: no scaled-load kernel for this tile config");
  } else if (d.b_int8) {
    gemm::LaunchQ8(cfg, d.b_kc, grid, ctx.stream, a);
  } else if (d.a_kc && !d.b_kc) {
    gemm::LaunchNN(cfg, vec, grid, ctx.stream, a);
  } else if (d.a_kc && d.b_kc) {
    gemm::LaunchNT(cfg, vec, grid, ctx.stream, a);
  } else {
    gemm::LaunchTN(cfg, vec, grid, ctx.stream, a);
  }
  if (Status s = LaunchStatus("Gemm"); !s) return s;
  if (plan.splits > 1) {
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(grid_for(static_cast<size_t>(d.M * d.N), kThreads, 8192)),
                       dim3(kThreads), 0, ctx.stream, a);
    return LaunchStatus("Gemm(split-K reduce)");
  }
  return Status::Ok();
}

bool GemmScaledOk(const GemmDesc& d, const GemmPlan& plan) {
  if (plan.n_split != 0 || !gemm::ScaledCfg(plan.cfg) || !GemmVecForm(d) || d.out || d.lora_t ||
      d.b_int8 || d.batch != 1 || d.causal != Causal::kNone)
    return false;
  int64_t elems = 0;
  const void* stream = SkinnyStream(d, &elems);
  if (!stream) return false;
  if (d.a_kc && d.b_kc) return stream == d.A;
  if (!d.a_kc && !d.b_kc) return stream == d.B;
  return false;
}

bool GemmPostOk(const GemmDesc& d, const GemmPlan& plan) {
  return d.post_bias && d.out && d.addend && !d.lora_t && !d.scale_stream && d.a_kc && !d.b_kc &&
         !d.b_int8 && d.batch == 1 && d.causal == Causal::kNone && !d.accumulate && !d.bias &&
         d.act == 0 && plan.splits == 1 && plan.n_split == 0 && gemm::ScaledCfg(plan.cfg) &&
         GemmVecForm(d) && (d.post_act >= 0 && d.post_act <= 3);
}

bool GemmLoraCfgOk(int cfg, bool b_kc) {
  return cfg == 2 || cfg == 4 || cfg == 5 || cfg == 8 || cfg == 9 || (cfg == 0 && b_kc);
}

bool GemmGroupFits(const GemmDesc* ds, const GemmPlan* ps, int n) {
  if (n < 2 || n > gemm::kMaxGroup) return false;
  for (int j = 0; j < n; ++j) {
    const GemmDesc& d = ds[j];
    const GemmPlan& p = ps[j];
    if (p.cfg != ps[0].cfg || !gemm::GroupCfg(p.cfg) || p.splits != 1 || p.n_split != 0 ||
        d.batch != 1 || d.causal != Causal::kNone || d.b_int8 || !d.a_kc || d.b_kc != ds[0].b_kc ||
        d.scale_stream || d.post_bias || !GemmVecForm(d) || !CheckEpilogue(d, p))
      return false;
  }
  return true;
}

Status LaunchGemmGroup(const GemmDesc* ds, const GemmPlan* ps, int n, const Ctx& ctx) {
  if (!GemmGroupFits(ds, ps, n)) return Status::Fail(kUnitEngine, "Gemm group: members do not fit one launch");
  gemm::GemmGroupArgs g{};
  uint64_t total = 0;
  for (int j = 0; j < n; ++j) {
    dim3 grid;
    int cfg = 0;
    bool vec = false;
    if (Status s = PrepareKArgs(ds[j], ps[j], ctx, &g.m[j], &grid, &cfg, &vec); !s) return s;
    total += static_cast<uint64_t>(grid.x);
    if (total > 0x7FFFFFFF / static_cast<uint64_t>(kCfgs[cfg].threads))
      return Status::Fail(kUnitEngine, "Gemm group: grid exceeds launch limits");
    g.wg_end[j] = static_cast<uint32_t>(total);
  }
  g.count = static_cast<uint32_t>(n);
  const dim3 grid(static_cast<unsigned>(total));
  const bool ok = ds[0].b_kc ? gemm::LaunchGroupNT(ps[0].cfg, grid, ctx.stream, g)
                             : gemm::LaunchGroupNN(ps[0].cfg, grid, ctx.stream, g);
  if (!ok) return Status::Fail(kUnitEngine, "Gemm group: no group kernel for this tile config");
  return LaunchStatus("Gemm group");
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
