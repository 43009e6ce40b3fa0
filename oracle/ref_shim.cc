// ref_shim.cc — TEST INFRASTRUCTURE ONLY.
//
// extern "C" entry points over the reference's own executor kernels
// (runtime/executor/*.cc, compiled in place from /root/reference by
// oracle/Makefile into oracle/_ref/libseeml_ref.so). They let the Python
// tests and bench.py's cpu_baseline leg call the real reference code through
// ctypes. This file restates nothing numeric: every function forwards to
// seeml::update_rt::kernels::* (runtime/executor/update_kernels.h:27-162).
// ref_execute mirrors the opcode switch of UpdateEngine::ExecuteRange
// (runtime/engine/update_engine.cc:306-509), which cannot be compiled here
// (update_engine.cc needs <expected>, absent from this toolchain).
#include <cstdint>
#include <cstring>

#include "compiler/backend/tuner/bandit.h"
#include "runtime/executor/update_kernels.h"
#include "source/identity/hash.h"
#include "source/parallel/parallel_for.h"
#include "source/plan/instruction.h"

namespace k = seeml::update_rt::kernels;
namespace up = seeml::update;

extern "C" {

void ref_set_threads(size_t n) { up::SetParallelThreadCount(n); }
size_t ref_threads() { return up::ParallelThreadCount(); }

uint64_t ref_plan_self_hash(const uint8_t* plan, size_t size, size_t at) {
  return up::PlanSelfHash(plan, size, at);
}
uint64_t ref_content_hash64(const uint8_t* data, size_t size) {
  return up::ContentHash64(data, size);
}

// The reference's Ucb1Bandit (compiler/backend/tuner/bandit.cc) driven the
// way AutotuneGemmTiling drives it (autotuner.cc:57-80): max(trials, arms)
// pulls, each rewarded by reward(ctx, arm). picks[t] is the t-th selection.
typedef double (*ref_arm_reward_fn)(void* ctx, uint64_t arm);
void ref_ucb1_run(uint64_t arms, double exploration, uint64_t trials, ref_arm_reward_fn reward,
                  void* ctx, uint64_t* picks, uint64_t* pulls, double* means,
                  uint64_t* best_arm) {
  up::Ucb1Bandit bandit(arms, exploration);
  const uint64_t budget = trials > arms ? trials : arms;
  for (uint64_t t = 0; t < budget; ++t) {
    const size_t arm = bandit.Select();
    picks[t] = arm;
    bandit.Update(arm, reward(ctx, arm));
  }
  for (uint64_t i = 0; i < arms; ++i) {
    pulls[i] = bandit.pulls(i);
    means[i] = bandit.meanReward(i);
  }
  *best_arm = bandit.BestArm();
}

void ref_gemm_nn(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K, const float* bias, int act) {
  k::GemmNN(A, B, C, M, N, K, bias, static_cast<up::EpilogueAct>(act));
}
void ref_gemm_nt(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K) {
  k::GemmNT(A, B, C, M, N, K);
}
void ref_gemm_tn(const float* A, const float* B, float* C, size_t M, size_t N,
                 size_t K) {
  k::GemmTN(A, B, C, M, N, K);
}
void ref_gemm_acc_nn(const float* A, const float* B, float* C, size_t M,
                     size_t N, size_t K, float alpha) {
  k::GemmAccNN(A, B, C, M, N, K, alpha);
}
void ref_gemm_nn_q8(const float* A, const int8_t* B, float* C, size_t M,
                    size_t N, size_t K, float scale, int act) {
  k::GemmNNQ8(A, B, C, M, N, K, scale, static_cast<up::EpilogueAct>(act));
}
void ref_gemm_nt_q8(const float* A, const int8_t* B, float* C, size_t M,
                    size_t N, size_t K, float scale) {
  k::GemmNTQ8(A, B, C, M, N, K, scale);
}
void ref_add_ew(const float* x, const float* y, float* o, size_t n) { k::AddEW(x, y, o, n); }
void ref_mul_ew(const float* x, const float* y, float* o, size_t n) { k::MulEW(x, y, o, n); }
void ref_add_bias(const float* x, const float* b, float* o, size_t r, size_t c) {
  k::AddBias(x, b, o, r, c);
}
void ref_scale(const float* x, float* o, float a, size_t n) { k::Scale(x, o, a, n); }
void ref_reduce_rows(const float* dy, float* db, size_t r, size_t c) { k::ReduceRows(dy, db, r, c); }
void ref_relu_fwd(const float* x, float* o, size_t n) { k::ReluFwd(x, o, n); }
void ref_relu_bwd(const float* dy, const float* x, float* dx, size_t n) { k::ReluBwd(dy, x, dx, n); }
void ref_gelu_fwd(const float* x, float* o, size_t n) { k::GeluFwd(x, o, n); }
void ref_gelu_bwd(const float* dy, const float* x, float* dx, size_t n) { k::GeluBwd(dy, x, dx, n); }
void ref_silu_fwd(const float* x, float* o, size_t n) { k::SiluFwd(x, o, n); }
void ref_silu_bwd(const float* dy, const float* x, float* dx, size_t n) { k::SiluBwd(dy, x, dx, n); }
void ref_embed_fwd(const int32_t* t, const float* tab, float* o, size_t r, size_t d) {
  k::EmbedFwd(t, tab, o, r, d);
}
void ref_fill(float* d, float v, size_t n) { k::Fill(d, v, n); }
void ref_copy(const float* s, float* d, size_t n) { k::Copy(s, d, n); }
void ref_layer_norm_fwd(const float* x, const float* g, const float* b, float* y,
                        float* mean, float* rstd, size_t r, size_t c) {
  k::LayerNormFwd(x, g, b, y, mean, rstd, r, c);
}
void ref_layer_norm_bwd(const float* dy, const float* x, const float* g,
                        const float* mean, const float* rstd, float* dx,
                        size_t r, size_t c) {
  k::LayerNormBwd(dy, x, g, mean, rstd, dx, r, c);
}
void ref_rms_norm_fwd(const float* x, const float* g, float* y, float* rstd,
                      size_t r, size_t c) {
  k::RmsNormFwd(x, g, y, rstd, r, c);
}
void ref_rms_norm_bwd(const float* dy, const float* x, const float* g,
                      const float* rstd, float* dx, size_t r, size_t c) {
  k::RmsNormBwd(dy, x, g, rstd, dx, r, c);
}
void ref_rope_fwd(const float* x, float* y, size_t B, size_t S, size_t H,
                  size_t d, float base) {
  k::RopeFwd(x, y, B, S, H, d, base);
}
void ref_rope_bwd(const float* dy, float* dx, size_t B, size_t S, size_t H,
                  size_t d, float base) {
  k::RopeBwd(dy, dx, B, S, H, d, base);
}
void ref_attn_fwd(const float* q, const float* kk, const float* v, float* o,
                  float* p, size_t B, size_t S, size_t H, size_t d) {
  k::AttnFwd(q, kk, v, o, p, B, S, H, d);
}
void ref_attn_dp(const float* dout, const float* v, float* dp, size_t B,
                 size_t S, size_t H, size_t d) {
  k::AttnDP(dout, v, dp, B, S, H, d);
}
void ref_attn_dv(const float* p, const float* dout, float* dv, size_t B,
                 size_t S, size_t H, size_t d) {
  k::AttnDV(p, dout, dv, B, S, H, d);
}
void ref_softmax_rows_bwd(const float* p, const float* dp, float* ds,
                          size_t rows, size_t cols) {
  k::SoftmaxRowsBwd(p, dp, ds, rows, cols);
}
void ref_attn_dq(const float* ds, const float* kk, float* dq, size_t B,
                 size_t S, size_t H, size_t d) {
  k::AttnDQ(ds, kk, dq, B, S, H, d);
}
void ref_attn_dk(const float* ds, const float* q, float* dk, size_t B,
                 size_t S, size_t H, size_t d) {
  k::AttnDK(ds, q, dk, B, S, H, d);
}
void ref_softmax_xent_fwd(const float* l, const int32_t* lab, float* loss,
                          float* p, size_t N, size_t C) {
  k::SoftmaxXEntFwd(l, lab, loss, p, N, C);
}
void ref_softmax_xent_bwd(const float* p, const int32_t* lab, const float* seed,
                          float* dl, size_t N, size_t C) {
  k::SoftmaxXEntBwd(p, lab, seed, dl, N, C);
}
void ref_mse_fwd(const float* p, const float* t, float* loss, size_t n) { k::MseFwd(p, t, loss, n); }
void ref_mse_bwd(const float* p, const float* t, const float* seed, float* dp, size_t n) {
  k::MseBwd(p, t, seed, dp, n);
}
void ref_kl_distill_fwd(const float* s, const float* t, float* loss, float* ps,
                        float* pt, size_t N, size_t C, float T) {
  k::KLDistillFwd(s, t, loss, ps, pt, N, C, T);
}
void ref_kl_distill_bwd(const float* ps, const float* pt, const float* seed,
                        float* dl, size_t N, size_t C, float T) {
  k::KLDistillBwd(ps, pt, seed, dl, N, C, T);
}
void ref_clip_norm(float* g, size_t n, float m) { k::ClipNorm(g, n, m); }
void ref_sgd_step(float* p, const float* g, size_t n, float lr, float wd) {
  k::SgdStep(p, g, n, lr, wd);
}
void ref_adamw_step(float* p, const float* g, float* m, float* v, size_t n,
                    float lr, float b1, float b2, float eps, float wd,
                    uint64_t step) {
  k::AdamWStep(p, g, m, v, n, lr, b1, b2, eps, wd, step);
}

// The opcode switch of UpdateEngine::ExecuteRange (update_engine.cc:306-509)
// over the reference kernels; `lr` is the step's EffectiveLr().
void ref_execute(const void* program, size_t count, uint8_t* arena,
                 const uint8_t* rodata, float lr, float beta1, float beta2,
                 float eps, float wd, uint64_t step) {
  const auto* prog = static_cast<const up::UpdateInstruction*>(program);
  auto rp = [&](uint64_t ref) -> const float* {
    const uint64_t off = up::RefOffset(ref);
    return reinterpret_cast<const float*>(
        (up::IsRodataRef(ref) ? rodata : arena) + off);
  };
  auto rq8 = [&](uint64_t ref) {
    return reinterpret_cast<const int8_t*>(rodata + up::RefOffset(ref));
  };
  auto wp = [&](uint64_t ref) {
    return reinterpret_cast<float*>(arena + up::RefOffset(ref));
  };
  auto ip = [&](uint64_t ref) {
    return reinterpret_cast<const int32_t*>(rp(ref));
  };
  auto f32 = [](uint64_t bits) {
    const uint32_t u = static_cast<uint32_t>(bits);
    float f;
    std::memcpy(&f, &u, sizeof f);
    return f;
  };
  for (size_t idx = 0; idx < count; ++idx) {
    up::UpdateInstruction ins;
    std::memcpy(&ins, prog + idx, sizeof ins);
    const auto act = up::EpilogueActOf(ins.flags);
    const size_t d0 = ins.out[0], d1 = ins.out[1], d2 = ins.out[2];
    switch (static_cast<up::OpCode>(ins.opcode)) {
      case up::OpCode::kNop: break;
      case up::OpCode::kGemmNN:
        k::GemmNN(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0, d1, d2,
                  ins.flags & up::kFlagEpilogueBias ? rp(ins.in[3]) : nullptr, act);
        break;
      case up::OpCode::kGemmNT: k::GemmNT(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0, d1, d2); break;
      case up::OpCode::kGemmTN: k::GemmTN(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0, d1, d2); break;
      case up::OpCode::kGemmAccNN:
        k::GemmAccNN(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0, d1, d2, f32(ins.in[3]));
        break;
      case up::OpCode::kGemmNNQ8:
        k::GemmNNQ8(rp(ins.in[0]), rq8(ins.in[1]), wp(ins.in[2]), d0, d1, d2, f32(ins.in[3]), act);
        break;
      case up::OpCode::kGemmNTQ8:
        k::GemmNTQ8(rp(ins.in[0]), rq8(ins.in[1]), wp(ins.in[2]), d0, d1, d2, f32(ins.in[3]));
        break;
      case up::OpCode::kAddEW: k::AddEW(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0); break;
      case up::OpCode::kMulEW: k::MulEW(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0); break;
      case up::OpCode::kAddBias: k::AddBias(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0, d1); break;
      case up::OpCode::kReluFwd: k::ReluFwd(rp(ins.in[0]), wp(ins.in[1]), d0); break;
      case up::OpCode::kReluBwd: k::ReluBwd(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0); break;
      case up::OpCode::kGeluFwd: k::GeluFwd(rp(ins.in[0]), wp(ins.in[1]), d0); break;
      case up::OpCode::kGeluBwd: k::GeluBwd(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0); break;
      case up::OpCode::kSiluFwd: k::SiluFwd(rp(ins.in[0]), wp(ins.in[1]), d0); break;
      case up::OpCode::kSiluBwd: k::SiluBwd(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0); break;
      case up::OpCode::kLayerNormFwd:
        k::LayerNormFwd(rp(ins.in[0]), rp(ins.in[1]), rp(ins.in[2]), wp(ins.in[3]),
                        wp(ins.out[1]), wp(ins.out[2]), d0 >> 32, d0 & 0xFFFFFFFFu);
        break;
      case up::OpCode::kLayerNormBwd:
        k::LayerNormBwd(rp(ins.in[0]), rp(ins.in[1]), rp(ins.in[2]), rp(ins.out[0]),
                        rp(ins.out[1]), wp(ins.in[3]), d2 >> 32, d2 & 0xFFFFFFFFu);
        break;
      case up::OpCode::kClipNorm: k::ClipNorm(wp(ins.in[0]), d0, f32(ins.in[1])); break;
      case up::OpCode::kScale: k::Scale(rp(ins.in[0]), wp(ins.in[1]), f32(ins.in[2]), d0); break;
      case up::OpCode::kReduceRows: k::ReduceRows(rp(ins.in[0]), wp(ins.in[1]), d0, d1); break;
      case up::OpCode::kSoftmaxXEntFwd:
        k::SoftmaxXEntFwd(rp(ins.in[0]), ip(ins.in[1]), wp(ins.in[2]), wp(ins.in[3]), d0, d1);
        break;
      case up::OpCode::kSoftmaxXEntBwd:
        k::SoftmaxXEntBwd(rp(ins.in[0]), ip(ins.in[1]), rp(ins.in[2]), wp(ins.in[3]), d0, d1);
        break;
      case up::OpCode::kMseFwd: k::MseFwd(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0); break;
      case up::OpCode::kMseBwd:
        k::MseBwd(rp(ins.in[0]), rp(ins.in[1]), rp(ins.in[2]), wp(ins.in[3]), d0);
        break;
      case up::OpCode::kKLDistillFwd:
        k::KLDistillFwd(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), wp(ins.in[3]),
                        wp(ins.out[0]), d1 >> 32, d1 & 0xFFFFFFFFu, f32(ins.out[2]));
        break;
      case up::OpCode::kKLDistillBwd:
        k::KLDistillBwd(rp(ins.in[0]), rp(ins.in[1]), rp(ins.in[2]), wp(ins.in[3]),
                        d0 >> 32, d0 & 0xFFFFFFFFu, f32(ins.out[1]));
        break;
      case up::OpCode::kSgdStep: k::SgdStep(wp(ins.in[0]), rp(ins.in[1]), d0, lr, wd); break;
      case up::OpCode::kAdamWStep:
        k::AdamWStep(wp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), wp(ins.in[3]), d0, lr,
                     beta1, beta2, eps, wd, step);
        break;
      case up::OpCode::kFill: k::Fill(wp(ins.in[0]), f32(ins.in[1]), d0); break;
      case up::OpCode::kCopy: k::Copy(rp(ins.in[0]), wp(ins.in[1]), d0); break;
      case up::OpCode::kRmsNormFwd:
        k::RmsNormFwd(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), wp(ins.in[3]),
                      d0 >> 32, d0 & 0xFFFFFFFFu);
        break;
      case up::OpCode::kRmsNormBwd:
        k::RmsNormBwd(rp(ins.in[0]), rp(ins.in[1]), rp(ins.in[2]), rp(ins.out[0]),
                      wp(ins.in[3]), d1 >> 32, d1 & 0xFFFFFFFFu);
        break;
      case up::OpCode::kRopeFwd:
        k::RopeFwd(rp(ins.in[0]), wp(ins.in[1]), d0 >> 32, d0 & 0xFFFFFFFFu, d1 >> 32,
                   d1 & 0xFFFFFFFFu, f32(ins.out[2]));
        break;
      case up::OpCode::kRopeBwd:
        k::RopeBwd(rp(ins.in[0]), wp(ins.in[1]), d0 >> 32, d0 & 0xFFFFFFFFu, d1 >> 32,
                   d1 & 0xFFFFFFFFu, f32(ins.out[2]));
        break;
      case up::OpCode::kAttnFwd:
        k::AttnFwd(rp(ins.in[0]), rp(ins.in[1]), rp(ins.in[2]), wp(ins.in[3]),
                   wp(ins.out[0]), d1 >> 32, d1 & 0xFFFFFFFFu, d2 >> 32, d2 & 0xFFFFFFFFu);
        break;
      case up::OpCode::kAttnDP:
        k::AttnDP(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0 >> 32, d0 & 0xFFFFFFFFu,
                  d1 >> 32, d1 & 0xFFFFFFFFu);
        break;
      case up::OpCode::kAttnDV:
        k::AttnDV(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0 >> 32, d0 & 0xFFFFFFFFu,
                  d1 >> 32, d1 & 0xFFFFFFFFu);
        break;
      case up::OpCode::kSoftmaxRowsBwd:
        k::SoftmaxRowsBwd(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0 >> 32,
                          d0 & 0xFFFFFFFFu);
        break;
      case up::OpCode::kAttnDQ:
        k::AttnDQ(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0 >> 32, d0 & 0xFFFFFFFFu,
                  d1 >> 32, d1 & 0xFFFFFFFFu);
        break;
      case up::OpCode::kAttnDK:
        k::AttnDK(rp(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0 >> 32, d0 & 0xFFFFFFFFu,
                  d1 >> 32, d1 & 0xFFFFFFFFu);
        break;
      case up::OpCode::kEmbedFwd:
        k::EmbedFwd(ip(ins.in[0]), rp(ins.in[1]), wp(ins.in[2]), d0, d1 & 0xFFFFFFFFu);
        break;
    }
  }
}

}  // extern "C"
