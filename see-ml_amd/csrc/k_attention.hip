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

size_t AttnWorkspace(size_t, size_t, size_t, size_t) { return 0; }

Status AttnFwd(const float* q, const float* k, const float* v, float* o, float* probs, size_t B,
               size_t S, size_t H, size_t d, const Ctx& c) {
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
              size_t d, const Ctx& c) {
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
