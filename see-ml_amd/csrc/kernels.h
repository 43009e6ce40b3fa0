// kernels.h — host-side launchers for the gfx950 kernel set.
//
// One launcher per executor kernel of the reference
// (runtime/executor/update_kernels.h:27-162), taking device pointers, the
// same dims, and a launch context (stream, workspace, per-step scalars).
// Launchers validate the shapes they are handed against what their grids
// assume before launching anything, and never allocate: scratch comes from
// the context's workspace, sized by the matching *_workspace_bytes query.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <initializer_list>

#include "plan_checks.h"

namespace seeml_hip {

// Per-step optimizer scalars, uploaded once per step before the step's
// graph replays (graph kernel arguments are frozen at capture). Computed on
// the host with the reference's float expressions (optimizer.cc:52-58,
// update_engine.cc:515-534) so AdamW/SGD reproduce the CPU bits.
struct alignas(64) StepScalars {
  float lr;
  float inv_bc1;
  float inv_bc2;
  float beta1;
  float beta2;
  float om_b1;
  float om_b2;
  float eps;
  float weight_decay;
  float pad[7];
};
StepScalars MakeStepScalars(const PlanHeader& h, uint64_t step);
// One launch that writes the step's scalars to `dst` (when s is set) and
// copies up to two device buffers (the batch's input and labels) into the
// arena; sizes are whole 4-byte elements.
Status StageStep(const StepScalars* s, StepScalars* dst, const void* in_src, void* in_dst,
                 size_t in_bytes, const void* lab_src, void* lab_dst, size_t lab_bytes,
                 hipStream_t stream);
// Interval timing on the device wall clock (wall_clock64): close = false
// stores the start in slot[0]; close = true adds the ticks since then to
// slot[1] and increments the count in slot[2].
Status WallStamp(uint64_t* slot, bool close, hipStream_t stream);
// Copies the loss scalar into mapped pinned host memory from the device.
Status PostLoss(const float* src, float* host_dst, hipStream_t stream);

struct Ctx {
  hipStream_t stream = nullptr;
  void* ws = nullptr;
  size_t ws_bytes = 0;
  const StepScalars* scalars = nullptr;
};

// SEEML_HIP_OK / SEEML_HIP_ERROR for a standalone C-ABI entry point; a
// failure's message is what seeml_hip_kernel_error() returns on this thread.
int ReportStandalone(const Status& s);

// ---- GEMM engine (k_gemm.hip) -------------------------------------------
enum class Causal : int {
  kNone = 0,
  kLowerOut = 1,  // write C(m,n) for n <= m, exact 0 above the diagonal
  kKLeM = 2,      // reduce only k <= m (rows of a causal P)
  kKGeM = 3,      // reduce only k >= m (columns of a causal P)
};

struct GemmDesc {
  const void* A = nullptr;
  const void* B = nullptr;
  float* C = nullptr;
  int64_t M = 0, N = 0, K = 0;
  int64_t lda = 0, ldb = 0, ldc = 0;
  bool a_kc = true;   // A(m,k) at A[m*lda + k]   (else A[k*lda + m])
  bool b_kc = false;  // B(k,n) at B[n*ldb + k]   (else B[k*ldb + n])
  bool b_int8 = false;
  int64_t batch = 1, heads = 1;  // z -> (z / heads, z % heads)
  int64_t a_sb = 0, a_sh = 0, b_sb = 0, b_sh = 0, c_sb = 0, c_sh = 0;
  float alpha = 1.0f;
  bool accumulate = false;  // C = C + alpha*AB instead of C = alpha*AB
  const float* bias = nullptr;
  int act = 0;
  Causal causal = Causal::kNone;
  // A following AddEW folded into the epilogue (tile kernels or their
  // split-K reduction; batch 1, ldc == N): out[m*N+n] = addend[m*N+n] (+) c, where c is the
  // value the GEMM stores at C(m, n) and (+) keeps the AddEW's operand order
  // (addend_first). C itself is stored only when write_c.
  // out_scaled: a Scale sits between the GEMM and the AddEW, so the AddEW
  // consumes fl(out_scale * c) (the Scale's stored value) instead of c, and
  // with c_gets_scaled the C store receives that scaled value (C then names
  // the Scale's output). Needs the 16-byte-load tile kernels (GemmVecForm).
  const float* addend = nullptr;
  float* out = nullptr;
  bool addend_first = true;
  bool write_c = true;
  bool out_scaled = false;
  float out_scale = 1.0f;
  bool c_gets_scaled = false;
  // After the fused AddEW (GemmPostOk): an AddBias of its sum o, and
  // optionally an activation of that: h = fl(o + post_bias[n]) stored to
  // post_h (when set), g = act(h) (post_act as dev_act) stored to post_g
  // (when set); o itself is stored to out only with write_out.
  const float* post_bias = nullptr;
  float* post_h = nullptr;
  float* post_g = nullptr;
  int post_act = 0;
  bool write_out = true;
  int64_t ldo = 0;  // row stride of addend and out (0: N, the fused-AddEW default)
  // A LoRA up-projection folded into the epilogue (with out; addend unused):
  // out = c (+) fl(out_scale * u) (out_scale only when out_scaled), where
  // u = T B' over lora_r (8 or 16; T [M, lora_r] with row stride
  // lora_ldt, 16-byte rows; B' [lora_r, N] with row stride lora_ldb), in
  // the k order of a tile GEMM of u, so u has that GEMM's bits. lora_y_first:
  // c is the AddEW's first operand. Tile configs of GemmLoraCfgOk, one
  // slice, A k-contiguous.
  const float* lora_t = nullptr;
  const float* lora_b = nullptr;
  int64_t lora_ldt = 0, lora_ldb = 0;
  int lora_r = 0;
  bool lora_y_first = true;
  // A Scale folded into the skinny rowdot / colsum kernels, or the tile
  // plans GemmScaledOk admits: their streamed operand (rowdot: A; colsum:
  // the [K, W] one) is read as fl(stream_scale * x), element by element, as
  // the Scale would have stored it.
  bool scale_stream = false;
  float stream_scale = 1.0f;
};

struct GemmPlan {
  int cfg = 0;      // tile configuration index
  int splits = 1;   // deterministic split-K slices
  size_t ws_bytes = 0;
  // Column split (one slice only): columns [0, n_split) run on `cfg`, the
  // rest on `tail_cfg`, as two launches. With cfg's tiles over [0, n_split)
  // a whole number of rounds of the chip, the last partial round runs on
  // smaller tiles. Every output keeps its k order: the bits are unchanged.
  int tail_cfg = -1;
  int64_t n_split = 0;
};
GemmPlan PlanGemm(const GemmDesc& d);
// `forced_cfg`/`forced_splits` >= 0 override the heuristic (autotuner arms).
GemmPlan PlanGemmWith(const GemmDesc& d, int forced_cfg, int forced_splits);
// A GEMM's summation order: the skinny kernels' own order, or the tile
// kernels' per-output k order at `splits` deterministic split-K slices (any
// tile config and any column split at one slice give the same bits). It is
// a pure function of the shape, layout and operand alignment — the
// heuristic's — so no timing can change a result's bits.
struct GemmOrder {
  bool skinny = false;
  int splits = 1;
};
GemmOrder GemmOrderOf(const GemmDesc& d);
// True when plan `p` keeps GemmOrderOf(d).
bool GemmPlanKeepsOrder(const GemmDesc& d, const GemmPlan& p);
// The column-split plan of `cfg` with `tail_cfg` on the remainder (or, with
// n_split > 0, at that column): n_split = 0 in the result when none fits
// (batched, causal or int8 GEMMs; tiles over the columns already a whole
// number of rounds; no whole-round prefix).
GemmPlan PlanGemmSplit(const GemmDesc& d, int cfg, int tail_cfg, int64_t n_split = 0);
int GemmConfigCount();
const char* GemmConfigName(int cfg);
Status LaunchGemm(const GemmDesc& d, const GemmPlan& plan, const Ctx& ctx);
// Tile configs whose kernels take the LoRA epilogue (GemmDesc::lora_t).
bool GemmLoraCfgOk(int cfg, bool b_kc);
// A tile plan that takes GemmDesc::scale_stream: a rowdot-shaped NT GEMM
// (A the stream) or a colsum-shaped TN GEMM with B the stream, on a small
// tile config with scaled-load kernels, one launch (no column split), the
// 16-byte-load form and a plain epilogue.
bool GemmScaledOk(const GemmDesc& d, const GemmPlan& plan);
// A tile plan that takes the AddBias (+ activation) after a fused AddEW
// (GemmDesc::post_bias): NN, a small tile config with the post-AddEW
// instantiation, one slice, no column split, the 16-byte-load form.
bool GemmPostOk(const GemmDesc& d, const GemmPlan& plan);
// GEMM groups: 2..4 GEMMs launched as one kernel, each output with the bits
// of its own launch. Fits: one tile config with a group kernel for all,
// each unsplit (one slice, no column split), unbatched, non-causal, in the
// 16-byte-load form with A k-contiguous and one B layout; any epilogue a
// single launch of that config takes (plain, fused AddEW, LoRA). The
// caller proves the members independent: no member reads or writes what
// another writes.
inline constexpr int kGemmGroupMax = 4;  // members of one group launch
bool GemmGroupFits(const GemmDesc* ds, const GemmPlan* ps, int n);
Status LaunchGemmGroup(const GemmDesc* ds, const GemmPlan* ps, int n, const Ctx& ctx);
// True when a tile-kernel launch of d takes the 16-byte-load form, whose
// epilogue can apply a fused Scale + AddEW (GemmDesc::out_scaled).
bool GemmVecForm(const GemmDesc& d);

// LoRA-shaped GEMMs (k_skinny.hip): one extent is the adapter rank. kOuter:
// K <= 64 (the output is the HBM stream); kRowDot: N <= 64 with A
// k-contiguous (A is the stream); kColSum: TN with min(M, N) <= 64 (the
// large [K, W] operand is the stream; k-group partials in the workspace).
enum class SkinnyKind : int { kNone = 0, kOuter = 1, kRowDot = 2, kColSum = 3 };
SkinnyKind SkinnyKindOf(const GemmDesc& d);
const char* SkinnyKindName(SkinnyKind k);
size_t SkinnyWorkspace(const GemmDesc& d);
// The operand a rowdot / colsum kernel streams (and its element count), or
// null for other shapes: the one GemmDesc::scale_stream applies to.
const void* SkinnyStream(const GemmDesc& d, int64_t* elems);
Status LaunchSkinny(const GemmDesc& d, const Ctx& ctx);
// A rowdot and a colsum GEMM over the same stream X [T, D] (the LoRA
// backward's dt = du B^T and dB = t^T du) in one pass over X: rd is the
// rowdot (A = X), cs the colsum (its large operand X). Fits: both ranks
// <= 16, one stream with one row stride, equal stream scaling. which: 1 =
// rd's output only, 2 = cs's only, 3 = both; each output has the same bits
// in every form. The caller proves the pair may run as one launch (neither
// output overlaps the other or an operand the pair reads).
bool SkinnyDualFits(const GemmDesc& rd, const GemmDesc& cs);
size_t SkinnyDualWorkspace(const GemmDesc& rd);
Status LaunchSkinnyDual(const GemmDesc& rd, const GemmDesc& cs, int which, const Ctx& ctx);
// 2..4 rowdots over the same A (the LoRA down-projections of one layer
// input: t_i = x A_i) in one pass over A. Fits: each on the skinny rowdot
// kernel with the same shape, N <= 16 and a plain epilogue. Each output has
// the bits of its rowdot's own launch. The caller proves the group may run
// as one launch at the first member's place.
bool SkinnyRowdotGroupFits(const GemmDesc* ds, int n);
Status LaunchSkinnyRowdotGroup(const GemmDesc* ds, int n, const Ctx& ctx);
// 2..4 colsums over the same large operand (the LoRA dA_j = x^T dt_j of one
// layer input) in one pass over it. Fits: each on the skinny colsum kernel
// with the same shape, rank <= 16 and a plain epilogue. Each output has the
// bits of its colsum's own launch.
bool SkinnyColsumGroupFits(const GemmDesc* ds, int n);
size_t SkinnyColsumGroupWorkspace(const GemmDesc* ds, int n);
Status LaunchSkinnyColsumGroup(const GemmDesc* ds, int n, const Ctx& ctx);
// The plan index that selects the skinny kernels (one past the tile configs).
int GemmSkinnyConfig();

// A kOuter GEMM u = A B followed in the plan by Scale and/or AddEW of its
// output, executed as one kernel (the engine proves the chain: exact operand
// matches, and no written range overlapping a read one). kind 1: s = alpha * u,
// then yout = y (+) s; kind 2: yout = y (+) u. (+) keeps the AddEW's operand
// order (y_first). u is stored unless write_u is false and s only where
// s != nullptr: the engine drops a store when the value is dead (its range is
// overwritten by the chain, or nothing observes it afterwards). The flat
// [M*N] arrays share C's indexing (ldc == N).
struct SkinnyChain {
  int kind = 0;
  float alpha = 1.0f;
  float* s = nullptr;
  const float* y = nullptr;
  float* yout = nullptr;
  bool write_u = true;
  bool y_first = true;
};
Status LaunchSkinnyChain(const GemmDesc& d, const SkinnyChain& ch, const Ctx& ctx);

// Row-major convenience forms of the reference's GEMM family.
GemmDesc GemmNNDesc(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K);
GemmDesc GemmNTDesc(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K);
GemmDesc GemmTNDesc(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K);

// ---- pointwise family (k_pointwise.hip) ---------------------------------
// A run of adjacent pointwise instructions on n elements each, executed as
// one kernel that evaluates them per element in registers. The engine proves
// the run: every operand range is identical to or disjoint from every other,
// so element i of each instruction depends only on element i of the run's
// inputs and earlier results. Value slots: 0..nin-1 hold the inputs as
// loaded, slot kPwIn + j step j's result (a unary step has b == a). Each step
// is the standalone kernel's element expression, so the stored bits are the
// run's. The kernels are compiled per program (PwProgramOf: the wirings the
// compiler's lowering produces); out[j] receives step j's result, or nothing
// when null (dead, or overwritten later in the run).
// kMulSilu: a * silu(b), the product with a SiLU output formed from its
// input (a recomputed SiLU; no instruction maps to it).
enum class PwOp : int { kAdd, kMul, kScale, kRelu, kReluBwd, kGelu, kGeluBwd, kSilu, kSiluBwd, kCopy, kMulSilu };
inline constexpr int kPwIn = 4, kPwOps = 4;
struct PwStep {
  PwOp op = PwOp::kCopy;
  int a = 0, b = 0;
};
struct PointwiseRun {
  size_t n = 0;
  int program = -1;  // PwProgramOf
  const float* in[kPwIn] = {};
  float alpha[kPwOps] = {1.0f, 1.0f, 1.0f, 1.0f};  // Scale steps
  float* out[kPwOps] = {};
};
// Index of the compiled program for these steps over nin inputs, or -1.
int PwProgramOf(int nin, const PwStep* steps, int nops);
// The SwiGLU backward's programs: over (dh, u, s, g), and over (dh, u, g)
// with s = silu(g) formed in registers (the same du bits).
inline constexpr int kPwSwiGluBwd = 1, kPwSwiGluBwdRecompute = 6;
Status LaunchPointwiseRun(const PointwiseRun& run, const Ctx& c);

Status AddEW(const float* x, const float* y, float* out, size_t n, const Ctx& c);
Status MulEW(const float* x, const float* y, float* out, size_t n, const Ctx& c);
Status AddBias(const float* x, const float* b, float* out, size_t rows, size_t cols, const Ctx& c);
Status Scale(const float* x, float* out, float alpha, size_t n, const Ctx& c);
Status ReluFwd(const float* x, float* out, size_t n, const Ctx& c);
Status ReluBwd(const float* dy, const float* x, float* dx, size_t n, const Ctx& c);
Status GeluFwd(const float* x, float* out, size_t n, const Ctx& c);
Status GeluBwd(const float* dy, const float* x, float* dx, size_t n, const Ctx& c);
Status SiluFwd(const float* x, float* out, size_t n, const Ctx& c);
Status SiluBwd(const float* dy, const float* x, float* dx, size_t n, const Ctx& c);
Status Fill(float* dst, float value, size_t n, const Ctx& c);
Status Copy(const float* src, float* dst, size_t n, const Ctx& c);
// dst[c * rows + r] = src[r * cols + c]: a [rows, cols] matrix transposed
// (the engine's k-contiguous copies of frozen GEMM weights).
Status Transpose(const float* src, float* dst, int64_t rows, int64_t cols, const Ctx& c);
Status EmbedFwd(const int32_t* tokens, const float* table, float* out, size_t rows, size_t dim,
                size_t vocab, const Ctx& c);
Status ReduceRows(const float* dy, float* db, size_t rows, size_t cols, const Ctx& c);
Status SoftmaxXEntBwd(const float* probs, const int32_t* labels, const float* seed, float* dlogits,
                      size_t N, size_t C, const Ctx& c);
Status MseBwd(const float* pred, const float* target, const float* seed, float* dpred, size_t n,
              const Ctx& c);
Status KLDistillBwd(const float* p_s, const float* p_t, const float* seed, float* dlogits,
                    size_t N, size_t C, float T, const Ctx& c);
Status SgdStep(float* p, const float* g, size_t n, const Ctx& c);
Status AdamWStep(float* p, const float* g, float* m, float* v, size_t n, const Ctx& c);

// Several AdamWStep instructions with pairwise-disjoint operands as one
// launch (same per-element expression, so the same bits). `segs` is a device
// array; AdamWMultiPlan fills first_block on the host copy and returns the
// grid size.
struct AdamWSegment {
  float* p;
  const float* g;
  float* m;
  float* v;
  uint64_t n;
  uint64_t first_block;
};
uint64_t AdamWMultiPlan(AdamWSegment* host_segs, size_t nseg);

// EvaluateMetrics' accuracy count (update_engine.cc:619-633): per row the
// first index of the largest value under strict '>' scanning from column 0
// (NaN never wins; a NaN in column 0 keeps index 0), compared with the
// row's label (negative labels never match). `partials` holds
// ArgmaxPartials(rows) u32; the exact integer total lands in *total.
size_t ArgmaxPartials(uint64_t rows);
Status ArgmaxCorrect(const float* probs, const int32_t* labels, uint64_t rows, uint64_t cols,
                     uint32_t* partials, uint64_t* total, const Ctx& c);
Status AdamWMulti(const AdamWSegment* segs, size_t nseg, uint64_t blocks, const Ctx& c);
Status RopeFwd(const float* x, float* y, size_t B, size_t S, size_t H, size_t d, float base,
               const Ctx& c);
Status RopeBwd(const float* dy, float* dx, size_t B, size_t S, size_t H, size_t d, float base,
               const Ctx& c);
// RoPE's angles for (S, d, base), precomputed: table[2 (s d/2 + c) + {0, 1}] =
// (cos t, sin t), t = s * base^(-2c/d) by the reference's recurrence: the
// values RopeFwd/Bwd compute on the fly, so results through the table are
// the same bits. RopeTableFloats(S, d) = S * d.
size_t RopeTableFloats(size_t S, size_t d);
Status RopeTable(float* table, size_t S, size_t d, float base, const Ctx& c);
// RopeFwd (dir +1) / RopeBwd (dir -1) reading a RopeTable: a pure stream
// (d % 4 == 0; x, y and the table 16-byte aligned). With x2 set, a second
// tensor of the same geometry, x2 -> y2, in the same launch, as if run after
// the first: every pair of the four ranges identical or disjoint, x2 != y.
Status RopeWithTable(const float* x, float* y, size_t B, size_t S, size_t H, size_t d,
                     const float* table, int dir, const Ctx& c, const float* x2 = nullptr,
                     float* y2 = nullptr);

// ---- row / reduction family (k_rows.hip) ----------------------------------
size_t MseFwdWorkspace(size_t n);
Status MseFwd(const float* pred, const float* target, float* loss, size_t n, const Ctx& c);
size_t ClipNormWorkspace(size_t n);
Status ClipNorm(float* g, size_t n, float max_norm, const Ctx& c);
size_t SoftmaxXEntFwdWorkspace(size_t N);
Status SoftmaxXEntFwd(const float* logits, const int32_t* labels, float* loss, float* probs,
                      size_t N, size_t C, const Ctx& c);
// SoftmaxXEntFwd, the Fill of the gradient seed (seed_slot = seed) and
// SoftmaxXEntBwd (dl from those probabilities and the seed) in one pass over
// the logits, with the three instructions' bits; probs null: not stored (no
// later reader). Fits: 16-byte aligned rows, C % 4 == 0, 2048 <= C <= 32768;
// dl, probs, the seed slot and the loss apart from the labels and from each
// other, and from the logits except dl, which may be the logits exactly.
bool XEntFwdBwdFits(const float* logits, const float* probs, const float* dl, size_t N, size_t C);
Status SoftmaxXEntFwdBwd(const float* logits, const int32_t* labels, float* loss, float* probs,
                         float seed, float* seed_slot, float* dl, size_t N, size_t C, const Ctx& c);
size_t KLDistillFwdWorkspace(size_t N);
Status KLDistillFwd(const float* s, const float* t, float* loss, float* p_s, float* p_t, size_t N,
                    size_t C, float T, const Ctx& c);
// The preceding AddEW folded into a norm forward's load: the norm's input
// x = a + b (the AddEW's operand order) is formed per row in registers and
// stored to `sum` only when store_sum; x itself is not read. The row
// operands (a, b, sum, y) may be the same range as one another but must not
// partially overlap; register-resident rows only (RowAddendForm).
struct RowPreAdd {
  const float* a = nullptr;
  const float* b = nullptr;
  float* sum = nullptr;
  bool store_sum = true;
};
Status LayerNormFwd(const float* x, const float* gamma, const float* beta, float* y, float* mean,
                    float* rstd, size_t rows, size_t cols, const Ctx& c,
                    const RowPreAdd* pre = nullptr);
// A following AddEW folded into a norm backward's write-back: out =
// addend (+) dx in the AddEW's operand order, dx itself stored only when
// store_dx. The row operands (dy, x, dx, addend, out) may be the same range
// as one another but must not partially overlap; register-resident rows only
// (RowAddendForm).
struct RowAddend {
  const float* addend = nullptr;
  float* out = nullptr;
  bool add_first = true;
  bool store_dx = true;
};
bool RowAddendForm(size_t cols, std::initializer_list<const void*> rows_base);
Status LayerNormBwd(const float* dy, const float* x, const float* gamma, const float* mean,
                    const float* rstd, float* dx, size_t rows, size_t cols, const Ctx& c,
                    const RowAddend* add = nullptr);
Status RmsNormFwd(const float* x, const float* gamma, float* y, float* rstd, size_t rows,
                  size_t cols, const Ctx& c, const RowPreAdd* pre = nullptr);
Status RmsNormBwd(const float* dy, const float* x, const float* gamma, const float* rstd,
                  float* dx, size_t rows, size_t cols, const Ctx& c,
                  const RowAddend* add = nullptr);
// causal_s > 0: the caller has proven that rows are (b, h, i) with i = row %
// causal_s, cols == causal_s, and that probs and dp hold exact +0 at every
// j > i (AttnFwd / AttnDP outputs). Those entries are then not read: their
// dS is (+0) * (0 - rowsum), the reference's expression on those values, and
// their +0 products leave the double rowsum's bits unchanged.
// Without `tail` (causal form only) a row stores only the float4s it read,
// for callers whose readers never look past them. SoftmaxRowsBwdCausalForm:
// whether the causal form applies to these operands (register-resident rows;
// the fallback reads and writes whole rows).
Status SoftmaxRowsBwd(const float* probs, const float* dp, float* ds, size_t rows, size_t cols,
                      const Ctx& c, size_t causal_s = 0, bool tail = true);
bool SoftmaxRowsBwdCausalForm(const float* probs, const float* dp, const float* ds, size_t cols);
// Causal row softmax in place over raw scores (attention forward, step 2).
Status AttnSoftmaxRows(float* p, size_t rows, size_t S, const Ctx& c);

// ---- attention family (k_attention.hip): GEMM-engine compositions -------
size_t AttnWorkspace(size_t B, size_t S, size_t H, size_t d);
// What the fused forward stores of P (the GEMM-engine form always stores it
// all): the rows up to each 32-query block's diagonal tile (kAttnStoreP) and
// the exact-zero tail beyond it (kAttnStoreTail). The engine leaves out
// what it proves no reader looks at; AttnDP's `tail` likewise.
inline constexpr int kAttnStoreP = 1, kAttnStoreTail = 2;
Status AttnFwd(const float* q, const float* k, const float* v, float* o, float* probs, size_t B,
               size_t S, size_t H, size_t d, const Ctx& c,
               int pstore = kAttnStoreP | kAttnStoreTail);
Status AttnDP(const float* dout, const float* v, float* dp, size_t B, size_t S, size_t H,
              size_t d, const Ctx& c, bool tail = true);
// Whether these operands take the fused kernels (d in {64, 128}, S % 4 == 0,
// 16-byte aligned): those read P / dS only at and below each 32-row block's
// diagonal tile, masking j > i.
bool AttnFusedPath(std::initializer_list<const float*> ptrs, size_t B, size_t S, size_t H,
                   size_t d);
Status AttnDV(const float* probs, const float* dout, float* dv, size_t B, size_t S, size_t H,
              size_t d, const Ctx& c);
Status AttnDQ(const float* ds, const float* k, float* dq, size_t B, size_t S, size_t H, size_t d,
              const Ctx& c);
Status AttnDK(const float* ds, const float* q, float* dk, size_t B, size_t S, size_t H, size_t d,
              const Ctx& c);

// Checks the last launch; returns "UpdateEngine: <what>: <hip error>".
Status LaunchStatus(const char* what);

}  // namespace seeml_hip
