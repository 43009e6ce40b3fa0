// engine.hip — the device execution engine and the C-ABI (include/seeml_hip.h).
//
// Reference boundary: UpdateEngine (runtime/engine/update_engine.h:119-242)
// loads a plan, proves it, allocates one arena and dispatches each program's
// instructions into the executor kernels (ExecuteRange,
// update_engine.cc:306-509). This engine keeps that contract on one MI355X:
//
//   open     every load-time proof (plan_checks.cc), then ONE hipMalloc'd
//            arena of round64(arena_size) bytes (zeroed, persistent image
//            uploaded) and a device copy of rodata — plan offsets are used
//            unchanged: pointer = base + RefOffset(ref).
//   build    decodes a program into its plan-ordered launch list (GEMM tile
//            plans chosen per instruction, workspace sized to the largest
//            need) and captures it once as a hipGraph on the engine stream.
//   step     step_ += 1, per-step scalars (EffectiveLr, AdamW bias
//            corrections) uploaded to a device block read by the optimizer
//            kernels, batch staged into the I/O slots, graph replayed, the
//            4-byte loss read back and checked for finiteness.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/seeml_hip.h"
#include "device_common.h"
#include "device_mem.h"
#include "kernels.h"
#include "checkpoint.h"
#include "stager.h"
#include "plan_checks.h"

namespace seeml_hip {
namespace {

constexpr size_t kAlign = 64;
size_t Round64(size_t v) { return (v + kAlign - 1) & ~(kAlign - 1); }

Status HipOk(hipError_t e, const char* what) {
  if (e == hipSuccess) return Status::Ok();
  return Status::Fail(kUnitEngine, std::string(what) + ": " + hipGetErrorString(e));
}

inline uint64_t Hi(uint64_t w) { return w >> 32; }
inline uint64_t Lo(uint64_t w) { return w & 0xFFFFFFFFu; }
float Bits(uint64_t b) {
  const uint32_t u = static_cast<uint32_t>(b);
  float f;
  std::memcpy(&f, &u, sizeof f);
  return f;
}

bool IsGemmOp(uint16_t op) {
  return op == static_cast<uint16_t>(Op::kGemmNN) || op == static_cast<uint16_t>(Op::kGemmNT) ||
         op == static_cast<uint16_t>(Op::kGemmTN) || op == static_cast<uint16_t>(Op::kGemmAccNN) ||
         op == static_cast<uint16_t>(Op::kGemmNNQ8) || op == static_cast<uint16_t>(Op::kGemmNTQ8);
}

// ---- UCB1 bandit (compiler/backend/tuner/bandit.cc:14-53) -----------------
// Deterministic: untried arms first in index order, score ties to the lowest
// index, no RNG.
// Autotune arms never change a result's bits: every arm of a GEMM keeps the
// summation order GemmOrderOf fixes from its shape (the split-K count, or
// the skinny kernels' order), and differs only in tile config or column
// split. The pick is the lowest-index arm within 1.5% of the best mean:
// standalone timings that close do not rank the tiles inside the step's
// graph, so near-ties keep the planner's hint (arm 0) or the earlier config.
constexpr double kAutotuneTileTolerance = 0.015;
constexpr double kPeakFp32MfmaFlops = 157.3e12;  // MI355X dense fp32 matrix peak

class Ucb1 {
 public:
  explicit Ucb1(size_t arms, double c = 1.0) : pulls_(arms, 0), mean_(arms, 0.0), c_(c) {}
  uint64_t pulls(size_t arm) const { return pulls_[arm]; }
  double mean(size_t arm) const { return mean_[arm]; }
  size_t Select() const {
    for (size_t i = 0; i < pulls_.size(); ++i)
      if (pulls_[i] == 0) return i;
    size_t best = 0;
    double best_score = -INFINITY;
    const double log_total = std::log(static_cast<double>(total_));
    for (size_t i = 0; i < pulls_.size(); ++i) {
      const double score =
          mean_[i] + c_ * std::sqrt(2.0 * log_total / static_cast<double>(pulls_[i]));
      if (score > best_score) {
        best_score = score;
        best = i;
      }
    }
    return best;
  }
  void Update(size_t arm, double reward) {
    ++pulls_[arm];
    ++total_;
    mean_[arm] += (reward - mean_[arm]) / static_cast<double>(pulls_[arm]);
  }
  // The lowest-index pulled arm whose mean is within `tol` (relative) of the
  // best mean: arms closer than timing noise resolve the same way every run.
  // At tol = 0 this is the reference's BestArm (the first strict maximum).
  size_t Best(double tol = 0.0) const {
    size_t best = pulls_.size();
    for (size_t i = 0; i < pulls_.size(); ++i)
      if (pulls_[i] > 0 && (best == pulls_.size() || mean_[i] > mean_[best])) best = i;
    if (best == pulls_.size()) return 0;
    for (size_t i = 0; i < best; ++i)
      if (pulls_[i] > 0 && mean_[i] >= (1.0 - tol) * mean_[best]) return i;
    return best;
  }

 private:
  std::vector<uint64_t> pulls_;
  std::vector<double> mean_;
  uint64_t total_ = 0;
  double c_;
};

}  // namespace

class Engine {
 public:
  ~Engine() { Release(); }

  Status Open(const uint8_t* plan, size_t plan_size, int device) {
    if (Status s = DecodeAndVerifyPlan(plan, plan_size, &plan_); !s) return s;
    device_ = device;
    if (Status s = HipOk(hipSetDevice(device), "hipSetDevice"); !s) return s;
    if (Status s = HipOk(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "stream"); !s)
      return s;
    const PlanHeader& h = plan_.header;
    arena_bytes_ = Round64(h.arena_size);
    if (arena_bytes_ == 0) arena_bytes_ = kAlign;
    if (Status s = HipOk(LockedMalloc(&arena_, arena_bytes_), "arena allocation failed"); !s)
      return s;
    if (Status s = HipOk(hipMemsetAsync(arena_, 0, arena_bytes_, stream_), "arena clear"); !s)
      return s;
    if (h.persist_init_size)
      if (Status s = HipOk(hipMemcpyAsync(arena_, plan + h.persist_init_offset,
                                          h.persist_init_size, hipMemcpyHostToDevice, stream_),
                           "persistent image upload");
          !s)
        return s;
    rodata_bytes_ = Round64(std::max<uint64_t>(h.rodata_size, 1));
    if (Status s = HipOk(LockedMalloc(&rodata_, rodata_bytes_), "rodata allocation failed"); !s)
      return s;
    if (h.rodata_size)
      if (Status s = HipOk(hipMemcpyAsync(rodata_, plan + h.rodata_offset, h.rodata_size,
                                          hipMemcpyHostToDevice, stream_),
                           "rodata upload");
          !s)
        return s;
    if (Status s = HipOk(LockedMalloc(&d_scalars_, sizeof(StepScalars)), "scalars"); !s) return s;
    // Pinned and mapped: the programs that end in a loss write it here from
    // the device (PostLoss), so reading it costs no copy launch.
    if (Status s = HipOk(LockedHostMalloc(&h_loss_, sizeof(float)), "pinned loss"); !s) return s;
    if (Status s = MakeWeightCopies(); !s) return s;
    if (Status s = MakeRopeTables(); !s) return s;
    for (int p = 0; p < 3; ++p) PlanCausalRows(p);
    PlanLiveness();
    for (int p = 0; p < 3; ++p) PlanCausalTails(p);
    for (int p = 0; p < 3; ++p) plans_[p].assign(plan_.program[p].size(), GemmPlan{});
    for (int p = 0; p < 3; ++p)
      for (size_t i = 0; i < plan_.program[p].size(); ++i)
        if (IsGemmOp(plan_.program[p][i].opcode)) plans_[p][i] = PlanGemm(DescOf(plan_.program[p][i]));
    for (int p = 0; p < 3; ++p) PlanDuals(p);
    if (Status s = SetStep(0); !s) return s;
    return HipOk(hipStreamSynchronize(stream_), "open");
  }

  // SoftmaxRowsBwd whose probs are the latest AttnFwd output and whose dP is
  // the latest AttnDP output, both of the same (B, H, S) with rows = B*H*S
  // and cols = S: those kernels store exact +0 above the causal diagonal,
  // so the row kernel may skip reading that half (kernels.h). Dataflow over
  // the straight-line program: the most recent instruction before idx whose
  // written bytes overlap an operand must be that producer, writing exactly
  // that range.
  void PlanCausalRows(int program) {
    const auto& prog = plan_.program[program];
    causal_rows_[program].assign(prog.size(), 0);
    std::vector<std::vector<std::pair<uint64_t, uint64_t>>> writes(prog.size());
    for (size_t i = 0; i < prog.size(); ++i) (void)WriteRangesOf(prog[i], &writes[i]);
    auto last_writer = [&](size_t idx, uint64_t off, uint64_t bytes) -> long {
      for (size_t j = idx; j-- > 0;)
        for (const auto& w : writes[j])
          if (w.first < off + bytes && off < w.first + w.second) return static_cast<long>(j);
      return -1;
    };
    for (size_t i = 0; i < prog.size(); ++i) {
      const UpdateInstruction& ins = prog[i];
      if (static_cast<Op>(ins.opcode) != Op::kSoftmaxRowsBwd) continue;
      if (IsRodataRef(ins.in[0]) || IsRodataRef(ins.in[1])) continue;
      const uint64_t rows = Hi(ins.out[0]), cols = Lo(ins.out[0]);
      const uint64_t bytes = rows * cols * sizeof(float);
      const long wp = last_writer(i, RefOffset(ins.in[0]), bytes);
      const long wd = last_writer(i, RefOffset(ins.in[1]), bytes);
      if (wp < 0 || wd < 0) continue;
      const UpdateInstruction& f = prog[static_cast<size_t>(wp)];
      const UpdateInstruction& g = prog[static_cast<size_t>(wd)];
      if (static_cast<Op>(f.opcode) != Op::kAttnFwd || static_cast<Op>(g.opcode) != Op::kAttnDP)
        continue;
      // AttnFwd: out[0] = probs, B<<32|S in out[1], H<<32|d in out[2];
      // AttnDP: in[2] = dP, B<<32|S in out[0], H<<32|d in out[1].
      if (f.out[0] != ins.in[0] || g.in[2] != ins.in[1]) continue;
      if (f.out[1] != g.out[0] || Hi(f.out[2]) != Hi(g.out[1])) continue;
      const uint64_t B = Hi(f.out[1]), S = Lo(f.out[1]), H = Hi(f.out[2]);
      if (S != cols || B * H * S != rows) continue;
      causal_rows_[program][i] = S;
    }
  }

  // ---- k-contiguous copies of frozen weights ---------------------------------
  // A GemmNN whose B is a frozen weight (rodata, [K, N] row-major) runs as
  // GemmNT on a transposed copy [N, K] made once here: the same kernel is a
  // few percent faster with both operands k-contiguous (8192x5504x2048:
  // ~137 against ~132 TFLOP/s), and the per-output k order is the same in
  // both layouts, so the results are bit-identical (tested). Rodata is never
  // written after open, so the copies never go stale. Dense shapes only
  // (min(K, N) >= 64, K % 4 == 0 for 16-byte rows).
  struct WeightCopy {
    uint64_t off = 0;
    int64_t K = 0, N = 0;
    const float* t = nullptr;
  };

  Status MakeWeightCopies() {
    wcopies_.clear();
    size_t total = 0;
    for (int p = 0; p < 3; ++p)
      for (const UpdateInstruction& ins : plan_.program[p]) {
        if (static_cast<Op>(ins.opcode) != Op::kGemmNN || !IsRodataRef(ins.in[1])) continue;
        const int64_t K = ins.out[2], N = ins.out[1];
        if (K < 64 || N < 64 || K % 4 != 0 || ins.out[0] < 64) continue;
        const uint64_t off = RefOffset(ins.in[1]);
        bool seen = false;
        for (const WeightCopy& w : wcopies_) seen = seen || (w.off == off && w.K == K && w.N == N);
        if (seen) continue;
        WeightCopy w;
        w.off = off;
        w.K = K;
        w.N = N;
        w.t = reinterpret_cast<const float*>(total);  // offset for now
        total += Round64(static_cast<uint64_t>(K * N) * sizeof(float));
        wcopies_.push_back(w);
      }
    if (wcopies_.empty()) return Status::Ok();
    if (Status s = HipOk(LockedMalloc(&wcopy_buf_, total), "weight copies allocation failed"); !s)
      return s;
    const Ctx c = MakeCtx();
    for (WeightCopy& w : wcopies_) {
      float* dst = reinterpret_cast<float*>(wcopy_buf_ + reinterpret_cast<uintptr_t>(w.t));
      w.t = dst;
      if (Status s = Transpose(reinterpret_cast<const float*>(rodata_ + w.off), dst, w.K, w.N, c); !s)
        return s;
    }
    return Status::Ok();
  }

  // RoPE angle tables, one per distinct (S, d, base) of the plan's RoPE
  // instructions with d % 4 == 0 (kernels.h RopeTable: the same bits).
  struct RopeTab {
    uint64_t S = 0, d = 0, base_bits = 0;
    float* t = nullptr;
  };

  Status MakeRopeTables() {
    ropetabs_.clear();
    size_t total = 0;
    for (int p = 0; p < 3; ++p)
      for (const UpdateInstruction& ins : plan_.program[p]) {
        const auto op = static_cast<Op>(ins.opcode);
        if (op != Op::kRopeFwd && op != Op::kRopeBwd) continue;
        const uint64_t S = Lo(ins.out[0]), d = Lo(ins.out[1]);
        if (S == 0 || d == 0 || d % 4 != 0 || S * d > 0xFFFFFFFFu) continue;
        bool seen = false;
        for (const RopeTab& r : ropetabs_) seen = seen || (r.S == S && r.d == d && r.base_bits == ins.out[2]);
        if (seen) continue;
        RopeTab r;
        r.S = S;
        r.d = d;
        r.base_bits = ins.out[2];
        r.t = reinterpret_cast<float*>(total);  // offset for now
        total += Round64(RopeTableFloats(S, d) * sizeof(float));
        ropetabs_.push_back(r);
      }
    if (ropetabs_.empty()) return Status::Ok();
    if (Status s = HipOk(LockedMalloc(&ropetab_buf_, total), "RoPE tables allocation failed"); !s)
      return s;
    const Ctx c = MakeCtx();
    for (RopeTab& r : ropetabs_) {
      r.t = reinterpret_cast<float*>(ropetab_buf_ + reinterpret_cast<uintptr_t>(r.t));
      if (Status s = RopeTable(r.t, r.S, r.d, Bits(r.base_bits), c); !s) return s;
    }
    return Status::Ok();
  }

  const float* RopeTableOf(uint64_t S, uint64_t d, uint64_t base_bits) const {
    for (const RopeTab& r : ropetabs_)
      if (r.S == S && r.d == d && r.base_bits == base_bits) return r.t;
    return nullptr;
  }

  const float* WeightCopyOf(uint64_t ref, int64_t K, int64_t N) const {
    if (!IsRodataRef(ref)) return nullptr;
    for (const WeightCopy& w : wcopies_)
      if (w.off == RefOffset(ref) && w.K == K && w.N == N) return w.t;
    return nullptr;
  }

  // ---- liveness of transient values ---------------------------------------
  // A fused launch may leave out the store of an intermediate value that
  // nothing observes. The plan's transient segment is assigned by liveness
  // within one program (arena_binder.cc:25-98; the values that must outlive
  // it, the loss and the gradients, are pinned there), so a transient value
  // never carries from one run of a program into another. Observed after
  // every program: the persistent segment and the I/O slots; after the train
  // and eval programs also the loss, after the eval program the probabilities
  // its accuracy reads, after the merge program the deltas the host reads
  // back. (Bytes one program leaves behind are no other program's input.)
  using Ranges = std::vector<std::pair<uint64_t, uint64_t>>;

  static bool Overlaps(const Ranges& rs, uint64_t off, uint64_t bytes) {
    for (const auto& r : rs)
      if (r.first < off + bytes && off < r.first + r.second) return true;
    return false;
  }

  void PlanLiveness() {
    const PlanHeader& h = plan_.header;
    const int kTr = static_cast<int>(Program::kTrain), kEv = static_cast<int>(Program::kEval),
              kMg = static_cast<int>(Program::kMerge);
    for (int p = 0; p < 3; ++p) {
      Ranges& o = observed_[p];
      o.clear();
      o.emplace_back(0, h.persistent_size);
      if (h.input_ref != kNullRef) o.emplace_back(RefOffset(h.input_ref), h.input_floats * 4);
      if (h.label_ref != kNullRef) o.emplace_back(RefOffset(h.label_ref), h.label_bytes);
      if (h.loss_ref != kNullRef && (p == kTr || p == kEv))
        o.emplace_back(RefOffset(h.loss_ref), sizeof(float));
      if (plan_.eval_probs_ref != kNullRef && p == kEv)
        o.emplace_back(RefOffset(plan_.eval_probs_ref),
                       plan_.eval_softmax_rows * plan_.eval_softmax_cols * sizeof(float));
      if (p == kMg)
        for (const EmitEntry& e : plan_.emit) o.emplace_back(e.arena_offset, e.byte_size);
    }
    for (int p = 0; p < 3; ++p) {
      const auto& prog = plan_.program[p];
      depends_[p].assign(prog.size(), Ranges{});
      writes_[p].assign(prog.size(), Ranges{});
      for (size_t i = 0; i < prog.size(); ++i) {
        if (!DependRangesOf(prog[i], &depends_[p][i]))
          depends_[p][i].assign(1, {0, ~uint64_t{0}});  // unknown: depends on everything
        if (!WriteRangesOf(prog[i], &writes_[p][i])) writes_[p][i].clear();  // overwrites nothing
      }
    }
  }

  // True when the value instruction k of `program` leaves in the arena bytes
  // [off, off + bytes) is observed by nothing: walking the program from
  // k + 1, no later instruction depends on a byte of it before that byte is
  // overwritten, and no byte still holding it when the program ends is one
  // the host reads then (the observed ranges are read only between
  // programs, so bytes overwritten within the program never show the value).
  // Instructions [skip_lo, skip_hi) count with their writes only: a caller
  // that knows they take the value another way.
  bool DeadAfter(int program, size_t k, uint64_t off, uint64_t bytes, size_t skip_lo = 0,
                 size_t skip_hi = 0) const {
    Ranges live{{off, bytes}};  // the bytes still holding the value
    for (size_t j = k + 1; j < depends_[program].size() && !live.empty(); ++j) {
      if (j < skip_lo || j >= skip_hi)
        for (const auto& r : live)
          if (Overlaps(depends_[program][j], r.first, r.second)) return false;
      for (const auto& w : writes_[program][j]) {
        Ranges rest;
        for (const auto& r : live) {
          const uint64_t lo = r.first, hi = r.first + r.second;
          const uint64_t wlo = w.first, whi = w.first + w.second;
          if (whi <= lo || hi <= wlo) { rest.push_back(r); continue; }
          if (lo < wlo) rest.emplace_back(lo, wlo - lo);
          if (whi < hi) rest.emplace_back(whi, hi - whi);
        }
        live.swap(rest);
      }
    }
    for (const auto& r : live)
      if (Overlaps(observed_[program], r.first, r.second)) return false;
    return true;
  }

  // ---- causal tails ---------------------------------------------------------
  // P (AttnFwd), dP (AttnDP) and dS (a causal SoftmaxRowsBwd) hold exact
  // zeros above each row's diagonal. Past each 32-row block's diagonal tile
  // those zeros are read only by whole-row readers: the fused DV/DQ/DK
  // kernels and the causal SoftmaxRowsBwd never look there (they stop at the
  // diagonal tile and mask j > i themselves). So a producer skips that tail
  // when every reader of its output, up to the output's full overwrite, is
  // one of those on exactly that tensor and geometry; an AttnFwd whose P has
  // no reader at all (the eval program) stores no P. A transient that nobody
  // reads is never observed (see liveness): only the bytes change, not a
  // result.
  void PlanCausalTails(int program) {
    const auto& prog = plan_.program[program];
    tails_[program].assign(prog.size(), static_cast<uint8_t>(kAttnStoreP | kAttnStoreTail));
    for (size_t k = 0; k < prog.size(); ++k) {
      const UpdateInstruction& ins = prog[k];
      const auto op = static_cast<Op>(ins.opcode);
      uint64_t ref = kNullRef, bs = 0, hd = 0;  // the produced tensor and its (B|S, H|d)
      if (op == Op::kAttnFwd) {
        bs = ins.out[1], hd = ins.out[2], ref = ins.out[0];
        if (!AttnFusedPath({RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), WP(ins.in[3]), WP(ref)},
                           Hi(bs), Lo(bs), Hi(hd), Lo(hd)))
          continue;
      } else if (op == Op::kAttnDP) {
        bs = ins.out[0], hd = ins.out[1], ref = ins.in[2];
        if (!AttnFusedPath({RP(ins.in[0]), RP(ins.in[1]), WP(ref)}, Hi(bs), Lo(bs), Hi(hd), Lo(hd)))
          continue;
      } else if (op == Op::kSoftmaxRowsBwd && causal_rows_[program][k]) {
        ref = ins.in[2];
        if (!SoftmaxRowsBwdCausalForm(RP(ins.in[0]), RP(ins.in[1]), WP(ref), Lo(ins.out[0])))
          continue;
      } else {
        continue;
      }
      if (IsRodataRef(ref)) continue;
      const uint64_t rows = op == Op::kSoftmaxRowsBwd ? Hi(ins.out[0]) : 0;
      const uint64_t S = op == Op::kSoftmaxRowsBwd ? Lo(ins.out[0]) : Lo(bs);
      const uint64_t bytes = (op == Op::kSoftmaxRowsBwd ? rows : Hi(bs) * Hi(hd) * S) * S * 4;
      // Whether reader j takes the tensor through a tail-blind path.
      auto blind = [&](size_t j) {
        const UpdateInstruction& r = prog[j];
        const auto rop = static_cast<Op>(r.opcode);
        if (rop == Op::kSoftmaxRowsBwd)
          return causal_rows_[program][j] != 0 && (r.in[0] == ref || r.in[1] == ref) &&
                 r.in[2] != ref &&
                 SoftmaxRowsBwdCausalForm(RP(r.in[0]), RP(r.in[1]), WP(r.in[2]), Lo(r.out[0]));
        if (rop != Op::kAttnDV && rop != Op::kAttnDQ && rop != Op::kAttnDK) return false;
        if (r.in[0] != ref || r.in[1] == ref || r.in[2] == ref) return false;
        const uint64_t rB = Hi(r.out[0]), rS = Lo(r.out[0]), rH = Hi(r.out[1]), rd = Lo(r.out[1]);
        const bool same = op == Op::kSoftmaxRowsBwd ? (rS == S && rB * rH * rS == rows)
                                                    : (r.out[0] == bs && r.out[1] == hd);
        return same && AttnFusedPath({RP(r.in[0]), RP(r.in[1]), WP(r.in[2])}, rB, rS, rH, rd);
      };
      bool tail = Overlaps(observed_[program], RefOffset(ref), bytes), read = tail;
      Ranges live{{RefOffset(ref), bytes}};
      for (size_t j = k + 1; j < prog.size() && !live.empty() && !tail; ++j) {
        bool touches = false;
        for (const auto& l : live) touches = touches || Overlaps(depends_[program][j], l.first, l.second);
        if (touches) {
          read = true;
          if (!blind(j)) tail = true;
        }
        for (const auto& w : writes_[program][j]) {
          Ranges rest;
          for (const auto& l : live) {
            const uint64_t lo = l.first, hi = l.first + l.second, wlo = w.first, whi = w.first + w.second;
            if (whi <= lo || hi <= wlo) { rest.push_back(l); continue; }
            if (lo < wlo) rest.emplace_back(lo, wlo - lo);
            if (whi < hi) rest.emplace_back(whi, hi - whi);
          }
          live.swap(rest);
        }
      }
      uint8_t f = static_cast<uint8_t>(kAttnStoreP | (tail ? kAttnStoreTail : 0));
      if (op == Op::kAttnFwd && !read) f = 0;  // P is read by nothing
      tails_[program][k] = f;
    }
  }

  // ---- instruction decode ------------------------------------------------
  const float* RP(uint64_t ref) const {
    return reinterpret_cast<const float*>((IsRodataRef(ref) ? rodata_ : arena_) + RefOffset(ref));
  }
  float* WP(uint64_t ref) const { return reinterpret_cast<float*>(arena_ + RefOffset(ref)); }
  const int32_t* IP(uint64_t ref) const { return reinterpret_cast<const int32_t*>(RP(ref)); }

  // The GEMM family's operand layouts (gemm.cc:173-228, instruction.h:29-33).
  GemmDesc DescOf(const UpdateInstruction& ins) const {
    const auto op = static_cast<Op>(ins.opcode);
    const int64_t M = ins.out[0], N = ins.out[1], K = ins.out[2];
    const float* A = RP(ins.in[0]);
    const void* B = RP(ins.in[1]);
    float* C = WP(ins.in[2]);
    GemmDesc d;
    switch (op) {
      case Op::kGemmNT: d = GemmNTDesc(A, static_cast<const float*>(B), C, M, N, K); break;
      case Op::kGemmTN: d = GemmTNDesc(A, static_cast<const float*>(B), C, M, N, K); break;
      case Op::kGemmNTQ8:
        d = GemmNTDesc(A, nullptr, C, M, N, K);
        d.B = B;
        d.b_int8 = true;
        d.alpha = Bits(ins.in[3]);
        break;
      default:
        d = GemmNNDesc(A, nullptr, C, M, N, K);
        d.B = B;
        if (op == Op::kGemmNN)
          if (const float* bt = WeightCopyOf(ins.in[1], K, N))
            d = GemmNTDesc(A, bt, C, M, N, K);  // B^T k-contiguous: the same products
        break;
    }
    if (op == Op::kGemmNN) {
      if (ins.flags & kFlagEpilogueBias) d.bias = RP(ins.in[3]);
      d.act = static_cast<int>(ActOf(ins.flags));
    } else if (op == Op::kGemmAccNN) {
      d.alpha = Bits(ins.in[3]);
      d.accumulate = true;
    } else if (op == Op::kGemmNNQ8) {
      d.b_int8 = true;
      d.alpha = Bits(ins.in[3]);
      d.act = static_cast<int>(ActOf(ins.flags));
    }
    return d;
  }

  size_t WorkspaceFor(int program, size_t idx) const {
    const UpdateInstruction& ins = plan_.program[program][idx];
    const auto op = static_cast<Op>(ins.opcode);
    if (IsGemmOp(ins.opcode)) {
      if (idx < cs_group_of_[program].size() && cs_group_of_[program][idx] >= 0) {
        const ColsumGroup& g = cs_groups_[program][cs_group_of_[program][idx]];
        if (idx == g.members.back()) {
          GemmDesc ds[4];
          for (size_t j = 0; j < g.members.size(); ++j) ds[j] = DescOf(plan_.program[program][g.members[j]]);
          return std::max(plans_[program][idx].ws_bytes,
                          SkinnyColsumGroupWorkspace(ds, static_cast<int>(g.members.size())));
        }
      }
      if (duals_[program][idx] >= 0)
        return std::max(plans_[program][idx].ws_bytes, SkinnyDualWorkspace(DualRowdot(program, idx)));
      return plans_[program][idx].ws_bytes;
    }
    switch (op) {
      case Op::kMseFwd: return MseFwdWorkspace(ins.out[0]);
      case Op::kClipNorm: return ClipNormWorkspace(ins.out[0]);
      case Op::kSoftmaxXEntFwd: return SoftmaxXEntFwdWorkspace(ins.out[0]);
      case Op::kKLDistillFwd: return KLDistillFwdWorkspace(Hi(ins.out[1]));
      default: return 0;
    }
  }

  // ExecuteRange's switch (update_engine.cc:309-508), one launch sequence per
  // instruction.
  Status Dispatch(int program, size_t idx, const Ctx& c) const {
    const UpdateInstruction& ins = plan_.program[program][idx];
    const uint64_t d0 = ins.out[0], d1 = ins.out[1], d2 = ins.out[2];
    switch (static_cast<Op>(ins.opcode)) {
      case Op::kNop: return Status::Ok();
      case Op::kGemmNN: case Op::kGemmNT: case Op::kGemmTN: case Op::kGemmAccNN:
      case Op::kGemmNNQ8: case Op::kGemmNTQ8:
        if (duals_[program][idx] >= 0) return LaunchDual(program, idx, 0, nullptr, 1.0f, c);
        return LaunchGemm(DescOf(ins), plans_[program][idx], c);
      case Op::kAddEW: return AddEW(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), d0, c);
      case Op::kMulEW: return MulEW(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), d0, c);
      case Op::kAddBias: return AddBias(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), d0, d1, c);
      case Op::kReluFwd: return ReluFwd(RP(ins.in[0]), WP(ins.in[1]), d0, c);
      case Op::kReluBwd: return ReluBwd(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), d0, c);
      case Op::kGeluFwd: return GeluFwd(RP(ins.in[0]), WP(ins.in[1]), d0, c);
      case Op::kGeluBwd: return GeluBwd(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), d0, c);
      case Op::kSiluFwd: return SiluFwd(RP(ins.in[0]), WP(ins.in[1]), d0, c);
      case Op::kSiluBwd: return SiluBwd(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), d0, c);
      case Op::kScale: return Scale(RP(ins.in[0]), WP(ins.in[1]), Bits(ins.in[2]), d0, c);
      case Op::kReduceRows: return ReduceRows(RP(ins.in[0]), WP(ins.in[1]), d0, d1, c);
      case Op::kLayerNormFwd:
        return LayerNormFwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), WP(ins.in[3]),
                            WP(ins.out[1]), WP(ins.out[2]), Hi(d0), Lo(d0), c);
      case Op::kLayerNormBwd:
        return LayerNormBwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), RP(ins.out[0]),
                            RP(ins.out[1]), WP(ins.in[3]), Hi(d2), Lo(d2), c);
      case Op::kClipNorm: return ClipNorm(WP(ins.in[0]), d0, Bits(ins.in[1]), c);
      case Op::kSoftmaxXEntFwd:
        return SoftmaxXEntFwd(RP(ins.in[0]), IP(ins.in[1]), WP(ins.in[2]), WP(ins.in[3]), d0, d1,
                              c);
      case Op::kSoftmaxXEntBwd:
        return SoftmaxXEntBwd(RP(ins.in[0]), IP(ins.in[1]), RP(ins.in[2]), WP(ins.in[3]), d0, d1,
                              c);
      case Op::kMseFwd: return MseFwd(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), d0, c);
      case Op::kMseBwd:
        return MseBwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), WP(ins.in[3]), d0, c);
      case Op::kKLDistillFwd:
        return KLDistillFwd(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), WP(ins.in[3]),
                            WP(ins.out[0]), Hi(d1), Lo(d1), Bits(d2), c);
      case Op::kKLDistillBwd:
        return KLDistillBwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), WP(ins.in[3]), Hi(d0),
                            Lo(d0), Bits(d1), c);
      case Op::kSgdStep: return SgdStep(WP(ins.in[0]), RP(ins.in[1]), d0, c);
      case Op::kAdamWStep:
        return AdamWStep(WP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), WP(ins.in[3]), d0, c);
      case Op::kFill: return Fill(WP(ins.in[0]), Bits(ins.in[1]), d0, c);
      case Op::kCopy: return Copy(RP(ins.in[0]), WP(ins.in[1]), d0, c);
      case Op::kRmsNormFwd:
        return RmsNormFwd(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), WP(ins.in[3]), Hi(d0),
                          Lo(d0), c);
      case Op::kRmsNormBwd:
        return RmsNormBwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), RP(ins.out[0]),
                          WP(ins.in[3]), Hi(d1), Lo(d1), c);
      case Op::kRopeFwd:
      case Op::kRopeBwd: {
        const int dir = static_cast<Op>(ins.opcode) == Op::kRopeFwd ? 1 : -1;
        if (const float* t = RopeTableOf(Lo(d0), Lo(d1), d2); t && aligned16(RP(ins.in[0])) &&
            aligned16(WP(ins.in[1])))
          return RopeWithTable(RP(ins.in[0]), WP(ins.in[1]), Hi(d0), Lo(d0), Hi(d1), Lo(d1), t,
                               dir, c);
        return dir > 0 ? RopeFwd(RP(ins.in[0]), WP(ins.in[1]), Hi(d0), Lo(d0), Hi(d1), Lo(d1),
                                 Bits(d2), c)
                       : RopeBwd(RP(ins.in[0]), WP(ins.in[1]), Hi(d0), Lo(d0), Hi(d1), Lo(d1),
                                 Bits(d2), c);
      }
      case Op::kAttnFwd:
        return AttnFwd(RP(ins.in[0]), RP(ins.in[1]), RP(ins.in[2]), WP(ins.in[3]),
                       WP(ins.out[0]), Hi(d1), Lo(d1), Hi(d2), Lo(d2), c, tails_[program][idx]);
      case Op::kAttnDP:
        return AttnDP(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), Hi(d0), Lo(d0), Hi(d1), Lo(d1), c,
                      (tails_[program][idx] & kAttnStoreTail) != 0);
      case Op::kAttnDV:
        return AttnDV(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), Hi(d0), Lo(d0), Hi(d1), Lo(d1), c);
      case Op::kSoftmaxRowsBwd:
        return SoftmaxRowsBwd(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), Hi(d0), Lo(d0), c,
                              causal_rows_[program][idx],
                              (tails_[program][idx] & kAttnStoreTail) != 0);
      case Op::kAttnDQ:
        return AttnDQ(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), Hi(d0), Lo(d0), Hi(d1), Lo(d1), c);
      case Op::kAttnDK:
        return AttnDK(RP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), Hi(d0), Lo(d0), Hi(d1), Lo(d1), c);
      case Op::kEmbedFwd:
        return EmbedFwd(IP(ins.in[0]), RP(ins.in[1]), WP(ins.in[2]), d0, Lo(d1), Hi(d1), c);
    }
    return Status::Fail(kUnitEngine, "unknown opcode " + std::to_string(ins.opcode));
  }

  Ctx MakeCtx() const {
    Ctx c;
    c.stream = stream_;
    c.ws = ws_;
    c.ws_bytes = ws_bytes_;
    c.scalars = d_scalars_;
    return c;
  }

  Status EnsureWorkspace(int program) {
    size_t need = 0;
    for (size_t i = 0; i < plan_.program[program].size(); ++i)
      need = std::max(need, WorkspaceFor(program, i));
    if (need <= ws_bytes_) return Status::Ok();
    // Growing the workspace moves it: every captured graph holds the old
    // address, so all of them are rebuilt on next use.
    if (Status s = HipOk(hipStreamSynchronize(stream_), "workspace sync"); !s) return s;
    if (ws_) (void)LockedFree(ws_);
    ws_ = nullptr;
    ws_bytes_ = 0;
    if (Status s = HipOk(LockedMalloc(&ws_, Round64(need)), "workspace allocation"); !s) return s;
    ws_bytes_ = Round64(need);
    for (int p = 0; p < 3; ++p) DropGraph(p);
    return Status::Ok();
  }

  void DropGraph(int p) {
    std::lock_guard<std::recursive_mutex> lock(DeviceMemMutex());
    for (Segment& g : segs_[p]) {
      if (g.exec) (void)hipGraphExecDestroy(g.exec);
      if (g.graph) (void)hipGraphDestroy(g.graph);
    }
    segs_[p].clear();
    built_[p] = false;
  }

  Status RunEager(int program) {
    const Ctx c = MakeCtx();
    size_t k = 0;
    const auto& marks = marked_[program];
    for (size_t i = 0; i < plan_.program[program].size(); ++i) {
      const bool timed = k < marks.size() && marks[k] == i;
      if (timed) (void)hipEventRecord(mark_ev_[program][2 * k], stream_);
      if (Status s = Dispatch(program, i, c); !s) return s;
      if (timed) (void)hipEventRecord(mark_ev_[program][2 * k++ + 1], stream_);
    }
    return Status::Ok();
  }

  // ExecuteRange (update_engine.cc:306-509) over instructions [begin, end)
  // of `program`: each dispatched once, eagerly (no fusion), in plan order
  // on the engine stream.
  Status RunRange(int program, size_t begin, size_t end) {
    if (program < 0 || program > 2 || begin > end || end > plan_.program[program].size())
      return Status::Fail(kUnitEngine, "instruction range out of bounds");
    if (Status s = EnsureWorkspace(program); !s) return s;
    loss_posted_ = false;
    const Ctx c = MakeCtx();
    for (size_t i = begin; i < end; ++i)
      if (Status s = Dispatch(program, i, c); !s) return s;
    return Status::Ok();
  }

  // Runs of consecutive AdamWStep instructions whose operands are pairwise
  // disjoint (one per LoRA tensor, optimizer.cc:15-20) launch as one
  // multi-tensor kernel in the captured graph. Order-independent by
  // disjointness, element expression unchanged: same bits as one launch per
  // instruction.
  struct FusedRun {
    size_t first = 0, count = 0;
    size_t seg_offset = 0;  // into fused_segs_[program]
    uint64_t blocks = 0;
  };

  Status PlanFusion(int program) {
    fused_runs_[program].clear();
    if (fused_segs_[program]) {
      // A replay of the previous graph may still read the old table.
      if (Status s = HipOk(hipStreamSynchronize(stream_), "fusion table sync"); !s) return s;
      (void)LockedFree(fused_segs_[program]);
    }
    fused_segs_[program] = nullptr;
    const auto& prog = plan_.program[program];
    std::vector<AdamWSegment> segs;
    size_t i = 0;
    while (i < prog.size()) {
      if (static_cast<Op>(prog[i].opcode) != Op::kAdamWStep) {
        ++i;
        continue;
      }
      size_t j = i;
      // [begin, end) byte ranges of every operand in the run; writes are p, m, v.
      std::vector<std::pair<uint64_t, uint64_t>> ranges;
      while (j < prog.size() && static_cast<Op>(prog[j].opcode) == Op::kAdamWStep &&
             !std::binary_search(marked_[program].begin(), marked_[program].end(), j)) {
        const UpdateInstruction& a = prog[j];
        const uint64_t bytes = a.out[0] * sizeof(float);
        bool clash = false;
        for (int k = 0; k < 4 && !clash; ++k) {
          const uint64_t b = reinterpret_cast<uint64_t>(k == 1 ? static_cast<const void*>(RP(a.in[k]))
                                                                : static_cast<const void*>(WP(a.in[k])));
          for (const auto& r : ranges)
            if (b < r.second && r.first < b + bytes) clash = true;
        }
        if (clash) break;
        for (int k = 0; k < 4; ++k) {
          const uint64_t b = reinterpret_cast<uint64_t>(k == 1 ? static_cast<const void*>(RP(a.in[k]))
                                                                : static_cast<const void*>(WP(a.in[k])));
          ranges.emplace_back(b, b + bytes);
        }
        ++j;
      }
      if (j - i >= 2) {
        FusedRun run;
        run.first = i;
        run.count = j - i;
        run.seg_offset = segs.size();
        for (size_t k = i; k < j; ++k) {
          const UpdateInstruction& a = prog[k];
          segs.push_back(AdamWSegment{WP(a.in[0]), RP(a.in[1]), WP(a.in[2]), WP(a.in[3]), a.out[0], 0});
        }
        run.blocks = AdamWMultiPlan(segs.data() + run.seg_offset, run.count);
        fused_runs_[program].push_back(run);
        i = j;
      } else {
        i = std::max(j, i + 1);
      }
    }
    PlanChains(program);
    // Before the pointwise runs: folding the AddEW into the norm's rows saves
    // the dx store and re-read (8 B/elem), a pointwise run over that AddEW and
    // the next pointwise instruction only the sum's re-read.
    PlanRowAddChains(program);
    PlanAddRowChains(program);
    PlanPointwiseRuns(program);
    PlanScaleFolds(program);
    PlanDualRuns(program);
    PlanRopePairs(program);
    PlanXentPasses(program);
    PlanRowdotGroups(program);
    if (Status s = PlanColsumGroups(program); !s) return s;
    PlanTileGroups(program);
    if (segs.empty()) return Status::Ok();
    const size_t bytes = segs.size() * sizeof(AdamWSegment);
    if (Status s = HipOk(LockedMalloc(&fused_segs_[program], bytes), "fused AdamW table"); !s) return s;
    if (Status s = HipOk(hipMemcpyAsync(fused_segs_[program], segs.data(), bytes,
                                        hipMemcpyHostToDevice, stream_),
                         "fused AdamW table upload");
        !s)
      return s;
    return HipOk(hipStreamSynchronize(stream_), "fused AdamW table upload");  // segs is local
  }

  // Dual skinny pairs (kernels.h LaunchSkinnyDual): adjacent rowdot and
  // colsum GEMMs on the skinny kernels streaming one operand (the LoRA
  // backward's dt = du B^T and dB = t^T du). Every run of either, eager or
  // fused, takes the dual kernel, so a pair launched as one pass and its two
  // single launches give the same bits. As one launch the pair reads all its
  // operands before it writes: the first's writes must not overlap what the
  // second depends on, and the two outputs must be disjoint.
  void PlanDuals(int program) {
    const auto& prog = plan_.program[program];
    duals_[program].assign(prog.size(), -1);
    for (size_t i = 0; i + 1 < prog.size(); ++i) {
      const UpdateInstruction& g0 = prog[i];
      const UpdateInstruction& g1 = prog[i + 1];
      if (!IsGemmOp(g0.opcode) || !IsGemmOp(g1.opcode) || g0.flags != 0 || g1.flags != 0) continue;
      if (plans_[program][i].cfg != GemmSkinnyConfig() ||
          plans_[program][i + 1].cfg != GemmSkinnyConfig())
        continue;
      const GemmDesc d0 = DescOf(g0), d1 = DescOf(g1);
      const bool rd_first = SkinnyKindOf(d0) == SkinnyKind::kRowDot;
      if (!SkinnyDualFits(rd_first ? d0 : d1, rd_first ? d1 : d0)) continue;
      Ranges w0, w1;
      if (!WriteRangesOf(g0, &w0) || !WriteRangesOf(g1, &w1)) continue;
      bool clash = false;
      for (const auto& w : w0)
        if (Overlaps(depends_[program][i + 1], w.first, w.second) || Overlaps(w1, w.first, w.second))
          clash = true;
      if (clash) continue;
      duals_[program][i] = static_cast<int64_t>(i + 1);
      duals_[program][i + 1] = static_cast<int64_t>(i);
      ++i;
    }
  }
  // The rowdot and colsum descriptors of the pair instruction idx belongs to.
  GemmDesc DualRowdot(int program, size_t idx) const {
    const size_t j = static_cast<size_t>(duals_[program][idx]);
    const GemmDesc d = DescOf(plan_.program[program][idx]);
    return SkinnyKindOf(d) == SkinnyKind::kRowDot ? d : DescOf(plan_.program[program][j]);
  }
  // Launches instruction idx's output (which 0) or both of its pair's (which
  // 3) on the dual kernel; fold_x: the pair's stream is a folded Scale's
  // input, scaled by fold_alpha as loaded.
  Status LaunchDual(int program, size_t idx, int which, const float* fold_x, float fold_alpha,
                    const Ctx& c) const {
    const size_t j = static_cast<size_t>(duals_[program][idx]);
    GemmDesc a = DescOf(plan_.program[program][idx]), b = DescOf(plan_.program[program][j]);
    const bool a_rd = SkinnyKindOf(a) == SkinnyKind::kRowDot;
    GemmDesc& rd = a_rd ? a : b;
    GemmDesc& cs = a_rd ? b : a;
    if (fold_x) {
      int64_t elems = 0;
      const void* stream = SkinnyStream(cs, &elems);
      if (cs.A == stream) cs.A = fold_x;
      else cs.B = fold_x;
      rd.A = fold_x;
      rd.scale_stream = cs.scale_stream = true;
      rd.stream_scale = cs.stream_scale = fold_alpha;
    }
    if (which == 0) which = a_rd ? 1 : 2;
    return LaunchSkinnyDual(rd, cs, which, c);
  }

  // Fused chains, each launched as one kernel when its results are provably
  // those of its instructions run in order. None of a chain's instructions
  // may be marked for timing.
  //
  // Skinny chains (kernels.h SkinnyChain): a GemmNN/NT on the skinny outer
  // kernel, then Scale of its output and/or AddEW of that with another
  // tensor, adjacent in the plan (LoRA's u = t B, s = alpha u, y' = y + s).
  // The AddEW/Scale operands are exactly the preceding outputs, and no range
  // the chain writes overlaps a range it reads (so no workgroup can see
  // another's write). u and s are stored unless dead: overwritten by the
  // chain's own output, or observed by nothing afterwards (DeadAfter).
  //
  // Dense chains (GemmDesc::out): a GEMM on the tile kernels (batch 1, plain
  // epilogue; with split-K the reduction applies it) and the AddEW right
  // after it that consumes its output C, e.g. the base and LoRA parts of an
  // input gradient. The epilogue forms the AddEW's sum from the value it
  // would store, so the bits are the two launches'. C is stored unless dead
  // or overwritten by the sum. The sum's output and C must not overlap the
  // GEMM's operands (other workgroups are still reading them), and the
  // AddEW's other operand must not overlap C, whose new value it would
  // otherwise have read.
  //
  // Pointwise runs (kernels.h PointwiseRun): see PlanPointwiseRuns.
  //
  // Scale folds: see PlanScaleFolds.
  enum class ChainKind { kSkinny, kDense, kPointwise, kScaleFold, kLoraBase, kDual, kRowAdd, kAddRow, kRopePair, kXentPass };
  struct ChainRun {
    size_t first = 0, count = 0;
    ChainKind kind = ChainKind::kSkinny;
    SkinnyChain ch;      // skinny
    GemmDesc d;          // dense: the GEMM with its fused AddEW
    PointwiseRun pw;     // pointwise
    RowAddend ra;        // row + AddEW: the AddEW in the norm backward's write-back
    RowPreAdd pa;        // AddEW + row: the AddEW in the norm forward's load
    bool store_p = true; // loss pass: P has a later reader
    uint64_t bytes = 0;  // skinny, pointwise: HBM bytes the fused launch moves
    const float* fold_x = nullptr;  // scale fold: the Scale's input and factor
    float fold_alpha = 1.0f;
    // LoRA run in a rowdot group (PlanRowdotGroups): 1 = launches the group's
    // rowdots (listed in grp_rowdots), -1 = its rowdot ran with the group;
    // both only when the executed range holds the group's whole span
    // [grp_first, grp_end), else the run launches its own rowdot.
    int rd_mode = 0;
    size_t grp_first = 0, grp_end = 0;
    std::vector<size_t> grp_rowdots;
    // SiLU recomputed (PlanSiluRecompute). A SwiGLU backward run launches
    // pw_alt (reading g, not s) when the executed range begins at or before
    // the SiluFwd at recompute_from; the forward run holding that SiluFwd
    // skips step cond_step's store (s) when the range ends at or after
    // cond_until, the backward run's end.
    static constexpr size_t kNoIndex = ~size_t{0};
    PointwiseRun pw_alt;
    uint64_t bytes_alt = 0;
    size_t recompute_from = kNoIndex;
    int cond_step = -1;
    size_t cond_until = 0;
  };

  void PlanChains(int program) {
    chains_[program].clear();
    const auto& prog = plan_.program[program];
    auto is_marked = [&](size_t i) {
      return std::binary_search(marked_[program].begin(), marked_[program].end(), i);
    };
    auto overlap = [](const Ranges& a, const Ranges& b) {
      for (const auto& x : a)
        if (Overlaps(b, x.first, x.second)) return true;
      return false;
    };
    for (size_t i = 0; i + 1 < prog.size(); ++i) {
      const UpdateInstruction& g = prog[i];
      const auto op = static_cast<Op>(g.opcode);
      if (op != Op::kGemmNN && op != Op::kGemmNT && op != Op::kGemmTN) continue;
      if (g.flags != 0 || is_marked(i)) continue;
      const GemmDesc d = DescOf(g);
      const uint64_t n = g.out[0] * g.out[1];
      const uint64_t bytes = n * sizeof(float);
      const uint64_t u = g.in[2];
      if (const size_t len = PlanLoraBase(program, i)) {
        i += len - 1;
        continue;
      }
      if (plans_[program][i].cfg != GemmSkinnyConfig()) {
        if (const size_t len = PlanDenseChain(program, i, d)) i += len - 1;
        continue;
      }
      if (op == Op::kGemmTN || SkinnyKindOf(d) != SkinnyKind::kOuter || d.ldc != d.N) continue;
      size_t k = i + 1;
      SkinnyChain ch;
      uint64_t v = u;  // the value the AddEW must consume
      if (static_cast<Op>(prog[k].opcode) == Op::kScale && prog[k].in[0] == u &&
          prog[k].out[0] == n && !is_marked(k) && k + 1 < prog.size()) {
        ch.kind = 1;
        ch.alpha = Bits(prog[k].in[2]);
        v = prog[k].in[1];
        ++k;
      } else {
        ch.kind = 2;
      }
      const UpdateInstruction& a = prog[k];
      if (static_cast<Op>(a.opcode) != Op::kAddEW || a.out[0] != n || is_marked(k)) continue;
      if (a.in[0] != v && a.in[1] != v) continue;
      ch.y_first = a.in[1] == v;
      const uint64_t y = ch.y_first ? a.in[0] : a.in[1];
      if (IsRodataRef(y) || IsRodataRef(a.in[2])) continue;
      // y is read from memory; u and s exist only in registers until stored.
      if (Overlaps(Ranges{{RefOffset(u), bytes}}, RefOffset(y), bytes) ||
          (ch.kind == 1 && Overlaps(Ranges{{RefOffset(v), bytes}}, RefOffset(y), bytes)))
        continue;
      ch.write_u = a.in[2] != u && !DeadAfter(program, k, RefOffset(u), bytes);
      const bool write_s = ch.kind == 1 && a.in[2] != v && !DeadAfter(program, k, RefOffset(v), bytes);
      Ranges writes, reads;
      if (ch.write_u) writes.emplace_back(RefOffset(u), bytes);
      if (write_s) writes.emplace_back(RefOffset(v), bytes);
      writes.emplace_back(RefOffset(a.in[2]), bytes);
      (void)ReadRangesOf(g, &reads);
      reads.emplace_back(RefOffset(y), bytes);
      if (overlap(writes, reads)) continue;
      // Distinct written tensors must not partially overlap one another.
      bool clash = false;
      for (size_t x = 0; x < writes.size(); ++x)
        for (size_t z = x + 1; z < writes.size(); ++z)
          if (overlap(Ranges{writes[x]}, Ranges{writes[z]})) clash = true;
      if (clash) continue;
      ch.s = write_s ? WP(v) : nullptr;
      ch.y = RP(y);
      ch.yout = WP(a.in[2]);
      if (!aligned16(ch.y) || !aligned16(ch.yout) || (ch.s && !aligned16(ch.s))) continue;
      ChainRun run;
      run.first = i;
      run.count = k - i + 1;
      run.ch = ch;
      run.bytes = 4 * (d.M * d.K + d.K * d.N) + bytes * (1 + writes.size());  // t, B, y; stores
      chains_[program].push_back(run);
      i = k;
    }
  }

  // Pointwise runs: maximal stretches (up to kPwOps) of adjacent pointwise
  // instructions of one element count n, outside the other fusions and not
  // marked. Every arena operand range (4n bytes from its offset) must be
  // identical to or disjoint from every other in the run, so element i of
  // each instruction depends only on element i of earlier values: each
  // thread then evaluates the run for its elements in registers, forwarding
  // a result to later readers of the same range, and stores each written
  // range's final value unless DeadAfter the run.
  static bool PwOpOf(const UpdateInstruction& ins, PwOp* op, int* arity) {
    *arity = 2;
    switch (static_cast<Op>(ins.opcode)) {
      case Op::kAddEW: *op = PwOp::kAdd; return true;
      case Op::kMulEW: *op = PwOp::kMul; return true;
      case Op::kReluBwd: *op = PwOp::kReluBwd; return true;
      case Op::kGeluBwd: *op = PwOp::kGeluBwd; return true;
      case Op::kSiluBwd: *op = PwOp::kSiluBwd; return true;
      default: break;
    }
    *arity = 1;
    switch (static_cast<Op>(ins.opcode)) {
      case Op::kScale: *op = PwOp::kScale; return true;
      case Op::kReluFwd: *op = PwOp::kRelu; return true;
      case Op::kGeluFwd: *op = PwOp::kGelu; return true;
      case Op::kSiluFwd: *op = PwOp::kSilu; return true;
      case Op::kCopy: *op = PwOp::kCopy; return true;
      default: return false;
    }
  }

  void PlanPointwiseRuns(int program) {
    const auto& prog = plan_.program[program];
    std::vector<char> taken(prog.size(), 0);
    for (const FusedRun& r : fused_runs_[program])
      for (size_t k = r.first; k < r.first + r.count; ++k) taken[k] = 1;
    for (const ChainRun& r : chains_[program])
      for (size_t k = r.first; k < r.first + r.count; ++k) taken[k] = 1;
    for (const size_t k : marked_[program]) taken[k] = 1;
    for (size_t i = 0; i < prog.size();) {
      ChainRun run;
      if (BuildPointwiseRun(program, i, taken, &run)) {
        i += run.count;
        chains_[program].push_back(run);
      } else {
        ++i;
      }
    }
    std::sort(chains_[program].begin(), chains_[program].end(),
              [](const ChainRun& a, const ChainRun& b) { return a.first < b.first; });
    PlanSiluRecompute(program);
  }

  // SiLU recomputed in the SwiGLU backward. Its pointwise run (ds = dh u,
  // du = dh s, dg = silu'(ds, g)) reads s = silu(g), which the forward's
  // SiluFwd stored from g. Where that SiluFwd is the last writer of any
  // byte of s before the run and nothing in between writes g, the run can
  // form du = dh silu(g) from g, which it reads anyway: the same function
  // of the same bits, so the same du, and s is not read (4n bytes). If the
  // forward's own pointwise run then leaves s to no other reader, it skips
  // s's store (4n bytes more). Both hold only when one executed range holds
  // the SiluFwd and the whole backward run (the host touches nothing in
  // between): the backward run recomputes when the range begins at or
  // before the SiluFwd, and the forward run skips the store when the range
  // ends at or after the backward run, which then recomputes. A range that
  // splits them keeps s stored and read.
  void PlanSiluRecompute(int program) {
    const auto& prog = plan_.program[program];
    auto& chains = chains_[program];
    for (ChainRun& r : chains) {
      if (r.kind != ChainKind::kPointwise || r.pw.program != kPwSwiGluBwd || r.count != 3) continue;
      const UpdateInstruction& m2 = prog[r.first + 1];  // du = dh * s
      const UpdateInstruction& sb = prog[r.first + 2];  // dg = silu'(ds, g)
      const uint64_t sref = m2.in[1], gref = sb.in[1];
      if (IsRodataRef(sref)) continue;
      const uint64_t bytes = r.pw.n * sizeof(float);
      const uint64_t soff = RefOffset(sref);
      const bool g_rod = IsRodataRef(gref);
      const uint64_t goff = g_rod ? 0 : RefOffset(gref);
      if (!g_rod && goff < soff + bytes && soff < goff + bytes) continue;
      size_t f = ChainRun::kNoIndex;
      bool ok = true;
      for (size_t j = r.first; j-- > 0;) {
        const Ranges& w = writes_[program][j];
        if (Overlaps(w, soff, bytes)) {
          const UpdateInstruction& a = prog[j];
          if (static_cast<Op>(a.opcode) == Op::kSiluFwd && a.in[1] == sref && a.in[0] == gref &&
              a.out[0] == r.pw.n)
            f = j;
          break;
        }
        if (!g_rod && Overlaps(w, goff, bytes)) {
          ok = false;
          break;
        }
      }
      if (!ok || f == ChainRun::kNoIndex) continue;
      r.pw_alt = r.pw;
      r.pw_alt.program = kPwSwiGluBwdRecompute;
      r.pw_alt.in[2] = RP(gref);
      r.pw_alt.in[3] = nullptr;
      r.recompute_from = f;
      r.bytes_alt = r.bytes - bytes;
      // The forward run holding the SiluFwd: s's store is needed only by
      // this backward run's plain form when nothing else reads it.
      for (ChainRun& fr : chains) {
        if (fr.kind != ChainKind::kPointwise || f < fr.first || f >= fr.first + fr.count) continue;
        const int st = static_cast<int>(f - fr.first);
        if (fr.pw.out[st] != WP(sref) || fr.cond_step >= 0) break;
        if (!DeadAfter(program, fr.first + fr.count - 1, soff, bytes, r.first, r.first + r.count))
          break;
        fr.cond_step = st;
        fr.cond_until = r.first + r.count;
        fr.bytes_alt = fr.bytes - bytes;
        break;
      }
    }
  }

  bool BuildPointwiseRun(int program, size_t i, const std::vector<char>& taken, ChainRun* out) {
    const auto& prog = plan_.program[program];
    PointwiseRun pw;
    PwStep steps[kPwOps];
    uint64_t outs[kPwOps] = {};
    int nin_after[kPwOps] = {};
    std::vector<std::pair<uint64_t, int>> slot_of;  // ref -> slot of its current value
    std::vector<uint64_t> offs;                     // arena operand offsets seen
    uint64_t n = 0;
    int nin = 0;
    size_t j = i;
    for (; j < prog.size() && j - i < static_cast<size_t>(kPwOps); ++j) {
      const UpdateInstruction& ins = prog[j];
      PwOp op;
      int arity;
      if (taken[j] || !PwOpOf(ins, &op, &arity)) break;
      if (j == i) n = ins.out[0];
      if (n == 0 || ins.out[0] != n) break;
      const uint64_t bytes = n * sizeof(float);
      const uint64_t a = ins.in[0], b = arity == 2 ? ins.in[1] : ins.in[0];
      const uint64_t o = arity == 2 ? ins.in[2] : ins.in[1];
      if (IsRodataRef(o)) break;
      bool ok = true;
      for (const uint64_t ref : {a, b, o}) {
        if (IsRodataRef(ref)) continue;
        const uint64_t off = RefOffset(ref);
        for (const uint64_t x : offs)
          if (x != off && x < off + bytes && off < x + bytes) ok = false;
      }
      if (!ok) break;
      // Operand slots (inputs first read here are loaded by the kernel).
      int next_nin = nin;
      auto next_slots = slot_of;
      const float* next_in[kPwIn];
      std::copy(pw.in, pw.in + kPwIn, next_in);
      auto slot = [&](uint64_t ref) -> int {
        for (const auto& e : next_slots)
          if (e.first == ref) return e.second;
        if (next_nin == kPwIn) return -1;
        next_in[next_nin] = RP(ref);
        next_slots.emplace_back(ref, next_nin);
        return next_nin++;
      };
      const int sa = slot(a), sb = slot(b);
      if (sa < 0 || sb < 0) break;
      const int step = static_cast<int>(j - i);
      steps[step].op = op;
      steps[step].a = sa;
      steps[step].b = sb;
      pw.alpha[step] = op == PwOp::kScale ? Bits(ins.in[2]) : 1.0f;
      outs[step] = o;
      bool replaced = false;
      for (auto& e : next_slots)
        if (e.first == o) e.second = kPwIn + step, replaced = true;
      if (!replaced) next_slots.emplace_back(o, kPwIn + step);
      nin = next_nin;
      nin_after[step] = nin;
      slot_of = next_slots;
      std::copy(next_in, next_in + kPwIn, pw.in);
      for (const uint64_t ref : {a, b, o})
        if (!IsRodataRef(ref)) offs.push_back(RefOffset(ref));
    }
    // The longest prefix (two steps or more) that is a compiled program.
    // Inputs are numbered in first-read order, so a prefix's are a prefix.
    size_t count = j - i;
    for (; count >= 2; --count)
      if ((pw.program = PwProgramOf(nin_after[count - 1], steps, static_cast<int>(count))) >= 0)
        break;
    if (count < 2) return false;
    const uint64_t bytes = n * sizeof(float);
    pw.n = n;
    int stored = 0;
    for (size_t st = 0; st < count; ++st) {
      // Step st's result is its range's final value unless a later step of
      // the prefix writes the same range.
      bool final_value = true;
      for (size_t later = st + 1; later < count; ++later)
        if (outs[later] == outs[st]) final_value = false;
      if (!final_value || DeadAfter(program, i + count - 1, RefOffset(outs[st]), bytes)) continue;
      pw.out[st] = WP(outs[st]);
      ++stored;
    }
    out->first = i;
    out->count = count;
    out->kind = ChainKind::kPointwise;
    out->pw = pw;
    out->bytes = bytes * static_cast<uint64_t>(nin_after[count - 1] + stored);
    return true;
  }

  // Scale folds: a Scale s = alpha x whose only readers are the rowdot /
  // colsum GEMMs right after it, each streaming exactly s, on the skinny
  // kernels or on a tile plan with scaled loads (GemmScaledOk: the rank-64
  // LoRA backward's dt = s B^T and dB = t^T s). Those kernels then read x
  // and scale each element as loaded (the same float product), and the
  // Scale launches nothing. Conditions: s is dead after the last of them;
  // they write neither x nor s; x is 16-byte aligned like s.
  void PlanScaleFolds(int program) {
    const auto& prog = plan_.program[program];
    std::vector<char> taken(prog.size(), 0);
    for (const FusedRun& r : fused_runs_[program])
      for (size_t k = r.first; k < r.first + r.count; ++k) taken[k] = 1;
    for (const ChainRun& r : chains_[program])
      for (size_t k = r.first; k < r.first + r.count; ++k) taken[k] = 1;
    for (const size_t k : marked_[program]) taken[k] = 1;
    for (size_t i = 0; i + 1 < prog.size(); ++i) {
      const UpdateInstruction& sc = prog[i];
      if (taken[i] || static_cast<Op>(sc.opcode) != Op::kScale) continue;
      const uint64_t x = sc.in[0], sref = sc.in[1];
      const uint64_t bytes = sc.out[0] * sizeof(float);
      if (IsRodataRef(sref) || !aligned16(RP(x))) continue;
      size_t j = i + 1;
      for (; j < prog.size() && !taken[j] && IsGemmOp(prog[j].opcode); ++j) {
        const GemmDesc d = DescOf(prog[j]);
        int64_t elems = 0;
        const void* stream = SkinnyStream(d, &elems);
        if (stream != WP(sref) || static_cast<uint64_t>(elems) != sc.out[0]) break;
        if ((d.A == stream ? d.B : d.A) == WP(sref)) break;  // s as the small operand too
        if (plans_[program][j].cfg != GemmSkinnyConfig()) {
          GemmDesc f = d;
          if (f.A == stream) f.A = RP(x);
          else f.B = RP(x);
          f.scale_stream = true;
          if (!GemmScaledOk(f, plans_[program][j])) break;
        }
        bool clash = false;
        for (const auto& w : writes_[program][j])
          if (Overlaps(Ranges{w}, RefOffset(sref), bytes) ||
              (!IsRodataRef(x) && Overlaps(Ranges{w}, RefOffset(x), bytes)))
            clash = true;
        if (clash) break;
      }
      if (j == i + 1 || !DeadAfter(program, j - 1, RefOffset(sref), bytes)) continue;
      ChainRun run;
      run.first = i;
      run.count = j - i;
      run.kind = ChainKind::kScaleFold;
      run.fold_x = RP(x);
      run.fold_alpha = Bits(sc.in[2]);
      chains_[program].push_back(run);
      i = j - 1;
    }
    std::sort(chains_[program].begin(), chains_[program].end(),
              [](const ChainRun& a, const ChainRun& b) { return a.first < b.first; });
  }

  // Dual pairs outside every other fusion run as one launch (kDual); a pair
  // among a scale fold's consumers launches once inside the fold.
  // Norm backward + AddEW (kernels.h RowAddend): RmsNormBwd or LayerNormBwd
  // followed by an AddEW that consumes its dx (the residual stream's
  // gradient sum) runs as one row kernel writing out = addend (+) dx, and dx
  // too while a later instruction reads it. The row operands (dy, x, dx,
  // addend, out) must be pairwise the same range or disjoint, and the writes
  // disjoint from the per-column and per-row parameters: each row is read
  // whole before any of it is written, by the threads that write it.
  void PlanRowAddChains(int program) {
    const auto& prog = plan_.program[program];
    std::vector<char> taken(prog.size(), 0);
    for (const FusedRun& r : fused_runs_[program])
      for (size_t k = r.first; k < r.first + r.count; ++k) taken[k] = 1;
    for (const ChainRun& r : chains_[program])
      for (size_t k = r.first; k < r.first + r.count; ++k) taken[k] = 1;
    for (const size_t k : marked_[program]) taken[k] = 1;
    bool added = false;
    for (size_t i = 0; i + 1 < prog.size(); ++i) {
      const UpdateInstruction& g = prog[i];
      const auto op = static_cast<Op>(g.opcode);
      if ((op != Op::kRmsNormBwd && op != Op::kLayerNormBwd) || taken[i] || taken[i + 1]) continue;
      const UpdateInstruction& a = prog[i + 1];
      if (static_cast<Op>(a.opcode) != Op::kAddEW) continue;
      const bool ln = op == Op::kLayerNormBwd;
      const uint64_t dims = ln ? g.out[2] : g.out[1];
      const uint64_t rows = Hi(dims), cols = Lo(dims), n = rows * cols;
      if (a.out[0] != n || n == 0) continue;
      const uint64_t dx = g.in[3];
      if ((a.in[0] == dx) == (a.in[1] == dx)) continue;  // exactly one operand is dx
      const bool add_first = a.in[1] == dx;
      const uint64_t y = add_first ? a.in[0] : a.in[1];
      const uint64_t o = a.in[2];
      if (IsRodataRef(o) || IsRodataRef(dx)) continue;
      const uint64_t bytes = n * sizeof(float);
      const uint64_t row_refs[5] = {g.in[0], g.in[1], dx, y, o};
      bool ok = true;
      for (int x1 = 0; x1 < 5 && ok; ++x1)
        for (int x2 = x1 + 1; x2 < 5 && ok; ++x2) {
          const uint64_t r1 = row_refs[x1], r2 = row_refs[x2];
          if (IsRodataRef(r1) || IsRodataRef(r2)) continue;  // reads only (o, dx are arena)
          if (RefOffset(r1) == RefOffset(r2)) continue;
          if (Overlaps(Ranges{{RefOffset(r1), bytes}}, RefOffset(r2), bytes)) ok = false;
        }
      if (!ok) continue;
      const bool store_dx = o != dx && !DeadAfter(program, i + 1, RefOffset(dx), bytes);
      Ranges writes{{RefOffset(o), bytes}};
      if (store_dx) writes.emplace_back(RefOffset(dx), bytes);
      Ranges params;
      auto param = [&](uint64_t ref, uint64_t count) {
        if (!IsRodataRef(ref)) params.emplace_back(RefOffset(ref), count * sizeof(float));
      };
      param(g.in[2], cols);  // gamma
      if (ln) {
        param(g.out[0], rows);  // mean
        param(g.out[1], rows);  // rstd
      } else {
        param(g.out[0], rows);  // rstd
      }
      bool clash = false;
      for (const auto& w : writes)
        if (Overlaps(params, w.first, w.second)) clash = true;
      if (clash) continue;
      RowAddend ra;
      ra.addend = RP(y);
      ra.out = WP(o);
      ra.add_first = add_first;
      ra.store_dx = store_dx;
      if (!RowAddendForm(cols, {RP(g.in[0]), RP(g.in[1]), RP(g.in[2]), WP(dx), ra.addend, ra.out}))
        continue;
      ChainRun run;
      run.first = i;
      run.count = 2;
      run.kind = ChainKind::kRowAdd;
      run.ra = ra;
      chains_[program].push_back(run);
      taken[i] = taken[i + 1] = 1;
      added = true;
      ++i;
    }
    if (added)
      std::sort(chains_[program].begin(), chains_[program].end(),
                [](const ChainRun& a, const ChainRun& b) { return a.first < b.first; });
  }

  // AddEW + norm forward (kernels.h RowPreAdd): an AddEW whose sum is the
  // next instruction's RmsNormFwd / LayerNormFwd input (the residual stream
  // x + f(x) entering the next block's norm) runs in that norm kernel's load:
  // the sum is formed per row in registers, stored while a later instruction
  // reads it, and normalised without being read back. The row operands (the
  // AddEW's a, b and sum, the norm's y) must be pairwise the same range or
  // disjoint, and the norm's per-row statistics apart from all of them.
  void PlanAddRowChains(int program) {
    const auto& prog = plan_.program[program];
    std::vector<char> taken(prog.size(), 0);
    for (const FusedRun& r : fused_runs_[program])
      for (size_t k = r.first; k < r.first + r.count; ++k) taken[k] = 1;
    for (const ChainRun& r : chains_[program])
      for (size_t k = r.first; k < r.first + r.count; ++k) taken[k] = 1;
    for (const size_t k : marked_[program]) taken[k] = 1;
    bool added = false;
    for (size_t i = 0; i + 1 < prog.size(); ++i) {
      const UpdateInstruction& a = prog[i];
      const UpdateInstruction& g = prog[i + 1];
      const auto op = static_cast<Op>(g.opcode);
      if (static_cast<Op>(a.opcode) != Op::kAddEW || taken[i] || taken[i + 1]) continue;
      if (op != Op::kRmsNormFwd && op != Op::kLayerNormFwd) continue;
      const bool ln = op == Op::kLayerNormFwd;
      const uint64_t rows = Hi(g.out[0]), cols = Lo(g.out[0]), n = rows * cols;
      const uint64_t sum = a.in[2];
      if (a.out[0] != n || n == 0 || g.in[0] != sum || IsRodataRef(sum)) continue;
      const uint64_t y = ln ? g.in[3] : g.in[2];
      if (IsRodataRef(y)) continue;
      const uint64_t bytes = n * sizeof(float);
      const uint64_t row_refs[4] = {a.in[0], a.in[1], sum, y};
      bool ok = true;
      for (int x1 = 0; x1 < 4 && ok; ++x1)
        for (int x2 = x1 + 1; x2 < 4 && ok; ++x2) {
          const uint64_t r1 = row_refs[x1], r2 = row_refs[x2];
          if (IsRodataRef(r1) || IsRodataRef(r2)) continue;
          if (RefOffset(r1) == RefOffset(r2)) continue;
          if (Overlaps(Ranges{{RefOffset(r1), bytes}}, RefOffset(r2), bytes)) ok = false;
        }
      if (!ok) continue;
      const bool store_sum = sum != y && !DeadAfter(program, i + 1, RefOffset(sum), bytes);
      Ranges rowr;  // every arena row operand
      for (uint64_t ref : row_refs)
        if (!IsRodataRef(ref)) rowr.emplace_back(RefOffset(ref), bytes);
      Ranges stats;  // written per row by the norm
      if (ln) {
        stats.emplace_back(RefOffset(g.out[1]), rows * sizeof(float));
        stats.emplace_back(RefOffset(g.out[2]), rows * sizeof(float));
      } else {
        stats.emplace_back(RefOffset(g.in[3]), rows * sizeof(float));
      }
      Ranges params;
      if (!IsRodataRef(g.in[1])) params.emplace_back(RefOffset(g.in[1]), cols * sizeof(float));
      if (ln && !IsRodataRef(g.in[2])) params.emplace_back(RefOffset(g.in[2]), cols * sizeof(float));
      bool clash = false;
      for (const auto& st : stats)
        if (Overlaps(rowr, st.first, st.second) || Overlaps(params, st.first, st.second)) clash = true;
      for (const auto& w : rowr)
        if (Overlaps(params, w.first, w.second)) clash = true;
      if (clash) continue;
      RowPreAdd pa;
      pa.a = RP(a.in[0]);
      pa.b = RP(a.in[1]);
      pa.sum = WP(sum);
      pa.store_sum = store_sum;
      if (!RowAddendForm(cols, {pa.a, pa.b, pa.sum, RP(g.in[1]), WP(y)})) continue;
      ChainRun run;
      run.first = i;
      run.count = 2;
      run.kind = ChainKind::kAddRow;
      run.pa = pa;
      chains_[program].push_back(run);
      taken[i] = taken[i + 1] = 1;
      added = true;
      ++i;
    }
    if (added)
      std::sort(chains_[program].begin(), chains_[program].end(),
                [](const ChainRun& a, const ChainRun& b) { return a.first < b.first; });
  }

  // RoPE pairs (RopeWithTable's x2/y2): two adjacent RopeFwd or two
  // RopeBwd of one geometry through one angle table (a layer's q and k) in
  // one launch. Each thread loads both tensors' float4s before it stores
  // either, first y then y2, so the bits are the two launches' when the four
  // ranges are pairwise identical or disjoint and the second does not read
  // the first's output.
  void PlanRopePairs(int program) {
    const auto& prog = plan_.program[program];
    std::vector<char> taken(prog.size(), 0);
    for (const FusedRun& r : fused_runs_[program])
      for (size_t k = r.first; k < r.first + r.count; ++k) taken[k] = 1;
    for (const ChainRun& r : chains_[program])
      for (size_t k = r.first; k < r.first + r.count; ++k) taken[k] = 1;
    for (const size_t k : marked_[program]) taken[k] = 1;
    auto rope = [&](size_t k) {
      const auto op = static_cast<Op>(prog[k].opcode);
      return op == Op::kRopeFwd || op == Op::kRopeBwd;
    };
    for (size_t i = 0; i + 1 < prog.size(); ++i) {
      if (taken[i] || taken[i + 1] || !rope(i) || prog[i + 1].opcode != prog[i].opcode) continue;
      const UpdateInstruction& a = prog[i];
      const UpdateInstruction& b = prog[i + 1];
      if (a.out[0] != b.out[0] || a.out[1] != b.out[1] || a.out[2] != b.out[2]) continue;
      const float* t = RopeTableOf(Lo(a.out[0]), Lo(a.out[1]), a.out[2]);
      const uint64_t S = Lo(a.out[0]), d = Lo(a.out[1]);
      if (!t || d % 4 != 0 || S * d > 0xFFFFFFFFu ||
          Hi(a.out[0]) * S * Hi(a.out[1]) * d / 4 > 0xFFFFFFFFu)
        continue;
      const uint64_t refs[4] = {a.in[0], a.in[1], b.in[0], b.in[1]};
      bool ok = b.in[0] != a.in[1];
      for (uint64_t r : refs) ok = ok && !IsRodataRef(r) && aligned16(RP(r));
      const uint64_t bytes = Hi(a.out[0]) * Lo(a.out[0]) * Hi(a.out[1]) * Lo(a.out[1]) * sizeof(float);
      for (int x = 0; x < 4 && ok; ++x)
        for (int z = x + 1; z < 4 && ok; ++z)
          ok = refs[x] == refs[z] || !Overlaps(Ranges{{RefOffset(refs[x]), bytes}}, RefOffset(refs[z]), bytes);
      if (!ok) continue;
      ChainRun run;
      run.first = i;
      run.count = 2;
      run.kind = ChainKind::kRopePair;
      chains_[program].push_back(run);
      taken[i] = taken[i + 1] = 1;
      ++i;
    }
    std::sort(chains_[program].begin(), chains_[program].end(),
              [](const ChainRun& a, const ChainRun& b) { return a.first < b.first; });
  }

  // Loss passes (SoftmaxXEntFwdBwd): SoftmaxXEntFwd, the Fill of the
  // gradient seed and SoftmaxXEntBwd over the forward's probabilities, in
  // plan order, as one pass over the logits: the backward runs on each row's
  // probabilities in registers, and P is stored only if a later
  // instruction reads it. The written ranges (dl, P, the seed, the loss)
  // must be apart from each other and from what the pass reads (logits,
  // labels), since the rows' reads and writes interleave across workgroups;
  // dl alone may be exactly the logits (each row is its workgroup's own).
  void PlanXentPasses(int program) {
    const auto& prog = plan_.program[program];
    std::vector<char> taken(prog.size(), 0);
    for (const FusedRun& r : fused_runs_[program])
      for (size_t k = r.first; k < r.first + r.count; ++k) taken[k] = 1;
    for (const ChainRun& r : chains_[program])
      for (size_t k = r.first; k < r.first + r.count; ++k) taken[k] = 1;
    for (const size_t k : marked_[program]) taken[k] = 1;
    for (size_t i = 0; i + 2 < prog.size(); ++i) {
      const UpdateInstruction& f = prog[i];
      const UpdateInstruction& z = prog[i + 1];
      const UpdateInstruction& b = prog[i + 2];
      if (taken[i] || taken[i + 1] || taken[i + 2] || static_cast<Op>(f.opcode) != Op::kSoftmaxXEntFwd ||
          static_cast<Op>(z.opcode) != Op::kFill || static_cast<Op>(b.opcode) != Op::kSoftmaxXEntBwd)
        continue;
      const uint64_t N = f.out[0], C = f.out[1];
      if (b.out[0] != N || b.out[1] != C || z.out[0] != 1 || b.in[0] != f.in[3] || b.in[1] != f.in[1] ||
          b.in[2] != z.in[0])
        continue;
      const uint64_t L = f.in[0], lab = f.in[1], loss = f.in[2], P = f.in[3], S = z.in[0], D = b.in[3];
      bool ok = true;
      for (uint64_t r : {loss, P, S, D}) ok = ok && !IsRodataRef(r);
      if (!ok) continue;
      const uint64_t mat = N * C * sizeof(float);
      const bool store_p = !DeadAfter(program, i + 2, RefOffset(P), mat);
      if (!XEntFwdBwdFits(RP(L), store_p ? RP(P) : nullptr, RP(D), N, C)) continue;
      // written ranges, then read ones
      Ranges w{{RefOffset(D), mat}, {RefOffset(S), sizeof(float)}, {RefOffset(loss), sizeof(float)}};
      if (store_p) w.emplace_back(RefOffset(P), mat);
      // dl may be the logits exactly (row by row in place); nothing else may
      // touch what the pass reads.
      Ranges r;
      if (!IsRodataRef(L)) r.emplace_back(RefOffset(L), mat);
      if (!IsRodataRef(lab)) r.emplace_back(RefOffset(lab), N * sizeof(int32_t));
      for (size_t x = 0; x < w.size() && ok; ++x) {
        const bool in_place = x == 0 && D == L;
        ok = in_place ? !Overlaps(Ranges{r.begin() + 1, r.end()}, w[x].first, w[x].second)
                      : !Overlaps(r, w[x].first, w[x].second);
        for (size_t y = x + 1; y < w.size() && ok; ++y)
          ok = !Overlaps(Ranges{w[x]}, w[y].first, w[y].second);
      }
      if (!ok) continue;
      ChainRun run;
      run.first = i;
      run.count = 3;
      run.kind = ChainKind::kXentPass;
      run.store_p = store_p;
      chains_[program].push_back(run);
      taken[i] = taken[i + 1] = taken[i + 2] = 1;
      i += 2;
    }
    std::sort(chains_[program].begin(), chains_[program].end(),
              [](const ChainRun& a, const ChainRun& b) { return a.first < b.first; });
  }

  void PlanDualRuns(int program) {
    const auto& prog = plan_.program[program];
    std::vector<char> taken(prog.size(), 0);
    for (const FusedRun& r : fused_runs_[program])
      for (size_t k = r.first; k < r.first + r.count; ++k) taken[k] = 1;
    for (const ChainRun& r : chains_[program])
      for (size_t k = r.first; k < r.first + r.count; ++k) taken[k] = 1;
    for (const size_t k : marked_[program]) taken[k] = 1;
    for (size_t i = 0; i + 1 < prog.size(); ++i) {
      if (duals_[program][i] != static_cast<int64_t>(i + 1) || taken[i] || taken[i + 1]) continue;
      ChainRun run;
      run.first = i;
      run.count = 2;
      run.kind = ChainKind::kDual;
      chains_[program].push_back(run);
      ++i;
    }
    std::sort(chains_[program].begin(), chains_[program].end(),
              [](const ChainRun& a, const ChainRun& b) { return a.first < b.first; });
  }

  // The consumers of a scale fold from idx on: a dual pair inside the fold
  // launches once (returns 2), any other consumer alone (returns 1).
  size_t FoldStep(int program, const ChainRun& run, size_t idx, const Ctx& c, Status* st) {
    if (duals_[program][idx] == static_cast<int64_t>(idx + 1) && idx + 1 < run.first + run.count) {
      *st = LaunchDual(program, idx, 3, run.fold_x, run.fold_alpha, c);
      return 2;
    }
    *st = LaunchFolded(program, run, idx, c);
    return 1;
  }

  // Consumer idx of a scale fold, reading x with the factor applied.
  Status LaunchFolded(int program, const ChainRun& run, size_t idx, const Ctx& c) {
    GemmDesc d = DescOf(plan_.program[program][idx]);
    int64_t elems = 0;
    const void* stream = SkinnyStream(d, &elems);
    if (d.A == stream) d.A = run.fold_x;
    else d.B = run.fold_x;
    d.scale_stream = true;
    d.stream_scale = run.fold_alpha;
    return LaunchGemm(d, plans_[program][idx], c);
  }

  // A LoRA'd projection as one run: the base GEMM y = x W at i, the rank-r
  // down-projection t = x A at i + 1, the up-projection u = t B at i + 2, an
  // optional Scale s = a u at i + 3, and the AddEW of y and s. The run
  // launches the down-projection first, then the base GEMM with u, the Scale
  // and the AddEW in its epilogue (GemmDesc::lora_t): y, u and s never reach
  // memory. The up-projection must run on a tile plan with one slice, so the
  // epilogue's u (the tile kernels' k order) has its bits; y, u and s must be
  // dead after the AddEW. Returns the run's length (0: none).
  // Rowdot groups (kernels.h LaunchSkinnyRowdotGroup): the down-projection
  // rowdots t_j = x A_j of consecutive LoRA runs over one layer input x (the
  // q, k and v projections) run as one pass over x when the first run
  // launches. Member j's rowdot moves from its own run's launch to the
  // first's, which is legal when no launch in between writes x, A_j or t_j
  // or reads t_j. A LoRA run's launch writes only its sum o and t and reads
  // only its GEMMs' operands (y, u and s stay in registers); any other
  // instruction counts with its plan-level ranges. Each member's t has the
  // bits of its own launch, so fused and eager replays agree.
  void PlanRowdotGroups(int program) {
    auto& chains = chains_[program];
    std::sort(chains.begin(), chains.end(),
              [](const ChainRun& a, const ChainRun& b) { return a.first < b.first; });
    const auto& prog = plan_.program[program];
    std::vector<int> chain_of(prog.size(), -1);
    for (size_t c = 0; c < chains.size(); ++c)
      for (size_t k = chains[c].first; k < chains[c].first + chains[c].count; ++k)
        chain_of[k] = static_cast<int>(c);
    auto member_ok = [&](const ChainRun& r) {
      return r.kind == ChainKind::kLoraBase && r.rd_mode == 0 &&
             plans_[program][r.first + 1].cfg == GemmSkinnyConfig();
    };
    // What the launches of instructions [from, to) write and read.
    auto launched = [&](size_t from, size_t to, Ranges* w, Ranges* rd) {
      for (size_t k = from; k < to; ++k) {
        const int c = chain_of[k];
        if (c >= 0 && chains[c].kind == ChainKind::kLoraBase) {
          const ChainRun& r = chains[c];
          if (k != r.first) continue;  // the run, counted at its first instruction
          const UpdateInstruction& add = prog[r.first + r.count - 1];
          const uint64_t bytes = static_cast<uint64_t>(r.d.M) * r.d.N * sizeof(float);
          (void)WriteRangesOf(prog[r.first + 1], w);
          w->emplace_back(RefOffset(add.in[2]), bytes);
          for (size_t g = r.first; g < r.first + 3; ++g) (void)DependRangesOf(prog[g], rd);
          continue;
        }
        (void)WriteRangesOf(prog[k], w);
        (void)DependRangesOf(prog[k], rd);
      }
    };
    auto overlap = [](const Ranges& a, const Ranges& b) {
      for (const auto& x : a)
        if (Overlaps(b, x.first, x.second)) return true;
      return false;
    };
    for (size_t a = 0; a < chains.size(); ++a) {
      if (!member_ok(chains[a])) continue;
      const ChainRun& r1 = chains[a];
      GemmDesc ds[4];
      ds[0] = DescOf(prog[r1.first + 1]);
      std::vector<size_t> members{a};
      for (size_t b = a + 1; b < chains.size() && members.size() < 4; ++b) {
        const ChainRun& rb = chains[b];
        if (!member_ok(rb)) break;
        const size_t ib = rb.first + 1;
        ds[members.size()] = DescOf(prog[ib]);
        if (!SkinnyRowdotGroupFits(ds, static_cast<int>(members.size()) + 1)) break;
        bool marked = false;
        for (size_t k = r1.first; k < rb.first + rb.count; ++k)
          marked = marked || std::binary_search(marked_[program].begin(), marked_[program].end(), k);
        if (marked) break;
        Ranges w, rd, in_b, out_b;
        launched(r1.first, rb.first, &w, &rd);
        (void)DependRangesOf(prog[ib], &in_b);  // x and A_b
        (void)WriteRangesOf(prog[ib], &out_b);  // t_b
        if (overlap(in_b, w) || overlap(out_b, w) || overlap(out_b, rd) || overlap(out_b, in_b)) break;
        members.push_back(b);
      }
      if (members.size() < 2) continue;
      const size_t grp_first = chains[members.front()].first;
      const size_t grp_end = chains[members.back()].first + chains[members.back()].count;
      for (size_t j = 0; j < members.size(); ++j) {
        ChainRun& r = chains[members[j]];
        r.rd_mode = j == 0 ? 1 : -1;
        r.grp_first = grp_first;
        r.grp_end = grp_end;
        if (j == 0)
          for (size_t m : members) r.grp_rowdots.push_back(chains[m].first + 1);
      }
      a = members.back();
    }
  }

  size_t PlanLoraBase(int program, size_t i) {
    const auto& prog = plan_.program[program];
    auto marked = [&](size_t k) {
      return std::binary_search(marked_[program].begin(), marked_[program].end(), k);
    };
    if (i + 4 >= prog.size()) return 0;
    const UpdateInstruction& g0 = prog[i];
    const UpdateInstruction& g1 = prog[i + 1];
    const UpdateInstruction& g2 = prog[i + 2];
    const auto op0 = static_cast<Op>(g0.opcode), op2 = static_cast<Op>(g2.opcode);
    if ((op0 != Op::kGemmNN && op0 != Op::kGemmNT) || op2 != Op::kGemmNN || !IsGemmOp(g1.opcode) ||
        static_cast<Op>(g1.opcode) == Op::kGemmAccNN)
      return 0;
    for (size_t k = i; k < i + 3; ++k)
      if (marked(k)) return 0;
    GemmDesc d = DescOf(g0);
    const GemmPlan& p0 = plans_[program][i];
    const GemmPlan& p2 = plans_[program][i + 2];
    if (d.batch != 1 || d.causal != Causal::kNone || d.accumulate || d.bias || d.b_int8 ||
        !d.a_kc || d.ldc != d.N || p0.splits != 1)
      return 0;
    auto lora_cfg_ok = [&](int cfg) { return GemmLoraCfgOk(cfg, d.b_kc); };
    if (!lora_cfg_ok(p0.cfg) || (p0.n_split > 0 && !lora_cfg_ok(p0.tail_cfg))) return 0;
    // up-projection u = t B: M x N over K = r, t the down-projection's output
    const GemmDesc du = DescOf(g2);
    const uint64_t t = g1.in[2];
    // Rank 16 or less: the epilogue's u costs r/8 MFMA groups and r scalar
    // B' loads per 32x32 block, with nothing to hide them; at rank 64 (C5)
    // that cost exceeded the unfused chain's (C5 step 469.6 -> 474.1 ms).
    if (g2.in[0] != t || du.M != d.M || du.N != d.N || du.K % 8 != 0 || du.K > 16 ||
        p2.cfg == GemmSkinnyConfig() || p2.splits != 1 || du.batch != 1 || du.accumulate ||
        du.bias || du.act != 0 || du.alpha != 1.0f || du.b_int8 || !du.a_kc || du.b_kc)
      return 0;
    const uint64_t n = static_cast<uint64_t>(d.M) * d.N, bytes = n * sizeof(float);
    const uint64_t y = g0.in[2], uref = g2.in[2];
    size_t k = i + 3;
    uint64_t v = uref;
    bool scaled = false;
    float scale = 1.0f;
    if (static_cast<Op>(prog[k].opcode) == Op::kScale && prog[k].in[0] == uref &&
        prog[k].out[0] == n && !marked(k) && k + 1 < prog.size()) {
      scaled = true;
      scale = Bits(prog[k].in[2]);
      v = prog[k].in[1];
      ++k;
    }
    const UpdateInstruction& a = prog[k];
    if (static_cast<Op>(a.opcode) != Op::kAddEW || marked(k) || a.out[0] != n) return 0;
    if (!((a.in[0] == y && a.in[1] == v) || (a.in[0] == v && a.in[1] == y))) return 0;
    const bool y_first = a.in[0] == y;
    const uint64_t o = a.in[2];
    if (IsRodataRef(o) || IsRodataRef(y) || IsRodataRef(uref) || IsRodataRef(v) || IsRodataRef(t)) return 0;
    // y, u and s exist only in registers: each dead after the AddEW (or
    // overwritten by its output), and the down-projection does not touch y.
    for (uint64_t ref : {y, uref, v})
      if (ref != o && !DeadAfter(program, k, RefOffset(ref), bytes)) return 0;
    Ranges w1;
    (void)WriteRangesOf(g1, &w1);
    if (Overlaps(w1, RefOffset(y), bytes)) return 0;
    // Unfused, the down- and up-projections run after y is stored and the
    // AddEW after u and s are: none of them may read y from memory, u and s
    // may not land on y, and s either is u (an in-place Scale) or is apart
    // from it. Fused, y, u and s never reach memory.
    Ranges r12;
    (void)ReadRangesOf(g1, &r12);
    (void)ReadRangesOf(g2, &r12);
    if (Overlaps(r12, RefOffset(y), bytes)) return 0;
    const Ranges yr{{RefOffset(y), bytes}};
    if (Overlaps(yr, RefOffset(uref), bytes) || Overlaps(yr, RefOffset(v), bytes)) return 0;
    if (scaled && v != uref && Overlaps(Ranges{{RefOffset(uref), bytes}}, RefOffset(v), bytes))
      return 0;
    // The fused launch reads x, W, t and B while it writes o; the
    // down-projection reads x and A: none of them may overlap o, and the
    // base GEMM's operands may not overlap t.
    Ranges reads;
    (void)ReadRangesOf(g0, &reads);
    (void)ReadRangesOf(g2, &reads);
    (void)ReadRangesOf(g1, &reads);
    if (Overlaps(reads, RefOffset(o), bytes)) return 0;
    Ranges r0;
    (void)ReadRangesOf(g0, &r0);
    for (const auto& wr : w1)
      if (Overlaps(r0, wr.first, wr.second)) return 0;
    if (!aligned16(du.A) || du.lda % 4 != 0 || !aligned16(WP(o))) return 0;
    d.out = WP(o);
    d.write_c = false;
    d.out_scaled = scaled;
    d.out_scale = scale;
    d.lora_t = static_cast<const float*>(du.A);
    d.lora_b = static_cast<const float*>(du.B);
    d.lora_ldt = du.lda;
    d.lora_ldb = du.ldb;
    d.lora_r = static_cast<int>(du.K);
    d.lora_y_first = y_first;
    if (!GemmVecForm(d)) return 0;
    ChainRun run;
    run.first = i;
    run.count = k - i + 1;
    run.kind = ChainKind::kLoraBase;
    run.d = d;
    chains_[program].push_back(run);
    return run.count;
  }

  // A dense chain at instruction i (the GEMM): the AddEW at i + 1, or a
  // Scale at i + 1 feeding the AddEW at i + 2, folded into the GEMM's
  // epilogue. Returns the chain's length (0: none). The GEMM's output c and
  // the Scale's output v are stored only while a later instruction reads
  // them (at most one of the two: the epilogue has one extra store).
  size_t PlanDenseChain(int program, size_t i, GemmDesc d) {
    const auto& prog = plan_.program[program];
    auto marked = [&](size_t k) {
      return std::binary_search(marked_[program].begin(), marked_[program].end(), k);
    };
    if (d.batch != 1 || d.ldc != d.N || d.causal != Causal::kNone ||
        d.accumulate || d.bias || d.act != 0 || d.b_int8)
      return 0;
    const UpdateInstruction& g = prog[i];
    const uint64_t c = g.in[2], n = g.out[0] * g.out[1], bytes = n * sizeof(float);
    size_t k = i + 1;
    uint64_t v = c;  // the value the AddEW consumes
    bool scaled = false;
    float scale = 1.0f;
    if (static_cast<Op>(prog[k].opcode) == Op::kScale && prog[k].in[0] == c &&
        prog[k].out[0] == n && !marked(k) && k + 1 < prog.size() && GemmVecForm(d)) {
      scaled = true;
      scale = Bits(prog[k].in[2]);
      v = prog[k].in[1];
      if (IsRodataRef(v)) return 0;
      ++k;
    }
    const UpdateInstruction& a = prog[k];
    if (static_cast<Op>(a.opcode) != Op::kAddEW || marked(k) || a.out[0] != n) return 0;
    if (a.in[0] != v && a.in[1] != v) return 0;
    const bool addend_first = a.in[1] == v;
    const uint64_t y = addend_first ? a.in[0] : a.in[1];
    const uint64_t o = a.in[2];
    if (y == v || y == c || IsRodataRef(o)) return 0;
    // c and v hold the GEMM's and the Scale's results only in registers:
    // nothing may read them from memory, and v may not partially cover c.
    if (!IsRodataRef(y) && (Overlaps(Ranges{{RefOffset(c), bytes}}, RefOffset(y), bytes) ||
                            (scaled && Overlaps(Ranges{{RefOffset(v), bytes}}, RefOffset(y), bytes))))
      return 0;
    if (scaled && v != c && Overlaps(Ranges{{RefOffset(c), bytes}}, RefOffset(v), bytes)) return 0;
    // Values live after the AddEW: c (unless overwritten by v or o) and v.
    const bool c_live = c != o && c != v && !DeadAfter(program, k, RefOffset(c), bytes);
    const bool v_live = scaled && v != o && !DeadAfter(program, k, RefOffset(v), bytes);
    if (c_live && v_live) return 0;
    uint64_t cdst = c;  // where the C store goes (with write_c)
    if (v_live) cdst = v;
    const bool write_c = c_live || v_live;
    Ranges writes{{RefOffset(o), bytes}};
    if (write_c) writes.emplace_back(RefOffset(cdst), bytes);
    Ranges reads;
    (void)ReadRangesOf(g, &reads);
    for (const auto& w : writes)
      if (Overlaps(reads, w.first, w.second)) return 0;
    if (write_c && cdst != o && Overlaps(Ranges{{RefOffset(o), bytes}}, RefOffset(cdst), bytes))
      return 0;
    if (!IsRodataRef(y) && y != o && Overlaps(Ranges{{RefOffset(o), bytes}}, RefOffset(y), bytes))
      return 0;
    d.C = WP(cdst);
    d.addend = RP(y);
    d.out = WP(o);
    d.addend_first = addend_first;
    d.write_c = write_c;
    d.out_scaled = scaled;
    d.out_scale = scale;
    d.c_gets_scaled = v_live;
    ChainRun run;
    run.first = i;
    run.count = k - i + 1;
    run.kind = ChainKind::kDense;
    run.d = d;
    run.count += PlanPostAddBias(program, k, c, cdst, write_c, y, o, reads, &run.d,
                                 plans_[program][i]);
    chains_[program].push_back(run);
    return run.count;
  }

  // The AddBias of the chain's sum o at k + 1 (h = o + b by column, the
  // biased MLP layers' up and down projections), and an activation of h at
  // k + 2 (g = act(h)), folded into the same epilogue (GemmDesc::post_bias)
  // when the GEMM's plan has the post-AddEW kernels (GemmPostOk). o and h
  // are stored only while a later instruction reads them. Every written
  // array (C's store, o, h, g) must be the same range as the addend y or
  // apart from it, apart from each other unless one overwrites the other,
  // apart from what the GEMM reads, and apart from the bias: each element
  // is read and written by one lane, in the unfused order. Returns the
  // instructions added to the chain (0: none); on 0, *d is unchanged.
  size_t PlanPostAddBias(int program, size_t k, uint64_t c, uint64_t cdst, bool write_c,
                         uint64_t y, uint64_t o, const Ranges& gemm_reads, GemmDesc* d,
                         const GemmPlan& plan) {
    const auto& prog = plan_.program[program];
    auto marked = [&](size_t j) {
      return std::binary_search(marked_[program].begin(), marked_[program].end(), j);
    };
    if (k + 1 >= prog.size() || marked(k + 1)) return 0;
    const UpdateInstruction& ab = prog[k + 1];
    if (static_cast<Op>(ab.opcode) != Op::kAddBias || ab.in[0] != o) return 0;
    if (static_cast<int64_t>(ab.out[0]) != d->M || static_cast<int64_t>(ab.out[1]) != d->N ||
        (d->ldo && d->ldo != d->N))
      return 0;
    const uint64_t bias = ab.in[1], h = ab.in[2];
    const uint64_t n = ab.out[0] * ab.out[1], bytes = n * sizeof(float);
    if (IsRodataRef(h)) return 0;
    size_t add = 1;
    int act = 0;
    uint64_t g = kNullRef;
    if (k + 2 < prog.size() && !marked(k + 2)) {
      const UpdateInstruction& a = prog[k + 2];
      const auto op = static_cast<Op>(a.opcode);
      const int code = op == Op::kReluFwd ? 1 : op == Op::kGeluFwd ? 2 : op == Op::kSiluFwd ? 3 : 0;
      if (code && a.in[0] == h && a.out[0] == n && !IsRodataRef(a.in[1])) {
        act = code;
        g = a.in[1];
        add = 2;
      }
    }
    const size_t last = k + add;
    const bool o_live = o != h && !(add == 2 && o == g) && !DeadAfter(program, last, RefOffset(o), bytes);
    const bool h_live = add == 1 || (h != g && !DeadAfter(program, last, RefOffset(h), bytes));
    // The arrays written, each with its range.
    std::vector<uint64_t> outs;
    if (write_c) outs.push_back(cdst);
    if (o_live) outs.push_back(o);
    if (h_live) outs.push_back(h);
    if (add == 2) outs.push_back(g);
    for (size_t x1 = 0; x1 < outs.size(); ++x1) {
      const uint64_t r1 = RefOffset(outs[x1]);
      if (Overlaps(gemm_reads, r1, bytes)) return 0;
      if (!IsRodataRef(bias) && Overlaps(Ranges{{RefOffset(bias), d->N * sizeof(float)}}, r1, bytes))
        return 0;
      if (!IsRodataRef(y) && outs[x1] != y && Overlaps(Ranges{{RefOffset(y), bytes}}, r1, bytes)) return 0;
      for (size_t x2 = x1 + 1; x2 < outs.size(); ++x2)
        if (Overlaps(Ranges{{RefOffset(outs[x2]), bytes}}, r1, bytes)) return 0;
    }
    (void)c;
    GemmDesc e = *d;
    e.post_bias = RP(bias);
    e.post_h = h_live ? WP(h) : nullptr;
    e.post_g = add == 2 ? WP(g) : nullptr;
    e.post_act = act;
    e.write_out = o_live;
    if (!aligned16(RP(bias)) || !GemmPostOk(e, plan)) return 0;
    *d = e;
    return add;
  }

  // Tile groups (kernels.h LaunchGemmGroup): 2..4 consecutive GEMM
  // launches on one tile config (a plain GEMM, a GEMM with its fused AddEW,
  // or a LoRA run's base GEMM with the up-projection in its epilogue) as
  // one launch, e.g. a decoder layer's q/k/v projections or its gate and up
  // projections. Each output keeps its own launch's bits. The launches run
  // at once, so no member may write what another reads or writes; the
  // rowdots a LoRA member launches first (its own, or its rowdot group's)
  // move ahead of the earlier members' GEMMs, so they may not write what
  // those read or write, nor read what those write. Ranges are the
  // launches' own operand extents. A group is used only when the executed
  // range holds its whole span; rowdot groups lie wholly inside a span.
  struct TileUnit {
    size_t first = 0, count = 1;  // instruction span
    GemmDesc d;                   // the launch (a chain's fused form)
    GemmPlan plan;
    int pre = 0;                  // 1: its own rowdot first; 2: its rowdot group first
    int chain = -1;               // chains_ index of a LoRA unit
  };
  struct TileGroup {
    size_t first = 0, end = 0;
    std::vector<TileUnit> units;
  };

  // What a tile-kernel launch of d (batch 1) reads and writes, as absolute
  // device address ranges.
  static void DescRanges(const GemmDesc& d, Ranges* rd, Ranges* wr) {
    auto at = [](const void* p) { return reinterpret_cast<uint64_t>(p); };
    auto span2 = [](int64_t rows, int64_t ld, int64_t cols) {
      return static_cast<uint64_t>((rows - 1) * ld + cols) * sizeof(float);
    };
    rd->emplace_back(at(d.A), d.a_kc ? span2(d.M, d.lda, d.K) : span2(d.K, d.lda, d.M));
    rd->emplace_back(at(d.B), d.b_kc ? span2(d.N, d.ldb, d.K) : span2(d.K, d.ldb, d.N));
    if (d.bias) rd->emplace_back(at(d.bias), static_cast<uint64_t>(d.N) * sizeof(float));
    const int64_t ldo = d.ldo ? d.ldo : d.N;
    if (d.lora_t) {
      rd->emplace_back(at(d.lora_t), span2(d.M, d.lora_ldt, d.lora_r));
      rd->emplace_back(at(d.lora_b), span2(d.lora_r, d.lora_ldb, d.N));
      wr->emplace_back(at(d.out), span2(d.M, ldo, d.N));
      return;
    }
    if (d.out) {
      rd->emplace_back(at(d.addend), span2(d.M, ldo, d.N));
      wr->emplace_back(at(d.out), span2(d.M, ldo, d.N));
    }
    if (!d.out || d.write_c) {
      if (d.accumulate) rd->emplace_back(at(d.C), span2(d.M, d.ldc, d.N));
      wr->emplace_back(at(d.C), span2(d.M, d.ldc, d.N));
    }
  }

  void PlanTileGroups(int program) {
    tgroups_[program].clear();
    const auto& prog = plan_.program[program];
    tgroup_of_[program].assign(prog.size(), -1);
    const auto& chains = chains_[program];
    std::vector<int> chain_at(prog.size(), -1), chain_of(prog.size(), -1);
    for (size_t c = 0; c < chains.size(); ++c) {
      chain_at[chains[c].first] = static_cast<int>(c);
      for (size_t k = chains[c].first; k < chains[c].first + chains[c].count; ++k)
        chain_of[k] = static_cast<int>(c);
    }
    std::vector<uint8_t> cs_span(prog.size(), 0);
    for (const ColsumGroup& g : cs_groups_[program])
      for (size_t k = g.members.front(); k <= g.members.back(); ++k) cs_span[k] = 1;
    auto marked = [&](size_t k) {
      return std::binary_search(marked_[program].begin(), marked_[program].end(), k);
    };
    auto overlap = [](const Ranges& a, const Ranges& b) {
      for (const auto& x : a)
        if (Overlaps(b, x.first, x.second)) return true;
      return false;
    };
    // The launch unit starting at instruction i, if it is one a group takes.
    auto unit_at = [&](size_t i, TileUnit* u) {
      if (cs_span[i]) return false;
      const int c = chain_at[i];
      if (c >= 0) {
        const ChainRun& r = chains[c];
        if (r.kind != ChainKind::kDense && r.kind != ChainKind::kLoraBase) return false;
        u->first = i;
        u->count = r.count;
        u->d = r.d;
        u->plan = plans_[program][i];
        u->chain = c;
        u->pre = r.kind != ChainKind::kLoraBase ? 0 : r.rd_mode == 0 ? 1 : r.rd_mode == 1 ? 2 : 0;
        for (size_t k = i; k < i + r.count; ++k)
          if (cs_span[k]) return false;
        return true;
      }
      if (chain_of[i] >= 0) return false;
      const UpdateInstruction& g = prog[i];
      if (!IsGemmOp(g.opcode) || duals_[program][i] >= 0) return false;
      if (plans_[program][i].cfg == GemmSkinnyConfig()) return false;
      u->first = i;
      u->count = 1;
      u->d = DescOf(g);
      u->plan = plans_[program][i];
      u->chain = -1;
      u->pre = 0;
      return true;
    };
    // The pre-launch (rowdot) ranges of unit u.
    auto pre_ranges = [&](const TileUnit& u, Ranges* rd, Ranges* wr) {
      if (u.pre == 1) DescRanges(DescOf(prog[u.first + 1]), rd, wr);
      if (u.pre == 2)
        for (size_t k : chains[u.chain].grp_rowdots) DescRanges(DescOf(prog[k]), rd, wr);
    };
    for (size_t i = 0; i < prog.size();) {
      TileUnit u0;
      if (!unit_at(i, &u0)) {
        ++i;
        continue;
      }
      std::vector<TileUnit> units{u0};
      std::vector<Ranges> R(1), W(1), PR(1), PW(1);
      DescRanges(u0.d, &R[0], &W[0]);
      pre_ranges(u0, &PR[0], &PW[0]);
      // A member marked for timing may only be the group's first instruction
      // (the timed launch is then the whole group).
      bool ok0 = true;
      for (size_t k = i + 1; k < i + u0.count; ++k) ok0 = ok0 && !marked(k);
      size_t next = i + u0.count;
      while (ok0 && units.size() < static_cast<size_t>(kGemmGroupMax) && next < prog.size()) {
        TileUnit u;
        if (!unit_at(next, &u)) break;
        bool bad = false;
        for (size_t k = next; k < next + u.count; ++k) bad = bad || marked(k);
        if (bad) break;
        std::vector<GemmDesc> ds;
        std::vector<GemmPlan> ps;
        for (const TileUnit& x : units) {
          ds.push_back(x.d);
          ps.push_back(x.plan);
        }
        ds.push_back(u.d);
        ps.push_back(u.plan);
        if (!GemmGroupFits(ds.data(), ps.data(), static_cast<int>(ds.size()))) break;
        Ranges r, w, pr, pw;
        DescRanges(u.d, &r, &w);
        pre_ranges(u, &pr, &pw);
        for (size_t j = 0; j < units.size() && !bad; ++j)
          bad = overlap(W[j], r) || overlap(W[j], w) || overlap(w, R[j]) ||
                overlap(pw, R[j]) || overlap(pw, W[j]) || overlap(pr, W[j]);
        if (bad) break;
        units.push_back(u);
        R.push_back(r);
        W.push_back(w);
        PR.push_back(pr);
        PW.push_back(pw);
        next += u.count;
      }
      // Rowdot groups wholly inside the span; trim members past it.
      while (units.size() >= 2) {
        const size_t end = units.back().first + units.back().count;
        bool inside = true;
        for (const TileUnit& x : units)
          if (x.chain >= 0 && chains[x.chain].rd_mode != 0)
            inside = inside && chains[x.chain].grp_first >= i && chains[x.chain].grp_end <= end;
        if (inside) break;
        units.pop_back();
      }
      if (units.size() < 2) {
        i += u0.count;
        continue;
      }
      TileGroup g;
      g.first = i;
      g.end = units.back().first + units.back().count;
      g.units = units;
      for (size_t k = g.first; k < g.end; ++k) tgroup_of_[program][k] = static_cast<int>(tgroups_[program].size());
      tgroups_[program].push_back(g);
      i = g.end;
    }
  }

  int TileGroupAt(int program, size_t idx, size_t begin, size_t end) const {
    if (idx >= tgroup_of_[program].size() || tgroup_of_[program][idx] < 0) return -1;
    const int g = tgroup_of_[program][idx];
    const TileGroup& grp = tgroups_[program][g];
    return grp.first == idx && grp.first >= begin && grp.end <= end ? g : -1;
  }

  Status LaunchTileGroup(int program, int g, const Ctx& c) const {
    const TileGroup& grp = tgroups_[program][g];
    const auto& prog = plan_.program[program];
    GemmDesc ds[kGemmGroupMax];
    GemmPlan ps[kGemmGroupMax];
    int n = 0;
    for (const TileUnit& u : grp.units) {
      if (u.pre == 1)
        if (Status s = LaunchGemm(DescOf(prog[u.first + 1]), plans_[program][u.first + 1], c); !s) return s;
      if (u.pre == 2) {
        const auto& rows = chains_[program][u.chain].grp_rowdots;
        GemmDesc rd[4];
        for (size_t j = 0; j < rows.size(); ++j) rd[j] = DescOf(prog[rows[j]]);
        if (Status s = LaunchSkinnyRowdotGroup(rd, static_cast<int>(rows.size()), c); !s) return s;
      }
      ds[n] = u.d;
      ps[n] = u.plan;
      ++n;
    }
    return LaunchGemmGroup(ds, ps, n, c);
  }

  // The chain instruction idx belongs to in the built program, or null.
  const ChainRun* ChainAt(int program, size_t idx) const {
    for (const ChainRun& run : chains_[program])
      if (idx >= run.first && idx < run.first + run.count) return &run;
    return nullptr;
  }

  // Colsum groups (kernels.h LaunchSkinnyColsumGroup): 2..4 standalone
  // colsums on the skinny kernel over one large operand X (the LoRA
  // dA_j = x^T dt_j of the q/k/v projections, which share the layer input)
  // launch as one pass over X at the last member's position. The plan
  // reuses one slot for the dt_j, so each earlier member copies its small
  // operand to a private buffer at its own position: the group then reads
  // every operand's value of that position. An earlier member's output is
  // written later than in plan order, so nothing between the first and the
  // last member may write X, or read or write an earlier member's output;
  // the outputs are disjoint from each other and from every member's
  // operands. Each output has the bits of its own launch. Applied only when
  // the executed range holds the whole group.
  struct ColsumGroup {
    std::vector<size_t> members;      // plan order
    std::vector<size_t> priv_off;     // per earlier member: its copy, in floats
    std::vector<size_t> priv_floats;  // into cs_priv_[program]
  };

  static bool ColsumBigIsA(const GemmDesc& d) { return d.N <= 64 && d.M >= 128; }

  Status PlanColsumGroups(int program) {
    cs_groups_[program].clear();
    const auto& prog = plan_.program[program];
    cs_group_of_[program].assign(prog.size(), -1);
    if (cs_priv_[program]) {
      // A replay of the previous graph may still read the old copies.
      if (Status s = HipOk(hipStreamSynchronize(stream_), "colsum group sync"); !s) return s;
      (void)LockedFree(cs_priv_[program]);
      cs_priv_[program] = nullptr;
    }
    const auto& chains = chains_[program];
    std::vector<int> chain_of(prog.size(), -1);
    std::vector<uint8_t> rd_span(prog.size(), 0);  // inside a rowdot group's span
    for (size_t c = 0; c < chains.size(); ++c) {
      for (size_t k = chains[c].first; k < chains[c].first + chains[c].count; ++k)
        chain_of[k] = static_cast<int>(c);
      if (chains[c].rd_mode != 0)
        for (size_t k = chains[c].grp_first; k < chains[c].grp_end && k < prog.size(); ++k) rd_span[k] = 1;
    }
    auto marked = [&](size_t k) {
      return std::binary_search(marked_[program].begin(), marked_[program].end(), k);
    };
    auto candidate = [&](size_t k) {
      const UpdateInstruction& g = prog[k];
      return IsGemmOp(g.opcode) && g.flags == 0 && chain_of[k] < 0 && cs_group_of_[program][k] < 0 &&
             duals_[program][k] < 0 && plans_[program][k].cfg == GemmSkinnyConfig() &&
             SkinnyKindOf(DescOf(g)) == SkinnyKind::kColSum;
    };
    auto overlap = [](const Ranges& a, const Ranges& b) {
      for (const auto& x : a)
        if (Overlaps(b, x.first, x.second)) return true;
      return false;
    };
    size_t total = 0;
    for (size_t i = 0; i < prog.size(); ++i) {
      if (rd_span[i] || marked(i) || !candidate(i)) continue;
      GemmDesc ds[4];
      ds[0] = DescOf(prog[i]);
      const bool big_a = ColsumBigIsA(ds[0]);
      const uint64_t xref = big_a ? prog[i].in[0] : prog[i].in[1];
      const int64_t ldx = big_a ? ds[0].lda : ds[0].ldb, W = big_a ? ds[0].M : ds[0].N;
      Ranges xr;
      if (!IsRodataRef(xref))
        xr.emplace_back(RefOffset(xref), static_cast<uint64_t>((ds[0].K - 1) * ldx + W) * sizeof(float));
      std::vector<size_t> members{i};
      Ranges outs, ins;  // the members' outputs and operands
      if (!WriteRangesOf(prog[i], &outs) || !DependRangesOf(prog[i], &ins)) continue;
      for (size_t k = i + 1; k < prog.size() && k < i + 64 && members.size() < 4; ++k) {
        if (marked(k) || rd_span[k]) break;
        if (candidate(k)) {
          ds[members.size()] = DescOf(prog[k]);
          Ranges wk, rk;
          if (SkinnyColsumGroupFits(ds, static_cast<int>(members.size()) + 1) && WriteRangesOf(prog[k], &wk) &&
              DependRangesOf(prog[k], &rk) && !overlap(wk, ins) && !overlap(wk, outs) && !overlap(wk, rk) &&
              !overlap(rk, outs)) {
            members.push_back(k);
            outs.insert(outs.end(), wk.begin(), wk.end());
            ins.insert(ins.end(), rk.begin(), rk.end());
            continue;
          }
        }
        // an instruction between members, run in plan order
        const Ranges& w = writes_[program][k];
        if (overlap(w, xr) || overlap(w, outs) || overlap(depends_[program][k], outs)) break;
      }
      if (members.size() < 2) continue;
      ColsumGroup g;
      g.members = members;
      for (size_t j = 0; j + 1 < members.size(); ++j) {
        const GemmDesc d = DescOf(prog[members[j]]);
        const int64_t ld = big_a ? d.ldb : d.lda, R = big_a ? d.N : d.M;
        const size_t floats = static_cast<size_t>((d.K - 1) * ld + R);
        g.priv_off.push_back(total);
        g.priv_floats.push_back(floats);
        total += (floats + 63) / 64 * 64;  // 256-byte aligned copies
      }
      for (size_t m : members) cs_group_of_[program][m] = static_cast<int>(cs_groups_[program].size());
      cs_groups_[program].push_back(std::move(g));
    }
    if (total == 0) return Status::Ok();
    return HipOk(LockedMalloc(&cs_priv_[program], total * sizeof(float)), "colsum group copies");
  }

  // The colsum group instruction idx belongs to when the executed range
  // [begin, end) holds the whole group, else -1.
  int ColsumGroupAt(int program, size_t idx, size_t begin, size_t end) const {
    if (idx >= cs_group_of_[program].size() || cs_group_of_[program][idx] < 0) return -1;
    const int g = cs_group_of_[program][idx];
    const ColsumGroup& grp = cs_groups_[program][g];
    return grp.members.front() >= begin && grp.members.back() < end ? g : -1;
  }

  // Member idx's step of colsum group g: an earlier member copies its small
  // operand; the last launches the group.
  Status ColsumGroupStep(int program, int g, size_t idx, const Ctx& c) const {
    const ColsumGroup& grp = cs_groups_[program][g];
    const auto& prog = plan_.program[program];
    float* priv = static_cast<float*>(cs_priv_[program]);
    const size_t n = grp.members.size();
    GemmDesc ds[4];
    for (size_t j = 0; j < n; ++j) ds[j] = DescOf(prog[grp.members[j]]);
    const bool big_a = ColsumBigIsA(ds[0]);
    for (size_t j = 0; j + 1 < n; ++j) {
      const void*& small = big_a ? ds[j].B : ds[j].A;
      if (grp.members[j] == idx)
        return Copy(static_cast<const float*>(small), priv + grp.priv_off[j], grp.priv_floats[j], c);
      small = priv + grp.priv_off[j];
    }
    if (idx != grp.members.back()) return Status::Fail(kUnitEngine, "not a colsum group member");
    return LaunchSkinnyColsumGroup(ds, static_cast<int>(n), c);
  }

  Status LaunchChain(int program, const ChainRun& run, const Ctx& c, size_t begin, size_t end) {
    switch (run.kind) {
      case ChainKind::kDense: return LaunchGemm(run.d, plans_[program][run.first], c);
      case ChainKind::kLoraBase: {
        const size_t i1 = run.first + 1;
        const bool grouped = run.rd_mode != 0 && run.grp_first >= begin && run.grp_end <= end;
        if (grouped && run.rd_mode == 1) {
          GemmDesc ds[4];
          const int n = static_cast<int>(run.grp_rowdots.size());
          for (int j = 0; j < n; ++j) ds[j] = DescOf(plan_.program[program][run.grp_rowdots[j]]);
          if (Status s = LaunchSkinnyRowdotGroup(ds, n, c); !s) return s;
        } else if (!grouped) {
          if (Status s = LaunchGemm(DescOf(plan_.program[program][i1]), plans_[program][i1], c); !s)
            return s;
        }
        return LaunchGemm(run.d, plans_[program][run.first], c);
      }
      case ChainKind::kPointwise:
        if (run.recompute_from != ChainRun::kNoIndex && begin <= run.recompute_from)
          return LaunchPointwiseRun(run.pw_alt, c);
        if (run.cond_step >= 0 && end >= run.cond_until) {
          PointwiseRun pw = run.pw;
          pw.out[run.cond_step] = nullptr;
          return LaunchPointwiseRun(pw, c);
        }
        return LaunchPointwiseRun(run.pw, c);
      case ChainKind::kScaleFold:
        for (size_t k = run.first + 1; k < run.first + run.count;) {
          Status s = Status::Ok();
          k += FoldStep(program, run, k, c, &s);
          if (!s) return s;
        }
        return Status::Ok();
      case ChainKind::kDual: return LaunchDual(program, run.first, 3, nullptr, 1.0f, c);
      case ChainKind::kXentPass: {
        const UpdateInstruction& f = plan_.program[program][run.first];
        const UpdateInstruction& z = plan_.program[program][run.first + 1];
        const UpdateInstruction& b = plan_.program[program][run.first + 2];
        return SoftmaxXEntFwdBwd(RP(f.in[0]), IP(f.in[1]), WP(f.in[2]), run.store_p ? WP(f.in[3]) : nullptr,
                                 Bits(z.in[1]), WP(z.in[0]), WP(b.in[3]), f.out[0], f.out[1], c);
      }
      case ChainKind::kRopePair: {
        const UpdateInstruction& a = plan_.program[program][run.first];
        const UpdateInstruction& b = plan_.program[program][run.first + 1];
        const int dir = static_cast<Op>(a.opcode) == Op::kRopeFwd ? 1 : -1;
        return RopeWithTable(RP(a.in[0]), WP(a.in[1]), Hi(a.out[0]), Lo(a.out[0]), Hi(a.out[1]),
                             Lo(a.out[1]), RopeTableOf(Lo(a.out[0]), Lo(a.out[1]), a.out[2]), dir, c,
                             RP(b.in[0]), WP(b.in[1]));
      }
      case ChainKind::kAddRow: {
        const UpdateInstruction& g = plan_.program[program][run.first + 1];
        if (static_cast<Op>(g.opcode) == Op::kLayerNormFwd)
          return LayerNormFwd(RP(g.in[0]), RP(g.in[1]), RP(g.in[2]), WP(g.in[3]), WP(g.out[1]),
                              WP(g.out[2]), Hi(g.out[0]), Lo(g.out[0]), c, &run.pa);
        return RmsNormFwd(RP(g.in[0]), RP(g.in[1]), WP(g.in[2]), WP(g.in[3]), Hi(g.out[0]),
                          Lo(g.out[0]), c, &run.pa);
      }
      case ChainKind::kRowAdd: {
        const UpdateInstruction& g = plan_.program[program][run.first];
        if (static_cast<Op>(g.opcode) == Op::kLayerNormBwd)
          return LayerNormBwd(RP(g.in[0]), RP(g.in[1]), RP(g.in[2]), RP(g.out[0]), RP(g.out[1]),
                              WP(g.in[3]), Hi(g.out[2]), Lo(g.out[2]), c, &run.ra);
        return RmsNormBwd(RP(g.in[0]), RP(g.in[1]), RP(g.in[2]), RP(g.out[0]), WP(g.in[3]),
                          Hi(g.out[1]), Lo(g.out[1]), c, &run.ra);
      }
      default: return LaunchSkinnyChain(DescOf(plan_.program[program][run.first]), run.ch, c);
    }
  }

  // The captured launch sequence of instructions [begin, end): plan order,
  // fused AdamW runs and chains (wholly inside the range) as one
  // launch each.
  Status RunFused(int program, size_t begin, size_t end) {
    const Ctx c = MakeCtx();
    const auto& runs = fused_runs_[program];
    const auto& chains = chains_[program];
    size_t r = 0, q = 0;
    while (r < runs.size() && runs[r].first < begin) ++r;
    while (q < chains.size() && chains[q].first < begin) ++q;
    const auto& marks = marked_[program];
    for (size_t i = begin; i < end;) {
      // A marked launch (its tile group, if it heads one) between two wall
      // clock stamps, captured as nodes of the program's one graph.
      if (const auto mk = std::lower_bound(marks.begin(), marks.end(), i);
          mk != marks.end() && *mk == i && mark_stamps_[program]) {
        const size_t k = static_cast<size_t>(mk - marks.begin());
        const int tg = TileGroupAt(program, i, begin, end);
        if (Status s = WallStamp(mark_stamps_[program] + 3 * k, false, stream_); !s) return s;
        if (Status s = tg >= 0 ? LaunchTileGroup(program, tg, c) : Dispatch(program, i, c); !s) return s;
        if (Status s = WallStamp(mark_stamps_[program] + 3 * k, true, stream_); !s) return s;
        i = tg >= 0 ? tgroups_[program][tg].end : i + 1;
        while (q < chains.size() && chains[q].first < i) ++q;
        while (r < runs.size() && runs[r].first < i) ++r;
        continue;
      }
      if (const int tg = TileGroupAt(program, i, begin, end); tg >= 0) {
        if (Status s = LaunchTileGroup(program, tg, c); !s) return s;
        i = tgroups_[program][tg].end;
        while (q < chains.size() && chains[q].first < i) ++q;
        while (r < runs.size() && runs[r].first < i) ++r;
        continue;
      }
      if (q < chains.size() && chains[q].first == i && i + chains[q].count <= end) {
        if (Status s = LaunchChain(program, chains[q], c, begin, end); !s) return s;
        i += chains[q].count;
        ++q;
        continue;
      }
      if (r < runs.size() && runs[r].first == i && i + runs[r].count <= end) {
        if (Status s = AdamWMulti(fused_segs_[program] + runs[r].seg_offset, runs[r].count,
                                  runs[r].blocks, c);
            !s)
          return s;
        i += runs[r].count;
        ++r;
        continue;
      }
      if (const int g = ColsumGroupAt(program, i, begin, end); g >= 0) {
        if (Status s = ColsumGroupStep(program, g, i, c); !s) return s;
        ++i;
        continue;
      }
      if (Status s = Dispatch(program, i, c); !s) return s;
      ++i;
    }
    return Status::Ok();
  }

  // Timing inside ordinary replays: the program's graph is split at the
  // marked instructions; each marked launch runs between graph segments on
  // the engine stream, bracketed by HIP events, so its duration is measured
  // in the bench's timed steps rather than in a separate relaunch loop.
  // Marked AdamW instructions are left out of multi-tensor fusion.
  Status MarkTimed(int program, const uint64_t* idx, size_t n) {
    if (program < 0 || program > 2) return Status::Fail(kUnitEngine, "unknown program id");
    std::vector<size_t> v;
    for (size_t j = 0; j < n; ++j) {
      if (idx[j] >= plan_.program[program].size())
        return Status::Fail(kUnitEngine, "timed instruction index out of range");
      v.push_back(idx[j]);
    }
    std::sort(v.begin(), v.end());
    v.erase(std::unique(v.begin(), v.end()), v.end());
    if (Status s = HipOk(hipStreamSynchronize(stream_), "mark sync"); !s) return s;
    for (hipEvent_t e : mark_ev_[program]) (void)hipEventDestroy(e);
    mark_ev_[program].clear();
    if (mark_stamps_[program]) (void)LockedFree(mark_stamps_[program]);
    mark_stamps_[program] = nullptr;
    marked_[program] = v;
    if (!v.empty()) {
      if (wall_khz_ == 0)
        (void)hipDeviceGetAttribute(&wall_khz_, hipDeviceAttributeWallClockRate, device_);
      const size_t bytes = 3 * v.size() * sizeof(uint64_t);
      if (Status s = HipOk(LockedMalloc(&mark_stamps_[program], bytes), "timing stamps"); !s) return s;
      if (Status s = HipOk(hipMemsetAsync(mark_stamps_[program], 0, bytes, stream_), "timing stamps"); !s)
        return s;
      if (h_stamps_cap_ < 3 * v.size()) {
        if (h_stamps_) (void)LockedHostFree(h_stamps_);
        h_stamps_ = nullptr;
        h_stamps_cap_ = 0;
        if (Status s = HipOk(LockedHostMalloc(&h_stamps_, bytes), "timing stamps"); !s) return s;
        h_stamps_cap_ = 3 * v.size();
      }
    }
    for (size_t j = 0; j < 2 * v.size(); ++j) {
      hipEvent_t e = nullptr;
      if (Status s = HipOk(hipEventCreate(&e), "timing event"); !s) return s;
      mark_ev_[program].push_back(e);
    }
    DropGraph(program);  // rebuilt with the event nodes on next use
    return Status::Ok();
  }

  // Durations (ms) of the marked launches: with stamp nodes, the mean over the
  // replays since the last read; with events, the most recent replay's.
  Status MarkedTimes(int program, float* ms, size_t n) {
    if (program < 0 || program > 2) return Status::Fail(kUnitEngine, "unknown program id");
    if (n < marked_[program].size()) return Status::Fail(kUnitEngine, "timing output too small");
    if (stamped_[program] && use_graph_) {
      // The mean over the replays since the previous read (the sums restart).
      const size_t m = marked_[program].size();
      const size_t bytes = 3 * m * sizeof(uint64_t);
      if (Status s = HipOk(hipMemcpyAsync(h_stamps_, mark_stamps_[program], bytes, hipMemcpyDeviceToHost,
                                          stream_),
                           "timing read");
          !s)
        return s;
      if (Status s = HipOk(hipMemsetAsync(mark_stamps_[program], 0, bytes, stream_), "timing reset"); !s)
        return s;
      if (Status s = HipOk(hipStreamSynchronize(stream_), "timing read"); !s) return s;
      for (size_t k = 0; k < m; ++k) {
        const uint64_t n = h_stamps_[3 * k + 2];
        ms[k] = n ? static_cast<float>(static_cast<double>(h_stamps_[3 * k + 1]) / n / wall_khz_) : 0.0f;
      }
      return Status::Ok();
    }
    for (size_t k = 0; k < marked_[program].size(); ++k) {
      float t = 0.0f;
      if (Status s = HipOk(hipEventElapsedTime(&t, mark_ev_[program][2 * k],
                                               mark_ev_[program][2 * k + 1]),
                           "timing read");
          !s)
        return s;
      ms[k] = t;
    }
    return Status::Ok();
  }

  // Captures instructions [begin, end) as one graph segment.
  Status Capture(int program, size_t begin, size_t end) {
    std::lock_guard<std::recursive_mutex> lock(DeviceMemMutex());
    if (Status s = HipOk(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal),
                         "graph capture begin");
        !s)
      return s;
    Status launched = RunFused(program, begin, end);
    if (launched && end == plan_.program[program].size() && PostsLoss(program))
      launched = PostLoss(RP(plan_.header.loss_ref), h_loss_, stream_);
    hipGraph_t g = nullptr;
    const hipError_t stop = hipStreamEndCapture(stream_, &g);
    if (!launched) {
      if (g) (void)hipGraphDestroy(g);
      return launched;
    }
    if (Status s = HipOk(stop, "graph capture end"); !s) return s;
    Segment seg;
    seg.graph = g;
    seg.first = begin;
    seg.count = end - begin;
    segs_[program].push_back(seg);
    return HipOk(hipGraphInstantiate(&segs_[program].back().exec, g, nullptr, nullptr, 0),
                 "graph instantiate");
  }

  Status Build(int program) {
    if (program < 0 || program > 2) return Status::Fail(kUnitEngine, "unknown program id");
    if (Status s = EnsureWorkspace(program); !s) return s;
    DropGraph(program);
    if (!use_graph_ || plan_.program[program].empty()) {
      built_[program] = true;
      return Status::Ok();
    }
    if (Status s = PlanFusion(program); !s) return s;
    // the colsum groups' partials can need more workspace than any launch alone
    if (Status s = EnsureWorkspace(program); !s) return s;
    // One graph for the whole program, each marked launch between two wall
    // clock stamp nodes (timing events do not record from inside a graph
    // on this runtime). Without the stamp buffer or clock rate: one graph
    // per unmarked stretch and each marked launch between them, timed by
    // events.
    const size_t n = plan_.program[program].size();
    stamped_[program] = false;
    if (!marked_[program].empty() && mark_stamps_[program] && wall_khz_ > 0) {
      if (Status s = Capture(program, 0, n); !s) return s;
      stamped_[program] = true;
      built_[program] = true;
      return Status::Ok();
    }
    size_t begin = 0;
    for (size_t k = 0; k <= marked_[program].size(); ++k) {
      const size_t end = k < marked_[program].size() ? marked_[program][k] : n;
      if (end > begin)
        if (Status s = Capture(program, begin, end); !s) return s;
      if (k < marked_[program].size()) {
        // A marked tile group's first instruction times the whole group.
        const int tg = TileGroupAt(program, end, 0, n);
        Segment seg;
        seg.first = end;
        seg.count = tg >= 0 ? tgroups_[program][tg].end - end : 1;
        seg.mark = static_cast<long>(k);
        segs_[program].push_back(seg);
        begin = end + seg.count;
      }
    }
    built_[program] = true;
    return Status::Ok();
  }

  // The train and eval programs end in a loss.
  bool PostsLoss(int program) const {
    return (program == static_cast<int>(Program::kTrain) || program == static_cast<int>(Program::kEval)) &&
           plan_.header.loss_ref != kNullRef;
  }

  Status Run(int program) {
    if (program < 0 || program > 2) return Status::Fail(kUnitEngine, "unknown program id");
    loss_posted_ = false;
    if (!built_[program])
      if (Status s = Build(program); !s) return s;
    if (plan_.program[program].empty()) return Status::Ok();
    if (!use_graph_) {
      if (Status s = RunEager(program); !s) return s;
      if (PostsLoss(program)) {
        if (Status s = PostLoss(RP(plan_.header.loss_ref), h_loss_, stream_); !s) return s;
        loss_posted_ = true;
      }
      return Status::Ok();
    }
    const Ctx c = MakeCtx();
    for (const Segment& g : segs_[program]) {
      if (g.mark < 0) {
        if (Status s = HipOk(hipGraphLaunch(g.exec, stream_), "graph launch"); !s) return s;
        continue;
      }
      (void)hipEventRecord(mark_ev_[program][2 * g.mark], stream_);
      const int tg = TileGroupAt(program, g.first, 0, plan_.program[program].size());
      if (Status s = tg >= 0 ? LaunchTileGroup(program, tg, c) : Dispatch(program, g.first, c); !s) return s;
      (void)hipEventRecord(mark_ev_[program][2 * g.mark + 1], stream_);
    }
    if (PostsLoss(program)) {
      // A graph ending the program posted the loss; a marked last launch did not.
      if (segs_[program].empty() || segs_[program].back().mark >= 0)
        if (Status s = PostLoss(RP(plan_.header.loss_ref), h_loss_, stream_); !s) return s;
      loss_posted_ = true;
    }
    return Status::Ok();
  }

  // The step's scalars travel as the staging kernel's arguments, copied at
  // launch: no host buffer outlives the call, and back-to-back steps need
  // no wait on an earlier upload.
  Status SetStep(uint64_t step) {
    const StepScalars sc = MakeStepScalars(plan_.header, step == 0 ? 1 : step);
    if (Status s = StageStep(&sc, d_scalars_, nullptr, nullptr, 0, nullptr, nullptr, 0, stream_); !s)
      return s;
    step_ = step;
    loss_posted_ = false;
    return Status::Ok();
  }

  // The feeder contract's bounds (contract.cc:173-207) on host-staged ids.
  Status CheckIds(const int32_t* ids, size_t n, uint64_t bound, const char* what) const {
    for (size_t i = 0; i < n; ++i)
      if (ids[i] < 0 || static_cast<uint64_t>(ids[i]) >= bound)
        return Status::Fail(kUnitEngine, std::string(what) + " " + std::to_string(ids[i]) +
                                             " at row " + std::to_string(i) +
                                             " is outside [0, " + std::to_string(bound) + ")");
    return Status::Ok();
  }

  Status Stage(const void* input, size_t input_bytes, const void* labels, size_t label_bytes,
               bool on_device) {
    if (Status s = CheckStaged(input, input_bytes, labels, label_bytes, on_device); !s) return s;
    const PlanHeader& h = plan_.header;
    loss_posted_ = false;
    const hipMemcpyKind kind = on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
    if (input_bytes)
      if (Status s = HipOk(hipMemcpyAsync(arena_ + RefOffset(h.input_ref), input, input_bytes,
                                          kind, stream_),
                           "input staging");
          !s)
        return s;
    if (h.label_kind != 0 && labels && label_bytes)
      if (Status s = HipOk(hipMemcpyAsync(arena_ + RefOffset(h.label_ref), labels, label_bytes,
                                          kind, stream_),
                           "label staging");
          !s)
        return s;
    return Status::Ok();
  }

  // The staged batch's sizes against the plan's slots, and (host batches)
  // the feeder contract's id bounds.
  Status CheckStaged(const void* input, size_t input_bytes, const void* labels, size_t label_bytes,
                     bool on_device) const {
    const PlanHeader& h = plan_.header;
    if (input_bytes != h.input_floats * 4)
      return Status::Fail(kUnitEngine, "staged input size does not match the plan input slot");
    if (h.label_kind != 0 && label_bytes != h.label_bytes)
      return Status::Fail(kUnitEngine, "staged label size does not match the plan label slot");
    if (!on_device) {
      if (h.input_kind == 1) {
        uint64_t bound = plan_.vocab_bound;
        if (plan_.num_classes && plan_.num_classes < bound) bound = plan_.num_classes;
        if (Status s = CheckIds(static_cast<const int32_t*>(input), h.input_floats, bound,
                                "token id");
            !s)
          return s;
      }
      if (h.label_kind == 1 && labels)
        if (Status s = CheckIds(static_cast<const int32_t*>(labels), label_bytes / 4,
                                plan_.num_classes, "class label");
            !s)
          return s;
    }
    return Status::Ok();
  }

  // After a whole train or eval program the loss is already on its way to
  // h_loss_ (PostLoss ends those programs); otherwise it is copied back.
  Status Loss(float* out) {
    if (loss_posted_) {
      if (Status s = HipOk(hipStreamSynchronize(stream_), "step"); !s) return s;
      *out = *h_loss_;
      return Status::Ok();
    }
    if (Status s = HipOk(hipMemcpyAsync(h_loss_, arena_ + RefOffset(plan_.header.loss_ref),
                                        sizeof(float), hipMemcpyDeviceToHost, stream_),
                         "loss read");
        !s)
      return s;
    if (Status s = HipOk(hipStreamSynchronize(stream_), "step"); !s) return s;
    *out = *h_loss_;
    return Status::Ok();
  }

  // The batch is validated and staged before step_ advances: a rejected
  // batch leaves the step counter (AdamW bias correction, LR schedule) as
  // it was.
  Status TrainStep(const void* input, size_t input_bytes, const void* labels, size_t label_bytes,
                   bool on_device, float* loss) {
    if (on_device) {
      // One launch stages a small device batch and the next step's scalars;
      // a large batch (C2's 134 MB inputs) goes through the runtime's copy,
      // which moves it faster than the staging kernel's.
      if (Status s = CheckStaged(input, input_bytes, labels, label_bytes, on_device); !s) return s;
      const PlanHeader& h = plan_.header;
      bool lab = h.label_kind != 0 && labels && label_bytes;
      bool inp = input_bytes != 0;
      constexpr size_t kKernelCopyMax = size_t{8} << 20;
      if (inp && input_bytes > kKernelCopyMax) {
        if (Status s = HipOk(hipMemcpyAsync(arena_ + RefOffset(h.input_ref), input, input_bytes,
                                            hipMemcpyDeviceToDevice, stream_),
                             "input staging");
            !s)
          return s;
        inp = false;
      }
      if (lab && label_bytes > kKernelCopyMax) {
        if (Status s = HipOk(hipMemcpyAsync(arena_ + RefOffset(h.label_ref), labels, label_bytes,
                                            hipMemcpyDeviceToDevice, stream_),
                             "label staging");
            !s)
          return s;
        lab = false;
      }
      const StepScalars sc = MakeStepScalars(plan_.header, step_ + 1);
      if (Status s = StageStep(&sc, d_scalars_, inp ? input : nullptr, arena_ + RefOffset(h.input_ref),
                               inp ? input_bytes : 0, lab ? labels : nullptr,
                               lab ? arena_ + RefOffset(h.label_ref) : nullptr, lab ? label_bytes : 0,
                               stream_);
          !s)
        return s;
      step_ = step_ + 1;
      loss_posted_ = false;
    } else {
      if (Status s = Stage(input, input_bytes, labels, label_bytes, on_device); !s) return s;
      if (Status s = SetStep(step_ + 1); !s) return s;
    }
    if (Status s = Run(static_cast<int>(Program::kTrain)); !s) return s;
    float l = 0.0f;
    if (Status s = Loss(&l); !s) return s;
    if (loss) *loss = l;
    if (!std::isfinite(l))
      return Status::Fail(kUnitEngine, "loss became non-finite at step " + std::to_string(step_) +
                                           " — aborting the update");
    return Status::Ok();
  }

  Status RunMerge() {
    if (Status s = Run(static_cast<int>(Program::kMerge)); !s) return s;
    if (Status s = HipOk(hipStreamSynchronize(stream_), "merge"); !s) return s;
    std::vector<float> buf;
    for (const EmitEntry& e : plan_.emit) {
      buf.resize(e.byte_size / 4);
      if (Status s = HipOk(hipMemcpyAsync(buf.data(), arena_ + e.arena_offset, e.byte_size,
                                          hipMemcpyDeviceToHost, stream_),
                           "delta read");
          !s)
        return s;
      if (Status s = HipOk(hipStreamSynchronize(stream_), "delta read"); !s) return s;
      for (float v : buf)
        if (!std::isfinite(v))
          return Status::Fail(kUnitEngine,
                              "merged delta contains a non-finite value — the adapters are "
                              "numerically poisoned; refusing to stage a commit");
    }
    return Status::Ok();
  }

  // ---- EvaluateMetrics / TrainImpl (update_engine.cc:557-787) ------------
  struct EvalOut {
    float loss = 0.0f;
    bool has_accuracy = false;
    float accuracy = 0.0f;
  };
  struct ReportOut {
    uint64_t steps = 0;
    float initial_avg_loss = 0.0f, final_avg_loss = 0.0f;
    bool has_validation = false;
    float val_initial_loss = 0.0f, val_final_loss = 0.0f;
    bool has_val_accuracy = false;
    float val_initial_accuracy = 0.0f, val_final_accuracy = 0.0f;
    bool stopped_early = false;
    bool improved() const {
      return has_validation ? val_final_loss < val_initial_loss
                            : final_avg_loss < initial_avg_loss;
    }
  };

  uint8_t* SlotPtr(uint64_t ref) const { return ref == kNullRef ? nullptr : arena_ + RefOffset(ref); }

  Status EnsureArgmaxBuffers(uint64_t rows) {
    const size_t need = ArgmaxPartials(rows);
    if (need <= argmax_cap_ && d_argmax_) return Status::Ok();
    if (d_argmax_) (void)LockedFree(d_argmax_);
    d_argmax_ = nullptr;
    argmax_cap_ = 0;
    // [total u64][partials u32 ...]
    if (Status s = HipOk(LockedMalloc(&d_argmax_, 8 + 4 * std::max<size_t>(need, 1)), "argmax buffers");
        !s)
      return s;
    argmax_cap_ = need;
    if (!h_count_)
      if (Status s = HipOk(LockedHostMalloc(&h_count_, sizeof(uint64_t)), "pinned count"); !s) return s;
    return Status::Ok();
  }

  Status EvaluateMetrics(Dataset& data, EvalOut* out) {
    const PlanHeader& h = plan_.header;
    const int kEval = static_cast<int>(Program::kEval);
    if (plan_.program[kEval].empty())
      return Status::Fail(kUnitEngine, "plan carries no eval program");
    if (Status s = VerifyFeederContract(h, data, plan_.num_classes, plan_.vocab_bound); !s)
      return s;
    // Every pass over a set scores the same samples: snapshot, rewind, and
    // restore afterwards (the restore replays the permutation epoch).
    const Dataset::ServingPos entry = data.SaveServingPos();
    data.Rewind();
    const bool has_labels = h.label_kind != 0;
    const bool track = h.label_kind == 1 && plan_.eval_probs_ref != kNullRef &&
                       plan_.eval_softmax_cols > 0 && plan_.eval_softmax_rows >= h.batch;
    const uint64_t rows_per_sample = h.input_kind == 1 ? h.seq_len : 1;
    const uint64_t per_step = h.batch / rows_per_sample;
    const uint64_t n = data.num_samples();
    const uint64_t batches = std::max<uint64_t>(1, (n + per_step - 1) / per_step);
    double total = 0.0;
    uint64_t correct = 0, counted = 0;
    Status st = track ? EnsureArgmaxBuffers(h.batch) : Status::Ok();
    if (st) {
      BatchStager feeder(data, h.batch, h.input_floats * 4, has_labels ? h.label_bytes : 0);
      st = feeder.Start();
      for (uint64_t b = 0; st && b < batches; ++b) {
        st = feeder.Next(SlotPtr(h.input_ref), has_labels ? SlotPtr(h.label_ref) : nullptr, stream_);
        if (st) st = Run(kEval);
        // Rows of the final batch past the set's end are wrapped duplicates:
        // the loss mean keeps them, accuracy judges each real row once.
        const uint64_t served = b * per_step;
        const uint64_t real = std::min<uint64_t>(per_step, n > served ? n - served : 0) * rows_per_sample;
        if (st && track && real) {
          Ctx c = MakeCtx();
          uint64_t* d_total = reinterpret_cast<uint64_t*>(d_argmax_);
          uint32_t* partials = reinterpret_cast<uint32_t*>(d_argmax_ + 8);
          st = ArgmaxCorrect(RP(plan_.eval_probs_ref),
                             reinterpret_cast<const int32_t*>(SlotPtr(h.label_ref)), real,
                             plan_.eval_softmax_cols, partials, d_total, c);
          if (st)
            st = HipOk(hipMemcpyAsync(h_count_, d_total, sizeof(uint64_t), hipMemcpyDeviceToHost,
                                      stream_),
                       "accuracy read");
        }
        float l = 0.0f;
        if (st) st = Loss(&l);  // synchronizes the stream (the count read too)
        if (!st) break;
        total += l;
        if (track && real) {
          correct += *h_count_;
          counted += real;
        }
      }
    }  // the feeder joins here and returns a staged, unconsumed batch
    data.RestoreServingPos(entry);
    if (!st) return st;
    out->loss = static_cast<float>(total / static_cast<double>(batches));
    out->has_accuracy = track && counted > 0;
    out->accuracy = out->has_accuracy ? static_cast<float>(static_cast<double>(correct) /
                                                           static_cast<double>(counted))
                                      : 0.0f;
    return Status::Ok();
  }

  // SaveCheckpoint / LoadCheckpoint (update_engine.cc:894-913): the
  // persistent segment [0, persistent_size) and step_, in the SEKP container.
  Status SaveCheckpoint(const std::string& path) {
    const uint64_t n = plan_.header.persistent_size;
    std::vector<uint8_t> host(n);
    if (Status s = Access(0, host.data(), n, false); !s) return s;
    return WriteCheckpoint(path, plan_.header.plan_hash, step_, host.data(), n);
  }
  Status LoadCheckpoint(const std::string& path) {
    loss_posted_ = false;  // runs instructions outside Run()
    const uint64_t n = plan_.header.persistent_size;
    std::vector<uint8_t> host(n);
    uint64_t step = 0;
    if (Status s = ReadCheckpoint(path, plan_.header.plan_hash, n, host.data(), &step); !s)
      return s;
    if (Status s = Access(0, host.data(), n, true); !s) return s;
    return SetStep(step);
  }

  // TrainOptions (update_engine.h:40-60): checkpoint file, period, resume.
  struct TrainOptions {
    std::string checkpoint_path;
    uint64_t checkpoint_every = 0;
    bool resume = false;
    int (*should_stop)(void*) = nullptr;  // polled once per step
    void* should_stop_ctx = nullptr;
  };

  Status Train(Dataset& data, uint64_t steps, Dataset* validation, float* curve,
               uint64_t curve_cap, ReportOut* rep, const TrainOptions& opt) {
    const PlanHeader& h = plan_.header;
    if (steps == 0) steps = h.default_steps;
    if (steps == 0)
      return Status::Fail(kUnitEngine, "no steps requested and the plan has no default");
    if (Status s = VerifyFeederContract(h, data, plan_.num_classes, plan_.vocab_bound); !s)
      return s;
    if (validation)
      if (Status s = VerifyFeederContract(h, *validation, plan_.num_classes, plan_.vocab_bound); !s)
        return s;
    if (opt.resume && !opt.checkpoint_path.empty()) {
      // A missing or unusable checkpoint is reported and training starts
      // from the current state (update_engine.cc:676-680). A resumed step
      // replays the feeder to where the interrupted run stood: step_
      // batches of h.batch rows, epoch reshuffles included, so the resumed
      // run is the uninterrupted one bit for bit (update_engine.cc:681-695).
      if (Status s = LoadCheckpoint(opt.checkpoint_path); !s) {
        std::fprintf(stderr, "seeml-update: no checkpoint resumed (%s)\n", s.error.c_str());
      } else if (step_ > 0) {
        uint64_t served = 0;
        if (!MulOk(step_, h.batch, &served))
          return Status::Fail(kUnitEngine, "resumed step count overflows the feeder position");
        if (Status s = data.SkipServed(served); !s) return s;
      }
    }
    ReportOut report;
    if (validation) {
      EvalOut v;
      if (Status s = EvaluateMetrics(*validation, &v); !s) return s;
      report.has_validation = true;
      report.val_initial_loss = v.loss;
      report.has_val_accuracy = v.has_accuracy;
      report.val_initial_accuracy = v.accuracy;
    }
    const bool has_labels = h.label_kind != 0;
    const uint64_t window = std::max<uint64_t>(1, std::min<uint64_t>(20, steps / 5));
    double first_sum = 0.0, last_sum = 0.0;
    uint64_t first_n = 0, last_n = 0, executed = 0;
    const uint64_t start = step_;
    Status st;
    {
      // The feeder stages step s+1's batch while step s runs; the served
      // sequence is exactly the serial one.
      BatchStager feeder(data, h.batch, h.input_floats * 4, has_labels ? h.label_bytes : 0);
      st = feeder.Start();
      for (uint64_t s = start; st && s < start + steps; ++s) {
        if (opt.should_stop && opt.should_stop(opt.should_stop_ctx)) {
          report.stopped_early = true;  // update_engine.cc:737-740
          break;
        }
        st = SetStep(s + 1);  // 1-indexed step for AdamW bias correction
        if (st)
          st = feeder.Next(SlotPtr(h.input_ref), has_labels ? SlotPtr(h.label_ref) : nullptr,
                           stream_);
        if (st) st = Run(static_cast<int>(Program::kTrain));
        float loss = 0.0f;
        if (st) st = Loss(&loss);
        if (!st) break;
        ++executed;
        if (!std::isfinite(loss)) {
          st = Status::Fail(kUnitEngine, "loss became non-finite at step " +
                                             std::to_string(step_) + " — aborting the update");
          break;
        }
        if (curve && s - start < curve_cap) curve[s - start] = loss;
        if (s - start < window) {
          first_sum += loss;
          ++first_n;
        }
        if (s - start >= steps - window) {
          last_sum += loss;
          ++last_n;
        }
        if (opt.checkpoint_every && !opt.checkpoint_path.empty() &&
            step_ % opt.checkpoint_every == 0) {
          st = SaveCheckpoint(opt.checkpoint_path);
          if (!st) break;
        }
      }
    }
    if (!st) return st;
    report.steps = executed;
    report.initial_avg_loss = first_n ? static_cast<float>(first_sum / first_n) : 0.0f;
    report.final_avg_loss = last_n ? static_cast<float>(last_sum / last_n) : report.initial_avg_loss;
    if (validation) {
      EvalOut v;
      if (Status s = EvaluateMetrics(*validation, &v); !s) return s;
      report.val_final_loss = v.loss;
      report.val_final_accuracy = v.accuracy;
    }
    *rep = report;
    return Status::Ok();
  }

  Status Access(uint64_t ref, void* host, size_t bytes, bool write) {
    const bool ro = IsRodataRef(ref);
    if (write && ro) return Status::Fail(kUnitEngine, "rodata is not writable");
    const uint64_t off = RefOffset(ref);
    const uint64_t space = ro ? plan_.header.rodata_size : plan_.header.arena_size;
    if (!RangeOk(off, bytes, space)) return Status::Fail(kUnitEngine, "probe out of bounds");
    uint8_t* dev = (ro ? rodata_ : arena_) + off;
    if (write) loss_posted_ = false;
    if (Status s = HipOk(hipStreamSynchronize(stream_), "probe sync"); !s) return s;
    if (Status s = HipOk(write ? hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, stream_)
                              : hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, stream_),
                         "probe copy");
        !s)
      return s;
    return HipOk(hipStreamSynchronize(stream_), "probe copy");
  }

  // Test hook: one GEMM instruction's plan, forced; the graph is rebuilt (and
  // its fusions re-planned) on the program's next run.
  Status SetGemmPlan(int program, size_t index, int cfg, int splits) {
    if (program < 0 || program > 2 || index >= plan_.program[program].size() ||
        !IsGemmOp(plan_.program[program][index].opcode) || cfg < 0 || cfg >= GemmConfigCount())
      return Status::Fail(kUnitEngine, "set_gemm_plan: not a GEMM instruction or config");
    plans_[program][index] = PlanGemmWith(DescOf(plan_.program[program][index]), cfg, splits);
    DropGraph(program);
    return Status::Ok();
  }

  // ---- GEMM tile autotuning ------------------------------------------------
  // With `inject`, each pull's reward comes from inject(ctx, group, arm, cfg,
  // splits, n_split) instead of a timed launch, and nothing is launched (the
  // reference's injected reward closure, test/compiler/backend/tuner_test.cc:130-145).
  using RewardFn = double (*)(void*, uint64_t, uint64_t, int, int, uint64_t);
  // The tile groups the per-shape picks form, re-tuned as launches: a
  // group holds two to four times one GEMM's tiles, so its best tile can
  // differ from the lone GEMM's. Groups of one signature (each member's
  // opcode, shape and epilogue kind, in order) are tuned once, on the first
  // such group, and share the pick. Arms: every tile config the members fit
  // as one group (their epilogues included) at one slice, the current pick
  // first; reward as in Autotune. Any tile config keeps the summation order.
  Status TuneTileGroups(int program, int budget, hipEvent_t t0, hipEvent_t t1) {
    if (Status s = EnsureWorkspace(program); !s) return s;
    if (Status s = PlanFusion(program); !s) return s;
    const auto& prog = plan_.program[program];
    const std::vector<TileGroup> groups = tgroups_[program];
    const Ctx c = MakeCtx();
    auto signature = [&](const TileGroup& g) {
      std::vector<uint64_t> key;
      for (const TileUnit& u : g.units) {
        const UpdateInstruction& ins = prog[u.first];
        key.insert(key.end(), {ins.opcode, ins.out[0], ins.out[1], ins.out[2],
                               static_cast<uint64_t>(u.d.lora_t ? 2 : u.d.out ? 1 : 0)});
      }
      return key;
    };
    std::map<std::vector<uint64_t>, int> picked;
    for (const TileGroup& g : groups) {
      const int n = static_cast<int>(g.units.size());
      const auto key = signature(g);
      if (const auto it = picked.find(key); it != picked.end()) {
        for (const TileUnit& u : g.units)
          plans_[program][u.first] = PlanGemmWith(DescOf(prog[u.first]), it->second, 1);
        continue;
      }
      GemmDesc ds[kGemmGroupMax];
      double flops = 0.0;
      for (int j = 0; j < n; ++j) {
        ds[j] = g.units[j].d;
        flops += GemmFlops(ds[j]);
      }
      std::vector<int> arms{g.units[0].plan.cfg};
      picked[key] = arms[0];
      for (int cfg = 0; cfg < GemmSkinnyConfig(); ++cfg) {
        if (cfg == arms[0]) continue;
        GemmPlan ps[kGemmGroupMax];
        bool ok = true;
        for (int j = 0; j < n && ok; ++j) {
          ps[j] = PlanGemmWith(DescOf(prog[g.units[j].first]), cfg, 1);
          ok = GemmPlanKeepsOrder(DescOf(prog[g.units[j].first]), ps[j]);
        }
        if (ok && GemmGroupFits(ds, ps, n)) arms.push_back(cfg);
      }
      if (arms.size() < 2) continue;
      auto launch = [&](int cfg) {
        GemmPlan ps[kGemmGroupMax];
        for (int j = 0; j < n; ++j) ps[j] = PlanGemmWith(DescOf(prog[g.units[j].first]), cfg, 1);
        return LaunchGemmGroup(ds, ps, n, c);
      };
      for (int cfg : arms)  // one untimed warm-up launch per arm
        if (Status s = launch(cfg); !s) return s;
      Ucb1 bandit(arms.size());
      const int trials = std::max<int>(budget, 2 * static_cast<int>(arms.size()));
      for (int t = 0; t < trials; ++t) {
        const size_t arm = bandit.Select();
        (void)hipEventRecord(t0, stream_);
        if (Status s = launch(arms[arm]); !s) return s;
        (void)hipEventRecord(t1, stream_);
        (void)hipEventSynchronize(t1);
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, t0, t1);
        bandit.Update(arm, ms > 0.0f ? flops / (ms * 1e-3) / kPeakFp32MfmaFlops : 0.0);
      }
      const int best = arms[bandit.Best(kAutotuneTileTolerance)];
      picked[key] = best;
      for (const TileUnit& u : g.units)
        plans_[program][u.first] = PlanGemmWith(DescOf(prog[u.first]), best, 1);
    }
    return Status::Ok();
  }

  // The Scale whose output GEMM g would read through PlanScaleFolds' fold
  // (its pattern, without the liveness and hazard checks made when the graph
  // is built): the Scale right before the run of GEMMs that holds g, each
  // streaming its output, the Scale's output in the arena (transient, so
  // autotuning may run it), its input 16-byte aligned. -1 if none.
  long FoldScaleOf(int program, size_t g) const {
    const auto& prog = plan_.program[program];
    size_t i = g;
    while (i > 0 && IsGemmOp(prog[i - 1].opcode)) --i;
    if (i == 0 || static_cast<Op>(prog[i - 1].opcode) != Op::kScale) return -1;
    const UpdateInstruction& sc = prog[i - 1];
    if (IsRodataRef(sc.in[1]) || RefOffset(sc.in[1]) < plan_.header.persistent_size ||
        !aligned16(RP(sc.in[0])))
      return -1;
    for (size_t j = i; j <= g; ++j) {
      const GemmDesc d = DescOf(prog[j]);
      int64_t elems = 0;
      const void* stream = SkinnyStream(d, &elems);
      if (stream != WP(sc.in[1]) || static_cast<uint64_t>(elems) != sc.out[0] ||
          (d.A == stream ? d.B : d.A) == WP(sc.in[1]))
        return -1;
    }
    return static_cast<long>(i - 1);
  }

  Status Autotune(int budget, RewardFn inject = nullptr, void* inject_ctx = nullptr) {
    loss_posted_ = false;  // runs instructions outside Run()
    const int program = static_cast<int>(Program::kTrain);
    const auto& prog = plan_.program[program];
    const uint64_t persist = plan_.header.persistent_size;
    std::map<std::tuple<uint16_t, uint64_t, uint64_t, uint64_t>, std::vector<size_t>> groups;
    for (size_t i = 0; i < prog.size(); ++i) {
      const UpdateInstruction& ins = prog[i];
      if (!IsGemmOp(ins.opcode) || ins.opcode == static_cast<uint16_t>(Op::kGemmAccNN)) continue;
      // Tune only in scratch-safe places: the output must be a transient,
      // never the persistent segment the optimizer state lives in.
      if (RefOffset(ins.in[2]) < persist) continue;
      groups[{ins.opcode, ins.out[0], ins.out[1], ins.out[2]}].push_back(i);
    }
    hipEvent_t t0, t1;
    if (Status s = HipOk(hipEventCreate(&t0), "event"); !s) return s;
    if (Status s = HipOk(hipEventCreate(&t1), "event"); !s) return s;
    Status result = Status::Ok();
    uint64_t group = 0;
    for (auto& [key, idxs] : groups) {
      const size_t first = idxs.front();
      const GemmDesc d = DescOf(prog[first]);
      const GemmOrder order = GemmOrderOf(d);
      // Arm 0 is the heuristic plan; the others are every tile config at
      // the order's split count and, at one split, the column splits (whole
      // rounds of 256x128 tiles, the rest on 128x128, 128x64 or 64x64 tiles). The
      // skinny kernels' order has one kernel: nothing to tune.
      const GemmPlan hint = PlanGemm(d);
      const uint64_t gid = group++;
      if (order.skinny) {
        for (size_t i : idxs) plans_[program][i] = hint;
        continue;
      }
      std::vector<GemmPlan> arms{hint};
      auto add = [&](const GemmPlan& p) {
        for (const auto& a : arms)
          if (a.cfg == p.cfg && a.splits == p.splits && a.n_split == p.n_split &&
              a.tail_cfg == p.tail_cfg)
            return;
        arms.push_back(p);
      };
      for (int cfg = 0; cfg < GemmSkinnyConfig(); ++cfg) add(PlanGemmWith(d, cfg, order.splits));
      if (order.splits == 1)
        for (int tail : {0, 4, 5}) {
          const GemmPlan sp = PlanGemmSplit(d, 2, tail);
          if (sp.n_split > 0) add(sp);
        }
      for (const auto& a : arms)
        if (!GemmPlanKeepsOrder(d, a)) {
          result = Status::Fail(kUnitEngine, "autotune: an arm would change the summation order");
          break;
        }
      if (!result) break;
      if (inject) {
        Ucb1 bandit(arms.size());
        const int trials = std::max<int>(budget, 2 * static_cast<int>(arms.size()));
        for (int t = 0; t < trials; ++t) {
          const size_t arm = bandit.Select();
          const GemmPlan& a = arms[arm];
          bandit.Update(arm, inject(inject_ctx, gid, arm, a.cfg, a.splits,
                                    static_cast<uint64_t>(a.n_split)));
        }
        const GemmPlan best = arms[bandit.Best(kAutotuneTileTolerance)];
        for (size_t i : idxs) plans_[program][i] = best;
        continue;
      }
      // A Scale that PlanScaleFolds would fold into this GEMM's stream loads
      // is launched only when the GEMM's plan cannot take the fold: an arm
      // that takes it is timed as the folded launch (reading x with the
      // factor applied), any other as its own launch plus the Scale's.
      const long fold_at = FoldScaleOf(program, first);
      GemmDesc fd = d;
      std::vector<char> folds(arms.size(), 0);
      if (fold_at >= 0) {
        const UpdateInstruction& sc = prog[static_cast<size_t>(fold_at)];
        int64_t elems = 0;
        const void* stream = SkinnyStream(d, &elems);
        if (fd.A == stream) fd.A = RP(sc.in[0]);
        else fd.B = RP(sc.in[0]);
        fd.scale_stream = true;
        fd.stream_scale = Bits(sc.in[2]);
        for (size_t a = 0; a < arms.size(); ++a) folds[a] = GemmScaledOk(fd, arms[a]) ? 1 : 0;
      }
      size_t need = 0;
      for (const auto& a : arms) need = std::max(need, a.ws_bytes);
      if (need > ws_bytes_) {
        if (Status s = HipOk(hipStreamSynchronize(stream_), "tune sync"); !s) { result = s; break; }
        if (ws_) (void)LockedFree(ws_);
        ws_ = nullptr;
        ws_bytes_ = 0;
        if (Status s = HipOk(LockedMalloc(&ws_, Round64(need)), "workspace"); !s) { result = s; break; }
        ws_bytes_ = Round64(need);
        for (int p = 0; p < 3; ++p) DropGraph(p);
      }
      const Ctx c = MakeCtx();
      const double flops = 2.0 * static_cast<double>(d.M) * d.N * d.K;
      auto launch = [&](size_t a) -> Status {
        if (folds[a]) return LaunchGemm(fd, arms[a], c);
        if (fold_at >= 0)
          if (Status s = Dispatch(program, static_cast<size_t>(fold_at), c); !s) return s;
        return LaunchGemm(d, arms[a], c);
      };
      // One warm-up launch per arm, timed: a pull of an arm then times
      // enough back-to-back launches to fill ~0.2 ms (at most 16), so that
      // the short GEMMs (the K = rank up-projections, ~20 us) are ranked by
      // more than one launch's event-timing noise.
      std::vector<int> reps(arms.size(), 1);
      for (size_t a = 0; a < arms.size() && result; ++a) {
        (void)hipEventRecord(t0, stream_);
        if (Status s = launch(a); !s) { result = s; break; }
        (void)hipEventRecord(t1, stream_);
        (void)hipEventSynchronize(t1);
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, t0, t1);
        if (ms > 0.0f) reps[a] = std::clamp(static_cast<int>(0.2f / ms), 1, 16);
      }
      if (!result) break;
      // Rewards are the fraction of fp32 MFMA peak (UCB1's [0, 1] scale);
      // every arm is pulled at least twice.
      Ucb1 bandit(arms.size());
      const int trials = std::max<int>(budget, 2 * static_cast<int>(arms.size()));
      for (int t = 0; t < trials; ++t) {
        const size_t arm = bandit.Select();
        (void)hipEventRecord(t0, stream_);
        for (int r = 0; r < reps[arm] && result; ++r)
          if (Status s = launch(arm); !s) result = s;
        if (!result) break;
        (void)hipEventRecord(t1, stream_);
        (void)hipEventSynchronize(t1);
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, t0, t1);
        ms /= static_cast<float>(reps[arm]);
        bandit.Update(arm, ms > 0.0f ? flops / (ms * 1e-3) / kPeakFp32MfmaFlops : 0.0);
      }
      if (!result) break;
      const GemmPlan best = arms[bandit.Best(kAutotuneTileTolerance)];
      for (size_t i : idxs) plans_[program][i] = best;
    }
    if (result && !inject) result = TuneTileGroups(program, budget, t0, t1);
    (void)hipEventDestroy(t0);
    (void)hipEventDestroy(t1);
    if (!result) return result;
    for (int p = 0; p < 3; ++p) DropGraph(p);
    return HipOk(hipStreamSynchronize(stream_), "autotune");
  }

  // Per-instruction durations (ms, mean over reps) from an eager pass with a
  // HIP event after every launch. A fused AdamW run is timed as the one
  // launch the graph makes, its time split over the run's instructions by
  // element count.
  Status Profile(int program, int reps, float* ms_out, size_t count) {
    loss_posted_ = false;  // runs instructions outside Run()
    if (program < 0 || program > 2) return Status::Fail(kUnitEngine, "unknown program id");
    const size_t n = plan_.program[program].size();
    if (count < n) return Status::Fail(kUnitEngine, "profile output too small");
    if (Status s = EnsureWorkspace(program); !s) return s;
    if (use_graph_ && !built_[program])
      if (Status s = Build(program); !s) return s;
    const auto& prog = plan_.program[program];
    std::vector<hipEvent_t> ev(n + 1);
    for (auto& e : ev)
      if (Status s = HipOk(hipEventCreate(&e), "event"); !s) return s;
    std::vector<double> acc(n, 0.0);
    const Ctx c = MakeCtx();
    const auto& runs = use_graph_ ? fused_runs_[program] : std::vector<FusedRun>{};
    const auto& chains = use_graph_ ? chains_[program] : std::vector<ChainRun>{};
    Status result = Status::Ok();
    for (int r = 0; r < reps && result; ++r) {
      (void)hipEventRecord(ev[0], stream_);
      size_t fr = 0, fq = 0;
      for (size_t i = 0; i < n;) {
        if (const int tg = use_graph_ ? TileGroupAt(program, i, 0, n) : -1; tg >= 0) {
          if (Status s = LaunchTileGroup(program, tg, c); !s) {
            result = s;
            break;
          }
          i = tgroups_[program][tg].end;
          while (fq < chains.size() && chains[fq].first < i) ++fq;
          while (fr < runs.size() && runs[fr].first < i) ++fr;
          (void)hipEventRecord(ev[i], stream_);
          continue;
        }
        if (fq < chains.size() && chains[fq].first == i) {
          const ChainRun& run = chains[fq++];
          if (run.kind == ChainKind::kScaleFold) {  // timed launch by launch
            (void)hipEventRecord(ev[i + 1], stream_);  // the Scale launches nothing
            for (size_t k = i + 1; k < i + run.count && result;) {
              const size_t step = FoldStep(program, run, k, c, &result);
              // A dual pair's one launch is timed on its first instruction.
              for (size_t e = 0; e < step; ++e) (void)hipEventRecord(ev[k + 1 + e], stream_);
              k += step;
            }
            if (!result) break;
            i += run.count;
            continue;
          }
          if (Status s = LaunchChain(program, run, c, 0, n); !s) {
            result = s;
            break;
          }
          i += run.count;
          (void)hipEventRecord(ev[i], stream_);
          continue;
        }
        if (fr < runs.size() && runs[fr].first == i) {
          if (Status s = AdamWMulti(fused_segs_[program] + runs[fr].seg_offset, runs[fr].count,
                                    runs[fr].blocks, c);
              !s) {
            result = s;
            break;
          }
          i += runs[fr++].count;
          (void)hipEventRecord(ev[i], stream_);
          continue;
        }
        const int cg = use_graph_ ? ColsumGroupAt(program, i, 0, n) : -1;
        if (Status s = cg >= 0 ? ColsumGroupStep(program, cg, i, c) : Dispatch(program, i, c); !s) {
          result = s;
          break;
        }
        (void)hipEventRecord(ev[++i], stream_);
      }
      if (!result) break;
      if (Status s = HipOk(hipEventSynchronize(ev[n]), "profile sync"); !s) { result = s; break; }
      fr = 0;
      fq = 0;
      for (size_t i = 0; i < n;) {
        if (const int tg = use_graph_ ? TileGroupAt(program, i, 0, n) : -1; tg >= 0) {
          // One launch: its time goes to the group's first instruction.
          const size_t e = tgroups_[program][tg].end;
          float ms = 0.0f;
          (void)hipEventElapsedTime(&ms, ev[i], ev[e]);
          acc[i] += ms;
          i = e;
          while (fq < chains.size() && chains[fq].first < i) ++fq;
          while (fr < runs.size() && runs[fr].first < i) ++fr;
          continue;
        }
        if (fq < chains.size() && chains[fq].first == i) {
          const ChainRun& run = chains[fq++];
          if (run.kind == ChainKind::kScaleFold) {
            for (size_t k = i; k < i + run.count; ++k) {
              float ms = 0.0f;
              (void)hipEventElapsedTime(&ms, ev[k], ev[k + 1]);
              acc[k] += ms;
            }
            i += run.count;
            continue;
          }
          float ms = 0.0f;
          (void)hipEventElapsedTime(&ms, ev[i], ev[i + run.count]);
          // One launch: its time goes to the chain's first instruction (the
          // others report "in ..." from GemmChoice).
          acc[i] += ms;
          i += run.count;
          continue;
        }
        if (fr < runs.size() && runs[fr].first == i) {
          const FusedRun& run = runs[fr++];
          float ms = 0.0f;
          (void)hipEventElapsedTime(&ms, ev[i], ev[i + run.count]);
          double elems = 0.0;
          for (size_t k = i; k < i + run.count; ++k) elems += static_cast<double>(prog[k].out[0]);
          for (size_t k = i; k < i + run.count; ++k)
            acc[k] += elems > 0.0 ? ms * static_cast<double>(prog[k].out[0]) / elems : 0.0;
          i += run.count;
          continue;
        }
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, ev[i], ev[i + 1]);
        acc[i] += ms;
        ++i;
      }
    }
    for (auto& e : ev) (void)hipEventDestroy(e);
    if (!result) return result;
    for (size_t i = 0; i < n; ++i) ms_out[i] = static_cast<float>(acc[i] / std::max(reps, 1));
    return Status::Ok();
  }

  Status TimeInstruction(int program, size_t idx, int reps, float* avg_ms) {
    loss_posted_ = false;  // runs instructions outside Run()
    if (program < 0 || program > 2 || idx >= plan_.program[program].size())
      return Status::Fail(kUnitEngine, "instruction index out of range");
    if (Status s = EnsureWorkspace(program); !s) return s;
    const Ctx c = MakeCtx();
    hipEvent_t t0, t1;
    if (Status s = HipOk(hipEventCreate(&t0), "event"); !s) return s;
    if (Status s = HipOk(hipEventCreate(&t1), "event"); !s) return s;
    Status result = Dispatch(program, idx, c);  // warm-up
    if (result) {
      (void)hipEventRecord(t0, stream_);
      for (int r = 0; r < reps && result; ++r) result = Dispatch(program, idx, c);
      (void)hipEventRecord(t1, stream_);
      if (result) result = HipOk(hipEventSynchronize(t1), "time sync");
    }
    float ms = 0.0f;
    if (result) (void)hipEventElapsedTime(&ms, t0, t1);
    (void)hipEventDestroy(t0);
    (void)hipEventDestroy(t1);
    if (!result) return result;
    *avg_ms = ms / static_cast<float>(std::max(reps, 1));
    return Status::Ok();
  }

  static double GemmFlops(const GemmDesc& d) {
    return 2.0 * static_cast<double>(d.batch) * d.M * d.N * d.K;
  }
  // A, B and C once each, at 4 B per f32 and 1 B per int8 weight.
  static double GemmOperandBytes(const GemmDesc& d) {
    return static_cast<double>(d.batch) *
           (4.0 * d.M * d.K + (d.b_int8 ? 1.0 : 4.0) * d.K * d.N + 4.0 * d.M * d.N);
  }

  // Algorithmic work (FLOPs, compulsory HBM bytes) of what instruction idx's
  // row carries in Profile()'s breakdown, where the fused graph's launch
  // differs from the instruction alone; false where the instruction's own
  // work applies. Bytes count each operand of the launch once:
  //  - colsum group, last member (the group's one launch): the shared large
  //    operand once, every member's small operand and output; the members'
  //    FLOPs. An earlier member copies its small operand: read + write of
  //    that copy, no FLOPs.
  //  - dual pass (its first instruction): both GEMMs' FLOPs, their operands
  //    with the shared stream read once.
  //  - LoRA run (its base GEMM): the base GEMM, the up-projection in its
  //    epilogue (t and B read, y/u/s in registers, one store of the sum) and
  //    the down-projection rowdots this run launches (its own, or its rowdot
  //    group's; the layer input they share is read once).
  //  - dense chain (the GEMM): A, B, the AddEW's addend and the stores made.
  bool LaunchWork(int program, size_t idx, double* flops, double* bytes) const {
    const auto& prog = plan_.program[program];
    if (idx >= prog.size()) return false;
    if (idx < tgroup_of_[program].size() && tgroup_of_[program][idx] >= 0) {
      const TileGroup& g = tgroups_[program][tgroup_of_[program][idx]];
      if (idx != g.first) return false;  // "in tile group": no launch of its own
      // The members' launches (their rowdots included), summed.
      double f = 0.0, b = 0.0;
      for (const TileUnit& u : g.units) {
        double uf = 0.0, ub = 0.0;
        if (!UnitWork(program, u.first, &uf, &ub)) {
          uf = GemmFlops(u.d);
          ub = GemmOperandBytes(u.d);
        }
        f += uf;
        b += ub;
      }
      *flops = f;
      *bytes = b;
      return true;
    }
    return UnitWork(program, idx, flops, bytes);
  }

  // A launch's work outside tile groups (LaunchWork).
  bool UnitWork(int program, size_t idx, double* flops, double* bytes) const {
    const auto& prog = plan_.program[program];
    if (idx < cs_group_of_[program].size() && cs_group_of_[program][idx] >= 0) {
      const ColsumGroup& g = cs_groups_[program][cs_group_of_[program][idx]];
      if (idx != g.members.back()) {
        for (size_t j = 0; j + 1 < g.members.size(); ++j)
          if (g.members[j] == idx) {
            *flops = 0.0;
            *bytes = 8.0 * static_cast<double>(g.priv_floats[j]);
            return true;
          }
        return false;
      }
      const GemmDesc d0 = DescOf(prog[g.members[0]]);
      const bool big_a = ColsumBigIsA(d0);
      double f = 0.0, b = big_a ? 4.0 * d0.K * d0.M : 4.0 * d0.K * d0.N;
      for (size_t m : g.members) {
        const GemmDesc d = DescOf(prog[m]);
        f += GemmFlops(d);
        b += (big_a ? 4.0 * d.K * d.N : 4.0 * d.K * d.M) + 4.0 * d.M * d.N;
      }
      *flops = f;
      *bytes = b;
      return true;
    }
    const ChainRun* run = ChainAt(program, idx);
    if (!run) return false;
    const bool dual_here =
        duals_[program][idx] == static_cast<int64_t>(idx + 1) &&
        ((run->kind == ChainKind::kDual && idx == run->first) ||
         (run->kind == ChainKind::kScaleFold && idx > run->first && idx + 1 < run->first + run->count));
    if (dual_here) {
      const GemmDesc a = DescOf(prog[idx]), b = DescOf(prog[idx + 1]);
      const GemmDesc& cs = SkinnyKindOf(a) == SkinnyKind::kRowDot ? b : a;
      int64_t elems = 0;
      (void)SkinnyStream(cs, &elems);
      *flops = GemmFlops(a) + GemmFlops(b);
      *bytes = GemmOperandBytes(a) + GemmOperandBytes(b) - 4.0 * static_cast<double>(elems);
      return true;
    }
    if (idx != run->first) return false;
    if (run->kind == ChainKind::kDense && run->d.post_bias) {
      const GemmDesc& d = run->d;
      const double mn = 4.0 * static_cast<double>(d.M) * static_cast<double>(d.N);
      *flops = GemmFlops(d);
      *bytes = 4.0 * d.M * d.K + 4.0 * d.K * d.N + mn /* addend */ + (d.write_c ? mn : 0.0) +
               (d.write_out ? mn : 0.0) + (d.post_h ? mn : 0.0) + (d.post_g ? mn : 0.0) +
               4.0 * static_cast<double>(d.N);
      return true;
    }
    if (run->kind == ChainKind::kLoraBase) {
      const GemmDesc g0 = DescOf(prog[idx]), up = DescOf(prog[idx + 2]);
      double f = GemmFlops(g0) + GemmFlops(up);
      double b = 4.0 * g0.M * g0.K + (g0.b_int8 ? 1.0 : 4.0) * g0.K * g0.N + 4.0 * g0.M * g0.N +
                 4.0 * up.M * up.K + 4.0 * up.K * up.N;
      std::vector<size_t> rowdots;
      if (run->rd_mode == 1) rowdots = run->grp_rowdots;
      else if (run->rd_mode == 0) rowdots.push_back(idx + 1);
      for (size_t k : rowdots) {
        const GemmDesc r = DescOf(prog[k]);
        f += GemmFlops(r);
        b += 4.0 * r.K * r.N + 4.0 * r.M * r.N + (r.A == g0.A ? 0.0 : 4.0 * r.M * r.K);
      }
      *flops = f;
      *bytes = b;
      return true;
    }
    if (run->kind == ChainKind::kXentPass) {
      const UpdateInstruction& g = prog[idx];
      const double mat = 4.0 * static_cast<double>(g.out[0]) * static_cast<double>(g.out[1]);
      // logits read, dl (and P) written; labels, per-row terms, loss, seed
      *flops = 0.0;
      *bytes = mat * (run->store_p ? 3.0 : 2.0) + 16.0 * static_cast<double>(g.out[0]) + 8.0;
      return true;
    }
    if (run->kind == ChainKind::kRopePair) {
      const UpdateInstruction& g = prog[idx];
      *flops = 0.0;
      *bytes = 2.0 * 8.0 * static_cast<double>(Hi(g.out[0]) * Lo(g.out[0]) * Hi(g.out[1]) * Lo(g.out[1]));
      return true;
    }
    if (run->kind == ChainKind::kAddRow) {
      const UpdateInstruction& g = prog[idx + 1];
      const bool ln = static_cast<Op>(g.opcode) == Op::kLayerNormFwd;
      const double rows = static_cast<double>(Hi(g.out[0])), cols = static_cast<double>(Lo(g.out[0]));
      // a and b read, y (and the sum) written; gamma (beta); the row stats.
      *flops = 0.0;
      *bytes = 4.0 * rows * cols * (run->pa.store_sum ? 4.0 : 3.0) + (ln ? 8.0 : 4.0) * cols +
               (ln ? 8.0 : 4.0) * rows;
      return true;
    }
    if (run->kind == ChainKind::kRowAdd) {
      const UpdateInstruction& g = prog[idx];
      const bool ln = static_cast<Op>(g.opcode) == Op::kLayerNormBwd;
      const uint64_t dims = ln ? g.out[2] : g.out[1];
      const double rows = static_cast<double>(Hi(dims)), cols = static_cast<double>(Lo(dims));
      // dy, x and the addend read, out (and dx) written; gamma; the row stats.
      *flops = 0.0;
      *bytes = 4.0 * rows * cols * (run->ra.store_dx ? 5.0 : 4.0) + 4.0 * cols +
               (ln ? 8.0 : 4.0) * rows;
      return true;
    }
    if (run->kind == ChainKind::kDense) {
      const GemmDesc& d = run->d;
      const double mn = 4.0 * static_cast<double>(d.batch) * d.M * d.N;
      *flops = GemmFlops(d);
      *bytes = GemmOperandBytes(d) - (d.write_c ? 0.0 : mn) + (d.addend ? mn : 0.0) +
               (d.out ? mn : 0.0);
      return true;
    }
    return false;
  }

  std::string GemmChoice(int program, size_t idx) const {
    const auto op = static_cast<Op>(plan_.program[program][idx].opcode);
    const uint8_t tf = tails_[program][idx];
    const char* no_tail = (tf & kAttnStoreTail) ? "" : "no zero tail";
    if (op == Op::kSoftmaxRowsBwd)
      return causal_rows_[program][idx]
                 ? "causal S=" + std::to_string(causal_rows_[program][idx]) +
                       (*no_tail ? std::string(", ") + no_tail : std::string())
                 : std::string();
    if (op == Op::kAttnFwd) return tf == 0 ? "P unused" : no_tail;
    if (op == Op::kAttnDP) return no_tail;
    if (idx < tgroup_of_[program].size() && tgroup_of_[program][idx] >= 0) {
      const TileGroup& g = tgroups_[program][tgroup_of_[program][idx]];
      for (const TileUnit& u : g.units)
        if (u.first == idx)
          return idx == g.first ? UnitChoice(program, idx) + ", tile group of " +
                                      std::to_string(g.units.size()) + " (launched first)"
                                : std::string("in tile group");
    }
    return UnitChoice(program, idx);
  }

  // The launch choice of idx outside tile groups (GemmChoice).
  std::string UnitChoice(int program, size_t idx) const {
    const ChainRun* run = ChainAt(program, idx);
    if (run && run->kind == ChainKind::kScaleFold) {
      if (idx == run->first) return "in the next GEMMs' loads";
      const int64_t pair = duals_[program][idx];
      if (pair >= 0 && pair >= static_cast<int64_t>(run->first) &&
          pair < static_cast<int64_t>(run->first + run->count))
        return pair > static_cast<int64_t>(idx) ? "skinny/dual dt+dB scaled loads" : "in the dual pass";
      const GemmPlan& gp = plans_[program][idx];
      if (gp.cfg != GemmSkinnyConfig())
        return std::string(GemmConfigName(gp.cfg)) + " splits=" + std::to_string(gp.splits) +
               " scaled loads";
      return std::string(SkinnyKindName(SkinnyKindOf(DescOf(plan_.program[program][idx])))) +
             " scaled loads";
    }
    if (run && run->kind == ChainKind::kDual)
      return idx == run->first ? "skinny/dual dt+dB" : "in the dual pass";
    if (run && idx != run->first) {
      switch (run->kind) {
        case ChainKind::kDense: return "in GEMM epilogue";
        case ChainKind::kLoraBase:
          if (idx != run->first + 1) return "in LoRA epilogue";
          if (run->rd_mode == 1)
            return "in LoRA run: rowdot group of " + std::to_string(run->grp_rowdots.size()) +
                   " (launched first)";
          if (run->rd_mode == -1) return "in LoRA run: in an earlier rowdot group";
          return "in LoRA run (launched first)";
        case ChainKind::kPointwise: return "in pointwise run";
        case ChainKind::kRowAdd: return "in row epilogue";
        case ChainKind::kAddRow: return "in row prologue";
        case ChainKind::kRopePair: return "in rope pair";
        case ChainKind::kXentPass: return "in loss pass";
        default: return "in chain";
      }
    }
    if (run && run->kind == ChainKind::kPointwise) {
      // As a whole program launches it (the bytes its HBM traffic counts).
      const std::string head = "pointwise run of " + std::to_string(run->count);
      if (run->recompute_from != ChainRun::kNoIndex)
        return head + " (SiLU recomputed) B=" + std::to_string(run->bytes_alt);
      if (run->cond_step >= 0)
        return head + " (SiLU output not stored) B=" + std::to_string(run->bytes_alt);
      return head + " B=" + std::to_string(run->bytes);
    }
    if (run && run->kind == ChainKind::kRowAdd)
      return run->ra.store_dx ? "with the next AddEW (dx stored)" : "with the next AddEW";
    if (run && run->kind == ChainKind::kAddRow)
      return run->pa.store_sum ? "with the next norm (sum stored)" : "with the next norm";
    if (run && run->kind == ChainKind::kRopePair) return "rope pair";
    if (run && run->kind == ChainKind::kXentPass)
      return run->store_p ? "one pass with the backward" : "one pass with the backward, P not stored";
    if (idx < cs_group_of_[program].size() && cs_group_of_[program][idx] >= 0) {
      const ColsumGroup& g = cs_groups_[program][cs_group_of_[program][idx]];
      return idx == g.members.back()
                 ? "skinny/colsum group of " + std::to_string(g.members.size()) + " (launched last)"
                 : std::string("copies its operand for a later colsum group");
    }
    if (!IsGemmOp(plan_.program[program][idx].opcode)) return std::string();
    const GemmPlan& p = plans_[program][idx];
    if (p.cfg == GemmSkinnyConfig()) {
      std::string k = SkinnyKindName(SkinnyKindOf(DescOf(plan_.program[program][idx])));
      if (run) k += " chain of " + std::to_string(run->count) + " B=" + std::to_string(run->bytes);
      return k;
    }
    const std::string tiles =
        p.n_split > 0 ? std::string(GemmConfigName(p.cfg)) + "|" + GemmConfigName(p.tail_cfg) + "@" +
                            std::to_string(p.n_split)
                      : std::string(GemmConfigName(p.cfg));
    if (run && run->kind == ChainKind::kLoraBase)
      return tiles + " splits=" + std::to_string(p.splits) + " +LoRA" +
             (run->count == 5 ? " +Scale" : "") + " +AddEW";
    if (run && run->d.post_bias) {  // the bytes as the launch moves them (UnitWork)
      static const char* kAct[] = {"", " +ReLU", " +GELU", " +SiLU"};
      return tiles + " splits=" + std::to_string(p.splits) +
             (run->d.out_scaled ? " +Scale+AddEW" : " +AddEW") + " +Bias" + kAct[run->d.post_act & 3];
    }
    return tiles + " splits=" + std::to_string(p.splits) +
           (run ? (run->count == 3 ? " +Scale+AddEW" : " +AddEW") : "");
  }

  void Release() {
    for (int p = 0; p < 3; ++p) DropGraph(p);
    if (stream_) (void)hipStreamSynchronize(stream_);
    if (arena_) (void)LockedFree(arena_);
    if (rodata_) (void)LockedFree(rodata_);
    if (wcopy_buf_) (void)LockedFree(wcopy_buf_);
    wcopy_buf_ = nullptr;
    wcopies_.clear();
    if (ropetab_buf_) (void)LockedFree(ropetab_buf_);
    ropetab_buf_ = nullptr;
    ropetabs_.clear();
    if (ws_) (void)LockedFree(ws_);
    if (d_scalars_) (void)LockedFree(d_scalars_);
    for (int p = 0; p < 3; ++p) {
      for (hipEvent_t ev : mark_ev_[p]) (void)hipEventDestroy(ev);
      mark_ev_[p].clear();
      marked_[p].clear();
      if (mark_stamps_[p]) (void)LockedFree(mark_stamps_[p]);
      mark_stamps_[p] = nullptr;
      if (fused_segs_[p]) (void)LockedFree(fused_segs_[p]);
      fused_segs_[p] = nullptr;
      fused_runs_[p].clear();
      if (cs_priv_[p]) (void)LockedFree(cs_priv_[p]);
      cs_priv_[p] = nullptr;
      cs_groups_[p].clear();
      cs_group_of_[p].clear();
    }
    if (d_argmax_) (void)LockedFree(d_argmax_);
    d_argmax_ = nullptr;
    argmax_cap_ = 0;
    if (h_count_) (void)LockedHostFree(h_count_);
    h_count_ = nullptr;
    if (h_loss_) (void)LockedHostFree(h_loss_);
    if (h_stamps_) (void)LockedHostFree(h_stamps_);
    h_stamps_ = nullptr;
    h_stamps_cap_ = 0;
    if (stream_) (void)hipStreamDestroy(stream_);
    arena_ = rodata_ = nullptr;
    ws_ = nullptr;
    d_scalars_ = nullptr;
    h_loss_ = nullptr;
    stream_ = nullptr;
  }

  DecodedPlan plan_;
  std::vector<GemmPlan> plans_[3];
  std::vector<int64_t> duals_[3];         // per instruction: its dual partner, or -1 (PlanDuals)
  int device_ = 0;
  hipStream_t stream_ = nullptr;
  uint8_t* arena_ = nullptr;
  size_t arena_bytes_ = 0;
  uint8_t* rodata_ = nullptr;
  uint8_t* wcopy_buf_ = nullptr;  // transposed frozen weights (MakeWeightCopies)
  std::vector<WeightCopy> wcopies_;
  uint8_t* ropetab_buf_ = nullptr;  // RoPE angle tables (MakeRopeTables)
  std::vector<RopeTab> ropetabs_;
  size_t rodata_bytes_ = 0;
  void* ws_ = nullptr;
  size_t ws_bytes_ = 0;
  StepScalars* d_scalars_ = nullptr;
  AdamWSegment* fused_segs_[3] = {nullptr, nullptr, nullptr};
  std::vector<size_t> marked_[3];
  std::vector<hipEvent_t> mark_ev_[3];
  uint8_t* d_argmax_ = nullptr;
  size_t argmax_cap_ = 0;
  uint64_t* h_count_ = nullptr;
  std::vector<FusedRun> fused_runs_[3];
  std::vector<ChainRun> chains_[3];
  std::vector<ColsumGroup> cs_groups_[3];  // PlanColsumGroups
  std::vector<TileGroup> tgroups_[3];     // PlanTileGroups
  std::vector<int> tgroup_of_[3];         // instruction -> its tile group, or -1
  std::vector<int> cs_group_of_[3];        // per instruction: its colsum group, or -1
  void* cs_priv_[3] = {nullptr, nullptr, nullptr};  // the groups' operand copies
  std::vector<Ranges> depends_[3];  // per instruction: DependRangesOf
  std::vector<Ranges> writes_[3];   // per instruction: WriteRangesOf
  Ranges observed_[3];  // per program (PlanLiveness)
  std::vector<uint64_t> causal_rows_[3];  // per instruction: S, or 0
  std::vector<uint8_t> tails_[3];         // per instruction: kAttnStore* (PlanCausalTails)
  bool loss_posted_ = false;  // the last program run wrote its loss to h_loss_
  float* h_loss_ = nullptr;
  struct Segment {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    size_t first = 0, count = 0;
    long mark = -1;  // >= 0: a marked launch, run eagerly between segments
  };
  std::vector<Segment> segs_[3];
  uint64_t* mark_stamps_[3] = {nullptr, nullptr, nullptr};  // per marked launch: start, tick sum, count
  uint64_t* h_stamps_ = nullptr;                            // pinned, for reading them back
  size_t h_stamps_cap_ = 0;
  bool stamped_[3] = {false, false, false};  // the built graph times its marks by stamps
  int wall_khz_ = 0;                         // the device wall clock's rate
  bool built_[3] = {false, false, false};
  bool use_graph_ = true;
  uint64_t step_ = 0;
  std::string error_;
};

// ---- standalone kernel context (per device, library-owned scratch) --------
namespace {

struct Standalone {
  std::mutex mu;
  std::map<int, std::pair<void*, size_t>> ws;       // device -> workspace
  std::map<int, StepScalars*> scalars;              // device -> scalar block
};
Standalone& Shared() {
  static Standalone s;
  return s;
}
thread_local std::string g_kernel_error;

int Report(const Status& s) {
  if (s.ok) return SEEML_HIP_OK;
  g_kernel_error = s.error;
  return SEEML_HIP_ERROR;
}
}  // namespace

// The standalone entry points' status: the message is kept for
// seeml_hip_kernel_error() on this thread.
int ReportStandalone(const Status& s) { return Report(s); }

std::recursive_mutex& DeviceMemMutex() {
  static std::recursive_mutex m;
  return m;
}

namespace {

Status StandaloneCtx(void* stream, size_t ws_need, Ctx* out) {
  int dev = 0;
  if (Status s = HipOk(hipGetDevice(&dev), "hipGetDevice"); !s) return s;
  Standalone& st = Shared();
  std::lock_guard<std::mutex> lock(st.mu);
  auto& w = st.ws[dev];
  if (ws_need > w.second) {
    if (w.first) {
      std::lock_guard<std::recursive_mutex> dev_lock(DeviceMemMutex());
      (void)hipDeviceSynchronize();
      (void)LockedFree(w.first);
    }
    w = {nullptr, 0};
    if (Status s = HipOk(LockedMalloc(&w.first, Round64(ws_need)), "standalone workspace"); !s)
      return s;
    w.second = Round64(ws_need);
  }
  auto& sc = st.scalars[dev];
  if (!sc)
    if (Status s = HipOk(LockedMalloc(&sc, sizeof(StepScalars)), "standalone scalars"); !s) return s;
  out->stream = static_cast<hipStream_t>(stream);
  out->ws = w.first;
  out->ws_bytes = w.second;
  out->scalars = sc;
  return Status::Ok();
}

void CopyError(const std::string& msg, char* err, uint64_t cap) {
  if (!err || cap == 0) return;
  const size_t n = std::min<size_t>(msg.size(), cap - 1);
  std::memcpy(err, msg.data(), n);
  err[n] = '\0';
}

}  // namespace
}  // namespace seeml_hip

using seeml_hip::Ctx;
using seeml_hip::Engine;
using seeml_hip::Status;

struct seeml_hip_engine {
  Engine impl;
};

namespace {
int Ret(seeml_hip_engine* e, const Status& s) {
  if (s.ok) return SEEML_HIP_OK;
  e->impl.error_ = s.error;
  return SEEML_HIP_ERROR;
}
}  // namespace

extern "C" {

int seeml_hip_verify_plan(const uint8_t* plan, uint64_t plan_size, char* err, uint64_t err_cap) {
  seeml_hip::DecodedPlan d;
  const Status s = seeml_hip::DecodeAndVerifyPlan(plan, plan_size, &d);
  if (!s) seeml_hip::CopyError(s.error, err, err_cap);
  return s.ok ? SEEML_HIP_OK : SEEML_HIP_ERROR;
}

int seeml_hip_validate_instruction(const void* instr64, uint64_t arena_size, uint64_t rodata_size,
                                   uint32_t plan_version, char* err, uint64_t err_cap) {
  seeml_hip::UpdateInstruction ins;
  std::memcpy(&ins, instr64, sizeof ins);
  const Status s = seeml_hip::ValidateInstruction(ins, arena_size, rodata_size, plan_version);
  if (!s) seeml_hip::CopyError(s.error, err, err_cap);
  return s.ok ? SEEML_HIP_OK : SEEML_HIP_ERROR;
}

uint64_t seeml_hip_plan_self_hash(const uint8_t* plan, uint64_t size, uint64_t hash_offset) {
  return seeml_hip::PlanSelfHash(plan, size, hash_offset);
}

uint64_t seeml_hip_content_hash64(const uint8_t* data, uint64_t size) {
  return seeml_hip::ContentHash64(data, size);
}

float seeml_hip_effective_lr(const uint8_t* header, uint64_t step) {
  seeml_hip::PlanHeader h;
  std::memcpy(&h, header, sizeof h);
  return seeml_hip::EffectiveLr(h, step);
}

int seeml_hip_open(const uint8_t* plan, uint64_t plan_size, int device, seeml_hip_engine** out,
                   char* err, uint64_t err_cap) {
  if (!out) return SEEML_HIP_ERROR;
  *out = nullptr;
  auto* e = new seeml_hip_engine();
  const Status s = e->impl.Open(plan, plan_size, device);
  if (!s) {
    seeml_hip::CopyError(s.error, err, err_cap);
    delete e;
    return SEEML_HIP_ERROR;
  }
  *out = e;
  return SEEML_HIP_OK;
}

void seeml_hip_close(seeml_hip_engine* e) { delete e; }

const char* seeml_hip_last_error(const seeml_hip_engine* e) {
  return e ? e->impl.error_.c_str() : "UpdateEngine: null engine";
}

int seeml_hip_build(seeml_hip_engine* e, int program) { return Ret(e, e->impl.Build(program)); }

int seeml_hip_set_graph_mode(seeml_hip_engine* e, int use_graph) {
  e->impl.use_graph_ = use_graph != 0;
  for (int p = 0; p < 3; ++p) e->impl.DropGraph(p);
  return SEEML_HIP_OK;
}

int seeml_hip_stage(seeml_hip_engine* e, const void* input, uint64_t input_bytes,
                    const void* labels, uint64_t label_bytes, int on_device) {
  return Ret(e, e->impl.Stage(input, input_bytes, labels, label_bytes, on_device != 0));
}

int seeml_hip_set_step(seeml_hip_engine* e, uint64_t step) { return Ret(e, e->impl.SetStep(step)); }
uint64_t seeml_hip_get_step(const seeml_hip_engine* e) { return e->impl.step_; }

int seeml_hip_run(seeml_hip_engine* e, int program) { return Ret(e, e->impl.Run(program)); }
int seeml_hip_run_range(seeml_hip_engine* e, int program, uint64_t begin, uint64_t end) {
  return Ret(e, e->impl.RunRange(program, begin, end));
}

int seeml_hip_sync(seeml_hip_engine* e) {
  return Ret(e, seeml_hip::HipOk(hipStreamSynchronize(e->impl.stream_), "sync"));
}

int seeml_hip_loss(seeml_hip_engine* e, float* loss) { return Ret(e, e->impl.Loss(loss)); }

int seeml_hip_train_step(seeml_hip_engine* e, const void* input, uint64_t input_bytes,
                         const void* labels, uint64_t label_bytes, int on_device, float* loss) {
  return Ret(e, e->impl.TrainStep(input, input_bytes, labels, label_bytes, on_device != 0, loss));
}

int seeml_hip_run_merge(seeml_hip_engine* e) { return Ret(e, e->impl.RunMerge()); }

int seeml_hip_read(seeml_hip_engine* e, uint64_t ref, void* dst, uint64_t bytes) {
  return Ret(e, e->impl.Access(ref, dst, bytes, false));
}

int seeml_hip_write(seeml_hip_engine* e, uint64_t ref, const void* src, uint64_t bytes) {
  return Ret(e, e->impl.Access(ref, const_cast<void*>(src), bytes, true));
}

void* seeml_hip_arena_device_ptr(seeml_hip_engine* e) { return e->impl.arena_; }
void* seeml_hip_stream(seeml_hip_engine* e) { return e->impl.stream_; }
uint64_t seeml_hip_workspace_bytes(const seeml_hip_engine* e) { return e->impl.ws_bytes_; }

int seeml_hip_autotune(seeml_hip_engine* e, int budget) { return Ret(e, e->impl.Autotune(budget)); }
int seeml_hip_autotune_injected(seeml_hip_engine* e, int budget, seeml_hip_tune_reward_fn reward,
                                void* ctx) {
  if (!reward) return Ret(e, Status::Fail(seeml_hip::kUnitEngine, "autotune: no reward function"));
  return Ret(e, e->impl.Autotune(budget, reward, ctx));
}

int seeml_hip_ucb1_run(uint64_t arms, double exploration, uint64_t trials,
                       seeml_hip_arm_reward_fn reward, void* ctx, uint64_t* picks,
                       uint64_t* pulls, double* means, uint64_t* best_arm) {
  if (arms == 0 || !reward) return SEEML_HIP_ERROR;
  seeml_hip::Ucb1 bandit(arms, exploration);
  const uint64_t budget = std::max(trials, arms);
  for (uint64_t t = 0; t < budget; ++t) {
    const size_t arm = bandit.Select();
    if (picks) picks[t] = arm;
    bandit.Update(arm, reward(ctx, arm));
  }
  for (uint64_t i = 0; i < arms; ++i) {
    if (pulls) pulls[i] = bandit.pulls(i);
    if (means) means[i] = bandit.mean(i);
  }
  if (best_arm) *best_arm = bandit.Best();
  return SEEML_HIP_OK;
}

int seeml_hip_set_gemm_plan(seeml_hip_engine* e, int program, uint64_t index, int cfg, int splits) {
  return Ret(e, e->impl.SetGemmPlan(program, index, cfg, splits));
}

int seeml_hip_launch_work(seeml_hip_engine* e, int program, uint64_t index, double* flops,
                          double* bytes) {
  if (program < 0 || program > 2 || index >= e->impl.plans_[program].size() || !flops || !bytes)
    return Ret(e, Status::Fail(seeml_hip::kUnitEngine, "instruction index out of range"));
  if (!e->impl.LaunchWork(program, index, flops, bytes)) *flops = *bytes = -1.0;
  return SEEML_HIP_OK;
}

int seeml_hip_gemm_choice(seeml_hip_engine* e, int program, uint64_t index, char* buf,
                          uint64_t cap) {
  if (program < 0 || program > 2 || index >= e->impl.plans_[program].size())
    return Ret(e, Status::Fail(seeml_hip::kUnitEngine, "instruction index out of range"));
  seeml_hip::CopyError(e->impl.GemmChoice(program, index), buf, cap);
  return SEEML_HIP_OK;
}

int seeml_hip_evaluate_metrics(seeml_hip_engine* e, seeml_hip_dataset* d,
                               seeml_hip_eval_metrics* out) {
  Engine::EvalOut m;
  if (const Status s = e->impl.EvaluateMetrics(d->impl, &m); !s) return Ret(e, s);
  out->loss = m.loss;
  out->has_accuracy = m.has_accuracy ? 1 : 0;
  out->accuracy = m.accuracy;
  return SEEML_HIP_OK;
}

int seeml_hip_train(seeml_hip_engine* e, seeml_hip_dataset* d, uint64_t steps,
                    seeml_hip_dataset* validation, float* loss_curve, uint64_t curve_cap,
                    seeml_hip_train_report* out) {
  return seeml_hip_train_ex(e, d, steps, validation, loss_curve, curve_cap, nullptr, out);
}

int seeml_hip_train_ex(seeml_hip_engine* e, seeml_hip_dataset* d, uint64_t steps,
                       seeml_hip_dataset* validation, float* loss_curve, uint64_t curve_cap,
                       const seeml_hip_train_options* options, seeml_hip_train_report* out) {
  Engine::ReportOut r;
  Engine::TrainOptions opt;
  if (options) {
    opt.checkpoint_path = options->checkpoint_path ? options->checkpoint_path : "";
    opt.checkpoint_every = options->checkpoint_every;
    opt.resume = options->resume != 0;
    opt.should_stop = options->should_stop;
    opt.should_stop_ctx = options->should_stop_ctx;
  }
  if (const Status s = e->impl.Train(d->impl, steps, validation ? &validation->impl : nullptr,
                                     loss_curve, curve_cap, &r, opt);
      !s)
    return Ret(e, s);
  out->steps = r.steps;
  out->initial_avg_loss = r.initial_avg_loss;
  out->final_avg_loss = r.final_avg_loss;
  out->has_validation = r.has_validation ? 1 : 0;
  out->val_initial_loss = r.val_initial_loss;
  out->val_final_loss = r.val_final_loss;
  out->has_val_accuracy = r.has_val_accuracy ? 1 : 0;
  out->val_initial_accuracy = r.val_initial_accuracy;
  out->val_final_accuracy = r.val_final_accuracy;
  out->improved = r.improved() ? 1 : 0;
  out->stopped_early = r.stopped_early ? 1 : 0;
  return SEEML_HIP_OK;
}

int seeml_hip_save_checkpoint(seeml_hip_engine* e, const char* path) {
  return Ret(e, e->impl.SaveCheckpoint(path ? path : ""));
}
int seeml_hip_load_checkpoint(seeml_hip_engine* e, const char* path) {
  return Ret(e, e->impl.LoadCheckpoint(path ? path : ""));
}
int seeml_hip_checkpoint_write(const char* path, uint64_t plan_hash, uint64_t step,
                               const uint8_t* payload, uint64_t size, char* err, uint64_t err_cap) {
  const Status s = seeml_hip::WriteCheckpoint(path ? path : "", plan_hash, step, payload, size);
  if (!s) seeml_hip::CopyError(s.error, err, err_cap);
  return s.ok ? SEEML_HIP_OK : SEEML_HIP_ERROR;
}
int seeml_hip_checkpoint_read(const char* path, uint64_t plan_hash, uint64_t size, uint8_t* dst,
                              uint64_t* step, char* err, uint64_t err_cap) {
  const Status s = seeml_hip::ReadCheckpoint(path ? path : "", plan_hash, size, dst, step);
  if (!s) seeml_hip::CopyError(s.error, err, err_cap);
  return s.ok ? SEEML_HIP_OK : SEEML_HIP_ERROR;
}

int seeml_hip_profile_program(seeml_hip_engine* e, int program, int reps, float* ms_out,
                              uint64_t count) {
  return Ret(e, e->impl.Profile(program, reps, ms_out, count));
}

int seeml_hip_mark_timed(seeml_hip_engine* e, int program, const uint64_t* indices,
                         uint64_t count) {
  return Ret(e, e->impl.MarkTimed(program, indices, count));
}

int seeml_hip_marked_times(seeml_hip_engine* e, int program, float* ms_out, uint64_t count) {
  return Ret(e, e->impl.MarkedTimes(program, ms_out, count));
}

int seeml_hip_time_instruction(seeml_hip_engine* e, int program, uint64_t index, int reps,
                               float* avg_ms) {
  return Ret(e, e->impl.TimeInstruction(program, index, reps, avg_ms));
}

uint64_t seeml_hip_program_length(const seeml_hip_engine* e, int program) {
  return program < 0 || program > 2 ? 0 : e->impl.plan_.program[program].size();
}

// ---- standalone kernels ---------------------------------------------------

const char* seeml_hip_kernel_error(void) { return seeml_hip::g_kernel_error.c_str(); }

#define SEEML_CTX(ws_need)                                                     \
  Ctx ctx;                                                                     \
  if (Status s_ = seeml_hip::StandaloneCtx(stream, (ws_need), &ctx); !s_)      \
    return seeml_hip::Report(s_);

static int RunGemm(seeml_hip::GemmDesc d, void* stream, int cfg = -1, int splits = -1) {
  const seeml_hip::GemmPlan plan = seeml_hip::PlanGemmWith(d, cfg, splits);
  SEEML_CTX(plan.ws_bytes);
  return seeml_hip::Report(seeml_hip::LaunchGemm(d, plan, ctx));
}

int seeml_hip_gemm_nn(const float* A, const float* B, float* C, uint64_t M, uint64_t N,
                      uint64_t K, const float* bias, int act, void* stream) {
  seeml_hip::GemmDesc d = seeml_hip::GemmNNDesc(A, B, C, M, N, K);
  d.bias = bias;
  d.act = act;
  return RunGemm(d, stream);
}
int seeml_hip_gemm_nt(const float* A, const float* B, float* C, uint64_t M, uint64_t N,
                      uint64_t K, void* stream) {
  return RunGemm(seeml_hip::GemmNTDesc(A, B, C, M, N, K), stream);
}
int seeml_hip_gemm_tn(const float* A, const float* B, float* C, uint64_t M, uint64_t N,
                      uint64_t K, void* stream) {
  return RunGemm(seeml_hip::GemmTNDesc(A, B, C, M, N, K), stream);
}
int seeml_hip_gemm_acc_nn(const float* A, const float* B, float* C, uint64_t M, uint64_t N,
                          uint64_t K, float alpha, void* stream) {
  seeml_hip::GemmDesc d = seeml_hip::GemmNNDesc(A, B, C, M, N, K);
  d.alpha = alpha;
  d.accumulate = true;
  return RunGemm(d, stream);
}
int seeml_hip_gemm_nn_q8(const float* A, const int8_t* B, float* C, uint64_t M, uint64_t N,
                         uint64_t K, float scale, int act, void* stream) {
  seeml_hip::GemmDesc d = seeml_hip::GemmNNDesc(A, nullptr, C, M, N, K);
  d.B = B;
  d.b_int8 = true;
  d.alpha = scale;
  d.act = act;
  return RunGemm(d, stream);
}
int seeml_hip_gemm_nt_q8(const float* A, const int8_t* B, float* C, uint64_t M, uint64_t N,
                         uint64_t K, float scale, void* stream) {
  seeml_hip::GemmDesc d = seeml_hip::GemmNTDesc(A, nullptr, C, M, N, K);
  d.B = B;
  d.b_int8 = true;
  d.alpha = scale;
  return RunGemm(d, stream);
}
int seeml_hip_gemm_forced(int layout, const float* A, const float* B, float* C, uint64_t M,
                          uint64_t N, uint64_t K, int cfg, int splits, void* stream) {
  seeml_hip::GemmDesc d = layout == 1   ? seeml_hip::GemmNTDesc(A, B, C, M, N, K)
                          : layout == 2 ? seeml_hip::GemmTNDesc(A, B, C, M, N, K)
                                        : seeml_hip::GemmNNDesc(A, B, C, M, N, K);
  return RunGemm(d, stream, cfg, splits);
}
int seeml_hip_gemm_group(int layout, int cfg, int n, const float* const* A, const float* const* B,
                         float* const* C, const uint64_t* dims, const float* const* addend,
                         float* const* out, void* stream) {
  if (n < 2 || n > seeml_hip::kGemmGroupMax || !A || !B || !C || !dims || (layout != 0 && layout != 1) ||
      cfg < 0 || cfg >= seeml_hip::GemmConfigCount() - 1)
    return seeml_hip::Report(seeml_hip::Status::Fail(seeml_hip::kUnitEngine, "gemm group: bad arguments"));
  seeml_hip::GemmDesc ds[seeml_hip::kGemmGroupMax];
  seeml_hip::GemmPlan ps[seeml_hip::kGemmGroupMax];
  for (int j = 0; j < n; ++j) {
    const uint64_t M = dims[3 * j], N = dims[3 * j + 1], K = dims[3 * j + 2];
    ds[j] = layout == 1 ? seeml_hip::GemmNTDesc(A[j], B[j], C[j], M, N, K)
                        : seeml_hip::GemmNNDesc(A[j], B[j], C[j], M, N, K);
    if (addend && addend[j]) {
      if (!out || !out[j])
        return seeml_hip::Report(seeml_hip::Status::Fail(seeml_hip::kUnitEngine, "gemm group: addend without out"));
      ds[j].addend = addend[j];
      ds[j].out = out[j];
      ds[j].write_c = false;
    }
    ps[j] = seeml_hip::PlanGemmWith(ds[j], cfg, 1);
  }
  SEEML_CTX(0);
  return seeml_hip::Report(seeml_hip::LaunchGemmGroup(ds, ps, n, ctx));
}
int seeml_hip_gemm_skinny_dual(const float* x, uint64_t T, uint64_t D, const float* b,
                               uint64_t r_rd, float* dt, const float* t, uint64_t r_cs, float* db,
                               int which, int scaled, float scale, void* stream) {
  seeml_hip::GemmDesc rd = seeml_hip::GemmNTDesc(x, b, dt, T, r_rd, D);
  seeml_hip::GemmDesc cs = seeml_hip::GemmTNDesc(t, x, db, r_cs, D, T);
  rd.scale_stream = cs.scale_stream = scaled != 0;
  rd.stream_scale = cs.stream_scale = scale;
  if (!seeml_hip::SkinnyDualFits(rd, cs))
    return seeml_hip::Report(seeml_hip::Status::Fail(seeml_hip::kUnitEngine,
                                                     "Gemm: the pair does not fit the dual skinny pass"));
  SEEML_CTX(seeml_hip::SkinnyDualWorkspace(rd));
  return seeml_hip::Report(seeml_hip::LaunchSkinnyDual(rd, cs, which, ctx));
}
int seeml_hip_gemm_skinny_group(int kind, const float* x, uint64_t T, uint64_t D,
                                const float* const* a, uint64_t r, float* const* out, int n,
                                void* stream) {
  if (kind < 0 || kind > 1 || n < 2 || n > 4 || !a || !out)
    return seeml_hip::Report(seeml_hip::Status::Fail(seeml_hip::kUnitEngine, "skinny group: bad arguments"));
  seeml_hip::GemmDesc ds[4];
  for (int j = 0; j < n; ++j)
    ds[j] = kind == 0 ? seeml_hip::GemmNNDesc(x, a[j], out[j], T, r, D)
                      : seeml_hip::GemmTNDesc(x, a[j], out[j], D, r, T);
  if (kind == 0 ? !seeml_hip::SkinnyRowdotGroupFits(ds, n) : !seeml_hip::SkinnyColsumGroupFits(ds, n))
    return seeml_hip::Report(seeml_hip::Status::Fail(seeml_hip::kUnitEngine,
                                                     "skinny group: the GEMMs do not form a group"));
  SEEML_CTX(kind == 0 ? 0 : seeml_hip::SkinnyColsumGroupWorkspace(ds, n));
  return seeml_hip::Report(kind == 0 ? seeml_hip::LaunchSkinnyRowdotGroup(ds, n, ctx)
                                     : seeml_hip::LaunchSkinnyColsumGroup(ds, n, ctx));
}
int seeml_hip_gemm_forced_split(int layout, const float* A, const float* B, float* C, uint64_t M,
                                uint64_t N, uint64_t K, int cfg, int tail_cfg, uint64_t n_split,
                                const float* addend, float* out, void* stream) {
  // With out set and C null, C is not stored (the engine's form of a fused
  // AddEW whose product is read by nothing else).
  const bool c_dead = out && !C;
  if (c_dead) C = out;
  seeml_hip::GemmDesc d = layout == 1   ? seeml_hip::GemmNTDesc(A, B, C, M, N, K)
                          : layout == 2 ? seeml_hip::GemmTNDesc(A, B, C, M, N, K)
                                        : seeml_hip::GemmNNDesc(A, B, C, M, N, K);
  if (addend || out) {
    d.addend = addend;
    d.out = out;
    d.write_c = !c_dead;
  }
  const seeml_hip::GemmPlan plan =
      n_split > 0 ? seeml_hip::PlanGemmSplit(d, cfg, tail_cfg, static_cast<int64_t>(n_split))
                  : seeml_hip::PlanGemmWith(d, cfg, 1);
  if (n_split > 0 && plan.n_split != static_cast<int64_t>(n_split)) {
    return seeml_hip::Report(seeml_hip::Status::Fail(seeml_hip::kUnitEngine,
                                                     "Gemm: the column split does not apply to this GEMM"));
  }
  SEEML_CTX(plan.ws_bytes);
  return seeml_hip::Report(seeml_hip::LaunchGemm(d, plan, ctx));
}
int seeml_hip_gemm_forced_lora(int layout, const float* A, const float* B, float* out, uint64_t M,
                               uint64_t N, uint64_t K, int cfg, int tail_cfg, uint64_t n_split,
                               const float* t, const float* bl, uint64_t r, int scaled, float scale,
                               int y_first, void* stream) {
  seeml_hip::GemmDesc d = layout == 1 ? seeml_hip::GemmNTDesc(A, B, out, M, N, K)
                                      : seeml_hip::GemmNNDesc(A, B, out, M, N, K);
  d.out = out;
  d.write_c = false;
  d.out_scaled = scaled != 0;
  d.out_scale = scale;
  d.lora_t = t;
  d.lora_b = bl;
  d.lora_ldt = static_cast<int64_t>(r);
  d.lora_ldb = static_cast<int64_t>(N);
  d.lora_r = static_cast<int>(r);
  d.lora_y_first = y_first != 0;
  const seeml_hip::GemmPlan plan =
      n_split > 0 ? seeml_hip::PlanGemmSplit(d, cfg, tail_cfg, static_cast<int64_t>(n_split))
                  : seeml_hip::PlanGemmWith(d, cfg, 1);
  if (n_split > 0 && plan.n_split != static_cast<int64_t>(n_split))
    return seeml_hip::Report(seeml_hip::Status::Fail(seeml_hip::kUnitEngine,
                                                     "Gemm: the column split does not apply to this GEMM"));
  SEEML_CTX(plan.ws_bytes);
  return seeml_hip::Report(seeml_hip::LaunchGemm(d, plan, ctx));
}
int seeml_hip_gemm_forced_scaled(int layout, const float* A, const float* B, float* C, uint64_t M,
                                 uint64_t N, uint64_t K, int cfg, int splits, float scale,
                                 void* stream) {
  if (layout != 1 && layout != 2)
    return seeml_hip::Report(seeml_hip::Status::Fail(seeml_hip::kUnitEngine,
                                                     "Gemm: scaled loads take layout 1 (NT) or 2 (TN)"));
  seeml_hip::GemmDesc d = layout == 1 ? seeml_hip::GemmNTDesc(A, B, C, M, N, K)
                                      : seeml_hip::GemmTNDesc(A, B, C, M, N, K);
  d.scale_stream = true;
  d.stream_scale = scale;
  const seeml_hip::GemmPlan plan = seeml_hip::PlanGemmWith(d, cfg, splits);
  if (!seeml_hip::GemmScaledOk(d, plan))
    return seeml_hip::Report(seeml_hip::Status::Fail(
        seeml_hip::kUnitEngine, "Gemm: no scaled-load plan for this shape and tile config"));
  SEEML_CTX(plan.ws_bytes);
  return seeml_hip::Report(seeml_hip::LaunchGemm(d, plan, ctx));
}
int seeml_hip_gemm_config_count(void) { return seeml_hip::GemmConfigCount(); }
const char* seeml_hip_gemm_config_name(int cfg) { return seeml_hip::GemmConfigName(cfg); }

#define SEEML_SIMPLE(call) \
  SEEML_CTX(0);            \
  return seeml_hip::Report(call)

int seeml_hip_add_ew(const float* x, const float* y, float* out, uint64_t n, void* stream) {
  SEEML_SIMPLE(seeml_hip::AddEW(x, y, out, n, ctx));
}
int seeml_hip_mul_ew(const float* x, const float* y, float* out, uint64_t n, void* stream) {
  SEEML_SIMPLE(seeml_hip::MulEW(x, y, out, n, ctx));
}
int seeml_hip_add_bias(const float* x, const float* b, float* out, uint64_t rows, uint64_t cols,
                       void* stream) {
  SEEML_SIMPLE(seeml_hip::AddBias(x, b, out, rows, cols, ctx));
}
int seeml_hip_scale(const float* x, float* out, float alpha, uint64_t n, void* stream) {
  SEEML_SIMPLE(seeml_hip::Scale(x, out, alpha, n, ctx));
}
int seeml_hip_reduce_rows(const float* dy, float* db, uint64_t rows, uint64_t cols, void* stream) {
  SEEML_SIMPLE(seeml_hip::ReduceRows(dy, db, rows, cols, ctx));
}
int seeml_hip_relu_fwd(const float* x, float* out, uint64_t n, void* stream) {
  SEEML_SIMPLE(seeml_hip::ReluFwd(x, out, n, ctx));
}
int seeml_hip_relu_bwd(const float* dy, const float* x, float* dx, uint64_t n, void* stream) {
  SEEML_SIMPLE(seeml_hip::ReluBwd(dy, x, dx, n, ctx));
}
int seeml_hip_gelu_fwd(const float* x, float* out, uint64_t n, void* stream) {
  SEEML_SIMPLE(seeml_hip::GeluFwd(x, out, n, ctx));
}
int seeml_hip_gelu_bwd(const float* dy, const float* x, float* dx, uint64_t n, void* stream) {
  SEEML_SIMPLE(seeml_hip::GeluBwd(dy, x, dx, n, ctx));
}
int seeml_hip_silu_fwd(const float* x, float* out, uint64_t n, void* stream) {
  SEEML_SIMPLE(seeml_hip::SiluFwd(x, out, n, ctx));
}
int seeml_hip_silu_bwd(const float* dy, const float* x, float* dx, uint64_t n, void* stream) {
  SEEML_SIMPLE(seeml_hip::SiluBwd(dy, x, dx, n, ctx));
}
int seeml_hip_embed_fwd(const int32_t* tokens, const float* table, float* out, uint64_t rows,
                        uint64_t dim, uint64_t vocab, void* stream) {
  SEEML_SIMPLE(seeml_hip::EmbedFwd(tokens, table, out, rows, dim, vocab, ctx));
}
int seeml_hip_fill(float* dst, float value, uint64_t n, void* stream) {
  SEEML_SIMPLE(seeml_hip::Fill(dst, value, n, ctx));
}
int seeml_hip_copy(const float* src, float* dst, uint64_t n, void* stream) {
  SEEML_SIMPLE(seeml_hip::Copy(src, dst, n, ctx));
}
int seeml_hip_layer_norm_fwd(const float* x, const float* gamma, const float* beta, float* y,
                             float* mean, float* rstd, uint64_t rows, uint64_t cols, void* stream) {
  SEEML_SIMPLE(seeml_hip::LayerNormFwd(x, gamma, beta, y, mean, rstd, rows, cols, ctx));
}
int seeml_hip_layer_norm_bwd(const float* dy, const float* x, const float* gamma,
                             const float* mean, const float* rstd, float* dx, uint64_t rows,
                             uint64_t cols, void* stream) {
  SEEML_SIMPLE(seeml_hip::LayerNormBwd(dy, x, gamma, mean, rstd, dx, rows, cols, ctx));
}
int seeml_hip_rms_norm_fwd(const float* x, const float* gamma, float* y, float* rstd,
                           uint64_t rows, uint64_t cols, void* stream) {
  SEEML_SIMPLE(seeml_hip::RmsNormFwd(x, gamma, y, rstd, rows, cols, ctx));
}
int seeml_hip_rms_norm_bwd(const float* dy, const float* x, const float* gamma,
                           const float* rstd, float* dx, uint64_t rows, uint64_t cols,
                           void* stream) {
  SEEML_SIMPLE(seeml_hip::RmsNormBwd(dy, x, gamma, rstd, dx, rows, cols, ctx));
}
int seeml_hip_rope_fwd(const float* x, float* y, uint64_t B, uint64_t S, uint64_t H, uint64_t d,
                       float base, void* stream) {
  SEEML_SIMPLE(seeml_hip::RopeFwd(x, y, B, S, H, d, base, ctx));
}
int seeml_hip_rope_bwd(const float* dy, float* dx, uint64_t B, uint64_t S, uint64_t H, uint64_t d,
                       float base, void* stream) {
  SEEML_SIMPLE(seeml_hip::RopeBwd(dy, dx, B, S, H, d, base, ctx));
}
int seeml_hip_attn_fwd(const float* q, const float* k, const float* v, float* o, float* probs,
                       uint64_t B, uint64_t S, uint64_t H, uint64_t d, void* stream) {
  SEEML_SIMPLE(seeml_hip::AttnFwd(q, k, v, o, probs, B, S, H, d, ctx));
}
int seeml_hip_attn_dp(const float* dout, const float* v, float* dp, uint64_t B, uint64_t S,
                      uint64_t H, uint64_t d, void* stream) {
  SEEML_SIMPLE(seeml_hip::AttnDP(dout, v, dp, B, S, H, d, ctx));
}
int seeml_hip_attn_dv(const float* probs, const float* dout, float* dv, uint64_t B, uint64_t S,
                      uint64_t H, uint64_t d, void* stream) {
  SEEML_SIMPLE(seeml_hip::AttnDV(probs, dout, dv, B, S, H, d, ctx));
}
int seeml_hip_softmax_rows_bwd(const float* probs, const float* dp, float* ds, uint64_t rows,
                               uint64_t cols, void* stream) {
  SEEML_SIMPLE(seeml_hip::SoftmaxRowsBwd(probs, dp, ds, rows, cols, ctx));
}
int seeml_hip_attn_dq(const float* ds, const float* k, float* dq, uint64_t B, uint64_t S,
                      uint64_t H, uint64_t d, void* stream) {
  SEEML_SIMPLE(seeml_hip::AttnDQ(ds, k, dq, B, S, H, d, ctx));
}
int seeml_hip_attn_dk(const float* ds, const float* q, float* dk, uint64_t B, uint64_t S,
                      uint64_t H, uint64_t d, void* stream) {
  SEEML_SIMPLE(seeml_hip::AttnDK(ds, q, dk, B, S, H, d, ctx));
}
int seeml_hip_softmax_xent_fwd(const float* logits, const int32_t* labels, float* loss,
                               float* probs, uint64_t N, uint64_t C, void* stream) {
  SEEML_CTX(seeml_hip::SoftmaxXEntFwdWorkspace(N));
  return seeml_hip::Report(seeml_hip::SoftmaxXEntFwd(logits, labels, loss, probs, N, C, ctx));
}
int seeml_hip_softmax_xent_bwd(const float* probs, const int32_t* labels, const float* seed,
                               float* dlogits, uint64_t N, uint64_t C, void* stream) {
  SEEML_SIMPLE(seeml_hip::SoftmaxXEntBwd(probs, labels, seed, dlogits, N, C, ctx));
}
int seeml_hip_argmax_correct(const float* probs, const int32_t* labels, uint64_t rows,
                             uint64_t cols, uint64_t* correct, void* stream) {
  SEEML_CTX(8 + 4 * seeml_hip::ArgmaxPartials(rows));
  uint64_t* total = static_cast<uint64_t*>(ctx.ws);
  uint32_t* partials = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(ctx.ws) + 8);
  if (const Status s = seeml_hip::ArgmaxCorrect(probs, labels, rows, cols, partials, total, ctx); !s)
    return seeml_hip::Report(s);
  uint64_t v = 0;
  if (hipMemcpyAsync(&v, total, sizeof v, hipMemcpyDeviceToHost, ctx.stream) != hipSuccess ||
      hipStreamSynchronize(ctx.stream) != hipSuccess)
    return seeml_hip::Report(Status::Fail(seeml_hip::kUnitEngine, "argmax: count read failed"));
  *correct = v;
  return SEEML_HIP_OK;
}

int seeml_hip_mse_fwd(const float* pred, const float* target, float* loss, uint64_t n,
                      void* stream) {
  SEEML_CTX(seeml_hip::MseFwdWorkspace(n));
  return seeml_hip::Report(seeml_hip::MseFwd(pred, target, loss, n, ctx));
}
int seeml_hip_mse_bwd(const float* pred, const float* target, const float* seed, float* dpred,
                      uint64_t n, void* stream) {
  SEEML_SIMPLE(seeml_hip::MseBwd(pred, target, seed, dpred, n, ctx));
}
int seeml_hip_kl_distill_fwd(const float* s_logits, const float* t_logits, float* loss,
                             float* p_s, float* p_t, uint64_t N, uint64_t C, float T,
                             void* stream) {
  SEEML_CTX(seeml_hip::KLDistillFwdWorkspace(N));
  return seeml_hip::Report(seeml_hip::KLDistillFwd(s_logits, t_logits, loss, p_s, p_t, N, C, T, ctx));
}
int seeml_hip_kl_distill_bwd(const float* p_s, const float* p_t, const float* seed,
                             float* dlogits, uint64_t N, uint64_t C, float T, void* stream) {
  SEEML_SIMPLE(seeml_hip::KLDistillBwd(p_s, p_t, seed, dlogits, N, C, T, ctx));
}
int seeml_hip_clip_norm(float* g, uint64_t n, float max_norm, void* stream) {
  SEEML_CTX(seeml_hip::ClipNormWorkspace(n));
  return seeml_hip::Report(seeml_hip::ClipNorm(g, n, max_norm, ctx));
}

static int UploadScalars(const Ctx& ctx, const seeml_hip::StepScalars& s) {
  const Status st = seeml_hip::HipOk(
      hipMemcpyAsync(const_cast<seeml_hip::StepScalars*>(ctx.scalars), &s, sizeof s,
                     hipMemcpyHostToDevice, ctx.stream),
      "scalars upload");
  if (!st) return seeml_hip::Report(st);
  // `s` lives on this host stack frame: complete the copy before returning.
  return seeml_hip::Report(seeml_hip::HipOk(hipStreamSynchronize(ctx.stream), "scalars sync"));
}

int seeml_hip_sgd_step(float* p, const float* g, uint64_t n, float lr, float weight_decay,
                       void* stream) {
  SEEML_CTX(0);
  seeml_hip::StepScalars s{};
  s.lr = lr;
  s.weight_decay = weight_decay;
  if (int r = UploadScalars(ctx, s); r != SEEML_HIP_OK) return r;
  return seeml_hip::Report(seeml_hip::SgdStep(p, g, n, ctx));
}

int seeml_hip_adamw_step(float* p, const float* g, float* m, float* v, uint64_t n, float lr,
                         float beta1, float beta2, float eps, float weight_decay, uint64_t step,
                         void* stream) {
  SEEML_CTX(0);
  seeml_hip::PlanHeader h{};
  h.lr = lr;
  h.beta1 = beta1;
  h.beta2 = beta2;
  h.eps = eps;
  h.weight_decay = weight_decay;
  h.lr_schedule = 0;
  const seeml_hip::StepScalars s = seeml_hip::MakeStepScalars(h, step);
  if (int r = UploadScalars(ctx, s); r != SEEML_HIP_OK) return r;
  return seeml_hip::Report(seeml_hip::AdamWStep(p, g, m, v, n, ctx));
}

}  // extern "C"
