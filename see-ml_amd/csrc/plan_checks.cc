// plan_checks.cc — see plan_checks.h for the reference functions restated.
//
// The validator is table-driven here: each opcode declares its operand list
// (which ref word, how many elements, read or write, element width); one
// generic pass then applies the reference's per-operand admission rules
// (non-null, nonzero extent, element-aligned, in bounds for its address
// space, never a rodata write) and its write-alias disjointness rule.
#include "plan_checks.h"

#include <cmath>
#include <cstring>
#include <thread>

namespace seeml_hip {

// ---------------------------------------------------------------- hashes --

namespace {

constexpr uint64_t kFnvOffsetBasis = 0xcbf29ce484222325ULL;
constexpr uint64_t kFnvPrime = 0x100000001b3ULL;
constexpr size_t kHashChunk = 1u << 20;
constexpr size_t kMaxChunks = 256;

uint64_t MixWord(uint64_t state, uint64_t word) {
  for (int b = 0; b < 8; ++b) {
    state ^= (word >> (8 * b)) & 0xff;
    state *= kFnvPrime;
  }
  return state;
}

// One chunk's 8-lane striped FNV-1a digest; `zero_at` (if inside the span)
// names 8 bytes read as zero.
uint64_t StripedDigest(const uint8_t* data, size_t size, size_t zero_lo,
                       size_t zero_hi) {
  uint64_t lane[8];
  for (size_t l = 0; l < 8; ++l)
    lane[l] = kFnvOffsetBasis ^ (0x9E3779B97F4A7C15ULL * (l + 1));
  auto byte_at = [&](size_t i) -> uint8_t {
    return (i >= zero_lo && i < zero_hi) ? 0 : data[i];
  };
  size_t i = 0;
  const bool patched = zero_lo < zero_hi;
  if (!patched) {
    for (; i + 8 <= size; i += 8)
      for (size_t l = 0; l < 8; ++l) {
        lane[l] ^= data[i + l];
        lane[l] *= kFnvPrime;
      }
  } else {
    for (; i + 8 <= size; i += 8)
      for (size_t l = 0; l < 8; ++l) {
        lane[l] ^= byte_at(i + l);
        lane[l] *= kFnvPrime;
      }
  }
  for (size_t l = 0; i < size; ++i, ++l) {
    lane[l] ^= byte_at(i);
    lane[l] *= kFnvPrime;
  }
  uint64_t h = kFnvOffsetBasis;
  for (size_t l = 0; l < 8; ++l) h = MixWord(h, lane[l]);
  return MixWord(h, size);
}

uint64_t ChunkedHash(const uint8_t* data, size_t size, size_t zero_at,
                     bool has_zero) {
  // ParallelChunkGrain/Count (parallel_for.h:55-67) at grain 1 MiB.
  const size_t cap = (size + kMaxChunks - 1) / kMaxChunks;
  const size_t grain = kHashChunk < cap ? cap : kHashChunk;
  const size_t chunks = size == 0 ? 0 : (size + grain - 1) / grain;
  std::vector<uint64_t> partial(chunks ? chunks : 1, 0);
  auto run = [&](size_t c) {
    const size_t b = c * grain;
    const size_t e = size < b + grain ? size : b + grain;
    size_t zlo = 0, zhi = 0;
    if (has_zero && zero_at < e && zero_at + 8 > b) {
      zlo = zero_at > b ? zero_at - b : 0;
      zhi = (zero_at + 8 < e ? zero_at + 8 : e) - b;
    }
    partial[c] = StripedDigest(data + b, e - b, zlo, zhi);
  };
  if (chunks <= 1) {
    // A single (possibly empty) chunk, exactly as the reference special-cases.
    size_t zlo = 0, zhi = 0;
    if (has_zero && zero_at < size) {
      zlo = zero_at;
      zhi = zero_at + 8 < size ? zero_at + 8 : size;
    }
    partial[0] = StripedDigest(data, size, zlo, zhi);
  } else {
    // Chunk digests are independent; threads only change who computes them.
    const size_t workers = std::min<size_t>(16, std::max(1u, std::thread::hardware_concurrency()));
    std::vector<std::thread> pool;
    for (size_t w = 0; w < workers; ++w)
      pool.emplace_back([&, w] {
        for (size_t c = w; c < chunks; c += workers) run(c);
      });
    for (auto& t : pool) t.join();
  }
  uint64_t h = kFnvOffsetBasis;
  for (size_t c = 0; c < (chunks ? chunks : 1); ++c) h = MixWord(h, partial[c]);
  return MixWord(h, size);
}

}  // namespace

uint64_t ContentHash64(const uint8_t* data, size_t size) {
  return ChunkedHash(data, size, 0, false);
}

uint64_t PlanSelfHash(const uint8_t* plan, size_t size, size_t hash_offset) {
  return ChunkedHash(plan, size, hash_offset, true);
}

// ------------------------------------------------------------- validator --

namespace {

struct Operand {
  uint64_t ref;
  uint64_t elems;
  bool write;
  uint64_t elem_bytes;
};

// Splits a packed dim word hi<<32 | lo.
inline uint64_t Hi(uint64_t w) { return w >> 32; }
inline uint64_t Lo(uint64_t w) { return w & 0xFFFFFFFFu; }

// Attention geometry from B<<32|S and H<<32|d: T*D activations and B*H*S*S
// probabilities, overflow-checked (plan_validator.cc:169-178).
bool AttnGeometry(uint64_t bs, uint64_t hd, uint64_t* td, uint64_t* pn) {
  const uint64_t B = Hi(bs), S = Lo(bs), H = Hi(hd), d = Lo(hd);
  uint64_t t = 0, dm = 0, bhs = 0;
  if (B == 0 || S == 0 || H == 0 || d == 0) return false;
  if (!MulOk(B, S, &t) || !MulOk(H, d, &dm) || !MulOk(t, dm, td)) return false;
  if (!MulOk(t, H, &bhs) || !MulOk(bhs, S, pn)) return false;
  return true;
}

// The operand table. Returns false when the opcode's dims are malformed
// (overflow, odd RoPE width, non-rodata q8/table) — a bounds failure in the
// reference's vocabulary.
bool OperandsOf(const UpdateInstruction& ins, Operand* ops, size_t* n) {
  const uint64_t d0 = ins.out[0], d1 = ins.out[1], d2 = ins.out[2];
  size_t k = 0;
  auto add = [&](uint64_t ref, uint64_t elems, bool write, uint64_t eb = 4) {
    ops[k++] = {ref, elems, write, eb};
  };
  uint64_t a = 0, b = 0, c = 0;
  switch (static_cast<Op>(ins.opcode)) {
    case Op::kNop: break;
    case Op::kGemmNN: case Op::kGemmNT: case Op::kGemmTN: case Op::kGemmAccNN:
    case Op::kGemmNNQ8: case Op::kGemmNTQ8: {
      const bool q8 = ins.opcode == static_cast<uint16_t>(Op::kGemmNNQ8) ||
                      ins.opcode == static_cast<uint16_t>(Op::kGemmNTQ8);
      if (!MulOk(d0, d2, &a) || !MulOk(d2, d1, &b) || !MulOk(d0, d1, &c)) return false;
      if (q8 && !IsRodataRef(ins.in[1])) return false;
      add(ins.in[0], a, false);
      add(ins.in[1], b, false, q8 ? 1 : 4);
      add(ins.in[2], c, true);
      if (ins.flags & kFlagEpilogueBias) add(ins.in[3], d1, false);
      break;
    }
    case Op::kAddEW: case Op::kMulEW: case Op::kReluBwd: case Op::kGeluBwd:
    case Op::kSiluBwd:
      add(ins.in[0], d0, false); add(ins.in[1], d0, false); add(ins.in[2], d0, true);
      break;
    case Op::kAddBias:
      if (!MulOk(d0, d1, &c)) return false;
      add(ins.in[0], c, false); add(ins.in[1], d1, false); add(ins.in[2], c, true);
      break;
    case Op::kReluFwd: case Op::kGeluFwd: case Op::kSiluFwd: case Op::kScale:
    case Op::kCopy:
      add(ins.in[0], d0, false); add(ins.in[1], d0, true);
      break;
    case Op::kLayerNormFwd:
      if (!MulOk(Hi(d0), Lo(d0), &c)) return false;
      add(ins.in[0], c, false); add(ins.in[1], Lo(d0), false); add(ins.in[2], Lo(d0), false);
      add(ins.in[3], c, true); add(ins.out[1], Hi(d0), true); add(ins.out[2], Hi(d0), true);
      break;
    case Op::kLayerNormBwd:
      if (!MulOk(Hi(d2), Lo(d2), &c)) return false;
      add(ins.in[0], c, false); add(ins.in[1], c, false); add(ins.in[2], Lo(d2), false);
      add(ins.in[3], c, true); add(ins.out[0], Hi(d2), false); add(ins.out[1], Hi(d2), false);
      break;
    case Op::kClipNorm: add(ins.in[0], d0, true); break;
    case Op::kReduceRows:
      if (!MulOk(d0, d1, &c)) return false;
      add(ins.in[0], c, false); add(ins.in[1], d1, true);
      break;
    case Op::kSoftmaxXEntFwd:
      if (!MulOk(d0, d1, &c)) return false;
      add(ins.in[0], c, false); add(ins.in[1], d0, false); add(ins.in[2], 1, true);
      add(ins.in[3], c, true);
      break;
    case Op::kSoftmaxXEntBwd:
      if (!MulOk(d0, d1, &c)) return false;
      add(ins.in[0], c, false); add(ins.in[1], d0, false); add(ins.in[2], 1, false);
      add(ins.in[3], c, true);
      break;
    case Op::kMseFwd:
      add(ins.in[0], d0, false); add(ins.in[1], d0, false); add(ins.in[2], 1, true);
      break;
    case Op::kMseBwd:
      add(ins.in[0], d0, false); add(ins.in[1], d0, false); add(ins.in[2], 1, false);
      add(ins.in[3], d0, true);
      break;
    case Op::kKLDistillFwd:
      if (!MulOk(Hi(d1), Lo(d1), &c)) return false;
      add(ins.in[0], c, false); add(ins.in[1], c, false); add(ins.in[2], 1, true);
      add(ins.in[3], c, true); add(ins.out[0], c, true);
      break;
    case Op::kKLDistillBwd:
      if (!MulOk(Hi(d0), Lo(d0), &c)) return false;
      add(ins.in[0], c, false); add(ins.in[1], c, false); add(ins.in[2], 1, false);
      add(ins.in[3], c, true);
      break;
    case Op::kSgdStep: add(ins.in[0], d0, true); add(ins.in[1], d0, false); break;
    case Op::kAdamWStep:
      add(ins.in[0], d0, true); add(ins.in[1], d0, false); add(ins.in[2], d0, true);
      add(ins.in[3], d0, true);
      break;
    case Op::kFill: add(ins.in[0], d0, true); break;
    case Op::kRmsNormFwd:
      if (!MulOk(Hi(d0), Lo(d0), &c)) return false;
      add(ins.in[0], c, false); add(ins.in[1], Lo(d0), false); add(ins.in[2], c, true);
      add(ins.in[3], Hi(d0), true);
      break;
    case Op::kRmsNormBwd:
      if (!MulOk(Hi(d1), Lo(d1), &c)) return false;
      add(ins.in[0], c, false); add(ins.in[1], c, false); add(ins.in[2], Lo(d1), false);
      add(ins.in[3], c, true); add(ins.out[0], Hi(d1), false);
      break;
    case Op::kRopeFwd: case Op::kRopeBwd:
      if (!AttnGeometry(d0, d1, &a, &b)) return false;
      if (Lo(d1) % 2 != 0) return false;  // rotation pairs need an even width
      add(ins.in[0], a, false); add(ins.in[1], a, true);
      break;
    case Op::kAttnFwd:
      if (!AttnGeometry(d1, d2, &a, &b)) return false;
      add(ins.in[0], a, false); add(ins.in[1], a, false); add(ins.in[2], a, false);
      add(ins.in[3], a, true); add(ins.out[0], b, true);
      break;
    case Op::kAttnDP:
      if (!AttnGeometry(d0, d1, &a, &b)) return false;
      add(ins.in[0], a, false); add(ins.in[1], a, false); add(ins.in[2], b, true);
      break;
    case Op::kAttnDV:
      if (!AttnGeometry(d0, d1, &a, &b)) return false;
      add(ins.in[0], b, false); add(ins.in[1], a, false); add(ins.in[2], a, true);
      break;
    case Op::kSoftmaxRowsBwd:
      if (!MulOk(Hi(d0), Lo(d0), &c)) return false;
      add(ins.in[0], c, false); add(ins.in[1], c, false); add(ins.in[2], c, true);
      break;
    case Op::kAttnDQ: case Op::kAttnDK:
      if (!AttnGeometry(d0, d1, &a, &b)) return false;
      add(ins.in[0], b, false); add(ins.in[1], a, false); add(ins.in[2], a, true);
      break;
    case Op::kEmbedFwd:
      if (!MulOk(Hi(d1), Lo(d1), &a) || !MulOk(d0, Lo(d1), &b)) return false;
      if (!IsRodataRef(ins.in[1])) return false;  // the table is compiler-packed rodata
      add(ins.in[0], d0, false); add(ins.in[1], a, false); add(ins.in[2], b, true);
      break;
  }
  *n = k;
  return true;
}

}  // namespace

namespace {

bool RangesOf(const UpdateInstruction& ins, bool writes,
              std::vector<std::pair<uint64_t, uint64_t>>* ranges) {
  Operand ops[8];
  size_t n = 0;
  if (!OperandsOf(ins, ops, &n)) return false;
  for (size_t i = 0; i < n; ++i) {
    if (ops[i].write != writes || IsRodataRef(ops[i].ref)) continue;
    uint64_t bytes = 0;
    if (!MulOk(ops[i].elems, ops[i].elem_bytes, &bytes)) return false;
    ranges->emplace_back(RefOffset(ops[i].ref), bytes);
  }
  return true;
}

}  // namespace

bool WriteRangesOf(const UpdateInstruction& ins,
                   std::vector<std::pair<uint64_t, uint64_t>>* ranges) {
  return RangesOf(ins, true, ranges);
}

bool ReadRangesOf(const UpdateInstruction& ins,
                  std::vector<std::pair<uint64_t, uint64_t>>* ranges) {
  return RangesOf(ins, false, ranges);
}

bool DependRangesOf(const UpdateInstruction& ins,
                    std::vector<std::pair<uint64_t, uint64_t>>* ranges) {
  if (!RangesOf(ins, false, ranges)) return false;
  switch (static_cast<Op>(ins.opcode)) {
    case Op::kGemmAccNN: case Op::kClipNorm: case Op::kSgdStep: case Op::kAdamWStep: {
      std::vector<std::pair<uint64_t, uint64_t>> w;
      if (!RangesOf(ins, true, &w)) return false;
      ranges->insert(ranges->end(), w.begin(), w.end());
      break;
    }
    default: break;
  }
  return true;
}

Status ValidateInstruction(const UpdateInstruction& ins, uint64_t arena_size,
                           uint64_t rodata_size, uint32_t plan_version) {
  const std::string op = std::to_string(ins.opcode);
  // Flags discipline first (plan_validator.cc:17-35).
  if (plan_version < kSeeuFlagsVersion) {
    if (ins.flags != 0)
      return Status::Fail(kUnitValidator,
                          "instruction carries flags in a pre-v" +
                              std::to_string(kSeeuFlagsVersion) + " plan (opcode " + op + ")");
  } else {
    const uint16_t allowed =
        ins.opcode == static_cast<uint16_t>(Op::kGemmNN)     ? kKnownFlagsMask
        : ins.opcode == static_cast<uint16_t>(Op::kGemmNNQ8) ? kFlagEpilogueActMask
                                                              : uint16_t{0};
    if (ins.flags & static_cast<uint16_t>(~allowed))
      return Status::Fail(kUnitValidator, "unknown or misplaced instruction flags " +
                                              std::to_string(ins.flags) + " (opcode " + op + ")");
  }
  // Version gates for the v6 transformer family and the v7 embedding.
  if (ins.opcode >= static_cast<uint16_t>(Op::kRmsNormFwd) &&
      ins.opcode <= static_cast<uint16_t>(Op::kAttnDK) &&
      plan_version < kSeeuTransformerVersion)
    return Status::Fail(kUnitValidator, "transformer opcode " + op + " in a pre-v" +
                                            std::to_string(kSeeuTransformerVersion) + " plan");
  if (ins.opcode == static_cast<uint16_t>(Op::kEmbedFwd) && plan_version < kSeeuTokenVersion)
    return Status::Fail(kUnitValidator, "token opcode " + op + " in a pre-v" +
                                            std::to_string(kSeeuTokenVersion) + " plan");
  if (ins.opcode > kMaxOpcode)
    return Status::Fail(kUnitValidator, "unknown opcode " + op);

  Operand ops[8];
  size_t n = 0;
  const Status oob =
      Status::Fail(kUnitValidator, "instruction operand out of bounds (opcode " + op + ")");
  if (!OperandsOf(ins, ops, &n)) return oob;
  struct Range { uint64_t off, bytes; bool write, rodata; };
  Range ranges[8];
  for (size_t i = 0; i < n; ++i) {
    const Operand& o = ops[i];
    if (o.ref == kNullRef) return oob;
    if (o.write && IsRodataRef(o.ref)) return oob;
    if (o.elems == 0) return oob;
    uint64_t bytes = 0;
    if (!MulOk(o.elems, o.elem_bytes, &bytes)) return oob;
    if (RefOffset(o.ref) % o.elem_bytes != 0) return oob;
    const uint64_t space = IsRodataRef(o.ref) ? rodata_size : arena_size;
    if (!RangeOk(RefOffset(o.ref), bytes, space)) return oob;
    ranges[i] = {RefOffset(o.ref), bytes, o.write, IsRodataRef(o.ref)};
  }
  // A written range may overlap no other operand in its address space.
  for (size_t i = 0; i < n; ++i)
    for (size_t j = i + 1; j < n; ++j) {
      const Range& x = ranges[i];
      const Range& y = ranges[j];
      if (!(x.write || y.write) || x.rodata != y.rodata) continue;
      if (x.off < y.off + y.bytes && y.off < x.off + x.bytes)
        return Status::Fail(kUnitValidator,
                            "instruction operands alias a written range (opcode " + op + ")");
    }
  return Status::Ok();
}

Status VerifyPlanContract(const PlanHeader& h, uint64_t plan_size) {
  uint64_t tb = 0, mb = 0, eb = 0, xb = 0;
  if (!MulOk(h.train_instr_count, sizeof(UpdateInstruction), &tb) ||
      !MulOk(h.merge_instr_count, sizeof(UpdateInstruction), &mb) ||
      !MulOk(h.eval_instr_count, sizeof(UpdateInstruction), &eb) ||
      !MulOk(h.emit_count, sizeof(EmitEntry), &xb))
    return Status::Fail(kUnitEngine, "plan section size overflows");
  if (!RangeOk(h.train_instr_offset, tb, plan_size) ||
      !RangeOk(h.merge_instr_offset, mb, plan_size) ||
      !RangeOk(h.eval_instr_offset, eb, plan_size) ||
      !RangeOk(h.rodata_offset, h.rodata_size, plan_size) ||
      !RangeOk(h.persist_init_offset, h.persist_init_size, plan_size) ||
      !RangeOk(h.emit_table_offset, xb, plan_size))
    return Status::Fail(kUnitEngine, "plan section out of bounds");
  if (h.batch == 0) return Status::Fail(kUnitEngine, "plan batch size is zero");
  if (h.input_floats == 0) return Status::Fail(kUnitEngine, "plan input width is zero");
  if (h.arena_size > UINT64_MAX - 63) return Status::Fail(kUnitEngine, "arena size overflows");
  if (h.persist_init_size > h.arena_size || h.persistent_size > h.arena_size)
    return Status::Fail(kUnitEngine, "persistent segment exceeds arena");
  uint64_t in_bytes = 0;
  if (IsRodataRef(h.input_ref) || RefOffset(h.input_ref) % 4 != 0 ||
      !MulOk(h.input_floats, 4, &in_bytes) ||
      !RangeOk(RefOffset(h.input_ref), in_bytes, h.arena_size))
    return Status::Fail(kUnitEngine, "plan input slot out of bounds");
  if (h.label_kind != 0 &&
      (IsRodataRef(h.label_ref) || RefOffset(h.label_ref) % 4 != 0 ||
       !RangeOk(RefOffset(h.label_ref), h.label_bytes, h.arena_size)))
    return Status::Fail(kUnitEngine, "plan label slot out of bounds");
  if (IsRodataRef(h.loss_ref) || RefOffset(h.loss_ref) % 4 != 0 ||
      !RangeOk(RefOffset(h.loss_ref), 4, h.arena_size))
    return Status::Fail(kUnitEngine, "plan loss slot out of bounds");
  return Status::Ok();
}

Status VerifyExecutorContract(const std::vector<UpdateInstruction>& train,
                              const std::vector<UpdateInstruction>& merge,
                              const std::vector<UpdateInstruction>& eval,
                              const std::vector<EmitEntry>& emit,
                              const PlanHeader& h) {
  for (const auto* program : {&train, &merge, &eval})
    for (const UpdateInstruction& ins : *program) {
      if (Status s = ValidateInstruction(ins, h.arena_size, h.rodata_size, h.version); !s)
        return s;
      const auto op = static_cast<Op>(ins.opcode);
      // The two data-dependent-offset dereferences (labels, tokens) must
      // read exactly the staged, feeder-validated slots.
      if (op == Op::kSoftmaxXEntFwd || op == Op::kSoftmaxXEntBwd) {
        if (h.label_kind != 1)
          return Status::Fail(kUnitEngine, "softmax cross-entropy in a plan without class labels");
        if (ins.in[1] != h.label_ref)
          return Status::Fail(kUnitEngine, "softmax labels are not the plan's staged label slot");
        if (ins.out[0] != h.batch)
          return Status::Fail(kUnitEngine, "softmax row count disagrees with the plan batch");
      }
      if (op == Op::kEmbedFwd) {
        if (h.input_kind != 1)
          return Status::Fail(kUnitEngine, "embedding gather in a plan without token input");
        if (ins.in[0] != h.input_ref)
          return Status::Fail(kUnitEngine, "embedding tokens are not the plan's staged input slot");
        if (ins.out[0] != h.batch)
          return Status::Fail(kUnitEngine, "embedding row count disagrees with the plan batch");
      }
    }
  for (const EmitEntry& e : emit) {
    if (!RangeOk(e.arena_offset, e.byte_size, h.arena_size))
      return Status::Fail(kUnitEngine, "emit entry outside the arena");
    if (e.arena_offset % 4 != 0 || e.byte_size % 4 != 0)
      return Status::Fail(kUnitEngine, "emit entry misaligned");
  }
  return Status::Ok();
}

Status DecodeAndVerifyPlan(const uint8_t* plan, size_t plan_size, DecodedPlan* out) {
  PlanHeader h{};
  if (plan_size < sizeof(h)) return Status::Fail(kUnitEngine, "plan smaller than its header");
  std::memcpy(&h, plan, sizeof(h));
  if (h.magic != kSeeuMagic) return Status::Fail(kUnitEngine, "bad plan magic");
  if (h.version < kSeeuOldestReadable || h.version > kSeeuVersion)
    return Status::Fail(kUnitEngine, "unsupported plan version " + std::to_string(h.version) +
                                         " (this runtime reads v" +
                                         std::to_string(kSeeuOldestReadable) + "..v" +
                                         std::to_string(kSeeuVersion) + ")");
  if (PlanSelfHash(plan, plan_size, offsetof(PlanHeader, plan_hash)) != h.plan_hash)
    return Status::Fail(kUnitEngine, "plan hash mismatch — the .seeu blob is corrupt");
  if (Status s = VerifyPlanContract(h, plan_size); !s) return s;

  DecodedPlan d;
  d.header = h;
  const uint64_t offs[3] = {h.train_instr_offset, h.merge_instr_offset, h.eval_instr_offset};
  const uint64_t counts[3] = {h.train_instr_count, h.merge_instr_count, h.eval_instr_count};
  for (int p = 0; p < 3; ++p) {
    d.program[p].resize(counts[p]);
    if (counts[p])
      std::memcpy(d.program[p].data(), plan + offs[p], counts[p] * sizeof(UpdateInstruction));
  }
  d.emit.resize(h.emit_count);
  if (h.emit_count)
    std::memcpy(d.emit.data(), plan + h.emit_table_offset, h.emit_count * sizeof(EmitEntry));
  if (Status s = VerifyExecutorContract(d.program[0], d.program[1], d.program[2], d.emit, h); !s)
    return s;

  // Softmax class widths: train and eval forward widths must agree, and a
  // class-label plan must carry a softmax (update_engine.cc:153-166).
  uint64_t fwd_classes = 0;
  for (int p : {0, 2})
    for (const auto& ins : d.program[p])
      if (static_cast<Op>(ins.opcode) == Op::kSoftmaxXEntFwd) {
        if (fwd_classes != 0 && fwd_classes != ins.out[1])
          return Status::Fail(kUnitEngine, "plan softmax class widths disagree across programs");
        fwd_classes = ins.out[1];
      }
  if (h.label_kind == 1 && fwd_classes == 0)
    return Status::Fail(kUnitEngine,
                        "class-label plan carries no softmax cross-entropy — its labels "
                        "could never be validated");
  for (const auto& ins : d.program[2])
    if (static_cast<Op>(ins.opcode) == Op::kSoftmaxXEntFwd) {
      d.eval_probs_ref = ins.in[3];
      d.eval_softmax_rows = ins.out[0];
      d.eval_softmax_cols = ins.out[1];
    }
  for (int p = 0; p < 3; ++p)
    for (const auto& ins : d.program[p]) {
      const auto op = static_cast<Op>(ins.opcode);
      if (op == Op::kSoftmaxXEntFwd || op == Op::kSoftmaxXEntBwd) {
        const uint64_t classes = ins.out[1];
        if (classes != 0 && (d.num_classes == 0 || classes < d.num_classes))
          d.num_classes = classes;
      }
      if (op == Op::kEmbedFwd) {
        const uint64_t vocab = ins.out[1] >> 32;
        if (vocab != 0 && (d.vocab_bound == 0 || vocab < d.vocab_bound)) d.vocab_bound = vocab;
      }
    }
  if (h.input_kind > 1)
    return Status::Fail(kUnitEngine, "unknown plan input kind " + std::to_string(h.input_kind));
  if (h.input_kind == 1) {
    if (d.vocab_bound == 0)
      return Status::Fail(kUnitEngine,
                          "token plan carries no embedding — its token ids could never be "
                          "validated");
    if (h.seq_len == 0 || h.batch % h.seq_len != 0)
      return Status::Fail(kUnitEngine,
                          "token plan sequence length must be nonzero and divide the batch");
  }
  *out = std::move(d);
  return Status::Ok();
}

float EffectiveLr(const PlanHeader& h, uint64_t step) {
  const float base = h.lr;
  if (h.lr_schedule != 1) return base;  // LrSchedule::kCosineWithWarmup == 1
  if (h.warmup_steps > 0 && step <= h.warmup_steps)
    return base * static_cast<float>(step) / static_cast<float>(h.warmup_steps);
  const uint64_t horizon = h.default_steps > h.warmup_steps ? h.default_steps - h.warmup_steps : 0;
  const float floor_v = base * h.min_lr_factor;
  if (horizon == 0 || step - h.warmup_steps >= horizon) return floor_v;
  const float t = static_cast<float>(step - h.warmup_steps) / static_cast<float>(horizon);
  constexpr float kPi = 3.14159265358979323846f;
  return floor_v + (base - floor_v) * 0.5f * (1.0f + std::cos(kPi * t));
}

}  // namespace seeml_hip
