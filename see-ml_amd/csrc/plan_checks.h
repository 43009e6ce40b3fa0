// plan_checks.h — load-time proof that a plan is fit for blind dispatch.
//
// The reference runs these checks before its first step and then executes
// instructions without further checks; the device backend keeps that
// contract: nothing is uploaded or launched until every check here passed.
//   ValidateInstruction     runtime/validator/plan_validator.cc:9-344
//   VerifyPlanContract      runtime/engine/contract.cc:35-100
//   VerifyExecutorContract  runtime/engine/contract.cc:102-168
//   softmax-width / token scans, Initialize  runtime/engine/update_engine.cc:80-225
//   PlanSelfHash, ContentHash64  source/identity/hash.h:67-161
// Errors read "<unit>: <message>" (runtime/diagnostics/diagnostic.h:30-41),
// units "PlanValidator" and "UpdateEngine" as in the reference.
#pragma once

#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "plan_abi.h"

namespace seeml_hip {

// A success-or-message status: this toolchain has no <expected>.
struct Status {
  bool ok = true;
  std::string error;
  static Status Ok() { return {}; }
  static Status Fail(const char* unit, const std::string& message) {
    return Status{false, std::string(unit) + ": " + message};
  }
  explicit operator bool() const { return ok; }
};

inline constexpr const char* kUnitEngine = "UpdateEngine";
inline constexpr const char* kUnitValidator = "PlanValidator";

inline bool MulOk(uint64_t a, uint64_t b, uint64_t* out) {
  if (b != 0 && a > UINT64_MAX / b) return false;
  *out = a * b;
  return true;
}
inline bool RangeOk(uint64_t off, uint64_t bytes, uint64_t size) {
  return off <= size && bytes <= size - off;
}

// ContentHash64 / PlanSelfHash (source/identity/hash.h:67-161): 8-lane
// striped FNV-1a per 1 MiB chunk (chunk count capped at 256 by ParallelFor's
// geometry), chunk digests folded in order, then the size.
uint64_t ContentHash64(const uint8_t* data, size_t size);
uint64_t PlanSelfHash(const uint8_t* plan, size_t size, size_t hash_offset);

// Arena byte ranges [offset, offset + bytes) an instruction writes (rodata is
// never written), from the validator's operand table, appended to *ranges
// (so one vector can gather several instructions'); false when the dims are
// malformed.
bool WriteRangesOf(const UpdateInstruction& ins,
                   std::vector<std::pair<uint64_t, uint64_t>>* ranges);
// The same for the arena ranges an instruction reads.
bool ReadRangesOf(const UpdateInstruction& ins,
                  std::vector<std::pair<uint64_t, uint64_t>>* ranges);
// Every arena range an instruction's results depend on: ReadRangesOf plus the
// operands it updates in place (GemmAccNN's C, the optimizer steps'
// parameters and moments, ClipNorm's tensor), which the operand table lists
// as writes only.
bool DependRangesOf(const UpdateInstruction& ins,
                    std::vector<std::pair<uint64_t, uint64_t>>* ranges);

Status ValidateInstruction(const UpdateInstruction& ins, uint64_t arena_size,
                           uint64_t rodata_size, uint32_t plan_version);
Status VerifyPlanContract(const PlanHeader& header, uint64_t plan_size);
Status VerifyExecutorContract(const std::vector<UpdateInstruction>& train,
                              const std::vector<UpdateInstruction>& merge,
                              const std::vector<UpdateInstruction>& eval,
                              const std::vector<EmitEntry>& emit,
                              const PlanHeader& header);

// Everything UpdateEngine::Initialize proves before it allocates the arena
// (update_engine.cc:80-225). On success the decoded programs and the scanned
// runtime bounds are returned through the out-parameters.
struct DecodedPlan {
  PlanHeader header;
  std::vector<UpdateInstruction> program[3];  // train, merge, eval
  std::vector<EmitEntry> emit;
  uint64_t num_classes = 0;   // narrowest softmax width anywhere
  uint64_t vocab_bound = 0;   // narrowest embedding table anywhere
  uint64_t eval_probs_ref = kNullRef;
  uint64_t eval_softmax_rows = 0;
  uint64_t eval_softmax_cols = 0;
};
Status DecodeAndVerifyPlan(const uint8_t* plan, size_t plan_size,
                           DecodedPlan* out);

// UpdateEngine::EffectiveLr (update_engine.cc:515-534), same float expressions.
float EffectiveLr(const PlanHeader& h, uint64_t step);

}  // namespace seeml_hip
