// plan_abi.h — the SeeML plan ABI as this backend reads it.
//
// The .seeu layout is a compiler<->runtime contract, so every field, width
// and opcode value below must match the reference byte-for-byte:
//   UpdateInstruction / OpCode / epilogue flags: source/plan/instruction.h:15-151
//   PlanHeader / EmitEntry / version policy:     source/plan/schema.h:18-178
// The static_asserts pin the sizes and field offsets the reference pins.
#pragma once

#include <cstddef>
#include <cstdint>

namespace seeml_hip {

inline constexpr uint64_t kRodataBit = 1ULL << 63;
inline constexpr uint64_t kNullRef = ~0ULL;
inline constexpr bool IsRodataRef(uint64_t ref) { return (ref & kRodataBit) != 0; }
inline constexpr uint64_t RefOffset(uint64_t ref) { return ref & ~kRodataBit; }

enum class Op : uint16_t {
  kNop = 0,
  kGemmNN = 1, kGemmNT = 2, kGemmTN = 3, kGemmAccNN = 4,
  kAddEW = 5, kAddBias = 6, kReluFwd = 7, kReluBwd = 8, kScale = 9,
  kReduceRows = 10,
  kSoftmaxXEntFwd = 11, kSoftmaxXEntBwd = 12, kMseFwd = 13, kMseBwd = 14,
  kKLDistillFwd = 15, kKLDistillBwd = 16,
  kSgdStep = 17, kAdamWStep = 18,
  kFill = 19, kCopy = 20,
  kMulEW = 21, kGeluFwd = 22, kGeluBwd = 23, kSiluFwd = 24, kSiluBwd = 25,
  kLayerNormFwd = 26, kLayerNormBwd = 27,
  kClipNorm = 28, kGemmNNQ8 = 29, kGemmNTQ8 = 30,
  kRmsNormFwd = 31, kRmsNormBwd = 32, kRopeFwd = 33, kRopeBwd = 34,
  kAttnFwd = 35, kAttnDP = 36, kAttnDV = 37, kSoftmaxRowsBwd = 38,
  kAttnDQ = 39, kAttnDK = 40,
  kEmbedFwd = 41,
};
inline constexpr uint16_t kMaxOpcode = 41;

inline constexpr uint16_t kFlagEpilogueBias = 1u << 0;
inline constexpr uint16_t kFlagEpilogueActShift = 1;
inline constexpr uint16_t kFlagEpilogueActMask = 3u << kFlagEpilogueActShift;
inline constexpr uint16_t kKnownFlagsMask = kFlagEpilogueBias | kFlagEpilogueActMask;
enum class Act : uint16_t { kNone = 0, kRelu = 1, kGelu = 2, kSilu = 3 };
inline constexpr Act ActOf(uint16_t flags) {
  return static_cast<Act>((flags & kFlagEpilogueActMask) >> kFlagEpilogueActShift);
}

inline constexpr uint32_t kSeeuMagic = 0x55454553;  // "SEEU"
inline constexpr uint32_t kSeeuVersion = 7;
inline constexpr uint32_t kSeeuOldestReadable = 4;
inline constexpr uint32_t kSeeuFlagsVersion = 5;
inline constexpr uint32_t kSeeuTransformerVersion = 6;
inline constexpr uint32_t kSeeuTokenVersion = 7;

#pragma pack(push, 1)
struct UpdateInstruction {
  uint16_t opcode = 0;
  uint16_t flags = 0;
  uint32_t pad = 0;
  uint64_t in[4] = {kNullRef, kNullRef, kNullRef, kNullRef};
  uint64_t out[3] = {0, 0, 0};
};

struct PlanHeader {
  uint32_t magic = kSeeuMagic;
  uint32_t version = kSeeuVersion;
  uint64_t arena_size = 0;
  uint64_t persistent_size = 0;
  uint64_t input_ref = kNullRef;
  uint64_t input_floats = 0;
  uint64_t label_ref = kNullRef;
  uint64_t label_bytes = 0;
  uint32_t label_kind = 0;
  uint32_t optimizer_kind = 1;
  uint64_t loss_ref = kNullRef;
  uint64_t train_instr_offset = 0;
  uint64_t train_instr_count = 0;
  uint64_t merge_instr_offset = 0;
  uint64_t merge_instr_count = 0;
  uint64_t rodata_offset = 0;
  uint64_t rodata_size = 0;
  uint64_t persist_init_offset = 0;
  uint64_t persist_init_size = 0;
  uint64_t emit_table_offset = 0;
  uint64_t emit_count = 0;
  float lr = 1e-3f;
  float beta1 = 0.9f;
  float beta2 = 0.999f;
  float eps = 1e-8f;
  float weight_decay = 0.01f;
  uint32_t pad2 = 0;
  uint64_t batch = 0;
  uint64_t default_steps = 0;
  uint64_t eval_instr_offset = 0;
  uint64_t eval_instr_count = 0;
  uint64_t source_model_hash = 0;
  uint64_t plan_hash = 0;
  uint32_t lr_schedule = 0;
  uint32_t pad3 = 0;
  uint64_t warmup_steps = 0;
  float min_lr_factor = 0.0f;
  float clip_norm = 0.0f;
  uint32_t input_kind = 0;
  uint32_t pad4 = 0;
  uint64_t seq_len = 0;
  uint64_t reserved[2] = {0, 0};
};

struct EmitEntry {
  uint64_t smf_data_offset = 0;
  uint64_t byte_size = 0;
  uint64_t arena_offset = 0;
};
#pragma pack(pop)

static_assert(sizeof(UpdateInstruction) == 64, "instruction word is 64 bytes");
static_assert(sizeof(PlanHeader) == 280, "PlanHeader layout is part of the ABI");
static_assert(sizeof(EmitEntry) == 24, "EmitEntry layout is part of the ABI");
static_assert(offsetof(PlanHeader, lr) == 152, "optimizer block offset");
static_assert(offsetof(PlanHeader, plan_hash) == 216, "plan_hash offset");
static_assert(offsetof(PlanHeader, seq_len) == 256, "v7 seq_len offset");

enum class Program : int { kTrain = 0, kMerge = 1, kEval = 2 };

}  // namespace seeml_hip
