// feeder.h — the batch feeder's dataset, host side (no GPU code).
//
// Serves fixed-shape samples into the plan's I/O slots, the contract of
// runtime/feeder/dataset.{h,cc}: sequentially with wraparound, or through a
// seeded splitmix64 Fisher–Yates permutation re-drawn at every epoch; token
// corpora (input_kind 1) serve whole records of seq+1 ids as inputs
// tokens[0..S) and shifted labels tokens[1..S]. The .sds bytes, the error
// texts and the served bytes and order are the reference's (integer and copy
// work only). The storage is this file's own: the corpus is held as the
// .sds sample section itself, one fixed-size record per sample.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "plan_checks.h"

namespace seeml_hip {

inline constexpr const char* kUnitDataset = "Dataset";
inline constexpr uint32_t kSdsMagic = 0x31534453;  // "SDS1" little-endian

// splitmix64 step (dataset.cc:344-352): advances *state, returns the mix.
uint64_t SplitMix64(uint64_t* state);

class Dataset {
 public:
  struct ServingPos {
    uint64_t cursor = 0;
    uint64_t epoch = 0;
  };

  // Construction (dataset.cc:34-120). On failure *out is untouched.
  static Status FromTokens(const int32_t* tokens, uint64_t count, uint64_t num_records,
                           uint64_t seq, Dataset* out);
  static Status FromMemory(const float* inputs, uint64_t input_count, const uint8_t* labels,
                           uint64_t label_bytes, uint64_t num_samples, uint64_t input_dim,
                           uint32_t label_kind, uint64_t label_dim, Dataset* out);
  static Status LoadFromFile(const std::string& path, Dataset* out);
  Status SaveToFile(const std::string& path) const;

  uint64_t num_samples() const { return num_samples_; }
  uint64_t input_dim() const { return input_dim_; }
  uint32_t label_kind() const { return label_kind_; }
  uint32_t input_kind() const { return input_kind_; }
  uint64_t label_dim() const { return label_dim_; }
  uint64_t label_bytes_per_sample() const;

  Status ValidateClassLabels(uint64_t num_classes) const;

  // Copies the next `batch` samples (token corpora: `batch` token rows, a
  // whole number of records) into host slots. label_slot may be null.
  void FillBatch(uint64_t batch, void* input_slot, void* label_slot);
  void Rewind() { cursor_ = 0; }
  void EnableShuffle(uint64_t seed);
  ServingPos SaveServingPos() const { return {cursor_, epoch_}; }
  void RestoreServingPos(ServingPos pos);
  Status SkipServed(uint64_t rows);
  Status SplitValidation(double fraction, Dataset* val);

 private:
  // Record geometry: the served input is the record's first input_dim_ * 4
  // bytes; the label bytes follow it (feature rows) or are the same ids one
  // position on (token records).
  uint64_t LabelOffset() const { return input_kind_ == 1 ? sizeof(int32_t) : input_dim_ * 4; }
  const uint8_t* Record(uint64_t i) const { return records_.data() + i * record_bytes_; }
  uint64_t CurrentRecord() const { return perm_.empty() ? cursor_ : perm_[cursor_]; }
  void Advance();
  void DrawPermutation();

  std::vector<uint8_t> records_;  // num_samples_ * record_bytes_, the .sds sample section
  uint64_t record_bytes_ = 0;
  uint64_t num_samples_ = 0;
  uint64_t input_dim_ = 0;
  uint32_t label_kind_ = 0;
  uint32_t input_kind_ = 0;
  uint64_t label_dim_ = 0;
  uint64_t cursor_ = 0;
  uint64_t epoch_ = 0;
  std::vector<uint64_t> perm_;  // this epoch's serving order; empty = sequential
  uint64_t origin_ = 0;         // splitmix64 state at epoch 0's first draw
};

// VerifyFeederContract (contract.cc:170-235): the dataset's geometry matches
// the compiled plan; class labels / token ids lie inside the plan's bounds.
Status VerifyFeederContract(const PlanHeader& h, const Dataset& data, uint64_t num_classes,
                            uint64_t vocab_bound);

}  // namespace seeml_hip

// The C-ABI's dataset handle (include/seeml_hip.h).
struct seeml_hip_dataset {
  seeml_hip::Dataset impl;
  std::string error;
};
