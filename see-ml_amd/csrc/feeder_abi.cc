// feeder_abi.cc — C-ABI of the batch feeder's dataset (include/seeml_hip.h).
#include <cstring>
#include <new>

#include "feeder.h"
#include "../../include/seeml_hip.h"

using seeml_hip::Dataset;
using seeml_hip::Status;

namespace {

void Copy(const std::string& m, char* err, uint64_t cap) {
  if (!err || cap == 0) return;
  const size_t n = m.size() < cap - 1 ? m.size() : cap - 1;
  std::memcpy(err, m.data(), n);
  err[n] = '\0';
}

int Make(const Status& s, Dataset&& d, seeml_hip_dataset** out, char* err, uint64_t cap) {
  if (!s) {
    Copy(s.error, err, cap);
    return SEEML_HIP_ERROR;
  }
  auto* h = new (std::nothrow) seeml_hip_dataset;
  if (!h) {
    Copy("Dataset: out of host memory", err, cap);
    return SEEML_HIP_ERROR;
  }
  h->impl = std::move(d);
  *out = h;
  return SEEML_HIP_OK;
}

int Ret(seeml_hip_dataset* d, const Status& s) {
  if (s.ok) return SEEML_HIP_OK;
  d->error = s.error;
  return SEEML_HIP_ERROR;
}

}  // namespace

extern "C" {

uint64_t seeml_hip_splitmix64(uint64_t* state) { return seeml_hip::SplitMix64(state); }

int seeml_hip_dataset_from_tokens(const int32_t* tokens, uint64_t count, uint64_t num_records,
                                  uint64_t seq, seeml_hip_dataset** out, char* err,
                                  uint64_t err_cap) {
  Dataset d;
  const Status s = Dataset::FromTokens(tokens, count, num_records, seq, &d);
  return Make(s, std::move(d), out, err, err_cap);
}

int seeml_hip_dataset_from_memory(const float* inputs, uint64_t input_count,
                                  const uint8_t* labels, uint64_t label_bytes,
                                  uint64_t num_samples, uint64_t input_dim, uint32_t label_kind,
                                  uint64_t label_dim, seeml_hip_dataset** out, char* err,
                                  uint64_t err_cap) {
  Dataset d;
  const Status s = Dataset::FromMemory(inputs, input_count, labels, label_bytes, num_samples,
                                       input_dim, label_kind, label_dim, &d);
  return Make(s, std::move(d), out, err, err_cap);
}

int seeml_hip_dataset_load(const char* path, seeml_hip_dataset** out, char* err,
                           uint64_t err_cap) {
  Dataset d;
  const Status s = Dataset::LoadFromFile(path ? path : "", &d);
  return Make(s, std::move(d), out, err, err_cap);
}

int seeml_hip_dataset_save(seeml_hip_dataset* d, const char* path) {
  return Ret(d, d->impl.SaveToFile(path ? path : ""));
}

void seeml_hip_dataset_free(seeml_hip_dataset* d) { delete d; }
const char* seeml_hip_dataset_error(const seeml_hip_dataset* d) { return d->error.c_str(); }
uint64_t seeml_hip_dataset_num_samples(const seeml_hip_dataset* d) { return d->impl.num_samples(); }
uint64_t seeml_hip_dataset_input_dim(const seeml_hip_dataset* d) { return d->impl.input_dim(); }
uint32_t seeml_hip_dataset_label_kind(const seeml_hip_dataset* d) { return d->impl.label_kind(); }
uint32_t seeml_hip_dataset_input_kind(const seeml_hip_dataset* d) { return d->impl.input_kind(); }
uint64_t seeml_hip_dataset_label_bytes_per_sample(const seeml_hip_dataset* d) {
  return d->impl.label_bytes_per_sample();
}

int seeml_hip_dataset_validate_class_labels(seeml_hip_dataset* d, uint64_t num_classes) {
  return Ret(d, d->impl.ValidateClassLabels(num_classes));
}

void seeml_hip_dataset_fill_batch(seeml_hip_dataset* d, uint64_t batch, void* input_slot,
                                  void* label_slot) {
  d->impl.FillBatch(batch, input_slot, label_slot);
}

void seeml_hip_dataset_rewind(seeml_hip_dataset* d) { d->impl.Rewind(); }
void seeml_hip_dataset_enable_shuffle(seeml_hip_dataset* d, uint64_t seed) {
  d->impl.EnableShuffle(seed);
}

void seeml_hip_dataset_get_serving_pos(const seeml_hip_dataset* d, uint64_t* cursor,
                                       uint64_t* epoch) {
  const Dataset::ServingPos p = d->impl.SaveServingPos();
  *cursor = p.cursor;
  *epoch = p.epoch;
}

void seeml_hip_dataset_restore_serving_pos(seeml_hip_dataset* d, uint64_t cursor,
                                           uint64_t epoch) {
  d->impl.RestoreServingPos({cursor, epoch});
}

int seeml_hip_dataset_skip_served(seeml_hip_dataset* d, uint64_t rows) {
  return Ret(d, d->impl.SkipServed(rows));
}

int seeml_hip_dataset_split_validation(seeml_hip_dataset* d, double fraction,
                                       seeml_hip_dataset** val) {
  Dataset v;
  const Status s = d->impl.SplitValidation(fraction, &v);
  if (!s) return Ret(d, s);
  auto* h = new (std::nothrow) seeml_hip_dataset;
  if (!h) return Ret(d, Status::Fail(seeml_hip::kUnitDataset, "out of host memory"));
  h->impl = std::move(v);
  *val = h;
  return SEEML_HIP_OK;
}

}  // extern "C"
