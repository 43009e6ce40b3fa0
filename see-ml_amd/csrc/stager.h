// stager.h — batch staging into the plan's device I/O slots.
//
// The MI355X form of runtime/feeder/batch_pipeline.{h,cc}: a feeder thread
// fills the next batch (Dataset::FillBatch, shuffle gathers, epoch
// reshuffles) into one of two pinned host buffers while the current step
// runs; Next() waits for it and enqueues one H2D copy per slot on the
// engine stream. At most one staged batch runs ahead, and a batch staged
// but never taken is un-consumed at teardown (RestoreServingPos), so the
// dataset's serving position is exactly the batches the engine consumed:
// pipelining is invisible in the served sequence (batch_pipeline.cc:21-37).
#pragma once

#include <hip/hip_runtime_api.h>

#include <condition_variable>
#include <cstdint>
#include <mutex>
#include <thread>

#include "feeder.h"

namespace seeml_hip {

class BatchStager {
 public:
  // batch: the plan's batch rows; in_bytes / label_bytes: the slot sizes
  // (label_bytes 0 = the plan takes no labels).
  BatchStager(Dataset& data, uint64_t batch, uint64_t in_bytes, uint64_t label_bytes);
  ~BatchStager();
  BatchStager(const BatchStager&) = delete;
  BatchStager& operator=(const BatchStager&) = delete;

  // Allocates the pinned buffers and starts the feeder thread.
  Status Start();
  // Takes the staged batch: H2D into d_input / d_labels on `stream`.
  Status Next(void* d_input, void* d_labels, hipStream_t stream);

 private:
  void Loop();
  uint8_t* input_buf(int k) const { return buf_[k]; }
  uint8_t* label_buf(int k) const { return label_bytes_ ? buf_[k] + in_bytes_ : nullptr; }

  Dataset& data_;
  const uint64_t batch_, in_bytes_, label_bytes_;
  uint8_t* buf_[2] = {nullptr, nullptr};
  hipEvent_t copied_[2] = {nullptr, nullptr};
  bool copy_pending_[2] = {false, false};
  std::thread feeder_;
  std::mutex mu_;
  std::condition_variable cv_;
  bool started_ = false, stop_ = false, full_ = false;
  int fill_ = 0;        // buffer the feeder fills next
  int ready_ = 0;       // buffer holding the staged batch (valid while full_)
  Dataset::ServingPos stage_start_;
};

}  // namespace seeml_hip
