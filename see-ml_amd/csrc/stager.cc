// stager.cc — pinned double-buffered batch staging (runtime/feeder/batch_pipeline.cc).
#include "stager.h"

#include "device_mem.h"

#include <string>

namespace seeml_hip {

namespace {

Status Hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return Status::Ok();
  return Status::Fail("BatchPipeline", std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace

BatchStager::BatchStager(Dataset& data, uint64_t batch, uint64_t in_bytes, uint64_t label_bytes)
    : data_(data), batch_(batch), in_bytes_(in_bytes), label_bytes_(label_bytes) {}

Status BatchStager::Start() {
  const uint64_t bytes = (in_bytes_ + label_bytes_) ? (in_bytes_ + label_bytes_) : 1;
  for (int k = 0; k < 2; ++k) {
    if (Status s = Hip(LockedHostMalloc(&buf_[k], bytes), "pinned staging");
        !s)
      return s;
    if (Status s = Hip(hipEventCreateWithFlags(&copied_[k], hipEventDisableTiming), "event"); !s)
      return s;
  }
  started_ = true;
  feeder_ = std::thread([this] { Loop(); });
  return Status::Ok();
}

void BatchStager::Loop() {
  for (;;) {
    int k;
    {
      std::unique_lock<std::mutex> lock(mu_);
      cv_.wait(lock, [&] { return !full_ || stop_; });
      if (stop_) return;
      k = fill_;
    }
    // The buffer's previous upload must have left it before it is refilled.
    if (copy_pending_[k]) {
      (void)hipEventSynchronize(copied_[k]);
      copy_pending_[k] = false;
    }
    // Snapshot first, so teardown can un-consume a batch never taken.
    stage_start_ = data_.SaveServingPos();
    data_.FillBatch(batch_, input_buf(k), label_buf(k));
    {
      std::lock_guard<std::mutex> lock(mu_);
      full_ = true;
      ready_ = k;
      fill_ = k ^ 1;
    }
    cv_.notify_all();
  }
}

Status BatchStager::Next(void* d_input, void* d_labels, hipStream_t stream) {
  int k;
  {
    std::unique_lock<std::mutex> lock(mu_);
    cv_.wait(lock, [&] { return full_; });
    k = ready_;
  }
  Status st = Hip(hipMemcpyAsync(d_input, input_buf(k), in_bytes_, hipMemcpyHostToDevice, stream),
                  "input staging");
  if (st && label_bytes_ && d_labels)
    st = Hip(hipMemcpyAsync(d_labels, label_buf(k), label_bytes_, hipMemcpyHostToDevice, stream),
             "label staging");
  if (st) st = Hip(hipEventRecord(copied_[k], stream), "staging event");
  {
    std::lock_guard<std::mutex> lock(mu_);
    copy_pending_[k] = true;
    full_ = false;
  }
  cv_.notify_all();
  return st;
}

BatchStager::~BatchStager() {
  if (started_) {
    {
      std::lock_guard<std::mutex> lock(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    feeder_.join();
    // A staged batch the engine never took goes back to the dataset.
    if (full_) data_.RestoreServingPos(stage_start_);
  }
  for (int k = 0; k < 2; ++k) {
    if (copied_[k]) {
      if (copy_pending_[k]) (void)hipEventSynchronize(copied_[k]);
      (void)hipEventDestroy(copied_[k]);
    }
    if (buf_[k]) (void)LockedHostFree(buf_[k]);
  }
}

}  // namespace seeml_hip
