// feeder.cc — the batch feeder's dataset (runtime/feeder/dataset.cc), host.
#include "feeder.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <utility>

namespace seeml_hip {

namespace {

constexpr uint64_t kSdsHeaderBytes = 40;
constexpr uint64_t kChunkBudget = 256 * 1024;  // bounded record staging for file I/O

Status Fail(const std::string& m) { return Status::Fail(kUnitDataset, m); }

}  // namespace

uint64_t SplitMix64(uint64_t* state) {
  uint64_t z = (*state += 0x9E3779B97F4A7C15ULL);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

uint64_t Dataset::label_bytes_per_sample() const {
  // A token record derives one class id per position (dataset.cc:23-33).
  if (input_kind_ == 1) return input_dim_ * sizeof(int32_t);
  if (label_kind_ == 1) return sizeof(int32_t);
  if (label_kind_ == 2) return label_dim_ * sizeof(float);
  return 0;
}

Status Dataset::FromTokens(const int32_t* tokens, uint64_t count, uint64_t num_records,
                           uint64_t seq, Dataset* out) {
  if (num_records == 0) return Fail("zero samples");
  if (seq == 0) return Fail("zero input dim");
  uint64_t want = 0;
  if (seq == UINT64_MAX || !MulOk(num_records, seq + 1, &want) || count != want)
    return Fail("token buffer size mismatch");
  for (uint64_t i = 0; i < want; ++i)
    if (tokens[i] < 0) return Fail("negative token id at position " + std::to_string(i));
  Dataset d;
  d.input_kind_ = 1;
  d.label_kind_ = 1;
  d.num_samples_ = num_records;
  d.input_dim_ = seq;
  d.tokens_.assign(tokens, tokens + want);
  *out = std::move(d);
  return Status::Ok();
}

Status Dataset::FromMemory(const float* inputs, uint64_t input_count, const uint8_t* labels,
                           uint64_t label_bytes, uint64_t num_samples, uint64_t input_dim,
                           uint32_t label_kind, uint64_t label_dim, Dataset* out) {
  Dataset d;
  d.num_samples_ = num_samples;
  d.input_dim_ = input_dim;
  d.label_kind_ = label_kind;
  d.label_dim_ = label_dim;
  if (num_samples == 0) return Fail("zero samples");
  if (input_dim == 0) return Fail("zero input dim");
  if (label_kind > 2) return Fail("unknown label kind");
  if (label_kind == 2 && (label_dim == 0 || label_dim > UINT64_MAX / sizeof(float)))
    return Fail("label dim out of range");
  uint64_t want_inputs = 0, want_labels = 0;
  if (!MulOk(num_samples, input_dim, &want_inputs) || input_count != want_inputs)
    return Fail("input buffer size mismatch");
  if (!MulOk(num_samples, d.label_bytes_per_sample(), &want_labels) || label_bytes != want_labels)
    return Fail("label buffer size mismatch");
  d.inputs_.assign(inputs, inputs + want_inputs);
  if (want_labels) d.labels_.assign(labels, labels + want_labels);
  *out = std::move(d);
  return Status::Ok();
}

Status Dataset::LoadFromFile(const std::string& path, Dataset* out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return Fail("cannot open '" + path + "'");
  f.seekg(0, std::ios::end);
  const std::streamoff end_pos = f.tellg();
  if (end_pos < 0) return Fail("cannot stat '" + path + "'");
  const uint64_t file_size = static_cast<uint64_t>(end_pos);
  f.seekg(0);
  auto read = [&](void* dst, uint64_t n) {
    f.read(static_cast<char*>(dst), static_cast<std::streamsize>(n));
    return static_cast<bool>(f);
  };

  uint32_t magic = 0, version = 0, label_kind = 0, input_kind = 0;
  uint64_t num_samples = 0, input_dim = 0, label_dim = 0;
  if (!read(&magic, 4) || magic != kSdsMagic) return Fail("bad magic in '" + path + "'");
  if (!read(&version, 4) || version < 1 || version > 2) return Fail("unsupported version");
  if (!read(&num_samples, 8) || !read(&input_dim, 8) || !read(&label_kind, 4) ||
      !read(&input_kind, 4) || !read(&label_dim, 8))
    return Fail("truncated header");

  Dataset d;
  d.num_samples_ = num_samples;
  d.input_dim_ = input_dim;
  d.label_kind_ = label_kind;
  d.label_dim_ = label_dim;
  d.input_kind_ = input_kind;
  if (num_samples == 0 || input_dim == 0) return Fail("empty dataset");
  if (label_kind > 2) return Fail("unknown label kind");
  if (label_kind == 2 && (label_dim == 0 || label_dim > UINT64_MAX / sizeof(float)))
    return Fail("label dim out of range");
  // v1's input_kind word was header padding (always 0).
  if (input_kind > 1 || (version < 2 && input_kind != 0)) return Fail("unknown input kind");

  if (input_kind == 1) {
    if (label_kind != 1 || label_dim != 0)
      return Fail("token corpora derive next-token class labels (label_kind 1, label_dim 0)");
    uint64_t record_bytes = 0, payload = 0;
    if (input_dim == UINT64_MAX || !MulOk(input_dim + 1, sizeof(int32_t), &record_bytes) ||
        !MulOk(num_samples, record_bytes, &payload) || payload > file_size - kSdsHeaderBytes)
      return Fail("sample section exceeds file size");
    d.tokens_.resize(payload / sizeof(int32_t));
    if (!read(d.tokens_.data(), payload)) return Fail("truncated inputs");
    for (const int32_t t : d.tokens_)
      if (t < 0) return Fail("negative token id");
    *out = std::move(d);
    return Status::Ok();
  }

  const uint64_t lbytes = d.label_bytes_per_sample();
  uint64_t input_bytes = 0, payload = 0;
  if (!MulOk(input_dim, sizeof(float), &input_bytes) || input_bytes > UINT64_MAX - lbytes ||
      !MulOk(num_samples, input_bytes + lbytes, &payload) ||
      payload > file_size - kSdsHeaderBytes)
    return Fail("sample section exceeds file size");
  d.inputs_.resize(num_samples * input_dim);
  d.labels_.resize(num_samples * lbytes);
  if (lbytes == 0) {
    if (!read(d.inputs_.data(), num_samples * input_bytes)) return Fail("truncated inputs");
    *out = std::move(d);
    return Status::Ok();
  }
  // Interleaved records, de-interleaved through a bounded chunk.
  const uint64_t record = input_bytes + lbytes;
  const uint64_t per_chunk = record >= kChunkBudget ? 1 : kChunkBudget / record;
  std::vector<uint8_t> chunk(per_chunk * record);
  for (uint64_t i = 0; i < num_samples;) {
    const uint64_t n = std::min(per_chunk, num_samples - i);
    if (!read(chunk.data(), n * record)) return Fail("truncated inputs");
    for (uint64_t s = 0; s < n; ++s) {
      const uint8_t* rec = chunk.data() + s * record;
      std::memcpy(d.inputs_.data() + (i + s) * input_dim, rec, input_bytes);
      std::memcpy(d.labels_.data() + (i + s) * lbytes, rec + input_bytes, lbytes);
    }
    i += n;
  }
  *out = std::move(d);
  return Status::Ok();
}

Status Dataset::SaveToFile(const std::string& path) const {
  std::ofstream f(path, std::ios::binary | std::ios::trunc);
  if (!f) return Fail("cannot write '" + path + "'");
  auto write = [&](const void* src, uint64_t n) {
    f.write(static_cast<const char*>(src), static_cast<std::streamsize>(n));
  };
  const uint32_t version = input_kind_ == 1 ? 2 : 1;
  write(&kSdsMagic, 4);
  write(&version, 4);
  write(&num_samples_, 8);
  write(&input_dim_, 8);
  write(&label_kind_, 4);
  write(&input_kind_, 4);
  write(&label_dim_, 8);
  if (input_kind_ == 1) {
    write(tokens_.data(), tokens_.size() * sizeof(int32_t));
  } else {
    const uint64_t lbytes = label_bytes_per_sample();
    if (lbytes == 0) {
      write(inputs_.data(), num_samples_ * input_dim_ * sizeof(float));
    } else {
      const uint64_t input_bytes = input_dim_ * sizeof(float);
      const uint64_t record = input_bytes + lbytes;
      const uint64_t per_chunk = record >= kChunkBudget ? 1 : kChunkBudget / record;
      std::vector<uint8_t> chunk(per_chunk * record);
      for (uint64_t i = 0; i < num_samples_;) {
        const uint64_t n = std::min(per_chunk, num_samples_ - i);
        for (uint64_t s = 0; s < n; ++s) {
          uint8_t* rec = chunk.data() + s * record;
          std::memcpy(rec, inputs_.data() + (i + s) * input_dim_, input_bytes);
          std::memcpy(rec + input_bytes, labels_.data() + (i + s) * lbytes, lbytes);
        }
        write(chunk.data(), n * record);
        i += n;
      }
    }
  }
  f.close();  // the stream tail flushes here; check after
  if (f.fail()) return Fail("short write to '" + path + "'");
  return Status::Ok();
}

Status Dataset::ValidateClassLabels(uint64_t num_classes) const {
  if (label_kind_ != 1 || num_classes == 0) return Status::Ok();
  auto outside = [&](const char* what, int64_t v, uint64_t where) {
    return Fail(std::string(what) + std::to_string(v) + " at " +
                (input_kind_ == 1 ? "position " : "sample ") + std::to_string(where) +
                " outside [0, " + std::to_string(num_classes) + ")");
  };
  if (input_kind_ == 1) {
    // Every token is an embedding index and, shifted, a class label.
    for (uint64_t i = 0; i < tokens_.size(); ++i)
      if (tokens_[i] < 0 || static_cast<uint64_t>(tokens_[i]) >= num_classes)
        return outside("token id ", tokens_[i], i);
    return Status::Ok();
  }
  for (uint64_t i = 0; i < num_samples_; ++i) {
    int32_t v;
    std::memcpy(&v, labels_.data() + i * sizeof(int32_t), sizeof v);
    if (v < 0 || static_cast<uint64_t>(v) >= num_classes) return outside("class label ", v, i);
  }
  return Status::Ok();
}

void Dataset::FillBatch(uint64_t batch, void* input_slot, void* label_slot) {
  uint8_t* in = static_cast<uint8_t*>(input_slot);
  uint8_t* lab = static_cast<uint8_t*>(label_slot);
  if (input_kind_ == 1) {
    // `batch` counts token rows; one record serves S of them (dataset.cc:290-313).
    const uint64_t S = input_dim_;
    const uint64_t row_bytes = S * sizeof(int32_t);
    for (uint64_t r = 0; r < batch / S; ++r) {
      const uint64_t i = order_.empty() ? cursor_ : order_[cursor_];
      const int32_t* rec = tokens_.data() + i * (S + 1);
      std::memcpy(in + r * row_bytes, rec, row_bytes);
      if (lab) std::memcpy(lab + r * row_bytes, rec + 1, row_bytes);
      if (++cursor_ == num_samples_) {
        cursor_ = 0;
        if (!order_.empty()) {
          Reshuffle();
          ++epoch_;
        }
      }
    }
    return;
  }
  const uint64_t lbytes = label_bytes_per_sample();
  const uint64_t in_bytes = input_dim_ * sizeof(float);
  if (order_.empty()) {
    // Sequential: copy contiguous runs up to the wrap point.
    for (uint64_t b = 0; b < batch;) {
      const uint64_t run = std::min(batch - b, num_samples_ - cursor_);
      std::memcpy(in + b * in_bytes, inputs_.data() + cursor_ * input_dim_, run * in_bytes);
      if (lab && lbytes) std::memcpy(lab + b * lbytes, labels_.data() + cursor_ * lbytes, run * lbytes);
      b += run;
      cursor_ += run;
      if (cursor_ == num_samples_) cursor_ = 0;
    }
    return;
  }
  for (uint64_t b = 0; b < batch; ++b) {
    const uint64_t i = order_[cursor_];
    std::memcpy(in + b * in_bytes, inputs_.data() + i * input_dim_, in_bytes);
    if (lab && lbytes) std::memcpy(lab + b * lbytes, labels_.data() + i * lbytes, lbytes);
    if (++cursor_ == num_samples_) {
      cursor_ = 0;
      Reshuffle();
      ++epoch_;
    }
  }
}

void Dataset::EnableShuffle(uint64_t seed) {
  // One splitmix step folds the seed so 0 is usable; the low bit keeps the
  // state nonzero ("shuffling on").
  shuffle_state_ = seed;
  shuffle_state_ = SplitMix64(&shuffle_state_) | 1ULL;
  shuffle_origin_ = shuffle_state_;
  epoch_ = 0;
  order_.resize(num_samples_);
  Reshuffle();
  cursor_ = 0;
}

void Dataset::Reshuffle() {
  for (uint64_t i = 0; i < num_samples_; ++i) order_[i] = i;
  for (uint64_t i = num_samples_ - 1; i > 0; --i) {
    const uint64_t j = SplitMix64(&shuffle_state_) % (i + 1);
    std::swap(order_[i], order_[j]);
  }
}

void Dataset::RestoreServingPos(ServingPos pos) {
  cursor_ = pos.cursor;
  if (order_.empty() || epoch_ == pos.epoch) return;
  // Each epoch's permutation is a function of (origin, epoch): replay.
  shuffle_state_ = shuffle_origin_;
  epoch_ = 0;
  Reshuffle();
  while (epoch_ < pos.epoch) {
    Reshuffle();
    ++epoch_;
  }
}

Status Dataset::SkipServed(uint64_t rows) {
  uint64_t records = rows;
  if (input_kind_ == 1) {
    if (rows % input_dim_ != 0)
      return Fail("served rows are not a whole number of token records — cannot replay the "
                  "serving position");
    records = rows / input_dim_;
  }
  RestoreServingPos({records % num_samples_, records / num_samples_});
  return Status::Ok();
}

Status Dataset::SplitValidation(double fraction, Dataset* val_out) {
  if (!(fraction > 0.0) || fraction >= 1.0) return Fail("validation fraction must be in (0, 1)");
  if (num_samples_ < 2) return Fail("too few samples to split");
  if (!order_.empty()) return Fail("split before enabling shuffle");
  uint64_t val_n = static_cast<uint64_t>(static_cast<double>(num_samples_) * fraction);
  if (val_n == 0) val_n = 1;
  if (val_n >= num_samples_) val_n = num_samples_ - 1;
  const uint64_t train_n = num_samples_ - val_n;
  const uint64_t lbytes = label_bytes_per_sample();

  Dataset val;
  val.num_samples_ = val_n;
  val.input_dim_ = input_dim_;
  val.label_kind_ = label_kind_;
  val.label_dim_ = label_dim_;
  val.input_kind_ = input_kind_;
  if (input_kind_ == 1) {
    // Whole records move: no sequence is cut.
    const uint64_t rec = input_dim_ + 1;
    val.tokens_.assign(tokens_.begin() + static_cast<std::ptrdiff_t>(train_n * rec), tokens_.end());
    tokens_.resize(train_n * rec);
  } else {
    val.inputs_.assign(inputs_.begin() + static_cast<std::ptrdiff_t>(train_n * input_dim_),
                       inputs_.end());
    val.labels_.assign(labels_.begin() + static_cast<std::ptrdiff_t>(train_n * lbytes),
                       labels_.end());
    inputs_.resize(train_n * input_dim_);
    labels_.resize(train_n * lbytes);
  }
  num_samples_ = train_n;
  cursor_ = 0;
  *val_out = std::move(val);
  return Status::Ok();
}

Status VerifyFeederContract(const PlanHeader& h, const Dataset& data, uint64_t num_classes,
                            uint64_t vocab_bound) {
  auto fail = [](const char* m) { return Status::Fail(kUnitEngine, m); };
  if (h.input_kind == 1) {
    if (data.input_kind() != 1)
      return fail("the compiled plan takes token ids, but the dataset carries feature rows");
    if (data.input_dim() != h.seq_len)
      return fail("dataset sequence length does not match the compiled plan");
    if (h.input_floats != h.batch)
      return fail("token plan input slot does not hold one id per batch row");
    if (h.label_kind == 1) {
      uint64_t want = 0;
      if (!MulOk(h.batch, sizeof(int32_t), &want) || want != h.label_bytes)
        return fail("token plan label slot does not hold one id per batch row");
    } else if (h.label_kind != 0) {
      return fail("token plans take class labels or none, not dense labels");
    }
    uint64_t bound = vocab_bound;
    if (num_classes != 0 && (bound == 0 || num_classes < bound)) bound = num_classes;
    return data.ValidateClassLabels(bound);
  }
  if (data.input_kind() != 0)
    return fail("the compiled plan takes feature rows, but the dataset carries token ids");
  uint64_t floats = 0;
  if (!MulOk(h.batch, data.input_dim(), &floats) || floats != h.input_floats)
    return fail("dataset input width does not match the compiled plan");
  if (h.label_kind != 0) {
    if (data.label_kind() != h.label_kind)
      return fail("dataset label kind does not match the compiled plan");
    uint64_t want = 0;
    if (!MulOk(h.batch, data.label_bytes_per_sample(), &want) || want != h.label_bytes)
      return fail("dataset label width does not match the compiled plan");
  }
  if (h.label_kind == 1) return data.ValidateClassLabels(num_classes);
  return Status::Ok();
}

}  // namespace seeml_hip
