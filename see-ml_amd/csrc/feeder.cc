// feeder.cc — the batch feeder's dataset, host side.
//
// A corpus is held exactly as the .sds sample section lays it out: one
// fixed-size record per sample — a feature row's f32 input followed by its
// label bytes, or a token record's seq + 1 i32 ids. Loading and saving are
// then one bulk transfer each, a validation split is a cut of one buffer,
// and one copy loop serves both kinds: a record's first input_dim * 4 bytes
// are the served input, and its label bytes sit right after them (feature
// rows) or one id further on (token records: the shifted next-token view).
//
// Serving walks a cursor over the records, through this epoch's permutation
// when shuffled. The permutation is the reference's (runtime/feeder/
// dataset.cc:344-417): Fisher–Yates from the identity, i = n-1 .. 1, each j
// the next splitmix64 draw mod (i + 1), a fresh one at every wrap. A
// splitmix64 state advances by the golden-ratio increment per draw and one
// permutation takes n - 1 draws, so epoch e's permutation starts at
// origin + e (n - 1) increments: any epoch is drawn directly, and restoring
// a serving position costs one permutation, not a replay of every epoch.
#include "feeder.h"

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <numeric>
#include <utility>

namespace seeml_hip {

namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ULL;  // splitmix64's state increment
constexpr uint64_t kSdsHeaderBytes = 40;

Status Fail(const std::string& m) { return Status::Fail(kUnitDataset, m); }

// The .sds header (40 bytes, little-endian).
struct SdsHeader {
  uint32_t magic, version;
  uint64_t num_samples, input_dim;
  uint32_t label_kind, input_kind;
  uint64_t label_dim;
};
static_assert(sizeof(SdsHeader) == kSdsHeaderBytes, "the .sds header is 40 bytes");

// Label bytes of one served sample (token records: one class id per
// position, the shifted view).
uint64_t ServedLabelBytes(uint32_t input_kind, uint32_t label_kind, uint64_t input_dim,
                          uint64_t label_dim) {
  if (input_kind == 1) return input_dim * sizeof(int32_t);
  if (label_kind == 1) return sizeof(int32_t);
  if (label_kind == 2) return label_dim * sizeof(float);
  return 0;
}

// A record's size, overflow-checked: token records are seq + 1 ids; a
// feature record is the input row followed by its label bytes.
bool RecordBytes(uint32_t input_kind, uint64_t input_dim, uint64_t label_bytes, uint64_t* out) {
  if (input_kind == 1) return input_dim < UINT64_MAX && MulOk(input_dim + 1, sizeof(int32_t), out);
  uint64_t in = 0;
  if (!MulOk(input_dim, sizeof(float), &in) || in > UINT64_MAX - label_bytes) return false;
  *out = in + label_bytes;
  return true;
}

int32_t IdAt(const uint8_t* p) {
  int32_t v;
  std::memcpy(&v, p, sizeof v);
  return v;
}

}  // namespace

uint64_t SplitMix64(uint64_t* state) {
  uint64_t z = (*state += kGolden);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

uint64_t Dataset::label_bytes_per_sample() const {
  return ServedLabelBytes(input_kind_, label_kind_, input_dim_, label_dim_);
}

Status Dataset::FromTokens(const int32_t* tokens, uint64_t count, uint64_t num_records,
                           uint64_t seq, Dataset* out) {
  if (num_records == 0) return Fail("zero samples");
  if (seq == 0) return Fail("zero input dim");
  uint64_t ids = 0;
  if (seq == UINT64_MAX || !MulOk(num_records, seq + 1, &ids) || count != ids)
    return Fail("token buffer size mismatch");
  const int32_t* neg = std::find_if(tokens, tokens + ids, [](int32_t t) { return t < 0; });
  if (neg != tokens + ids)
    return Fail("negative token id at position " + std::to_string(neg - tokens));
  Dataset d;
  d.input_kind_ = 1;
  d.label_kind_ = 1;
  d.num_samples_ = num_records;
  d.input_dim_ = seq;
  d.record_bytes_ = (seq + 1) * sizeof(int32_t);
  const uint8_t* bytes = reinterpret_cast<const uint8_t*>(tokens);
  d.records_.assign(bytes, bytes + ids * sizeof(int32_t));
  *out = std::move(d);
  return Status::Ok();
}

Status Dataset::FromMemory(const float* inputs, uint64_t input_count, const uint8_t* labels,
                           uint64_t label_bytes, uint64_t num_samples, uint64_t input_dim,
                           uint32_t label_kind, uint64_t label_dim, Dataset* out) {
  if (num_samples == 0) return Fail("zero samples");
  if (input_dim == 0) return Fail("zero input dim");
  if (label_kind > 2) return Fail("unknown label kind");
  if (label_kind == 2 && (label_dim == 0 || label_dim > UINT64_MAX / sizeof(float)))
    return Fail("label dim out of range");
  const uint64_t lb = ServedLabelBytes(0, label_kind, input_dim, label_dim);
  uint64_t floats = 0, lab_total = 0, rec = 0, total = 0;
  if (!MulOk(num_samples, input_dim, &floats) || input_count != floats)
    return Fail("input buffer size mismatch");
  if (!MulOk(num_samples, lb, &lab_total) || label_bytes != lab_total)
    return Fail("label buffer size mismatch");
  if (!RecordBytes(0, input_dim, lb, &rec) || !MulOk(num_samples, rec, &total))
    return Fail("input buffer size mismatch");
  Dataset d;
  d.num_samples_ = num_samples;
  d.input_dim_ = input_dim;
  d.label_kind_ = label_kind;
  d.label_dim_ = label_dim;
  d.record_bytes_ = rec;
  d.records_.resize(total);
  const uint64_t in_bytes = input_dim * sizeof(float);
  for (uint64_t i = 0; i < num_samples; ++i) {
    uint8_t* r = d.records_.data() + i * rec;
    std::memcpy(r, inputs + i * input_dim, in_bytes);
    if (lb) std::memcpy(r + in_bytes, labels + i * lb, lb);
  }
  *out = std::move(d);
  return Status::Ok();
}

Status Dataset::LoadFromFile(const std::string& path, Dataset* out) {
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f) return Fail("cannot open '" + path + "'");
  const std::streamoff end = f.tellg();
  if (end < 0) return Fail("cannot stat '" + path + "'");
  const uint64_t file_size = static_cast<uint64_t>(end);
  f.seekg(0);
  SdsHeader h{};
  f.read(reinterpret_cast<char*>(&h), sizeof h);
  const uint64_t got = static_cast<uint64_t>(std::max<std::streamsize>(f.gcount(), 0));
  // The header's fields are judged in file order: a file cut short inside
  // one reports that field.
  if (got < 4 || h.magic != kSdsMagic) return Fail("bad magic in '" + path + "'");
  if (got < 8 || h.version < 1 || h.version > 2) return Fail("unsupported version");
  if (got < kSdsHeaderBytes) return Fail("truncated header");
  if (h.num_samples == 0 || h.input_dim == 0) return Fail("empty dataset");
  if (h.label_kind > 2) return Fail("unknown label kind");
  if (h.label_kind == 2 && (h.label_dim == 0 || h.label_dim > UINT64_MAX / sizeof(float)))
    return Fail("label dim out of range");
  // v1's input_kind word was header padding (always 0).
  if (h.input_kind > 1 || (h.version < 2 && h.input_kind != 0)) return Fail("unknown input kind");
  if (h.input_kind == 1 && (h.label_kind != 1 || h.label_dim != 0))
    return Fail("token corpora derive next-token class labels (label_kind 1, label_dim 0)");
  const uint64_t lb = ServedLabelBytes(h.input_kind, h.label_kind, h.input_dim, h.label_dim);
  uint64_t rec = 0, payload = 0;
  if (!RecordBytes(h.input_kind, h.input_dim, h.input_kind == 1 ? 0 : lb, &rec) ||
      !MulOk(h.num_samples, rec, &payload) || payload > file_size - kSdsHeaderBytes)
    return Fail("sample section exceeds file size");
  if (payload > SIZE_MAX) return Fail("dataset too large for this host");
  Dataset d;
  d.num_samples_ = h.num_samples;
  d.input_dim_ = h.input_dim;
  d.label_kind_ = h.label_kind;
  d.input_kind_ = h.input_kind;
  d.label_dim_ = h.label_dim;
  d.record_bytes_ = rec;
  d.records_.resize(payload);
  f.read(reinterpret_cast<char*>(d.records_.data()), static_cast<std::streamsize>(payload));
  if (!f) return Fail("truncated inputs");
  if (h.input_kind == 1)
    for (uint64_t at = 0; at < payload; at += sizeof(int32_t))
      if (IdAt(d.records_.data() + at) < 0) return Fail("negative token id");
  *out = std::move(d);
  return Status::Ok();
}

Status Dataset::SaveToFile(const std::string& path) const {
  std::ofstream f(path, std::ios::binary | std::ios::trunc);
  if (!f) return Fail("cannot write '" + path + "'");
  const SdsHeader h{kSdsMagic, input_kind_ == 1 ? 2u : 1u, num_samples_, input_dim_,
                    label_kind_, input_kind_, label_dim_};
  f.write(reinterpret_cast<const char*>(&h), sizeof h);
  f.write(reinterpret_cast<const char*>(records_.data()),
          static_cast<std::streamsize>(records_.size()));
  f.close();  // the buffered tail is written here: judge the stream after it
  if (f.fail()) return Fail("short write to '" + path + "'");
  return Status::Ok();
}

Status Dataset::ValidateClassLabels(uint64_t num_classes) const {
  if (label_kind_ != 1 || num_classes == 0) return Status::Ok();
  auto outside = [&](int64_t v) { return v < 0 || static_cast<uint64_t>(v) >= num_classes; };
  const std::string bound = " outside [0, " + std::to_string(num_classes) + ")";
  if (input_kind_ == 1) {
    // Every id is an embedding index and, one position on, a class label.
    for (uint64_t at = 0; at < records_.size(); at += sizeof(int32_t))
      if (const int32_t v = IdAt(records_.data() + at); outside(v))
        return Fail("token id " + std::to_string(v) + " at position " +
                    std::to_string(at / sizeof(int32_t)) + bound);
    return Status::Ok();
  }
  for (uint64_t i = 0; i < num_samples_; ++i)
    if (const int32_t v = IdAt(Record(i) + LabelOffset()); outside(v))
      return Fail("class label " + std::to_string(v) + " at sample " + std::to_string(i) + bound);
  return Status::Ok();
}

void Dataset::Advance() {
  if (++cursor_ < num_samples_) return;
  cursor_ = 0;
  if (perm_.empty()) return;  // sequential serving wraps around
  ++epoch_;
  DrawPermutation();
}

void Dataset::FillBatch(uint64_t batch, void* input_slot, void* label_slot) {
  // Token corpora count `batch` in token rows: one record serves input_dim_.
  const uint64_t samples = input_kind_ == 1 ? batch / input_dim_ : batch;
  const uint64_t in_bytes = input_dim_ * 4, lab_bytes = label_bytes_per_sample();
  const uint64_t lab_off = LabelOffset();
  uint8_t* in = static_cast<uint8_t*>(input_slot);
  uint8_t* lab = lab_bytes ? static_cast<uint8_t*>(label_slot) : nullptr;
  for (uint64_t b = 0; b < samples; ++b) {
    const uint8_t* rec = Record(CurrentRecord());
    std::memcpy(in + b * in_bytes, rec, in_bytes);
    if (lab) std::memcpy(lab + b * lab_bytes, rec + lab_off, lab_bytes);
    Advance();
  }
}

void Dataset::DrawPermutation() {
  perm_.resize(num_samples_);
  std::iota(perm_.begin(), perm_.end(), uint64_t{0});
  uint64_t state = origin_ + epoch_ * (num_samples_ - 1) * kGolden;
  for (uint64_t i = num_samples_ - 1; i > 0; --i)
    std::swap(perm_[i], perm_[SplitMix64(&state) % (i + 1)]);
}

void Dataset::EnableShuffle(uint64_t seed) {
  // The seed goes through one splitmix64 step (so 0 is a usable seed), with
  // the low bit set (dataset.cc:356-366).
  uint64_t s = seed;
  origin_ = SplitMix64(&s) | 1ULL;
  epoch_ = 0;
  cursor_ = 0;
  DrawPermutation();
}

void Dataset::RestoreServingPos(ServingPos pos) {
  cursor_ = pos.cursor;
  if (perm_.empty() || epoch_ == pos.epoch) return;
  epoch_ = pos.epoch;
  DrawPermutation();
}

Status Dataset::SkipServed(uint64_t rows) {
  if (input_kind_ == 1 && rows % input_dim_ != 0)
    return Fail("served rows are not a whole number of token records — cannot replay the "
                "serving position");
  const uint64_t records = input_kind_ == 1 ? rows / input_dim_ : rows;
  RestoreServingPos({records % num_samples_, records / num_samples_});
  return Status::Ok();
}

Status Dataset::SplitValidation(double fraction, Dataset* val_out) {
  if (!(fraction > 0.0) || fraction >= 1.0) return Fail("validation fraction must be in (0, 1)");
  if (num_samples_ < 2) return Fail("too few samples to split");
  if (!perm_.empty()) return Fail("split before enabling shuffle");
  // The tail fraction of the records (whole records: no sequence is cut),
  // at least one on each side.
  const uint64_t val_n =
      std::clamp<uint64_t>(static_cast<uint64_t>(static_cast<double>(num_samples_) * fraction), 1,
                           num_samples_ - 1);
  const uint64_t cut = (num_samples_ - val_n) * record_bytes_;
  Dataset val;
  val.record_bytes_ = record_bytes_;
  val.num_samples_ = val_n;
  val.input_dim_ = input_dim_;
  val.label_kind_ = label_kind_;
  val.input_kind_ = input_kind_;
  val.label_dim_ = label_dim_;
  val.records_.assign(records_.begin() + static_cast<std::ptrdiff_t>(cut), records_.end());
  records_.resize(cut);
  records_.shrink_to_fit();
  num_samples_ -= val_n;
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
