// fuzz_formats.cc — TEST INFRASTRUCTURE ONLY. A seeded mutation harness over
// the three parsers that take untrusted bytes (the roles of
// test/fuzz/binary_formats.cc): the .seeu plan loader + validator
// (DecodeAndVerifyPlan), the .sds corpus reader (Dataset::LoadFromFile) and
// the SEKP checkpoint reader (ReadCheckpoint). Built by tests/test_fuzz_formats.py
// with AddressSanitizer and UBSan from the backend's host-only sources.
//
// Contract under test: any byte string may be rejected but must never crash,
// over-read or overflow, and every rejection is one "<unit>: <message>" line
// naming the parser's unit. Like the reference harness, a mutated plan is
// re-sealed with PlanSelfHash (most of the time) so mutations reach the
// validators behind the integrity hash.
//
// usage: fuzz_formats <seed-dir> <iterations per seed> <rng seed>
//   seed files: *.seeu (plans), *.sds (corpora), *.sekp (checkpoints; the
//   file name carries the plan hash and payload size: <hash>_<size>.sekp)
#include <dirent.h>
#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <random>
#include <string>
#include <vector>

#include "../../see-ml_amd/csrc/checkpoint.h"
#include "../../see-ml_amd/csrc/feeder.h"
#include "../../see-ml_amd/csrc/plan_checks.h"

using namespace seeml_hip;

namespace {

std::vector<uint8_t> ReadFile(const std::string& p) {
  std::ifstream f(p, std::ios::binary);
  return std::vector<uint8_t>(std::istreambuf_iterator<char>(f), {});
}

void WriteFile(const std::string& p, const std::vector<uint8_t>& b) {
  std::ofstream f(p, std::ios::binary | std::ios::trunc);
  f.write(reinterpret_cast<const char*>(b.data()), static_cast<std::streamsize>(b.size()));
}

// One of several mutation families, chosen by the generator.
void Mutate(std::vector<uint8_t>& b, std::mt19937_64& g) {
  if (b.empty()) {
    b.push_back(static_cast<uint8_t>(g()));
    return;
  }
  const uint64_t specials[] = {0,          1,          2,          63,         64,
                               0xFFFFFFFF, 0x100000000ULL, UINT64_MAX, UINT64_MAX - 1,
                               1ULL << 63, b.size(),   b.size() - 1, b.size() + 64};
  const int rounds = 1 + static_cast<int>(g() % 4);
  for (int r = 0; r < rounds; ++r) {
    switch (g() % 7) {
      case 0:  // flip a bit
        b[g() % b.size()] ^= static_cast<uint8_t>(1u << (g() % 8));
        break;
      case 1:  // overwrite a byte
        b[g() % b.size()] = static_cast<uint8_t>(g());
        break;
      case 2: {  // an aligned u64 field, mostly in the headers, to a boundary value
        const uint64_t span = std::min<uint64_t>(b.size(), (g() % 2) ? 320 : b.size());
        if (span < 8) break;
        const uint64_t at = (g() % (span / 8)) * 8;
        const uint64_t v = specials[g() % (sizeof specials / sizeof specials[0])];
        std::memcpy(b.data() + at, &v, 8);
        break;
      }
      case 3: {  // an aligned u32 field to a boundary value
        if (b.size() < 4) break;
        const uint64_t at = (g() % (b.size() / 4)) * 4;
        const uint32_t v = static_cast<uint32_t>(specials[g() % (sizeof specials / sizeof specials[0])]);
        std::memcpy(b.data() + at, &v, 4);
        break;
      }
      case 4:  // truncate
        b.resize(g() % (b.size() + 1));
        if (b.empty()) return;
        break;
      case 5:  // append garbage
        for (int k = static_cast<int>(g() % 64); k > 0; --k) b.push_back(static_cast<uint8_t>(g()));
        break;
      default: {  // copy a random 64-byte block over another (instruction soup)
        if (b.size() < 128) break;
        const uint64_t from = g() % (b.size() - 64), to = g() % (b.size() - 64);
        std::memmove(b.data() + to, b.data() + from, 64);
        break;
      }
    }
  }
}

bool WellFormed(const std::string& e, const char* unit) {
  const std::string want = std::string(unit) + ": ";
  return e.size() > want.size() && e.compare(0, want.size(), want) == 0 &&
         e.find('\n') == std::string::npos;
}

bool WellFormedAny(const std::string& e, std::initializer_list<const char*> units) {
  for (const char* u : units)
    if (WellFormed(e, u)) return true;
  return false;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 4) {
    std::fprintf(stderr, "usage: %s <seed-dir> <iterations> <rng-seed>\n", argv[0]);
    return 2;
  }
  const std::string dir = argv[1];
  const long iters = std::atol(argv[2]);
  std::mt19937_64 g(std::strtoull(argv[3], nullptr, 10));
  const std::string tmp = dir + "/mutant_" + std::to_string(::getpid());
  long rejected[3] = {0, 0, 0}, accepted[3] = {0, 0, 0};
  DIR* d = ::opendir(dir.c_str());
  if (!d) return 2;
  std::vector<std::string> seeds;
  while (dirent* e = ::readdir(d)) seeds.push_back(e->d_name);
  ::closedir(d);
  for (const std::string& name : seeds) {
    const std::string path = dir + "/" + name;
    int kind = -1;
    if (name.size() > 5 && name.compare(name.size() - 5, 5, ".seeu") == 0) kind = 0;
    if (name.size() > 4 && name.compare(name.size() - 4, 4, ".sds") == 0) kind = 1;
    if (name.size() > 5 && name.compare(name.size() - 5, 5, ".sekp") == 0) kind = 2;
    if (kind < 0) continue;
    const std::vector<uint8_t> seed = ReadFile(path);
    uint64_t ck_hash = 0, ck_size = 0;
    if (kind == 2 && std::sscanf(name.c_str(), "%lx_%lu", &ck_hash, &ck_size) != 2) return 2;
    for (long it = 0; it < iters; ++it) {
      std::vector<uint8_t> b = seed;
      Mutate(b, g);
      std::string err;
      if (kind == 0) {
        if (b.size() >= sizeof(PlanHeader) && g() % 10 != 0) {
          const uint64_t h = PlanSelfHash(b.data(), b.size(), offsetof(PlanHeader, plan_hash));
          std::memcpy(b.data() + offsetof(PlanHeader, plan_hash), &h, 8);
        }
        DecodedPlan out;
        const Status s = DecodeAndVerifyPlan(b.data(), b.size(), &out);
        if (!s && !WellFormedAny(s.error, {kUnitEngine, kUnitValidator})) err = s.error;
        (s ? accepted : rejected)[0]++;
      } else if (kind == 1) {
        WriteFile(tmp, b);
        Dataset ds;
        const Status s = Dataset::LoadFromFile(tmp, &ds);
        if (!s && !WellFormed(s.error, kUnitDataset)) err = s.error;
        if (s) {
          // An accepted corpus is served: two epochs, shuffled.
          const uint64_t per = ds.input_kind() == 1 ? ds.input_dim() : 1;
          const uint64_t batch = per * 3;
          std::vector<uint8_t> in(batch * ds.input_dim() * 4 / per + 64);
          std::vector<uint8_t> lab(3 * ds.label_bytes_per_sample() + 64);
          ds.EnableShuffle(g());
          for (uint64_t k = 0; k < 2 * ds.num_samples() / 3 + 1; ++k)
            ds.FillBatch(batch, in.data(), lab.data());
          (void)ds.ValidateClassLabels(1 + g() % 1000);
        }
        (s ? accepted : rejected)[1]++;
      } else {
        WriteFile(tmp, b);
        std::vector<uint8_t> dst(ck_size);
        uint64_t step = 0;
        const Status s = ReadCheckpoint(tmp, ck_hash, ck_size, dst.data(), &step);
        if (!s && !WellFormed(s.error, kUnitCheckpoint)) err = s.error;
        (s ? accepted : rejected)[2]++;
      }
      if (!err.empty()) {
        std::fprintf(stderr, "malformed diagnostic from %s (iteration %ld): '%s'\n", name.c_str(),
                     it, err.c_str());
        std::remove(tmp.c_str());
        return 1;
      }
    }
  }
  std::remove(tmp.c_str());
  std::printf("plans rejected %ld accepted %ld | corpora rejected %ld accepted %ld | "
              "checkpoints rejected %ld accepted %ld\n",
              rejected[0], accepted[0], rejected[1], accepted[1], rejected[2], accepted[2]);
  return 0;
}
