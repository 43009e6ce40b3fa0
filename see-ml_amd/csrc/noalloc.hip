// noalloc.hip — GemmTN for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).
//
// seeml_hip_gemm_tn takes its scratch (the skinny colsum kernels' k-group
// partials, split-K partials) from a library workspace that grows with
// hipMalloc on demand. This variant takes it from `scratch`, a file-scope
// device array of kNoAllocScratchBytes that each GPU holds from the
// library's load until the process ends. Its device address is looked up
// once per device with hipGetSymbolAddress (the array's name is a host-side
// stand-in, never a device address) and kept per device. The plan and the
// kernels are seeml_hip_gemm_tn's, so the results are bit for bit the same.
//
// Every call on one GPU shares that GPU's array. The kernels write every
// scratch byte they later read (each k-group partial and split-K slice is
// stored whole before the reduction reads it), so nothing needs clearing
// between calls; calls that overlap on one GPU (two streams, two threads)
// race on it.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <string>

#include "../../include/seeml_hip.h"
#include "kernels.h"

namespace seeml_hip {
namespace {

constexpr size_t kNoAllocScratchBytes = size_t{SEEML_HIP_NOALLOC_SCRATCH_BYTES};

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

struct ScratchTable {
  std::mutex mu;
  std::map<int, void*> ptr;  // device ordinal -> the device address of `scratch`
};

ScratchTable& Table() {
  static ScratchTable t;
  return t;
}

// The calling thread's current device's copy of `scratch`: looked up with
// hipGetSymbolAddress on the first call on that device, with the device
// current, then reused.
Status ScratchOfCurrentDevice(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess)
    return Status::Fail(kUnitEngine, "GemmTN(no-alloc): hipGetDevice failed");
  ScratchTable& t = Table();
  std::lock_guard<std::mutex> lock(t.mu);
  auto it = t.ptr.find(dev);
  if (it != t.ptr.end()) {
    *out = it->second;
    return Status::Ok();
  }
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr)
    return Status::Fail(kUnitEngine, std::string("GemmTN(no-alloc): hipGetSymbolAddress failed: ") +
                                         hipGetErrorString(e));
  t.ptr.emplace(dev, p);
  *out = p;
  return Status::Ok();
}

}  // namespace
}  // namespace seeml_hip

extern "C" int seeml_hip_gemm_tn_noalloc(const float* A, const float* B, float* C, uint64_t M,
                                         uint64_t N, uint64_t K, void* stream) {
  using namespace seeml_hip;
  const GemmDesc d = GemmTNDesc(A, B, C, static_cast<int64_t>(M), static_cast<int64_t>(N),
                                static_cast<int64_t>(K));
  // The same plan as seeml_hip_gemm_tn (the heuristic: skinny colsum for
  // LoRA gradients, the tile kernels with their deterministic split-K count
  // otherwise).
  const GemmPlan plan = PlanGemmWith(d, -1, -1);
  if (plan.ws_bytes > kNoAllocScratchBytes)
    return ReportStandalone(Status::Fail(
        kUnitEngine, "GemmTN(no-alloc): this shape needs " + std::to_string(plan.ws_bytes) +
                         " bytes of scratch, more than the " +
                         std::to_string(kNoAllocScratchBytes) + " the no-allocation entry point holds"));
  Ctx ctx;
  ctx.stream = static_cast<hipStream_t>(stream);
  if (Status s = ScratchOfCurrentDevice(&ctx.ws); !s) return ReportStandalone(s);
  ctx.ws_bytes = kNoAllocScratchBytes;
  return ReportStandalone(LaunchGemm(d, plan, ctx));
}
