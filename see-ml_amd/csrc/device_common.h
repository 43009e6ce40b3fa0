// device_common.h — shared device helpers for the gfx950 kernels.
//
// Determinism: every reduction here is a fixed tree (per-thread sequential
// partial in a fixed element assignment, then an xor-butterfly across the
// 64-lane wavefront, then wavefront partials combined in index order through
// LDS). No float atomics anywhere, so every launch of the same shape produces
// the same bits.
//
// All device code is compiled with -ffp-contract=off: an expression rounds
// where it is written, which is what lets the elementwise, AdamW, bias and
// loss-backward kernels reproduce the CPU executor's bits exactly.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace seeml_hip {

inline constexpr int kWave = 64;

// The activation expressions of kernel_policy.h:47-67, restated for device.
// expf/tanhf here are the device library's, so these match the CPU bits only
// to within a few ulp (the libm boundary is tolerance-only by design).
__device__ __forceinline__ float dev_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float dev_relu(float x) { return x > 0.0f ? x : 0.0f; }
__device__ __forceinline__ float dev_gelu(float x) {
  const float t = tanhf(0.7978845608028654f * (x + 0.044715f * x * x * x));
  return 0.5f * x * (1.0f + t);
}
__device__ __forceinline__ float dev_silu(float x) { return x * dev_sigmoid(x); }
__device__ __forceinline__ float dev_act(int act, float v) {
  switch (act) {
    case 1: return dev_relu(v);
    case 2: return dev_gelu(v);
    case 3: return dev_silu(v);
    default: return v;
  }
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Block-wide sum over NT threads (NT a multiple of 64); every thread gets the
// total. `scratch` holds NT/64 elements of T.
template <typename T, int NT>
__device__ __forceinline__ T block_sum(T v, T* scratch) {
  v = wave_sum(v);
  constexpr int kWaves = NT / kWave;
  if constexpr (kWaves == 1) {
    return v;
  } else {
    const int w = threadIdx.x / kWave;
    __syncthreads();
    if ((threadIdx.x % kWave) == 0) scratch[w] = v;
    __syncthreads();
    T t = scratch[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) t += scratch[i];
    return t;
  }
}

template <int NT>
__device__ __forceinline__ float block_max(float v, float* scratch) {
  v = wave_max(v);
  constexpr int kWaves = NT / kWave;
  if constexpr (kWaves == 1) {
    return v;
  } else {
    const int w = threadIdx.x / kWave;
    __syncthreads();
    if ((threadIdx.x % kWave) == 0) scratch[w] = v;
    __syncthreads();
    float t = scratch[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) t = fmaxf(t, scratch[i]);
    return t;
  }
}

// Streaming 16-byte accesses: non-temporal loads and stores (vector memory
// instructions with the streaming cache policy). On streams larger than the
// 256 MiB memory-side cache they give ~20% more HBM throughput than
// default-policy float4; below that size the default policy wins overall,
// because it leaves a freshly written tensor in the cache for its consumer
// (the next GEMM reads it back from there). kStreamBytes is the switch.
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_stream(const float* p) {
  const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_stream(float* p, float4 v) {
  const f32x4 t = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(t, reinterpret_cast<f32x4*>(p));
}

__device__ __forceinline__ float4 ld4(const float* p, bool nt) {
  return nt ? ld_stream(p) : *reinterpret_cast<const float4*>(p);
}
__device__ __forceinline__ void st4(float* p, float4 v, bool nt) {
  if (nt) st_stream(p, v);
  else *reinterpret_cast<float4*>(p) = v;
}
inline constexpr size_t kStreamBytes = size_t{256} << 20;
// Streaming policy for a kernel moving `traffic` bytes in total.
inline bool StreamPolicy(size_t traffic) { return traffic > kStreamBytes; }

__host__ __device__ inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline unsigned grid_for(size_t work_items, int block, size_t cap = 65536) {
  size_t g = (work_items + block - 1) / block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return static_cast<unsigned>(g);
}

}  // namespace seeml_hip
