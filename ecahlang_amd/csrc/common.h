// Shared device helpers for the paged-KV kernels (gfx950, wave64).
//
// Cache layout (NHD, one tensor per layer, the form the reference manager allocates at
// ecahlang/manager.py:51-54):  cache[page][kv][slot][head][dim], kv = 0 for K and 1 for V.
// Every kernel addresses K and V through two base pointers plus a page stride, so the
// single-tensor form (V base = K base + page_size*Hkv*D, page stride = 2*page_size*Hkv*D)
// and a split (k_cache, v_cache) pair (page stride = page_size*Hkv*D) share one code path.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

namespace pkv {

enum DType : int32_t { kF16 = 0, kBF16 = 1, kF32 = 2 };

constexpr int kWave = 64;

// Error codes returned through the C ABI (0 = success, >0 = hipError_t, <0 = argument error).
enum Err : int32_t {
  kOk = 0,
  kBadDType = -1,
  kBadHeadDim = -2,
  kBadGroup = -3,
  kBadAlign = -4,
  kBadArg = -5,
  kWorkspaceTooSmall = -6,
  kBadPageSize = -7,
};

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(_Float16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(__hip_bfloat16 x) { return __bfloat162float(x); }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float x) { return (_Float16)x; }
template <> __device__ __forceinline__ __hip_bfloat16 from_f32<__hip_bfloat16>(float x) {
  return __float2bfloat16(x);  // round-to-nearest-even, as torch's .to(bfloat16)
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Largest b in [0, n) with a[b] <= x, for a non-decreasing a[0..n]; a[0] <= x assumed.
__device__ __forceinline__ int upper_index(const int32_t* a, int n, int64_t x) {
  int lo = 0, hi = n;  // invariant: a[lo] <= x, answer in [lo, hi)
  while (hi - lo > 1) {
    int mid = (lo + hi) >> 1;
    if ((int64_t)a[mid] <= x) lo = mid; else hi = mid;
  }
  return lo;
}

}  // namespace pkv
