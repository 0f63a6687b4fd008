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

// Whole-wave reductions in registers (no LDS round trips): within each 16-lane row by DPP row
// rotations (after rotating by 8, 4, 2 and 1 every lane holds its row's total), then across rows
// by v_permlane16_swap (odd rows with even rows) and v_permlane32_swap (the two halves).  Every
// lane gets the result.  All 64 lanes must be active.  Integer results do not depend on the
// order, so they equal any other reduction's.
namespace wred {
template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
constexpr int kRor8 = 0x128, kRor4 = 0x124, kRor2 = 0x122, kRor1 = 0x121;  // row_ror:n
template <typename Op>
__device__ __forceinline__ uint32_t reduce_u32(uint32_t v, Op op) {
  v = op(v, dpp<kRor8>(v));
  v = op(v, dpp<kRor4>(v));
  v = op(v, dpp<kRor2>(v));
  v = op(v, dpp<kRor1>(v));
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = op((uint32_t)r[0], (uint32_t)r[1]);
  const auto h = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return op((uint32_t)h[0], (uint32_t)h[1]);
}
}  // namespace wred
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  return wred::reduce_u32(v, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}
__device__ __forceinline__ float wave_max_f32(float v) {  // (fmaxf: NaN only when every lane is NaN)
  return __uint_as_float(wred::reduce_u32(__float_as_uint(v), [](uint32_t a, uint32_t b) {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  }));
}
__device__ __forceinline__ int wave_sum_i32(int v) {
  return (int)wred::reduce_u32((uint32_t)v, [](uint32_t a, uint32_t b) { return a + b; });
}
__device__ __forceinline__ uint64_t wave_sum_u64_dpp(uint64_t v) {
  auto step = [&](auto fetch) __attribute__((always_inline)) {
    const uint32_t lo = fetch((uint32_t)v), hi = fetch((uint32_t)(v >> 32));
    v += ((uint64_t)hi << 32) | lo;
  };
  step([](uint32_t x) { return wred::dpp<wred::kRor8>(x); });
  step([](uint32_t x) { return wred::dpp<wred::kRor4>(x); });
  step([](uint32_t x) { return wred::dpp<wred::kRor2>(x); });
  step([](uint32_t x) { return wred::dpp<wred::kRor1>(x); });
  {
    const auto rl = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
    const auto rh = __builtin_amdgcn_permlane16_swap((uint32_t)(v >> 32), (uint32_t)(v >> 32), false, false);
    v = (((uint64_t)(uint32_t)rh[0] << 32) | (uint32_t)rl[0]) + (((uint64_t)(uint32_t)rh[1] << 32) | (uint32_t)rl[1]);
  }
  {
    const auto hl = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    const auto hh = __builtin_amdgcn_permlane32_swap((uint32_t)(v >> 32), (uint32_t)(v >> 32), false, false);
    v = (((uint64_t)(uint32_t)hh[0] << 32) | (uint32_t)hl[0]) + (((uint64_t)(uint32_t)hh[1] << 32) | (uint32_t)hl[1]);
  }
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
