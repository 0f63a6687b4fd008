// Matrix-core building blocks shared by the paged decode and prefill kernels (gfx950).
//
//   Mma<T>::qk   v_mfma_f32_16x16x32_{f16,bf16}: 16x16 fp32 tile += A (16 x 32) * B (32 x 16);
//                lane l supplies row/column l % 16, reduction elements 8*(l/16) .. +7
//   Mma<T>::pv   v_mfma_f32_16x16x16{f16,bf16_1k}: reduction elements 4*(l/16) .. +3
//   Accumulator layout (both): lane l holds C[4*(l/16) + i][l % 16], i = 0..3.
//   lds_read_tr16 + vswz: the V^T operand of the P.V product read straight from a row-major,
//   XOR-swizzled LDS copy of 16 value rows.
#pragma once
#include "common.h"

namespace pkv {
namespace mfma {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
// 16 bytes as a plain vector (arrays of it stay in registers; arrays of the uint4 struct copied
// to and from memory may be left in scratch)
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

template <typename To, typename From>
__device__ __forceinline__ To bitcast_(const From& x) {
  static_assert(sizeof(To) == sizeof(From), "size");
  To y;
  __builtin_memcpy(&y, &x, sizeof(To));
  return y;
}

template <typename T> struct Mma;
template <> struct Mma<_Float16> {
  static __device__ __forceinline__ f4 qk(uint4 a, uint4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast_<h8>(a), bitcast_<h8>(b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f4 pv(uint2 a, uint2 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(bitcast_<h4>(a), bitcast_<h4>(b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float x, float y) {  // v_cvt_pk_f16_f32
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return bitcast_<uint32_t>(__builtin_convertvector((f2{x, y}), h2));
  }
};
template <> struct Mma<__hip_bfloat16> {
  static __device__ __forceinline__ f4 qk(uint4 a, uint4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(bitcast_<bf8>(a), bitcast_<bf8>(b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f4 pv(uint2 a, uint2 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bitcast_<s4>(a), bitcast_<s4>(b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float x, float y) {  // v_cvt_pk_bf16_f32
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return bitcast_<uint32_t>(__builtin_convertvector((f2{x, y}), b2));
  }
};

// Chunk swizzle of the staged V tile: 16-byte chunk c of token row t lives at c ^ vswz(t).
// Row writes (one row per 16 lanes) stay 16-byte aligned and conflict-free, and the
// transposing operand read (rows 4g..4g+3, 32 bytes each, per 16-lane group g) lands the
// four rows of a group, and the two groups of a 32-lane half, on disjoint banks.
template <int D>
__device__ __forceinline__ int vswz(int t) {
  return D == 128 ? 2 * (t & 7) : 2 * ((t >> 1) & 3);
}

// Chunk swizzle of a staged K tile: 16-byte chunk c of key row t lives at c ^ kswz(t).  The
// A-operand read (16 keys, one chunk per 16-lane group) then touches 16 distinct 16-byte bank
// groups: rows are 256 B (D = 128: one full bank cycle per row, so XOR by t) or 128 B (D = 64:
// row parity picks the half, XOR by t / 2 within it).
template <int D>
__device__ __forceinline__ int kswz(int t) {
  return D == 128 ? (t & 15) : ((t >> 1) & 7);
}

typedef short s4v __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element (i & 3) of the
// 8-byte rows addressed by lanes 4j + (i >> 2), j = 0..3.  With lane i of group g pointing
// at V[4g + i/4][16*mt + 4*(i%4)], lane i gets V[4g + j][16*mt + i]: the V^T operand of the
// 16x16x16 P.V product, in one instruction.
__device__ __forceinline__ uint2 lds_read_tr16(const char* p) {
  s4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s4v*)(p));
  uint2 u;
  __builtin_memcpy(&u, &r, sizeof(u));
  return u;
}

// Maxima without the canonicalising copies IEEE mode adds around fmaxf (the inputs are matrix-core
// results or -inf, never signalling NaNs).
__device__ __forceinline__ float max2f(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
template <int N>
__device__ __forceinline__ float max_of(const float* v) {
  static_assert(N == 16, "max_of");
  const float a = max3f(max3f(v[0], v[1], v[2]), max3f(v[3], v[4], v[5]), max3f(v[6], v[7], v[8]));
  const float b = max3f(max3f(v[9], v[10], v[11]), max3f(v[12], v[13], v[14]), v[15]);
  return max2f(a, b);
}
// Maximum and sum over the four 16-lane groups (lanes l, l ^ 16, l ^ 32, l ^ 48) by two lane
// swaps in registers (v_permlane16_swap: odd rows with even rows; v_permlane32_swap: the two
// halves), where a shuffle would take two LDS round trips.  Every lane gets the result; all 64
// lanes must be active.  The sum adds l ^ 16 first, then l ^ 32, as a shuffle-based
// x + x^16, then + ^32 does, with the same operands, so it is bit-identical to that.
__device__ __forceinline__ float max_across_groups(float x) {
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = max2f(__uint_as_float(h[0]), __uint_as_float(h[1]));
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max2f(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_across_groups(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(h[0]) + __uint_as_float(h[1]);
}

}  // namespace mfma
}  // namespace pkv
