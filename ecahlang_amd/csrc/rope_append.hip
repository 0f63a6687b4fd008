// Rotary position embedding fused with the K/V append: the model's apply_rotary_pos_emb on
// the new tokens' q and k (transformers/models/qwen2/modeling_qwen2.py:210-211, called in
// Qwen2Attention.forward just before the attention hook), then the hook's append
// (ecahlang/main.py:62-66 -> flashinfer.page.append_paged_kv_cache), in one launch.
//
//   pkv_append_paged_kv_cache_rope  <- apply_rotary_pos_emb + append_paged_kv_cache
//
// Query rows are rotated into q_out (which may alias q); key rows are rotated and written
// straight into their pages; value rows are copied into their pages.  The rotated keys never
// make a separate round trip through HBM.  The rotation is the model's non-interleaved one,
// rotate_half(x) = cat(-x[D/2:], x[:D/2]):
//   out[d]       = x[d] * cos[d]             + (-x[d + D/2]) * sin[d]         d < D/2
//   out[d + D/2] = x[d + D/2] * cos[d + D/2] + x[d] * sin[d + D/2]
// where cos / sin are the token's rows of the model's position embeddings, already in the
// activations' dtype.  Every product is rounded to that dtype and then the sum is rounded,
// which is how the model's eager tensor ops round.  That keeps the result bit-identical to
// the model's own rotation followed by the plain append.
//
// There is one lane per (token, row, run of N dims d .. d+N-1 in the first half), N = 16 bytes
// of elements (4 on the element path for unaligned views).  The lane loads those dims and
// their partners d + D/2 .. d + D/2 + N-1, and writes both.  Rows are
// ordered Hq query rows, then Hkv key rows, then Hkv value rows.  Index order, fastest first:
// dim group, row, token.
#include "common.h"
#include "../../include/pagedkv.h"

#include <type_traits>

using namespace pkv;

namespace {

template <typename T>
__device__ __forceinline__ float rnd(float x) {  // round to T and back
  return to_f32(from_f32<T>(x));
}

// N consecutive elements; one 16-byte access when VEC (pointers and strides aligned to N
// elements, N * sizeof(T) == 16), else N element accesses.
template <typename T, int N, bool VEC>
struct Run {
  T e[N];
  __device__ __forceinline__ void load(const T* p) {
    if constexpr (VEC) {
      static_assert(N * sizeof(T) == 16, "one 16-byte vector");
      const uint4 w = *reinterpret_cast<const uint4*>(p);
      __builtin_memcpy(e, &w, 16);
    } else {
#pragma unroll
      for (int j = 0; j < N; ++j) e[j] = p[j];
    }
  }
  __device__ __forceinline__ void store(T* p) const {
    if constexpr (VEC) {
      uint4 w;
      __builtin_memcpy(&w, e, 16);
      *reinterpret_cast<uint4*>(p) = w;
    } else {
#pragma unroll
      for (int j = 0; j < N; ++j) p[j] = e[j];
    }
  }
};

// The token's cos / sin at dims d0.. and d0 + D/2..
template <typename T, int N, bool VEC>
struct CosSin {
  Run<T, N, VEC> c0, c1, s0, s1;
  __device__ __forceinline__ void load(const T* cs, const T* sn, int half) {
    c0.load(cs);
    c1.load(cs + half);
    s0.load(sn);
    s1.load(sn + half);
  }
};

// lo / hi: dims d0.. and d0 + D/2.. of one row, rotated in place with the token's cos / sin.
template <typename T, int N, bool VEC>
__device__ __forceinline__ void rotate(Run<T, N, VEC>& lo, Run<T, N, VEC>& hi, const CosSin<T, N, VEC>& t) {
#pragma clang fp contract(off)
  const Run<T, N, VEC>&c0 = t.c0, &c1 = t.c1, &s0 = t.s0, &s1 = t.s1;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const float a = to_f32(lo.e[j]), b = to_f32(hi.e[j]);
    // rounding is sign-symmetric, so x*cos + round(-x2*sin) == x*cos - round(x2*sin)
    const float x = rnd<T>(a * to_f32(c0.e[j])) - rnd<T>(b * to_f32(s0.e[j]));
    const float y = rnd<T>(b * to_f32(c1.e[j])) + rnd<T>(a * to_f32(s1.e[j]));
    lo.e[j] = from_f32<T>(x);
    hi.e[j] = from_f32<T>(y);
  }
}

template <typename T, int N, bool VEC>
__global__ void rope_append_kernel(const T* q, int64_t q_sn, int64_t q_sh, T* q_out, int64_t qo_sn, int64_t qo_sh,
                                   int32_t hq, const T* __restrict__ k, int64_t k_sn, int64_t k_sh,
                                   const T* __restrict__ v, int64_t v_sn, int64_t v_sh, const T* __restrict__ cos_,
                                   const T* __restrict__ sin_, int64_t cs_sn, const int32_t* __restrict__ bidx,
                                   const int32_t* __restrict__ pos, int32_t nnz, T* __restrict__ k_cache,
                                   T* __restrict__ v_cache, int64_t page_stride, int64_t num_pages,
                                   const int32_t* __restrict__ kv_indices, int64_t num_indices,
                                   const int32_t* __restrict__ kv_indptr, int32_t batch, int32_t hkv, int32_t d,
                                   int32_t ps, int32_t* __restrict__ err) {
  const int half = d / 2, groups = half / N, rows = hq + 2 * hkv;
  const int64_t total = (int64_t)nnz * rows * groups;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int d0 = N * (int)(idx % groups);
    const int64_t r0 = idx / groups;
    const int row = (int)(r0 % rows);
    const int64_t i = r0 / rows;
    Run<T, N, VEC> lo, hi;
    CosSin<T, N, VEC> cs;
    if (row < hq) {  // query row: rotated into q_out
      const T* src = q + i * q_sn + row * q_sh + d0;
      lo.load(src);
      hi.load(src + half);
      cs.load(cos_ + i * cs_sn + d0, sin_ + i * cs_sn + d0, half);
      rotate(lo, hi, cs);
      T* dst = q_out + i * qo_sn + row * qo_sh + d0;
      lo.store(dst);
      hi.store(dst + half);
      continue;
    }
    const bool is_v = row - hq >= hkv;
    const int h = is_v ? row - hq - hkv : row - hq;
    // The row and the token's cos / sin (read for value rows too, unused, so that no load
    // sits under a divergent branch) are requested before the page-table lookups, which they
    // do not depend on; the empty asm keeps the compiler from sinking them behind those.
    const T* src = is_v ? v + i * v_sn + h * v_sh + d0 : k + i * k_sn + h * k_sh + d0;
    lo.load(src);
    hi.load(src + half);
    cs.load(cos_ + i * cs_sn + d0, sin_ + i * cs_sn + d0, half);
    asm volatile("" ::: "memory");
    const int b = bidx[i], p = pos[i];
    bool ok = b >= 0 && b < batch && p >= 0;
    int page = -1;
    if (ok) {
      const int base = kv_indptr[b], np = kv_indptr[b + 1] - base, pi = p / ps;
      ok = pi < np && (int64_t)base + pi < num_indices;
      if (ok) {
        page = kv_indices[base + pi];
        ok = page >= 0 && page < num_pages;
      }
    }
    if (!ok) {  // metadata outside the sequence's pages: skipped, counted once per token
      if (row == hq && d0 == 0 && err) atomicAdd(err, 1);
      continue;
    }
    T* dst = (is_v ? v_cache : k_cache) + page * page_stride + ((int64_t)(p % ps) * hkv + h) * d + d0;
    if (!is_v) rotate(lo, hi, cs);
    lo.store(dst);
    hi.store(dst + half);
  }
}

}  // namespace

extern "C" int pkv_append_paged_kv_cache_rope(
    const void* q, int64_t q_stride_n, int64_t q_stride_h, void* q_out, int64_t qo_stride_n, int64_t qo_stride_h,
    int32_t num_qo_heads, const void* append_key, int64_t k_stride_n, int64_t k_stride_h, const void* append_value,
    int64_t v_stride_n, int64_t v_stride_h, const void* cos, const void* sin, int64_t cs_stride_n,
    const int32_t* batch_indices, const int32_t* positions, int32_t nnz, void* k_cache, void* v_cache,
    int64_t page_stride, int64_t num_pages, const int32_t* kv_indices, int64_t num_indices, const int32_t* kv_indptr,
    int32_t batch, int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int32_t dtype, int32_t* err_count,
    void* stream) {
  const int es = dtype == kF32 ? 4 : (dtype == kF16 || dtype == kBF16) ? 2 : 0;
  if (!es) return kBadDType;
  if (nnz < 0 || num_qo_heads < 0 || num_kv_heads <= 0 || page_size <= 0 || batch < 0) return kBadArg;
  if (head_dim <= 0 || head_dim % 8) return kBadHeadDim;
  if (nnz == 0) return kOk;
  // 16-byte pieces (N = 16 / element size dims from each half per lane) when every pointer and
  // stride allows it, else 4 elements at a time with element accesses.
  const int n16 = 16 / es;
  const uintptr_t m = (uintptr_t)q | (uintptr_t)q_out | (uintptr_t)append_key | (uintptr_t)append_value |
                      (uintptr_t)cos | (uintptr_t)sin | (uintptr_t)k_cache | (uintptr_t)v_cache;
  const int64_t st = q_stride_n | q_stride_h | qo_stride_n | qo_stride_h | k_stride_n | k_stride_h | v_stride_n |
                     v_stride_h | cs_stride_n | page_stride;
  if (m % es) return kBadAlign;
  const bool vec = m % 16 == 0 && st % n16 == 0 && head_dim % (2 * n16) == 0;
  const int per_lane = vec ? n16 : 4;
  const int64_t total = (int64_t)nnz * (num_qo_heads + 2 * num_kv_heads) * (head_dim / (2 * per_lane));
  const int threads = 256;
  const int64_t want = (total + threads - 1) / threads;
  const int blocks = (int)(want < 65536 ? want : 65536);
  hipStream_t s = (hipStream_t)stream;
#define PKV_ROPE(T, N, V)                                                                                       \
  hipLaunchKernelGGL((rope_append_kernel<T, N, V>), dim3(blocks), dim3(threads), 0, s, (const T*)q, q_stride_n, \
                     q_stride_h, (T*)q_out, qo_stride_n, qo_stride_h, num_qo_heads, (const T*)append_key,       \
                     k_stride_n, k_stride_h, (const T*)append_value, v_stride_n, v_stride_h, (const T*)cos,      \
                     (const T*)sin, cs_stride_n, batch_indices, positions, nnz, (T*)k_cache, (T*)v_cache,        \
                     page_stride, num_pages, kv_indices, num_indices, kv_indptr, batch, num_kv_heads, head_dim,  \
                     page_size, err_count)
#define PKV_ROPE_T(T) \
  if (vec) PKV_ROPE(T, 16 / sizeof(T), true); else PKV_ROPE(T, 4, false);
  if (dtype == kF16) {
    PKV_ROPE_T(_Float16)
  } else if (dtype == kBF16) {
    PKV_ROPE_T(__hip_bfloat16)
  } else {
    PKV_ROPE_T(float)
  }
#undef PKV_ROPE_T
#undef PKV_ROPE
  return (int)hipGetLastError();
}
