// Work partition and split-state merge shared by the paged decode kernels.
//
// Decode partitions the batch's concatenated page list (kv_indices[0 .. kv_indptr[B])) into
// num_ctas equal page ranges, one per workgroup, independent of sequence boundaries: every
// workgroup streams the same number of pages whatever the length mix.  A sequence cut by a
// range boundary yields one partial softmax state per workgroup that touches it; those are
// written to the workspace at slot (workgroup + sequence), which is unique because walking
// the page list in order every new segment starts at a new workgroup, a new sequence, or
// both.  The workgroup that arrives last for a sequence (an atomic counter per sequence)
// merges the partials and resets the counter to zero, so the workspace needs zeroing once
// (at plan time) and never inside a captured graph.
#pragma once
#include "common.h"

namespace pkv {

struct DecodeParams {
  const void* q;
  int64_t q_sn, q_sh;          // element strides of q[b][h][:]
  const void* k_cache;
  const void* v_cache;
  int64_t page_stride;         // elements between consecutive pages
  int64_t num_pages;           // pool size: page ids outside [0, num_pages) are never read
  int64_t num_indices;         // length of indices: the page list is cut there
  const int32_t* indptr;       // [B+1]
  const int32_t* indices;      // [indptr[B]]
  const int32_t* last;         // [B]
  int32_t batch, hq, hkv, ps;
  float scale_log2;            // sm_scale * log2(e): scores live in base-2 units
  void* out;
  int64_t o_sn, o_sh;
  int32_t* counters;           // [B]
  float2* part_ml;             // [num_ctas + B][hq] (running max, sum of exp)
  float* part_o;               // [num_ctas + B][hq][D], normalised partial output
  int32_t num_ctas;
  int32_t q_vec;               // q rows / strides allow 16-byte loads
  int32_t o_vec;               // out rows / strides allow 8-byte stores
};

__device__ __forceinline__ int64_t range_start(int w, int n, int64_t total) {
  return (int64_t)w * total / n;
}
// Workgroup whose range holds page p (largest w with range_start(w) <= p).
__device__ __forceinline__ int range_owner(int64_t p, int n, int64_t total) {
  int64_t w = ((p + 1) * n + total - 1) / total - 1;
  return (int)(w < n - 1 ? w : n - 1);
}

// Total pages of the batch, cut to the length of the indices array.
__device__ __forceinline__ int64_t total_pages(const DecodeParams& P) {
  int64_t t = P.indptr[P.batch];
  t = t < P.num_indices ? t : P.num_indices;
  return t > 0 ? t : 0;
}

// Page id at position i of the concatenated page list, or -1 when it is outside the pool.
__device__ __forceinline__ int64_t page_at(const int32_t* indices, int64_t i, int64_t num_pages) {
  int64_t pg = indices[i];
  return (pg >= 0 && pg < num_pages) ? pg : -1;
}

__device__ __forceinline__ int seq_len_of(const DecodeParams& P, int b) {
  int np = P.indptr[b + 1] - P.indptr[b];
  return np > 0 ? (np - 1) * P.ps + P.last[b] : 0;
}

// Cross-workgroup data (split partials, arrival counters) moves only through device-scope
// atomic loads and stores.  Those are coherent across the XCDs' separate L2 caches by
// themselves, so the hand-off needs no L2 write-back / invalidate (which a device-scope
// fence would issue, once per segment per workgroup): a writer waits for its stores to
// complete before bumping the counter, and the last arriver reads with device-scope loads.
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Merge the partial states of sequence b (workgroups w_lo..w_hi) into the output row.
template <typename T, int D>
__device__ void merge_partials(const DecodeParams& P, int b, int w_lo, int w_hi) {
  T* out = reinterpret_cast<T*>(P.out);
  const float* ml = reinterpret_cast<const float*>(P.part_ml);
  for (int idx = threadIdx.x; idx < P.hq * D; idx += blockDim.x) {
    int h = idx / D, d = idx - h * D;
    float M = -INFINITY;
    for (int w = w_lo; w <= w_hi; ++w) M = fmaxf(M, ld_dev(ml + 2 * ((int64_t)(w + b) * P.hq + h)));
    float num = 0.f, den = 0.f;
    for (int w = w_lo; w <= w_hi; ++w) {
      int64_t s = (int64_t)(w + b) * P.hq + h;
      float mx = ld_dev(ml + 2 * s), l = ld_dev(ml + 2 * s + 1);
      if (l > 0.f) {
        float c = exp2f(mx - M) * l;
        num += c * ld_dev(P.part_o + s * D + d);
        den += c;
      }
    }
    out[b * P.o_sn + h * P.o_sh + d] = from_f32<T>(den > 0.f ? num / den : 0.f);
  }
}

// Partial state of one (slot, q head): normalised output and (max, sum) in base-2 units.
__device__ __forceinline__ void store_partial_ml(const DecodeParams& P, int64_t sidx, float m, float l) {
  float* ml = reinterpret_cast<float*>(P.part_ml);
  st_dev(ml + 2 * sidx, m);
  st_dev(ml + 2 * sidx + 1, l);
}

// Arrival protocol after a workgroup wrote its partial for sequence b.  Returns true in
// every thread of the workgroup that arrived last (it must then merge).
__device__ __forceinline__ bool arrive_last(const DecodeParams& P, int b, int nseg, int* flag_lds) {
  wait_stores();  // this thread's partial stores are complete (device-visible)
  __syncthreads();
  if (threadIdx.x == 0) {
    int old = atomicAdd(&P.counters[b], 1);
    int last = old == nseg - 1;
    // Every other arrival already happened: safe to reset for the next launch.
    if (last) __hip_atomic_store(&P.counters[b], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag_lds = last;
  }
  __syncthreads();
  const bool last = *flag_lds != 0;
  asm volatile("" ::: "memory");  // no partial load is hoisted above the arrival
  return last;
}

// Zero the output rows of sequences that own no pages (no workgroup range touches them).
// One thread per sequence, so the check costs one round of loads, not one per sequence.
template <typename T, int D>
__device__ void zero_empty_sequences(const DecodeParams& P) {
  T* out = reinterpret_cast<T*>(P.out);
  for (int b = threadIdx.x; b < P.batch; b += blockDim.x) {
    if (P.indptr[b + 1] > P.indptr[b]) continue;
    for (int h = 0; h < P.hq; ++h)
      for (int d = 0; d < D; ++d) out[b * P.o_sn + h * P.o_sh + d] = from_f32<T>(0.f);
  }
}

// Number of page ranges actually used: never more ranges than pages, so no range is empty
// and the workgroups touching a sequence are exactly range_owner(first)..range_owner(last).
__device__ __forceinline__ int effective_ranges(int num_ctas, int64_t total) {
  return (int)(num_ctas < total ? num_ctas : total);
}

// The matrix-core kernel also caps a range at kPidCap pages (its page ids are staged in
// LDS), using ceil(total / kPidCap) ranges when that exceeds the workgroup count.
constexpr int kPidCap = 2048;
__host__ __device__ __forceinline__ int64_t decode_ranges_max(int num_ctas, int64_t total) {
  int64_t need = (total + kPidCap - 1) / kPidCap;
  return need > num_ctas ? need : num_ctas;
}
__device__ __forceinline__ int decode_ranges(int num_ctas, int64_t total) {
  int64_t n = total < num_ctas ? total : num_ctas;
  int64_t need = (total + kPidCap - 1) / kPidCap;
  return (int)(n > need ? n : need);
}

// Largest b in [0, B) with indptr[b] <= p, found by the whole wave: each lane loads one
// entry and a ballot counts the prefix (indptr is non-decreasing), so B <= 64 costs one
// round of loads and B <= 4096 two.
__device__ __forceinline__ int find_seq_wave(const int32_t* indptr, int B, int64_t p) {
  const int lane = threadIdx.x & 63;
  int lo = 0, n = B;
  while (n > 64) {
    const int stride = (n + 63) / 64;
    const int idx = lo + lane * stride;
    const bool le = idx < lo + n && (int64_t)indptr[idx] <= p;
    const int cnt = __popcll(__ballot(le));
    lo += (cnt - 1) * stride;
    n = stride < B - lo ? stride : B - lo;
  }
  const bool le = lane < n && (int64_t)indptr[lo + lane] <= p;
  return lo + __popcll(__ballot(le)) - 1;
}

int decode_valu_dispatch(const DecodeParams& P, int dtype, int d, hipStream_t s);
int decode_mfma_dispatch(const DecodeParams& P, int dtype, int d, hipStream_t s);
bool decode_mfma_supported(int dtype, int d, int g, int hkv);

}  // namespace pkv
