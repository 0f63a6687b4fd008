// Work partition and split-state merge shared by the paged decode kernels.
//
// Decode partitions the batch's concatenated page list (kv_indices[0 .. kv_indptr[B])) into
// page ranges independent of sequence boundaries, so every workgroup streams about the same
// number of pages whatever the length mix.  A sequence cut by range boundaries (or, with the
// matrix-core kernel's schedule, also into shared-prefix chunks) yields one partial softmax
// state per part; a sequence's parts occupy consecutive partial slots.  The vector kernel's
// slot of (range w, sequence b) is w + b, which is unique because walking the page list in
// order every new segment starts at a new range, a new sequence, or both; the plan assigns
// the matrix-core kernel's slots.  The workgroup that arrives last for a sequence (an atomic
// counter per sequence) merges the partials and resets the counter to zero, so the workspace
// needs zeroing once (at plan time) and never inside a captured graph.
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
  float2* part_ml;             // [slot_cap][ml_stride] (running max, sum of exp)
  float* part_o;               // [slot_cap][hq][D], normalised partial output
  int32_t slot_cap;            // partial slots in the workspace (>= num_ctas + B)
  int32_t num_ctas;
  int32_t q_vec;               // q rows / strides allow 16-byte loads
  int32_t o_vec;               // out rows / strides allow 8-byte stores
  int32_t dynamic;             // matrix-core kernel: waves take pages on demand
  int32_t ml_stride;           // float2 entries per part_ml slot: hq rounded up to a line
  const int32_t* sched;        // matrix-core kernel: the plan's range records (decode_sched.h)
  const int32_t* sched_hdr;    // ... and its global header
  const int32_t* sched_head;   // ... and the dense heads of its ranges
  const int32_t* sched_pref;   // ... and its prefix item records
  int32_t cascade;             // the schedule was planned with prefix items
  int32_t r_cap;               // ranges the workspace holds
  // Matrix-core kernel, append fused in (pkv_batch_decode_append): token b's new K and V rows
  // (byte strides per token and head) belong at the last slot of sequence b's last page; null
  // when the call appends nothing.
  const char* ak;
  const char* av;
  int64_t ak_sn, ak_sh, av_sn, av_sh;
};

// The kernel arguments as wave-uniform values that the compiler cannot reload from the argument
// block.  Kernel arguments are invariant, so under scalar-register pressure the compiler re-issues
// their scalar loads instead of keeping them, and a reload that misses the scalar cache costs
// ~0.25 us per line (measured on MI355X) -- several of those sat in every range's fold and merge.
// Staged through LDS (one word per thread) and read back with readfirstlane, each field is an
// ordinary value: kept in scalar registers or spilled to vector lanes, never reloaded.  All
// threads of the workgroup must call it (it synchronises once).
template <typename Prm>
__device__ __forceinline__ Prm uniform_params(const Prm& arg, int* lds_words) {
  static_assert(sizeof(Prm) % 4 == 0 && sizeof(Prm) / 4 <= 256, "parameter block");
  constexpr int N = sizeof(Prm) / 4;
  if ((int)threadIdx.x < N) lds_words[threadIdx.x] = reinterpret_cast<const int*>(&arg)[threadIdx.x];
  __syncthreads();
  int w[N];
#pragma unroll
  for (int k = 0; k < N; ++k) w[k] = __builtin_amdgcn_readfirstlane(lds_words[k]);
  Prm out;
  __builtin_memcpy(&out, w, sizeof(Prm));
  return out;
}

// A part_ml slot (one segment's (max, sum) pairs of every q head) spans whole 128-byte L2 lines,
// so no line holds two slots.  The merger of a sequence reads its slots with plain loads; were a
// line shared with another sequence's slot, that load could bring the other slot's line into
// this XCD's L2 before its writer (on another XCD) stored it, and the other sequence's merger
// on this XCD would then read the stale copy.
constexpr int kLineBytes = 128;
__host__ __device__ __forceinline__ int ml_slot_stride(int hq) {
  constexpr int per = kLineBytes / 8;  // float2 entries per line
  return (hq + per - 1) / per * per;
}

// Partition of the batch's `total` pages into n contiguous ranges (1 <= n <= total): the
// first r = total % n ranges hold q + 1 pages, the others q = total / n.  32-bit arithmetic
// only (total < 2^31 as page-list offsets are int32): a 64-bit division is a long software
// sequence on this target.
struct Ranges {
  int n, q, r, big;  // big = r * (q + 1): first page of the q-page ranges
  __device__ __forceinline__ Ranges(int n_, int total)
      : n(n_), q(total / n_), r(total % n_), big((total % n_) * (total / n_ + 1)) {}
  __device__ __forceinline__ int start(int w) const { return w * q + (w < r ? w : r); }
  // Range holding page p (clamped to the last range for p >= total).
  __device__ __forceinline__ int owner(int p) const {
    const int w = p < big ? p / (q + 1) : r + (p - big) / q;
    return w < n - 1 ? w : n - 1;
  }
};

// Total pages of the batch, cut to the length of the indices array.
__device__ __forceinline__ int total_pages(const DecodeParams& P) {
  int64_t t = P.indptr[P.batch];
  t = t < P.num_indices ? t : P.num_indices;
  return t > 0 ? (int)t : 0;
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

// Cross-workgroup hand-off of split partials without device-scope fences (each of which
// writes back and invalidates a whole L2, once per segment per workgroup):
//  * writers store partials with device-scope atomic stores, which write through the
//    XCD's L2, and wait for them to complete before bumping the sequence's counter;
//  * the last arriver then reads them with plain loads: no L2 on its XCD has held those
//    lines since the kernel began (each partial slot is read once, by that merger only,
//    and caches start the kernel invalidated), so the loads fetch the written values, and
//    being plain they can all be in flight at once.
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16-byte device-scope (write-through, sc1) vector store: the same effect as four st_dev,
// issued as a buffer store with the sc1 cache policy so the compiler still tracks its
// register hazards (a hand-written store can have its data registers reused before the
// hardware has read them).  `base` is the start of the partial area, `off` a byte offset.
typedef float fvec4 __attribute__((ext_vector_type(4)));
constexpr int kCpolSc1 = 16;  // device scope: write through this XCD's L2
__device__ __forceinline__ void st_dev4(float* base, uint32_t off, fvec4 v) {
  __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7fffffff, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kCpolSc1);
}
// vmcnt(0) through the builtin (expcnt and lgkmcnt left at their maxima: 0x0F70), so the
// compiler's own wait bookkeeping knows every load and store has completed and inserts no
// stale waits afterwards; the empty asm keeps memory accesses from moving across it.
__device__ __forceinline__ void wait_stores() {
  __builtin_amdgcn_s_waitcnt(0x0F70);
  asm volatile("" ::: "memory");
}

// Workgroup barrier for LDS hand-offs only.  __syncthreads() also carries a release fence,
// which on this target waits for every outstanding global load (vmcnt(0)) and so would
// drain each wave's K/V prefetch at every barrier; here only LDS traffic is settled.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

constexpr int kMergeRegs = 8;  // segments a merge folds from registers

// Running merge of a sequence's normalised partial rows: part s holds NV values po[s][.] of the
// normalised row and its (max, sum) ml[s] in base-2 units.  Parts are folded in groups of
// kMergeRegs with a running reference max.  Every merge of decode partials uses this one
// sequence of operations, so an output row does not depend on which workgroup merged it or how
// (from memory after the last arrival, or straight from the last part's own state).
template <int NV>
struct MergeAcc {
  float mu = 0.f, den = 0.f;  // running reference max (0 while no part is seen) and weight sum
  float acc[NV];
  __device__ __forceinline__ MergeAcc() {
#pragma unroll
    for (int x = 0; x < NV; ++x) acc[x] = 0.f;
  }
  // Fold of parts g0 .. g0 + nsw - 1 (the group's values in ml[0 .. nsw), po[0 .. nsw)), those
  // below nseg only.  v_exp_f32 directly: its arguments are <= 0.
  __device__ __forceinline__ void fold(const float2* ml, const float (*po)[NV], int g0, int nsw, int nseg) {
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < kMergeRegs; ++s) {
      if (s >= nsw) break;
      M = g0 + s < nseg ? fmaxf(M, ml[s].x) : M;
    }
    if (g0 > 0) {  // rescale what the earlier groups folded to the new reference max
      const float mn = M > mu || den == 0.f ? M : mu;
      const float m2 = mn == -INFINITY ? 0.f : mn;
      const float f = den > 0.f ? __builtin_amdgcn_exp2f(mu - m2) : 0.f;
      den *= f;
#pragma unroll
      for (int x = 0; x < NV; ++x) acc[x] *= f;
      mu = m2;
    } else {
      mu = M == -INFINITY ? 0.f : M;
    }
#pragma unroll
    for (int s = 0; s < kMergeRegs; ++s) {
      if (s >= nsw) break;
      const float c = (g0 + s < nseg && ml[s].y > 0.f) ? __builtin_amdgcn_exp2f(ml[s].x - mu) * ml[s].y : 0.f;
      den += c;
      // Partial rows are finite (normalised averages of finite value rows; a segment whose
      // tokens were all masked stores zeros), and entries past nseg repeat a real part, so
      // c * row needs no select.
#pragma unroll
      for (int x = 0; x < NV; ++x) acc[x] = __builtin_fmaf(c, po[s][x], acc[x]);
    }
  }
  // Output value x (a sum of exact zeros comes out +0, whatever the signs of its terms).
  __device__ __forceinline__ float out(int x) const {
    const float inv = den > 0.f ? 1.f / den : 0.f;
    return (acc[x] + 0.f) * inv;
  }
};

// Merges of the sequences queued in `list` (rows of sequence, first slot, parts), all at once.
// An item is 8 consecutive output dims of one head of one queued sequence; each thread takes
// one item per round.  Segments are folded in groups of kMergeRegs: a group's loads are all
// issued before its fold, and a wave loads only as many segments of a group as the longest
// sequence among its items has (a wave-uniform bound, so the loads need no divergent branch).
// So a round costs one memory latency per group; sequences of up to kMergeRegs parts (the
// usual case) take one group, and their result is the plain fold of all parts at once.
template <typename T, int D>
struct MergeItem {
  float2 ml[kMergeRegs];
  float po[kMergeRegs][8];
  MergeAcc<8> m;
  int b = -1, h = 0, d = 0, nseg = 0;
  // Item `item` of `nitems` (>= 1): which sequence, head and dims, and its segment count.
  // Items past the end repeat the last one and are not stored.
  __device__ __forceinline__ int locate(const int (*list)[3], int per, int item, int nitems) {
    const bool real = item < nitems;
    const int it = real ? item : nitems - 1;
    const int i = it / per, r = it - i * per;
    nseg = list[i][2];
    b = real ? list[i][0] : -1;
    h = r / (D / 8);
    d = (r - h * (D / 8)) * 8;
    return i;
  }
  // Loads of segments g0 .. g0 + nsw - 1 (nsw wave-uniform, 1 .. kMergeRegs), from indices
  // clamped into this item's segments.
  __device__ __forceinline__ void load(const DecodeParams& P, const int (*list)[3], int i, int g0, int nsw) {
    const int64_t slot0 = list[i][1];
#pragma unroll
    for (int s = 0; s < kMergeRegs; ++s) {
      if (s < nsw) {
        const int64_t slot = slot0 + (g0 + s < nseg ? g0 + s : nseg - 1);
        ml[s] = P.part_ml[slot * P.ml_stride + h];
        const float4* src = reinterpret_cast<const float4*>(P.part_o + (slot * P.hq + h) * D + d);
        const float4 a = src[0], c = src[1];
        po[s][0] = a.x; po[s][1] = a.y; po[s][2] = a.z; po[s][3] = a.w;
        po[s][4] = c.x; po[s][5] = c.y; po[s][6] = c.z; po[s][7] = c.w;
      } else {  // (never folded: set so that no value is left undefined)
        ml[s] = make_float2(-INFINITY, 0.f);
#pragma unroll
        for (int x = 0; x < 8; ++x) po[s][x] = 0.f;
      }
    }
  }
  __device__ __forceinline__ void fold(int g0, int nsw) { m.fold(ml, po, g0, nsw, nseg); }
  __device__ __forceinline__ void store(const DecodeParams& P) const {
    if (b < 0) return;
    T* orow = reinterpret_cast<T*>(P.out) + b * P.o_sn + h * P.o_sh + d;
    if (sizeof(T) == 2 && P.o_vec) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        T v[4] = {from_f32<T>(m.out(4 * half)), from_f32<T>(m.out(4 * half + 1)),
                  from_f32<T>(m.out(4 * half + 2)), from_f32<T>(m.out(4 * half + 3))};
        *reinterpret_cast<uint2*>(orow + 4 * half) = *reinterpret_cast<const uint2*>(v);
      }
    } else {
#pragma unroll
      for (int x = 0; x < 8; ++x) orow[x] = from_f32<T>(m.out(x));
    }
  }
};

template <typename T, int D>
__device__ __forceinline__ void merge_queued(const DecodeParams& P, const int (*list)[3], int nm) {
  const int per = P.hq * (D / 8);
  const int nitems = nm * per;
  const int nt = blockDim.x;
  auto round = [&](int base) __attribute__((always_inline)) {
    MergeItem<T, D> a;
    const int i = a.locate(list, per, base + threadIdx.x, nitems);
    int nsmax = a.nseg;  // the wave's longest item
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) nsmax = max(nsmax, __shfl_xor(nsmax, off, 64));
    nsmax = __builtin_amdgcn_readfirstlane(nsmax);
    int nsw = nsmax < kMergeRegs ? nsmax : kMergeRegs;
    a.load(P, list, i, 0, nsw);
    asm volatile("" ::: "memory");  // every load of the group is issued before the fold
    a.fold(0, nsw);
    for (int g0 = kMergeRegs; g0 < nsmax; g0 += kMergeRegs) {
      nsw = nsmax - g0 < kMergeRegs ? nsmax - g0 : kMergeRegs;
      a.load(P, list, i, g0, nsw);
      asm volatile("" ::: "memory");
      a.fold(g0, nsw);
    }
    a.store(P);
  };
  // The first round (all of it when nitems <= blockDim.x, the usual case) is peeled off the
  // loop: inside a loop, registers that the previous round's loads filled can make the
  // compiler wait for those loads before issuing the next ones.  With no items (nm == 0:
  // this workgroup arrived last for none of its splits) nothing runs: an item's loads use
  // list rows that only exist when nitems > 0.
  if (nitems <= 0) return;
  round(0);
  for (int base = nt; base < nitems; base += nt) round(base);
}

// Merge of sequence b's partials (slots slot_lo .. slot_lo + nseg - 1) straight from global
// memory (any segment count).
template <typename T, int D>
__device__ __forceinline__ void merge_partials(const DecodeParams& P, int b, int slot_lo, int nseg) {
  T* out = reinterpret_cast<T*>(P.out);
  const int64_t slot0 = slot_lo;
  for (int idx = threadIdx.x; idx < P.hq * D; idx += blockDim.x) {
    const int h = idx / D, d = idx - h * D;
    const float2* ml = P.part_ml + slot0 * P.ml_stride + h;
    const float* po = P.part_o + (slot0 * P.hq + h) * D + d;
    float M = -INFINITY;
#pragma unroll 4
    for (int s = 0; s < nseg; ++s) M = fmaxf(M, ml[(int64_t)s * P.ml_stride].x);
    float num = 0.f, den = 0.f;
#pragma unroll 4
    for (int s = 0; s < nseg; ++s) {
      const float2 v = ml[(int64_t)s * P.ml_stride];
      const float o = po[(int64_t)s * P.hq * D];
      const float c = v.y > 0.f ? exp2f(v.x - M) * v.y : 0.f;
      num += c * o;
      den += c;
    }
    out[b * P.o_sn + h * P.o_sh + d] = from_f32<T>(den > 0.f ? num / den : 0.f);
  }
}

// (max, sum) in base-2 units of one (slot, q head) of a split segment.
__device__ __forceinline__ void store_partial_ml(const DecodeParams& P, int64_t slot, int hq, float m, float l) {
  float* ml = reinterpret_cast<float*>(P.part_ml + slot * P.ml_stride + hq);
  st_dev(ml, m);
  st_dev(ml + 1, l);
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
__device__ __forceinline__ void zero_empty_sequences(const DecodeParams& P) {
  T* out = reinterpret_cast<T*>(P.out);
  for (int b = threadIdx.x; b < P.batch; b += blockDim.x) {
    if (P.indptr[b + 1] > P.indptr[b]) continue;
    for (int h = 0; h < P.hq; ++h)
      for (int d = 0; d < D; ++d) out[b * P.o_sn + h * P.o_sh + d] = from_f32<T>(0.f);
  }
}

// Number of page ranges actually used: never more ranges than pages, so no range is empty
// and the workgroups touching a sequence are exactly Ranges::owner(first)..owner(last).
__device__ __forceinline__ int effective_ranges(int num_ctas, int total) {
  return num_ctas < total ? num_ctas : total;
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
bool decode_mfma_supported(int dtype, int d, int g, int hkv, int batch);

}  // namespace pkv
