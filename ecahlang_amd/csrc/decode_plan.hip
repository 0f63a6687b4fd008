// The decode schedule (decode_sched.h), built on the device by one workgroup.
//
// This is the device half of BatchDecodeWithPagedKVCacheWrapper.plan (ecahlang/main.py:341-347,
// :444-455, :538-548): FlashInfer's plan copies kv_indptr to the host and computes its split
// schedule there; here the schedule is computed where the page table already is, so plan never
// synchronises and the step's page table can be rebuilt on the device right before it (also
// inside a captured graph).
//
// First phase (one workgroup of 1024 threads; every loop strides over the batch):
//  1. total = min(kv_indptr[B], num_indices), first = kv_indptr[0]; the n = total - first pages
//     are cut into R = max(min(num_ctas, n), ceil(n / kRangePages)) ranges.
//  2. Sequence b owns pages [s0, s1) = kv_indptr[b .. b+1] clipped to [first, total).  An
//     exclusive scan of (s1 > s0) gives each non-empty sequence its rank.  Sequences with no
//     page are listed.
//  3. Range starts cut the page list into R parts of equal weight (a page weighs 1, a sequence
//     start seg_cost_pages); a range's first sequence is the one holding its first page.
//  4. Each sequence's first and last range are found in the LDS copy of the range starts.
// Second phase (one workgroup per range, decode_plan_records_kernel): the range's sequences
// become its segments (sequence b is segment rank[b] - rank[first sequence of the range]) and
// its page ids are copied, coalesced.
#include "attn_common.h"
#include "decode_sched.h"
#include "../../include/pagedkv.h"

using namespace pkv;

namespace {

struct PlanParams {
  const int32_t* indptr;
  const int32_t* last;
  const int32_t* indices;
  int64_t num_indices;
  int32_t batch, num_ctas, r_cap, page_size, seg_cost;
  int32_t* ghdr;    // kGlobHdr words, then the empty-sequence list [B]
  int32_t* recs;    // r_cap records of kRecStride words
  int32_t* heads;   // r_cap heads of kHeadWords words
  int32_t* rank;    // [B] scratch
  int32_t* bf;      // [r_cap] scratch: first sequence of each range
  int32_t* starts;  // [r_cap + 1] scratch: first page-list position of each range
  int32_t* swin;    // [B] scratch: first | last range << 16 of each sequence with pages
};

constexpr int kPlanThreads = 1024;
constexpr int kStartsLds = 4096;  // range starts kept in LDS for the owner searches

__global__ __launch_bounds__(kPlanThreads) void decode_plan_kernel(PlanParams P) {
  __shared__ int s_total, s_first, s_r, s_nempty, s_bad;
  __shared__ int s_wsum[kPlanThreads / 64];
  __shared__ int s_starts[kStartsLds + 1];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int B = P.batch;
  if (tid == 0) {
    int64_t t = P.indptr[B];
    t = t < P.num_indices ? t : P.num_indices;
    t = t > 0 ? t : 0;
    int64_t f = P.indptr[0];
    f = f < 0 ? 0 : (f > t ? t : f);
    const int64_t n = t - f;
    int64_t r = 0;
    if (n > 0) {
      r = n < P.num_ctas ? n : P.num_ctas;
      const int64_t need = (n + kRangePages - 1) / kRangePages;
      r = r > need ? r : need;
      r = r < P.r_cap ? r : P.r_cap;  // (the host sized r_cap for num_indices >= n)
    }
    s_total = (int)t;
    s_first = (int)f;
    s_r = (int)r;
    s_nempty = 0;
    s_bad = 0;
  }
  __syncthreads();
  const int total = s_total, first = s_first, R = s_r, n = total - first;
  int* starts = R <= kStartsLds ? s_starts : P.starts;
  auto clip = [&](int64_t x) -> int { return (int)(x < first ? first : (x > total ? total : x)); };

  // ---- ranks of the sequences that own pages; the ones that own none are listed
  int carry = 0;
  for (int base = 0; base < B; base += kPlanThreads) {
    const int b = base + tid;
    int s0 = 0, s1 = 0;
    if (b < B) {
      s0 = clip(P.indptr[b]);
      s1 = clip(P.indptr[b + 1]);
    }
    const bool ne = b < B && s1 > s0;
    const uint64_t bal = __ballot(ne);
    const int below = __popcll(bal & ((1ull << lane) - 1));
    if (lane == 0) s_wsum[wv] = __popcll(bal);
    __syncthreads();
    int off = 0, blk = 0;
#pragma unroll
    for (int v = 0; v < kPlanThreads / 64; ++v) {
      off += v < wv ? s_wsum[v] : 0;
      blk += s_wsum[v];
    }
    if (b < B) P.rank[b] = carry + off + below;
    if (!ne && b < B) {
      const int e = atomicAdd(&s_nempty, 1);
      P.ghdr[kGlobHdr + e] = b;
    }
    carry += blk;
    __syncthreads();  // s_wsum is rewritten next round; global writes above are visible below
  }
  const int nne = carry;
  for (int w = tid; w < P.r_cap; w += kPlanThreads) P.bf[w] = -1;
  __syncthreads();

  // ---- range starts: pages weigh 1 and every sequence start after the first weighs seg_cost,
  // and the weight is cut into R equal parts, so a range that holds the start of a sequence (an
  // extra segment: a combine of the waves' states mid-range) gets fewer pages.  Sequence k (in
  // rank order) covers weights [W0 - seg_cost, W0 + len) with W0 = (s0 - first) + seg_cost * k
  // (the first part is the gap before its start); range w starts where weight w * WT / R falls.
  // If a range comes out empty or over kRangePages pages, the equal split (cost 0) is used.
  for (int pass = 0; pass < 2; ++pass) {
    const int c = pass == 0 ? P.seg_cost : 0;
    const int64_t WT = (int64_t)n + (int64_t)c * (nne > 0 ? nne - 1 : 0);
    for (int b = tid; b < B && R > 0; b += kPlanThreads) {
      const int s0 = clip(P.indptr[b]), s1 = clip(P.indptr[b + 1]);
      if (s1 <= s0) continue;
      const int k = P.rank[b];
      const int64_t w0 = (int64_t)(s0 - first) + (int64_t)c * k;
      const int64_t lo = k == 0 ? 0 : w0 - c, hi = w0 + (s1 - s0);
      // ranges whose target floor(w * WT / R) lies in [lo, hi)
      int64_t w = (lo * R + WT - 1) / WT;
      w = w > 0 ? w - 1 : 0;
      for (; w < R; ++w) {
        const int64_t tw = w * WT / R;
        if (tw >= hi) break;
        if (tw < lo) continue;
        starts[w] = tw < w0 ? s0 : (int)(s0 + (tw - w0));
        P.bf[w] = b;
      }
    }
    if (tid == 0) starts[R] = total;
    __syncthreads();
    for (int w = tid; w < R; w += kPlanThreads) {
      const int len = starts[w + 1] - starts[w];
      if (len < 1 || len > kRangePages) s_bad = 1;
    }
    __syncthreads();
    if (!s_bad) break;
    __syncthreads();  // every thread has read s_bad before it is cleared
    if (tid == 0) s_bad = 0;
  }
  // range holding page-list position p (largest w with starts[w] <= p)
  auto owner = [&](int p) -> int {
    int lo = 0, hi = R;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (starts[mid] <= p) lo = mid; else hi = mid;
    }
    return lo;
  };
  // each sequence's first and last range (for the second phase's segment records)
  for (int b = tid; b < B; b += kPlanThreads) {
    const int s0 = clip(P.indptr[b]), s1 = clip(P.indptr[b + 1]);
    P.swin[b] = s1 > s0 ? owner(s0) | (owner(s1 - 1) << 16) : -1;
  }
  if (starts != P.starts)
    for (int w = tid; w <= R; w += kPlanThreads) P.starts[w] = starts[w];
  if (tid == 0) {
    P.ghdr[kGhRanges] = R;
    P.ghdr[kGhEmpty] = s_nempty;
    P.ghdr[kGhTotal] = total;
    P.ghdr[kGhFirst] = first;
  }
}

// Second phase: one workgroup per range slot w < r_cap writes the range's head and record (its
// sequence segments and a copy of its page ids), all ranges at once.
constexpr int kRecThreads = 256;

__global__ __launch_bounds__(kRecThreads) void decode_plan_records_kernel(PlanParams P) {
  __shared__ int s_nseg;
  const int w = blockIdx.x, tid = threadIdx.x;
  const int R = P.ghdr[kGhRanges];
  int32_t* head = P.heads + (int64_t)w * kHeadWords;
  int32_t* rec = P.recs + (int64_t)w * kRecStride;
  if (w >= R) {  // unused slot: an empty header (R in every header bounds the decode's range loop)
    if (tid == 0) {
      head[kHdrLen] = 0;
      head[kHdrNseg] = 0;
      head[kHdrRanges] = R;
    }
    return;
  }
  const int B = P.batch, first = P.ghdr[kGhFirst], total = P.ghdr[kGhTotal];
  const int rs = P.starts[w], re = P.starts[w + 1];
  const int f = P.bf[w];
  if (tid == 0) s_nseg = 0;
  __syncthreads();
  auto clip = [&](int64_t x) -> int { return (int)(x < first ? first : (x > total ? total : x)); };
  // ---- segments: the sequences f, f + 1, ... that own pages in [rs, re)
  if (f >= 0 && f < B) {
    const int rf = P.rank[f];
    for (int base = f; base < B; base += kRecThreads) {
      const int b = base + tid;
      bool past = true;
      if (b < B) {
        const int e1 = P.indptr[b + 1];
        const int s0 = clip(P.indptr[b]), s1 = clip(e1);
        past = s0 >= re;
        if (!past && s1 > s0) {
          const int idx = P.rank[b] - rf;
          const int beg = (s0 > rs ? s0 : rs) - rs, end = (s1 < re ? s1 : re) - rs;
          const int win = P.swin[b];
          if (idx >= 0 && idx < kRangePages && end > beg && win >= 0) {
            int nvl = P.last[b];
            nvl = nvl < 0 ? 0 : (nvl > P.page_size ? P.page_size : nvl);
            // the segment's last page is the sequence's last page only if the list was not cut
            const int nv = (s1 == e1 && s1 <= re) ? nvl : P.page_size;
            const int4 sg = make_int4(b, beg | (end << 16), nv, win);
            *reinterpret_cast<int4*>(rec + kRecSegOff + 4 * idx) = sg;
            if (idx < kHeadSegs) *reinterpret_cast<int4*>(head + kRecSegOff + 4 * idx) = sg;
            atomicMax(&s_nseg, idx + 1);
          }
        }
      }
      if (__syncthreads_and(past ? 1 : 0)) break;  // (uniform: every thread sees the same result)
    }
  }
  // ---- page ids
  const int len = re - rs;
  for (int i = tid; i < len; i += kRecThreads) {
    const int pid = P.indices[rs + i];
    rec[kRecPidOff + i] = pid;
    if (i < kHeadPids) head[kHeadPidOff + i] = pid;
  }
  __syncthreads();
  if (tid == 0) {
    head[kHdrLen] = len;
    head[kHdrNseg] = s_nseg;
    head[kHdrRanges] = R;
  }
}

}  // namespace

namespace pkv {

int decode_plan_launch(const int32_t* indptr, const int32_t* indices, int64_t num_indices,
                       const int32_t* last, int batch, int num_ctas, int page_size, int seg_cost,
                       int r_cap, int32_t* ghdr, int32_t* recs, int32_t* heads, int32_t* rank,
                       int32_t* bf, int32_t* starts, int32_t* swin, hipStream_t s) {
  PlanParams P;
  P.indptr = indptr;
  P.last = last;
  P.indices = indices;
  P.num_indices = num_indices;
  P.batch = batch;
  P.num_ctas = num_ctas;
  P.r_cap = r_cap;
  P.page_size = page_size;
  P.seg_cost = seg_cost;
  P.ghdr = ghdr;
  P.recs = recs;
  P.heads = heads;
  P.rank = rank;
  P.bf = bf;
  P.starts = starts;
  P.swin = swin;
  hipLaunchKernelGGL(decode_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, P);
  hipLaunchKernelGGL(decode_plan_records_kernel, dim3(r_cap), dim3(kRecThreads), 0, s, P);
  return (int)hipGetLastError();
}

}  // namespace pkv
