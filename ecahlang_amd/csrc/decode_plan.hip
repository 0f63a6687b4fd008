// The decode schedule (decode_sched.h), built on the device.
//
// This is the device half of BatchDecodeWithPagedKVCacheWrapper.plan (ecahlang/main.py:341-347,
// :444-455, :538-548): FlashInfer's plan copies kv_indptr to the host and computes its split
// schedule there; here the schedule is computed where the page table already is, so plan never
// synchronises and the step's page table can be rebuilt on the device right before it (also
// inside a captured graph).
//
// First phase (decode_plan_kernel, one workgroup of 1024 threads; every loop strides over the
// batch):
//  1. total = min(kv_indptr[B], num_indices), first = kv_indptr[0]; sequence b owns pages
//     [s0, s1) = kv_indptr[b .. b+1] clipped to [first, total).  An exclusive scan of (s1 > s0)
//     gives each non-empty sequence its rank; sequences with no page are listed.
//  2. Shared prefixes (only with the kv_shared_pages hint): sequence b is linked to b - 1 when
//     they share at least kPrefixMinPages leading pages (the hint, clipped so that each keeps
//     one page of its own).  A run of linked sequences shares P = min(hint) pages, which are
//     marked kPidShared.  With the cascade (and a group width G >= 2), P is cut into np chunks
//     of C pages and the run's sequences into groups of G: one prefix item per (chunk, KV head,
//     group), and every sequence's pages after P are its suffix.  When the items or their
//     partial slots do not fit, nothing is grouped.
//  3. The suffix pages (every page of an ungrouped sequence) are cut into R ranges of equal
//     weight: a page weighs 1, a sequence start seg_cost pages, and the R_p ranges that carry a
//     prefix item (spread evenly over the ranges) are given that much less.
//  4. Each sequence's first and last suffix range, its part count (prefix chunks + the
//     non-empty suffix ranges it spans) and, by an exclusive scan of those, its first partial
//     slot.
// Second phase (one workgroup per range, decode_plan_records_kernel): the range's sequences
// become its segments and its page ids are copied; a range that carries a prefix item also
// writes the item's record.
#include "attn_common.h"
#include "decode_sched.h"
#include "../../include/pagedkv.h"

using namespace pkv;

namespace {

struct PlanParams {
  const int32_t* indptr;
  const int32_t* last;
  const int32_t* indices;
  const int32_t* shared;  // optional hint [B]: leading pages of b that are b - 1's
  int64_t num_indices;
  int32_t batch, num_ctas, r_cap, page_size, seg_cost, group, slot_cap, hkv, cascade;
  int32_t* ghdr;    // kGlobHdr words, then the empty-sequence list [B]
  int32_t* recs;    // r_cap records of kRecStride words
  int32_t* heads;   // r_cap heads of kHeadWords words
  int32_t* precs;   // r_cap prefix item records of kPrecStride words
  int32_t* bf;      // [r_cap] first sequence of each range
  int32_t* starts;  // [r_cap + 1] first suffix position of each range
  int32_t* nzb;     // [r_cap + 1] non-empty ranges before each range
  // per sequence [B]
  int32_t *rank, *swin, *ss, *sp, *sl, *npb, *sbase, *runof, *lcp;
  // per run [B]
  int32_t *run_r0, *run_p, *run_c, *run_np, *run_i0;
};

constexpr int kPlanThreads = 1024;
constexpr int kStartsLds = 4096;  // range starts kept in LDS for the owner searches
constexpr int kNone = 0x7fffffff;

// Weight-space start of range w (0 <= w <= R): the ranges hold equal weight, except that the
// R_p ranges carrying a prefix item hold xt / R_p less each.  Non-decreasing in w, tgt(0) = 0
// and tgt(R) = ws.
struct Targets {
  int64_t ws, xt;  // suffix weight, prefix item weight
  int R, Rp;
  bool carry;      // the carriers hold ws-share minus their item (else they hold no suffix page)
  __device__ Targets(int64_t ws_, int64_t xt_, int R_, int Rp_) : ws(ws_), xt(xt_), R(R_), Rp(Rp_) {
    // (T = (ws + xt) / R >= xt / R_p + 2 keeps every step of the integer form below >= 0)
    carry = Rp == 0 || (ws + xt) * Rp >= (xt + 2 * (int64_t)Rp) * R;
  }
  // prefix items carried by ranges before w: item i sits on range ceil(i * R / R_p)
  __device__ int64_t cnt(int64_t w) const { return (Rp == 0 || w == 0) ? 0 : (w - 1) * Rp / R + 1; }
  __device__ int64_t tgt(int64_t w) const {
    if (Rp == 0 || R == Rp) return w * ws / R;
    if (carry) return w * (ws + xt) / R - (cnt(w) * xt + Rp - 1) / Rp;
    return (w - cnt(w)) * ws / (R - Rp);
  }
};

// Block-wide exclusive scan of v (all 1024 threads call it); `carry` holds the sum of the
// earlier rounds and is advanced by this round's total (the same in every thread).
__device__ __forceinline__ int block_scan(int v, int& carry, int* s_wsum) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    x += lane >= off ? y : 0;
  }
  if (lane == 63) s_wsum[wv] = x;
  __syncthreads();
  int off = 0, blk = 0;
#pragma unroll
  for (int k = 0; k < kPlanThreads / 64; ++k) {
    off += k < wv ? s_wsum[k] : 0;
    blk += s_wsum[k];
  }
  const int ex = carry + off + x - v;
  carry += blk;
  __syncthreads();  // s_wsum is rewritten by the next call
  return ex;
}

__global__ __launch_bounds__(kPlanThreads) void decode_plan_kernel(PlanParams P) {
  __shared__ int s_total, s_first, s_nempty, s_bad;
  __shared__ int s_wsum[kPlanThreads / 64];
  __shared__ unsigned long long s_xt;
  __shared__ int s_starts[kStartsLds + 1];
  __shared__ int64_t s_tgt[kStartsLds + 1];
  const int tid = threadIdx.x, lane = tid & 63;
  const int B = P.batch;
  if (tid == 0) {
    int64_t t = P.indptr[B];
    t = t < P.num_indices ? t : P.num_indices;
    t = t > 0 ? t : 0;
    int64_t f = P.indptr[0];
    f = f < 0 ? 0 : (f > t ? t : f);
    s_total = (int)t;
    s_first = (int)f;
    s_nempty = 0;
    s_bad = 0;
    s_xt = 0;
  }
  __syncthreads();
  const int total = s_total, first = s_first;
  auto clip = [&](int64_t x) -> int { return (int)(x < first ? first : (x > total ? total : x)); };
  const bool hint = P.shared != nullptr;
  const bool group = hint && P.cascade && P.group >= 2;

  // ---- 1, 2a: ranks, the empty list, links and runs
  int nne = 0, nruns = 0;
  for (int base = 0; base < B; base += kPlanThreads) {
    const int b = base + tid;
    int s0 = 0, s1 = 0, lc = 0;
    if (b < B) {
      s0 = clip(P.indptr[b]);
      s1 = clip(P.indptr[b + 1]);
      if (hint && b > 0) {
        const int p0 = clip(P.indptr[b - 1]);
        // each keeps its own the pages that can receive the step's token: its last page, and the
        // one before it when the last is empty (kv_last_page_len 0)
        const int cap = min(s1 - s0 - (P.last[b] > 0 ? 1 : 2), s0 - p0 - (P.last[b - 1] > 0 ? 1 : 2));
        lc = P.shared[b];
        lc = lc < 0 ? 0 : (lc > cap ? cap : lc);
      }
    }
    const bool ne = b < B && s1 > s0;
    const bool link = b < B && lc >= kPrefixMinPages;
    const bool head = b < B && !link;
    const int rk = block_scan(ne ? 1 : 0, nne, s_wsum);
    const int rid = block_scan(head ? 1 : 0, nruns, s_wsum) - (head ? 0 : 1);
    if (b < B) {
      P.rank[b] = rk;
      P.runof[b] = rid;
      P.lcp[b] = link ? lc : 0;
      if (head) {
        P.run_r0[rid] = b;
        P.run_p[rid] = kNone;
      }
      if (!ne) P.ghdr[kGlobHdr + atomicAdd(&s_nempty, 1)] = b;
    }
  }
  __syncthreads();

  // ---- 2b: each run's shared pages, the minimum hint over its linked members (a segmented
  // minimum inside each wave, then one atomic per piece of a run)
  if (hint) {
    for (int base = 0; base < B; base += kPlanThreads) {
      const int b = base + tid;
      int v = b < B && P.lcp[b] > 0 ? P.lcp[b] : kNone;
      const int rid = b < B ? P.runof[b] : -1;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(v, off, 64);
        const int r2 = __shfl_up(rid, off, 64);
        if (lane >= off && r2 == rid) v = min(v, y);
      }
      const int rn = __shfl_down(rid, 1, 64);
      const bool tail = lane == 63 || rn != rid;
      if (b < B && tail && v != kNone) atomicMin(&P.run_p[rid], v);
    }
    __syncthreads();
  }

  // ---- 2c: chunks and items of each run
  const int G = P.group;
  int nitems = 0, nparts = 0;
  for (int base = 0; base < nruns; base += kPlanThreads) {
    const int r = base + tid;
    int items = 0, parts = 0;
    unsigned long long xt = 0;
    if (r < nruns) {
      int pp = 0, np = 0, c = 0;
      if (hint) {
        const int r0 = P.run_r0[r];
        const int size = (r + 1 < nruns ? P.run_r0[r + 1] : B) - r0;
        pp = size >= 2 ? P.run_p[r] : 0;
        pp = pp == kNone ? 0 : pp;  // (kept as the run's shared pages even when not grouping)
        if (pp > 0 && group) {
          np = (pp + kPrefixChunkMin - 1) / kPrefixChunkMin;
          np = np > kMaxPrefixParts ? kMaxPrefixParts : np;
          const int need = (pp + kItemPages - 1) / kItemPages;
          np = np < need ? need : np;
          if (np > kMaxPrefixNp) np = 0;  // (not grouped; its pages are still marked)
          c = np ? (pp + np - 1) / np : 0;
        }
        items = np * P.hkv * ((size + G - 1) / G);
        parts = np * size;
        // an item's weight in suffix pages (decode_sched.h)
        const unsigned long long x =
            ((unsigned long long)c * kPrefixCostNum + kPrefixCostDen - 1) / kPrefixCostDen + kPrefixItemFixed;
        xt = (unsigned long long)items * x;
      }
      P.run_p[r] = pp;
      P.run_np[r] = np;
      P.run_c[r] = c;
    }
    const int i0 = block_scan(items, nitems, s_wsum);
    if (r < nruns) P.run_i0[r] = i0;
    block_scan(parts, nparts, s_wsum);
    if (xt) atomicAdd(&s_xt, xt);
  }
  __syncthreads();
  // The cascade must fit: one carrier range per item, and a partial slot for every chunk of
  // every grouped sequence beside the suffix ranges' R + B.
  const bool casc = group && nitems > 0 && nitems <= P.r_cap &&
                    (int64_t)nparts <= (int64_t)P.slot_cap - P.r_cap - B;
  const int Rp = casc ? nitems : 0;
  const int64_t XT = casc ? (int64_t)s_xt : 0;

  // ---- 2d: suffixes and their positions in the suffix page list
  int ns = 0;
  for (int base = 0; base < B; base += kPlanThreads) {
    const int b = base + tid;
    int s0 = 0, s1 = 0, pp = 0, np = 0, shp = 0;
    if (b < B) {
      s0 = clip(P.indptr[b]);
      s1 = clip(P.indptr[b + 1]);
      if (hint) {
        const int r = P.runof[b];
        shp = P.run_p[r];
        if (casc) {
          np = P.run_np[r];
          pp = np > 0 ? shp : 0;
        }
      }
    }
    const int len = s1 > s0 ? s1 - s0 - pp : 0;
    const int pos = block_scan(len, ns, s_wsum);
    if (b < B) {
      P.ss[b] = s0 + pp;
      P.sl[b] = len;
      P.sp[b] = pos;
      P.npb[b] = np;
      P.lcp[b] = s0 + shp;  // end of the pages b shares with its run (kv_indices position)
    }
  }

  // ---- 3: the suffix ranges
  int R = 0;
  if (ns > 0) {
    R = ns < P.num_ctas ? ns : P.num_ctas;
    const int need = (ns + kRangePages - 1) / kRangePages;
    R = R > need ? R : need;
  }
  R = R > Rp ? R : Rp;
  R = R < P.r_cap ? R : P.r_cap;  // (the host sized r_cap for num_indices >= ns, and Rp <= r_cap)
  int* starts = R <= kStartsLds ? s_starts : P.starts;
  for (int w = tid; w < P.r_cap; w += kPlanThreads) P.bf[w] = -1;
  __syncthreads();
  // Sequence k (in rank order) covers weights [W0 - c, W0 + len) with W0 = pos + c * k (the
  // first part is the gap before its start); range w starts where weight tgt(w) falls.  If a
  // range comes out over kRangePages pages, the plain equal split is used.
  for (int pass = 0; pass < 2 && R > 0; ++pass) {
    const int c = pass == 0 ? P.seg_cost : 0;
    const Targets T((int64_t)ns + (int64_t)c * (nne > 0 ? nne - 1 : 0), pass == 0 ? XT : 0, R, Rp);
    // every range's start weight, computed once (a thread each: three 64-bit divisions) for the
    // searches below, when it fits in LDS
    const bool tab = R <= kStartsLds;
    if (tab) {
      for (int w = tid; w <= R; w += kPlanThreads) s_tgt[w] = T.tgt(w);
      __syncthreads();
    }
    auto tgt_at = [&](int w) -> int64_t { return tab ? s_tgt[w] : T.tgt(w); };
    for (int b = tid; b < B; b += kPlanThreads) {
      const int len = P.sl[b];
      if (len <= 0) continue;
      const int k = P.rank[b], pos = P.sp[b];
      const int64_t w0 = (int64_t)pos + (int64_t)c * k;
      const int64_t lo = k == 0 ? 0 : w0 - c, hi = w0 + len;
      int wl = 0, wh = R;  // smallest w in [0, R] with tgt(w) >= lo
      while (wl < wh) {
        const int mid = (wl + wh) >> 1;
        if (tgt_at(mid) >= lo) wh = mid; else wl = mid + 1;
      }
      for (int w = wl; w < R; ++w) {
        const int64_t tw = tgt_at(w);
        if (tw >= hi) break;
        starts[w] = tw < w0 ? pos : (int)(pos + (tw - w0));
        P.bf[w] = b;
      }
    }
    if (tid == 0) starts[R] = ns;
    __syncthreads();
    for (int w = tid; w < R; w += kPlanThreads) {
      const int len = starts[w + 1] - starts[w];
      if (len < 0 || len > kRangePages) s_bad = 1;
    }
    __syncthreads();
    if (!s_bad) break;
    __syncthreads();  // every thread has read s_bad before it is cleared
    if (tid == 0) s_bad = 0;
  }
  // range holding suffix position p (largest w with starts[w] <= p: empty ranges are skipped)
  auto owner = [&](int p) -> int {
    int lo = 0, hi = R;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (starts[mid] <= p) lo = mid; else hi = mid;
    }
    return lo;
  };
  // ---- 4: non-empty ranges before each range (a range can be empty: a carrier whose item
  // outweighs its share), suffix windows, part counts and first partial slots
  int nnz = 0;
  for (int base = 0; base <= R; base += kPlanThreads) {
    const int w = base + tid;
    const int ex = block_scan(w < R && starts[w + 1] > starts[w] ? 1 : 0, nnz, s_wsum);
    if (w <= R) P.nzb[w] = ex;
  }
  __syncthreads();
  int nslots = 0;
  for (int base = 0; base < B; base += kPlanThreads) {
    const int b = base + tid;
    int parts = 0;
    if (b < B) {
      const int len = P.sl[b];
      if (len > 0) {
        const int pos = P.sp[b];
        const int wlo = owner(pos), whi = owner(pos + len - 1);
        P.swin[b] = wlo | (whi << 16);
        parts = P.npb[b] + P.nzb[whi] - P.nzb[wlo] + 1;
      } else {
        P.swin[b] = -1;
      }
    }
    const int sb = block_scan(parts, nslots, s_wsum);
    if (b < B) P.sbase[b] = sb;
  }
  if (starts != P.starts)
    for (int w = tid; w <= R; w += kPlanThreads) P.starts[w] = starts[w];
  if (tid == 0) {
    P.ghdr[kGhRanges] = R;
    P.ghdr[kGhEmpty] = s_nempty;
    P.ghdr[kGhTotal] = total;
    P.ghdr[kGhFirst] = first;
    P.ghdr[kGhItems] = Rp;
    P.ghdr[kGhSuffix] = ns;
    P.ghdr[kGhRuns] = nruns;
  }
}

// Second phase: one workgroup per range slot w < r_cap writes the range's head and record (its
// sequence segments and its page ids) and, when the range carries one, a prefix item's record.
constexpr int kRecThreads = 256;

__global__ __launch_bounds__(kRecThreads) void decode_plan_records_kernel(PlanParams P) {
  __shared__ int s_nseg;
  __shared__ int s_beg[kRangePages], s_src[kRangePages], s_shend[kRangePages];
  const int w = blockIdx.x, tid = threadIdx.x;
  const int R = P.ghdr[kGhRanges], Rp = P.ghdr[kGhItems];
  int32_t* head = P.heads + (int64_t)w * kHeadWords;
  int32_t* rec = P.recs + (int64_t)w * kRecStride;
  if (w >= R) {  // unused slot: an empty header (R in every header bounds the decode's range loop)
    if (tid == 0) {
      head[kHdrLen] = 0;
      head[kHdrNseg] = 0;
      head[kHdrRanges] = R;
      head[kHdrPrefix] = 0;
    }
    return;
  }
  const int B = P.batch, first = P.ghdr[kGhFirst], total = P.ghdr[kGhTotal];
  const int rs = P.starts[w], re = P.starts[w + 1];
  const int f = P.bf[w];
  if (tid == 0) s_nseg = 0;
  __syncthreads();
  auto clip = [&](int64_t x) -> int { return (int)(x < first ? first : (x > total ? total : x)); };
  // parts of sequence b (prefix chunks, then the non-empty suffix ranges w_lo .. w_hi) and the
  // non-empty ranges before its w_lo
  auto parts_of = [&](int b, int* zlo) -> int {
    const int win = P.swin[b];
    *zlo = P.nzb[win & 0xFFFF];
    return P.npb[b] + P.nzb[(win >> 16) & 0xFFFF] - *zlo + 1;
  };
  // ---- segments: the sequences f, f + 1, ... whose suffixes have pages in [rs, re)
  if (f >= 0 && f < B && re > rs) {
    const int rf = P.rank[f];
    for (int base = f; base < B; base += kRecThreads) {
      const int b = base + tid;
      bool past = true;
      if (b < B) {
        const int pos = P.sp[b], len = P.sl[b];
        past = pos >= re;
        if (!past && len > 0) {
          const int idx = P.rank[b] - rf;
          const int beg = (pos > rs ? pos : rs) - rs, end = (pos + len < re ? pos + len : re) - rs;
          if (idx >= 0 && idx < kRangePages && end > beg && P.swin[b] >= 0) {
            const int e0 = P.indptr[b], e1 = P.indptr[b + 1];
            const int lp = P.last[b];
            int nvl = lp < 0 ? 0 : (lp > P.page_size ? P.page_size : lp);
            // the segment's last page is the sequence's last page only if the list was not cut
            const int nv = (clip(e1) == e1 && pos + len <= re) ? nvl : P.page_size;
            // the step's token: position (n - 1) * ps + last - 1 of the sequence's n listed
            // pages (an uncut list, 0 <= last <= ps), whose pages are the suffix's last len
            int app = 0;
            const int n = e1 - e0;
            const int at = (n - 1) * P.page_size + lp - 1;
            if (clip(e1) == e1 && e0 >= 0 && n >= 1 && lp >= 0 && lp <= P.page_size && at >= 0) {
              const int k = pos + (at / P.page_size - (n - len)) - rs;  // range page of the token
              const int back = end - 1 - k;
              if (k >= beg && k < end && back <= 1) app = 1 + ((back << 4) | (at % P.page_size));
            }
            int zlo;
            const int np = parts_of(b, &zlo);
            const int4 sg = make_int4(seg_pack_b(b, nv, P.npb[b]), seg_pack_range(beg, end, app), P.sbase[b],
                                      seg_pack_part(P.npb[b] + P.nzb[w] - zlo, np));
            *reinterpret_cast<int4*>(rec + kRecSegOff + 4 * idx) = sg;
            if (idx < kHeadSegs) *reinterpret_cast<int4*>(head + kRecSegOff + 4 * idx) = sg;
            s_beg[idx] = beg;
            s_src[idx] = P.ss[b] + (rs + beg - pos);
            s_shend[idx] = P.lcp[b];
            atomicMax(&s_nseg, idx + 1);
          }
        }
      }
      if (__syncthreads_and(past ? 1 : 0)) break;  // (uniform: every thread sees the same result)
    }
  }
  __syncthreads();
  // ---- page ids: position i belongs to the last segment that begins at or before it
  const int len = re - rs, nseg = s_nseg;
  for (int i = tid; i < len; i += kRecThreads) {
    int lo = 0, hi = nseg;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (s_beg[mid] <= i) lo = mid; else hi = mid;
    }
    const int k = s_src[lo] + (i - s_beg[lo]);
    int pid = nseg > 0 ? P.indices[k] : -1;
    pid = (pid < 0 || pid >= kPidShared) ? -1 : (k < s_shend[lo] ? pid | kPidShared : pid);
    rec[kRecPidOff + i] = pid;
    if (i < kHeadPids) head[kHeadPidOff + i] = pid;
  }
  // ---- the prefix item this range carries (item i sits on range ceil(i * R / R_p))
  bool carrier = false;
  int item = 0;
  if (Rp > 0) {
    const int64_t c0 = w == 0 ? 0 : (int64_t)(w - 1) * Rp / R + 1;
    const int64_t c1 = (int64_t)w * Rp / R + 1;
    carrier = c1 > c0;
    item = (int)c0;
  }
  if (carrier) {
    int32_t* pr = P.precs + (int64_t)w * kPrecStride;
    const int nruns = P.ghdr[kGhRuns];
    int lo = 0, hi = nruns;  // the run holding the item: the largest r with run_i0[r] <= item
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (P.run_i0[mid] <= item) lo = mid; else hi = mid;
    }
    const int r = lo, r0 = P.run_r0[r];
    const int size = (r + 1 < nruns ? P.run_r0[r + 1] : B) - r0;
    const int pp = P.run_p[r], C = P.run_c[r];
    const int G = P.group, ng = (size + G - 1) / G;
    const int k = item - P.run_i0[r];
    // chunk-major, then head: the items that read one head's rows of a chunk sit on nearby
    // ranges (one XCD's L2)
    const int c = k / (ng * P.hkv), kr = k - c * ng * P.hkv;
    const int head = kr / ng, o = kr - head * ng;
    const int pbeg = c * C, plen = min(pp, pbeg + C) - pbeg;
    const int nmem = min(G, size - o * G);
    if (tid < nmem) {
      const int b = r0 + o * G + tid;
      int zlo;
      const int np = parts_of(b, &zlo);
      *reinterpret_cast<int4*>(pr + kPrecSegOff + 4 * tid) =
          make_int4(seg_pack_b(b, P.page_size, P.npb[b]), plen << 16, P.sbase[b], seg_pack_part(c, np));
    }
    const int src = P.ss[r0] - pp + pbeg;
    for (int i = tid; i < plen; i += kRecThreads) pr[kPrecPidOff + i] = P.indices[src + i];
    if (tid == 0) {
      pr[kHdrLen] = plen;
      pr[kHdrNseg] = nmem;
      pr[kHdrHead] = head;
    }
  }
  __syncthreads();
  if (tid == 0) {
    head[kHdrLen] = len;
    head[kHdrNseg] = nseg;
    head[kHdrRanges] = R;
    head[kHdrPrefix] = carrier ? 1 : 0;
  }
}

}  // namespace

namespace pkv {

// Plan scratch in int32 words: 9 per-sequence and 5 per-run arrays.
int64_t decode_plan_scratch_words(int batch) { return (int64_t)14 * batch; }

int decode_plan_launch(const int32_t* indptr, const int32_t* indices, int64_t num_indices,
                       const int32_t* last, const int32_t* shared, int batch, int num_ctas,
                       int page_size, int seg_cost, int group, int hkv, int cascade, int r_cap, int slot_cap,
                       int32_t* ghdr, int32_t* recs, int32_t* heads, int32_t* precs, int32_t* bf,
                       int32_t* starts, int32_t* nzb, int32_t* scratch, hipStream_t s) {
  PlanParams P;
  P.indptr = indptr;
  P.last = last;
  P.indices = indices;
  P.shared = shared;
  P.num_indices = num_indices;
  P.batch = batch;
  P.num_ctas = num_ctas;
  P.r_cap = r_cap;
  P.page_size = page_size;
  P.seg_cost = seg_cost;
  P.group = group < kMaxGroup ? group : kMaxGroup;
  P.slot_cap = slot_cap;
  P.hkv = hkv;
  P.cascade = cascade;
  P.ghdr = ghdr;
  P.recs = recs;
  P.heads = heads;
  P.precs = precs;
  P.bf = bf;
  P.starts = starts;
  P.nzb = nzb;
  int32_t* a[14];
  for (int i = 0; i < 14; ++i) a[i] = scratch + (int64_t)i * batch;
  P.rank = a[0]; P.swin = a[1]; P.ss = a[2]; P.sp = a[3]; P.sl = a[4]; P.npb = a[5];
  P.sbase = a[6]; P.runof = a[7]; P.lcp = a[8];
  P.run_r0 = a[9]; P.run_p = a[10]; P.run_c = a[11]; P.run_np = a[12]; P.run_i0 = a[13];
  hipLaunchKernelGGL(decode_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, P);
  hipLaunchKernelGGL(decode_plan_records_kernel, dim3(r_cap), dim3(kRecThreads), 0, s, P);
  return (int)hipGetLastError();
}

}  // namespace pkv
