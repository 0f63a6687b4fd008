// Decode schedule: the per-plan work list the matrix-core decode kernel reads.
//
// pkv_decode_plan (BatchDecodeWithPagedKVCacheWrapper.plan) enqueues decode_plan_kernel, which
// cuts the batch's page list (kv_indices[kv_indptr[0] .. kv_indptr[B]), clipped to num_indices)
// into R equal ranges and writes one fixed-size record per range into the workspace:
//   header   [len, nseg, R, 0, ...]                      kRecHdr int32 (in the range's head)
//   segments nseg x {b, beg | end << 16, nv, w_lo | w_hi << 16}
//            one per sequence with pages in the range: range pages [beg, end) are sequence
//            b's, nv is the valid token count of the segment's last page (16 unless that page
//            is the sequence's last), and the sequence spans ranges w_lo .. w_hi
//   page ids the range's len page ids, copied from kv_indices
// so a decode workgroup learns everything it needs to start streaming pages from one record,
// in one memory round trip, instead of searching kv_indptr first.  The decode launches of all
// layers of a step share the plan.  A global header before the records holds R and the
// sequences that own no page (their output rows are zeros).
#pragma once
#include <stdint.h>

namespace pkv {

constexpr int kRangePages = 512;                       // pages per range at most
// Weight of a sequence start when the plan cuts the page list, in K/V bytes: a range that holds
// one more segment synchronises its waves mid-range to combine their states, which costs about
// as long as a workgroup takes to stream this many bytes (measured at Qwen2.5-3B B=64: 12
// pages of 16 KB was the fastest of 0, 3, 6, 9, 12, 16, 24, 32).
constexpr int64_t kSegCostBytes = 12 * 16384;
inline int seg_cost_pages(int num_kv_heads, int head_dim, int page_size) {
  const int64_t page = (int64_t)2 * page_size * num_kv_heads * head_dim * 2;
  const int64_t c = (kSegCostBytes + page / 2) / page;
  return c < 1 ? 1 : (c > 64 ? 64 : (int)c);
}
constexpr int kRecHdr = 16;                            // header words
constexpr int kRecSegOff = kRecHdr;                    // segment records (4 words each)
constexpr int kRecPidOff = kRecSegOff + 4 * kRangePages;
constexpr int kRecStride = (kRecPidOff + kRangePages + 63) / 64 * 64;  // words, 256-byte multiple
enum RecHdr { kHdrLen = 0, kHdrNseg = 1, kHdrRanges = 2 };
// Head of each range: the header, its first kHeadSegs segments and first kHeadPids page ids,
// 512 bytes per range in one dense array, which is all a decode workgroup reads before its
// first page copies (one contiguous area for every workgroup's first read).
constexpr int kHeadWords = 128;
constexpr int kHeadSegs = 12;                          // words 16 .. 63
constexpr int kHeadPidOff = 64;
constexpr int kHeadPids = 64;                          // words 64 .. 127
constexpr int kGlobHdr = 16;                           // global header words (then the empty list)
enum GlobHdr { kGhRanges = 0, kGhEmpty = 1, kGhTotal = 2, kGhFirst = 3 };

// Ranges a plan may use: one per workgroup, more when that would put over kRangePages pages in
// one range (num_indices bounds the page count).
inline int64_t decode_ranges_cap(int num_ctas, int64_t num_indices) {
  const int64_t need = (num_indices + kRangePages - 1) / kRangePages;
  return need > num_ctas ? need : num_ctas;
}

}  // namespace pkv
