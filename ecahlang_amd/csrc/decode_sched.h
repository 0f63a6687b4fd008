// Decode schedule: the per-plan work list the matrix-core decode kernel reads.
//
// pkv_decode_plan (BatchDecodeWithPagedKVCacheWrapper.plan) builds it on the device.
//
// Suffix ranges.  The batch's page list (kv_indices[kv_indptr[0] .. kv_indptr[B]), clipped to
// num_indices), minus the shared prefix pages described below, is cut into R ranges of equal
// weight; each range gets one fixed-size record:
//   header   [len, nseg, R, prefix, ...]                 kRecHdr int32 (in the range's head)
//   segments nseg x int4 {b | nv << 22 | np << 27, beg | app << 10 | end << 16, slot0,
//                         part | (nparts - 1) << 16}
//            one per sequence with pages in the range: range pages [beg, end) are sequence
//            b's, nv is the valid token count of the segment's last page (16 unless that page
//            is the sequence's last).  app (bits 10-15 of the second word, 0: none) places the
//            decode step's new token when it falls in this segment: at position
//            (pages - 1) * page_size + kv_last_page_len - 1 of the sequence, i.e. range page
//            end - 1 - ((app - 1) >> 4), row (app - 1) & 15 (the page before an empty last page
//            when kv_last_page_len is 0).  The sequence's softmax state is cut into nparts parts
//            whose partials live in slots slot0 .. slot0 + nparts - 1; this segment is part
//            `part` (nparts == 1: the segment is the whole sequence and writes the output).
//            The first np parts are shared-prefix chunks, each written by Hkv prefix items
//            (one per KV head), so the sequence's merge waits for nparts + np (Hkv - 1)
//            arrivals.
//   page ids the range's len page ids, each with kPidShared set when other sequences of the
//            batch read the same page (then it is copied with the cached policy, so the
//            readers after the first find it in L2; other pages stream past the caches), and -1
//            for an id that cannot be a page (negative, or kPidShared and above)
// so a decode workgroup learns everything it needs to start streaming pages from one record,
// in one memory round trip.  The decode launches of all layers of a step share the plan.  A
// global header before the records holds R and the sequences that own no page (their output
// rows are zeros).
//
// Shared prefixes.  With the optional kv_shared_pages hint (for each sequence b >= 1, how many of
// its leading pages are the same pages as sequence b - 1's), the common prefix of a run of
// consecutive sequences that share at least kPrefixMinPages pages is marked kPidShared.
// Cascade (PKV_PLAN_CASCADE): the common prefix is instead read once per group of G sequences
// rather than once per sequence: the prefix is cut into chunks, and a prefix item
// (G sequences x one chunk x one KV head) is carried by one range.  Its record:
//   header   [len, nseg, head]                           (nseg <= G <= kMaxGroup sequences)
//   segments nseg x int4, as above (beg = 0, end = len, part = the chunk's index)
//   page ids the chunk's len page ids
// The workgroup that owns the range reads the head's rows of each chunk page into LDS once (its
// waves share the pages) and attends all G = 2 * (16 / g) sequences to them, so a grouped
// sequence has one prefix part per chunk (a chunk holds up to kItemPages pages).  A grouped
// sequence's parts are its prefix chunks followed
// by its suffix ranges, merged like any split sequence.
#pragma once
#include <stdint.h>

namespace pkv {

constexpr int kRangePages = 512;                       // pages per range (and per chunk) at most
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
enum RecHdr { kHdrLen = 0, kHdrNseg = 1, kHdrRanges = 2, kHdrPrefix = 3, kHdrHead = 2 };
// Head of each range: the header, its first kHeadSegs segments and first kHeadPids page ids,
// 512 bytes per range in one dense array, which is all a decode workgroup reads before its
// first page copies (one contiguous area for every workgroup's first read).
constexpr int kHeadWords = 128;
constexpr int kHeadSegs = 12;                          // words 16 .. 63
constexpr int kHeadPidOff = 64;
constexpr int kHeadPids = 64;                          // words 64 .. 127
constexpr int kGlobHdr = 16;                           // global header words (then the empty list)
constexpr int kPidShared = 1 << 30;                    // page id flag: read by several sequences
enum GlobHdr { kGhRanges = 0, kGhEmpty = 1, kGhTotal = 2, kGhFirst = 3, kGhItems = 4, kGhSuffix = 5, kGhRuns = 6 };

// Prefix item records (indexed by the range that carries the item).
constexpr int kMaxGroup = 32;                          // sequences per prefix item at most
constexpr int kPrecSegOff = 16;                        // <= kMaxGroup segments: words 16 .. 143
constexpr int kPrecPidOff = 256;
constexpr int kPrecStride = kPrecPidOff + kRangePages; // words, 256-byte multiple
constexpr int kPrefixMinPages = 16;                    // shorter shared prefixes are not grouped
constexpr int kPrefixChunkMin = 64;                    // pages per chunk, unless that makes too many
constexpr int kMaxPrefixParts = 16;                    // chunks per prefix (more only past 16 x 128 pages)
constexpr int kMaxPrefixNp = 31;                       // chunks per prefix at most (5 bits)
constexpr int kItemPages = 128;                        // pages per chunk at most (ids in 2 registers a lane)
// A prefix item's weight when the plan balances the ranges, in streamed pages (a suffix page
// weighs 1): a fixed kPrefixItemFixed for its set-up, its fold and its arrivals, plus its C
// pages of one head's rows times kPrefixCostNum / kPrefixCostDen (the workgroup's waves share
// the pages, each attending all G sequences to its own).
constexpr int kPrefixCostNum = 1, kPrefixCostDen = 4, kPrefixItemFixed = 29;

// Head block of the matrix-core decode: the largest power of two HB with HB * g <= 16 query heads
// (the MFMA's 16 columns), HB * head_dim <= 256 and HB | Hkv.
__host__ __device__ inline int decode_head_block(int d, int g, int hkv) {
  int hb = 1;
  while (2 * hb * g <= 16 && 2 * hb * d <= 256 && hkv % (2 * hb) == 0) hb *= 2;
  return hb;
}

// Segment word packing.
constexpr int kSegBBits = 22;
__host__ __device__ inline int seg_pack_range(int beg, int end, int app) { return beg | (app << 10) | (end << 16); }
__host__ __device__ inline int seg_pack_b(int b, int nv, int np) {
  return (int)((unsigned)b | ((unsigned)nv << kSegBBits) | ((unsigned)np << (kSegBBits + 5)));
}
__host__ __device__ inline int seg_pack_part(int part, int nparts) { return part | ((nparts - 1) << 16); }

// Ranges a plan may use: one per workgroup, more when that would put over kRangePages pages in
// one range (num_indices bounds the page count).
inline int64_t decode_ranges_cap(int num_ctas, int64_t num_indices) {
  const int64_t need = (num_indices + kRangePages - 1) / kRangePages;
  return need > num_ctas ? need : num_ctas;
}
constexpr int64_t kMaxRanges = 60000;                  // segment words hold part / nparts in 16 bits

}  // namespace pkv
