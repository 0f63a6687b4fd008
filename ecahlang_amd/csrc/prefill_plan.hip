// The host half of BatchPrefillWithPagedKVCacheWrapper.plan (ecahlang/main.py:432-443): the
// matrix-core prefill's work list, built on the host from the batch's indptr arrays (the
// wrapper reads them back once per batch, as FlashInfer's plan does).
//
// An item is (request, KV head, rows / g query tokens, a chunk of the keys those tokens see).
// A key range longer than the chunk is cut into chunks of `chunk` keys (the last one shorter)
// that form a split group, whose partials a second kernel merges.  The chunk is a whole number
// of the kernel's 64-key steps.  Items are issued longest first, and the hardware hands each
// to the first compute unit that is free, so the kernel lasts as long as the most loaded unit
// under that greedy order.  The plan therefore tries chunks around total keys / CUs and keeps
// the one whose simulated makespan is lowest: each item costs a fixed set-up and write-out, a
// split item the merge's share on top, plus its steps (the costs measured on the Qwen2.5-3B
// chunked-prefill shape: 1.9 us a step, 11 us an item, 6 us more for a split one).  Chunks are
// doubled while the partials would not fit in the workspace.
#include <algorithm>
#include <array>
#include <functional>
#include <queue>
#include <vector>
#include "../../include/pagedkv.h"

namespace {

constexpr int kItemWords = 12;
constexpr int kGroupWords = 8;
constexpr int kStepKeys = 64;
constexpr int kChunkMin = 256, kChunkMax = 8192;
// Makespan model, in microseconds.
constexpr double kStepUs = 1.9, kItemUs = 11.0, kSplitUs = 6.0;
// Candidate chunks, as multiples of total keys / CUs (in 1/16).
constexpr int kCandidates[] = {8, 10, 12, 14, 16, 17, 18, 20, 24};

struct Group {
  int h, t0, tq, kv_end, kv_len, qo_len, qo_start, kp0, b;
};

int64_t align256(int64_t n) { return (n + 255) / 256 * 256; }

struct Layout {
  int64_t n_items = 0, n_groups = 0, slots = 0, off_g = 0, off_ml = 0, off_o = 0, bytes = 0;
};

Layout layout_for(const std::vector<Group>& groups, int chunk, int rows, int head_dim, int pbytes) {
  Layout L;
  for (const Group& gr : groups) {
    const int64_t nch = std::max<int64_t>(1, ((int64_t)gr.kv_end + chunk - 1) / chunk);
    L.n_items += nch;
    if (nch > 1) {
      ++L.n_groups;
      L.slots += nch;
    }
  }
  L.off_g = align256(L.n_items * kItemWords * 4);
  L.off_ml = L.off_g + align256(L.n_groups * kGroupWords * 4);
  L.off_o = L.off_ml + align256(L.slots * rows * 8);
  L.bytes = L.off_o + L.slots * (int64_t)rows * head_dim * pbytes;
  return L;
}

// Simulated kernel time of the work list cut at `chunk`: items longest first, each to the
// least loaded of ncu compute units.
double makespan(const std::vector<Group>& groups, int chunk, int ncu) {
  struct It {
    int len;
    bool split;
  };
  std::vector<It> its;
  for (const Group& gr : groups) {
    const int nch = std::max(1, (gr.kv_end + chunk - 1) / chunk);
    for (int c = 0; c < nch; ++c) its.push_back({std::min(gr.kv_end, (c + 1) * chunk) - c * chunk, nch > 1});
  }
  std::stable_sort(its.begin(), its.end(), [](const It& a, const It& b) { return a.len > b.len; });
  std::priority_queue<double, std::vector<double>, std::greater<double>> load;
  for (int i = 0; i < ncu; ++i) load.push(0.0);
  double worst = 0.0;
  for (const It& it : its) {
    const double t = load.top() + kItemUs + (it.split ? kSplitUs : 0.0) +
                     kStepUs * ((it.len + kStepKeys - 1) / kStepKeys);
    load.pop();
    load.push(t);
    worst = std::max(worst, t);
  }
  return worst;
}

int round_chunk(int64_t keys) {
  int64_t c = (keys + kStepKeys / 2) / kStepKeys * kStepKeys;
  return (int)std::min<int64_t>(kChunkMax, std::max<int64_t>(kChunkMin, c));
}

}  // namespace

extern "C" int pkv_prefill_work_list(const int32_t* qo_indptr, const int32_t* kv_indptr,
                                     const int32_t* kv_last_page_len, int32_t batch, int32_t group,
                                     int32_t num_kv_heads, int32_t page_size, int32_t causal,
                                     int32_t head_dim, int32_t num_cus, int64_t workspace_bytes,
                                     int32_t rows, int32_t partial_bytes, int32_t chunk,
                                     int32_t* items, int64_t items_cap, int32_t* groups_out,
                                     int64_t groups_cap, int64_t* info) {
  if (!qo_indptr || !kv_indptr || !kv_last_page_len || !info || batch < 0 || group < 1 ||
      num_kv_heads < 1 || page_size < 1 || head_dim < 1 || num_cus < 1 || rows < group ||
      rows % group || (partial_bytes != 2 && partial_bytes != 4) ||
      (chunk != 0 && (chunk % kStepKeys || chunk < kChunkMin || chunk > kChunkMax)))
    return PKV_E_ARG;
  const int tq_max = rows / group;
  std::vector<Group> grs;
  int64_t total = 0;
  for (int b = 0; b < batch; ++b) {
    const int qo_len = qo_indptr[b + 1] - qo_indptr[b];
    const int npg = kv_indptr[b + 1] - kv_indptr[b];
    if (qo_len < 0 || npg < 0) return PKV_E_ARG;
    const int kv_len = npg > 0 ? (npg - 1) * page_size + kv_last_page_len[b] : 0;
    for (int t0 = 0; t0 < qo_len; t0 += tq_max) {
      const int tq = std::min(tq_max, qo_len - t0);
      const int kv_end = causal ? std::min(kv_len, std::max(0, t0 + tq + kv_len - qo_len)) : kv_len;
      for (int h = 0; h < num_kv_heads; ++h) {
        grs.push_back({h, t0, tq, kv_end, kv_len, qo_len, qo_indptr[b], kv_indptr[b], b});
        total += kv_end;
      }
    }
  }
  // the chunk: the given one, else the candidate with the lowest simulated makespan among those
  // whose partials fit (ties go to the longer chunk: fewer splits); if none fits, doubled from
  // the longest candidate while the partials do not fit
  const int64_t per_cu = (total + num_cus - 1) / num_cus;
  int best = 0;
  if (chunk != 0) {
    best = chunk;
  } else {
    double best_t = 0.0;
    int widest = kChunkMin;
    for (int f : kCandidates) {
      const int c = round_chunk(per_cu * f / 16);
      widest = std::max(widest, c);
      if (layout_for(grs, c, rows, head_dim, partial_bytes).bytes > workspace_bytes) continue;
      const double t = makespan(grs, c, num_cus);
      if (best == 0 || t < best_t || (t == best_t && c > best)) {
        best = c;
        best_t = t;
      }
    }
    if (best == 0) {
      best = widest;
      while (best < kChunkMax && layout_for(grs, best, rows, head_dim, partial_bytes).bytes > workspace_bytes)
        best = std::min(kChunkMax, best * 2);
    }
  }
  const Layout L = layout_for(grs, best, rows, head_dim, partial_bytes);
  info[0] = L.n_items;
  info[1] = L.n_groups;
  info[2] = best;
  info[3] = L.slots;
  info[4] = L.off_g;
  info[5] = L.off_ml;
  info[6] = L.off_o;
  info[7] = L.bytes;
  if (L.bytes > workspace_bytes) return PKV_E_WORKSPACE;
  if (L.n_items > items_cap || L.n_groups > groups_cap || !items || (L.n_groups > 0 && !groups_out))
    return PKV_E_ARG;
  // the list: split groups' chunks take consecutive slots in group order; then the items are
  // ordered longest key range first (stable, so equal lengths keep that order)
  std::vector<std::array<int32_t, kItemWords>> its;
  its.reserve(L.n_items);
  int64_t nslots = 0, ng = 0;
  for (const Group& gr : grs) {
    const int nch = std::max(1, (gr.kv_end + best - 1) / best);
    if (nch == 1) {
      its.push_back({gr.b, gr.h, gr.t0, gr.tq, 0, gr.kv_end, -1, gr.kv_len, gr.qo_len, gr.qo_start, gr.kp0, 0});
      continue;
    }
    for (int c = 0; c < nch; ++c)
      its.push_back({gr.b, gr.h, gr.t0, gr.tq, c * best, std::min(gr.kv_end, (c + 1) * best),
                     (int32_t)(nslots + c), gr.kv_len, gr.qo_len, gr.qo_start, gr.kp0, 0});
    const int32_t rec[kGroupWords] = {(int32_t)nslots, nch, gr.qo_start, gr.t0, gr.tq, gr.h, 0, 0};
    std::copy(rec, rec + kGroupWords, groups_out + ng * kGroupWords);
    ++ng;
    nslots += nch;
  }
  std::stable_sort(its.begin(), its.end(), [](const std::array<int32_t, kItemWords>& a,
                                              const std::array<int32_t, kItemWords>& b) {
    return a[5] - a[4] > b[5] - b[4];
  });
  for (size_t i = 0; i < its.size(); ++i) std::copy(its[i].begin(), its[i].end(), items + i * kItemWords);
  return 0;
}
