// Top-k / top-p sampling from logits, one row per workgroup: the sampler the serving loop calls
// after the last layer (flashinfer.sampling.top_k_top_p_sampling_from_logits at
// ecahlang/main.py:377-379, 400-402, 489-491, 582-584; top-k filter first, then top-p on the
// renormalised top-k distribution, deterministic=True).
//
// Definition (the oracle, oracle/sampling_ref.py, restates the same rule):
//   p_i ∝ exp(x_i - max x)                                   (softmax of the row's logits)
//   K   = { i : x_i >= k-th largest logit }                  (all tokens when k <= 0 or k >= V)
//   S   = { i in K : x_i >= t }, t the largest logit with mass({j in K : x_j >= t}) >= top_p * mass(K)
//                                                             (S = K when top_p >= 1)
//   token = first i in S, in vocabulary order, whose cumulative mass over S exceeds u * mass(S)
// Ties at a threshold are kept.  No sort: both thresholds are found by radix selection over an
// order-preserving 32-bit key of the logit (three digit passes of 11, 11 and 10 bits, histograms
// in LDS), and every mass is an integer: exp(x_i - max) in 32-bit fixed point, summed in 64 bits,
// so the result depends on nothing but the row and u (no floating-point summation order).
// Every pass reads the row with 16-byte loads (8 fp16/bf16 or 4 fp32 logits per thread, 8 tiles
// in flight); after the first pass the row is served from L2.
#include "common.h"
#include "../../include/pagedkv.h"

using namespace pkv;

namespace {

constexpr int kThreads = 1024;
constexpr int kBins = 2048;        // 11-bit digits
constexpr int kMaxTiles = 512;     // tiles of kThreads * 8 logits: vocabularies up to 4 M


// Order-preserving key of a float (larger float, larger key); NaN sorts lowest.
__device__ __forceinline__ uint32_t fkey(float f) {
  const uint32_t b = __float_as_uint(f);
  if (f != f) return 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
// Mass of a logit in 32-bit fixed point: floor(exp(x - max) * 2^32), capped at 4294967040 (the
// largest float below 2^32), so it converts with one 32-bit instruction (a float -> 64-bit
// integer conversion is a sequence of ten; this runs for every logit on several passes).
__device__ __forceinline__ uint64_t fmass(float x, float mx) {
  const float d = x - mx;
  if (!(d > -23.f)) return 0;  // (also NaN): exp(-23) * 2^32 < 0.5
  return (uint64_t)(uint32_t)fminf(__expf(d) * 4294967296.0f, 4294967040.0f);
}

template <typename T>
struct Row {
  const T* p;
  int v;
  bool vec;
  static constexpr int E = 16 / sizeof(T);  // logits per 16-byte load
  // Calls f(index, logit) for this thread's logits of tile `tile` (thread t: E consecutive).
  template <typename F>
  __device__ __forceinline__ void tile(int tile, F&& f) const {
    const int base = (tile * kThreads + (int)threadIdx.x) * E;
    if (vec && base + E <= v) {
      const uint4 u = *reinterpret_cast<const uint4*>(p + base);
      const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
      for (int k = 0; k < E; ++k) f(base + k, to_f32(e[k]));
    } else {
#pragma unroll
      for (int k = 0; k < E; ++k)
        if (base + k < v) f(base + k, to_f32(p[base + k]));
    }
  }
  __device__ __forceinline__ int tiles() const { return (v + kThreads * E - 1) / (kThreads * E); }
  // Calls f(index, logit) for all of this thread's logits, kUnroll tiles' loads in flight at a time.
  static constexpr int kUnroll = 8;
  template <typename F>
  __device__ __forceinline__ void each(F&& f) const {
    const int nt = tiles();
    // (unconditional loads from clamped addresses: a load under a branch would be waited for
    // at the branch's end, one at a time; whole vectors past the row end are never used)
    const int last = v >= E ? (v - E) / E * E : 0;
    for (int t0 = 0; t0 < nt; t0 += kUnroll) {
      uint4 buf[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int base = ((t0 + u) * kThreads + (int)threadIdx.x) * E;
        buf[u] = vec ? *reinterpret_cast<const uint4*>(p + min(base, last)) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int base = ((t0 + u) * kThreads + (int)threadIdx.x) * E;
        if (vec && base + E <= v) {
          const T* e = reinterpret_cast<const T*>(&buf[u]);
#pragma unroll
          for (int k = 0; k < E; ++k) f(base + k, to_f32(e[k]));
        } else {
          for (int k = 0; k < E; ++k)
            if (base + k < v) f(base + k, to_f32(p[base + k]));
        }
      }
    }
  }
};

__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max_f32(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) red[w] = v;
  __syncthreads();
  float r = -INFINITY;
  for (int i = 0; i < kThreads / 64; ++i) r = fmaxf(r, red[i]);
  return r;
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) { return wave_sum_u64_dpp(v); }
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t* red) {
  v = wave_sum_u64(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) red[w] = v;
  __syncthreads();
  uint64_t r = 0;
  for (int i = 0; i < kThreads / 64; ++i) r += red[i];
  return r;
}

struct SampleLds {
  uint64_t hist[kBins];     // counts (top-k) or masses (top-p) per digit
  uint64_t tile[kMaxTiles];  // kept mass per tile
  uint64_t red[kThreads / 64];
  float redf[kThreads / 64];
  uint64_t scan[kThreads / 64];
  uint32_t sel[4];
};

template <typename T, typename RowT>
__device__ __forceinline__ void sample_row(const RowT& row, SampleLds& L, int b, int vocab, const int32_t* top_k,
                                           int32_t top_k_all, const float* top_p, float top_p_all,
                                           const float* uniform, int32_t* out) {
  uint64_t* s_hist = L.hist;
  uint64_t* s_tile = L.tile;
  uint64_t* s_red = L.red;
  float* s_redf = L.redf;
  uint64_t* s_scan = L.scan;
  uint32_t* s_sel = L.sel;
  const int ntiles = row.tiles();

  // ---- max logit
  float mx = -INFINITY;
  row.each([&](int, float x) { mx = fmaxf(mx, x); });
  mx = block_max(mx, s_redf);

  // ---- radix selection, most significant digit first.  `above` is what lies above the
  // current prefix (a count for top-k, a mass for top-p); the digit where the running total
  // from the top reaches `need` extends the prefix.
  auto select = [&](bool by_mass, uint32_t floor_key, uint64_t need, uint64_t& total) -> uint32_t {
    uint32_t prefix = 0, pmask = 0;
    uint64_t above = 0;
    const int shifts[3] = {21, 10, 0}, widths[3] = {11, 11, 10};
    total = 0;
    for (int lvl = 0; lvl < 3; ++lvl) {
      const int sh = shifts[lvl], nb = 1 << widths[lvl];
      for (int i = threadIdx.x; i < kBins; i += kThreads) s_hist[i] = 0;
      __syncthreads();
      row.each([&](int, float x) {
        const uint32_t k = fkey(x);
        if (k >= floor_key && (k & pmask) == prefix)
          atomicAdd((unsigned long long*)&s_hist[(k >> sh) & (nb - 1)], by_mass ? (unsigned long long)fmass(x, mx) : 1ull);
      });
      __syncthreads();
      if (threadIdx.x < 64) {
        // lane l owns bins [l * nb / 64, (l + 1) * nb / 64); suffix sums from the top bin down
        const int per = nb / 64, lo = threadIdx.x * per;
        uint64_t mine = 0;
        for (int i = 0; i < per; ++i) mine += s_hist[lo + i];
        if (lvl == 0) total = wave_sum_u64(mine);  // (uniform: everything at or above floor_key)
        // inclusive suffix scan of lane sums across the wave (from lane 63 down)
        uint64_t suf = mine;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const uint64_t v = __shfl_down(suf, o, kWave);
          if ((int)threadIdx.x + o < 64) suf += v;
        }
        // the lane whose range holds the crossing: above + suffix(l) >= need > above + suffix(l + 1)
        const uint64_t next = __shfl_down(suf, 1, kWave);
        const uint64_t suf_next = threadIdx.x < 63 ? next : 0;
        if (above + suf >= need && above + suf_next < need) {
          uint64_t run = above + suf_next;
          int d = lo + per - 1;
          for (; d > lo; --d) {
            if (run + s_hist[d] >= need) break;
            run += s_hist[d];
          }
          s_sel[0] = (uint32_t)d;
          s_sel[1] = (uint32_t)(run & 0xffffffffu);
          s_sel[2] = (uint32_t)(run >> 32);
        }
        if (lvl == 0) s_red[0] = total;
      }
      __syncthreads();
      const uint32_t d = s_sel[0];
      above = (uint64_t)s_sel[1] | ((uint64_t)s_sel[2] << 32);
      total = s_red[0];
      prefix |= d << sh;
      pmask |= (uint32_t)(nb - 1) << sh;
      __syncthreads();
    }
    return prefix;
  };

  // ---- top-k threshold (key of the k-th largest logit; ties kept)
  const int k = top_k ? top_k[b] : top_k_all;
  uint32_t thr = 0;
  uint64_t dummy;
  if (k > 0 && k < vocab) thr = select(false, 0u, (uint64_t)k, dummy);

  // ---- top-p threshold over the top-k set
  const float pp = top_p ? top_p[b] : top_p_all;
  if (pp < 1.f) {
    // mass of the top-k set first (the first level's histogram total), then the selection
    uint64_t mk = 0;
    row.each([&](int, float x) { if (fkey(x) >= thr) mk += fmass(x, mx); });
    mk = block_sum_u64(mk, s_red);
    double needd = ceil((double)fmaxf(pp, 0.f) * (double)mk);
    uint64_t need = needd < 1.0 ? 1 : (uint64_t)needd;
    if (need > mk) need = mk;
    if (mk > 0) {
      uint64_t tot;
      const uint32_t tp = select(true, thr, need, tot);
      thr = tp > thr ? tp : thr;
    }
  }

  // ---- sample: kept mass per tile, the tile holding the target, then the thread and token
  for (int t = threadIdx.x; t < ntiles; t += kThreads) s_tile[t] = 0;
  __syncthreads();
  {
    constexpr int E = RowT::E;
    uint64_t m = 0;
    int cur = 0;
    row.each([&](int i, float x) {
      const int t = i / (kThreads * E);
      if (t != cur) {  // (tiles come in increasing order)
        if (m) atomicAdd((unsigned long long*)&s_tile[cur], (unsigned long long)m);
        m = 0;
        cur = t;
      }
      if (fkey(x) >= thr) m += fmass(x, mx);
    });
    if (m) atomicAdd((unsigned long long*)&s_tile[cur], (unsigned long long)m);
  }
  __syncthreads();
  uint64_t ms = 0;
  for (int t = 0; t < ntiles; ++t) ms += s_tile[t];  // (every thread: uniform)
  int32_t token = -1;
  if (ms > 0) {
    const double uu = fminf(fmaxf(uniform[b], 0.f), 1.f);
    uint64_t target = (uint64_t)(uu * (double)ms);
    if (target >= ms) target = ms - 1;
    int tt = 0;
    uint64_t before = 0;
    while (tt < ntiles - 1 && before + s_tile[tt] <= target) before += s_tile[tt++];
    // inside tile tt: each thread's kept mass, exclusive scan, then the owner walks its logits
    uint64_t mine = 0;
    row.tile(tt, [&](int, float x) { if (fkey(x) >= thr) mine += fmass(x, mx); });
    // block exclusive scan: inclusive within each wave, then the waves' totals
    uint64_t inc = mine;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t v = __shfl_up(inc, o, kWave);
      if (lane >= o) inc += v;
    }
    if (lane == 63) s_scan[wv] = inc;
    __syncthreads();
    uint64_t off = before;
    for (int i = 0; i < wv; ++i) off += s_scan[i];
    const uint64_t start = off + inc - mine;
    if (mine > 0 && start <= target && target < start + mine) {
      uint64_t run = start;
      int found = -1;
      row.tile(tt, [&](int i, float x) {
        if (found < 0 && fkey(x) >= thr) {
          run += fmass(x, mx);
          if (run > target) found = i;
        }
      });
      out[b] = found;
    }
  } else if (threadIdx.x == 0) {
    out[b] = token;  // (no token carries mass: an all-NaN or empty row)
  }
}

// Which kernel samples a row: its whole distribution (no top-k, no top-p filter), a top-k filter
// with k <= kTopKMax (then any top-p), or anything else (the one-workgroup kernel).
enum RowKind : int { kWholeRow = 0, kTopKRow = 1, kOtherRow = 2 };
constexpr int kTopKMax = 256;
__host__ __device__ __forceinline__ int row_kind_of(int k, float pp, int vocab) {
  if (k <= 0 || k >= vocab) return pp < 1.f ? kOtherRow : kWholeRow;
  return k <= kTopKMax ? kTopKRow : kOtherRow;
}
__device__ __forceinline__ int row_kind(int b, int vocab, const int32_t* top_k, int32_t top_k_all,
                                        const float* top_p, float top_p_all) {
  return row_kind_of(top_k ? top_k[b] : top_k_all, top_p ? top_p[b] : top_p_all, vocab);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void sample_kernel(const T* logits, int64_t row_stride, int vocab,
                                                          const int32_t* top_k, int32_t top_k_all,
                                                          const float* top_p, float top_p_all,
                                                          const float* uniform, int32_t* out, int split,
                                                          const int32_t* fallback) {
  __shared__ SampleLds L;
  const int b = blockIdx.x;
  // with the split kernels in use, whole-distribution and small-top-k rows are theirs, except
  // the rows they handed back (fallback[b])
  if (split && row_kind(b, vocab, top_k, top_k_all, top_p, top_p_all) != kOtherRow && !fallback[b]) return;
  const T* p = logits + (int64_t)b * row_stride;
  const Row<T> row{p, vocab, ((uintptr_t)p % 16) == 0};
  sample_row<T>(row, L, b, vocab, top_k, top_k_all, top_p, top_p_all, uniform, out);
}

// ---- Whole-distribution rows (the serving loop's default request: top_k 0, top_p 1) over many
// workgroups per row.  One workgroup per row leaves half the chip idle and is bound by the
// vector ALU of the CUs it has, so these rows are cut into slices of kSliceTiles tiles of
// kSplitTile logits, one workgroup per (slice, row), in two launches:
//   split_max_kernel     each slice's largest logit
//   split_sample_kernel  the row's largest logit from the slices', each tile's mass (the same
//                        integer masses as sample_row), then the workgroup that finishes its
//                        slice last (a per-row counter) finds the tile and the token holding the
//                        row's uniform, walking in vocabulary order.
// The masses and the target are the integers sample_row computes, so the token is identical.
constexpr int kSplitThreads = 256;
constexpr int kSplitTile = kSplitThreads * 8;  // 8 logits per thread
constexpr int kSliceTiles = 8;
constexpr int kMaxSplitTiles = 2048;           // vocabularies up to 4 M

constexpr int kCandCap = 512;    // candidates a slice hands over for a top-k row
constexpr int kMergeRegs = 16;   // candidates per lane of the merging wave (64 * 16 per row)

struct SplitWs {
  uint64_t* tmass;    // [rows][ntiles] tile masses (whole rows)
  uint64_t* cand;     // [rows][slices][kCandCap] candidates, index << 32 | key (top-k rows)
  float* smax;        // [rows][slices] slice maxima (whole rows)
  int32_t* ncand;     // [rows][slices] candidates per slice, -1: more than kCandCap
  int32_t* counter;   // [rows] slices finished
  int32_t* fallback;  // [rows] 1: handed back to the one-workgroup kernel
};
__host__ __device__ inline int split_tiles(int vocab) { return (vocab + kSplitTile - 1) / kSplitTile; }
__host__ __device__ inline int split_slices(int vocab) { return (split_tiles(vocab) + kSliceTiles - 1) / kSliceTiles; }
__host__ __device__ inline int64_t split_ws_bytes(int rows, int vocab) {
  const int64_t S = split_slices(vocab);
  return (int64_t)rows * (split_tiles(vocab) * 8 + S * kCandCap * 8 + S * 4 + S * 4 + 4 + 4);
}
__host__ __device__ inline SplitWs split_ws(void* ws, int rows, int vocab) {
  const int64_t S = split_slices(vocab);
  char* c = reinterpret_cast<char*>(ws);
  SplitWs w;
  w.tmass = reinterpret_cast<uint64_t*>(c);
  c += (int64_t)rows * split_tiles(vocab) * 8;
  w.cand = reinterpret_cast<uint64_t*>(c);
  c += (int64_t)rows * S * kCandCap * 8;
  w.smax = reinterpret_cast<float*>(c);
  c += (int64_t)rows * S * 4;
  w.ncand = reinterpret_cast<int32_t*>(c);
  c += (int64_t)rows * S * 4;
  w.counter = reinterpret_cast<int32_t*>(c);
  c += (int64_t)rows * 4;
  w.fallback = reinterpret_cast<int32_t*>(c);
  return w;
}

// Thread t's 8 logits of tile j: indices j * kSplitTile + 8 t .. + 7 (ok: inside the row).
template <typename T>
__device__ __forceinline__ void load8(const T* p, int vocab, bool vec, int j, float (&x)[8], bool (&ok)[8]) {
  const int base = j * kSplitTile + 8 * (int)threadIdx.x;
  if (vec && base + 8 <= vocab) {
    T e[8];
#pragma unroll
    for (int v = 0; v < (int)(8 * sizeof(T) / 16); ++v) {
      const uint4 w = *reinterpret_cast<const uint4*>(p + base + v * (16 / sizeof(T)));
      __builtin_memcpy(e + v * (16 / sizeof(T)), &w, 16);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      x[k] = to_f32(e[k]);
      ok[k] = true;
    }
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      ok[k] = base + k < vocab;
      x[k] = ok[k] ? to_f32(p[base + k]) : 0.f;
    }
  }
}

// A slice's tiles for thread t, all loads issued before any is used: 16-byte vectors from
// clamped in-bounds addresses (a load under a divergent branch would be waited for at the
// branch's end, one tile at a time); get() then reads them, or the row with element loads
// where a vector would cross its end (or the row is not 16-byte aligned).
template <typename T>
struct SliceLoad {
  static constexpr int R = 8 * sizeof(T) / 16;  // vectors per thread per tile
  uint4 raw[kSliceTiles][R];
  __device__ __forceinline__ void issue(const T* p, int vocab, bool vec, int j0, int j1) {
    if (!(vec && vocab >= 8)) return;  // (uniform)
    const int last = (vocab - 8) / 8 * 8;
#pragma unroll
    for (int jj = 0; jj < kSliceTiles; ++jj) {
      const int j = min(j0 + jj, j1 - 1);
      const int base = min(j * kSplitTile + 8 * (int)threadIdx.x, last);
#pragma unroll
      for (int v = 0; v < R; ++v) raw[jj][v] = *reinterpret_cast<const uint4*>(p + base + v * (16 / sizeof(T)));
    }
  }
  __device__ __forceinline__ void get(const T* p, int vocab, bool vec, int j, int jj, float (&x)[8],
                                      bool (&ok)[8]) const {
    const int base = j * kSplitTile + 8 * (int)threadIdx.x;
    if (vec && vocab >= 8 && base + 8 <= vocab) {
      T e[8];
      __builtin_memcpy(e, raw[jj], 8 * sizeof(T));
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        x[k] = to_f32(e[k]);
        ok[k] = true;
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        ok[k] = base + k < vocab;
        x[k] = ok[k] ? to_f32(p[base + k]) : 0.f;
      }
    }
  }
};

__device__ __forceinline__ float block_max256(float v, float* red) {
  v = wave_max_f32(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
__device__ __forceinline__ uint64_t block_sum256(uint64_t v, uint64_t* red) {
  v = wave_sum_u64(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

template <typename T>
__global__ __launch_bounds__(kSplitThreads) void split_max_kernel(const T* logits, int64_t row_stride, int vocab,
                                                                  const int32_t* top_k, int32_t top_k_all,
                                                                  const float* top_p, float top_p_all,
                                                                  SplitWs ws) {
  __shared__ float red[4];
  const int s = blockIdx.x, b = blockIdx.y, S = gridDim.x, ntiles = split_tiles(vocab);
  if (s == 0 && threadIdx.x == 0) {  // (read by the later launches on this stream)
    ws.counter[b] = 0;
    ws.fallback[b] = 0;
  }
  if (row_kind(b, vocab, top_k, top_k_all, top_p, top_p_all) != kWholeRow) return;
  const T* p = logits + (int64_t)b * row_stride;
  const bool vec = ((uintptr_t)p % 16) == 0;
  float mx = -INFINITY;
  const int j0 = s * kSliceTiles, j1 = min(j0 + kSliceTiles, ntiles);
  SliceLoad<T> sl;
  sl.issue(p, vocab, vec, j0, j1);
#pragma unroll
  for (int jj = 0; jj < kSliceTiles; ++jj) {
    if (j0 + jj >= j1) break;  // (uniform)
    float x[8];
    bool ok[8];
    sl.get(p, vocab, vec, j0 + jj, jj, x, ok);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (ok[k]) mx = fmaxf(mx, x[k]);
  }
  mx = block_max256(mx, red);
  if (threadIdx.x == 0) ws.smax[(int64_t)b * S + s] = mx;
}

template <typename T>
__global__ __launch_bounds__(kSplitThreads) void split_sample_kernel(const T* logits, int64_t row_stride, int vocab,
                                                                     const int32_t* top_k, int32_t top_k_all,
                                                                     const float* top_p, float top_p_all,
                                                                     const float* uniform, int32_t* out, SplitWs ws) {
  __shared__ float redf[4];
  __shared__ uint64_t redu[4];
  __shared__ uint64_t s_tile[kMaxSplitTiles];
  __shared__ int s_last;
  const int s = blockIdx.x, b = blockIdx.y, S = gridDim.x, ntiles = split_tiles(vocab);
  if (row_kind(b, vocab, top_k, top_k_all, top_p, top_p_all) != kWholeRow) return;
  const T* p = logits + (int64_t)b * row_stride;
  const bool vec = ((uintptr_t)p % 16) == 0;
  // this slice's logits (requested first), and the row's largest logit from the slices'
  // (written by the previous launch)
  const int j0 = s * kSliceTiles, j1 = min(j0 + kSliceTiles, ntiles);
  SliceLoad<T> sl;
  sl.issue(p, vocab, vec, j0, j1);
  float mx = -INFINITY;
  for (int i = threadIdx.x; i < S; i += kSplitThreads) mx = fmaxf(mx, ws.smax[(int64_t)b * S + i]);
  mx = block_max256(mx, redf);
  // this slice's tile masses, written through to device scope
  uint64_t* tm = ws.tmass + (int64_t)b * ntiles;
#pragma unroll
  for (int jj = 0; jj < kSliceTiles; ++jj) {
    if (j0 + jj >= j1) break;  // (uniform)
    float x[8];
    bool ok[8];
    sl.get(p, vocab, vec, j0 + jj, jj, x, ok);
    uint64_t m = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (ok[k]) m += fmass(x[k], mx);
    m = block_sum256(m, redu);
    if (threadIdx.x == 0) __hip_atomic_store(tm + j0 + jj, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // arrival: the last slice of the row to finish samples it
  if (threadIdx.x == 0) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // this slice's tile masses are complete (device-visible)
    const int old = atomicAdd(&ws.counter[b], 1);
    s_last = old == S - 1;
  }
  __syncthreads();
  if (!s_last) return;
  for (int j = threadIdx.x; j < ntiles; j += kSplitThreads)
    s_tile[j] = __hip_atomic_load(tm + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  uint64_t ms = 0;
  for (int j = 0; j < ntiles; ++j) ms += s_tile[j];  // (every thread: uniform)
  if (ms == 0) {
    if (threadIdx.x == 0) out[b] = -1;  // (no token carries mass: an all-NaN row)
    return;
  }
  const double uu = fminf(fmaxf(uniform[b], 0.f), 1.f);
  uint64_t target = (uint64_t)(uu * (double)ms);
  if (target >= ms) target = ms - 1;
  int tt = 0;
  uint64_t before = 0;
  while (tt < ntiles - 1 && before + s_tile[tt] <= target) before += s_tile[tt++];
  // inside tile tt: each thread's mass, exclusive scan in thread (= vocabulary) order, then the
  // owner walks its 8 logits
  float x[8];
  bool ok[8];
  load8(p, vocab, vec, tt, x, ok);
  uint64_t mine = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (ok[k]) mine += fmass(x[k], mx);
  uint64_t inc = mine;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t v = __shfl_up(inc, o, kWave);
    if (lane >= o) inc += v;
  }
  __syncthreads();
  if (lane == 63) redu[wv] = inc;
  __syncthreads();
  uint64_t off = before;
  for (int i = 0; i < wv; ++i) off += redu[i];
  const uint64_t start = off + inc - mine;
  if (mine > 0 && start <= target && target < start + mine) {
    uint64_t run = start;
    int found = -1;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (found < 0 && ok[k]) {
        run += fmass(x[k], mx);
        if (run > target) found = tt * kSplitTile + 8 * (int)threadIdx.x + k;
      }
    }
    out[b] = found;
  }
}

__device__ __forceinline__ int block_sum_i256(int v, int* red) {
  v = wave_sum_i32(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}
__device__ __forceinline__ uint32_t block_max_u256(uint32_t v, uint32_t* red) {
  v = wave_max_u32(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return max(max(red[0], red[1]), max(red[2], red[3]));
}
// The float whose fkey is k (k != 0).
__device__ __forceinline__ float key_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// ---- Top-k rows (0 < k <= kTopKMax, any top-p) over many workgroups per row, one launch.
// Each (slice, row) workgroup holds its slice's keys in registers and bisects for a key t_s
// with k <= #{key >= t_s} <= kCandCap (or takes every non-NaN logit when there are at most
// kCandCap of them), and hands those logits over as candidates.  No slice can hold k logits
// above the row's k-th largest key T*, so t_s <= T* and every logit with key >= T* is a
// candidate: over the candidates, the largest T with #{key >= T} >= k is T* itself.  The last
// slice of the row to finish then runs sample_row's rule on the candidates alone: T*, the top-p
// threshold (the largest T with mass{key >= T} >= need, as its mass-weighted selection finds),
// and the inverse CDF in vocabulary order, with the same integer masses, so the token is the
// same.  One wave does that merge with shuffle reductions (a search takes up to 32 steps, and
// workgroup barriers at every step made it the kernel's critical path); slices hand over between
// k and 2k logits to keep the candidates within its registers.  Rows it cannot finish this way
// (a slice's ties beyond kCandCap, more candidates than the wave holds, fewer than k finite
// logits, a kept set beyond kKeptCap) are handed back to sample_kernel through `fallback`.
constexpr int kKeptCap = 1024;
constexpr int kRadixBins = 2048;  // the largest digit (11 bits) of the merge's radix selection

template <typename T>
__global__ __launch_bounds__(kSplitThreads) __attribute__((amdgpu_waves_per_eu(5))) void split_topk_kernel(
    const T* logits, int64_t row_stride, int vocab,
                                                                   const int32_t* top_k, int32_t top_k_all,
                                                                   const float* top_p, float top_p_all,
                                                                   const float* uniform, int32_t* out, SplitWs ws) {
  __shared__ __align__(16) int s_h[kRadixBins];
  __shared__ int s_wsum[kSplitThreads / kWave];
  __shared__ int s_n, s_dig, s_above, s_cnt, s_total;
  const int s = blockIdx.x, b = blockIdx.y, S = gridDim.x, ntiles = split_tiles(vocab);
  if (row_kind(b, vocab, top_k, top_k_all, top_p, top_p_all) != kTopKRow) return;
  const int k = top_k ? top_k[b] : top_k_all;
  const T* p = logits + (int64_t)b * row_stride;
  const bool vec = ((uintptr_t)p % 16) == 0;
  const int t = threadIdx.x, lane = t & (kWave - 1), wv = t / kWave;
  // the slice's keys (0: past the row's end, or NaN)
  const int j0 = s * kSliceTiles, j1 = min(j0 + kSliceTiles, ntiles);
  SliceLoad<T> sl;
  sl.issue(p, vocab, vec, j0, j1);
  // The slice's keys, cut to their 16 most significant bits (still in the logits' order, ties
  // merged) and packed two to a register: key i in the half i & 1 of kp[i / 2] (0: past the
  // row's end, or NaN).  Held as 16 bits, every slice's workgroup of the batch is resident at
  // once; a candidate's full key is recomputed from its logit when it is handed over.
  uint32_t kp[kSliceTiles * 4];
#pragma unroll
  for (int jj = 0; jj < kSliceTiles; ++jj) {
    float x[8];
    bool ok[8];
    if (j0 + jj < j1) {
      sl.get(p, vocab, vec, j0 + jj, jj, x, ok);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) ok[e] = false;
    }
#pragma unroll
    for (int e = 0; e < 8; e += 2)
      kp[jj * 4 + e / 2] = (ok[e] ? fkey(x[e]) >> 16 : 0u) | (ok[e + 1] ? fkey(x[e + 1]) & 0xFFFF0000u : 0u);
  }
  auto key16 = [&](int i) __attribute__((always_inline)) -> uint32_t {
    return (i & 1) ? kp[i >> 1] >> 16 : kp[i >> 1] & 0xFFFFu;
  };
  // The threshold t_s: the start of the range of 16-bit keys (a digit of 11 bits, then one of 5)
  // that holds the slice's k-th largest, refined until at most 2k keys lie at or above it: each
  // level histograms, in LDS, the keys inside the range chosen so far, and one scan of the
  // histogram finds the digit (where a bisection counted every key once per halving, with a
  // workgroup reduction each time).  Keys at or above t_s include every logit at or above the
  // slice's k-th largest, so every logit at or above the row's k-th largest is a candidate.
  uint32_t ts = 1u, prefix = 0u, himask = 0u;
  int above = 0, cnt = 0;
#pragma unroll 1
  for (int level = 0; level < 2; ++level) {
    const int shift = level == 0 ? 5 : 0;
    const uint32_t nb = level == 0 ? 2048u : 32u;
#pragma unroll
    for (int i = 0; i < kRadixBins / kSplitThreads / 4; ++i)
      reinterpret_cast<int4*>(s_h)[t * (kRadixBins / kSplitThreads / 4) + i] = make_int4(0, 0, 0, 0);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kSliceTiles * 8; ++i) {
      const uint32_t kk = key16(i);
      if (kk != 0u && (kk & himask) == prefix) atomicAdd(&s_h[(kk >> shift) & (nb - 1u)], 1);
    }
    __syncthreads();
    // thread t owns bins [8t, 8t + 8); the count in its bins and in every bin above them
    int bins[8];
    {
      const int4 a = reinterpret_cast<const int4*>(s_h)[2 * t], c = reinterpret_cast<const int4*>(s_h)[2 * t + 1];
      bins[0] = a.x; bins[1] = a.y; bins[2] = a.z; bins[3] = a.w;
      bins[4] = c.x; bins[5] = c.y; bins[6] = c.z; bins[7] = c.w;
    }
    int own = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) own += bins[e];
    int incl = own;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int v = __shfl_down(incl, o, kWave);
      incl += lane + o < kWave ? v : 0;
    }
    if (lane == 0) s_wsum[wv] = incl;
    __syncthreads();
    for (int w2 = wv + 1; w2 < kSplitThreads / kWave; ++w2) incl += s_wsum[w2];
    if (t == 0) s_total = incl;  // (thread 0's: every key in the range)
    if (above + incl >= k && above + incl - own < k) {  // the thread whose bins hold the k-th largest
      int acc = above + incl - own;
#pragma unroll
      for (int e = 7; e >= 0; --e) {
        if (acc + bins[e] >= k) {
          s_dig = 8 * t + e;
          s_above = acc;
          s_cnt = acc + bins[e];
          break;
        }
        acc += bins[e];
      }
    }
    __syncthreads();
    if (level == 0 && s_total < k) {  // (uniform) fewer than k finite keys: all of them
      ts = 1u;
      cnt = s_total;
      break;
    }
    cnt = s_cnt;
    prefix |= (uint32_t)s_dig << shift;
    himask |= (nb - 1u) << shift;
    above = s_above;
    ts = prefix;
    if (cnt <= 2 * k) break;  // (uniform) at most 2k keys at or above ts
    __syncthreads();  // (s_dig, s_above, s_cnt read by every thread before the next level writes them)
  }
  const bool bad = cnt > kCandCap;  // (ties at the threshold beyond the slice's capacity)
  if (t == 0) s_n = 0;
  __syncthreads();
  uint64_t* cand = ws.cand + ((int64_t)b * S + s) * kCandCap;
  if (!bad) {
#pragma unroll
    for (int i = 0; i < kSliceTiles * 8; ++i) {
      if (key16(i) >= ts) {
        const int pos = atomicAdd(&s_n, 1);
        const int idx = (j0 + i / 8) * kSplitTile + 8 * t + (i % 8);
        cand[pos] = ((uint64_t)(uint32_t)idx << 32) | fkey(to_f32(p[idx]));
      }
    }
  }
  __syncthreads();
  if (t == 0) ws.ncand[(int64_t)b * S + s] = bad ? -1 : s_n;
}

// The merge of a top-k row's candidates (the launch after split_topk_kernel), one wave per row:
// the row's k-th largest key T* over its slices' candidates, the top-p threshold over the top-k
// set, and the inverse CDF in vocabulary order, with sample_row's integer masses, so the token is
// the same.  A launch of its own rather than the last slice to finish: the slice kernel then
// holds only its slice's keys and a chip's worth of its workgroups are resident at once.
__global__ __launch_bounds__(kWave) void split_topk_merge_kernel(int vocab, const int32_t* top_k, int32_t top_k_all,
                                                                 const float* top_p, float top_p_all,
                                                                 const float* uniform, int32_t* out, SplitWs ws) {
  __shared__ int s_off[kMaxSplitTiles / kSliceTiles + 1];
  __shared__ int s_sidx[kKeptCap];
  __shared__ uint64_t s_smass[kKeptCap];
  __shared__ uint32_t s_skey[kKeptCap];
  __shared__ __align__(16) int s_hist[kRadixBins];  // (16-byte vector accesses)
  const int b = blockIdx.x, S = split_slices(vocab);
  if (row_kind(b, vocab, top_k, top_k_all, top_p, top_p_all) != kTopKRow) return;
  const int k = top_k ? top_k[b] : top_k_all;
  const int lane = threadIdx.x;
  if (lane == 0) ws.fallback[b] = 0;
  // the slices' candidate counts, 64 at a time, and their running offsets
  int off = 0, anybad = 0;
  for (int i0 = 0; i0 < S; i0 += kWave) {
    const int i = i0 + lane;
    const int c = i < S ? ws.ncand[(int64_t)b * S + i] : 0;
    anybad |= c < 0 ? 1 : 0;
    const int cc = c < 0 ? 0 : c;
    int incl = cc;  // inclusive prefix over the lanes below
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int v = __shfl_up(incl, o, kWave);
      incl += lane >= o ? v : 0;
    }
    if (i < S) s_off[i] = off + incl - cc;
    off += __shfl(incl, kWave - 1, kWave);
  }
  if (lane == 0) s_off[S] = off;
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the offsets are in LDS for every lane
  __builtin_amdgcn_wave_barrier();
  const int n = off;
  if (wave_max_u32((uint32_t)anybad) || n == 0 || n > kWave * kMergeRegs) {
    if (lane == 0) ws.fallback[b] = 1;
    return;
  }
  auto wsum_i = [](int v) __attribute__((always_inline)) { return wave_sum_i32(v); };
  auto wmax_u = [](uint32_t v) __attribute__((always_inline)) { return wave_max_u32(v); };
  uint32_t ck[kMergeRegs];
  int cidx[kMergeRegs];
  // the slice holding candidate lane + 64 r and its first candidate's offset: the slices' offsets
  // come to every lane through scalar registers (one readlane each), in slice order
  int csl[kMergeRegs], cso[kMergeRegs];
#pragma unroll
  for (int r = 0; r < kMergeRegs; ++r) csl[r] = cso[r] = 0;
  for (int i0 = 0; i0 < S; i0 += kWave) {
    const int offv = i0 + lane < S ? s_off[i0 + lane] : 0;
    const int nin = min(kWave, S - i0);
    for (int ii = 0; ii < nin; ++ii) {
      const int oi = __builtin_amdgcn_readlane(offv, ii);
#pragma unroll
      for (int r = 0; r < kMergeRegs; ++r) {
        if (oi <= min(lane + kWave * r, n - 1)) {
          csl[r] = i0 + ii;
          cso[r] = oi;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kMergeRegs; ++r) {  // unconditional loads of clamped candidates
    const int ci = min(lane + kWave * r, n - 1);
    const uint64_t v = ws.cand[((int64_t)b * S + csl[r]) * kCandCap + (ci - cso[r])];
    const bool real = lane + kWave * r < n;
    ck[r] = real ? (uint32_t)v : 0u;
    cidx[r] = (int)(v >> 32);
  }
  uint32_t mxk = 0;
  int nfin = 0;
#pragma unroll
  for (int r = 0; r < kMergeRegs; ++r) {
    mxk = max(mxk, ck[r]);
    nfin += ck[r] != 0u ? 1 : 0;
  }
  mxk = wmax_u(mxk);
  if (wsum_i(nfin) < k) {  // K would take NaN logits: not a candidate case
    if (lane == 0) ws.fallback[b] = 1;
    return;
  }
  // The k-th largest key T* (ties kept): the largest T with #{key >= T} >= k, by radix
  // selection over the bits in which the candidates' keys differ (the others are those of the
  // largest key, and so of T*), in digits of up to 11 bits from the most significant: a
  // histogram of the candidates that agree with the digits chosen so far, then the digit at
  // which the count from the top reaches k.  One to three histograms replace the up to 32
  // halvings of a bisection, each of which was a wave-wide reduction in turn.
  uint32_t diff = 0;  // the bits in which some finite candidate differs from the largest
#pragma unroll
  for (int r = 0; r < kMergeRegs; ++r) diff |= ck[r] != 0u ? ck[r] ^ mxk : 0u;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) diff |= (uint32_t)__shfl_xor((int)diff, o, kWave);
  diff = (uint32_t)__builtin_amdgcn_readfirstlane((int)diff);
  uint32_t thr = mxk;
  if (diff != 0u) {
    const int top = 32 - __builtin_clz(diff), bot = __builtin_ctz(diff);  // bits [bot, top) vary
    thr = mxk & ~((top == 32 ? ~0u : ((1u << top) - 1u)) & ~((1u << bot) - 1u));
    int above = 0;  // candidates above the digits chosen so far
    for (int hi = top; hi > bot;) {
      const int width = min(hi - bot, 11), shift = hi - width;
      const uint32_t nb = 1u << width;
      const uint32_t himask = hi == 32 ? 0u : ~0u << hi;  // the bits above this digit
      hi = shift;
      int4* hv = reinterpret_cast<int4*>(s_hist + lane * 32);  // this lane's 32 bins, 4 a vector
#pragma unroll
      for (int i = 0; i < 8; ++i) hv[i] = make_int4(0, 0, 0, 0);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int r = 0; r < kMergeRegs; ++r)
        if (ck[r] != 0u && (ck[r] & himask) == (thr & himask))
          atomicAdd(&s_hist[(ck[r] >> shift) & (nb - 1u)], 1);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_wave_barrier();
      // this lane's bins [32 lane, 32 lane + 32), in registers; the count in the bins of the
      // lanes above
      int bins[32];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int4 v = hv[i];
        bins[4 * i] = v.x;
        bins[4 * i + 1] = v.y;
        bins[4 * i + 2] = v.z;
        bins[4 * i + 3] = v.w;
      }
      int own = 0;
#pragma unroll
      for (int i = 0; i < 32; ++i) own += bins[i];
      int incl = own;  // bins of this lane and every lane above it
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const int v = __shfl_down(incl, o, kWave);
        incl += lane + o < kWave ? v : 0;
      }
      const bool mine = above + incl >= k && above + incl - own < k;
      int dig = 0, abv = 0;
      {
        int acc = above + incl - own;
        bool found = false;
#pragma unroll
        for (int i = 31; i >= 0; --i) {
          const bool hit = !found && acc + bins[i] >= k;
          dig = hit ? lane * 32 + i : dig;
          abv = hit ? acc : abv;
          found = found || hit;
          acc += bins[i];
        }
      }
      const uint64_t who = __ballot(mine);
      const int src = (int)__builtin_ctzll(who);
      dig = __shfl(dig, src, kWave);
      above = __shfl(abv, src, kWave);
      thr |= (uint32_t)dig << shift;
    }
  }
  const float mx = key_float(mxk);
  // the top-k set K, compacted into LDS in a fixed order (ballots): index, key, mass
  uint64_t kmass = 0;
  int m = 0;
#pragma unroll
  for (int r = 0; r < kMergeRegs; ++r) {
    const bool keep = ck[r] >= thr;
    const uint64_t bal = __ballot(keep);
    const uint64_t cm = keep ? fmass(key_float(ck[r]), mx) : 0;
    if (keep) {
      const int pos = m + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                         __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
      if (pos < kKeptCap) {
        s_sidx[pos] = cidx[r];
        s_skey[pos] = ck[r];
        s_smass[pos] = cm;
      }
    }
    kmass += cm;
    m += __popcll(bal);
  }
  kmass = wave_sum_u64(kmass);
  if (m > kKeptCap) {
    if (lane == 0) ws.fallback[b] = 1;
    return;
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // K is in LDS for every lane
  __builtin_amdgcn_wave_barrier();
  // The top-p threshold over K: the largest T with mass{key >= T} >= need, which is the key of
  // one of K's members; each lane weighs its members' keys over all of K.
  uint64_t ms = kmass;
  const float pp = top_p ? top_p[b] : top_p_all;
  if (pp < 1.f && kmass > 0) {
    const double needd = ceil((double)fmaxf(pp, 0.f) * (double)kmass);
    uint64_t need = needd < 1.0 ? 1 : (uint64_t)needd;
    if (need > kmass) need = kmass;
    uint32_t tp = 0;
    for (int e0 = 0; e0 < m; e0 += kWave) {
      const int e = e0 + lane;
      const uint32_t ke = e < m ? s_skey[e] : ~0u;
      uint64_t f = 0;  // mass{key >= ke} over K, its members taken 64 at a time through readlane
      for (int x0 = 0; x0 < m; x0 += kWave) {
        const uint32_t kx = x0 + lane < m ? s_skey[x0 + lane] : 0u;
        const uint64_t mx2 = x0 + lane < m ? s_smass[x0 + lane] : 0;
        const uint32_t mlo = (uint32_t)mx2, mhi = (uint32_t)(mx2 >> 32);
        const int nx = min(kWave, m - x0);
#pragma unroll 8
        for (int xx = 0; xx < nx; ++xx) {
          const uint32_t kk = (uint32_t)__builtin_amdgcn_readlane(kx, xx);
          const uint64_t mm = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(mhi, xx) << 32) |
                              (uint64_t)(uint32_t)__builtin_amdgcn_readlane(mlo, xx);  // (readlane is signed)
          f += kk >= ke ? mm : 0;
        }
      }
      if (e < m && f >= need) tp = max(tp, ke);
    }
    tp = wmax_u(tp);
    if (tp > thr) {  // the kept set shrinks to S = {key >= tp}: recompact it in place, in order
      thr = tp;
      int n2 = 0;
      uint64_t m2 = 0;
      for (int e0 = 0; e0 < m; e0 += kWave) {
        const int e = e0 + lane;
        const bool keep = e < m && s_skey[e] >= thr;
        const int ie = keep ? s_sidx[e] : 0;
        const uint32_t kk = keep ? s_skey[e] : 0u;
        const uint64_t mm = keep ? s_smass[e] : 0;
        const uint64_t bal = __ballot(keep);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_wave_barrier();  // (every lane has read its entry before any is moved)
        if (keep) {
          const int pos = n2 + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                              __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
          s_sidx[pos] = ie;
          s_skey[pos] = kk;
          s_smass[pos] = mm;
        }
        m2 += mm;
        n2 += __popcll(bal);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_wave_barrier();
      }
      m = n2;
      ms = wave_sum_u64(m2);
    }
  }
  if (ms == 0) {
    if (lane == 0) out[b] = -1;
    return;
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the kept set is in LDS for every lane
  __builtin_amdgcn_wave_barrier();
  const double uu = fminf(fmaxf(uniform[b], 0.f), 1.f);
  uint64_t target = (uint64_t)(uu * (double)ms);
  if (target >= ms) target = ms - 1;
  for (int e0 = 0; e0 < m; e0 += kWave) {
    const int e = e0 + lane;
    const int ie = e < m ? s_sidx[e] : 0x7fffffff;
    const uint64_t me = e < m ? s_smass[e] : 0;
    uint64_t pre = 0;  // mass of the kept logits before this one in vocabulary order, their members
                       // taken 64 at a time through readlane
    for (int f0 = 0; f0 < m; f0 += kWave) {
      const int fi = f0 + lane < m ? s_sidx[f0 + lane] : 0x7fffffff;
      const uint64_t fm = f0 + lane < m ? s_smass[f0 + lane] : 0;
      const uint32_t flo = (uint32_t)fm, fhi = (uint32_t)(fm >> 32);
      const int nf = min(kWave, m - f0);
#pragma unroll 8
      for (int ff = 0; ff < nf; ++ff) {
        const int ii = __builtin_amdgcn_readlane(fi, ff);
        const uint64_t mm = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(fhi, ff) << 32) |
                            (uint64_t)(uint32_t)__builtin_amdgcn_readlane(flo, ff);  // (readlane is signed)
        pre += ii < ie ? mm : 0;
      }
    }
    if (e < m && me > 0 && pre <= target && target < pre + me) out[b] = ie;
  }
}

template <typename T>
int launch_sample(const T* logits, int64_t row_stride, int rows, int vocab, const int32_t* top_k, int32_t top_k_all,
                  const float* top_p, float top_p_all, const float* uniform, int32_t* out, void* ws,
                  int64_t ws_bytes, hipStream_t s) {
  // which kinds of rows there are: scalars settle it on the host, per-row tensors need all
  bool any_whole = true, any_topk = true, any_other = true;
  if (!top_k && !top_p) {
    const int kind = row_kind_of(top_k_all, top_p_all, vocab);
    any_whole = kind == kWholeRow;
    any_topk = kind == kTopKRow;
    any_other = kind == kOtherRow;
  }
  const bool split = ws && (any_whole || any_topk) && rows <= 65535 && split_tiles(vocab) <= kMaxSplitTiles &&
                     ws_bytes >= split_ws_bytes(rows, vocab);
  SplitWs w{};
  if (split) {
    w = split_ws(ws, rows, vocab);
    const dim3 grid((unsigned)split_slices(vocab), (unsigned)rows);
    // (split_max_kernel also resets every row's counter and fallback flag for the kernels below;
    // the top-k merge sets its rows' flags itself, so a batch of top-k rows alone skips it)
    if (any_whole) {
      hipLaunchKernelGGL(split_max_kernel<T>, grid, dim3(kSplitThreads), 0, s, logits, row_stride, vocab, top_k,
                         top_k_all, top_p, top_p_all, w);
      hipLaunchKernelGGL(split_sample_kernel<T>, grid, dim3(kSplitThreads), 0, s, logits, row_stride, vocab, top_k,
                         top_k_all, top_p, top_p_all, uniform, out, w);
    }
    if (any_topk) {
      hipLaunchKernelGGL(split_topk_kernel<T>, grid, dim3(kSplitThreads), 0, s, logits, row_stride, vocab, top_k,
                         top_k_all, top_p, top_p_all, uniform, out, w);
      hipLaunchKernelGGL(split_topk_merge_kernel, dim3((unsigned)rows), dim3(kWave), 0, s, vocab, top_k, top_k_all,
                         top_p, top_p_all, uniform, out, w);
    }
  }
  if (!split || any_other || any_topk)  // (top-k rows may be handed back)
    hipLaunchKernelGGL(sample_kernel<T>, dim3(rows), dim3(kThreads), 0, s, logits, row_stride, vocab, top_k,
                       top_k_all, top_p, top_p_all, uniform, out, split ? 1 : 0, w.fallback);
  return (int)hipGetLastError();
}

// The serving loop's scaling before sampling (ecahlang/main.py:169-170, 483-487), in one pass:
//   out[b][i] = float32(T(logits[b][i] / penalty[penalty_rows[b]][i])) / temperature[b]
// (`logits / mask_penalty` in the logits' dtype T, then `/ temperature` with a float32
// temperature, which promotes to float32).  Both divisions are IEEE divisions, as the tensor
// ops do them; a penalty or temperature of 1 leaves the value unchanged (x / 1 == x).  One
// thread per 8 logits; memory-bound.
template <typename T, bool VEC>
__global__ void scale_logits_kernel(const T* __restrict__ logits, int64_t row_stride, int vocab,
                                    const T* __restrict__ penalty, int64_t penalty_stride, int penalty_slots,
                                    const int32_t* __restrict__ penalty_rows, const float* __restrict__ temperature,
                                    float* __restrict__ out, int64_t out_stride) {
  constexpr int N = 8;  // logits per thread: 16 bytes of fp16 / bf16, two 16-byte vectors of fp32
  const int b = blockIdx.y;
  const int i0 = (blockIdx.x * blockDim.x + threadIdx.x) * N;
  if (i0 >= vocab) return;
  const T* x = logits + (int64_t)b * row_stride;
  const int prow = penalty ? penalty_rows[b] : 0;
  const T* pen = penalty ? penalty + (int64_t)prow * penalty_stride : nullptr;
  const float t = temperature ? temperature[b] : 1.f;
  float* o = out + (int64_t)b * out_stride;
  if (penalty && (prow < 0 || prow >= penalty_slots)) {  // no such penalty row: the row reads as NaN
    for (int k = 0; k < N && i0 + k < vocab; ++k) o[i0 + k] = __builtin_nanf("");
    return;
  }
  auto scale = [&](T xv, T pv) __attribute__((always_inline)) -> float {
    float y = to_f32(xv);
    if (pen) {
      const float d = to_f32(pv);
      if (d != 1.f) y = to_f32(from_f32<T>(y / d));
    }
    if (t != 1.f) y = y / t;
    return y;
  };
  if (VEC && i0 + N <= vocab) {
    T xs[N], ps[N];
    static_assert(N * sizeof(T) % 16 == 0, "whole 16-byte vectors");
#pragma unroll
    for (int v = 0; v < (int)(N * sizeof(T) / 16); ++v) {
      const uint4 w = *reinterpret_cast<const uint4*>(x + i0 + v * (16 / sizeof(T)));
      __builtin_memcpy(xs + v * (16 / sizeof(T)), &w, 16);
      const uint4 pw = pen ? *reinterpret_cast<const uint4*>(pen + i0 + v * (16 / sizeof(T))) : make_uint4(0, 0, 0, 0);
      __builtin_memcpy(ps + v * (16 / sizeof(T)), &pw, 16);
    }
    float ys[N];
#pragma unroll
    for (int k = 0; k < N; ++k) ys[k] = scale(xs[k], ps[k]);
#pragma unroll
    for (int v = 0; v < N / 4; ++v)
      *reinterpret_cast<float4*>(o + i0 + 4 * v) = make_float4(ys[4 * v], ys[4 * v + 1], ys[4 * v + 2], ys[4 * v + 3]);
  } else {
    for (int k = 0; k < N && i0 + k < vocab; ++k) o[i0 + k] = scale(x[i0 + k], pen ? pen[i0 + k] : from_f32<T>(1.f));
  }
}

}  // namespace

extern "C" int pkv_scale_logits(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab, int32_t dtype,
                                const void* penalty, int64_t penalty_stride, int32_t penalty_slots,
                                const int32_t* penalty_rows, const float* temperature, float* out,
                                int64_t out_stride, void* stream) {
  if (rows < 0 || vocab <= 0 || row_stride < vocab || out_stride < vocab || !out) return kBadArg;
  if (penalty && (!penalty_rows || penalty_stride < vocab || penalty_slots <= 0)) return kBadArg;
  if (rows == 0) return kOk;
  if (rows > 65535) return kBadArg;
  const dim3 grid((unsigned)((vocab + 8 * 256 - 1) / (8 * 256)), (unsigned)rows);
  hipStream_t s = (hipStream_t)stream;
  const int es = dtype == kF32 ? 4 : 2;
  // 16-byte vectors when every row start is 16-byte aligned (base pointers and row strides)
  const bool vec = ((uintptr_t)logits % 16 == 0) && (row_stride * es % 16 == 0) && ((uintptr_t)out % 16 == 0) &&
                   (out_stride * 4 % 16 == 0) &&
                   (!penalty || (((uintptr_t)penalty % 16 == 0) && (penalty_stride * es % 16 == 0)));
#define PKV_SCALE(T)                                                                                          \
  do {                                                                                                        \
    if (vec)                                                                                                  \
      hipLaunchKernelGGL((scale_logits_kernel<T, true>), grid, dim3(256), 0, s, (const T*)logits, row_stride, \
                         vocab, (const T*)penalty, penalty_stride, penalty_slots, penalty_rows, temperature, out,  \
                         out_stride);                                                                         \
    else                                                                                                      \
      hipLaunchKernelGGL((scale_logits_kernel<T, false>), grid, dim3(256), 0, s, (const T*)logits, row_stride, \
                         vocab, (const T*)penalty, penalty_stride, penalty_slots, penalty_rows, temperature, out, \
                         out_stride);                                                                         \
  } while (0)
  if (dtype == kF16) PKV_SCALE(_Float16);
  else if (dtype == kBF16) PKV_SCALE(__hip_bfloat16);
  else if (dtype == kF32) PKV_SCALE(float);
  else return kBadDType;
#undef PKV_SCALE
  return (int)hipGetLastError();
}

static int sample_entry(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab, int32_t dtype,
                        const int32_t* top_k, int32_t top_k_all, const float* top_p, float top_p_all,
                        const float* uniform, int32_t* out, void* workspace, int64_t workspace_bytes,
                        void* stream) {
  if (rows < 0 || vocab <= 0 || row_stride < vocab || !uniform || !out) return kBadArg;
  if (rows == 0) return kOk;
  const int es = dtype == kF32 ? 4 : 2;
  if ((int64_t)vocab > (int64_t)kMaxTiles * kThreads * (16 / es)) return kBadArg;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == kF16)
    return launch_sample((const _Float16*)logits, row_stride, rows, vocab, top_k, top_k_all, top_p, top_p_all,
                         uniform, out, workspace, workspace_bytes, s);
  if (dtype == kBF16)
    return launch_sample((const __hip_bfloat16*)logits, row_stride, rows, vocab, top_k, top_k_all, top_p,
                         top_p_all, uniform, out, workspace, workspace_bytes, s);
  if (dtype == kF32)
    return launch_sample((const float*)logits, row_stride, rows, vocab, top_k, top_k_all, top_p, top_p_all,
                         uniform, out, workspace, workspace_bytes, s);
  return kBadDType;
}

extern "C" int pkv_top_k_top_p_sampling(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab,
                                        int32_t dtype, const int32_t* top_k, int32_t top_k_all,
                                        const float* top_p, float top_p_all, const float* uniform,
                                        int32_t* out, void* stream) {
  return sample_entry(logits, row_stride, rows, vocab, dtype, top_k, top_k_all, top_p, top_p_all, uniform, out,
                      nullptr, 0, stream);
}

extern "C" int64_t pkv_sampling_workspace_bytes(int32_t rows, int32_t vocab) {
  return rows > 0 && vocab > 0 ? split_ws_bytes(rows, vocab) : 0;
}

extern "C" int pkv_top_k_top_p_sampling_ws(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab,
                                           int32_t dtype, const int32_t* top_k, int32_t top_k_all,
                                           const float* top_p, float top_p_all, const float* uniform,
                                           int32_t* out, void* workspace, int64_t workspace_bytes, void* stream) {
  if (workspace && ((uintptr_t)workspace % 8)) return kBadAlign;
  return sample_entry(logits, row_stride, rows, vocab, dtype, top_k, top_k_all, top_p, top_p_all, uniform, out,
                      workspace, workspace_bytes, stream);
}
