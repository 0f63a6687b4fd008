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
  v = wave_max(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) red[w] = v;
  __syncthreads();
  float r = -INFINITY;
  for (int i = 0; i < kThreads / 64; ++i) r = fmaxf(r, red[i]);
  return r;
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
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

template <typename T>
__global__ __launch_bounds__(kThreads) void sample_kernel(const T* logits, int64_t row_stride, int vocab,
                                                          const int32_t* top_k, int32_t top_k_all,
                                                          const float* top_p, float top_p_all,
                                                          const float* uniform, int32_t* out) {
  __shared__ SampleLds L;
  const int b = blockIdx.x;
  const T* p = logits + (int64_t)b * row_stride;
  const Row<T> row{p, vocab, ((uintptr_t)p % 16) == 0};
  sample_row<T>(row, L, b, vocab, top_k, top_k_all, top_p, top_p_all, uniform, out);
}

template <typename T>
int launch_sample(const T* logits, int64_t row_stride, int rows, int vocab, const int32_t* top_k, int32_t top_k_all,
                  const float* top_p, float top_p_all, const float* uniform, int32_t* out, hipStream_t s) {
  hipLaunchKernelGGL(sample_kernel<T>, dim3(rows), dim3(kThreads), 0, s, logits, row_stride, vocab, top_k,
                     top_k_all, top_p, top_p_all, uniform, out);
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

extern "C" int pkv_top_k_top_p_sampling(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab,
                                        int32_t dtype, const int32_t* top_k, int32_t top_k_all,
                                        const float* top_p, float top_p_all, const float* uniform,
                                        int32_t* out, void* stream) {
  if (rows < 0 || vocab <= 0 || row_stride < vocab || !uniform || !out) return kBadArg;
  if (rows == 0) return kOk;
  const int es = dtype == kF32 ? 4 : 2;
  if ((int64_t)vocab > (int64_t)kMaxTiles * kThreads * (16 / es)) return kBadArg;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == kF16)
    return launch_sample((const _Float16*)logits, row_stride, rows, vocab, top_k, top_k_all, top_p, top_p_all,
                         uniform, out, s);
  if (dtype == kBF16)
    return launch_sample((const __hip_bfloat16*)logits, row_stride, rows, vocab, top_k, top_k_all, top_p,
                         top_p_all, uniform, out, s);
  if (dtype == kF32)
    return launch_sample((const float*)logits, row_stride, rows, vocab, top_k, top_k_all, top_p, top_p_all,
                         uniform, out, s);
  return kBadDType;
}
