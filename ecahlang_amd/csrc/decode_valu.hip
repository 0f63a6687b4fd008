// Generic paged attention on the vector ALUs: any of fp32 / fp16 / bf16, head_dim 64/128/256,
// GQA group up to 16.  It serves fp32 caches (where no 16-bit matrix instruction applies)
// and shapes the matrix-core kernels do not cover, for both decode and prefill.
//
// Decode semantics (FlashInfer BatchDecodeWithPagedKVCacheWrapper.run, called at
// ecahlang/main.py:68): o[b,h] = softmax(q[b,h] . K_b[:, h/g]^T * sm_scale) V_b[:, h/g] over the
// seq_len_b = (npages-1)*page_size + last_page_len tokens of sequence b, fp32 accumulation,
// output in the cache dtype.
//
// Prefill semantics (BatchPrefillWithPagedKVCacheWrapper.run with causal=True, planned at
// ecahlang/main.py:432-443): query row i of request b (0-based within the request) sees keys
// j <= i + kv_len_b - qo_len_b (bottom-right aligned); without causal it sees all kv_len_b keys.
//
// Organisation: 4 waves per workgroup; each wave owns one KV head at a time and the G query
// heads of its group.  Keys are scored 64 at a time with one token per lane (q read from LDS
// as a broadcast), the online-softmax state is wave-uniform, and P.V runs with the head
// dimension spread over lanes.
#include "attn_common.h"
#include "../../include/pagedkv.h"

using namespace pkv;

namespace {

constexpr int kWavesV = 4;

template <typename T> struct Vec16 { using type = uint4; static constexpr int n = 16 / sizeof(T); };

template <typename T>
__device__ __forceinline__ void load_row_f32(const T* p, float* dst, int n) {
  for (int j = 0; j < n; ++j) dst[j] = to_f32(p[j]);
}

// Online-softmax attention of one wave over tokens [t0, t1) of one sequence / KV head.
// q_lds: [G][D] floats pre-scaled to base-2 logits; p_lds: [G][64] scratch.
template <typename T, int D, int G>
__device__ void attend_tokens(const T* __restrict__ kc, const T* __restrict__ vc,
                              int64_t page_stride, const int32_t* __restrict__ pages,
                              int64_t npages_avail, int64_t num_pages, int ps,
                              int hkv, int h, int t0, int t1, const float* q_lds, float* p_lds,
                              float (&m)[G], float (&l)[G], float (&o)[G][D / 64], bool active) {
  constexpr int DPL = D / 64;
  constexpr int VE = Vec16<T>::n;  // elements per 16-byte vector
  const int lane = threadIdx.x & 63;
  for (int ts = t0; ts < t1; ts += 64) {
    int t = ts + lane;
    bool valid = active && t < t1;
    float s[G];
#pragma unroll
    for (int gi = 0; gi < G; ++gi) s[gi] = 0.f;
    int64_t page = -1;
    if (valid && t / ps < npages_avail) page = page_at(pages, t / ps, num_pages);
    valid = valid && page >= 0;
    if (valid) {
      const T* kp = kc + page * page_stride + ((int64_t)(t % ps) * hkv + h) * D;
      for (int d = 0; d < D; d += VE) {
        uint4 raw = *reinterpret_cast<const uint4*>(kp + d);
        const T* kv = reinterpret_cast<const T*>(&raw);
#pragma unroll
        for (int j = 0; j < VE; ++j) {
          float kf = to_f32(kv[j]);
#pragma unroll
          for (int gi = 0; gi < G; ++gi) s[gi] += q_lds[gi * D + d + j] * kf;
        }
      }
    }
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      float sv = valid ? s[gi] : -INFINITY;
      float mx = wave_max(sv);
      float mnew = fmaxf(m[gi], mx);
      float alpha = (m[gi] == -INFINITY) ? 0.f : exp2f(m[gi] - mnew);
      float p = (valid && mnew != -INFINITY) ? exp2f(sv - mnew) : 0.f;
      l[gi] = l[gi] * alpha + wave_sum(p);
      m[gi] = mnew;
      p_lds[gi * 64 + lane] = p;
#pragma unroll
      for (int j = 0; j < DPL; ++j) o[gi][j] *= alpha;
    }
    __syncthreads();
    int nv = t1 - ts < 64 ? t1 - ts : 64;
    if (active) {
      for (int tt = 0; tt < nv; ++tt) {
        int tok = ts + tt;
        int64_t page = tok / ps < npages_avail ? page_at(pages, tok / ps, num_pages) : -1;
        if (page < 0) continue;  // its score was masked: p == 0
        const T* vp = vc + page * page_stride + ((int64_t)(tok % ps) * hkv + h) * D + lane * DPL;
        float vf[DPL];
        load_row_f32(vp, vf, DPL);
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
          float p = p_lds[gi * 64 + tt];
#pragma unroll
          for (int j = 0; j < DPL; ++j) o[gi][j] += p * vf[j];
        }
      }
    }
    __syncthreads();
  }
}

template <typename T, int D, int G>
__device__ void load_q_group(const T* q, int64_t q_sh, int h, int g, float scale, float* q_lds) {
  const int lane = threadIdx.x & 63;
  for (int idx = lane; idx < G * D; idx += 64) {
    int gi = idx / D, d = idx - gi * D;
    q_lds[idx] = gi < g ? to_f32(q[(int64_t)(h * g + gi) * q_sh + d]) * scale : 0.f;
  }
}

template <typename T, int D, int G>
__global__ __launch_bounds__(256) void decode_valu_kernel(DecodeParams P) {
  constexpr int DPL = D / 64;
  extern __shared__ float smem[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  float* q_lds = smem + wave * G * (D + 64);
  float* p_lds = q_lds + G * D;
  __shared__ int flag;

  const int w = blockIdx.x;
  const int total = total_pages(P);
  if (w == 0) zero_empty_sequences<T, D>(P);
  if (total == 0) return;
  const int N = effective_ranges(P.num_ctas, total);
  if (w >= N) return;
  const Ranges R(N, total);
  int64_t p = R.start(w), end = R.start(w + 1);
  const int64_t first = P.indptr[0];  // pages before indptr[0] belong to no sequence
  if (p < first) p = first < end ? first : end;
  const int g = P.hq / P.hkv;
  const T* kc = reinterpret_cast<const T*>(P.k_cache);
  const T* vc = reinterpret_cast<const T*>(P.v_cache);
  const T* qb = reinterpret_cast<const T*>(P.q);
  T* out = reinterpret_cast<T*>(P.out);
  int b = find_seq_wave(P.indptr, P.batch, p);
  const int head_iters = (P.hkv + kWavesV - 1) / kWavesV;

  while (p < end) {
    const int s0 = P.indptr[b], s1 = P.indptr[b + 1];
    const int64_t seg_end = end < s1 ? end : s1;
    const int len = seq_len_of(P, b);
    const int t0 = (int)(p - s0) * P.ps;
    int t1 = (int)(seg_end - s0) * P.ps;
    if (t1 > len) t1 = len;
    const int w_lo = R.owner(s0), w_hi = R.owner(s1 - 1);
    const bool whole = w_lo == w_hi;
    const int64_t slot = (int64_t)w + b;

    for (int it = 0; it < head_iters; ++it) {
      const int h = it * kWavesV + wave;
      const bool active = h < P.hkv;
      if (active) load_q_group<T, D, G>(qb + b * P.q_sn, P.q_sh, h, g, P.scale_log2, q_lds);
      __syncthreads();
      float m[G], l[G], o[G][DPL];
#pragma unroll
      for (int gi = 0; gi < G; ++gi) {
        m[gi] = -INFINITY;
        l[gi] = 0.f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) o[gi][j] = 0.f;
      }
      attend_tokens<T, D, G>(kc, vc, P.page_stride, P.indices + s0, total - s0, P.num_pages, P.ps,
                             P.hkv, active ? h : 0, t0, t1, q_lds, p_lds, m, l, o, active);
      if (active) {
        for (int gi = 0; gi < g && gi < G; ++gi) {
          int hq = h * g + gi;
          float inv = l[gi] > 0.f ? 1.f / l[gi] : 0.f;
          if (whole) {
#pragma unroll
            for (int j = 0; j < DPL; ++j)
              out[b * P.o_sn + hq * P.o_sh + lane * DPL + j] = from_f32<T>(o[gi][j] * inv);
          } else {
            int64_t s = slot * P.hq + hq;
#pragma unroll
            for (int j = 0; j < DPL; ++j) st_dev(P.part_o + s * D + lane * DPL + j, o[gi][j] * inv);
            if (lane == 0) store_partial_ml(P, slot, hq, m[gi], l[gi]);
          }
        }
      }
      __syncthreads();
    }
    if (!whole && arrive_last(P, b, w_hi - w_lo + 1, &flag)) merge_partials<T, D>(P, b, w_lo + b, w_hi - w_lo + 1);
    p = seg_end;
    ++b;
    while (b < P.batch && P.indptr[b + 1] <= p) ++b;
  }
}

// Prefill: one workgroup per query row, all KV heads; the row's visible key count decides
// the token range, and the output is written directly (no split).
struct PrefillParams {
  const void* q;
  int64_t q_sn, q_sh;
  const int32_t* qo_indptr;
  const void* k_cache;
  const void* v_cache;
  int64_t page_stride;
  int64_t num_pages;
  int64_t num_indices;
  const int32_t* indptr;
  const int32_t* indices;
  const int32_t* last;
  int32_t batch, hq, hkv, ps, causal, nnz;
  float scale_log2;
  void* out;
  int64_t o_sn, o_sh;
};

template <typename T, int D, int G>
__global__ __launch_bounds__(256) void prefill_valu_kernel(PrefillParams P) {
  constexpr int DPL = D / 64;
  extern __shared__ float smem[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float* q_lds = smem + wave * G * (D + 64);
  float* p_lds = q_lds + G * D;
  const int row = blockIdx.x;
  if (row >= P.nnz) return;
  const int b = upper_index(P.qo_indptr, P.batch, row);
  const int qo_len = P.qo_indptr[b + 1] - P.qo_indptr[b];
  const int i = row - P.qo_indptr[b];
  const int s0 = P.indptr[b], np = P.indptr[b + 1] - s0;
  const int kv_len = np > 0 ? (np - 1) * P.ps + P.last[b] : 0;
  int vis = P.causal ? i + kv_len - qo_len + 1 : kv_len;
  vis = vis < 0 ? 0 : (vis > kv_len ? kv_len : vis);
  const int g = P.hq / P.hkv;
  const T* kc = reinterpret_cast<const T*>(P.k_cache);
  const T* vc = reinterpret_cast<const T*>(P.v_cache);
  const T* qb = reinterpret_cast<const T*>(P.q) + row * P.q_sn;
  T* out = reinterpret_cast<T*>(P.out);
  const int head_iters = (P.hkv + kWavesV - 1) / kWavesV;
  for (int it = 0; it < head_iters; ++it) {
    const int h = it * kWavesV + wave;
    const bool active = h < P.hkv;
    if (active) load_q_group<T, D, G>(qb, P.q_sh, h, g, P.scale_log2, q_lds);
    __syncthreads();
    float m[G], l[G], o[G][DPL];
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      m[gi] = -INFINITY;
      l[gi] = 0.f;
#pragma unroll
      for (int j = 0; j < DPL; ++j) o[gi][j] = 0.f;
    }
    attend_tokens<T, D, G>(kc, vc, P.page_stride, P.indices + s0, P.num_indices - s0, P.num_pages,
                           P.ps, P.hkv, active ? h : 0, 0, vis, q_lds, p_lds, m, l, o, active);
    if (active) {
      for (int gi = 0; gi < g && gi < G; ++gi) {
        float inv = l[gi] > 0.f ? 1.f / l[gi] : 0.f;
#pragma unroll
        for (int j = 0; j < DPL; ++j)
          out[row * P.o_sn + (h * g + gi) * P.o_sh + lane * DPL + j] = from_f32<T>(o[gi][j] * inv);
      }
    }
    __syncthreads();
  }
}

template <typename T, int D>
int launch_decode_valu_d(const DecodeParams& P, int g, hipStream_t s) {
  int G = g <= 1 ? 1 : g <= 2 ? 2 : g <= 4 ? 4 : g <= 8 ? 8 : g <= 16 ? 16 : 0;
  if (!G) return kBadGroup;
  size_t lds = (size_t)kWavesV * G * (D + 64) * sizeof(float);
#define PKV_DV(GG)                                                                            \
  hipLaunchKernelGGL((decode_valu_kernel<T, D, GG>), dim3(P.num_ctas), dim3(256), lds, s, P); \
  break
  switch (G) {
    case 1: PKV_DV(1);
    case 2: PKV_DV(2);
    case 4: PKV_DV(4);
    case 8: PKV_DV(8);
    default: PKV_DV(16);
  }
#undef PKV_DV
  return (int)hipGetLastError();
}

template <typename T, int D>
int launch_prefill_valu_d(const PrefillParams& P, int g, hipStream_t s) {
  int G = g <= 1 ? 1 : g <= 2 ? 2 : g <= 4 ? 4 : g <= 8 ? 8 : g <= 16 ? 16 : 0;
  if (!G) return kBadGroup;
  size_t lds = (size_t)kWavesV * G * (D + 64) * sizeof(float);
#define PKV_PV(GG)                                                                           \
  hipLaunchKernelGGL((prefill_valu_kernel<T, D, GG>), dim3(P.nnz), dim3(256), lds, s, P);    \
  break
  switch (G) {
    case 1: PKV_PV(1);
    case 2: PKV_PV(2);
    case 4: PKV_PV(4);
    case 8: PKV_PV(8);
    default: PKV_PV(16);
  }
#undef PKV_PV
  return (int)hipGetLastError();
}

template <typename T>
int launch_decode_valu(const DecodeParams& P, int d, int g, hipStream_t s) {
  switch (d) {
    case 64: return launch_decode_valu_d<T, 64>(P, g, s);
    case 128: return launch_decode_valu_d<T, 128>(P, g, s);
    case 256: return launch_decode_valu_d<T, 256>(P, g, s);
    default: return kBadHeadDim;
  }
}

template <typename T>
int launch_prefill_valu(const PrefillParams& P, int d, int g, hipStream_t s) {
  switch (d) {
    case 64: return launch_prefill_valu_d<T, 64>(P, g, s);
    case 128: return launch_prefill_valu_d<T, 128>(P, g, s);
    case 256: return launch_prefill_valu_d<T, 256>(P, g, s);
    default: return kBadHeadDim;
  }
}

}  // namespace

namespace pkv {
int decode_valu_dispatch(const DecodeParams& P, int dtype, int d, hipStream_t s) {
  int g = P.hq / P.hkv;
  switch (dtype) {
    case kF16: return launch_decode_valu<_Float16>(P, d, g, s);
    case kBF16: return launch_decode_valu<__hip_bfloat16>(P, d, g, s);
    case kF32: return launch_decode_valu<float>(P, d, g, s);
    default: return kBadDType;
  }
}
}  // namespace pkv

extern "C" int pkv_batch_prefill_valu(
    const void* q, int64_t q_stride_n, int64_t q_stride_h, const int32_t* qo_indptr, int32_t nnz_q,
    const void* k_cache, const void* v_cache, int64_t page_stride, int64_t num_pages,
    const int32_t* kv_indptr, const int32_t* kv_indices, int64_t num_indices,
    const int32_t* kv_last_page_len, int32_t batch,
    int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
    int32_t causal, float sm_scale, void* out, int64_t o_stride_n, int64_t o_stride_h,
    int32_t dtype, void* stream) {
  if (batch <= 0 || nnz_q < 0 || num_kv_heads <= 0 || num_qo_heads % num_kv_heads) return kBadArg;
  if (nnz_q == 0) return kOk;
  PrefillParams P;
  P.q = q; P.q_sn = q_stride_n; P.q_sh = q_stride_h; P.qo_indptr = qo_indptr;
  P.k_cache = k_cache; P.v_cache = v_cache; P.page_stride = page_stride;
  P.num_pages = num_pages; P.num_indices = num_indices;
  P.indptr = kv_indptr; P.indices = kv_indices; P.last = kv_last_page_len;
  P.batch = batch; P.hq = num_qo_heads; P.hkv = num_kv_heads; P.ps = page_size;
  P.causal = causal; P.nnz = nnz_q; P.scale_log2 = sm_scale * 1.4426950408889634f;
  P.out = out; P.o_sn = o_stride_n; P.o_sh = o_stride_h;
  int g = num_qo_heads / num_kv_heads;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case kF16: return launch_prefill_valu<_Float16>(P, head_dim, g, s);
    case kBF16: return launch_prefill_valu<__hip_bfloat16>(P, head_dim, g, s);
    case kF32: return launch_prefill_valu<float>(P, head_dim, g, s);
    default: return kBadDType;
  }
}
