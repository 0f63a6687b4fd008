// Paged decode on the matrix cores (fp16 / bf16 caches, page_size 16, head_dim 64 or 128,
// GQA group <= 16).  Same contract as the vector kernel (FlashInfer
// BatchDecodeWithPagedKVCacheWrapper.run, ecahlang/main.py:68); same page-range partition
// and split merge (attn_common.h).
//
// Why matrix cores in decode: with a GQA group of g query heads per KV head every K/V byte
// feeds g multiply-adds in Q.K^T and g more in P.V.  At g = 8 (Qwen2.5-3B) that is 4 MACs per
// cache byte, which on the vector ALUs (64 fp32 FMA/clk/CU) costs about as many cycles as
// streaming the byte from HBM; on the matrix cores it is ~10% of that, leaving the kernel
// bound by HBM alone.  The g query heads of one KV head form the 16 MFMA columns (g < 16
// leaves columns idle; compute is not the bound).
//
// Per wave, per page (16 tokens of one KV head):
//   S[t][n]  = sum_d K[t][d] Q[n][d]    v_mfma_f32_16x16x32: A = K rows straight from HBM
//                                       (lane = token l%16, 8 dims), B = Q (lane = head l%16)
//   online softmax on S in the accumulator layout (lane holds 4 tokens of one head)
//   O^T[d][n] += sum_t V[t][d] P[t][n]  v_mfma_f32_16x16x16: B = P exactly as the softmax
//                                       left it; A = V^T, read from an XOR-swizzled LDS
//                                       copy of the page (coalesced 16-byte HBM loads)
// The reduction index of both products only has to agree between the two operands, so the
// dim order inside K and Q operands is chosen to make each K load 64 contiguous bytes.
// Waves of one workgroup split the pages of each segment; their states meet in LDS by a
// pairwise tree, and the last wave writes the output (or the partial for a split sequence).
#include "attn_common.h"
#include "../../include/pagedkv.h"

using namespace pkv;

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

template <typename To, typename From>
__device__ __forceinline__ To bitcast_(const From& x) {
  static_assert(sizeof(To) == sizeof(From), "size");
  To y;
  __builtin_memcpy(&y, &x, sizeof(To));
  return y;
}

template <typename T> struct Mma;
template <> struct Mma<_Float16> {
  static __device__ __forceinline__ f4 qk(uint4 a, uint4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast_<h8>(a), bitcast_<h8>(b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f4 pv(uint2 a, uint2 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(bitcast_<h4>(a), bitcast_<h4>(b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float x, float y) {
    _Float16 a = (_Float16)x, b = (_Float16)y;
    return (uint32_t)bitcast_<uint16_t>(a) | ((uint32_t)bitcast_<uint16_t>(b) << 16);
  }
};
template <> struct Mma<__hip_bfloat16> {
  static __device__ __forceinline__ f4 qk(uint4 a, uint4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(bitcast_<bf8>(a), bitcast_<bf8>(b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f4 pv(uint2 a, uint2 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bitcast_<s4>(a), bitcast_<s4>(b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float x, float y) {
    __hip_bfloat16 a = __float2bfloat16(x), b = __float2bfloat16(y);
    return (uint32_t)bitcast_<uint16_t>(a) | ((uint32_t)bitcast_<uint16_t>(b) << 16);
  }
};

__device__ __forceinline__ uint16_t load_u16(const void* p) { return *reinterpret_cast<const uint16_t*>(p); }

// Chunk swizzle of the staged V tile: 16-byte chunk c of token row t lives at c ^ swz(t).
// The P.V operand read (4 rows 4 apart x 16 consecutive dims per lane group) then hits
// disjoint banks, and the row writes stay 16-byte aligned.
__device__ __forceinline__ int vswz(int t) { return 2 * ((t >> 2) & 3); }

template <typename T, int D, int W>
__global__ __launch_bounds__(W * 64) void decode_mfma_kernel(DecodeParams P) {
  constexpr int KSTEPS = D / 32;        // Q.K^T matrix steps (k = 32 dims each)
  constexpr int MT = D / 16;            // P.V output tiles of 16 dims
  constexpr int CPR = D / 8;            // 16-byte chunks per token row
  constexpr int VCH = 16 * CPR / 64;    // V chunks per lane per page
  constexpr int ROWB = D * 2;           // bytes per staged V row
  constexpr int TILEB = 16 * ROWB;      // bytes per staged V page
  constexpr int XCH = MT * 4 + 2;       // floats per lane exchanged in the wave tree

  extern __shared__ __align__(16) char smem[];
  __shared__ int flag;
  __shared__ int s_pid[kPidCap];
  // readfirstlane: the wave index (and all derived from it) is wave-uniform, so page ids
  // and addresses that depend on it become scalar values and scalar loads.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int lr = lane & 15, lg = lane >> 4;
  char* vtile = smem + wave * TILEB;
  float* xbuf = reinterpret_cast<float*>(smem);  // tree exchange, aliases the V tiles

  const int64_t total = total_pages(P);
  if (blockIdx.x == 0) zero_empty_sequences<T, D>(P);
  if (total == 0) return;
  const int N0 = P.num_ctas;
  // Ranges: one per workgroup, but never more than there are pages and never more than
  // kPidCap pages each (a workgroup then walks ranges w, w + N0, ...).
  const int N = decode_ranges(N0, total);
  // XCD-aware range order: workgroups are dealt round-robin to the 8 XCDs, so giving each
  // XCD a run of consecutive ranges keeps a split sequence's partials on one L2.
  const int w0 = (N0 % 8 == 0) ? (int)(blockIdx.x % 8) * (N0 / 8) + (int)(blockIdx.x / 8)
                               : (int)blockIdx.x;
  for (int w = w0; w < N; w += N0) {
  const int64_t p0 = range_start(w, N, total), p1 = range_start(w + 1, N, total);
  // Stage the range's page ids in LDS (one coalesced pass); a wave then reads the id of
  // any page as a uniform LDS load, which never waits behind in-flight K/V loads.
  __syncthreads();  // the previous range's readers are done with s_pid
  for (int t = threadIdx.x; t < p1 - p0; t += blockDim.x) s_pid[t] = (int)page_at(P.indices, p0 + t, P.num_pages);
  __syncthreads();

  const int hkv = P.hkv, g = P.hq / hkv;
  const int J = W / hkv;                 // waves sharing one KV head (hkv <= W)
  const int h = wave / J, j = wave % J;  // this wave's KV head and its rank among the J
  const bool active = h < hkv;
  const T* kc = reinterpret_cast<const T*>(P.k_cache);
  const T* vc = reinterpret_cast<const T*>(P.v_cache);
  const T* qall = reinterpret_cast<const T*>(P.q);
  T* out = reinterpret_cast<T*>(P.out);
  const int64_t rowstride = (int64_t)hkv * D;  // elements between tokens in a page
  const int64_t hoff = (int64_t)(active ? h : 0) * D;

  // The wave streams range pages p0 + j + J*k, k = 0..nk-1, across sequence boundaries.
  const int64_t len = p1 - p0;
  const int nk = (active && len > j) ? (int)((len - j + J - 1) / J) : 0;
  auto pid_of = [&](int k) -> int {  // id of wave page k (clamped to the last one)
    k = k < nk ? k : nk - 1;
    return s_pid[j + J * k];
  };
  // A page id outside the pool is read as page 0; its tokens are masked (nv = 0).
  auto load_page = [&](int pgid, uint4 (&kr)[KSTEPS], uint4 (&vr)[VCH]) {
    const int pg = pgid < 0 ? 0 : pgid;
    const T* kb = kc + (int64_t)pg * P.page_stride + hoff;
    const T* vb = vc + (int64_t)pg * P.page_stride + hoff;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
      kr[s] = *reinterpret_cast<const uint4*>(kb + lr * rowstride + 32 * s + 8 * lg);
#pragma unroll
    for (int r = 0; r < VCH; ++r) {
      const int c = lane + 64 * r, t = c / CPR, cc = c % CPR;
      vr[r] = *reinterpret_cast<const uint4*>(vb + t * rowstride + 8 * cc);
    }
  };
  // Ping-pong buffers: page k lives in A when k is even, B when odd; two pages in flight.
  uint4 kA[KSTEPS], vA[VCH], kB[KSTEPS], vB[VCH];
  if (nk > 0) {
    load_page(pid_of(0), kA, vA);
    load_page(pid_of(1), kB, vB);  // nk == 1 reloads page 0: harmless, keeps the pipeline uniform
  }

  // Sequence metadata for sequences bf + lane, refreshed every 64 sequences.
  int bf = find_seq_wave(P.indptr, P.batch, p0);
  int m_start = 0, m_end = 0, m_last = 0;
  auto meta_load = [&]() {
    const int sb = bf + lane;
    m_start = P.indptr[sb < P.batch ? sb : P.batch];
    m_end = P.indptr[sb + 1 < P.batch ? sb + 1 : P.batch];
    m_last = P.last[sb < P.batch ? sb : P.batch - 1];
  };
  meta_load();

  int b = bf;
  int64_t p = p0;
  int k = 0;  // next wave page to process
  while (p < p1) {
    if (b - bf >= 64) { bf = b; meta_load(); }
    const int si = b - bf;
    const int s0 = __builtin_amdgcn_readlane(m_start, si);
    const int s1 = __builtin_amdgcn_readlane(m_end, si);
    if (s1 <= p) { ++b; continue; }  // a sequence with no pages
    int last_len = __builtin_amdgcn_readlane(m_last, si);
    last_len = last_len < 0 ? 0 : (last_len > 16 ? 16 : last_len);
    const int64_t seg_end = p1 < s1 ? p1 : s1;
    const int w_lo = range_owner(s0, N, total), w_hi = range_owner(s1 - 1, N, total);
    const bool whole = w_lo == w_hi;
    const int64_t slot = (int64_t)w + b;
    const int64_t e = seg_end - p0;
    int k_end = (active && e > j) ? (int)((e - j + J - 1) / J) : 0;
    k_end = k_end < nk ? k_end : nk;

    // Q operand: lane = head lr of the group, dims 32*s + 8*lg .. +7.
    uint4 qop[KSTEPS];
    {
      const bool qv = active && lr < g;
      const T* qrow = qall + b * P.q_sn + (int64_t)(active ? h * g + (qv ? lr : 0) : 0) * P.q_sh;
      if (P.q_vec) {
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
          uint4 x = *reinterpret_cast<const uint4*>(qrow + 32 * s + 8 * lg);
          qop[s] = qv ? x : make_uint4(0, 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
          uint32_t e2[4];
#pragma unroll
          for (int x = 0; x < 4; ++x)
            e2[x] = (uint32_t)load_u16(qrow + 32 * s + 8 * lg + 2 * x) |
                    ((uint32_t)load_u16(qrow + 32 * s + 8 * lg + 2 * x + 1) << 16);
          qop[s] = qv ? make_uint4(e2[0], e2[1], e2[2], e2[3]) : make_uint4(0, 0, 0, 0);
        }
      }
      // Settle q here (s_waitcnt vmcnt(0)), once per segment: otherwise the page loop's
      // header inherits "q is the newest load" and waits for every page in flight.
      __builtin_amdgcn_s_waitcnt(0x0F70);
    }
    f4 o[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) o[mt] = f4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, lsum = 0.f;

    auto process = [&](const uint4 (&kr)[KSTEPS], const uint4 (&vr)[VCH], int kk, int pgid) {
      const int64_t gp = p0 + j + (int64_t)J * kk;
      int nv = (gp == s1 - 1) ? last_len : 16;
      if (pgid < 0) nv = 0;
      f4 sacc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) sacc = Mma<T>::qk(kr[s], qop[s], sacc);
      float sv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[i] = (4 * lg + i < nv) ? sacc[i] * P.scale_log2 : -INFINITY;
      float cmax = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
      cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
      cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
      const float mnew = fmaxf(m, cmax);
      const float muse = mnew == -INFINITY ? 0.f : mnew;
      const float alpha = exp2f(m - muse);
      float pr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) pr[i] = exp2f(sv[i] - muse);
      lsum = lsum * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
      m = mnew;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) o[mt] *= alpha;
      // Stage V (tokens past the end zeroed: 0 * NaN would poison P.V).
#pragma unroll
      for (int r = 0; r < VCH; ++r) {
        const int c = lane + 64 * r, t = c / CPR, cc = c % CPR;
        const uint4 val = t < nv ? vr[r] : make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4*>(vtile + t * ROWB + ((cc ^ vswz(t)) << 4)) = val;
      }
      __builtin_amdgcn_wave_barrier();
      const uint2 pb = make_uint2(Mma<T>::pack(pr[0], pr[1]), Mma<T>::pack(pr[2], pr[3]));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int chunk = (2 * mt + (lr >> 3)) ^ (2 * lg);  // vswz(4*lg + i) == 2*lg
        const char* base = vtile + (4 * lg) * ROWB + (chunk << 4) + (lr & 7) * 2;
        const uint32_t a0 = load_u16(base), a1 = load_u16(base + ROWB);
        const uint32_t a2 = load_u16(base + 2 * ROWB), a3 = load_u16(base + 3 * ROWB);
        o[mt] = Mma<T>::pv(make_uint2(a0 | (a1 << 16), a2 | (a3 << 16)), pb, o[mt]);
      }
      __builtin_amdgcn_wave_barrier();
    };

    // One step: consume page kk from its buffer, refill that buffer with page kk + 2
    // (clamped to the last page), rotate the ids.  Pages alternate A, B, A, ...; the two
    // straight-line loops below keep that order visible to the compiler, so each wait
    // covers only the older buffer and the other page's loads stay in flight.
    auto step = [&](uint4 (&kr)[KSTEPS], uint4 (&vr)[VCH], int kk) {
      process(kr, vr, kk, pid_of(kk));
      load_page(pid_of(kk + 2), kr, vr);
    };
    if (k < k_end) {
      if ((k & 1) == 0) {
        for (; k + 1 < k_end; k += 2) {
          step(kA, vA, k);
          step(kB, vB, k + 1);
        }
        if (k < k_end) step(kA, vA, k++);
      } else {
        for (; k + 1 < k_end; k += 2) {
          step(kB, vB, k);
          step(kA, vA, k + 1);
        }
        if (k < k_end) step(kB, vB, k++);
      }
    }

    // Pairwise tree over the J waves of each KV head: wave j += wave j + stride.
    for (int stride = 1; stride < J; stride <<= 1) {
      __syncthreads();
      if ((j % (2 * stride)) == stride) {
        float* xb = xbuf + (size_t)(wave / 2) * XCH * 64;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) xb[(mt * 4 + i) * 64 + lane] = o[mt][i];
        xb[(MT * 4) * 64 + lane] = m;
        xb[(MT * 4 + 1) * 64 + lane] = lsum;
      }
      __syncthreads();
      if ((j % (2 * stride)) == 0 && j + stride < J) {
        const float* xb = xbuf + (size_t)((wave + stride) / 2) * XCH * 64;
        const float m2 = xb[(MT * 4) * 64 + lane], l2 = xb[(MT * 4 + 1) * 64 + lane];
        const float mm = fmaxf(m, m2);
        const float mu = mm == -INFINITY ? 0.f : mm;
        const float c1 = exp2f(m - mu), c2 = exp2f(m2 - mu);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[mt][i] = o[mt][i] * c1 + xb[(mt * 4 + i) * 64 + lane] * c2;
        lsum = lsum * c1 + l2 * c2;
        m = mm;
      }
    }
    // The exchange buffer aliases the V tiles the next segment writes.
    if (J > 1) __syncthreads();

    // Wave j == 0 of each head writes the (partial) result for its g query heads.
    float ltot = lsum + __shfl_xor(lsum, 16, 64);
    ltot += __shfl_xor(ltot, 32, 64);
    if (active && j == 0 && lr < g) {
      const int hq = h * g + lr;
      const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
      if (whole) {
        T* orow = out + b * P.o_sn + (int64_t)hq * P.o_sh + 4 * lg;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if (P.o_vec) {
            const uint2 pk = make_uint2(Mma<T>::pack(o[mt][0] * inv, o[mt][1] * inv),
                                        Mma<T>::pack(o[mt][2] * inv, o[mt][3] * inv));
            *reinterpret_cast<uint2*>(orow + 16 * mt) = pk;
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) orow[16 * mt + i] = from_f32<T>(o[mt][i] * inv);
          }
        }
      } else {
        const int64_t sidx = slot * P.hq + hq;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) st_dev(P.part_o + sidx * D + 16 * mt + 4 * lg + i, o[mt][i] * inv);
        if (lg == 0) store_partial_ml(P, sidx, m, ltot);
      }
    }
    if (!whole && arrive_last(P, b, w_hi - w_lo + 1, &flag)) merge_partials<T, D>(P, b, w_lo, w_hi);
    p = seg_end;
    ++b;
  }
  }  // ranges
}

template <typename T, int D>
int launch_mfma(const DecodeParams& P, hipStream_t s) {
  constexpr int W = 8;
  constexpr int MT = D / 16;
  size_t tiles = (size_t)W * 16 * D * 2;
  size_t xch = (size_t)(W / 2) * (MT * 4 + 2) * 64 * sizeof(float);
  size_t lds = tiles > xch ? tiles : xch;
  hipLaunchKernelGGL((decode_mfma_kernel<T, D, W>), dim3(P.num_ctas), dim3(W * 64), lds, s, P);
  return (int)hipGetLastError();
}

}  // namespace

namespace pkv {

bool decode_mfma_supported(int dtype, int d, int g, int hkv) {
  return (dtype == kF16 || dtype == kBF16) && (d == 64 || d == 128) && g >= 1 && g <= 16 &&
         hkv >= 1 && hkv <= 8;
}

int decode_mfma_dispatch(const DecodeParams& P, int dtype, int d, hipStream_t s) {
  if (P.ps != 16) return decode_valu_dispatch(P, dtype, d, s);
  if (dtype == kF16) return d == 64 ? launch_mfma<_Float16, 64>(P, s) : launch_mfma<_Float16, 128>(P, s);
  return d == 64 ? launch_mfma<__hip_bfloat16, 64>(P, s) : launch_mfma<__hip_bfloat16, 128>(P, s);
}

}  // namespace pkv
