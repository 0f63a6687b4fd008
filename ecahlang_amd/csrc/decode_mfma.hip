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

// Chunk swizzle of the staged V tile: 16-byte chunk c of token row t lives at c ^ vswz(t).
// Row writes (one row per 16 lanes) stay 16-byte aligned and conflict-free, and the
// transposing operand read (rows 4g..4g+3, 32 bytes each, per 16-lane group g) lands the
// four rows of a group, and the two groups of a 32-lane half, on disjoint banks.
template <int D>
__device__ __forceinline__ int vswz(int t) {
  return D == 128 ? 2 * (t & 7) : 2 * ((t >> 1) & 3);
}

typedef short s4v __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element (i & 3) of the
// 8-byte rows addressed by lanes 4j + (i >> 2), j = 0..3.  With lane i of group g pointing
// at V[4g + i/4][16*mt + 4*(i%4)], lane i gets V[4g + j][16*mt + i]: the V^T operand of the
// 16x16x16 P.V product, in one instruction.
__device__ __forceinline__ uint2 lds_read_tr16(const char* p) {
  s4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s4v*)(p));
  uint2 u;
  __builtin_memcpy(&u, &r, sizeof(u));
  return u;
}

// Dynamic LDS of the kernel, in bytes (host and device compute the same layout):
//   tiles  one V page per wave, XOR-swizzled                       W * 16 * D * 2
//   slots  online-softmax state of every wave that is not its
//          head's leader (j > 0), parked for the leader's combine  (W - W/J) * XCH * 256
//   meta   indptr[0..B] and last_page_len[0..B) (B <= kMetaCap)
//   q      query rows of the range's first qseg sequences, plus one slot filled on demand
//          for a range with more segments
constexpr int kMetaCap = 2048;    // batch limit: page-table rows are staged in LDS
constexpr int kMaxSplit = 32;     // split segments whose arrival a workgroup defers
constexpr int kQSegMax = 4;

__host__ __device__ constexpr int align_up(int x, int a) { return (x + a - 1) / a * a; }

struct MfmaLds {
  int tiles, slots, meta, q, total;
};
template <int D, int W>
__host__ __device__ inline MfmaLds mfma_lds(int hkv, int hq, int qseg) {
  constexpr int XCH = (D / 16) * 4 + 4;  // MT float4s + (max, sum) padded to a float4
  const int J = W / hkv;
  MfmaLds L;
  L.tiles = 0;
  L.slots = W * 16 * D * 2;
  L.meta = align_up(L.slots + (W - W / J) * XCH * 64 * 4, 16);
  L.q = L.meta + align_up((2 * kMetaCap + 1) * 4, 16);
  L.total = L.q + (qseg + 1) * hq * D * 2;
  return L;
}
// Query rows staged per range: as many sequences as fit in 32 KB, between 1 and kQSegMax.
__host__ __device__ inline int mfma_qseg(int hq, int d) {
  int n = 32768 / (hq * d * 2);
  return n < 1 ? 1 : (n > kQSegMax ? kQSegMax : n);
}

template <typename T, int D, int W>
__global__ __launch_bounds__(W * 64) void decode_mfma_kernel(DecodeParams P) {
  constexpr int KSTEPS = D / 32;        // Q.K^T matrix steps (k = 32 dims each)
  constexpr int MT = D / 16;            // P.V output tiles of 16 dims
  constexpr int CPR = D / 8;            // 16-byte chunks per token row
  constexpr int VCH = 16 * CPR / 64;    // V chunks per lane per page
  constexpr int ROWB = D * 2;           // bytes per staged V row
  constexpr int TILEB = 16 * ROWB;      // bytes per staged V page
  constexpr int XCH = MT * 4 + 4;       // floats per lane of a parked softmax state

  extern __shared__ __align__(16) char smem[];
  __shared__ int s_pid[kPidCap];
  __shared__ int s_split[kMaxSplit][3];  // deferred arrivals: sequence, w_lo, w_hi
  __shared__ int s_last[kMaxSplit];
  __shared__ int s_nsplit;
  // readfirstlane: the wave index (and all derived from it) is wave-uniform, so page ids
  // and addresses that depend on it become scalar values.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int lr = lane & 15, lg = lane >> 4;

  const int B = P.batch, hkv = P.hkv, g = P.hq / hkv;
  const int qseg = mfma_qseg(P.hq, D);
  const MfmaLds L = mfma_lds<D, W>(hkv, P.hq, qseg);
  char* vtile = smem + L.tiles + wave * TILEB;
  int* s_indptr = reinterpret_cast<int*>(smem + L.meta);  // [kMetaCap + 1]
  int* s_lastlen = s_indptr + kMetaCap + 1;               // [kMetaCap]
  const T* s_q = reinterpret_cast<const T*>(smem + L.q);  // [qseg][hq][D]
  T* s_qw = reinterpret_cast<T*>(smem + L.q);

  const int J = W / hkv;                 // waves sharing one KV head (hkv <= W)
  const int h = wave / J, j = wave % J;  // this wave's KV head and its rank among the J
  const bool active = h < hkv;
  // parked-state slot of a non-leader wave (j > 0)
  float* myslot = reinterpret_cast<float*>(smem + L.slots) + (h * (J - 1) + (j - 1)) * XCH * 64;

  // ---- round 1: the page table's row pointers and last-page lengths into LDS
  for (int i = threadIdx.x; i <= B; i += blockDim.x) s_indptr[i] = P.indptr[i];
  for (int i = threadIdx.x; i < B; i += blockDim.x) s_lastlen[i] = P.last[i];
  if (threadIdx.x == 0) s_nsplit = 0;
  if (blockIdx.x == 0) zero_empty_sequences<T, D>(P);
  lds_barrier();
  auto rd = [&](const int* lds_arr, int i) __attribute__((always_inline)) -> int {  // uniform LDS read
    return __builtin_amdgcn_readfirstlane(lds_arr[i]);
  };
  int64_t total = rd(s_indptr, B);
  total = total < P.num_indices ? total : P.num_indices;
  if (total <= 0) return;
  const int N0 = P.num_ctas;
  // Ranges: one per workgroup, never more than there are pages and never more than
  // kPidCap pages each (a workgroup then walks ranges w, w + N0, ...).
  const int N = decode_ranges(N0, total);
  // XCD-aware range order: workgroups are dealt round-robin to the 8 XCDs, so giving each
  // XCD a run of consecutive ranges keeps a split sequence's partials on one L2.
  const int w0 = (N0 % 8 == 0) ? (int)(blockIdx.x % 8) * (N0 / 8) + (int)(blockIdx.x / 8)
                               : (int)blockIdx.x;

  const T* kc = reinterpret_cast<const T*>(P.k_cache);
  const T* vc = reinterpret_cast<const T*>(P.v_cache);
  const T* qall = reinterpret_cast<const T*>(P.q);
  T* out = reinterpret_cast<T*>(P.out);
  const int64_t rowstride = (int64_t)hkv * D;  // elements between tokens in a page
  const int64_t hoff = (int64_t)(active ? h : 0) * D;
  // Per-lane element offsets inside a page: K in the Q.K^T operand layout (token lr,
  // dims 8*lg + 32*s), V in plain 16-byte row chunks.
  const uint32_t koff = (uint32_t)(lr * rowstride + 8 * lg);
  uint32_t voff[VCH];
#pragma unroll
  for (int r = 0; r < VCH; ++r) {
    const int c = lane + 64 * r;
    voff[r] = (uint32_t)((c / CPR) * rowstride + 8 * (c % CPR));
  }

  // Deferred arrivals: bump the counters of the parked split segments in parallel, then
  // merge the sequences this workgroup completed.
  auto flush_splits = [&]() __attribute__((always_inline)) {
    wait_stores();  // this thread's partial stores are complete (device-visible)
    lds_barrier();
    const int ns = s_nsplit;
    if ((int)threadIdx.x < ns) {
      const int sb = s_split[threadIdx.x][0];
      const int nseg = s_split[threadIdx.x][2] - s_split[threadIdx.x][1] + 1;
      const int old = atomicAdd(&P.counters[sb], 1);
      const int last = old == nseg - 1;
      if (last) __hip_atomic_store(&P.counters[sb], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last[threadIdx.x] = last;
    }
    lds_barrier();  // also keeps partial loads below the arrivals
    for (int i = 0; i < ns; ++i) {
      if (!s_last[i]) continue;
      const int sb = s_split[i][0], lo = s_split[i][1], hi = s_split[i][2];
      if (hi - lo + 1 <= kMergeRegs)
        merge_partials_regs<T, D>(P, sb, lo, hi);
      else
        merge_partials<T, D>(P, sb, lo, hi);
    }
    lds_barrier();
    if (threadIdx.x == 0) s_nsplit = 0;
    lds_barrier();
  };

  for (int w = w0; w < N; w += N0) {
  const int64_t p0 = range_start(w, N, total), p1 = range_start(w + 1, N, total);
  const int bf = lds_upper_index(s_indptr, B, p0);
  // The range's first qseg sequences (with pages in the range), whose q rows get staged.
  // (Named scalars, not an array: a dynamically indexed array would live in scratch.)
  int qb0 = bf, qb1 = bf, qb2 = bf, qb3 = bf;
  int nq = 0;
  {
    int bb = bf;
    int64_t pp = p0;
    while (pp < p1 && nq < qseg && bb < B) {
      const int e = rd(s_indptr, bb + 1);
      if (e > pp) {
        qb0 = nq == 0 ? bb : qb0;
        qb1 = nq == 1 ? bb : qb1;
        qb2 = nq == 2 ? bb : qb2;
        qb3 = nq == 3 ? bb : qb3;
        ++nq;
        pp = e < p1 ? e : p1;
      }
      ++bb;
    }
  }
  // ---- round 2: the range's page ids and the staged q rows into LDS
  lds_barrier();  // the previous range's readers are done with s_pid / s_q
  for (int t = threadIdx.x; t < p1 - p0; t += blockDim.x)
    s_pid[t] = (int)page_at(P.indices, p0 + t, P.num_pages);
  {
    const int per = P.hq * (D / 8);  // 16-byte chunks per sequence
    for (int c = threadIdx.x; c < nq * per; c += blockDim.x) {
      const int i = c / per, r = c - i * per;
      const int hh = r / (D / 8), d = (r - hh * (D / 8)) * 8;
      const int sb = i == 0 ? qb0 : i == 1 ? qb1 : i == 2 ? qb2 : qb3;
      const T* src = qall + sb * P.q_sn + (int64_t)hh * P.q_sh + d;
      T* dst = s_qw + ((int64_t)(i * P.hq + hh)) * D + d;
      if (P.q_vec) {
        *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
      } else {
#pragma unroll
        for (int x = 0; x < 8; ++x) dst[x] = src[x];
      }
    }
  }
  lds_barrier();

  // The wave streams range pages p0 + j + J*k, k = 0..nk-1, across sequence boundaries.
  const int64_t len = p1 - p0;
  const int nk = (active && len > j) ? (int)((len - j + J - 1) / J) : 0;
  auto pid_of = [&](int k) __attribute__((always_inline)) -> int {  // id of wave page k (clamped to the last one)
    k = k < nk ? k : nk - 1;
    return __builtin_amdgcn_readfirstlane(s_pid[j + J * k]);  // uniform: an SGPR
  };
  // A page id outside the pool is read as page 0; its tokens are masked (nv = 0).
  auto load_page = [&](int pgid, uint4 (&kr)[KSTEPS], uint4 (&vr)[VCH]) __attribute__((always_inline)) {
    const int pg = pgid < 0 ? 0 : pgid;
    const T* kb = kc + (int64_t)pg * P.page_stride + hoff;  // uniform base
    const T* vb = vc + (int64_t)pg * P.page_stride + hoff;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
      kr[s] = *reinterpret_cast<const uint4*>(kb + koff + 32 * s);
#pragma unroll
    for (int r = 0; r < VCH; ++r) vr[r] = *reinterpret_cast<const uint4*>(vb + voff[r]);
  };

  // ---- the range's pages, one loop per wave; sequence (segment) boundaries are crossed
  // inside it.  Every wave ends each segment of the range once and in order, so the
  // combine barriers match up even though waves reach them at different pages.
  int nseg = 0;  // segments in the range
  {
    int bb = bf;
    int64_t pp = p0;
    while (pp < p1 && bb < B) {
      const int e = rd(s_indptr, bb + 1);
      if (e > pp) {
        ++nseg;
        pp = e < p1 ? e : p1;
      }
      ++bb;
    }
  }
  int b = bf - 1, si = -1;
  int s1 = 0, last_len = 0, w_lo = 0, w_hi = 0;
  int64_t seg_end = p0;
  bool whole = false;
  const bool qv = active && lr < g;
  const T* qrow_lds = s_q;
  f4 o[MT];
  float m = -INFINITY, lsum = 0.f;

  auto start_segment = [&]() __attribute__((always_inline)) {  // uniform across the workgroup
    int s0;
    do {
      ++b;
      s0 = rd(s_indptr, b);
      s1 = rd(s_indptr, b + 1);
    } while (s1 <= seg_end);  // skip sequences with no pages
    ++si;
    last_len = rd(s_lastlen, b);
    last_len = last_len < 0 ? 0 : (last_len > 16 ? 16 : last_len);
    seg_end = p1 < s1 ? p1 : s1;
    w_lo = range_owner(s0, N, total);
    w_hi = range_owner(s1 - 1, N, total);
    whole = w_lo == w_hi;
    // Q of this segment is read from LDS at every page (lane = head lr of the group,
    // dims 32*s + 8*lg .. +7); a segment past the staged ones fills the spare slot first.
    int qslot = si;
    if (si >= nq) {
      qslot = qseg;
      lds_barrier();  // the spare slot's previous readers are done
      const int per = P.hq * (D / 8);
      for (int c = threadIdx.x; c < per; c += blockDim.x) {
        const int hh = c / (D / 8), d = (c - hh * (D / 8)) * 8;
        const T* src = qall + b * P.q_sn + (int64_t)hh * P.q_sh + d;
        T* dst = s_qw + ((int64_t)(qseg * P.hq + hh)) * D + d;
#pragma unroll
        for (int x = 0; x < 8; ++x) dst[x] = src[x];
      }
      lds_barrier();
    }
    qrow_lds = s_q + ((int64_t)(qslot * P.hq + (active ? h * g + (qv ? lr : 0) : 0))) * D + 8 * lg;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) o[mt] = f4{0.f, 0.f, 0.f, 0.f};
    m = -INFINITY;
    lsum = 0.f;
  };

  auto end_segment = [&]() __attribute__((always_inline)) {  // uniform across the workgroup
    // Combine the J waves of each head: non-leaders park their state, the leader (j == 0)
    // folds it in and writes the output row or the split partial.
    if (J > 1) {
      if (active && j > 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          *reinterpret_cast<f4*>(myslot + (mt * 64 + lane) * 4) = o[mt];
        *reinterpret_cast<float2*>(myslot + (MT * 64 + lane) * 4) = make_float2(m, lsum);
      }
      lds_barrier();
      if (active && j == 0) {
        for (int jj = 1; jj < J; ++jj) {
          const float* xb = reinterpret_cast<const float*>(smem + L.slots) + (h * (J - 1) + (jj - 1)) * XCH * 64;
          const float2 ml2 = *reinterpret_cast<const float2*>(xb + (MT * 64 + lane) * 4);
          const float m2 = ml2.x, l2 = ml2.y;
          const float mm = fmaxf(m, m2);
          const float mu = mm == -INFINITY ? 0.f : mm;
          const float c1 = __builtin_amdgcn_exp2f(m - mu), c2 = __builtin_amdgcn_exp2f(m2 - mu);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            o[mt] = o[mt] * c1 + *reinterpret_cast<const f4*>(xb + (mt * 64 + lane) * 4) * c2;
          lsum = lsum * c1 + l2 * c2;
          m = mm;
        }
      }
    }
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
        const int64_t sidx = ((int64_t)w + b) * P.hq + hq;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          st_dev4(P.part_o, (uint32_t)((sidx * D + 16 * mt + 4 * lg) * sizeof(float)), o[mt] * inv);
        if (lg == 0) store_partial_ml(P, sidx, m, ltot);
      }
    }
    if (!whole && threadIdx.x == 0) {
      const int n = s_nsplit;
      s_split[n][0] = b;
      s_split[n][1] = w_lo;
      s_split[n][2] = w_hi;
      s_nsplit = n + 1;
    }
    lds_barrier();  // slots are read before the next segment parks new states
    if (s_nsplit == kMaxSplit) flush_splits();
  };
  auto advance = [&]() __attribute__((always_inline)) {
    end_segment();
    start_segment();
  };

  auto process = [&](const uint4 (&kr)[KSTEPS], const uint4 (&vr)[VCH], int64_t gp, int pgid) __attribute__((always_inline)) {
    int nv = (gp == s1 - 1) ? last_len : 16;
    if (pgid < 0) nv = 0;
    // Stage V first (tokens past the end zeroed: 0 * NaN would poison P.V); only a
    // sequence's last page can be partial.
    if (nv == 16) {
#pragma unroll
      for (int r = 0; r < VCH; ++r) {
        const int c = lane + 64 * r, t = c / CPR, cc = c % CPR;
        *reinterpret_cast<uint4*>(vtile + t * ROWB + ((cc ^ vswz<D>(t)) << 4)) = vr[r];
      }
    } else {
#pragma unroll
      for (int r = 0; r < VCH; ++r) {
        const int c = lane + 64 * r, t = c / CPR, cc = c % CPR;
        const uint4 val = t < nv ? vr[r] : make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4*>(vtile + t * ROWB + ((cc ^ vswz<D>(t)) << 4)) = val;
      }
    }
    f4 sacc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      uint4 qs = *reinterpret_cast<const uint4*>(qrow_lds + 32 * s);
      qs = qv ? qs : make_uint4(0, 0, 0, 0);
      sacc = Mma<T>::qk(kr[s], qs, sacc);
    }
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sv[i] = (4 * lg + i < nv) ? sacc[i] * P.scale_log2 : -INFINITY;
    float cmax = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
    const float mnew = fmaxf(m, cmax);
    const float muse = mnew == -INFINITY ? 0.f : mnew;
    // v_exp_f32 directly: arguments are <= 0, results in [0, 1] (denormals flush to 0).
    const float alpha = __builtin_amdgcn_exp2f(m - muse);
    float pr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pr[i] = __builtin_amdgcn_exp2f(sv[i] - muse);
    lsum = lsum * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
    // Rescale the accumulator only when some head's running max moved (rare after the
    // first pages of a sequence).
    if (__ballot(mnew != m)) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) o[mt] *= alpha;
    }
    m = mnew;
    __builtin_amdgcn_wave_barrier();
    const uint2 pb = make_uint2(Mma<T>::pack(pr[0], pr[1]), Mma<T>::pack(pr[2], pr[3]));
    const int tr_row = 4 * lg + (lr >> 2);
    const char* tr_base = vtile + tr_row * ROWB + (lr & 1) * 8;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int chunk = (2 * mt + ((lr & 3) >> 1)) ^ vswz<D>(tr_row);
      o[mt] = Mma<T>::pv(lds_read_tr16(tr_base + (chunk << 4)), pb, o[mt]);
    }
    __builtin_amdgcn_wave_barrier();
  };

  // One step: consume wave page kk from its buffer (A for even kk, B for odd), refill that
  // buffer with page kk + 2 (clamped to the last page), so two pages are always in flight.
  auto step = [&](uint4 (&kr)[KSTEPS], uint4 (&vr)[VCH], int kk) __attribute__((always_inline)) {
    const int64_t gp = p0 + j + (int64_t)J * kk;
    while (gp >= seg_end) advance();
    process(kr, vr, gp, pid_of(kk));
    load_page(pid_of(kk + 2), kr, vr);
    __builtin_amdgcn_sched_barrier(0);
  };
  start_segment();
  // Ping-pong buffers: page k lives in A when k is even, B when odd; two pages in flight.
  // Issued only now, after the scalar set-up: work between these loads and their first use
  // risks a wait that drains them.
  uint4 kA[KSTEPS], vA[VCH], kB[KSTEPS], vB[VCH];
  if (nk > 0) {
    load_page(pid_of(0), kA, vA);
    load_page(pid_of(1), kB, vB);  // nk == 1 reloads page 0: harmless, keeps the pipeline uniform
  }
  for (int k = 0; k < nk; k += 2) {
    step(kA, vA, k);
    if (k + 1 < nk) step(kB, vB, k + 1);
  }
  while (si < nseg - 1) advance();
  end_segment();
  }  // ranges
  if (s_nsplit > 0) flush_splits();
}

template <typename T, int D>
int launch_mfma(const DecodeParams& P, hipStream_t s) {
  constexpr int W = 8;
  const MfmaLds L = mfma_lds<D, W>(P.hkv, P.hq, mfma_qseg(P.hq, D));
  hipLaunchKernelGGL((decode_mfma_kernel<T, D, W>), dim3(P.num_ctas), dim3(W * 64), L.total, s, P);
  return (int)hipGetLastError();
}

}  // namespace

namespace pkv {

bool decode_mfma_supported(int dtype, int d, int g, int hkv, int batch) {
  return (dtype == kF16 || dtype == kBF16) && (d == 64 || d == 128) && g >= 1 && g <= 16 &&
         hkv >= 1 && hkv <= 8 && batch <= kMetaCap;
}

int decode_mfma_dispatch(const DecodeParams& P, int dtype, int d, hipStream_t s) {
  if (P.ps != 16) return decode_valu_dispatch(P, dtype, d, s);
  if (dtype == kF16) return d == 64 ? launch_mfma<_Float16, 64>(P, s) : launch_mfma<_Float16, 128>(P, s);
  return d == 64 ? launch_mfma<__hip_bfloat16, 64>(P, s) : launch_mfma<__hip_bfloat16, 128>(P, s);
}

}  // namespace pkv
