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
// Waves of one workgroup split the pages of each segment; their states meet in LDS at the
// segment's end, where every wave folds the copies of the output tiles it owns and writes
// them (as output rows, or as the partial of a sequence split across workgroups).
#include "attn_common.h"
#include "mfma_common.h"
#include "../../include/pagedkv.h"

using namespace pkv;

namespace {

using namespace pkv::mfma;

// Dynamic LDS of the kernel, in bytes (host and device compute the same layout):
//   tiles  one V page per wave, XOR-swizzled                        W * 16 * D * 2
//   slots  softmax states met at a segment end: (max, sum) of every
//          wave, and each output tile of a head from the J - 1 waves
//          that do not own it                                        W * 512 + hkv * (J - 1) * MT * 1024
//   meta   indptr[0..B] and last_page_len[0..B) (B <= kMetaCap)
//   q      query rows of the range's first qseg sequences, plus one slot filled on demand
//          for a range with more segments
constexpr int kMetaCap = 2048;    // batch limit: page-table rows are staged in LDS
constexpr int kMaxSplit = 32;     // split segments whose arrival a workgroup defers
constexpr int kQSegMax = 4;

__host__ __device__ constexpr int align_up(int x, int a) { return (x + a - 1) / a * a; }

struct MfmaLds {
  int tiles, slots, copies, meta, q, total;
};
template <int D, int W>
__host__ __device__ inline MfmaLds mfma_lds(int hkv, int hq, int qseg) {
  constexpr int MT = D / 16;
  const int J = W / hkv;
  MfmaLds L;
  L.tiles = 0;
  L.slots = W * 16 * D * 2;                 // (max, sum) pairs: W * 64 float2
  L.copies = L.slots + W * 64 * 8;          // tile copies: [hkv][MT][J - 1][64] float4
  L.meta = align_up(L.copies + hkv * (J - 1) * MT * 1024, 16);
  L.q = L.meta + align_up((2 * kMetaCap + 1) * 4, 16);
  L.total = L.q + (qseg + 1) * hq * D * 2;
  return L;
}
// Query rows staged per range: as many sequences as fit in 32 KB, between 1 and kQSegMax.
__host__ __device__ inline int mfma_qseg(int hq, int d) {
  int n = 32768 / (hq * d * 2);
  return n < 1 ? 1 : (n > kQSegMax ? kQSegMax : n);
}

// J = W / hkv waves share each KV head (a template parameter: the combine's loops and
// register arrays are sized by it).
template <typename T, int D, int W, int J>
__global__ __launch_bounds__(W * 64) void decode_mfma_kernel(DecodeParams P) {
  constexpr int NT = W * 64;
  constexpr int KSTEPS = D / 32;        // Q.K^T matrix steps (k = 32 dims each)
  constexpr int MT = D / 16;            // P.V output tiles of 16 dims
  constexpr int CPR = D / 8;            // 16-byte chunks per token row
  constexpr int VCH = 16 * CPR / 64;    // V chunks per lane per page
  constexpr int ROWB = D * 2;           // bytes per staged V row
  constexpr int TILEB = 16 * ROWB;      // bytes per staged V page

  extern __shared__ __align__(16) char smem[];
  __shared__ int s_pid[kPidCap];
  __shared__ int s_split[kMaxSplit][3];  // deferred arrivals: sequence, w_lo, w_hi
  __shared__ int s_merge[kMaxSplit][3];  // merges owed after the arrivals
  __shared__ int s_nmerge;
  __shared__ int s_next[8];              // per KV head: next range page to hand out
  __shared__ int s_bf, s_bl, s_nseg;     // the range's first / last sequence, segment count
  // readfirstlane: the wave index (and all derived from it) is wave-uniform, so page ids
  // and addresses that depend on it become scalar values.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int lr = lane & 15, lg = lane >> 4;

  const int B = P.batch, hkv = P.hkv, g = P.hq / hkv;
  const int qseg = mfma_qseg(P.hq, D);
  const MfmaLds L = mfma_lds<D, W>(hkv, P.hq, qseg);
  char* vtile = smem + L.tiles + wave * TILEB;
  float2* s_ml = reinterpret_cast<float2*>(smem + L.slots);   // [W][64]
  f4* s_copy = reinterpret_cast<f4*>(smem + L.copies);        // [hkv][MT][J - 1][64]
  int* s_indptr = reinterpret_cast<int*>(smem + L.meta);      // [kMetaCap + 1]
  int* s_lastlen = s_indptr + kMetaCap + 1;                   // [kMetaCap]
  const T* s_q = reinterpret_cast<const T*>(smem + L.q);      // [qseg + 1][hq][D]
  T* s_qw = reinterpret_cast<T*>(smem + L.q);

  // Heads are dealt round-robin (h = wave % hkv): waves of one SIMD differ in issue
  // priority by age, and this gives every head the same mix of older and younger waves.
  const int h = wave % hkv, j = wave / hkv;  // this wave's KV head and its rank among the J
  const bool active = j < J;

  const int N0 = P.num_ctas;
  // XCD-aware range order: workgroups are dealt round-robin to the 8 XCDs, so giving each
  // XCD a run of consecutive ranges keeps a split sequence's partials on one L2.
  const int w0 = (N0 % 8 == 0) ? (int)(blockIdx.x % 8) * (N0 / 8) + (int)(blockIdx.x / 8)
                               : (int)blockIdx.x;
  // The first range's page ids are requested together with round 1, assuming the page list
  // holds exactly indptr[B] entries (kv_indices sized to the batch): the partition then
  // depends on num_indices alone.  Round 1 confirms the guess, or they are read again.
  static_assert(kPidCap <= 4 * NT, "four page ids per thread");
  const int tg = (int)(P.num_indices < INT_MAX ? P.num_indices : INT_MAX);
  int pv[4];
  int gp0 = 0, glen = 1, ng = 0;
  {
    if (tg > 0) {
      ng = decode_ranges(N0, tg);
      if (w0 < ng) {
        const Ranges rg(ng, tg);
        gp0 = rg.start(w0);
        glen = rg.start(w0 + 1) - gp0;
      }
    }
    const int32_t* src = tg > 0 ? P.indices + gp0 : P.indptr;  // (a valid address either way)
#pragma unroll
    for (int r = 0; r < 4; ++r) {  // unconditional loads from clamped indices
      const int t = threadIdx.x + r * NT;
      pv[r] = src[tg > 0 ? (t < glen ? t : glen - 1) : 0];
    }
  }

  // ---- round 1: the page table's row pointers and last-page lengths into LDS
  // (B <= kMetaCap <= 4 * NT).  The loads are unconditional, from clamped indices, and all
  // are issued before the first LDS write: a load under a divergent branch gets a wait for
  // its result at the branch's end, which would serialise them.
  {
    static_assert(kMetaCap <= 4 * NT, "four rows per thread");
    int iv[5], lv[4];
#pragma unroll
    for (int r = 0; r < 5; ++r) {
      const int i = threadIdx.x + r * NT;
      iv[r] = P.indptr[i < B ? i : B];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = threadIdx.x + r * NT;
      lv[r] = P.last[i < B - 1 ? i : B - 1];
    }
#pragma unroll
    for (int r = 0; r < 5; ++r) {
      const int i = threadIdx.x + r * NT;
      if (i <= B) s_indptr[i] = iv[r];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = threadIdx.x + r * NT;
      if (i < B) s_lastlen[i] = lv[r];
    }
  }
  if (threadIdx.x == 0) {
    s_nseg = 0;
    s_bf = INT_MAX;
    s_bl = -1;
  }
  if (tg > 0 && w0 < ng) {  // the first range's page ids, as the speculative read gave them
#pragma unroll
    for (int r = 0; r < 4; ++r) {  // ids outside the pool are read as absent (-1)
      const int t = threadIdx.x + r * NT;
      if (t < glen) s_pid[t] = ((int64_t)pv[r] >= 0 && (int64_t)pv[r] < P.num_pages) ? pv[r] : -1;
    }
  }
  if (blockIdx.x == 0) zero_empty_sequences<T, D>(P);
  lds_barrier();
  auto rd = [&](const int* lds_arr, int i) __attribute__((always_inline)) -> int {  // uniform LDS read
    return __builtin_amdgcn_readfirstlane(lds_arr[i]);
  };
  int total = rd(s_indptr, B);
  total = (int64_t)total < P.num_indices ? total : (int)P.num_indices;
  if (total <= 0) return;
  // Ranges: one per workgroup, never more than there are pages and never more than
  // kPidCap pages each (a workgroup then walks ranges w, w + N0, ...).
  const int N = decode_ranges(N0, total);
  const Ranges R(N, total);

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

  // A page id outside the pool is read as page 0; its tokens are masked (nv = 0).  Past the
  // range's end the last page is loaded again (an L2 hit, never used), so the load after a
  // wave's last page is still a valid one.
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

  // One page buffer per wave: a wave has one page in flight.  With the eight waves of every
  // CU each holding one (~16 MB in flight over the chip, more than the HBM's bandwidth-delay
  // product), this is faster than two per wave: 40.9 against 42.1 us per launch at the
  // Qwen2.5-3B B=64 batch, and the wave needs 221 registers instead of 254.
  uint4 kA[KSTEPS], vA[VCH];

  // Deferred arrivals (split segments recorded in s_split; the count is kept in a register
  // in every wave, as whether a segment is split is the same in all of them): every wave
  // waits for its own partial stores, then one lane per split bumps that sequence's counter
  // (all in parallel); the splits that arrived last are compacted into s_merge and merged
  // by the whole workgroup at once.  Inside the page loop (a full record) the register-light
  // global-memory merge is used: the page buffers are live there.
  int nsplit = 0;
  auto flush_splits = [&](bool in_loop) __attribute__((always_inline)) {
    wait_stores();  // this wave's partial stores are complete (device-visible)
    lds_barrier();  // ... in every wave; the split records are visible
    if (wave == 0) {
      int sb = 0, lo = 0, hi = 0, last = 0;
      if (lane < nsplit) {
        sb = s_split[lane][0];
        lo = s_split[lane][1];
        hi = s_split[lane][2];
        const int old = atomicAdd(&P.counters[sb], 1);
        last = old == hi - lo;
        // Every other arrival already happened: safe to reset for the next launch.
        if (last) __hip_atomic_store(&P.counters[sb], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      const uint64_t bal = __ballot(last);
      if (last) {
        const int pos = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                  __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
        s_merge[pos][0] = sb;
        s_merge[pos][1] = lo;
        s_merge[pos][2] = hi;
      }
      if (lane == 0) s_nmerge = __popcll(bal);
    }
    lds_barrier();  // also keeps partial loads below the arrivals
    const int nm = __builtin_amdgcn_readfirstlane(s_nmerge);
    if (in_loop) {
      for (int i = 0; i < nm; ++i) merge_partials<T, D>(P, s_merge[i][0], s_merge[i][1], s_merge[i][2]);
    } else {
      merge_queued<T, D>(P, s_merge, nm);
    }
    lds_barrier();  // s_split / s_merge are free again
    nsplit = 0;
  };

  for (int w = w0; w < N; w += N0) {
  const int64_t p0 = R.start(w), p1 = R.start(w + 1);
  const int len = (int)(p1 - p0);
  lds_barrier();  // the previous range's readers are done with s_pid / s_q / s_bf / s_bl

  // ---- round 2: the range's page ids (requested at the start for the first range when
  // the page list is exactly indptr[B] long; otherwise now), written to LDS below ...
  if (w != w0 || total != tg) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {  // unconditional loads from clamped indices, as in round 1
      const int t = threadIdx.x + r * NT;
      pv[r] = P.indices[p0 + (t < len ? t : len - 1)];
    }
  }
  // ... while all threads look up the range's sequences in the staged rows: the first and
  // last sequence with pages in [p0, p1) and how many have any (the segments).
  for (int i = threadIdx.x; i < B; i += NT) {
    const int64_t s = s_indptr[i], e = s_indptr[i + 1];
    if (e > s && e > p0 && s < p1) {
      atomicAdd(&s_nseg, 1);
      atomicMin(&s_bf, i);
      atomicMax(&s_bl, i);
    }
  }
  lds_barrier();
  const int bf = rd(&s_bf, 0), nseg = rd(&s_nseg, 0);
  if (nseg == 0) continue;  // pages before indptr[0]: no sequence owns them
  const int nq = min(qseg, rd(&s_bl, 0) - bf + 1);  // sequences bf .. bf + nq - 1 get staged
  const int per = P.hq * (D / 8);  // 16-byte q chunks per sequence
  const int nqc = nq * per;        // <= 4 * NT: qseg * hq * D * 2 <= 32 KB
  auto q_src = [&](int c) __attribute__((always_inline)) -> const T* {
    const int i = c / per, rr = c - i * per;
    const int hh = rr / (D / 8), d = (rr - hh * (D / 8)) * 8;
    return qall + (bf + i) * P.q_sn + (int64_t)hh * P.q_sh + d;
  };
  auto write_pids = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {  // ids outside the pool are read as absent (-1)
      const int t = threadIdx.x + r * NT;
      if (t < len) s_pid[t] = ((int64_t)pv[r] >= 0 && (int64_t)pv[r] < P.num_pages) ? pv[r] : -1;
    }
  };
  // Staged row i, head hh lives at s_q[(i * hq + hh) * D]: chunk c maps to c * 8.  When a
  // thread stages at most one chunk (the common case) it is kept in a register and written
  // after the first K/V loads are issued, so those do not wait for the q rows.
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // (a plain vector: stays in registers)
  const bool q_one = P.q_vec && nqc <= NT;
  const u32x4 qc0 = *reinterpret_cast<const u32x4*>(
      q_one ? q_src((int)threadIdx.x < nqc ? (int)threadIdx.x : nqc - 1)
            : reinterpret_cast<const T*>(P.part_o));  // (unconditional: any aligned address)
  if (!q_one && P.q_vec) {
    u32x4 qc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = threadIdx.x + r * NT;
      qc[r] = *reinterpret_cast<const u32x4*>(q_src(c < nqc ? c : nqc - 1));
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = threadIdx.x + r * NT;
      if (c < nqc) *reinterpret_cast<u32x4*>(s_qw + (int64_t)c * 8) = qc[r];
    }
  } else if (!q_one) {
    for (int c = threadIdx.x; c < nqc; c += NT) {
      const T* src = q_src(c);
#pragma unroll
      for (int x = 0; x < 8; ++x) s_qw[(int64_t)c * 8 + x] = src[x];
    }
  }
  write_pids();
  // Pages before the first sequence (only when indptr[0] > 0) are skipped.
  const int gap0 = (int)max((int64_t)rd(s_indptr, bf) - p0, (int64_t)0);
  if (threadIdx.x < 8) s_next[threadIdx.x] = gap0;
  lds_barrier();
  if (threadIdx.x == 0) {  // (read by every thread before the barrier above)
    s_nseg = 0;
    s_bf = INT_MAX;
    s_bl = -1;
  }

  // The J waves of a head split the range's pages, each in increasing order: by default
  // wave j takes pages j, j + J, j + 2J, ... (a fixed split: the result is reproducible);
  // with P.dynamic the waves take them on demand from the head's LDS counter, so a wave
  // that gets fewer issue slots takes fewer pages and the J waves finish together.
  int next_static = gap0 + j;
  auto grab = [&]() __attribute__((always_inline)) -> int {  // next page of this head (uniform)
    if (P.dynamic) {
      int v = 0;
      if (lane == 0) v = atomicAdd(&s_next[h], 1);
      return __builtin_amdgcn_readfirstlane(v);
    }
    const int v = next_static;
    next_static += J;
    return v;
  };
  auto pid_at = [&](int i) __attribute__((always_inline)) -> int {  // id of range page i (uniform)
    return __builtin_amdgcn_readfirstlane(s_pid[i < len ? i : len - 1]);
  };
  // ---- the range's pages, one loop per wave; sequence (segment) boundaries are crossed
  // inside it.  Every wave ends each segment of the range once and in order, so the
  // combine barriers match up even though waves reach them at different pages.
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
    w_lo = R.owner(s0);
    w_hi = R.owner(s1 - 1);
    whole = w_lo == w_hi;
    // Q of this segment is read from LDS at every page (lane = head lr of the group,
    // dims 32*s + 8*lg .. +7); a sequence past the staged ones fills the spare slot first.
    int qslot = b - bf;
    if (qslot >= nq) {
      qslot = qseg;
      lds_barrier();  // the spare slot's previous readers are done
      for (int c = threadIdx.x; c < per; c += NT) {
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
    // Combine the J waves of each head, all of them at once: wave j owns the output tiles
    // mt = j, j + J, ...  Every wave parks its (max, sum) and the tiles it does not own;
    // then each wave folds the J copies of its own tiles.
    if constexpr (J > 1) {
      if (active) {
        s_ml[(h * J + j) * 64 + lane] = make_float2(m, lsum);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int c = mt % J;
          if (c != j) s_copy[((h * MT + mt) * (J - 1) + (j < c ? j : j - 1)) * 64 + lane] = o[mt];
        }
      }
      lds_barrier();
      if (active) {
        float2 mls[J];
#pragma unroll
        for (int jj = 0; jj < J; ++jj) mls[jj] = s_ml[(h * J + jj) * 64 + lane];
        float mx = -INFINITY;
#pragma unroll
        for (int jj = 0; jj < J; ++jj) mx = fmaxf(mx, mls[jj].x);
        const float mu = mx == -INFINITY ? 0.f : mx;
        float sc[J];
        float ls = 0.f, cj = 0.f;
#pragma unroll
        for (int jj = 0; jj < J; ++jj) {
          sc[jj] = __builtin_amdgcn_exp2f(mls[jj].x - mu);
          ls += mls[jj].y * sc[jj];
          cj = jj == j ? sc[jj] : cj;
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if (mt % J != j) continue;
          f4 cp[J - 1];
#pragma unroll
          for (int jj = 0; jj < J - 1; ++jj) cp[jj] = s_copy[((h * MT + mt) * (J - 1) + jj) * 64 + lane];
          f4 acc = o[mt] * cj;
#pragma unroll
          for (int jj = 0; jj < J - 1; ++jj) {
            const int src = jj < j ? jj : jj + 1;  // wave rank that parked copy jj
            float s2 = 0.f;
#pragma unroll
            for (int x = 0; x < J; ++x) s2 = x == src ? sc[x] : s2;
            acc += cp[jj] * s2;
          }
          o[mt] = acc;
        }
        m = mx;
        lsum = ls;
      }
    }
    if (!whole && threadIdx.x == 0) {
      s_split[nsplit][0] = b;
      s_split[nsplit][1] = w_lo;
      s_split[nsplit][2] = w_hi;
    }
    lds_barrier();  // slots are read before the next segment parks new states
    float ltot = lsum + __shfl_xor(lsum, 16, 64);
    ltot += __shfl_xor(ltot, 32, 64);
    if (active && lr < g) {
      const int hq = h * g + lr;
      const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
      if (whole) {
        T* orow = out + b * P.o_sn + (int64_t)hq * P.o_sh + 4 * lg;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if (mt % J != j) continue;
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
        for (int mt = 0; mt < MT; ++mt) {
          if (mt % J != j) continue;
          st_dev4(P.part_o, (uint32_t)((sidx * D + 16 * mt + 4 * lg) * sizeof(float)), o[mt] * inv);
        }
        if (j == 0 && lg == 0) store_partial_ml(P, sidx, m, ltot);
      }
    }
    if (!whole && ++nsplit == kMaxSplit) flush_splits(true);
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

  // One step: consume range page idx from the buffer, then take the head's next page and
  // request it into the same buffer.  The next page's id is read from LDS before the compute,
  // so its request does not wait for that read afterwards (0.2 us per launch).
  auto step = [&](uint4 (&kr)[KSTEPS], uint4 (&vr)[VCH], int& idx) __attribute__((always_inline)) {
    const int64_t gp = p0 + idx;
    while (gp >= seg_end) advance();
    const int nidx = grab();
    const int cpid = pid_at(idx), npid = pid_at(nidx);
    process(kr, vr, gp, cpid);
    idx = nidx;
    load_page(npid, kr, vr);
    __builtin_amdgcn_sched_barrier(0);
  };
  start_segment();
  // A wave's pages come in increasing order, so the first one past the range ends its loop.
  int ia = len;
  if (active) ia = grab();
  load_page(pid_at(ia), kA, vA);
  if (q_one && (int)threadIdx.x < nqc) *reinterpret_cast<u32x4*>(s_qw + (int64_t)threadIdx.x * 8) = qc0;
  lds_barrier();  // the q rows are staged
  while (ia < len) step(kA, vA, ia);
  while (si < nseg - 1) advance();
  end_segment();
  }  // ranges
  if (nsplit > 0) flush_splits(false);
}

template <typename T, int D>
int launch_mfma(const DecodeParams& P, hipStream_t s) {
  constexpr int W = 8;
  const MfmaLds L = mfma_lds<D, W>(P.hkv, P.hq, mfma_qseg(P.hq, D));
  const dim3 grid(P.num_ctas), block(W * 64);
  switch (W / P.hkv) {  // 1 <= hkv <= 8: J is 8, 4, 2 or 1
    case 8: hipLaunchKernelGGL((decode_mfma_kernel<T, D, W, 8>), grid, block, L.total, s, P); break;
    case 4: hipLaunchKernelGGL((decode_mfma_kernel<T, D, W, 4>), grid, block, L.total, s, P); break;
    case 2: hipLaunchKernelGGL((decode_mfma_kernel<T, D, W, 2>), grid, block, L.total, s, P); break;
    default: hipLaunchKernelGGL((decode_mfma_kernel<T, D, W, 1>), grid, block, L.total, s, P); break;
  }
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
