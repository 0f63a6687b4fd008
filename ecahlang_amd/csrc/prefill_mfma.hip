// Paged chunked prefill on the matrix cores (fp16 / bf16 caches, page_size 16, head_dim 64 or
// 128, GQA group g in {1, 2, 4, 8, 16}).  Same contract as the vector kernel
// (BatchPrefillWithPagedKVCacheWrapper.run, ecahlang/main.py:432-443, :68): query row i of
// request b (qo_len_b rows) attends keys j <= i + kv_len_b - qo_len_b when causal (bottom-right
// aligned), else all kv_len_b keys.
//
// Work items come from the host plan (one int32 record each, longest first):
//   item = (request, KV head, 256 / g query tokens, a chunk [k0, k1) of the keys they see)
// A workgroup of 8 waves owns the item's 256 query rows (row r = token r / g, head r % g of the
// KV head's group), so every staged K/V page serves all 256 rows.  Per 64 keys (four pages),
// staged in LDS by all threads in a ring of three stages:
//   S^T[key][row] = K . Q^T      v_mfma_f32_16x16x32, A = K from LDS, B = Q in registers
//   online softmax per row in the accumulator layout (lane = row l % 16, keys 4*(l/16) + i)
//   O^T[dim][row] += V^T . P     v_mfma_f32_16x16x32 over two pages at a time: the reduction
//                                slot 8*(l/16) + e holds key 4*(l/16) + e of the first page for
//                                e < 4 and of the second for e >= 4, which is where the softmax
//                                left P and where two ds_read_b64_tr_b16 leave V^T
// Pages go global -> LDS directly (global_load_lds_dwordx4: lane l's 16 bytes land at base + 16 l),
// three steps in flight, so no registers hold them on the way.  Each wave owns 32 rows
// outright, so waves never combine.  An item that is one chunk of a
// longer key range writes a partial (normalised rows plus running max and sum); the merge
// kernel folds the partials of each split group.
#include <type_traits>
#include "attn_common.h"
#include "mfma_common.h"
#include "../../include/pagedkv.h"

using namespace pkv;
using namespace pkv::mfma;

namespace {

constexpr int kRows = 256;   // query rows per item (8 waves x 32)
constexpr int kStepPages = 4;  // pages (16 keys each) staged per step; chunks start at multiples of 64 keys
constexpr int kMaxChunk = 8192;  // keys per item (its page ids are staged in LDS)
// Lazy running max (log2 units): a row's reference max moves only when its scores exceed it by
// more than this, so probabilities stay <= 2^kLazyMax (exact enough in fp16 / bf16 P, and far
// from fp32 overflow in the sums) and the output rows are rescaled only on such jumps.
constexpr float kLazyMax = 8.f;

// Source of the value rows that must read as zero (past the chunk, absent pages): P is 0 there,
// and 0 * NaN would poison P.V.
__device__ uint4 g_zero_rows[64];

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// One wave-wide 16-byte-per-lane copy global -> LDS: lane l's 16 bytes at src (per lane) land at
// LDS byte dst + 16 * l (dst uniform across the wave, passed in M0).  Written as inline assembly
// so that the compiler does not track it: the caller orders it with explicit vmcnt waits and
// barriers (the compiler cannot tell which LDS array a later transposed read touches and would
// otherwise wait for every copy in flight, draining the prefetch pipeline).
__device__ __forceinline__ void lds_copy16(const void* src, const char* dst) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(
      (unsigned)(uintptr_t)(const __attribute__((address_space(3))) char*)(dst));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}
constexpr int kItem = 12;    // int32 fields per work item
constexpr int kGroup = 8;    // int32 fields per split group

struct PrefillMfmaParams {
  const void* q;
  int64_t q_sn, q_sh;
  const void* k_cache;
  const void* v_cache;
  int64_t page_stride, num_pages;
  const int32_t* indices;
  int64_t num_indices;
  int32_t hq, hkv;
  int32_t causal;
  float scale_log2;
  void* out;
  int64_t o_sn, o_sh;
  const int32_t* items;
  float2* part_ml;  // [slot][kRows]
  float* part_o;    // [slot][kRows][D] (fp16 elements for fp16 caches, else fp32)
  int32_t o_vec;
};

// Split groups' partial outputs are kept in fp16 when the cache is fp16 (averages of fp16 V
// rows, so they fit; half the bytes written by the items and read by the merge), else fp32.
template <typename T>
constexpr bool kHalfPartials = std::is_same<T, _Float16>::value;

template <typename T, int D, int G>
__global__ __launch_bounds__(512) void prefill_mfma_kernel(PrefillMfmaParams P) {
  constexpr int KSTEPS = D / 32;      // Q.K^T reduction steps
  constexpr int MT = D / 16;          // output tiles of 16 dims
  constexpr int CPR = D / 8;          // 16-byte chunks per row
  constexpr int ROWB = D * 2;         // bytes per staged row
  constexpr int TILEB = 16 * ROWB;    // bytes per staged page (16 rows)
  constexpr int NP = kStepPages;
  constexpr int STEPB = NP * TILEB;   // one step's pages
  constexpr int RPI = 64 / CPR;       // rows per 1 KB direct load (one 16-byte chunk per lane)
  constexpr int LPP = 16 / RPI;       // loads per page and K or V
  constexpr int LPW = NP * 2 * LPP / 8;  // loads per wave per step
  static_assert(NP * 2 * LPP % 8 == 0, "loads per wave");
  constexpr int TQ = kRows / G;       // query tokens per item

  // three stages as distinct arrays (the step loop is unrolled by three): the compiler can then
  // tell the stage being read from the stages being filled and does not wait for the latter
  __shared__ __align__(16) char s_k0[STEPB], s_k1[STEPB], s_k2[STEPB];
  __shared__ __align__(16) char s_v0[STEPB], s_v1[STEPB], s_v2[STEPB];
  __shared__ int s_page[kMaxChunk / 16 + kStepPages];  // the chunk's page ids, -1 = absent

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;

  const int32_t* it = P.items + (int64_t)kItem * blockIdx.x;
  const int h = it[1], t0 = it[2], tq = it[3], k0 = it[4], k1 = it[5], slot = it[6];
  const int kv_len = it[7], qo_len = it[8], qo_start = it[9], kp0 = it[10];
  const int64_t npages_req = (kv_len + 15) / 16;

  const T* kc = reinterpret_cast<const T*>(P.k_cache);
  const T* vc = reinterpret_cast<const T*>(P.v_cache);
  const int64_t rowstride = (int64_t)P.hkv * D;
  const int64_t hoff = (int64_t)h * D;

  // ---- this wave's 32 rows: Q^T operand in registers (B of the 16x16x32 product)
  uint4 qr[2][KSTEPS];
  int rtok[2];  // token (within the item) of this lane's row in each row tile
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int r = 32 * wave + 16 * rt + lr;
    const int tt = r / G, hh = r % G;
    rtok[rt] = tt;
    const bool ok = tt < tq;
    const T* src = reinterpret_cast<const T*>(P.q) + (int64_t)(qo_start + t0 + (ok ? tt : 0)) * P.q_sn +
                   (int64_t)(h * G + hh) * P.q_sh + 8 * lg;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      const uint4 v = *reinterpret_cast<const uint4*>(src + 32 * s);
      qr[rt][s] = ok ? v : make_uint4(0, 0, 0, 0);
    }
  }

  // ---- staging: step st covers keys kb = k0 + 64 st .. +63 (pages kb/16 .. kb/16 + 3)
  // (the plan keeps k1 - k0 <= kMaxChunk; the clamp keeps s_page in bounds regardless)
  const int nsteps = min((k1 - k0 + 16 * NP - 1) / (16 * NP), kMaxChunk / (16 * NP));
  // the chunk's page ids (pages past the request's last one repeat it; their keys are masked)
  const int npc = nsteps * NP;
  for (int i = threadIdx.x; i < npc; i += blockDim.x) {
    const int64_t pi = k0 / 16 + i;
    int64_t e = kp0 + (pi < npages_req ? pi : npages_req - 1);
    e = e < P.num_indices ? e : P.num_indices - 1;
    const int64_t pg = e >= 0 ? P.indices[e] : -1;
    s_page[i] = (pg >= 0 && pg < P.num_pages) ? (int)pg : -1;
  }
  // the Q loads are complete here; a compiler-visible vmcnt(0) (expcnt, lgkmcnt at their maxima)
  // tells the compiler so, which keeps it from waiting on them, and on every copy in flight,
  // inside the step loop
  __builtin_amdgcn_s_waitcnt(0x0F70);
  lds_barrier();
  auto page_of = [&](int key) __attribute__((always_inline)) -> int {  // -1: absent page
    return s_page[(key - k0) / 16];
  };
  // Step st's pages into stage buf: wave-load wi (this wave: wi = wave * LPW + x) covers RPI
  // rows of one page's K or V; lane l fills LDS slot l, i.e. row RPI*(wi % LPP) + l / CPR,
  // position l % CPR, which holds the row's chunk position ^ swizzle(row).
  auto issue_step = [&](int st, char* kstage, char* vstage) __attribute__((always_inline)) {
    const int kb = k0 + 16 * NP * st;
#pragma unroll
    for (int x = 0; x < LPW; ++x) {
      const int wi = wave * LPW + x;
      const int p = wi / (2 * LPP), kv = (wi / LPP) & 1, r0 = RPI * (wi % LPP);
      const int row = r0 + lane / CPR, pos = lane % CPR;
      const int pg = page_of(kb + 16 * p);
      const int key = kb + 16 * p + row;
      const void* src;
      char* dst;
      if (kv) {
        const int col = pos ^ vswz<D>(row);
        src = (pg < 0 || key >= k1) ? (const void*)(g_zero_rows + lane)
                                    : (const void*)(vc + (int64_t)pg * P.page_stride + row * rowstride + hoff + 8 * col);
        dst = vstage + p * TILEB + r0 * ROWB;
      } else {
        const int col = pos ^ kswz<D>(row);
        src = (pg < 0) ? (const void*)(g_zero_rows + lane)
                       : (const void*)(kc + (int64_t)pg * P.page_stride + row * rowstride + hoff + 8 * col);
        dst = kstage + p * TILEB + r0 * ROWB;
      }
      lds_copy16(src, dst);
    }
  };

  f4 o[2][MT];
  float m[2], lsum[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) o[rt][mt] = f4{0.f, 0.f, 0.f, 0.f};
    m[rt] = -INFINITY;
    lsum[rt] = 0.f;
  }
  // key limit of each row: j < lim (causal: bottom-right aligned diagonal)
  int lim[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int tabs = t0 + rtok[rt];
    int l = P.causal ? tabs + kv_len - qo_len + 1 : kv_len;
    l = l < k1 ? l : k1;
    lim[rt] = rtok[rt] < tq ? l : -1;
  }

  // the smallest key limit among this wave's rows that exist: a step entirely below it (and
  // with no absent page) needs no masking
  int lim_min = INT_MAX;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) lim_min = min(lim_min, rtok[rt] < tq ? lim[rt] : INT_MAX);
#pragma unroll
  for (int x = 1; x < 64; x <<= 1) lim_min = min(lim_min, __shfl_xor(lim_min, x, 64));
  lim_min = __builtin_amdgcn_readfirstlane(lim_min);
  const float scale = P.scale_log2;

  // step st: compute on stage (ks, vs) = stage st % 3, refill stage (kn, vn) with step st + 2
  auto do_step = [&](int st, const char* ks, const char* vs, char* kn, char* vn) __attribute__((always_inline)) {
    // this wave's loads of step st are done (step st + 1's may still be in flight) ...
    if (st + 1 < nsteps) wait_vmcnt<LPW>();
    else wait_vmcnt<0>();
    // ... and every wave's: step st is staged, and every wave is past step st - 1, whose
    // stage is refilled next
    lds_barrier();
    if (st + 2 < nsteps) issue_step(st + 2, kn, vn);
    const int kb = k0 + 16 * NP * st;
    bool absent[NP];
    bool full = kb + 16 * NP <= lim_min;  // (uniform)
#pragma unroll
    for (int kt = 0; kt < NP; ++kt) {
      absent[kt] = page_of(kb + 16 * kt) < 0;
      full = full && !absent[kt];
    }
    // S^T tiles: [key tile kt][row tile rt]
    f4 sacc[NP][2];
#pragma unroll
    for (int kt = 0; kt < NP; ++kt) {
      const char* krow = ks + kt * TILEB + lr * ROWB;
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) sacc[kt][rt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        const uint4 a = *reinterpret_cast<const uint4*>(krow + (((4 * s + lg) ^ kswz<D>(lr)) << 4));
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) sacc[kt][rt] = Mma<T>::qk(a, qr[rt][s], sacc[kt][rt]);
      }
    }
    // online softmax per row tile on the raw scores (the scale is folded into the exponent's
    // FMA; it is positive, so maxima commute with it); P packed as the B operand of P.V
    uint2 pb[NP][2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      float sv[NP][4];
      float cmax = -INFINITY;
      if (full) {
#pragma unroll
        for (int kt = 0; kt < NP; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) sv[kt][i] = sacc[kt][rt][i];
      } else {
#pragma unroll
        for (int kt = 0; kt < NP; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kb + 16 * kt + 4 * lg + i;
            sv[kt][i] = (key < lim[rt] && !absent[kt]) ? sacc[kt][rt][i] : -INFINITY;
          }
      }
#pragma unroll
      for (int kt = 0; kt < NP; ++kt)
        cmax = fmaxf(cmax, fmaxf(fmaxf(sv[kt][0], sv[kt][1]), fmaxf(sv[kt][2], sv[kt][3])));
      cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
      cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
      const float cms = cmax * scale;
      const bool grow = cms > m[rt] + kLazyMax;  // (false while every score so far is masked)
      if (__ballot(grow)) {
        const float mnew = grow ? cms : m[rt];
        const float alpha = __builtin_amdgcn_exp2f(m[rt] - mnew);  // 0 from -inf, 1 if unchanged
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) o[rt][mt] *= alpha;
        lsum[rt] *= alpha;
        m[rt] = mnew;
      }
      const float nmuse = m[rt] == -INFINITY ? 0.f : -m[rt];
      float psum = 0.f;
#pragma unroll
      for (int kt = 0; kt < NP; ++kt) {
        float pr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pr[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[kt][i], scale, nmuse));
          psum += pr[i];
        }
        pb[kt][rt] = make_uint2(Mma<T>::pack(pr[0], pr[1]), Mma<T>::pack(pr[2], pr[3]));
      }
      lsum[rt] += psum;
    }
    // O^T += V^T . P, two pages per 16x16x32 product
    const int tr_row = 4 * lg + (lr >> 2);
#pragma unroll
    for (int u = 0; u < NP / 2; ++u) {
      const char* tra = vs + (2 * u) * TILEB + tr_row * ROWB + (lr & 1) * 8;
      const char* trb = tra + TILEB;
      uint4 pp[2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
        pp[rt] = make_uint4(pb[2 * u][rt].x, pb[2 * u][rt].y, pb[2 * u + 1][rt].x, pb[2 * u + 1][rt].y);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int chunk = ((2 * mt + ((lr & 3) >> 1)) ^ vswz<D>(tr_row)) << 4;
        const uint2 va = lds_read_tr16(tra + chunk), vb = lds_read_tr16(trb + chunk);
        const uint4 vt = make_uint4(va.x, va.y, vb.x, vb.y);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) o[rt][mt] = Mma<T>::qk(vt, pp[rt], o[rt][mt]);
      }
    }
  };
  if (nsteps > 0) issue_step(0, s_k0, s_v0);
  if (nsteps > 1) issue_step(1, s_k1, s_v1);
  for (int st = 0; st < nsteps; st += 3) {
    do_step(st, s_k0, s_v0, s_k2, s_v2);
    if (st + 1 < nsteps) do_step(st + 1, s_k1, s_v1, s_k0, s_v0);
    if (st + 2 < nsteps) do_step(st + 2, s_k2, s_v2, s_k1, s_v1);
  }

  // ---- rows out: normalised output rows, or the partial of a split group
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    float ltot = lsum[rt] + __shfl_xor(lsum[rt], 16, 64);
    ltot += __shfl_xor(ltot, 32, 64);
    const int r = 32 * wave + 16 * rt + lr;
    const int tt = rtok[rt], hh = r % G;
    if (tt >= tq) continue;
    const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
    if (slot < 0) {
      T* orow = reinterpret_cast<T*>(P.out) + (int64_t)(qo_start + t0 + tt) * P.o_sn + (int64_t)(h * G + hh) * P.o_sh + 4 * lg;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (P.o_vec) {
          *reinterpret_cast<uint2*>(orow + 16 * mt) = make_uint2(Mma<T>::pack(o[rt][mt][0] * inv, o[rt][mt][1] * inv),
                                                                 Mma<T>::pack(o[rt][mt][2] * inv, o[rt][mt][3] * inv));
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) orow[16 * mt + i] = from_f32<T>(o[rt][mt][i] * inv);
        }
      }
    } else {
      const int64_t pr = (int64_t)slot * kRows + r;
      if constexpr (kHalfPartials<T>) {
        _Float16* prow = reinterpret_cast<_Float16*>(P.part_o) + pr * D + 4 * lg;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          *reinterpret_cast<uint2*>(prow + 16 * mt) = make_uint2(Mma<T>::pack(o[rt][mt][0] * inv, o[rt][mt][1] * inv),
                                                                 Mma<T>::pack(o[rt][mt][2] * inv, o[rt][mt][3] * inv));
      } else {
        float* prow = P.part_o + pr * D + 4 * lg;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          *reinterpret_cast<float4*>(prow + 16 * mt) = make_float4(o[rt][mt][0] * inv, o[rt][mt][1] * inv,
                                                                   o[rt][mt][2] * inv, o[rt][mt][3] * inv);
      }
      if (lg == 0) P.part_ml[pr] = make_float2(m[rt], ltot);
    }
  }
}

// Folds the partials of each split group: group = {first_slot, nslots, qo_start, t0, tq, h}.
// A workgroup takes kMergeRows rows of one group; D/4 lanes per row, 4 dims each.  Loads are
// issued kMergeUnroll slots at a time from clamped (always valid) addresses, so that they are
// in flight together.
constexpr int kMergeUnroll = 4;
template <int D>
constexpr int merge_rows() { return 256 / (D / 4); }

template <typename T, int D, int G>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillMfmaParams P, const int32_t* groups) {
  constexpr int RB = merge_rows<D>(), TPR = D / 4;
  const int32_t* gr = groups + (int64_t)kGroup * (blockIdx.x / (kRows / RB));
  const int s0 = gr[0], ns = gr[1], qo_start = gr[2], t0 = gr[3], tq = gr[4], h = gr[5];
  const int r = (blockIdx.x % (kRows / RB)) * RB + threadIdx.x / TPR, d = (threadIdx.x % TPR) * 4;
  const int tt = r / G, hh = r % G;
  if (tt >= tq || ns <= 0) return;
  const float2* ml = P.part_ml + (int64_t)s0 * kRows + r;
  const int64_t po = ((int64_t)s0 * kRows + r) * D + d;  // element offset of slot s0's dims
  float M = -INFINITY;
  for (int s = 0; s < ns; s += kMergeUnroll) {
    float2 v[kMergeUnroll];
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) v[u] = ml[(int64_t)min(s + u, ns - 1) * kRows];
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) M = fmaxf(M, v[u].x);
  }
  float den = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s = 0; s < ns; s += kMergeUnroll) {
    float2 w[kMergeUnroll];
    float4 v[kMergeUnroll];
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
      const int64_t sl = min(s + u, ns - 1);
      w[u] = ml[sl * kRows];
      if constexpr (kHalfPartials<T>) {
        const uint2 raw = *reinterpret_cast<const uint2*>(reinterpret_cast<const _Float16*>(P.part_o) + po + sl * kRows * D);
        _Float16 hv[4];
        __builtin_memcpy(hv, &raw, 8);
        v[u] = make_float4((float)hv[0], (float)hv[1], (float)hv[2], (float)hv[3]);
      } else {
        v[u] = *reinterpret_cast<const float4*>(P.part_o + po + sl * kRows * D);
      }
    }
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
      // a slot whose rows saw no key (l = 0) carries no weight; repeats past ns count zero
      // (such a slot's row may hold anything, hence the branch rather than a zero weight)
      const float c = (s + u < ns && w[u].y > 0.f) ? exp2f(w[u].x - M) * w[u].y : 0.f;
      if (c != 0.f) {
        den += c;
        acc.x += c * v[u].x;
        acc.y += c * v[u].y;
        acc.z += c * v[u].z;
        acc.w += c * v[u].w;
      }
    }
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  T* orow = reinterpret_cast<T*>(P.out) + (int64_t)(qo_start + t0 + tt) * P.o_sn + (int64_t)(h * G + hh) * P.o_sh + d;
  if (P.o_vec) {
    T v[4] = {from_f32<T>(acc.x * inv), from_f32<T>(acc.y * inv), from_f32<T>(acc.z * inv),
              from_f32<T>(acc.w * inv)};
    *reinterpret_cast<uint2*>(orow) = *reinterpret_cast<const uint2*>(v);
  } else {
    orow[0] = from_f32<T>(acc.x * inv);
    orow[1] = from_f32<T>(acc.y * inv);
    orow[2] = from_f32<T>(acc.z * inv);
    orow[3] = from_f32<T>(acc.w * inv);
  }
}

template <typename T, int D, int G>
int launch(const PrefillMfmaParams& P, int n_items, const int32_t* groups, int n_groups, hipStream_t s) {
  if (n_items > 0)
    hipLaunchKernelGGL((prefill_mfma_kernel<T, D, G>), dim3(n_items), dim3(512), 0, s, P);
  if (n_groups > 0)
    hipLaunchKernelGGL((prefill_merge_kernel<T, D, G>), dim3(n_groups * (kRows / merge_rows<D>())), dim3(256), 0, s,
                       P, groups);
  return (int)hipGetLastError();
}

template <typename T, int D>
int launch_g(const PrefillMfmaParams& P, int g, int n_items, const int32_t* groups, int n_groups, hipStream_t s) {
  switch (g) {
    case 1: return launch<T, D, 1>(P, n_items, groups, n_groups, s);
    case 2: return launch<T, D, 2>(P, n_items, groups, n_groups, s);
    case 4: return launch<T, D, 4>(P, n_items, groups, n_groups, s);
    case 8: return launch<T, D, 8>(P, n_items, groups, n_groups, s);
    case 16: return launch<T, D, 16>(P, n_items, groups, n_groups, s);
  }
  return kBadGroup;
}

}  // namespace

extern "C" int pkv_prefill_mfma_supported(int32_t dtype, int32_t head_dim, int32_t num_qo_heads,
                                          int32_t num_kv_heads, int32_t page_size) {
  if (num_kv_heads <= 0 || num_qo_heads % num_kv_heads) return 0;
  const int g = num_qo_heads / num_kv_heads;
  return (dtype == kF16 || dtype == kBF16) && (head_dim == 64 || head_dim == 128) && page_size == 16 &&
         (g == 1 || g == 2 || g == 4 || g == 8 || g == 16);
}

extern "C" int pkv_batch_prefill_mfma(const void* q, int64_t q_stride_n, int64_t q_stride_h,
                                      const void* k_cache, const void* v_cache, int64_t page_stride,
                                      int64_t num_pages, const int32_t* kv_indices, int64_t num_indices,
                                      int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                      int32_t page_size, int32_t causal, float sm_scale,
                                      const int32_t* items, int32_t n_items, const int32_t* groups,
                                      int32_t n_groups, void* part_ml, void* part_o, void* out,
                                      int64_t o_stride_n, int64_t o_stride_h, int32_t dtype, void* stream) {
  if (!pkv_prefill_mfma_supported(dtype, head_dim, num_qo_heads, num_kv_heads, page_size)) return kBadArg;
  if (n_items < 0 || n_groups < 0 || (n_items > 0 && !items) || (n_groups > 0 && (!groups || !part_ml || !part_o)))
    return kBadArg;
  const int es = 2;
  if ((uintptr_t)q % 16 || (q_stride_n * es) % 16 || (q_stride_h * es) % 16) return kBadAlign;
  PrefillMfmaParams P;
  P.q = q; P.q_sn = q_stride_n; P.q_sh = q_stride_h;
  P.k_cache = k_cache; P.v_cache = v_cache; P.page_stride = page_stride; P.num_pages = num_pages;
  P.indices = kv_indices; P.num_indices = num_indices;
  P.hq = num_qo_heads; P.hkv = num_kv_heads; P.causal = causal;
  P.scale_log2 = sm_scale * 1.4426950408889634f;
  P.out = out; P.o_sn = o_stride_n; P.o_sh = o_stride_h;
  P.items = items;
  P.part_ml = reinterpret_cast<float2*>(part_ml);
  P.part_o = reinterpret_cast<float*>(part_o);
  P.o_vec = ((uintptr_t)out % 8 == 0) && ((o_stride_n * es) % 8 == 0) && ((o_stride_h * es) % 8 == 0);
  hipStream_t s = (hipStream_t)stream;
  const int g = num_qo_heads / num_kv_heads;
  if (dtype == kF16)
    return head_dim == 64 ? launch_g<_Float16, 64>(P, g, n_items, groups, n_groups, s)
                          : launch_g<_Float16, 128>(P, g, n_items, groups, n_groups, s);
  return head_dim == 64 ? launch_g<__hip_bfloat16, 64>(P, g, n_items, groups, n_groups, s)
                        : launch_g<__hip_bfloat16, 128>(P, g, n_items, groups, n_groups, s);
}
