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
// staged in LDS by all threads:
//   S^T[key][row] = K . Q^T      v_mfma_f32_16x16x32, A = K from LDS, B = Q in registers
//   online softmax per row in the accumulator layout (lane = row l % 16, keys 4*(l/16) + i)
//   O^T[dim][row] += V^T . P     v_mfma_f32_16x16x32 over two pages at a time: the reduction
//                                slot 8*(l/16) + e holds key 4*(l/16) + e of the first page for
//                                e < 4 and of the second for e >= 4, which is where the softmax
//                                left P and where two ds_read_b64_tr_b16 leave V^T
// Pages go global -> LDS directly (global_load_lds_dwordx4: lane l's 16 bytes land at base + 16 l)
// into rings of three K and three V stages, so no registers hold them on the way.  Each wave owns
// 32 rows outright, so waves never combine.
// Schedule: a step is a matrix phase (K . Q^T of step j and P.V of step j - 1, as a software
// pipeline of eight-product units whose LDS operands are read one unit ahead) and a softmax
// phase, each ending at a workgroup barrier; waves 4-7 run one phase behind waves 0-3, so each
// SIMD (waves w and w + 4) overlaps one wave's matrix phase with the other's softmax.  Page ids
// are read from the LDS page table a phase before they are needed (a lookup in the matrix phase
// would wait behind the other waves' operand reads).
// An item that is one chunk of a longer key range writes a partial (normalised rows plus
// running max and sum); the merge kernel folds the partials of each split group.
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
// A workgroup barrier that also ends the compiler's scheduling region, so that no instruction
// moves between the phases it separates.
__device__ __forceinline__ void phase_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  lds_barrier();
  __builtin_amdgcn_sched_barrier(0);
}
// One wave-wide 16-byte-per-lane copy global -> LDS: lane l's 16 bytes at sbase + voff (a
// wave-uniform base in an SGPR pair plus a 32-bit per-lane byte offset) land at LDS byte
// m0 + 16 * l (m0 uniform).  Written as inline assembly so that the compiler does not track it:
// the caller orders it with explicit vmcnt waits and barriers (the compiler cannot tell which LDS
// array a later transposed read touches and would otherwise wait for every copy in flight,
// draining the prefetch pipeline).
__device__ __forceinline__ void lds_copy16(const void* sbase, unsigned voff, unsigned m0) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(m0) : "memory", "m0");
}
// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ unsigned lds_addr(const char* p) {
  return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) char*)(p);
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
  constexpr int KL = NP * LPP / 8;    // K (and V) loads per wave per step
  static_assert(NP * LPP % 8 == 0, "loads per wave");
  constexpr int TQ = kRows / G;       // query tokens per item

  // rings of three stages for K and for V
  __shared__ __align__(16) char s_k[3 * STEPB];
  __shared__ __align__(16) char s_v[3 * STEPB];
  __shared__ __align__(16) int s_page[kMaxChunk / 16 + kStepPages];  // the chunk's page ids, -1 = absent

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
  // V stage 2 starts zero-filled: the first M phase multiplies it by a zero P (uninitialised LDS
  // could hold NaN bit patterns, and 0 * NaN is NaN)
  for (int i = threadIdx.x; i < STEPB / 16; i += blockDim.x)
    reinterpret_cast<uint4*>(s_v + 2 * STEPB)[i] = make_uint4(0, 0, 0, 0);
  // the Q loads are complete here; a compiler-visible vmcnt(0) (expcnt, lgkmcnt at their maxima)
  // tells the compiler so, which keeps it from waiting on them, and on every copy in flight,
  // inside the step loop
  __builtin_amdgcn_s_waitcnt(0x0F70);
  lds_barrier();
  // Step st's K (or V) pages into a stage: K wave-load wi (this wave: wi = wave * KL + x) covers
  // RPI rows of page wi / LPP (the same page, my_page, for all of a wave's loads); lane l fills
  // LDS slot l, i.e. row RPI*(wi % LPP) + l / CPR, position l % CPR, which holds the row's chunk
  // position ^ swizzle(row).  The page id pg (wave-uniform, read from the table a phase ahead)
  // gives the base and each lane adds its byte offset; absent pages (and, for V, keys past the
  // chunk, per row) read zero rows.
  static_assert(LPP % KL == 0, "a wave's loads of a step cover one page");
  const int my_page = wave * KL / LPP;
  // this wave's page of step st (a VGPR holding a uniform value; st clamped into the chunk)
  auto page_id = [&](int st) __attribute__((always_inline)) -> int {
    return s_page[min(st, nsteps - 1) * NP + my_page];
  };
  const char* kbase = reinterpret_cast<const char*>(kc + hoff);
  const char* vbase = reinterpret_cast<const char*>(vc + hoff);
  const int64_t page_bytes = P.page_stride * (int64_t)sizeof(T);
  // (branch-free: the base and the offsets are selected, so the copies can sit between the
  // products of the matrix phase; kstage / vstage are LDS byte addresses)
  const char* const zero_rows = reinterpret_cast<const char*>(g_zero_rows);
  auto issue_k = [&](int st, unsigned kstage, int pg) __attribute__((always_inline)) {
    const bool have = pg >= 0;
    const char* base = have ? kbase + pg * page_bytes : zero_rows;
#pragma unroll
    for (int x = 0; x < KL; ++x) {
      const int wi = wave * KL + x;
      const int p = wi / LPP, r0 = RPI * (wi % LPP);
      const int row = r0 + lane / CPR, col = (lane % CPR) ^ kswz<D>(row);
      const unsigned off = have ? (unsigned)((row * rowstride + 8 * col) * sizeof(T)) : 16u * lane;
      lds_copy16(base, off, kstage + p * TILEB + r0 * ROWB);
    }
  };
  // V rows at or past the chunk's end must not be NaN (their P is 0, and 0 * NaN is NaN): in a
  // page that the chunk ends inside, they repeat the page's last row inside the chunk; a page
  // entirely past the end, or absent, reads zero rows.
  auto issue_v = [&](int st, unsigned vstage, int pg) __attribute__((always_inline)) {
    const int kb = k0 + 16 * NP * st;
#pragma unroll
    for (int x = 0; x < KL; ++x) {
      const int wi = wave * KL + x;
      const int p = wi / LPP, r0 = RPI * (wi % LPP);
      const int row = r0 + lane / CPR, col = (lane % CPR) ^ vswz<D>(row);
      const int vr = k1 - kb - 16 * p;  // rows of this page inside the chunk (uniform)
      const bool have = pg >= 0 && vr > 0;
      const char* base = have ? vbase + pg * page_bytes : zero_rows;
      const int rs = min(row, vr - 1);
      const unsigned off = have ? (unsigned)((rs * rowstride + 8 * col) * sizeof(T)) : 16u * lane;
      lds_copy16(base, off, vstage + p * TILEB + r0 * ROWB);
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

  // Ping-pong schedule.  A step is two phases: M(j) on the matrix cores (S^T = K . Q^T of step
  // j, and O^T += V^T . P of step j - 1) and S(j) on the vector ALUs (the online softmax of step
  // j's scores into P).  Every wave runs M(0) S(0) M(1) S(1) ... S(n-1) M(n), each phase ending
  // at a workgroup barrier, and waves 4-7 start one phase after waves 0-3: each SIMD holds
  // waves w and w + 4, so one runs a matrix phase while the other runs a softmax phase.
  // Stage rings of three for K and for V: at M(j) every wave issues its share of K(j + 2) and
  // V(j + 1).  Counting phases from the leading waves' M(0) = 0, K(j) is read in phases 2j and
  // 2j + 1 and V(j) in 2j + 2 and 2j + 3, so the slot a refill issued at phase 2j or later
  // overwrites has had its last read; and the refill is needed from phase 2j + 4, so each wave
  // waits for its loads issued before its latest M phase ahead of the barrier that ends phase
  // 2j + 3 (the leading waves' S(j + 1), the trailing waves' M(j + 1)).
  f4 sacc[NP][2];    // S^T tiles of the step in flight: [key tile kt][row tile rt]
  uint2 pb[NP][2];   // P of the previous step, packed as the B operand of P.V (zero before step 0)
#pragma unroll
  for (int kt = 0; kt < NP; ++kt)
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) pb[kt][rt] = make_uint2(0, 0);
  const int tr_row = 4 * lg + (lr >> 2);
  // M(j): the page loads of later steps, then the products as a software pipeline of units of
  // eight 16x16x32 products: units 0-3 are P.V of step j - 1 (pages 2u, 2u + 1 with u = unit / 2,
  // output tiles 4 (unit % 2) .. + 3), units 4-7 are K . Q^T of step j (page unit - 4).  Each unit's
  // LDS operands are read kAhead units ahead into a ring of kAhead + 1 operand buffers, and every
  // unit ends the compiler's scheduling region, so the reads stay that far ahead of the products.
  // One unit ahead is enough: two and three ahead measured no faster (+1 %, +1.5 %) on the
  // Qwen2.5-3B chunked-prefill workload.
  constexpr int kAhead = 1;
  constexpr int NB = kAhead + 1;
  constexpr int MTU = MT / 2;  // output tiles per P.V unit
  static_assert(MTU == KSTEPS, "a P.V unit and a K . Q^T unit take the same operand count");
  uint4 opnd[NB][KSTEPS];
  auto read_unit = [&](int i, int buf, const char* ks, const char* vs) __attribute__((always_inline)) {
    if (i < 4) {
      const int u = i >> 1;
      const char* tra = vs + (2 * u) * TILEB + tr_row * ROWB + (lr & 1) * 8;
      const char* trb = tra + TILEB;
#pragma unroll
      for (int m = 0; m < MTU; ++m) {
        const int mt = MTU * (i & 1) + m;
        const int chunk = ((2 * mt + ((lr & 3) >> 1)) ^ vswz<D>(tr_row)) << 4;
        const uint2 va = lds_read_tr16(tra + chunk), vb = lds_read_tr16(trb + chunk);
        opnd[buf][m] = make_uint4(va.x, va.y, vb.x, vb.y);
      }
    } else {
      const char* krow = ks + (i - 4) * TILEB + lr * ROWB;
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s)
        opnd[buf][s] = *reinterpret_cast<const uint4*>(krow + (((4 * s + lg) ^ kswz<D>(lr)) << 4));
    }
  };
  auto mma_unit = [&](int i, int buf) __attribute__((always_inline)) {
    if (i < 4) {
      const int u = i >> 1;
      uint4 pp[2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
        pp[rt] = make_uint4(pb[2 * u][rt].x, pb[2 * u][rt].y, pb[2 * u + 1][rt].x, pb[2 * u + 1][rt].y);
#pragma unroll
      for (int m = 0; m < MTU; ++m)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
          o[rt][MTU * (i & 1) + m] = Mma<T>::qk(opnd[buf][m], pp[rt], o[rt][MTU * (i & 1) + m]);
    } else {
      const int kt = i - 4;
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) sacc[kt][rt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) sacc[kt][rt] = Mma<T>::qk(opnd[buf][s], qr[rt][s], sacc[kt][rt]);
    }
  };
  // Every M phase runs all eight units, so the pipeline has no branches: at j = 0, P.V multiplies
  // the zero P it starts with by the zero-filled V stage 2 and adds exactly +0 to O; at
  // j = nsteps, K . Q^T reads a stale K stage and its scores are never used.  Unit i's operands go
  // to buffer i % NB.
  // (the caller has read the operands of units 0 .. kAhead - 1)
  auto products = [&](const char* ks, const char* vs) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_barrier(0);
      if (i + kAhead < 8) read_unit(i + kAhead, (i + kAhead) % NB, ks, vs);
      mma_unit(i, i % NB);
      // the unit's 2 * KSTEPS products interleaved with the next unit's operand reads (a P.V
      // unit's 2 * MTU reads one per product, a K . Q^T unit's KSTEPS one per two), which spreads
      // the LDS requests over the unit (2 % faster than the compiler's own order, which bunches
      // them)
      if (i + kAhead < 4) {
#pragma unroll
        for (int x = 0; x < 2 * MTU; ++x) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        }
      } else if (i + kAhead < 8) {
#pragma unroll
        for (int x = 0; x < KSTEPS; ++x) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  static_assert(NP == 4, "the product pipeline is written for four pages a step");
  // Page ids reach the phases a phase early, so that no lookup waits behind the bulk LDS reads of
  // the other waves: pk_next / pv_next (uniform) are the pages this wave loads at its next M phase
  // (K of step j + 2, V of step j + 1 at M(j)); step_pages holds step j's four page ids for S(j).
  int pk_next = 0, pv_next = 0;
  int4 step_pages;
  // (the copies are issued while the first units' operand reads are in flight)
  auto phase_m = [&](int j, const char* ks, const char* vs, unsigned kn, unsigned vn) __attribute__((always_inline)) {
    step_pages = *reinterpret_cast<const int4*>(s_page + min(j, nsteps - 1) * NP);
#pragma unroll
    for (int a = 0; a < kAhead; ++a) read_unit(a, a, ks, vs);
    if (j + 2 < nsteps) issue_k(j + 2, kn, pk_next);
    if (j + 1 < nsteps) issue_v(j + 1, vn, pv_next);
    products(ks, vs);
  };
  auto phase_s = [&](int j) __attribute__((always_inline)) {
    // the next M phase's pages, read now and made scalar at the end of this phase
    const int pk_raw = page_id(j + 3), pv_raw = page_id(j + 2);
    const int kb = k0 + 16 * NP * j;
    bool absent[NP];
    absent[0] = __builtin_amdgcn_readfirstlane(step_pages.x) < 0;
    absent[1] = __builtin_amdgcn_readfirstlane(step_pages.y) < 0;
    absent[2] = __builtin_amdgcn_readfirstlane(step_pages.z) < 0;
    absent[3] = __builtin_amdgcn_readfirstlane(step_pages.w) < 0;
    bool full = kb + 16 * NP <= lim_min;  // (uniform)
#pragma unroll
    for (int kt = 0; kt < NP; ++kt) full = full && !absent[kt];
    // online softmax per row tile on the raw scores (the scale is folded into the exponent's
    // FMA; it is positive, so maxima commute with it)
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      // masked scores (causal limit, keys past the chunk, absent pages) become -inf in place
      // (key kb + 16 kt + 4 lg + i is below the limit iff 16 kt + i < rem: compares with
      // immediates, all inside the branch)
      if (!full) {
        const int rem = lim[rt] - kb - 4 * lg;
#pragma unroll
        for (int kt = 0; kt < NP; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (!(16 * kt + i < rem && !absent[kt])) sacc[kt][rt][i] = -INFINITY;
      }
      float sv[NP * 4];
#pragma unroll
      for (int kt = 0; kt < NP; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[4 * kt + i] = sacc[kt][rt][i];
      float cmax = max_of<NP * 4>(sv);
      cmax = max_across_groups(cmax);
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
      float psum[4];
#pragma unroll
      for (int kt = 0; kt < NP; ++kt) {
        float pr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pr[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[4 * kt + i], scale, nmuse));
          psum[i] = kt == 0 ? pr[i] : psum[i] + pr[i];
        }
        pb[kt][rt] = make_uint2(Mma<T>::pack(pr[0], pr[1]), Mma<T>::pack(pr[2], pr[3]));
      }
      lsum[rt] += (psum[0] + psum[1]) + (psum[2] + psum[3]);
    }
    __builtin_amdgcn_sched_barrier(0);
    pk_next = __builtin_amdgcn_readfirstlane(pk_raw);
    pv_next = __builtin_amdgcn_readfirstlane(pv_raw);
  };
  // this wave's loads issued before its M(j) are complete (M(j)'s may stay in flight)
  auto wait_before = [&](int j) __attribute__((always_inline)) {
    if (j + 2 < nsteps) wait_vmcnt<2 * KL>();
    else wait_vmcnt<0>();
  };
  const bool lead = wave < 4;
  auto round = [&](int j, const char* ks, const char* vs, unsigned kn, unsigned vn) __attribute__((always_inline)) {
    phase_m(j, ks, vs, kn, vn);
    if (!lead) wait_before(j);
    phase_barrier();
    if (j < nsteps) {
      phase_s(j);
      if (lead) wait_before(j);
      phase_barrier();
    }
  };
  if (nsteps > 0) {
    const unsigned sk = lds_addr(s_k), sv = lds_addr(s_v);
    issue_k(0, sk, __builtin_amdgcn_readfirstlane(page_id(0)));
    issue_v(0, sv, __builtin_amdgcn_readfirstlane(page_id(0)));
    pk_next = __builtin_amdgcn_readfirstlane(page_id(2));
    pv_next = __builtin_amdgcn_readfirstlane(page_id(1));
    if (nsteps > 1) {
      issue_k(1, sk + STEPB, __builtin_amdgcn_readfirstlane(page_id(1)));
      wait_vmcnt<2 * KL>();
    } else {
      wait_vmcnt<KL>();
    }
    phase_barrier();  // K(0) staged
    if (!lead) phase_barrier();  // the trailing waves' idle first phase
    int cs = 0;  // stage of step j (j % 3)
#pragma unroll 1
    for (int j = 0; j <= nsteps; ++j) {
      const int ns = cs == 2 ? 0 : cs + 1;  // (j + 1) % 3
      const int ps = cs == 0 ? 2 : cs - 1;  // (j + 2) % 3, also (j - 1) % 3
      round(j, s_k + cs * STEPB, s_v + ps * STEPB, sk + ps * STEPB, sv + ns * STEPB);
      cs = ns;
    }
    if (lead) phase_barrier();  // the leading waves' idle last phase
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
// A workgroup takes merge_rows() rows of one group; D/8 lanes per row, 8 dims each (16-byte
// loads of fp16 partials).  Each round loads kMergeUnroll slots' (max, sum) and rows together,
// from clamped (always valid) addresses, and folds them under a running max: one memory round
// trip per round, and for a group of at most kMergeUnroll slots the plain fold under the
// group's max.
constexpr int kMergeUnroll = 4;
template <int D>
constexpr int merge_rows() { return 256 / (D / 8); }

template <typename T, int D, int G>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillMfmaParams P, const int32_t* groups) {
  constexpr int RB = merge_rows<D>(), TPR = D / 8;
  const int32_t* gr = groups + (int64_t)kGroup * (blockIdx.x / (kRows / RB));
  const int s0 = gr[0], ns = gr[1], qo_start = gr[2], t0 = gr[3], tq = gr[4], h = gr[5];
  const int r = (blockIdx.x % (kRows / RB)) * RB + threadIdx.x / TPR, d = (threadIdx.x % TPR) * 8;
  const int tt = r / G, hh = r % G;
  if (tt >= tq || ns <= 0) return;
  const float2* ml = P.part_ml + (int64_t)s0 * kRows + r;
  const int64_t po = ((int64_t)s0 * kRows + r) * D + d;  // element offset of slot s0's dims
  float M = -INFINITY;
  float den = 0.f;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < ns; s += kMergeUnroll) {
    float2 w[kMergeUnroll];
    float v[kMergeUnroll][8];
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
      const int64_t sl = min(s + u, ns - 1);
      w[u] = ml[sl * kRows];
      if constexpr (kHalfPartials<T>) {
        const uint4 raw = *reinterpret_cast<const uint4*>(reinterpret_cast<const _Float16*>(P.part_o) + po + sl * kRows * D);
        _Float16 hv[8];
        __builtin_memcpy(hv, &raw, 16);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[u][e] = (float)hv[e];
      } else {
        const float4* src = reinterpret_cast<const float4*>(P.part_o + po + sl * kRows * D);
        const float4 a = src[0], b = src[1];
        v[u][0] = a.x; v[u][1] = a.y; v[u][2] = a.z; v[u][3] = a.w;
        v[u][4] = b.x; v[u][5] = b.y; v[u][6] = b.z; v[u][7] = b.w;
      }
    }
    // the running max over the slots loaded so far (repeats of the last slot included, as in a
    // separate max pass); what earlier rounds folded is rescaled to it
    float Mn = M;
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) Mn = fmaxf(Mn, w[u].x);
    if (Mn > M) {
      const float f = den > 0.f ? exp2f(M - Mn) : 0.f;
      den *= f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] *= f;
      M = Mn;
    }
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
      // a slot whose rows saw no key (l = 0) carries no weight; repeats past ns count zero
      // (such a slot's row may hold anything, hence the branch rather than a zero weight)
      const float c = (s + u < ns && w[u].y > 0.f) ? exp2f(w[u].x - M) * w[u].y : 0.f;
      if (c != 0.f) {
        den += c;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += c * v[u][e];
      }
    }
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  T* orow = reinterpret_cast<T*>(P.out) + (int64_t)(qo_start + t0 + tt) * P.o_sn + (int64_t)(h * G + hh) * P.o_sh + d;
  if (P.o_vec) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      T o4[4] = {from_f32<T>(acc[4 * half] * inv), from_f32<T>(acc[4 * half + 1] * inv),
                 from_f32<T>(acc[4 * half + 2] * inv), from_f32<T>(acc[4 * half + 3] * inv)};
      *reinterpret_cast<uint2*>(orow + 4 * half) = *reinterpret_cast<const uint2*>(o4);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) orow[e] = from_f32<T>(acc[e] * inv);
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
