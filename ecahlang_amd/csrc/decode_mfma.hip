// Paged decode on the matrix cores (fp16 / bf16 caches, page_size 16, head_dim 64 or 128,
// GQA group <= 16), driven by the plan's schedule (decode_sched.h).  Same contract as the
// vector kernel (FlashInfer BatchDecodeWithPagedKVCacheWrapper.run, ecahlang/main.py:68).
//
// Work unit: one page of one head block, i.e. 16 tokens x HB KV heads, where HB is the largest
// power of two with HB * g <= 16 query heads (the MFMA's 16 columns), HB * head_dim <= 256 and
// HB | Hkv.  At Qwen2.5-3B (Hkv 2, g 8, D 128) a unit is a whole page, both heads: 8 KB of K
// and 8 KB of V, each a contiguous run of 16 token rows of 512 bytes.  A wave copies a unit
// global -> LDS with non-temporal global_load_lds_dwordx4 (each instruction reads 1 KB of whole
// 128-byte lines), which streams measurably faster than per-head 64-byte row pieces into
// registers, and needs no registers for the data in flight.
//
// Per unit (column n = query head hb*HB*g + n of the block, n < HB*g):
//   S[t][n]   = sum over the unit row r of K[t][r] * Qbd[r][n]    v_mfma_f32_16x16x32, A = K
//               rows from LDS, B = Qbd, block-diagonal: Q of column n in the dims of its own KV
//               head, zero in the other heads' dims, so one tile holds every head's scores
//   online softmax per column in the accumulator layout (lane: column l%16, tokens 4*(l/16)+i)
//   O^T[d][n] += sum_hh sum_t V_hh[t][d] * P[t][n] [head(n) == hh]   v_mfma_f32_16x16x32 over
//               two heads at once (reduction slots 0-3 = head 2u, 4-7 = head 2u+1; A = two
//               ds_read_b64_tr_b16 of the staged V, B = P masked to each head's columns)
// Every output column is a distinct query head, so the accumulators hold D x 16 values.
//
// A workgroup (8 waves) owns ranges of the schedule; the J = 8 / (Hkv / HB) waves of a head
// block split the range's pages (wave j takes pages j, j+J, ...: a fixed order, so the result is
// reproducible).  Each wave keeps one unit in flight: the next unit's K is requested as soon as
// the current K is consumed, its V as soon as the current V is.  At a segment (sequence) end the
// J states meet in LDS; the owner of each 16-dim tile writes it: output rows, or the partial of a
// sequence split across ranges, merged by the last workgroup to finish (attn_common.h).
#include "decode_tile.h"
#include "../../include/pagedkv.h"

using namespace pkv;

namespace {

using namespace pkv::mfma;
using namespace pkv::dtile;

constexpr int kQArea = 8192;        // LDS bytes for query rows of the range's first segments
constexpr int kSegLds = 64;         // segment records staged in LDS (more are read from memory)
constexpr int kMaxSplit = 64;       // split segments whose arrival a workgroup defers

// Sum of the J (<= W) copies of a tile, read four at a time with every read of a batch issued
// before any add (copies past J repeat copy 0 and are dropped).
template <typename F>
__device__ __forceinline__ f4 fold_copies(int J, F&& copy) {
  f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int b0 = 0; b0 < W; b0 += 4) {
    if (b0 >= J) break;
    f4 x[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) x[k] = copy(b0 + k < J ? b0 + k : 0);
#pragma unroll
    for (int k = 0; k < 4; ++k) acc += b0 + k < J ? x[k] : f4{0.f, 0.f, 0.f, 0.f};
  }
  return acc;
}

template <int HB, int D>
constexpr int mfma_lds_bytes() { return W * 2 * Shape<HB, D>::TILE + kQArea; }

// CASC: the schedule may hold prefix items (a cascade plan).  Without it the prefix-item code is
// not compiled in, which keeps the range loop's registers free of its pressure.
template <typename T, int D, int HB, bool CASC>
__global__ __launch_bounds__(NT) void decode_mfma_kernel(DecodeParams P) {
  using S = Shape<HB, D>;
  constexpr int RB = S::RB, CPR = S::CPR, RPI = S::RPI, NI = S::NI, TILE = S::TILE;
  constexpr int KS = S::KS, KSH = S::KSH, MT = S::MT;

  extern __shared__ __align__(16) char smem[];  // [W][K tile, V tile] | query rows
  __shared__ int s_pid[kRangePages];
  __shared__ int4 s_seg[kSegLds];
  __shared__ float2 s_ml[W][16];
  __shared__ f4 s_x[2][W][64];                // tile exchange at interior segment ends
  __shared__ int s_split[kMaxSplit][4];       // deferred arrivals: sequence, first slot, parts, arrivals
  __shared__ int s_merge[kMaxSplit][3];       // merges owed after the arrivals
  __shared__ int s_nmerge;
  __shared__ int s_next[W];                   // PKV_DECODE_DYNAMIC: next page per head block

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
  const int B = P.batch, g = P.hq / P.hkv;
  const int NHB = P.hkv / HB, J = W / NHB;
  const int hb = wave % NHB, j = wave / NHB;
  const bool active = j < J;
  char* kbuf = smem + wave * 2 * TILE;
  char* vbuf = kbuf + TILE;
  char* qarea = smem + W * 2 * TILE;
  const int qrow = P.hq * D * 2;                       // bytes of one sequence's query rows
  const int qcap = min(4, kQArea / qrow);              // sequences whose rows are staged
  const int ncol = HB * g;                             // columns in use
  const int hn = lr / g;                               // KV head (in the block) of my column
  const bool colv = active && lr < ncol;
  const int qh = hb * ncol + (colv ? lr : 0);          // query head of my column

  const T* kc = reinterpret_cast<const T*>(P.k_cache);
  const T* vc = reinterpret_cast<const T*>(P.v_cache);
  const T* qall = reinterpret_cast<const T*>(P.q);
  T* out = reinterpret_cast<T*>(P.out);
  const int rowstride32 = P.hkv * D;                   // elements between token rows
  const int64_t hboff = (int64_t)hb * HB * D;

  // copy of unit (page pg, head block at element offset hoff) rows into a staged tile, rows
  // swizzled; streamed (nt) or, for pages other workgroups read too, cached
  auto issue_tile = [&](const T* base, int64_t pg, char* dst, bool isv, int64_t hoff = -1,
                        bool nt = true) __attribute__((always_inline)) {
    if (hoff < 0) hoff = hboff;
    const T* pbase = base + pg * P.page_stride + hoff;  // (row offsets fit in 32 bits)
    // The per-copy offsets are recomputed at every call (a few VALU operations): hoisted out of
    // the page loop they would hold 2 * NI registers for the whole loop.
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int t = i * RPI + ln / CPR, pos = ln % CPR;
      const int col = pos ^ (isv ? vx<RB>(t) : kx<RB>(t));
      const T* src = pbase + (t * rowstride32 + 8 * col);
      if (nt) dma16_nt(src, dst + i * 1024); else dma16(src, dst + i * 1024);
    }
  };
  auto page_ok = [&](int pid) __attribute__((always_inline)) -> bool {
    return pid >= 0 && (int64_t)pid < P.num_pages;
  };

  // Prefix items (cascade schedules): the item attends one KV head; a column is (sequence,
  // query head of that head), 16 / g sequences per 16-column block and two blocks, so
  // G = 2 * (16 / g) sequences share an item.
  const int i_spb = 16 / g, i_sib = lr / g, i_gi = lr - i_sib * g;
  struct ItemRegs {
    int hv = 0;
    int pid[2] = {0, 0};
    int4 sv[2];
  };
  auto load_item = [&](int w) __attribute__((always_inline)) -> ItemRegs {
    const int32_t* pr = P.sched_pref + (int64_t)w * kPrecStride;
    ItemRegs r;
    r.hv = pr[lane];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int e = k * i_spb + i_sib;
      r.sv[k] = *reinterpret_cast<const int4*>(pr + kPrecSegOff + 4 * (e < kMaxGroup ? e : kMaxGroup - 1));
      r.pid[k] = pr[kPrecPidOff + 64 * k + lane];
    }
    return r;
  };
  // Item pages: one head's K and V rows of 16 tokens each (TILE1 bytes per half); a wave's unit
  // buffer holds SPW = HB such pages, and a step takes NPS of them.
  constexpr int RB1 = D * 2, CPR1 = RB1 / 16, RPI1 = 64 / CPR1, NI1 = 16 / RPI1, TILE1 = 16 * RB1;
  constexpr int SPW = 2 * TILE / (2 * TILE1);
  constexpr int NPS = SPW >= 2 ? 2 : 1;
  static_assert(SPW >= 1 && MT * 1024 <= 2 * TILE, "prefix item buffers");
  auto item_plen = [&](const ItemRegs& r) __attribute__((always_inline)) -> int {
    const int v = __builtin_amdgcn_readlane(r.hv, kHdrLen);
    return v < 0 ? 0 : (v > kItemPages ? kItemPages : v);
  };
  auto item_head = [&](const ItemRegs& r) __attribute__((always_inline)) -> int {
    const int v = __builtin_amdgcn_readlane(r.hv, kHdrHead);
    return v < 0 ? 0 : (v >= P.hkv ? P.hkv - 1 : v);
  };
  // page p's id (p wave-uniform, < kItemPages)
  auto item_pid = [&](const ItemRegs& r, int p) __attribute__((always_inline)) -> int {
    return __builtin_amdgcn_readlane(p < 64 ? r.pid[0] : r.pid[1], p & 63);
  };
  // The K (or V) rows of step j's pages of this wave into their slots: the wave takes pages
  // wave, wave + W, ...; step j holds its pages NPS j .. NPS j + NPS - 1, the i-th in slot i
  // (K rows, then V rows), copied with the cached policy (every group of the run reads them).
  auto item_issue = [&](const ItemRegs& r, int plen, int hd, int j, bool isv) __attribute__((always_inline)) {
    const int nmine = plen > wave ? (plen - 1 - wave) / W + 1 : 0;
    const T* base = isv ? vc : kc;
    char* wb = smem + wave * 2 * TILE;
#pragma unroll
    for (int x = 0; x < NPS; ++x) {
      const int li = NPS * j + x;
      if (li >= nmine) break;
      const int pid = item_pid(r, wave + W * li);
      const int64_t pg = page_ok(pid) ? pid : 0;
      const T* pb = base + pg * P.page_stride + (int64_t)hd * D;
      char* dst = wb + x * 2 * TILE1 + (isv ? TILE1 : 0);
      int ln = lane;
      asm volatile("" : "+v"(ln));
#pragma unroll
      for (int i = 0; i < NI1; ++i) {
        const int t = i * RPI1 + ln / CPR1, pos = ln % CPR1;
        const int col = pos ^ (isv ? vx<RB1>(t) : kx<RB1>(t));
        dma16(pb + (t * rowstride32 + 8 * col), dst + i * 1024);
      }
    }
  };

  const int N0 = P.num_ctas;
  // XCD-aware range order: workgroups are dealt round-robin to the 8 XCDs, so giving each XCD a
  // run of consecutive ranges keeps a split sequence's partials mostly on one L2.
  const int w0 = (N0 % 8 == 0) ? (int)(blockIdx.x % 8) * (N0 / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
  // The first range's head (fetch 1), its segment records and its first 256 page ids are
  // requested before anything else: none depends on another, and the set-up code below (several
  // hundred instructions) then runs while they are in flight.
  int hv0 = 0, pv0 = 0;
  const bool early = w0 < P.r_cap;
  // A prefix item's record in registers (cascade schedules): its header (lane l: word l), the
  // segments of this lane's two member columns, and its page ids (page p: lane p % 64 of
  // word p / 64).  Every range's slot is read: a range that carries no item ignores it.
  ItemRegs ir0;
  if (early) {
    const int32_t* head0 = P.sched_head + (int64_t)w0 * kHeadWords;
    const int32_t* rec0 = P.sched + (int64_t)w0 * kRecStride;
    hv0 = head0[lane];
    pv0 = head0[kHeadPidOff + lane];
    if constexpr (CASC) ir0 = load_item(w0);
    if (wave == 0) dma16(rec0 + kRecSegOff + 4 * lane, reinterpret_cast<const char*>(s_seg));
    if (wave == 1 % W) dma16(rec0 + kRecPidOff + 4 * lane, reinterpret_cast<const char*>(s_pid));
  }
  // ... and, once the head is in, this wave's first unit: HBM then streams the first pages while
  // the set-up code runs (the range loop takes them over as its first unit)
  int cpid0 = 0;
  bool unit0 = false, item0 = false;  // the first range's first unit, or its item's first pages, issued
  if (early) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // the head is in (compiler-visible vmcnt(0))
    int len0 = __builtin_amdgcn_readlane(hv0, kHdrLen);
    len0 = len0 < 0 ? 0 : (len0 > kRangePages ? kRangePages : len0);
    int nseg0 = __builtin_amdgcn_readlane(hv0, kHdrNseg);
    nseg0 = nseg0 < 0 ? 0 : (nseg0 > len0 ? len0 : nseg0);
    bool plain = w0 < __builtin_amdgcn_readlane(hv0, kHdrRanges) && nseg0 > 0;
    if constexpr (CASC) plain = plain && !__builtin_amdgcn_readlane(hv0, kHdrPrefix);
    const int pi0 = active ? j : len0;
    if constexpr (CASC) {
      // a range that carries a prefix item: the item's first pages go out now, and stream in
      // while the set-up code runs
      if (w0 < __builtin_amdgcn_readlane(hv0, kHdrRanges) && __builtin_amdgcn_readlane(hv0, kHdrPrefix)) {
        const int pl0 = item_plen(ir0), hd0 = item_head(ir0);
        item_issue(ir0, pl0, hd0, 0, false);
        item_issue(ir0, pl0, hd0, 0, true);
        item0 = true;
      }
    }
    if (plain && pi0 < len0) {
      const int raw = __builtin_amdgcn_readlane(pv0, pi0);
      cpid0 = pid_page(raw);
      const int64_t pg = page_ok(cpid0) ? cpid0 : 0;
      issue_tile(kc, pg, kbuf, false, -1, !pid_cached(raw));
      issue_tile(vc, pg, vbuf, true, -1, !pid_cached(raw));
      unit0 = true;
    }
  }
  int nsplit = 0;

  // Deferred arrivals of split segments: every wave waits for its own partial stores, then one
  // lane per split bumps that sequence's counter (all in parallel); the splits that arrived last
  // are merged by the whole workgroup at once.  Inside the page loop (a full record) the
  // register-light global-memory merge is used.
  auto flush_splits = [&](bool in_loop) __attribute__((always_inline)) {
    wait_stores();
    lds_barrier();
    if (wave == 0) {
      int sb = 0, lo = 0, hi = 0, last = 0;
      if (lane < nsplit) {
        sb = s_split[lane][0];
        lo = s_split[lane][1];  // first slot
        hi = s_split[lane][2];  // parts
        const int old = atomicAdd(&P.counters[sb], 1);
        last = old == s_split[lane][3] - 1;
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
    lds_barrier();
    const int nm = __builtin_amdgcn_readfirstlane(s_nmerge);
    if (in_loop) {
      for (int i = 0; i < nm; ++i) merge_partials<T, D>(P, s_merge[i][0], s_merge[i][1], s_merge[i][2]);
    } else {
      merge_queued<T, D>(P, s_merge, nm);
    }
    lds_barrier();
    nsplit = 0;
  };

  // ---- prefix item (decode_sched.h): G sequences x one chunk of pages x one KV head, all
  // shared.  A column of the products is (sequence, query head of the item's head): 16 / g
  // sequences per 16-column block and two blocks, so G = 2 * (16 / g) sequences share each K/V
  // fragment read from LDS.  The chunk's pages are dealt to the waves like a range's (wave r
  // takes pages r, r + W, ...); each wave streams its own pages into its own unit buffer (HB page
  // slots of one head's K and V rows, copied with the cached policy: every group of the run reads
  // the chunk) and attends all G sequences to them, two pages a step, with no barrier until the
  // end, where the W states of each column are folded through LDS in wave order.
  const float scale = P.scale_log2;
  auto prefix_item = [&](int w, bool pre) __attribute__((always_inline)) {
    // the record: requested at the kernel's start for the first range, else now
    const ItemRegs ir = pre ? ir0 : load_item(w);
    if (!pre) __builtin_amdgcn_s_waitcnt(0x0F70);
    const int plen = item_plen(ir), hd = item_head(ir);
    int pn = __builtin_amdgcn_readlane(ir.hv, kHdrNseg);
    pn = pn < 0 ? 0 : (pn > kMaxGroup ? kMaxGroup : pn);
    if (nsplit + kMaxGroup > kMaxSplit) flush_splits(true);  // room for this item's arrivals
    lds_barrier();  // the previous readers of the unit buffers are done
    // my columns and their sequences (segment e = k * spb + column / g)
    const int spb = i_spb, sib = i_sib, gi = i_gi;
    const int qhd = hd * g + gi;                        // query head of my column
    Seg sgk[2];
    bool ok[2];
    uint4 qk2[2][KSH];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int e = k * spb + sib;
      ok[k] = sib < spb && e < pn;
      sgk[k] = unpack_seg(ir.sv[k], plen, B, P.slot_cap);
      const T* src = qall + (int64_t)sgk[k].b * P.q_sn + (int64_t)qhd * P.q_sh + 8 * lg;
#pragma unroll
      for (int s = 0; s < KSH; ++s)
        qk2[k][s] = ok[k] ? *reinterpret_cast<const uint4*>(src + 32 * s) : make_uint4(0, 0, 0, 0);
    }
    f4 po[2][MT];
    float pm[2], pl[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) po[k][mt] = f4{0.f, 0.f, 0.f, 0.f};
      pm[k] = -INFINITY;
      pl[k] = 0.f;
    }
    auto pid_at = [&](int p) __attribute__((always_inline)) -> int { return item_pid(ir, p); };
    const int nmine = plen > wave ? (plen - 1 - wave) / W + 1 : 0;
    const int nsteps = (nmine + NPS - 1) / NPS;
    char* wbuf = smem + wave * 2 * TILE;
    // (the query rows' loads were issued before the pages': the compiler's wait for them, at
    // their first use, also covers these copies)
    auto issue_half = [&](int j, bool isv) __attribute__((always_inline)) { item_issue(ir, plen, hd, j, isv); };
    // vmcnt allowing the copies of n pages (of one half) to stay in flight
    auto wait_pages = [&](int n) __attribute__((always_inline)) {
      if (n <= 0) wait_vm<0>();
      else if (n == 1) wait_vm<NI1>();
      else wait_vm<2 * NI1>();
    };
    auto pages_of = [&](int j) __attribute__((always_inline)) -> int {
      return j < nsteps ? min(NPS, nmine - NPS * j) : 0;
    };
    if (nsteps > 0 && !(pre && item0)) {  // (the first range's went out at the start)
      issue_half(0, false);
      issue_half(0, true);
    }
    for (int j = 0; j < nsteps; ++j) {
      const int np2 = pages_of(j);
      const int pid0 = pid_at(wave + W * (NPS * j));
      const int pid1 = np2 == 2 ? pid_at(wave + W * (NPS * j + 1)) : pid0;
      const bool v0 = page_ok(pid0), v1 = np2 == 2 && page_ok(pid1);
      wait_pages(np2);  // K of step j has landed (its V may still be in flight)
      // Straight-line step: both slots and both blocks always; a lone last page leaves slot 1
      // stale and a page outside the pool holds page 0's rows, so their scores are replaced by
      // -inf and their V fragments by zeros, by selects.
      const char* kb0 = wbuf;
      const char* kb1 = wbuf + (NPS == 2 ? 2 * TILE1 : 0);
      // lane-derived LDS offsets are recomputed here, not kept from the kernel's start
      int l2 = lane;
      asm volatile("" : "+v"(l2));
      const int lr2 = l2 & 15, lg2 = l2 >> 4;
      uint4 ka[2][KSH];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const char* krow = (x ? kb1 : kb0) + lr2 * RB1;
#pragma unroll
        for (int s = 0; s < KSH; ++s)
          ka[x][s] = *reinterpret_cast<const uint4*>(krow + (((4 * s + lg2) ^ kx<RB1>(lr2)) << 4));
      }
      f4 sa[2][2];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          sa[x][k] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < KSH; ++s) sa[x][k] = Mma<T>::qk(ka[x][s], qk2[k][s], sa[x][k]);
        }
      }
      wait_lgkm0();  // the K rows have been read: the slots' K halves can be refilled
      issue_half(j + 1, false);
      // online softmax per block over the step's 16 or 32 tokens (every chunk page is full)
      uint4 pb[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        float sv[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sv[i] = v0 ? sa[0][k][i] : -INFINITY;
          sv[4 + i] = v1 ? sa[1][k][i] : -INFINITY;
        }
        float cmax = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                           fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
        cmax = max_across_groups(cmax);
        const float cms = cmax * scale;
        const bool grow = cms > pm[k] + kLazyMax;
        if (__ballot(grow)) {
          const float mnew = grow ? cms : pm[k];
          const float alpha = __builtin_amdgcn_exp2f(pm[k] - mnew);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) po[k][mt] *= alpha;
          pl[k] *= alpha;
          pm[k] = mnew;
        }
        const float nmu = pm[k] == -INFINITY ? 0.f : -pm[k];
        float e8[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) e8[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[i], scale, nmu));
        pl[k] += ((e8[0] + e8[1]) + (e8[2] + e8[3])) + ((e8[4] + e8[5]) + (e8[6] + e8[7]));
        pb[k] = make_uint4(Mma<T>::pack(e8[0], e8[1]), Mma<T>::pack(e8[2], e8[3]),
                           Mma<T>::pack(e8[4], e8[5]), Mma<T>::pack(e8[6], e8[7]));
      }
      wait_pages(pages_of(j + 1));  // V of step j has landed (step j + 1's K may be in flight)
      // V^T fragments of both slots: reduction slots 0-3 the first page, 4-7 the second
      const int tr_row = 4 * lg2 + (lr2 >> 2);
      const char* vb0 = kb0 + TILE1 + tr_row * RB1 + (lr2 & 1) * 8;
      const char* vb1 = kb1 + TILE1 + tr_row * RB1 + (lr2 & 1) * 8;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int c = (2 * mt + ((lr2 & 3) >> 1)) ^ vx<RB1>(tr_row);
        const uint2 a0 = lds_read_tr16(vb0 + (c << 4));
        const uint2 a1 = lds_read_tr16(vb1 + (c << 4));
        const uint4 va = make_uint4(v0 ? a0.x : 0u, v0 ? a0.y : 0u, v1 ? a1.x : 0u, v1 ? a1.y : 0u);
        po[0][mt] = Mma<T>::qk(va, pb[0], po[0][mt]);
        po[1][mt] = Mma<T>::qk(va, pb[1], po[1][mt]);
      }
      wait_lgkm0();  // the V rows have been read: the slots' V halves can be refilled
      issue_half(j + 1, true);
    }
    // ---- the W waves' states of each column, folded in wave order: (max, sum) through the
    // exchange buffer, then the blocks' tiles through the unit buffers (now idle); tile (k, mt)
    // is folded, normalised and written by wave (k MT + mt) % W
    float2* s_iml = reinterpret_cast<float2*>(&s_x[0][0][0]);  // [W][2][16]
    float ltot[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) ltot[k] = sum_across_groups(pl[k]);
    if (lg == 0) {
#pragma unroll
      for (int k = 0; k < 2; ++k) s_iml[(wave * 2 + k) * 16 + lr] = make_float2(pm[k], ltot[k]);
    }
    lds_barrier();
    float Mk[2], Lk[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      float2 v[W];
#pragma unroll
      for (int ww = 0; ww < W; ++ww) v[ww] = s_iml[(ww * 2 + k) * 16 + lr];
      float M = -INFINITY;
#pragma unroll
      for (int ww = 0; ww < W; ++ww) M = fmaxf(M, v[ww].x);
      const float mu = M == -INFINITY ? 0.f : M;
      float L = 0.f;
#pragma unroll
      for (int ww = 0; ww < W; ++ww) L += v[ww].y * __builtin_amdgcn_exp2f(v[ww].x - mu);
      const float cs = __builtin_amdgcn_exp2f(pm[k] - mu);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) po[k][mt] *= cs;
      Mk[k] = M;
      Lk[k] = L;
    }
    // both blocks' tiles in one exchange when a wave's buffer holds them, else a block at a time
    constexpr int KR = 2 * MT * 1024 <= 2 * TILE ? 2 : 1;  // blocks per exchange round
#pragma unroll
    for (int k0 = 0; k0 < 2; k0 += KR) {
      if (k0 > 0) lds_barrier();  // the previous round's folds have read the buffers
#pragma unroll
      for (int kk = 0; kk < KR; ++kk)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          *reinterpret_cast<f4*>(wbuf + (kk * MT + mt) * 1024 + lane * 16) = po[k0 + kk][mt];
      lds_barrier();
#pragma unroll
      for (int kk = 0; kk < KR; ++kk) {
        const int k = k0 + kk;
        const float inv = Lk[k] > 0.f ? 1.f / Lk[k] : 0.f;
        const int64_t slot = (int64_t)sgk[k].slot0 + sgk[k].part;
        const int64_t sidx = slot * P.hq + qhd;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if ((k * MT + mt) % W != wave) continue;
          f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ww = 0; ww < W; ++ww)
            acc += *reinterpret_cast<const f4*>(smem + ww * 2 * TILE + (kk * MT + mt) * 1024 + lane * 16);
          if (ok[k]) st_dev4(P.part_o, (uint32_t)((sidx * D + 16 * mt + 4 * lg) * sizeof(float)), acc * inv);
        }
        if (wave == 0 && ok[k]) {
          if (lg == 0) store_partial_ml(P, slot, qhd, Mk[k], Lk[k]);
          if (gi == 0 && lg == 0) {
            const int e = k * spb + sib;
            s_split[nsplit + e][0] = sgk[k].b;
            s_split[nsplit + e][1] = sgk[k].slot0;
            s_split[nsplit + e][2] = sgk[k].nparts;
            s_split[nsplit + e][3] = sgk[k].nparts + sgk[k].np * (P.hkv - 1);
          }
        }
      }
    }
    nsplit += pn;
    lds_barrier();  // every wave is done with the buffers; the arrivals are queued
  };

  int rmax = P.r_cap;  // ranges of this plan (from the first record; never past the workspace)
  for (int w = w0; w < rmax; w += N0) {
    const int32_t* rec = P.sched + (int64_t)w * kRecStride;
    const int32_t* head = P.sched_head + (int64_t)w * kHeadWords;
    lds_barrier();  // the previous range's readers of s_pid / s_seg / the query rows are done
    // ---- fetch 1: the range's head: header and first segments (words 0..63), first 64 page ids
    // (the first range's were requested at the start, with its first two fetch-2 jobs)
    const bool first = early && w == w0;
    const int hv = first ? hv0 : head[lane];
    const int pv = first ? pv0 : head[kHeadPidOff + lane];
    const int rr = __builtin_amdgcn_readlane(hv, kHdrRanges);
    rmax = rr < rmax ? rr : rmax;
    int len = __builtin_amdgcn_readlane(hv, kHdrLen);
    len = len < 0 ? 0 : (len > kRangePages ? kRangePages : len);
    int nseg = __builtin_amdgcn_readlane(hv, kHdrNseg);
    nseg = nseg < 0 ? 0 : (nseg > len ? len : nseg);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // fetch 1 complete (compiler-visible vmcnt(0))
    if (w >= rmax) break;
    // the early copies into s_seg / s_pid stand for this range's first two fetch-2 jobs (a prefix
    // item keeps its record in registers and leaves those arrays alone)
    const bool early_jobs = first;
    if constexpr (CASC) {
      if (__builtin_amdgcn_readlane(hv, kHdrPrefix)) {
        prefix_item(w, first);
        // The item's arrivals now: its G sequences' other parts are mostly still running, so
        // their merges fall to those parts' workgroups instead of piling up on this one.
        if (nsplit > 0) flush_splits(false);
      }
    }
    if (nseg == 0) continue;
    // segment s < kHeadSegs from the fetch-1 registers
    auto seg_reg = [&](int s) __attribute__((always_inline)) -> int4 {
      return make_int4(__builtin_amdgcn_readlane(hv, kRecSegOff + 4 * s),
                       __builtin_amdgcn_readlane(hv, kRecSegOff + 4 * s + 1),
                       __builtin_amdgcn_readlane(hv, kRecSegOff + 4 * s + 2),
                       __builtin_amdgcn_readlane(hv, kRecSegOff + 4 * s + 3));
    };
    const int qs = min(nseg, qcap);
    // ---- fetch 2 (copies into LDS): segment records, page ids, query rows of the first qs
    // segments, then this wave's first unit.  Job k of the first three kinds is wave k % W's.
    const int npj = (len + 255) / 256;
    const int qchunks = qs * (qrow / 16);
    const int nqj = (qchunks + 63) / 64;
    const int njobs = 1 + npj + nqj;
    for (int k = wave; k < njobs; k += W) {
      if (early_jobs && k <= 1) continue;  // (issued at the start)
      if (k == 0) {
        dma16(rec + kRecSegOff + 4 * lane, reinterpret_cast<const char*>(s_seg));
      } else if (k <= npj) {
        const int i = k - 1;
        dma16(rec + kRecPidOff + 256 * i + 4 * lane, reinterpret_cast<const char*>(s_pid + 256 * i));
      } else {
        const int i = k - 1 - npj;
        int c = 64 * i + lane;
        c = c < qchunks ? c : qchunks - 1;
        const int per = qrow / 16, s = c / per, r = c - s * per;
        const int h = r / (D / 8), dc = r - h * (D / 8);
        int4 sv = seg_reg(0);
#pragma unroll
        for (int x = 1; x < 4; ++x) sv = s == x ? seg_reg(x) : sv;
        const int b = unpack_seg(sv, len, B, P.slot_cap).b;
        dma16(qall + (int64_t)b * P.q_sn + (int64_t)h * P.q_sh + 8 * dc, qarea + 1024 * i);
      }
    }
    if (threadIdx.x < W) s_next[threadIdx.x] = J;  // (pages 0 .. J-1 go to the ranks in order)
    int pi = active ? j : len;  // this wave's current page (range page index)
    int cpid = 0;
    bool have = pi < len;
    // (the first range's first unit went out at the start, before these copies: then every
    // copy is waited for, the unit included)
    const bool issued = first && unit0;
    if (issued) {
      cpid = cpid0;
    } else if (have) {
      const int raw = __builtin_amdgcn_readlane(pv, pi);
      cpid = pid_page(raw);
      const int64_t pg = page_ok(cpid) ? cpid : 0;
      issue_tile(kc, pg, kbuf, false, -1, !pid_cached(raw));
      issue_tile(vc, pg, vbuf, true, -1, !pid_cached(raw));
    }
    if (have && !issued) wait_vm<2 * NI>(); else wait_vm<0>();
    lds_barrier();

    // ---- per-segment state
    int si = 0;
    Seg sg;
    auto seg_at = [&](int s) __attribute__((always_inline)) -> Seg {
      int4 v;
      if (s < kSegLds) {
        v = lds_ld<int4>(s_seg + s);
        v = make_int4(__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                      __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w));
      } else {
        v = glb_ld16_sync<int4>(rec + kRecSegOff + 4 * s);
        v = make_int4(__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                      __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w));
      }
      return unpack_seg(v, len, B, P.slot_cap);
    };
    uint4 qop[KS];
    f4 o[MT];
    float m = -INFINITY, lsum = 0.f;
    auto start_segment = [&]() __attribute__((always_inline)) {
      sg = seg_at(si);
      {
        // Fused append: the wave that will attend the page that receives the step's token
        // (range page k goes to rank k % J) copies the token's K and V rows of its head block
        // into its 1 KB of the exchange buffer now (lane l's 16 bytes at byte 16 l: K chunks,
        // then V chunks), so they have landed when that page comes up.  The buffer is free
        // until this segment's end: exchanges write it only there.
        if (P.ak && active && sg.app_page >= 0 && sg.app_page % J == j) {
          const int c = lane % (2 * CPR), cc = c % CPR;
          const bool isv = c >= CPR;
          const int64_t h = (int64_t)hb * HB + cc / (D / 8);
          const int64_t kb = uniform64((int64_t)(P.ak + (int64_t)sg.b * P.ak_sn)), ksh = uniform64(P.ak_sh);
          const int64_t vb = uniform64((int64_t)(P.av + (int64_t)sg.b * P.av_sn)), vsh = uniform64(P.av_sh);
          const char* src = (const char*)((isv ? vb : kb) + h * (isv ? vsh : ksh));
          dma16(src + 16 * (cc % (D / 8)), reinterpret_cast<const char*>(&s_x[0][wave][0]));
        }
      }
      // query operand: column lr's query head, dims of its own KV head only
      uint4 qv[KSH];
      if (si < qs) {
        const char* src = qarea + si * qrow + qh * D * 2 + 16 * lg;
#pragma unroll
        for (int s = 0; s < KSH; ++s) qv[s] = lds_ld<uint4>(src + 64 * s);
        asm volatile("" ::: "memory");
      } else {
        const T* src = qall + (int64_t)sg.b * P.q_sn + (int64_t)qh * P.q_sh + 8 * lg;
#pragma unroll
        for (int s = 0; s < KSH; ++s) qv[s] = glb_ld16_sync<uint4>(src + 32 * s);
      }
#pragma unroll
      for (int s = 0; s < KS; ++s) qop[s] = (colv && hn == s / KSH) ? qv[s % KSH] : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) o[mt] = f4{0.f, 0.f, 0.f, 0.f};
      m = -INFINITY;
      lsum = 0.f;
    };

    auto end_segment = [&]() __attribute__((always_inline)) {
      const float ltot = sum_across_groups(lsum);
      const bool whole = sg.nparts == 1;
      float M = m, L = ltot;
      if (J > 1) {
        // (every read of the J copies is issued at once: slots past J repeat slot 0 and are
        // dropped by the selects)
        if (active && lg == 0) s_ml[wave][lr] = make_float2(m, ltot);
        lds_barrier();
        if (active) {
          float2 v[W];
#pragma unroll
          for (int jj = 0; jj < W; ++jj) v[jj] = s_ml[hb + NHB * (jj < J ? jj : 0)][lr];
          M = -INFINITY;
#pragma unroll
          for (int jj = 0; jj < W; ++jj) M = jj < J ? fmaxf(M, v[jj].x) : M;
          const float mu = M == -INFINITY ? 0.f : M;
          L = 0.f;
#pragma unroll
          for (int jj = 0; jj < W; ++jj) L += jj < J ? v[jj].y * __builtin_amdgcn_exp2f(v[jj].x - mu) : 0.f;
          const float cs = __builtin_amdgcn_exp2f(m - mu);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) o[mt] *= cs;
        }
        // tile mt is folded and written by rank mt % J of the head block
        if (si == nseg - 1) {
          // the range's last segment: no copy is in flight into any page buffer, so every wave
          // parks all its tiles in its own buffer and one barrier covers the whole exchange
          char* mine = smem + wave * 2 * TILE;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) *reinterpret_cast<f4*>(mine + mt * 1024 + lane * 16) = o[mt];
          lds_barrier();
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            if (active && j == mt % J) {
              o[mt] = fold_copies(J, [&](int jj) __attribute__((always_inline)) -> f4 {
                return *reinterpret_cast<const f4*>(smem + (hb + NHB * jj) * 2 * TILE + mt * 1024 + lane * 16);
              });
            }
          }
        } else {
          // next units are in flight into the page buffers: one tile per step through two
          // alternating exchange buffers (step mt + 2 rewrites a buffer only after the barrier
          // of step mt + 1, which every reader of step mt has passed)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            s_x[mt & 1][wave][lane] = o[mt];
            lds_barrier();
            if (active && j == mt % J) {
              o[mt] = fold_copies(J, [&](int jj) __attribute__((always_inline)) -> f4 {
                return s_x[mt & 1][hb + NHB * jj][lane];
              });
            }
          }
        }
      }
      if (!whole && threadIdx.x == 0) {
        s_split[nsplit][0] = sg.b;
        s_split[nsplit][1] = sg.slot0;
        s_split[nsplit][2] = sg.nparts;
        s_split[nsplit][3] = sg.nparts + sg.np * (P.hkv - 1);
      }
      if (colv) {
        const float inv = L > 0.f ? 1.f / L : 0.f;
        if (whole) {
          T* orow = out + (int64_t)sg.b * P.o_sn + (int64_t)qh * P.o_sh + 4 * lg;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            if (mt % J != j) continue;
            if (P.o_vec) {
              *reinterpret_cast<uint2*>(orow + 16 * mt) = make_uint2(Mma<T>::pack(o[mt][0] * inv, o[mt][1] * inv),
                                                                     Mma<T>::pack(o[mt][2] * inv, o[mt][3] * inv));
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i) orow[16 * mt + i] = from_f32<T>(o[mt][i] * inv);
            }
          }
        } else {
          const int64_t slot = (int64_t)sg.slot0 + sg.part, sidx = slot * P.hq + qh;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            if (mt % J != j) continue;
            st_dev4(P.part_o, (uint32_t)((sidx * D + 16 * mt + 4 * lg) * sizeof(float)), o[mt] * inv);
          }
          if (j == 0 && lg == 0) store_partial_ml(P, slot, qh, M, L);
        }
      }
      lds_barrier();  // s_split / s_ml / s_x are read before the next segment writes them
      if (!whole && ++nsplit == kMaxSplit) flush_splits(true);
      ++si;
      if (si < nseg) start_segment();
    };

    start_segment();
    while (have) {
      while (si < nseg && pi >= sg.end) end_segment();
      if (si >= nseg) {  // (a page no segment covers: only for a malformed schedule)
        wait_vm<0>();
        break;
      }
      // K of unit pi has landed (its V may still be in flight)
      wait_vm<NI>();
      {
        // Fused append at the page that receives the step's token: once the page's V and the
        // new rows (copied at the segment's start) have landed, the rows replace their row of
        // the staged K and V tiles and are written to that slot of the page in the cache.
        if (P.ak && pi == sg.app_page) {
          wait_vm<0>();
          if (lane < 2 * CPR) {
            const bool isv = lane >= CPR;
            const int c = lane - (isv ? CPR : 0), r = sg.app_row;
            const uint4 x = *reinterpret_cast<const uint4*>(&s_x[0][wave][lane]);
            char* tile = isv ? vbuf : kbuf;
            *reinterpret_cast<uint4*>(tile + r * RB + ((c ^ (isv ? vx<RB>(r) : kx<RB>(r))) << 4)) = x;
            if (page_ok(cpid)) {
              T* dst = const_cast<T*>(isv ? vc : kc) + (int64_t)cpid * P.page_stride + (r * rowstride32 + 8 * c) +
                       hboff;
              *reinterpret_cast<uint4*>(dst) = x;
            }
          }
        }
      }
      f4 sacc = f4{0.f, 0.f, 0.f, 0.f};
      const char* krow = kbuf + lr * RB;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const uint4 a = *reinterpret_cast<const uint4*>(krow + (((4 * s + lg) ^ kx<RB>(lr)) << 4));
        sacc = Mma<T>::qk(a, qop[s], sacc);
      }
      // the K operand reads run up to four ahead of their (chained) products; left to itself the
      // compiler reuses one operand register and waits out each read's LDS latency in turn
      {
        constexpr int AH = KS < 4 ? KS : 4;
        __builtin_amdgcn_sched_group_barrier(0x100, AH, 0);  // DS reads
#pragma unroll
        for (int x = 0; x < KS - AH; ++x) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, AH, 0);
      }
      // next page: fixed (rank j takes j, j+J, ...: reproducible) or, with PKV_DECODE_DYNAMIC,
      // the head block's next page on demand (waves finish together; the summation order varies)
      int nxt = pi + J;
      if (P.dynamic) {
        int v = 0;
        if (lane == 0) v = atomicAdd(&s_next[hb], 1);
        nxt = __builtin_amdgcn_readfirstlane(v);
      }
      const bool more = nxt < len;
      int nraw = 0;
      if (more) nraw = __builtin_amdgcn_readfirstlane(s_pid[nxt]);
      const int npid = pid_page(nraw);
      const bool nnt = !pid_cached(nraw);
      wait_lgkm0();  // the K tile has been read: it can be refilled
      if (more) issue_tile(kc, page_ok(npid) ? npid : 0, kbuf, false, -1, nnt);
      // softmax over the unit's 16 tokens (only a sequence's last page is partial)
      int nv = pi == sg.end - 1 ? sg.nv : 16;
      nv = page_ok(cpid) ? nv : 0;
      float sv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[i] = (4 * lg + i < nv) ? sacc[i] : -INFINITY;
      float cmax = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
      cmax = max_across_groups(cmax);
      const float cms = cmax * scale;
      const bool grow = cms > m + kLazyMax;  // (false while every score so far is masked)
      if (__ballot(grow)) {
        const float mnew = grow ? cms : m;
        const float alpha = __builtin_amdgcn_exp2f(m - mnew);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) o[mt] *= alpha;
        lsum *= alpha;
        m = mnew;
      }
      const float nmu = m == -INFINITY ? 0.f : -m;
      float pr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) pr[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[i], scale, nmu));
      lsum += (pr[0] + pr[1]) + (pr[2] + pr[3]);
      const uint2 pb = make_uint2(Mma<T>::pack(pr[0], pr[1]), Mma<T>::pack(pr[2], pr[3]));
      // V of unit pi has landed (the next unit's K may still be in flight)
      if (more) wait_vm<NI>(); else wait_vm<0>();
      if (nv < 16) {  // rows past the sequence's end read as zeros (0 * NaN would poison P.V)
        for (int c = lane; c < (16 - nv) * CPR; c += 64)
          *reinterpret_cast<uint4*>(vbuf + nv * RB + 16 * c) = make_uint4(0, 0, 0, 0);
      }
      const int tr_row = 4 * lg + (lr >> 2);
      const char* trb = vbuf + tr_row * RB + (lr & 1) * 8;
      if constexpr (HB == 1) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int chunk = (2 * mt + ((lr & 3) >> 1)) ^ vx<RB>(tr_row);
          o[mt] = Mma<T>::pv(lds_read_tr16(trb + (chunk << 4)), pb, o[mt]);
        }
      } else {
#pragma unroll
        for (int u = 0; u < HB / 2; ++u) {
          const uint2 p0 = hn == 2 * u ? pb : make_uint2(0, 0);
          const uint2 p1 = hn == 2 * u + 1 ? pb : make_uint2(0, 0);
          const uint4 pp = make_uint4(p0.x, p0.y, p1.x, p1.y);
          // the V^T operand reads run two output tiles ahead of their products (the same
          // register reuse as for K otherwise serialises them)
          uint2 va[MT], vb[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const int c0 = ((2 * u) * D) / 8 + 2 * mt + ((lr & 3) >> 1);
            const int c1 = c0 + D / 8;
            va[mt] = lds_read_tr16(trb + ((c0 ^ vx<RB>(tr_row)) << 4));
            vb[mt] = lds_read_tr16(trb + ((c1 ^ vx<RB>(tr_row)) << 4));
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            o[mt] = Mma<T>::qk(make_uint4(va[mt].x, va[mt].y, vb[mt].x, vb[mt].y), pp, o[mt]);
          {
            constexpr int AH = MT < 2 ? MT : 2;
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * AH, 0);
#pragma unroll
            for (int x = 0; x < MT - AH; ++x) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
              __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, AH, 0);
          }
        }
      }
      wait_lgkm0();  // the V tile has been read: it can be refilled
      if (more) issue_tile(vc, page_ok(npid) ? npid : 0, vbuf, true, -1, nnt);
      pi = nxt;
      cpid = npid;
      have = more;
    }
    while (si < nseg) end_segment();
  }  // ranges
  if (nsplit > 0) flush_splits(false);
  // output rows of sequences that own no page
  const int ne = P.sched_hdr[kGhEmpty];
  for (int e = blockIdx.x; e < ne && e < B; e += gridDim.x) {
    int b = P.sched_hdr[kGlobHdr + e];
    if (b < 0 || b >= B) continue;
    for (int x = threadIdx.x; x < P.hq * D; x += NT) {
      const int h = x / D, d = x - h * D;
      out[(int64_t)b * P.o_sn + (int64_t)h * P.o_sh + d] = from_f32<T>(0.f);
    }
  }
}

template <typename T, int D, int HB>
int launch(const DecodeParams& P, hipStream_t s) {
  constexpr int lds = mfma_lds_bytes<HB, D>();
  if (P.cascade)
    hipLaunchKernelGGL((decode_mfma_kernel<T, D, HB, true>), dim3(P.num_ctas), dim3(NT), lds, s, P);
  else
    hipLaunchKernelGGL((decode_mfma_kernel<T, D, HB, false>), dim3(P.num_ctas), dim3(NT), lds, s, P);
  return (int)hipGetLastError();
}

template <typename T>
int launch_t(const DecodeParams& P, int d, hipStream_t s) {
  const int hb = decode_head_block(d, P.hq / P.hkv, P.hkv);
  if (d == 128) return hb == 2 ? launch<T, 128, 2>(P, s) : launch<T, 128, 1>(P, s);
  return hb == 4 ? launch<T, 64, 4>(P, s) : (hb == 2 ? launch<T, 64, 2>(P, s) : launch<T, 64, 1>(P, s));
}

}  // namespace

namespace pkv {

bool decode_mfma_supported(int dtype, int d, int g, int hkv, int batch) {
  (void)batch;
  if (!((dtype == kF16 || dtype == kBF16) && (d == 64 || d == 128) && g >= 1 && g <= 16 && hkv >= 1))
    return false;
  return hkv / decode_head_block(d, g, hkv) <= W;
}

// Sequences that share one prefix item, G = 2 * (16 / g), or 0 when the shape cannot group.
int decode_mfma_group(int d, int g, int hkv) {
  if (!((d == 64 || d == 128) && g >= 1 && g <= 16 && hkv >= 1)) return 0;
  const int G = 2 * (16 / g);  // two 16-column blocks of 16 / g sequences each
  return G <= kMaxGroup ? G : 0;
}

int decode_mfma_dispatch(const DecodeParams& P, int dtype, int d, hipStream_t s) {
  if (P.ps != 16) return decode_valu_dispatch(P, dtype, d, s);
  // plain schedules with the fixed page order: each wave streams one run of its range's pages
  return dtype == kF16 ? launch_t<_Float16>(P, d, s) : launch_t<__hip_bfloat16>(P, d, s);
}

}  // namespace pkv
