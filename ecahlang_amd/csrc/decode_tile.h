// Pieces of the matrix-core decode kernels (the plain and cascade variants in decode_mfma.hip): the
// global -> LDS page copies with explicit waits, the swizzles of the staged K and V tiles, the
// segment words of the schedule and the unit geometry.
#pragma once
#include "attn_common.h"
#include "mfma_common.h"
#include "decode_sched.h"

namespace pkv {
namespace dtile {

constexpr int W = 8;                // waves per workgroup
constexpr int NT = W * 64;
constexpr float kLazyMax = 8.f;     // a column's reference max moves only on jumps > 2^8

template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// One wave-wide copy global -> LDS: lane l's 16 bytes at src (per lane) land at LDS byte
// dst + 16 l (dst wave-uniform, in M0).  Inline assembly, so the compiler neither tracks nor
// waits for it: the kernels order these copies with explicit vmcnt waits.  `nt` streams the
// K/V pages past the caches; small metadata copies use the default policy.
__device__ __forceinline__ void dma16_nt(const void* src, const char* dst) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(
      (unsigned)(uintptr_t)(const __attribute__((address_space(3))) char*)(dst));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(m0) : "memory", "m0");
}
__device__ __forceinline__ void dma16(const void* src, const char* dst) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(
      (unsigned)(uintptr_t)(const __attribute__((address_space(3))) char*)(dst));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}

// XOR swizzles of 16-byte chunk positions inside a staged row of RB bytes (the low four bits
// only, so a row's chunks stay in their own 256-byte half and every copy still reads whole
// lines).  K rows are read as the QK A operand (16 rows, one chunk per 16-lane group): distinct
// bank groups for the 16 rows.  V rows are read by ds_read_b64_tr_b16 (per 32 lanes, 8 rows x 2
// adjacent chunks): distinct bank groups for those 16 chunks.
template <int RB>
__device__ __forceinline__ int kx(int t) {
  return RB >= 256 ? (t & 15) : ((t >> 1) & 7);
}
template <int RB>
__device__ __forceinline__ int vx(int t) {
  return RB >= 256 ? 2 * (t & 7) : 2 * ((t >> 1) & 3);
}

// Where code picks between an LDS copy and a global-memory copy of the same data (a segment
// record, query rows), plain loads of both get merged into one generic (flat) load, and a flat
// load makes the compiler wait for every vector memory operation in flight (vmcnt(0)) before
// using its result: that drains the page copies in the page loop and the write-through partial
// stores at a range's end.  The LDS copy is read through an LDS-qualified pointer and the global
// one with glb_ld16_sync, each in its own branch.
template <typename V>
__device__ __forceinline__ V lds_ld(const void* p) {
  static_assert(sizeof(V) == 16, "16-byte loads");
  const mfma::u4v x = *(const __attribute__((address_space(3))) mfma::u4v*)(p);
  V r;
  __builtin_memcpy(&r, &x, sizeof(r));
  return r;
}
// A 16-byte global load that has completed when the statement ends (it waits for every vector
// memory operation in flight), for the rare paths inside a page loop: a load the compiler tracks
// there shares destination registers with the common path, and the compiler, which cannot see the
// inline-assembly page copies, then guards those registers with waits that drain every copy.
template <typename V>
__device__ __forceinline__ V glb_ld16_sync(const void* p) {
  static_assert(sizeof(V) == 16, "16-byte loads");
  V r;
  asm volatile("global_load_dwordx4 %0, %1, off\n\ts_waitcnt vmcnt(0)" : "=v"(r) : "v"(p) : "memory");
  return r;
}

// A wave-uniform 64-bit value held in scalar registers.  Selecting per lane between two kernel
// arguments otherwise lets the compiler turn the choice into a per-lane load from the kernel
// argument block (a vector memory load, with the waits that brings in the page loop).
__device__ __forceinline__ int64_t uniform64(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x), hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

struct Seg {
  int b, beg, end, nv, slot0, part, nparts, np;
  int app_page, app_row;  // range page and row of the step's new token (-1: not in this segment)
};
// A segment word (decode_sched.h), clamped so that a stale or malformed schedule cannot index
// past the batch, the record or the partial slots.
__device__ __forceinline__ Seg unpack_seg(int4 v, int len, int batch, int slot_cap) {
  Seg s;
  const int b = v.x & ((1 << kSegBBits) - 1);
  s.b = b >= batch ? batch - 1 : b;
  const int nv = (int)(((unsigned)v.x >> kSegBBits) & 31);
  s.nv = nv > 16 ? 16 : nv;
  s.np = (int)((unsigned)v.x >> (kSegBBits + 5));
  s.beg = v.y & 0x3FF;
  s.end = (v.y >> 16) & 0xFFFF;
  s.end = s.end > len ? len : s.end;
  s.beg = s.beg > s.end ? s.end : s.beg;
  const int app = (v.y >> 10) & 63;
  s.app_page = app ? s.end - 1 - ((app - 1) >> 4) : -1;
  s.app_page = s.app_page >= s.beg ? s.app_page : -1;
  s.app_row = (app - 1) & 15;
  s.nparts = ((v.w >> 16) & 0xFFFF) + 1;
  s.nparts = s.nparts > slot_cap ? slot_cap : s.nparts;
  s.slot0 = v.z < 0 ? 0 : (v.z > slot_cap - s.nparts ? slot_cap - s.nparts : v.z);
  s.part = v.w & 0xFFFF;
  s.part = s.part >= s.nparts ? s.nparts - 1 : s.part;
  s.np = s.np >= s.nparts ? s.nparts - 1 : s.np;
  return s;
}

// Unit geometry: a unit is one page of one head block (16 token rows of HB heads x D dims).
template <int HB, int D>
struct Shape {
  static constexpr int RW = HB * D;        // elements of a unit row
  static constexpr int RB = RW * 2;        // bytes of a unit row
  static constexpr int CPR = RB / 16;      // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;     // rows per 1 KB copy
  static constexpr int NI = 16 / RPI;      // copies per K (or V) tile
  static constexpr int TILE = 16 * RB;     // bytes of a K (or V) tile
  static constexpr int KS = RW / 32;       // QK steps
  static constexpr int KSH = D / 32;       // QK steps per head
  static constexpr int MT = D / 16;        // output tiles of 16 dims
};

// A range record's page id word: the page, and whether other sequences read it too.
__device__ __forceinline__ int pid_page(int raw) { return raw < 0 ? raw : raw & ~kPidShared; }
__device__ __forceinline__ bool pid_cached(int raw) { return raw >= 0 && (raw & kPidShared); }

}  // namespace dtile
}  // namespace pkv
