// Page-table metadata kernels and the K/V append scatter.
//
//   pkv_get_seq_lens                 <- flashinfer.get_seq_lens              (ecahlang/manager.py:143, 170)
//   pkv_get_batch_indices_positions  <- flashinfer.get_batch_indices_positions (ecahlang/manager.py:144-146, 171-173)
//   pkv_append_paged_kv_cache        <- flashinfer.page.append_paged_kv_cache (ecahlang/manager.py:155-165, 175-185, 271-280)
//   pkv_append_paged_kv_cache_slots  <- the same append with each token's slot resolved beforehand
//                                       (the CUDA-graph decode step, ecahlang/manager.py:270-280)
//
// The append is pure data movement: every byte of the new K/V rows lands, unchanged, in
// cache[page][kv][slot][head][:] with page = kv_indices[kv_indptr[b] + pos / page_size] and
// slot = pos % page_size.  Each lane moves one 16-byte vector (or one element on the
// misaligned path), K and V rows of every head are handled by one launch, and consecutive
// lanes cover consecutive bytes of a destination row so both sides coalesce.
#include "common.h"
#include "../../include/pagedkv.h"

using namespace pkv;

namespace {

__global__ void seq_lens_kernel(const int32_t* __restrict__ indptr, const int32_t* __restrict__ last,
                                int32_t batch, int32_t ps, int32_t* __restrict__ out) {
  int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  int np = indptr[b + 1] - indptr[b];
  int full = np - 1 > 0 ? np - 1 : 0;
  out[b] = full * ps + last[b];
}

__global__ void batch_positions_kernel(const int32_t* __restrict__ append_indptr,
                                       const int32_t* __restrict__ seq_lens, int32_t batch,
                                       int32_t nnz, int32_t* __restrict__ bidx,
                                       int32_t* __restrict__ pos) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nnz) return;
  int b = upper_index(append_indptr, batch, i);
  int start = append_indptr[b];
  int len = append_indptr[b + 1] - start;
  bidx[i] = b;
  pos[i] = seq_lens[b] - len + (i - start);
}

// Destination of token i: (ok, page, slot).  With SLOTS, slots[i] = page * ps + slot (from the
// page-table gather), one lookup instead of the three dependent ones through batch_indices /
// positions, kv_indptr and kv_indices.  Metadata that points outside the sequence's pages,
// past num_indices entries or outside the pool gives ok = false.
template <bool SLOTS>
__device__ __forceinline__ bool resolve_dst(int64_t i, const int32_t* __restrict__ bidx,
                                            const int32_t* __restrict__ pos, const int32_t* __restrict__ slots,
                                            const int32_t* __restrict__ kv_indices, int64_t num_indices,
                                            const int32_t* __restrict__ kv_indptr, int32_t batch,
                                            int64_t num_pages, int32_t ps, int& page, int& slot) {
  bool ok;
  page = -1;
  slot = 0;
  if constexpr (SLOTS) {
    const int sl = slots[i];
    ok = sl >= 0 && sl / ps < num_pages;
    page = sl / ps;
    slot = sl - page * ps;
  } else {
    const int b = bidx[i];
    const int p = pos[i];
    ok = b >= 0 && b < batch && p >= 0;
    if (ok) {
      const int base = kv_indptr[b];
      const int np = kv_indptr[b + 1] - base;
      const int pi = p / ps;
      ok = pi < np && (int64_t)base + pi < num_indices;
      if (ok) {
        page = kv_indices[base + pi];
        ok = page >= 0 && page < num_pages;
      }
    }
    slot = p % ps;
  }
  return ok;
}

// Tokens whose K and V rows together are CT = 64 / TPW chunks of 16 bytes (e.g. 2 heads of
// 128 fp16 dims: CT = 64, TPW = 1): each wave moves TPW tokens at a time, lane l the chunk
// l % CT of token l / CT (its k|v, head and offset fixed for the whole kernel), U such groups
// per round.  A round's tokens are wave-uniform, so their page-table words are read with
// scalar loads, which are counted apart from the vector loads and stores: the lookup chain
// (batch index and position, then kv_indptr, then kv_indices) never waits for the rows in
// flight.  The rounds are software-pipelined: the next round's source rows are requested
// before this round's are stored, and the next round's lookups run while both are in flight.
// The row loads and stores are issued as instructions of their own with the waits written
// out (the compiler's counting would wait for every store before reusing its data registers);
// the cache rows are written non-temporally (nothing reads them back soon: the decode that
// does copies them past the caches itself).
typedef unsigned u4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u4v row_load(const char* p) {
  u4v v;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p));
  return v;
}

__device__ __forceinline__ void row_store_nt(char* p, u4v v) {
  // (s_nop: a VALU write of the data registers right after a store of more than 8 bytes needs
  // wait states the compiler does not count for an asm statement)
  asm volatile("global_store_dwordx4 %0, %1, off nt\n\ts_nop 1" ::"v"(p), "v"(v));
}

// Wait until at most N vector memory operations of this wave are outstanding (they complete
// in issue order).
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N));
}

template <bool SLOTS, int U, int TPW>
__global__ __launch_bounds__(256) void append_wave_kernel(
    const char* __restrict__ k, int64_t k_sn, int64_t k_sh, const char* __restrict__ v, int64_t v_sn,
    int64_t v_sh, const int32_t* __restrict__ bidx, const int32_t* __restrict__ pos, int32_t nnz,
    char* __restrict__ k_cache, char* __restrict__ v_cache, int64_t page_stride, int64_t num_pages,
    const int32_t* __restrict__ kv_indices, int64_t num_indices, const int32_t* __restrict__ kv_indptr,
    int32_t batch, int32_t hkv, int32_t row_bytes, int32_t ps, const int32_t* __restrict__ slots,
    int32_t* __restrict__ err) {
  constexpr int CT = 64 / TPW, NT = U * TPW;  // chunks per token, tokens per wave round
  const int lane = threadIdx.x & 63;
  const int t = lane / CT, c = lane % CT;
  const int cpr = row_bytes / 16;
  const int kv = c / (CT / 2), rc = c % (CT / 2), h = rc / cpr, cc = rc - h * cpr;
  const char* sbase = (kv ? v + h * v_sh : k + h * k_sh) + cc * 16;
  const int64_t ssn = kv ? v_sn : k_sn;
  char* dbase = (kv ? v_cache : k_cache) + (int64_t)h * row_bytes + cc * 16;
  const int64_t slot_bytes = (int64_t)hkv * row_bytes;
  const int64_t gw = (int64_t)blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * (blockDim.x >> 6);
  int64_t base = gw * NT;
  if (base >= nnz) return;

  // Source rows of the round starting at token b0.  Tokens past nnz read the last token's row
  // (in bounds, never stored), so every round issues exactly U loads.
  auto load = [&](int64_t b0, u4v (&val)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int64_t i = b0 + u * TPW + t;
      i = i < nnz ? i : nnz - 1;
      val[u] = row_load(sbase + i * ssn);
    }
  };
  // Destinations of the round's tokens (nullptr: past nnz, or metadata outside the sequence's
  // pages, counted once per token, k|v and head, as the element-wise kernel counts).  Every lookup index is clamped into its array (the launch
  // guarantees batch >= 1 and num_indices >= 1 without SLOTS), the checks are 32-bit and
  // combined with & rather than &&, so each stage's NT scalar loads issue together with no
  // branch between them.
  const int npg = num_pages < INT32_MAX ? (int)num_pages : INT32_MAX;
  const int nidx = num_indices < INT32_MAX ? (int)num_indices : INT32_MAX;
  auto resolve = [&](int64_t b0, char* (&dst)[U]) {
    const int64_t left = nnz - b0;  // tokens from b0 on (> 0)
    int pg[NT], sl[NT];
    bool in[NT], ok[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) in[j] = j < left;
    if constexpr (SLOTS) {
#pragma unroll
      for (int j = 0; j < NT; ++j) sl[j] = slots[__builtin_amdgcn_readfirstlane(in[j] ? (int)b0 + j : nnz - 1)];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        pg[j] = sl[j] / ps;
        ok[j] = in[j] & (sl[j] >= 0) & (pg[j] < npg);
        sl[j] -= pg[j] * ps;
      }
    } else {
      int bi[NT], po[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        // (the index is wave-uniform; readfirstlane says so, so the loads go through the
        // scalar cache)
        const int i = __builtin_amdgcn_readfirstlane(in[j] ? (int)b0 + j : nnz - 1);
        bi[j] = bidx[i];
        po[j] = pos[i];
      }
      int lo[NT], hi[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        ok[j] = in[j] & (bi[j] >= 0) & (bi[j] < batch) & (po[j] >= 0);
        bi[j] = ok[j] ? bi[j] : 0;
        po[j] = ok[j] ? po[j] : 0;
      }
#pragma unroll
      for (int j = 0; j < NT; ++j) lo[j] = kv_indptr[bi[j]], hi[j] = kv_indptr[bi[j] + 1];
      int at[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int pi = po[j] / ps;
        // lo + pi < hi <= INT32_MAX once pi < hi - lo (both counted from lo >= 0)
        ok[j] = ok[j] & (lo[j] >= 0) & (pi < hi[j] - lo[j]);
        ok[j] = ok[j] & (lo[j] + (ok[j] ? pi : 0) < nidx);
        at[j] = ok[j] ? lo[j] + pi : 0;
        sl[j] = po[j] - pi * ps;
      }
#pragma unroll
      for (int j = 0; j < NT; ++j) pg[j] = kv_indices[at[j]];
#pragma unroll
      for (int j = 0; j < NT; ++j) ok[j] = ok[j] & (pg[j] >= 0) & (pg[j] < npg);
    }
    int bad = 0;
#pragma unroll
    for (int j = 0; j < NT; ++j) bad += in[j] & !ok[j];
    if (bad && lane == 0 && err) atomicAdd(err, bad * 2 * hkv);  // one count per token, k|v and head
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int p = pg[u * TPW], q = sl[u * TPW];
      bool o = ok[u * TPW];
#pragma unroll
      for (int j = 1; j < TPW; ++j)
        if (t == j) p = pg[u * TPW + j], q = sl[u * TPW + j], o = ok[u * TPW + j];
      dst[u] = o ? dbase + p * page_stride + q * slot_bytes : nullptr;
    }
  };

  // One round: request the next round's rows into `next`; wait until only those U loads are
  // outstanding (this round's rows have arrived, and the previous round's stores, issued
  // between the two, have completed); store this round's rows from `cur`; look up the next
  // round's destinations.  Written out twice with the register sets swapped: the rows are
  // never copied between registers while their loads are in flight.
  u4v va[U], vb[U];
  char* dst[U];
  auto round = [&](u4v (&cur)[U], u4v (&next)[U]) {
    const int64_t nb = base + nw * NT;
    load(nb < nnz ? nb : base, next);  // (this round's rows again after the last round)
    wait_vm<U>();
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (dst[u]) row_store_nt(dst[u], cur[u]);
    if (nb >= nnz) return false;
    resolve(nb, dst);
    base = nb;
    return true;
  };
  load(base, va);
  resolve(base, dst);
  while (round(va, vb) && round(vb, va)) {
  }
  wait_vm<0>();  // the last loads (their rows unused) land before the wave ends
}

// One lane per VEC-byte chunk of a (token, k|v, head) row.  Index order, fastest first:
// chunk, head, k|v, token -- destination rows of consecutive heads are adjacent in a slot.
// With SLOTS, token i's destination is slots[i] = page * ps + slot (from the page-table gather),
// one lookup instead of the three dependent ones through batch_indices / positions, kv_indptr
// and kv_indices.
template <int VEC, bool SLOTS>
__global__ void append_kernel(const char* __restrict__ k, int64_t k_sn, int64_t k_sh,
                              const char* __restrict__ v, int64_t v_sn, int64_t v_sh,
                              const int32_t* __restrict__ bidx, const int32_t* __restrict__ pos,
                              int32_t nnz, char* __restrict__ k_cache, char* __restrict__ v_cache,
                              int64_t page_stride, int64_t num_pages,
                              const int32_t* __restrict__ kv_indices, int64_t num_indices,
                              const int32_t* __restrict__ kv_indptr, int32_t batch, int32_t hkv,
                              int32_t row_bytes, int32_t ps, const int32_t* __restrict__ slots,
                              int32_t* __restrict__ err) {
  using V = typename std::conditional<VEC == 16, uint4,
            typename std::conditional<VEC == 8, uint2,
            typename std::conditional<VEC == 4, uint32_t, uint16_t>::type>::type>::type;
  const int cpr = row_bytes / VEC;
  const int64_t total = (int64_t)nnz * 2 * hkv * cpr;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    int c = (int)(idx % cpr);
    int64_t r = idx / cpr;
    int h = (int)(r % hkv);
    r /= hkv;
    int kv = (int)(r & 1);
    int i = (int)(r >> 1);
    // The source chunk is read first, in parallel with the page-table lookups below (it does
    // not depend on them); the empty asm keeps the compiler from sinking the load into the
    // store's branch, which would chain it behind the lookups.
    const char* src = (kv ? v + i * v_sn + h * v_sh : k + i * k_sn + h * k_sh) + c * VEC;
    const V val = *reinterpret_cast<const V*>(src);
    asm volatile("" ::: "memory");
    int page, slot;
    const bool ok = resolve_dst<SLOTS>(i, bidx, pos, slots, kv_indices, num_indices, kv_indptr, batch,
                                       num_pages, ps, page, slot);
    if (!ok) {  // metadata that points outside the sequence's pages: skip, count it
      if (c == 0 && err) atomicAdd(err, 1);
      continue;
    }
    char* dst = (kv ? v_cache : k_cache) + page * page_stride +
                ((int64_t)slot * hkv + h) * row_bytes + c * VEC;
    *reinterpret_cast<V*>(dst) = val;
  }
}

}  // namespace

extern "C" int pkv_get_seq_lens(const int32_t* kv_indptr, const int32_t* kv_last_page_len,
                                int32_t batch, int32_t page_size, int32_t* seq_lens,
                                void* stream) {
  if (batch < 0 || page_size <= 0) return kBadArg;
  if (batch == 0) return kOk;
  int threads = 256, blocks = (batch + threads - 1) / threads;
  hipLaunchKernelGGL(seq_lens_kernel, dim3(blocks), dim3(threads), 0, (hipStream_t)stream,
                     kv_indptr, kv_last_page_len, batch, page_size, seq_lens);
  return (int)hipGetLastError();
}

extern "C" int pkv_get_batch_indices_positions(const int32_t* append_indptr,
                                               const int32_t* seq_lens, int32_t batch,
                                               int32_t nnz, int32_t* batch_indices,
                                               int32_t* positions, void* stream) {
  if (batch <= 0 || nnz < 0) return nnz == 0 ? kOk : kBadArg;
  if (nnz == 0) return kOk;
  int threads = 256, blocks = (nnz + threads - 1) / threads;
  hipLaunchKernelGGL(batch_positions_kernel, dim3(blocks), dim3(threads), 0, (hipStream_t)stream,
                     append_indptr, seq_lens, batch, nnz, batch_indices, positions);
  return (int)hipGetLastError();
}

namespace {

// Compute units of the stream's device (looked up once per device).
int num_cus(hipStream_t s) {
  static int cached[64] = {};
  hipDevice_t dev = 0;
  if ((s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev)) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

int launch_append(const void* append_key, int64_t k_stride_n, int64_t k_stride_h, const void* append_value,
                  int64_t v_stride_n, int64_t v_stride_h, const int32_t* batch_indices, const int32_t* positions,
                  const int32_t* slots, int32_t nnz, void* k_cache, void* v_cache, int64_t page_stride,
                  int64_t num_pages, const int32_t* kv_indices, int64_t num_indices, const int32_t* kv_indptr,
                  int32_t batch, int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int32_t dtype,
                  int32_t* err_count, void* stream) {
  int es = dtype == kF32 ? 4 : (dtype == kF16 || dtype == kBF16) ? 2 : 0;
  if (!es) return kBadDType;
  if (nnz < 0 || num_kv_heads <= 0 || head_dim <= 0 || page_size <= 0 || batch < 0) return kBadArg;
  if (nnz == 0) return kOk;
  // Strides arrive in elements; the kernel works in bytes.
  int64_t ksn = k_stride_n * es, ksh = k_stride_h * es, vsn = v_stride_n * es, vsh = v_stride_h * es;
  int64_t pstride = page_stride * es;
  int row_bytes = head_dim * es;
  auto aligned = [&](int vec) {
    uintptr_t m = (uintptr_t)append_key | (uintptr_t)append_value | (uintptr_t)k_cache |
                  (uintptr_t)v_cache;
    int64_t s = ksn | ksh | vsn | vsh | pstride | row_bytes;
    return (m % vec) == 0 && (s % vec) == 0;
  };
  int vec = aligned(16) ? 16 : aligned(8) ? 8 : aligned(4) ? 4 : 2;
  if (vec < es) return kBadAlign;
  int64_t total = (int64_t)nnz * 2 * num_kv_heads * (row_bytes / vec);
  int threads = 256;
  int64_t want = (total + threads - 1) / threads;
  int blocks = (int)(want < 65536 ? want : 65536);
  hipStream_t s = (hipStream_t)stream;
  const int ct = vec == 16 ? 2 * num_kv_heads * (row_bytes / 16) : 0;
  if ((ct == 64 || ct == 32 || ct == 16 || ct == 8) && (slots || (batch >= 1 && num_indices >= 1))) {
    // Measured at 65536 tokens of Qwen2.5-3B shape (CT = 64): U = 2 with at most 16
    // workgroups of 4 waves per CU (22.0 us against 22.7 for U = 4 and 22.9 for U = 1; 4 and 8
    // workgroups per CU were 0.9 and 0.3 us slower).
    constexpr int U = 2;
    const int tpw = 64 / ct;
    const int64_t per_wave = (int64_t)tpw * U, waves = (nnz + per_wave - 1) / per_wave;
    int64_t nb = (waves + 3) / 4;  // 4 waves per block
    const int64_t cap = 16 * (int64_t)num_cus(s);
    nb = nb < cap ? nb : cap;
#define PKV_APPEND_WAVE(SL, T)                                                                        \
  hipLaunchKernelGGL((append_wave_kernel<SL, U, T>), dim3((unsigned)nb), dim3(256), 0, s,             \
                     (const char*)append_key, ksn, ksh, (const char*)append_value, vsn, vsh,          \
                     batch_indices, positions, nnz, (char*)k_cache, (char*)v_cache, pstride,          \
                     num_pages, kv_indices, num_indices, kv_indptr, batch, num_kv_heads, row_bytes,   \
                     page_size, slots, err_count)
    switch (tpw * 2 + (slots != nullptr)) {
      case 2: PKV_APPEND_WAVE(false, 1); break;
      case 3: PKV_APPEND_WAVE(true, 1); break;
      case 4: PKV_APPEND_WAVE(false, 2); break;
      case 5: PKV_APPEND_WAVE(true, 2); break;
      case 8: PKV_APPEND_WAVE(false, 4); break;
      case 9: PKV_APPEND_WAVE(true, 4); break;
      case 16: PKV_APPEND_WAVE(false, 8); break;
      default: PKV_APPEND_WAVE(true, 8); break;
    }
#undef PKV_APPEND_WAVE
    return (int)hipGetLastError();
  }
#define PKV_APPEND(VB, SL)                                                                      \
  hipLaunchKernelGGL((append_kernel<VB, SL>), dim3(blocks), dim3(threads), 0, s,                \
                     (const char*)append_key, ksn, ksh, (const char*)append_value, vsn, vsh,    \
                     batch_indices, positions, nnz, (char*)k_cache, (char*)v_cache, pstride,    \
                     num_pages, kv_indices, num_indices, kv_indptr, batch, num_kv_heads,        \
                     row_bytes, page_size, slots, err_count)
  if (slots) {
    switch (vec) {
      case 16: PKV_APPEND(16, true); break;
      case 8: PKV_APPEND(8, true); break;
      case 4: PKV_APPEND(4, true); break;
      default: PKV_APPEND(2, true); break;
    }
  } else {
    switch (vec) {
      case 16: PKV_APPEND(16, false); break;
      case 8: PKV_APPEND(8, false); break;
      case 4: PKV_APPEND(4, false); break;
      default: PKV_APPEND(2, false); break;
    }
  }
#undef PKV_APPEND
  return (int)hipGetLastError();
}

}  // namespace

extern "C" int pkv_append_paged_kv_cache(
    const void* append_key, int64_t k_stride_n, int64_t k_stride_h, const void* append_value,
    int64_t v_stride_n, int64_t v_stride_h, const int32_t* batch_indices, const int32_t* positions,
    int32_t nnz, void* k_cache, void* v_cache, int64_t page_stride, int64_t num_pages,
    const int32_t* kv_indices, int64_t num_indices, const int32_t* kv_indptr, int32_t batch,
    int32_t num_kv_heads,
    int32_t head_dim, int32_t page_size, int32_t dtype, int32_t* err_count, void* stream) {
  if (nnz > 0 && (!batch_indices || !positions)) return kBadArg;
  return launch_append(append_key, k_stride_n, k_stride_h, append_value, v_stride_n, v_stride_h, batch_indices,
                       positions, nullptr, nnz, k_cache, v_cache, page_stride, num_pages, kv_indices, num_indices,
                       kv_indptr, batch, num_kv_heads, head_dim, page_size, dtype, err_count, stream);
}

extern "C" int pkv_append_paged_kv_cache_slots(
    const void* append_key, int64_t k_stride_n, int64_t k_stride_h, const void* append_value,
    int64_t v_stride_n, int64_t v_stride_h, const int32_t* slots, int32_t nnz, void* k_cache, void* v_cache,
    int64_t page_stride, int64_t num_pages, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
    int32_t dtype, int32_t* err_count, void* stream) {
  if (nnz > 0 && !slots) return kBadArg;
  return launch_append(append_key, k_stride_n, k_stride_h, append_value, v_stride_n, v_stride_h, nullptr, nullptr,
                       slots, nnz, k_cache, v_cache, page_stride, num_pages, nullptr, 0, nullptr, 0, num_kv_heads,
                       head_dim, page_size, dtype, err_count, stream);
}
