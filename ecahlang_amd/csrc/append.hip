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

// Tokens whose K and V rows together are CT <= 64 chunks of 16 bytes (CT dividing 64: e.g.
// 2 heads of 128 fp16 dims = 64 chunks): each wave takes 64 / CT tokens at a time, lane l the
// chunk l % CT of token l / CT (its k|v, head and offset fixed for the whole kernel), and U
// such groups per round, so a wave has U tokens' source loads and page-table lookups in flight
// at once.  The lanes of a token read the same metadata words: one request per token.  The
// cache rows are written with non-temporal stores (nothing reads them back soon: the decode
// that does copies them past the caches itself).  Measured at 65536 tokens of Qwen2.5-3B
// shape: U = 2 with 8 workgroups of 4 waves per CU was the fastest of U = 1 .. 8 and 4 .. 64
// workgroups per CU.
typedef unsigned u4v __attribute__((ext_vector_type(4)));

template <bool SLOTS, int U>
__global__ __launch_bounds__(256) void append_tok_kernel(
    const char* __restrict__ k, int64_t k_sn, int64_t k_sh, const char* __restrict__ v, int64_t v_sn,
    int64_t v_sh, const int32_t* __restrict__ bidx, const int32_t* __restrict__ pos, int32_t nnz,
    char* __restrict__ k_cache, char* __restrict__ v_cache, int64_t page_stride, int64_t num_pages,
    const int32_t* __restrict__ kv_indices, int64_t num_indices, const int32_t* __restrict__ kv_indptr,
    int32_t batch, int32_t hkv, int32_t row_bytes, int32_t ps, const int32_t* __restrict__ slots,
    int32_t* __restrict__ err) {
  const int lane = threadIdx.x & 63;
  const int cpr = row_bytes / 16, CT = 2 * hkv * cpr, tpw = 64 / CT;
  const int t = lane / CT, c = lane - t * CT;          // token of the group, chunk of the token
  const int kv = c / (hkv * cpr), rc = c - kv * hkv * cpr, h = rc / cpr, cc = rc - h * cpr;
  const char* sbase = (kv ? v + h * v_sh : k + h * k_sh) + cc * 16;
  const int64_t ssn = kv ? v_sn : k_sn;
  char* dbase = (kv ? v_cache : k_cache) + (int64_t)h * row_bytes + cc * 16;
  const int64_t per = (int64_t)tpw * U;                  // tokens per wave round
  const int64_t gw = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nw = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t base = gw * per; base < nnz; base += nw * per) {
    uint4 val[U];
    int64_t ii[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ii[u] = base + (int64_t)u * tpw + t;
      val[u] = ii[u] < nnz ? *reinterpret_cast<const uint4*>(sbase + ii[u] * ssn) : make_uint4(0, 0, 0, 0);
    }
    asm volatile("" ::: "memory");  // every source load is issued before the lookups
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (ii[u] >= nnz) continue;
      int page, slot;
      if (!resolve_dst<SLOTS>(ii[u], bidx, pos, slots, kv_indices, num_indices, kv_indptr, batch, num_pages,
                              ps, page, slot)) {
        if (cc == 0 && err) atomicAdd(err, 1);  // one count per token, k|v and head
        continue;
      }
      const u4v x = {val[u].x, val[u].y, val[u].z, val[u].w};
      __builtin_nontemporal_store(x, reinterpret_cast<u4v*>(dbase + page * page_stride + (int64_t)slot * hkv * row_bytes));
    }
  }
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
  if (ct > 0 && ct <= 64 && 64 % ct == 0) {
    constexpr int U = 2;
    const int64_t per_wave = (int64_t)(64 / ct) * U, waves = (nnz + per_wave - 1) / per_wave;
    int64_t nb = (waves + 3) / 4;  // 4 waves per block
    const int64_t cap = 8 * (int64_t)num_cus(s);
    nb = nb < cap ? nb : cap;
    if (slots)
      hipLaunchKernelGGL((append_tok_kernel<true, U>), dim3((unsigned)nb), dim3(256), 0, s, (const char*)append_key,
                         ksn, ksh, (const char*)append_value, vsn, vsh, batch_indices, positions, nnz,
                         (char*)k_cache, (char*)v_cache, pstride, num_pages, kv_indices, num_indices, kv_indptr,
                         batch, num_kv_heads, row_bytes, page_size, slots, err_count);
    else
      hipLaunchKernelGGL((append_tok_kernel<false, U>), dim3((unsigned)nb), dim3(256), 0, s, (const char*)append_key,
                         ksn, ksh, (const char*)append_value, vsn, vsh, batch_indices, positions, nnz,
                         (char*)k_cache, (char*)v_cache, pstride, num_pages, kv_indices, num_indices, kv_indptr,
                         batch, num_kv_heads, row_bytes, page_size, slots, err_count);
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
