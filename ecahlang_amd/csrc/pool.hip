// Device-side page pool of the KV cache manager (ecahlang/manager.py:56, 99-120, 187-212).
//
// The reference keeps the free pages in a Python list used as a stack (pop() from the end,
// extend() in page order on free) and each sequence's pages in a Python list.  Here both
// live in device memory:
//   stack[max_blocks]         free page ids; the live part is stack[0 .. n_free)
//   table[rows][stride]       page list of each sequence slot (one row per slot, plus a row
//                             for the CUDA-graph padding pages)
// The host keeps only counts (n_free, pages per sequence), so it can raise the reference's
// exceptions before anything is touched and compute every stack position itself; the page
// ids never leave the device.  Operations are queued on the host and applied here in one
// launch, in their original order.
//
//   pkv_pool_apply   <- allocate / append_tokens / free / init_cuda_graph_buffers, and the
//                       page-sharing extension (a sequence's row starts with a copy of the
//                       pages it shares; a shared page written to is replaced by a private
//                       copy; no counterpart in the reference)
//   pkv_pool_copy_pages, pkv_shared_prefix_pages <- the same extension: the K/V data of those
//                       copies, and the decode plan's shared-page hint from the page lists
//   pkv_pool_gather  <- get_append_metadata / fill_cuda_graph_metadata (the page walk that
//                       builds kv_indices, manager.py:124-133, 231-246)
//   pkv_pool_step    <- one decode step of a fixed batch, all on the device: append_tokens(b, n)
//                       for every row (manager.py:187-205) then fill_cuda_graph_metadata for
//                       the bucket (manager.py:228-253), with the per-slot page counts and
//                       last-page lengths kept on the device, so the step can be replayed from
//                       a graph with no host work in between
//   pkv_pool_steps_begin <- the hand-over of a batch to those steps (begin_device_steps, an
//                       extension): the device's page counts, last-page lengths and free count
//                       set from the bucket's metadata in one launch
#include "common.h"
#include "../../include/pagedkv.h"

using namespace pkv;

namespace {

// One workgroup applies the operations in order (a pop may read stack slots that an earlier
// push of the same batch wrote).  Operation i is ops[5i .. 5i+4] = {kind, row, pos, col, n}:
//   kind 0, pop:  table[row][col + k] = stack[pos - 1 - k]   (k < n: the order of pop())
//   kind 1, push: stack[pos + k] = table[row][col + k]       (the order of extend())
//   kind 2, copy: table[row][col + k] = table[pos][k]         (pos = the sharer's source row)
//   kind 3, copy on write: the page table[row][col] is replaced by stack[pos - 1] (one pop),
//           and pairs[2n], pairs[2n + 1] = (old page, new page) for the data copy
// Operations that fall outside the stack, the table or the pairs are skipped and counted in
// *err.  The operations are staged in LDS a chunk at a time, so each one costs its own loads,
// its stores and a barrier.
constexpr int kApplyThreads = 256, kApplyChunk = 1024;
__global__ __launch_bounds__(kApplyThreads) void pool_apply_kernel(
    int32_t* stack, int32_t stack_size, int32_t* table, int64_t stride, int32_t rows, const int32_t* ops,
    int32_t n_ops, int32_t* pairs, int32_t pairs_cap, int32_t* err) {
  __shared__ int s_op[kApplyChunk * 5];
  const int tid = threadIdx.x;
  for (int base = 0; base < n_ops; base += kApplyChunk) {
    const int cnt = n_ops - base < kApplyChunk ? n_ops - base : kApplyChunk;
    __syncthreads();  // (the previous chunk is done with s_op)
    for (int t = tid; t < 5 * cnt; t += kApplyThreads) s_op[t] = ops[5 * (int64_t)base + t];
    __syncthreads();
    for (int i = 0; i < cnt; ++i) {
      const int* o = s_op + 5 * i;
      const int kind = o[0], row = o[1], pos = o[2], col = o[3], n = o[4];
      bool ok = kind >= 0 && kind <= 3 && row >= 0 && row < rows && col >= 0 && n >= 0;
      if (kind == 0) ok = ok && (int64_t)col + n <= stride && pos - n >= 0 && pos <= stack_size;
      else if (kind == 1) ok = ok && (int64_t)col + n <= stride && pos >= 0 && pos + n <= stack_size;
      else if (kind == 2) ok = ok && (int64_t)col + n <= stride && pos >= 0 && pos < rows && pos != row;
      else ok = ok && col < stride && pos >= 1 && pos <= stack_size && pairs && n < pairs_cap;
      if (!ok) {
        if (tid == 0 && err) atomicAdd(err, 1);
        // a rejected copy on write still owns its pair: mark it empty, so the data copy skips it
        // rather than replaying an earlier call's pair onto a page that may have changed hands
        if (tid == 0 && kind == 3 && pairs && n >= 0 && n < pairs_cap) pairs[2 * n] = pairs[2 * n + 1] = -1;
      } else if (kind == 3) {
        if (tid == 0) {
          int32_t* cell = table + (int64_t)row * stride + col;
          pairs[2 * n] = *cell;
          pairs[2 * n + 1] = stack[pos - 1];
          *cell = stack[pos - 1];
        }
      } else {
        int32_t* trow = table + (int64_t)row * stride + col;
        const int32_t* src = table + (int64_t)pos * stride;  // (kind 2 only)
        for (int k = tid; k < n; k += kApplyThreads) {
          if (kind == 0) trow[k] = stack[pos - 1 - k];
          else if (kind == 1) stack[pos + k] = trow[k];
          else trow[k] = src[k];
        }
      }
      __syncthreads();  // this operation's writes are visible to the next one
    }
  }
}

// The data of copy-on-write pairs: for pair p and layer l (blockIdx.y, blockIdx.z), the page
// pairs[2p] of the layer is copied to the page pairs[2p + 1], 16 bytes per thread (the page is
// whole 16-byte runs: 2 x page_size x Hkv x head_dim elements).  Pairs naming a page outside
// the pool are skipped and counted in *err; a (-1, -1) pair (a rejected copy on write, counted
// when it was rejected) is skipped silently.
__global__ void pool_copy_pages_kernel(char* cache, int64_t layer_stride, int64_t page_bytes, const int32_t* pairs,
                                       int64_t num_pages, int32_t* err) {
  const int p = blockIdx.y, l = blockIdx.z;
  const int src = pairs[2 * p], dst = pairs[2 * p + 1];
  if (src == -1 && dst == -1) return;  // a rejected copy on write (already counted)
  if (src < 0 || src >= num_pages || dst < 0 || dst >= num_pages) {
    if (err && l == 0 && blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(err, 1);
    return;
  }
  const char* from = cache + l * layer_stride + (int64_t)src * page_bytes;
  char* to = cache + l * layer_stride + (int64_t)dst * page_bytes;
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < page_bytes / 16;
       c += (int64_t)gridDim.x * blockDim.x)
    reinterpret_cast<uint4*>(to)[c] = reinterpret_cast<const uint4*>(from)[c];
}

// out[b] = how many leading page ids rows b and b - 1 of the page table have in common (the
// decode plan's kv_shared_pages hint), out[0] = 0; one wave per row, 64 ids compared at a time.
__global__ void shared_prefix_kernel(const int32_t* __restrict__ indptr, const int32_t* __restrict__ indices,
                                     int64_t num_indices, int32_t batch, int32_t* __restrict__ out) {
  const int b = (int)(((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6), lane = threadIdx.x & 63;
  if (b >= batch) return;
  int k = 0;
  if (b > 0) {
    const int64_t x0 = indptr[b], x1 = indptr[b + 1], y0 = indptr[b - 1];
    int64_t n = x1 - x0 < x0 - y0 ? x1 - x0 : x0 - y0;
    if (x1 > num_indices || x0 < 0 || y0 < 0) n = 0;
    for (int64_t i = 0; i < n; i += 64) {
      const bool diff = i + lane < n && indices[x0 + i + lane] != indices[y0 + i + lane];
      const uint64_t bal = __ballot(diff);
      if (bal) {
        k = (int)(i + __builtin_ctzll(bal));
        break;
      }
      k = (int)(i + 64 < n ? i + 64 : n);
    }
  }
  if (lane == 0) out[b] = k;
}

// indices[indptr[b] + k] = table[desc[4b]][desc[4b+1] + k] for k < desc[4b+2]; one thread per
// output entry finds its sequence by binary search over indptr.
// With `slots`, also each row's append slot: slots[b] = page * ps + positions[b] % ps for the
// page holding position positions[b] of row b, or -1 when that position is outside the row's
// pages (rows with no pages included: a thread per row writes the -1s, the thread gathering
// the page writes the rest).
__global__ void pool_gather_kernel(const int32_t* table, int64_t stride, int32_t rows, const int32_t* desc,
                                   const int32_t* indptr, int32_t batch, int32_t* indices,
                                   int64_t num_indices, const int32_t* positions, int32_t ps,
                                   int32_t* slots, int32_t* err) {
  const int64_t total = indptr[batch] < num_indices ? indptr[batch] : num_indices;
  const int64_t span = total > batch || !slots ? total : batch;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < span;
       t += (int64_t)gridDim.x * blockDim.x) {
    if (slots && t < batch) {
      const int p = positions[t];
      const int64_t np = (int64_t)indptr[t + 1] - indptr[t];
      if (p < 0 || p / ps >= np || (int64_t)indptr[t] + p / ps >= total) slots[t] = -1;
    }
    if (t >= total) continue;
    int lo = 0, hi = batch;  // largest b with indptr[b] <= t
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (indptr[mid] <= t) lo = mid; else hi = mid;
    }
    const int row = desc[4 * lo], col = desc[4 * lo + 1], n = desc[4 * lo + 2];
    const int64_t k = t - indptr[lo];
    int page = -1;
    if (row >= 0 && row < rows && k < n && col + k < stride) {
      page = table[(int64_t)row * stride + col + k];
    } else if (err) {
      atomicAdd(err, 1);
    }
    indices[t] = page;
    if (slots) {
      const int p = positions[lo];
      if (p >= 0 && p / ps == k) slots[lo] = page < 0 ? -1 : page * ps + p % ps;
    }
  }
}

// One workgroup: appends n tokens to every real row of the bucket, in row order (the order of
// the reference's append_tokens loop), popping the pages that fill from the top of the stack
// exactly as append_tokens would (row i's pops come after rows 0 .. i-1's), then writes the
// bucket's metadata: kv_indptr, kv_last_page_len, each row's newest-token position, and the
// gather descriptor pool_gather_kernel reads.  Padding rows (rows[i] < 0) take one padding
// page each, in order (last_page_len 1, position 0).  A row whose pops the stack (or its table row)
// cannot hold is left unchanged, as are all rows after it, and *err is bumped: the host checks
// the pool before it enqueues a step, so this is only a guard.
constexpr int kStepThreads = 1024;
__global__ __launch_bounds__(kStepThreads) void pool_step_kernel(
    int32_t* stack, int32_t* n_free, int32_t* table, int64_t stride, int32_t rows_total,
    const int32_t* rows, int32_t batch, int32_t n_tokens, int32_t bs, int32_t* npages, int32_t* plen,
    int32_t padding_row, int32_t* desc, int32_t* indptr, int32_t* last, int32_t* positions, int32_t* err) {
  __shared__ int s_wsum[kStepThreads / 64];
  __shared__ int s_free, s_fail, s_taken;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (tid == 0) {
    s_free = *n_free;
    s_fail = batch;
    s_taken = 0;
  }
  __syncthreads();
  const int nf = s_free;
  auto scan = [&](int v, int& carry) -> int {  // block-wide exclusive scan (all threads call it)
    int x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(x, off, 64);
      x += lane >= off ? y : 0;
    }
    if (lane == 63) s_wsum[wv] = x;
    __syncthreads();
    int o = 0, blk = 0;
#pragma unroll
    for (int k = 0; k < kStepThreads / 64; ++k) {
      o += k < wv ? s_wsum[k] : 0;
      blk += s_wsum[k];
    }
    const int ex = carry + o + x - v;
    carry += blk;
    __syncthreads();
    return ex;
  };
  auto real_row = [&](int i) -> int {
    const int row = i < batch ? rows[i] : -1;
    return row >= 0 && row < rows_total ? row : -1;
  };
  // ---- pops: row i needs (plen + n) / bs pages, taken from the top after rows 0 .. i-1's
  int before = 0;
  for (int base = 0; base < batch; base += kStepThreads) {
    const int i = base + tid;
    const int row = real_row(i);
    int need = 0, np = 0, pl = 0;
    if (row >= 0) {
      np = npages[row];
      pl = plen[row];
      need = (pl + n_tokens) / bs;
    }
    const int off = scan(need, before);
    if (row >= 0 && (off + need > nf || (int64_t)np + need > stride)) atomicMin(&s_fail, i);
    __syncthreads();
    if (row >= 0 && i < s_fail) {
      int32_t* trow = table + (int64_t)row * stride + np;
      for (int k = 0; k < need; ++k) trow[k] = stack[nf - 1 - off - k];
      npages[row] = np + need;
      plen[row] = (pl + n_tokens) % bs;
      if (need) atomicAdd(&s_taken, need);
    }
    __syncthreads();
    if (s_fail < batch) break;  // (uniform)
  }
  if (tid == 0) {
    *n_free = nf - s_taken;
    if (s_fail < batch && err) atomicAdd(err, 1);
  }
  // ---- the bucket's metadata, from the new counts (padding entry j takes padding page j)
  int carry = 0, pads = 0;
  for (int base = 0; base < batch; base += kStepThreads) {
    const int i = base + tid;
    const int row = real_row(i);
    int np = 1, pl = 1, pos = 0;
    if (row >= 0) {
      np = npages[row];
      pl = plen[row];
      pos = (np - 1) * bs + pl - 1;
    }
    const int start = scan(i < batch ? np : 0, carry);
    const int pad = scan(i < batch && row < 0 ? 1 : 0, pads);
    if (i < batch) {
      indptr[i] = start;
      last[i] = pl;
      positions[i] = pos;
      desc[4 * i] = row >= 0 ? row : padding_row;
      desc[4 * i + 1] = row >= 0 ? 0 : pad;
      desc[4 * i + 2] = np;
      desc[4 * i + 3] = 0;
    }
  }
  if (tid == 0) indptr[batch] = carry;
}

// The hand-over of a batch to the device steps, from the bucket's metadata as the gather wrote
// it: rows[i] = desc[4i] for the real entries (i < real) and -1 for the padding ones; each real
// entry's row takes npages[row] = desc[4i + 2] and plen[row] = last[i] (rows outside
// [0, rows_total) are skipped and counted in *err); *n_free_out = n_free.
__global__ void pool_steps_begin_kernel(const int32_t* desc, const int32_t* last, int32_t batch, int32_t real,
                                        int32_t n_free, int32_t* rows, int32_t* npages, int32_t* plen,
                                        int32_t rows_total, int32_t* n_free_out, int32_t* err) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i == 0) *n_free_out = n_free;
  if (i >= batch) return;
  if (i >= real) {
    rows[i] = -1;
    return;
  }
  const int row = desc[4 * i];
  rows[i] = row;
  if (row >= 0 && row < rows_total) {
    npages[row] = desc[4 * i + 2];
    plen[row] = last[i];
  } else if (err) {
    atomicAdd(err, 1);
  }
}

}  // namespace

extern "C" int pkv_pool_apply(int32_t* stack, int32_t stack_size, int32_t* table, int64_t stride,
                              int32_t rows, const int32_t* ops, int32_t n_ops, int32_t* pairs,
                              int32_t pairs_cap, int32_t* err, void* stream) {
  if (n_ops < 0 || stack_size < 0 || stride <= 0 || rows <= 0 || pairs_cap < 0) return kBadArg;
  if (n_ops == 0) return kOk;
  hipLaunchKernelGGL(pool_apply_kernel, dim3(1), dim3(kApplyThreads), 0, (hipStream_t)stream, stack, stack_size,
                     table, stride, rows, ops, n_ops, pairs, pairs_cap, err);
  return (int)hipGetLastError();
}

extern "C" int pkv_pool_copy_pages(void* cache, int64_t layer_stride, int32_t layers, int64_t page_bytes,
                                   const int32_t* pairs, int32_t n_pairs, int64_t num_pages, int32_t* err,
                                   void* stream) {
  if (layers < 0 || n_pairs < 0 || page_bytes <= 0 || page_bytes % 16 || layer_stride % 16 || num_pages < 0 ||
      (uintptr_t)cache % 16)
    return kBadArg;
  if (layers == 0 || n_pairs == 0) return kOk;
  if (n_pairs > 65535 || layers > 65535) return kBadArg;
  const int64_t chunks = page_bytes / 16;
  const unsigned bx = (unsigned)((chunks + 255) / 256 < 64 ? (chunks + 255) / 256 : 64);
  hipLaunchKernelGGL(pool_copy_pages_kernel, dim3(bx, (unsigned)n_pairs, (unsigned)layers), dim3(256), 0,
                     (hipStream_t)stream, (char*)cache, layer_stride, page_bytes, pairs, num_pages, err);
  return (int)hipGetLastError();
}

extern "C" int pkv_shared_prefix_pages(const int32_t* kv_indptr, const int32_t* kv_indices, int64_t num_indices,
                                       int32_t batch, int32_t* out, void* stream) {
  if (batch < 0 || num_indices < 0) return kBadArg;
  if (batch == 0) return kOk;
  const unsigned blocks = (unsigned)((batch + 3) / 4);  // 4 waves per block, one per row
  hipLaunchKernelGGL(shared_prefix_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, kv_indptr, kv_indices,
                     num_indices, batch, out);
  return (int)hipGetLastError();
}

extern "C" int pkv_pool_gather(const int32_t* table, int64_t stride, int32_t rows, const int32_t* desc,
                               const int32_t* indptr, int32_t batch, int32_t* indices,
                               int64_t num_indices, int64_t max_total, const int32_t* positions,
                               int32_t page_size, int32_t* slots, int32_t* err, void* stream) {
  if (batch < 0 || stride <= 0 || rows <= 0 || num_indices < 0 || max_total < 0) return kBadArg;
  if (slots && (!positions || page_size <= 0)) return kBadArg;
  if (batch == 0 || (max_total == 0 && !slots)) return kOk;
  int64_t n = max_total < num_indices ? max_total : num_indices;
  if (slots && n < batch) n = batch;
  const int threads = 256;
  int64_t blocks = (n + threads - 1) / threads;
  blocks = blocks < 1024 ? (blocks > 0 ? blocks : 1) : 1024;
  hipLaunchKernelGGL(pool_gather_kernel, dim3((unsigned)blocks), dim3(threads), 0, (hipStream_t)stream,
                     table, stride, rows, desc, indptr, batch, indices, num_indices, positions, page_size,
                     slots, err);
  return (int)hipGetLastError();
}

extern "C" int pkv_pool_step(int32_t* stack, int32_t* n_free, int32_t* table, int64_t stride,
                             int32_t rows_total, const int32_t* rows, int32_t batch, int32_t n_tokens,
                             int32_t page_size, int32_t* npages, int32_t* last_len, int32_t padding_row,
                             int32_t* desc, int32_t* kv_indptr, int32_t* kv_last_page_len,
                             int32_t* positions, int32_t* kv_indices, int64_t num_indices,
                             int64_t max_total, int32_t* slots, int32_t* err, void* stream) {
  if (batch <= 0 || n_tokens < 0 || page_size <= 0 || stride <= 0 || rows_total <= 0 || num_indices < 0 ||
      max_total < 0 || padding_row < 0 || padding_row >= rows_total)
    return kBadArg;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(pool_step_kernel, dim3(1), dim3(kStepThreads), 0, s, stack, n_free, table, stride,
                     rows_total, rows, batch, n_tokens, page_size, npages, last_len, padding_row, desc,
                     kv_indptr, kv_last_page_len, positions, err);
  // kv_indices and the append slots, as fill_cuda_graph_metadata's gather
  int64_t n = max_total < num_indices ? max_total : num_indices;
  if (n < batch) n = batch;
  const int threads = 256;
  int64_t blocks = (n + threads - 1) / threads;
  blocks = blocks < 1024 ? (blocks > 0 ? blocks : 1) : 1024;
  hipLaunchKernelGGL(pool_gather_kernel, dim3((unsigned)blocks), dim3(threads), 0, s, table, stride,
                     rows_total, desc, kv_indptr, batch, kv_indices, num_indices, positions, page_size,
                     slots, err);
  return (int)hipGetLastError();
}

extern "C" int pkv_pool_steps_begin(const int32_t* desc, const int32_t* last_len, int32_t batch, int32_t real,
                                    int32_t n_free, int32_t* rows, int32_t* npages, int32_t* plen,
                                    int32_t rows_total, int32_t* n_free_out, int32_t* err, void* stream) {
  if (batch < 0 || real < 0 || real > batch || n_free < 0 || rows_total <= 0 || !n_free_out ||
      (batch > 0 && (!desc || !last_len || !rows || !npages || !plen)))
    return kBadArg;
  const unsigned blocks = (unsigned)(batch > 0 ? (batch + 255) / 256 : 1);
  hipLaunchKernelGGL(pool_steps_begin_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, desc, last_len,
                     batch, real, n_free, rows, npages, plen, rows_total, n_free_out, err);
  return (int)hipGetLastError();
}
