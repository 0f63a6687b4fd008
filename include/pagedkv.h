/*
 * pagedkv.h -- C ABI of libpagedkv.so, the MI355X (gfx950) paged-KV hot path.
 *
 * Every pointer is a device pointer owned by the caller (PyTorch tensors' data_ptr()),
 * every stride is in ELEMENTS, `stream` is a hipStream_t, and no entry point allocates,
 * frees or synchronises: each call only enqueues kernels on `stream`, so all of them can be
 * captured into a hipGraph.  Return value: 0 on success, a positive hipError_t from the
 * launch, or a negative pkv argument code (see PKV_E_* below).
 *
 * dtype codes: 0 = float16, 1 = bfloat16, 2 = float32.
 *
 * Cache addressing (NHD): element (page, slot, head, dim) of K is
 *   k_cache[page * page_stride + (slot * num_kv_heads + head) * head_dim + dim]
 * and likewise for V.  For the reference's single-tensor layer cache
 * kv_cache[layer] = [pages, 2, page_size, Hkv, D] (ecahlang/manager.py:51-54) pass
 * k_cache = base, v_cache = base + page_size*Hkv*D, page_stride = 2*page_size*Hkv*D.
 *
 * Each entry point replaces one FlashInfer 0.6.5 call made by the reference (FlashInfer is
 * an external dependency of ecahLang, pinned at uv.lock:324-325; the call sites cited are
 * the reference's).
 */
#ifndef PAGEDKV_H
#define PAGEDKV_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PKV_E_DTYPE (-1)
#define PKV_E_HEAD_DIM (-2)
#define PKV_E_GROUP (-3)
#define PKV_E_ALIGN (-4)
#define PKV_E_ARG (-5)
#define PKV_E_WORKSPACE (-6)
#define PKV_E_PAGE_SIZE (-7)

/* flashinfer.get_seq_lens(kv_indptr, kv_last_page_len, page_size)
 * (ecahlang/manager.py:143, :170):
 * seq_lens[b] = max(kv_indptr[b+1] - kv_indptr[b] - 1, 0) * page_size + kv_last_page_len[b]. */
int pkv_get_seq_lens(const int32_t* kv_indptr, const int32_t* kv_last_page_len, int32_t batch,
                     int32_t page_size, int32_t* seq_lens, void* stream);

/* flashinfer.get_batch_indices_positions(append_indptr, seq_lens, nnz)
 * (ecahlang/manager.py:144-146, :171-173): for appended token i of request b,
 * batch_indices[i] = b and
 * positions[i] = seq_lens[b] - (append_indptr[b+1] - append_indptr[b]) + (i - append_indptr[b]). */
int pkv_get_batch_indices_positions(const int32_t* append_indptr, const int32_t* seq_lens,
                                    int32_t batch, int32_t nnz, int32_t* batch_indices,
                                    int32_t* positions, void* stream);

/* flashinfer.page.append_paged_kv_cache(append_key, append_value, batch_indices, positions,
 * paged_kv_cache, kv_indices, kv_indptr, kv_last_page_len, kv_layout="NHD")
 * (ecahlang/manager.py:155-165, :175-185, :271-280).  append_key/value are [nnz, Hkv, D]
 * with strides (stride_n, stride_h) and a unit inner stride.  Token i goes to page
 * kv_indices[kv_indptr[b] + positions[i] / page_size], slot positions[i] % page_size, where
 * b = batch_indices[i].  A token whose metadata points outside its sequence's pages, past
 * num_indices entries of kv_indices, or outside the num_pages-page pool is skipped and
 * counted in *err_count (may be NULL) instead of written. */
int pkv_append_paged_kv_cache(const void* append_key, int64_t k_stride_n, int64_t k_stride_h,
                              const void* append_value, int64_t v_stride_n, int64_t v_stride_h,
                              const int32_t* batch_indices, const int32_t* positions, int32_t nnz,
                              void* k_cache, void* v_cache, int64_t page_stride, int64_t num_pages,
                              const int32_t* kv_indices, int64_t num_indices,
                              const int32_t* kv_indptr, int32_t batch,
                              int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                              int32_t dtype, int32_t* err_count, void* stream);

/* The same append with each token's destination resolved beforehand: token i goes to page
 * slots[i] / page_size, slot slots[i] % page_size (slots as pkv_pool_gather writes them).  What
 * the CUDA-graph decode step's append (ecahlang/manager.py:270-280, the reference's
 * append_paged_kv_cache with the bucket's static batch_indices / positions / kv_indptr /
 * kv_indices) computes, with one lookup per token instead of three dependent ones.  A slot
 * that is negative or outside the num_pages-page pool is skipped and counted in *err_count
 * (may be NULL). */
int pkv_append_paged_kv_cache_slots(const void* append_key, int64_t k_stride_n, int64_t k_stride_h,
                                    const void* append_value, int64_t v_stride_n, int64_t v_stride_h,
                                    const int32_t* slots, int32_t nnz, void* k_cache, void* v_cache,
                                    int64_t page_stride, int64_t num_pages, int32_t num_kv_heads,
                                    int32_t head_dim, int32_t page_size, int32_t dtype,
                                    int32_t* err_count, void* stream);

/* The model's rotary embedding on the new tokens' q and k, then the append, in one launch:
 * apply_rotary_pos_emb (transformers/models/qwen2/modeling_qwen2.py:210-211, run just before
 * the attention hook) followed by the hook's append (ecahlang/main.py:62-66 ->
 * pkv_append_paged_kv_cache).  q rows [nnz, num_qo_heads, head_dim] are rotated into q_out
 * (q_out == q rotates in place); key rows are rotated and scattered like
 * pkv_append_paged_kv_cache; value rows are scattered unchanged.  cos / sin are the tokens'
 * rows [nnz, head_dim] of the model's position embeddings (row stride cs_stride_n), in the
 * cache dtype.  Rotation: x*cos + rotate_half(x)*sin with rotate_half(x) = cat(-x2, x1),
 * each product and the sum rounded to the dtype, so the outputs are bit-identical to the
 * model's rotation followed by the plain append.  head_dim must be a multiple of 8.  Bad
 * metadata is skipped and counted once per token in *err_count (may be NULL). */
int pkv_append_paged_kv_cache_rope(const void* q, int64_t q_stride_n, int64_t q_stride_h, void* q_out,
                                   int64_t qo_stride_n, int64_t qo_stride_h, int32_t num_qo_heads,
                                   const void* append_key, int64_t k_stride_n, int64_t k_stride_h,
                                   const void* append_value, int64_t v_stride_n, int64_t v_stride_h,
                                   const void* cos, const void* sin, int64_t cs_stride_n,
                                   const int32_t* batch_indices, const int32_t* positions, int32_t nnz,
                                   void* k_cache, void* v_cache, int64_t page_stride, int64_t num_pages,
                                   const int32_t* kv_indices, int64_t num_indices, const int32_t* kv_indptr,
                                   int32_t batch, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                   int32_t dtype, int32_t* err_count, void* stream);

/* Smallest workspace pkv_decode_plan and pkv_batch_decode need for this geometry (num_indices =
 * length of the kv_indices buffer): the host half of BatchDecodeWithPagedKVCacheWrapper.plan
 * (ecahlang/main.py:341-347, :444-455).  The reference hands the wrapper a 128 MiB buffer
 * (ecahlang/main.py:203).  A larger workspace also holds the partial results of shared-prefix
 * chunks (see pkv_decode_plan); the layout depends on the size, so pass plan and decode the
 * same workspace_bytes. */
int64_t pkv_decode_workspace_bytes(int32_t batch, int32_t num_qo_heads, int32_t head_dim,
                                   int32_t num_ctas, int64_t num_indices);

/* Where pkv_decode_plan puts its schedule inside a workspace of workspace_bytes for this geometry.
 * A host-only diagnostic for tests and tools that read the schedule back; no counterpart in the
 * reference.  out[0..7] = byte offsets of the global header, the range heads and the range
 * records and the prefix item records, then the range capacity, the partial slot capacity, the
 * words per range head and the words per range record (record formats: decode_sched.h).
 * Returns 0, or PKV_E_ARG / PKV_E_WORKSPACE as pkv_decode_plan would. */
int pkv_decode_schedule_layout(int32_t batch, int32_t num_qo_heads, int32_t head_dim,
                               int32_t num_ctas, int64_t num_indices, int64_t workspace_bytes,
                               int64_t* out);

/* Zeroes the split-merge counters at the head of the workspace (the device half of plan).
 * pkv_batch_decode leaves them zero again when it finishes, so this is needed only when the
 * buffer is fresh or the batch grows. */
int pkv_decode_workspace_init(void* workspace, int32_t batch, void* stream);

/* The device half of BatchDecodeWithPagedKVCacheWrapper.plan (ecahlang/main.py:341-347,
 * :444-455, :538-548): two kernels read the page table (kv_indptr, kv_indices,
 * kv_last_page_len) and write the matrix-core kernel's schedule into the workspace: the batch's
 * pages cut into ranges (about one per workgroup, at most 512 pages each; a range that holds a
 * sequence start gets fewer pages, since its waves combine their states there), each with its
 * sequence segments and a copy of its page ids.  FlashInfer's plan computes its schedule on the
 * host after copying kv_indptr back; this one never synchronises and can be captured.  Every
 * decode launch on the same workspace with PKV_DECODE_PLANNED reads it, so the page table it
 * was built from must not change before those launches (re-plan after rebuilding it, as the
 * reference does before each step).
 *
 * kv_shared_pages (an extension; may be NULL) describes shared prefixes: entry b >= 1 says
 * that the first kv_shared_pages[b] pages of sequence b are the same page ids as the first ones
 * of sequence b - 1 (entry 0 is ignored; the caller guarantees it, as it guarantees the rest of
 * the page table).  The common prefix of a run of consecutive sequences that share at least 16
 * pages is then copied with the cached load policy, so every reader after the first finds it in
 * L2 (other pages stream past the caches).  With PKV_PLAN_CASCADE in plan_flags, the common
 * prefix is instead read once per group of 2 * (16 / g) sequences, g = num_qo_heads /
 * num_kv_heads (one workgroup attends the group to each chunk of up to 64 prefix pages, per KV
 * head, and the parts are merged like split sequences); the results are those of the plain
 * schedule up to the order of the fp32 summation.  Each sequence keeps as its own the page
 * that receives the step's token (its last page, and the one before an empty last page), so
 * the fused append of pkv_batch_decode_append works with either plan.  AutoKVCacheManager fills
 * kv_shared_pages for sequences allocated on a prefix. */
#define PKV_PLAN_CASCADE 1
int pkv_decode_plan(const int32_t* kv_indptr, const int32_t* kv_indices, int64_t num_indices,
                    const int32_t* kv_last_page_len, const int32_t* kv_shared_pages, int32_t batch,
                    int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                    int32_t num_ctas, int32_t plan_flags, void* workspace, int64_t workspace_bytes,
                    void* stream);

/* 1 when pkv_batch_decode can run the matrix-core kernel for this shape (fp16/bf16, head_dim
 * 64 or 128, group <= 16, and num_kv_heads at most 8 head blocks of up to 256 / head_dim heads;
 * page_size 16 and 16-byte aligned q rows are checked per call), 0 when it runs the vector-ALU
 * kernel. */
int pkv_decode_uses_mfma(int32_t dtype, int32_t head_dim, int32_t num_qo_heads,
                         int32_t num_kv_heads, int32_t batch);

/* BatchDecodeWithPagedKVCacheWrapper.run(q, paged_kv_cache) (ecahlang/main.py:68, captured
 * at :162-171): out[b, h, :] = softmax(q[b,h] . K_b^T * sm_scale) V_b over the
 * seq_len_b = (npages_b - 1) * page_size + kv_last_page_len[b] tokens of sequence b, with
 * KV head h / (num_qo_heads / num_kv_heads); fp32 accumulation, output in `dtype`.  A
 * sequence with no tokens yields zeros.  num_ctas workgroups each stream an equal share of
 * the batch's pages.  flags: PKV_DECODE_PLANNED says pkv_decode_plan has written this page
 * table's schedule into the workspace (same batch, num_indices and num_ctas), which the
 * matrix-core kernel needs; without it the vector-ALU kernel runs.  PKV_DECODE_VALU selects the
 * vector-ALU kernel (cross-checks); PKV_DECODE_DYNAMIC lets that kernel's waves take pages on
 * demand (the summation order, and so the last bits of the result, then vary from call to
 * call).  Otherwise the result is bitwise reproducible for a given num_ctas.  Page ids outside
 * [0, num_pages) and page-list entries past num_indices are never read (their tokens are
 * treated as absent); pages before kv_indptr[0] belong to no sequence. */
#define PKV_DECODE_VALU 1
#define PKV_DECODE_DYNAMIC 2
#define PKV_DECODE_PLANNED 4
int pkv_batch_decode(const void* q, int64_t q_stride_n, int64_t q_stride_h, const void* k_cache,
                     const void* v_cache, int64_t page_stride, int64_t num_pages,
                     const int32_t* kv_indptr, const int32_t* kv_indices, int64_t num_indices,
                     const int32_t* kv_last_page_len, int32_t batch,
                     int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                     int32_t page_size, float sm_scale, int32_t num_ctas, void* workspace,
                     int64_t workspace_bytes, void* out, int64_t o_stride_n, int64_t o_stride_h,
                     int32_t dtype, int32_t flags, void* stream);

/* The CUDA-graph decode step's append (ecahlang/manager.py:270-280, append_paged_kv_cache
 * through the bucket's metadata, whose positions are seq_len_b - 1: main.py:62-64) followed by
 * BatchDecodeWithPagedKVCacheWrapper.run (main.py:68), in one call: token b's new K and V rows
 * (append_key / append_value [batch, num_kv_heads, head_dim], element strides) go to position
 * seq_len_b - 1 = (n_b - 1) * page_size + kv_last_page_len[b] - 1 of sequence b's n_b pages
 * (the last page's slot kv_last_page_len - 1; with kv_last_page_len 0, the empty page the
 * reference's append_tokens adds when a page fills, the previous page's last slot), then out
 * is computed as by pkv_batch_decode over the caches holding them; out and the caches are
 * bitwise those of pkv_append_paged_kv_cache at those positions + pkv_batch_decode.  A sequence
 * whose page list is empty or cut at num_indices, whose kv_last_page_len is outside
 * [0, page_size], whose position is negative or whose page id is outside the pool gets no
 * append.  On the matrix-core kernel (PKV_DECODE_PLANNED, no
 * PKV_DECODE_DYNAMIC, a plan without PKV_PLAN_CASCADE, 16-byte aligned rows) the append rides
 * in the decode launch; otherwise it is a launch of its own before the decode. */
int pkv_batch_decode_append(const void* q, int64_t q_stride_n, int64_t q_stride_h,
                            const void* append_key, int64_t k_stride_n, int64_t k_stride_h,
                            const void* append_value, int64_t v_stride_n, int64_t v_stride_h,
                            void* k_cache, void* v_cache, int64_t page_stride, int64_t num_pages,
                            const int32_t* kv_indptr, const int32_t* kv_indices, int64_t num_indices,
                            const int32_t* kv_last_page_len, int32_t batch, int32_t num_qo_heads,
                            int32_t num_kv_heads, int32_t head_dim, int32_t page_size, float sm_scale,
                            int32_t num_ctas, void* workspace, int64_t workspace_bytes, void* out,
                            int64_t o_stride_n, int64_t o_stride_h, int32_t dtype, int32_t flags,
                            void* stream);

/* pkv_decode_plan + pkv_batch_decode in one call that allocates nothing and takes no workspace:
 * the counters, split partials and schedule live in a file-scope device array of
 * PKV_NOALLOC_SCRATCH_BYTES per device, held by every device the library runs on until the
 * process ends.  No counterpart in the reference (FlashInfer's wrappers take a workspace): it is
 * for callers that cannot allocate or own a workspace, such as code under graph capture or a
 * tight serving loop.  Arguments as pkv_batch_decode (num_ctas workgroups); the result is bitwise
 * the same as pkv_decode_plan + pkv_batch_decode with the same num_ctas.  Returns PKV_E_WORKSPACE,
 * enqueueing nothing, when this geometry needs more than the array holds
 * (pkv_decode_workspace_bytes > PKV_NOALLOC_SCRATCH_BYTES).  All calls on one device share that
 * device's array, so calls that overlap on one device (another stream, another thread) race. */
#define PKV_NOALLOC_SCRATCH_BYTES (16 << 20)
int pkv_batch_decode_noalloc(const void* q, int64_t q_stride_n, int64_t q_stride_h,
                             const void* k_cache, const void* v_cache, int64_t page_stride,
                             int64_t num_pages, const int32_t* kv_indptr, const int32_t* kv_indices,
                             int64_t num_indices, const int32_t* kv_last_page_len, int32_t batch,
                             int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                             int32_t page_size, float sm_scale, int32_t num_ctas, void* out,
                             int64_t o_stride_n, int64_t o_stride_h, int32_t dtype, void* stream);

/* BatchPrefillWithPagedKVCacheWrapper.run(q, paged_kv_cache) after
 * plan(qo_indptr, kv_indptr, kv_indices, kv_last_page_len, ..., causal=...)
 * (ecahlang/main.py:432-443, :68), vector-ALU kernel: query row i of request b
 * (qo_len_b = qo_indptr[b+1] - qo_indptr[b]) attends keys j <= i + kv_len_b - qo_len_b when
 * causal != 0 (bottom-right aligned), else all kv_len_b keys. */
int pkv_batch_prefill_valu(const void* q, int64_t q_stride_n, int64_t q_stride_h,
                           const int32_t* qo_indptr, int32_t nnz_q, const void* k_cache,
                           const void* v_cache, int64_t page_stride, int64_t num_pages,
                           const int32_t* kv_indptr, const int32_t* kv_indices,
                           int64_t num_indices, const int32_t* kv_last_page_len,
                           int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                           int32_t head_dim, int32_t page_size, int32_t causal, float sm_scale,
                           void* out, int64_t o_stride_n, int64_t o_stride_h, int32_t dtype,
                           void* stream);

/* BatchPrefillWithPagedKVCacheWrapper.run on the matrix cores (same contract as
 * pkv_batch_prefill_valu; ecahlang/main.py:432-443, :68) for fp16/bf16, head_dim 64 or 128,
 * page_size 16 and GQA groups 1, 2, 4, 8, 16 (pkv_prefill_mfma_supported).  The work list comes
 * from the wrapper's plan: n_items records of 12 int32 {request, kv_head, first query token,
 * query tokens, key chunk begin, key chunk end, partial slot or -1, kv_len, qo_len, first q row,
 * first page-list entry, 0}, each covering 256 / g query tokens; n_groups records of 8 int32
 * {first slot, slots, first q row, first query token, query tokens, kv_head, 0, 0} name the
 * split items whose partials (part_ml: float2 x 256 per slot, part_o: fp32 x 256 x head_dim per
 * slot) a second kernel merges.  q must be 16-byte aligned with strides that keep rows
 * aligned (PKV_E_ALIGN otherwise). */
int pkv_prefill_mfma_supported(int32_t dtype, int32_t head_dim, int32_t num_qo_heads,
                               int32_t num_kv_heads, int32_t page_size);
/* The host half of BatchPrefillWithPagedKVCacheWrapper.plan (ecahlang/main.py:432-443; host
 * memory in and out, no device call): the work list pkv_batch_prefill_mfma takes, for a batch of
 * `batch` requests (qo_indptr, kv_indptr [batch + 1], kv_last_page_len [batch]) with GQA group
 * `group` and `rows` query rows per item.  chunk: keys per item (a multiple of 64 in
 * [256, 8192]), or 0 to pick the one with the lowest simulated kernel time among chunks around
 * total keys / num_cus, doubled while the split partials (partial_bytes per element: 2 or 4)
 * would not fit in workspace_bytes.  Writes the items (12 int32 each, longest key range first)
 * and split groups (8 int32 each) and info[8] = {n_items, n_groups, chunk, slots, byte offset
 * of the groups, of part_ml, of part_o, workspace bytes needed}.  Returns 0, PKV_E_WORKSPACE
 * (info filled) or PKV_E_ARG (bad arguments, or more records than items_cap / groups_cap). */
int pkv_prefill_work_list(const int32_t* qo_indptr, const int32_t* kv_indptr,
                          const int32_t* kv_last_page_len, int32_t batch, int32_t group,
                          int32_t num_kv_heads, int32_t page_size, int32_t causal, int32_t head_dim,
                          int32_t num_cus, int64_t workspace_bytes, int32_t rows,
                          int32_t partial_bytes, int32_t chunk, int32_t* items, int64_t items_cap,
                          int32_t* groups, int64_t groups_cap, int64_t* info);
int pkv_batch_prefill_mfma(const void* q, int64_t q_stride_n, int64_t q_stride_h,
                           const void* k_cache, const void* v_cache, int64_t page_stride,
                           int64_t num_pages, const int32_t* kv_indices, int64_t num_indices,
                           int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                           int32_t page_size, int32_t causal, float sm_scale,
                           const int32_t* items, int32_t n_items, const int32_t* groups,
                           int32_t n_groups, void* part_ml, void* part_o, void* out,
                           int64_t o_stride_n, int64_t o_stride_h, int32_t dtype, void* stream);

/* Page pool of AutoKVCacheManager (ecahlang/manager.py:56, 99-120, 187-212), device side.
 * stack[0 .. n_free) holds the free page ids (the reference's free_blocks list: pop() takes
 * the last entry, extend() appends in page order); table is rows x stride int32, one row of
 * page ids per sequence slot.  Applies n_ops queued operations in order; operation i is
 * ops[5i .. 5i+4] = {kind, row, pos, col, n}:
 *   kind 0, pop  (allocate :104, append_tokens :201-203, init_cuda_graph_buffers :212):
 *     table[row][col + k] = stack[pos - 1 - k] for k < n
 *   kind 1, push (free :116): stack[pos + k] = table[row][col + k] for k < n
 *   kind 2, copy: table[row][col + k] = table[pos][k] for k < n (a sequence that shares the
 *     leading pages of the sequence in row pos; the reference has no page sharing, so this
 *     kind and the next have no counterpart there)
 *   kind 3, copy on write: table[row][col] = stack[pos - 1] (one pop), after writing the old
 *     and the new page id to pairs[2n], pairs[2n + 1] (n < pairs_cap) for
 *     pkv_pool_copy_pages
 * Operations outside the stack, table or pairs are skipped and counted in *err (may be NULL). */
int pkv_pool_apply(int32_t* stack, int32_t stack_size, int32_t* table, int64_t stride,
                   int32_t rows, const int32_t* ops, int32_t n_ops, int32_t* pairs, int32_t pairs_cap,
                   int32_t* err, void* stream);

/* The K/V data of n_pairs copy-on-write pairs (the page-sharing extension of AutoKVCacheManager;
 * no counterpart in the reference): for every layer l < layers, the page_bytes bytes of page
 * pairs[2p] at cache + l * layer_stride are copied to page pairs[2p + 1] (byte offsets
 * page * page_bytes).  16-byte aligned; pairs naming pages outside [0, num_pages) are skipped
 * and counted in *err (may be NULL). */
int pkv_pool_copy_pages(void* cache, int64_t layer_stride, int32_t layers, int64_t page_bytes,
                        const int32_t* pairs, int32_t n_pairs, int64_t num_pages, int32_t* err,
                        void* stream);

/* The decode plan's kv_shared_pages from a page table (the page-sharing extension; no
 * counterpart in the reference): out[b] = the number of leading page ids rows b and b - 1
 * have in common, out[0] = 0.  Rows past num_indices count as sharing nothing. */
int pkv_shared_prefix_pages(const int32_t* kv_indptr, const int32_t* kv_indices, int64_t num_indices,
                            int32_t batch, int32_t* out, void* stream);

/* The page walk of get_append_metadata / fill_cuda_graph_metadata (ecahlang/manager.py:124-133,
 * :231-246): kv_indices[indptr[b] + k] = table[desc[4b]][desc[4b+1] + k] for k < desc[4b+2],
 * with indptr[batch+1] (the exclusive scan of the desc counts) already on the device.  At most
 * min(max_total, num_indices) entries are written; entries with no source are set to -1 and
 * counted in *err (may be NULL).  With slots (may be NULL; then positions and page_size are
 * unused), also slots[b] = page * page_size + positions[b] % page_size, where page is the
 * gathered id at position positions[b] of row b, or -1 when that position lies outside the
 * row's gathered pages: the destinations pkv_append_paged_kv_cache_slots takes (the slot that
 * append_paged_kv_cache_cuda_graph, manager.py:270-280, resolves on every layer). */
int pkv_pool_gather(const int32_t* table, int64_t stride, int32_t rows, const int32_t* desc,
                    const int32_t* indptr, int32_t batch, int32_t* kv_indices, int64_t num_indices,
                    int64_t max_total, const int32_t* positions, int32_t page_size, int32_t* slots,
                    int32_t* err, void* stream);

/* One decode step of a fixed batch, entirely on the device: the serving loop's
 * append_tokens(b, n_tokens) for every sequence of the batch, in batch order (ecahlang/main.py
 * :328-335 -> manager.py:187-205), then fill_cuda_graph_metadata for the bucket
 * (manager.py:228-253).  rows[i] is the table row of batch entry i, or -1 for a padding entry
 * (one page from padding_row, last_page_len 1, position 0).  npages[row] and last_len[row] are
 * the device's copies of each row's page count and last-page length, and *n_free the device's
 * free-stack size: each row takes (last_len + n_tokens) / page_size pages from the top of the
 * stack after the rows before it, exactly as the reference's loop pops them, and keeps
 * (last_len + n_tokens) % page_size as its new last-page length.  Then kv_indptr[batch + 1],
 * kv_last_page_len[batch], positions[batch] (each row's newest token), kv_indices (at most
 * min(max_total, num_indices) entries) and slots[batch] are written as pkv_pool_gather writes
 * them (desc[4 * batch] is scratch).  No extension of the reference: it is the same step with no
 * host work, so the step can be captured in a graph with the model and replayed.  A row whose
 * pages the stack or its table row cannot hold is left unchanged, as are the rows after it, and
 * *err is bumped: callers check the pool before they enqueue the step (AutoKVCacheManager does,
 * and takes the reference's path, which raises, when it would run dry). */
int pkv_pool_step(int32_t* stack, int32_t* n_free, int32_t* table, int64_t stride, int32_t rows_total,
                  const int32_t* rows, int32_t batch, int32_t n_tokens, int32_t page_size,
                  int32_t* npages, int32_t* last_len, int32_t padding_row, int32_t* desc,
                  int32_t* kv_indptr, int32_t* kv_last_page_len, int32_t* positions,
                  int32_t* kv_indices, int64_t num_indices, int64_t max_total, int32_t* slots,
                  int32_t* err, void* stream);

/* The hand-over of a batch to pkv_pool_step (AutoKVCacheManager.begin_device_steps, an
 * extension with no counterpart in the reference), from the gather descriptor and
 * kv_last_page_len that fill_cuda_graph_metadata wrote for the bucket: rows[i] = desc[4i] for
 * the real entries i < real and -1 for the padding entries i < batch; npages[desc[4i]] =
 * desc[4i + 2] and last_len[desc[4i]] = kv_last_page_len[i] for the real entries (rows outside
 * [0, rows_total) are skipped and counted in *err, which may be NULL); *n_free_out = n_free. */
int pkv_pool_steps_begin(const int32_t* desc, const int32_t* kv_last_page_len, int32_t batch, int32_t real,
                         int32_t n_free, int32_t* rows, int32_t* npages, int32_t* last_len,
                         int32_t rows_total, int32_t* n_free_out, int32_t* err, void* stream);

/* Top-k / top-p sampling from logits (flashinfer.sampling.top_k_top_p_sampling_from_logits at
 * ecahlang/main.py:377-379, 400-402, 489-491, 582-584: top-k first, then top-p on the
 * renormalised top-k distribution, deterministic=True).  logits: rows x vocab (row stride in
 * elements, dtype PKV fp16/bf16/fp32); top_k / top_p per row, or NULL to use top_k_all /
 * top_p_all for every row (k <= 0 or k >= vocab: no top-k filter; top_p >= 1: no top-p
 * filter); uniform: one number in [0, 1) per row, which selects the token by inverse CDF over
 * the kept tokens in vocabulary order (so the caller owns the random stream).  out: int32 token
 * per row (-1 for a row with no finite logit).  Ties at a threshold are kept. */
int pkv_top_k_top_p_sampling(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab,
                             int32_t dtype, const int32_t* top_k, int32_t top_k_all,
                             const float* top_p, float top_p_all, const float* uniform,
                             int32_t* out, void* stream);

/* Workspace bytes pkv_top_k_top_p_sampling_ws can use for rows x vocab. */
int64_t pkv_sampling_workspace_bytes(int32_t rows, int32_t vocab);

/* pkv_top_k_top_p_sampling with a workspace (8-byte aligned, workspace_bytes >=
 * pkv_sampling_workspace_bytes): rows sampled from their whole distribution (top_k <= 0 or
 * >= vocab and top_p >= 1, the serving loop's default request) are then spread over many
 * workgroups per row instead of one.  Same tokens, bit for bit; the workspace needs no
 * initialisation (its counters are reset by the call itself). */
int pkv_top_k_top_p_sampling_ws(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab,
                                int32_t dtype, const int32_t* top_k, int32_t top_k_all, const float* top_p,
                                float top_p_all, const float* uniform, int32_t* out, void* workspace,
                                int64_t workspace_bytes, void* stream);

/* The serving loop's scaling of the logits before sampling (ecahlang/main.py:169-170, 483-487,
 * 566-579: `logits / mask_penalty[slot_of_row]` in the logits' dtype, then `/ temperature` with
 * a float32 temperature, which promotes to float32), in one pass instead of a gather and two
 * divisions: out[b][i] = float32(dtype(logits[b][i] / penalty[penalty_rows[b] * penalty_stride
 * + i])) / temperature[b], with IEEE divisions, so the values are bit-identical to those tensor
 * ops.  penalty (the logits' dtype, penalty_slots rows) and temperature (float32, one per row)
 * may each be NULL; a row whose penalty_rows entry is outside [0, penalty_slots) is written as
 * NaN (the sampler then returns -1 for it).  out is float32, rows <= 65535. */
int pkv_scale_logits(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab, int32_t dtype,
                     const void* penalty, int64_t penalty_stride, int32_t penalty_slots,
                     const int32_t* penalty_rows, const float* temperature, float* out, int64_t out_stride,
                     void* stream);

/* A measurement helper with no counterpart in the reference: reads `bytes` of device memory at
 * src (16-byte aligned, a multiple of 16 bytes) with `blocks` workgroups of 1024 threads, each
 * workgroup a contiguous slice, with 16-byte non-temporal loads; *sink (device, 4 bytes) may be
 * written.  Timed by the caller, it gives the HBM read rate a launch of that size reaches. */
int pkv_probe_stream_read(const void* src, int64_t bytes, int32_t blocks, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* PAGEDKV_H */
