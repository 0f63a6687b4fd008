// Batch paged decode: C-ABI entry points, workspace layout and kernel choice.
//
//   pkv_decode_workspace_bytes / pkv_decode_workspace_init  <- BatchDecodeWithPagedKVCacheWrapper.plan
//   pkv_batch_decode                                        <- BatchDecodeWithPagedKVCacheWrapper.run
//   (ecahlang/main.py:203-204 construct, :341-347 / :444-455 plan, :68 run)
//
// Workspace (caller-owned bytes, 256-byte aligned regions):
//   [counters: int32 x batch] [part_ml: float2 x (ctas+batch) x Hq] [part_o: f32 x (ctas+batch) x Hq x D]
#include "attn_common.h"
#include "../../include/pagedkv.h"

using namespace pkv;

namespace {

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct WsLayout {
  size_t cnt, ml, o, total;
};
inline WsLayout ws_layout(int batch, int hq, int d, int ctas) {
  WsLayout L;
  size_t segs = (size_t)ctas + batch;
  L.cnt = 0;
  L.ml = align256(sizeof(int32_t) * (size_t)batch);
  L.o = L.ml + align256(sizeof(float) * 2 * segs * hq);
  L.total = L.o + align256(sizeof(float) * segs * hq * d);
  return L;
}

__global__ void zero_i32_kernel(int32_t* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

}  // namespace

extern "C" int64_t pkv_decode_workspace_bytes(int32_t batch, int32_t num_qo_heads,
                                              int32_t head_dim, int32_t num_ctas,
                                              int64_t num_indices) {
  if (batch < 0 || num_qo_heads <= 0 || head_dim <= 0 || num_ctas <= 0 || num_indices < 0)
    return kBadArg;
  const int64_t ranges = decode_ranges_max(num_ctas, num_indices);
  return (int64_t)ws_layout(batch, num_qo_heads, head_dim, (int)ranges).total;
}

extern "C" int pkv_decode_workspace_init(void* workspace, int32_t batch, void* stream) {
  if (batch <= 0) return kOk;
  // A fill kernel rather than a memset node, so the call is also safe under graph capture.
  hipLaunchKernelGGL(zero_i32_kernel, dim3((batch + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     (int32_t*)workspace, batch);
  return (int)hipGetLastError();
}

extern "C" int pkv_decode_uses_mfma(int32_t dtype, int32_t head_dim, int32_t num_qo_heads,
                                    int32_t num_kv_heads, int32_t batch) {
  if (num_kv_heads <= 0 || num_qo_heads % num_kv_heads) return 0;
  return decode_mfma_supported(dtype, head_dim, num_qo_heads / num_kv_heads, num_kv_heads, batch)
             ? 1 : 0;
}

extern "C" int pkv_batch_decode(const void* q, int64_t q_stride_n, int64_t q_stride_h,
                                const void* k_cache, const void* v_cache, int64_t page_stride,
                                int64_t num_pages, const int32_t* kv_indptr,
                                const int32_t* kv_indices, int64_t num_indices,
                                const int32_t* kv_last_page_len, int32_t batch,
                                int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                int32_t page_size, float sm_scale, int32_t num_ctas,
                                void* workspace, int64_t workspace_bytes, void* out,
                                int64_t o_stride_n, int64_t o_stride_h, int32_t dtype,
                                int32_t flags, void* stream) {
  if (batch <= 0 || num_kv_heads <= 0 || num_qo_heads <= 0 || num_ctas <= 0) return kBadArg;
  if (num_qo_heads % num_kv_heads) return kBadGroup;
  if (page_size <= 0) return kBadPageSize;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return kBadHeadDim;
  if (num_indices < 0 || num_pages < 0) return kBadArg;
  // Partial slots are indexed by range + sequence; ranges never exceed this bound.
  WsLayout L = ws_layout(batch, num_qo_heads, head_dim, (int)decode_ranges_max(num_ctas, num_indices));
  if ((int64_t)L.total > workspace_bytes) return kWorkspaceTooSmall;
  DecodeParams P;
  P.q = q; P.q_sn = q_stride_n; P.q_sh = q_stride_h;
  P.k_cache = k_cache; P.v_cache = v_cache; P.page_stride = page_stride;
  P.num_pages = num_pages; P.num_indices = num_indices;
  P.indptr = kv_indptr; P.indices = kv_indices; P.last = kv_last_page_len;
  P.batch = batch; P.hq = num_qo_heads; P.hkv = num_kv_heads; P.ps = page_size;
  P.scale_log2 = sm_scale * 1.4426950408889634f;
  P.out = out; P.o_sn = o_stride_n; P.o_sh = o_stride_h;
  char* ws = (char*)workspace;
  P.counters = (int32_t*)(ws + L.cnt);
  P.part_ml = (float2*)(ws + L.ml);
  P.part_o = (float*)(ws + L.o);
  P.num_ctas = num_ctas;
  P.dynamic = (flags & PKV_DECODE_DYNAMIC) != 0;
  const int es = dtype == kF32 ? 4 : 2;
  P.q_vec = ((uintptr_t)q % 16 == 0) && ((q_stride_n * es) % 16 == 0) && ((q_stride_h * es) % 16 == 0);
  P.o_vec = ((uintptr_t)out % 8 == 0) && ((o_stride_n * es) % 8 == 0) && ((o_stride_h * es) % 8 == 0);
  hipStream_t s = (hipStream_t)stream;
  int g = num_qo_heads / num_kv_heads;
  if (!(flags & PKV_DECODE_VALU) && decode_mfma_supported(dtype, head_dim, g, num_kv_heads, batch))
    return decode_mfma_dispatch(P, dtype, head_dim, s);
  return decode_valu_dispatch(P, dtype, head_dim, s);
}
