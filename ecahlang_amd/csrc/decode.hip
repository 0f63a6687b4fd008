// Batch paged decode: C-ABI entry points, workspace layout and kernel choice.
//
//   pkv_decode_workspace_bytes / pkv_decode_workspace_init / pkv_decode_plan
//                                          <- BatchDecodeWithPagedKVCacheWrapper.plan
//   pkv_batch_decode                       <- BatchDecodeWithPagedKVCacheWrapper.run
//   pkv_batch_decode_append                <- the CUDA-graph decode step's append
//                                             (ecahlang/manager.py:270-280) + run
//   (ecahlang/main.py:203-204 construct, :341-347 / :444-455 plan, :68 run)
//
// Workspace (caller-owned bytes, 256-byte aligned regions; R = decode_ranges_cap ranges):
//   [counters: int32 x batch]
//   [schedule: global header + empty list (kGlobHdr + batch int32), R heads of kHeadWords
//    int32, R range records of kRecStride int32, R prefix item records of kPrecStride int32,
//    first-sequence[R], range starts[R + 1], non-empty ranges before[R + 1], plan scratch
//    (decode_plan_scratch_words)]
//   [part_ml: float2 x S x ml_slot_stride(Hq)] [part_o: f32 x S x Hq x D]
// with S = R + batch partial slots, plus up to kMaxPrefixParts x batch more for shared-prefix
// chunks when the workspace has room (each part_ml slot is whole 128-byte lines).  The layout
// depends on the workspace size, so plan and run are given the same size.
#include <mutex>
#include <unordered_map>
#include "attn_common.h"
#include "decode_sched.h"
#include "../../include/pagedkv.h"

using namespace pkv;

namespace pkv {
int64_t decode_plan_scratch_words(int batch);
int decode_plan_launch(const int32_t* indptr, const int32_t* indices, int64_t num_indices,
                       const int32_t* last, const int32_t* shared, int batch, int num_ctas,
                       int page_size, int seg_cost, int group, int hkv, int cascade, int r_cap, int slot_cap,
                       int32_t* ghdr, int32_t* recs, int32_t* heads, int32_t* precs, int32_t* bf,
                       int32_t* starts, int32_t* nzb, int32_t* scratch, hipStream_t s);
int decode_mfma_group(int d, int g, int hkv);
}

namespace {

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct WsLayout {
  size_t cnt, ghdr, heads, recs, precs, bf, starts, nzb, scratch, ml, o, total;
  int64_t rcap, slots;
};
// Layout for a workspace of ws_bytes (< 0: the smallest one, without shared-prefix slots).
inline WsLayout ws_layout(int batch, int hq, int d, int ctas, int64_t num_indices, int64_t ws_bytes = -1) {
  WsLayout L;
  L.rcap = decode_ranges_cap(ctas, num_indices);
  L.cnt = 0;
  L.ghdr = align256(sizeof(int32_t) * (size_t)batch);
  L.heads = L.ghdr + align256(sizeof(int32_t) * ((size_t)kGlobHdr + batch));
  L.recs = L.heads + align256(sizeof(int32_t) * (size_t)L.rcap * kHeadWords);
  L.precs = L.recs + align256(sizeof(int32_t) * (size_t)L.rcap * kRecStride);
  L.bf = L.precs + align256(sizeof(int32_t) * (size_t)L.rcap * kPrecStride);
  L.starts = L.bf + align256(sizeof(int32_t) * (size_t)L.rcap);
  L.nzb = L.starts + align256(sizeof(int32_t) * ((size_t)L.rcap + 1));
  L.scratch = L.nzb + align256(sizeof(int32_t) * ((size_t)L.rcap + 1));
  L.ml = L.scratch + align256(sizeof(int32_t) * (size_t)decode_plan_scratch_words(batch));
  const size_t ml_slot = sizeof(float) * 2 * ml_slot_stride(hq), o_slot = sizeof(float) * hq * d;
  const int64_t base = L.rcap + batch;
  int64_t extra = 0;
  if (ws_bytes > 0) {
    // (a 256-byte alignment pad per array)
    const int64_t room = ws_bytes - (int64_t)L.ml - 512 - base * (int64_t)(ml_slot + o_slot);
    extra = room > 0 ? room / (int64_t)(ml_slot + o_slot) : 0;
    const int64_t cap = (int64_t)kMaxPrefixParts * batch;
    extra = extra < cap ? extra : cap;
  }
  L.slots = base + extra;
  L.o = L.ml + align256(ml_slot * (size_t)L.slots);
  L.total = L.o + align256(o_slot * (size_t)L.slots);
  return L;
}

// Which workspaces hold a cascade schedule (the decode launches the kernel variant that reads
// prefix items only for those): recorded by pkv_decode_plan, read by pkv_batch_decode.
std::mutex g_plan_mu;
std::unordered_map<const void*, bool> g_plan_cascade;

__global__ void zero_i32_kernel(int32_t* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

// Sizes the schedule's words can hold: ranges and parts in 16 bits, sequences in 27, and the
// partial outputs addressed with 32-bit byte offsets.
bool ws_args_ok(int32_t batch, int32_t hq, int32_t d, int32_t ctas, int64_t num_indices) {
  if (!(batch >= 0 && batch < (1 << kSegBBits) && hq > 0 && d > 0 && ctas > 0 && num_indices >= 0))
    return false;
  const int64_t rcap = decode_ranges_cap(ctas, num_indices);
  if (rcap > kMaxRanges) return false;
  const int64_t slots = rcap + (int64_t)(1 + kMaxPrefixParts) * batch;
  return slots * hq * d * (int64_t)sizeof(float) < ((int64_t)1 << 32);
}

}  // namespace

extern "C" int64_t pkv_decode_workspace_bytes(int32_t batch, int32_t num_qo_heads,
                                              int32_t head_dim, int32_t num_ctas,
                                              int64_t num_indices) {
  if (!ws_args_ok(batch, num_qo_heads, head_dim, num_ctas, num_indices)) return kBadArg;
  return (int64_t)ws_layout(batch, num_qo_heads, head_dim, num_ctas, num_indices).total;
}

extern "C" int pkv_decode_schedule_layout(int32_t batch, int32_t num_qo_heads, int32_t head_dim,
                                          int32_t num_ctas, int64_t num_indices, int64_t workspace_bytes,
                                          int64_t* out) {
  if (!out || !ws_args_ok(batch, num_qo_heads, head_dim, num_ctas, num_indices)) return kBadArg;
  const WsLayout L = ws_layout(batch, num_qo_heads, head_dim, num_ctas, num_indices, workspace_bytes);
  if ((int64_t)L.total > workspace_bytes) return kWorkspaceTooSmall;
  out[0] = (int64_t)L.ghdr;
  out[1] = (int64_t)L.heads;
  out[2] = (int64_t)L.recs;
  out[3] = (int64_t)L.precs;
  out[4] = L.rcap;
  out[5] = L.slots;
  out[6] = kHeadWords;
  out[7] = kRecStride;
  return kOk;
}

extern "C" int pkv_decode_workspace_init(void* workspace, int32_t batch, void* stream) {
  if (batch <= 0) return kOk;
  // A fill kernel rather than a memset node, so the call is also safe under graph capture.
  hipLaunchKernelGGL(zero_i32_kernel, dim3((batch + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     (int32_t*)workspace, batch);
  return (int)hipGetLastError();
}

extern "C" int pkv_decode_plan(const int32_t* kv_indptr, const int32_t* kv_indices,
                               int64_t num_indices, const int32_t* kv_last_page_len,
                               const int32_t* kv_shared_pages, int32_t batch,
                               int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                               int32_t page_size, int32_t num_ctas, int32_t plan_flags,
                               void* workspace, int64_t workspace_bytes, void* stream) {
  if (batch <= 0) return kOk;
  if (page_size <= 0) return kBadPageSize;
  if (num_kv_heads <= 0 || num_qo_heads % num_kv_heads) return kBadArg;
  if (!ws_args_ok(batch, num_qo_heads, head_dim, num_ctas, num_indices)) return kBadArg;
  const WsLayout L = ws_layout(batch, num_qo_heads, head_dim, num_ctas, num_indices, workspace_bytes);
  if ((int64_t)L.total > workspace_bytes) return kWorkspaceTooSmall;
  char* ws = (char*)workspace;
  const int group = decode_mfma_group(head_dim, num_qo_heads / num_kv_heads, num_kv_heads);
  const bool cascade = (plan_flags & PKV_PLAN_CASCADE) && kv_shared_pages && group >= 2;
  {
    std::lock_guard<std::mutex> lock(g_plan_mu);
    if (cascade) g_plan_cascade[workspace] = true;
    else g_plan_cascade.erase(workspace);
  }
  return decode_plan_launch(kv_indptr, kv_indices, num_indices, kv_last_page_len, kv_shared_pages,
                            batch, num_ctas, page_size, seg_cost_pages(num_kv_heads, head_dim, page_size),
                            group, num_kv_heads, cascade ? 1 : 0, (int)L.rcap,
                            (int)L.slots, (int32_t*)(ws + L.ghdr),
                            (int32_t*)(ws + L.recs), (int32_t*)(ws + L.heads), (int32_t*)(ws + L.precs),
                            (int32_t*)(ws + L.bf), (int32_t*)(ws + L.starts), (int32_t*)(ws + L.nzb),
                            (int32_t*)(ws + L.scratch),
                            (hipStream_t)stream);
}

extern "C" int pkv_decode_uses_mfma(int32_t dtype, int32_t head_dim, int32_t num_qo_heads,
                                    int32_t num_kv_heads, int32_t batch) {
  if (num_kv_heads <= 0 || num_qo_heads % num_kv_heads) return 0;
  return decode_mfma_supported(dtype, head_dim, num_qo_heads / num_kv_heads, num_kv_heads, batch)
             ? 1 : 0;
}

namespace {

// New K and V rows of a decode step, one token per sequence (element strides).
struct AppendRows {
  const void* k;
  int64_t k_sn, k_sh;
  const void* v;
  int64_t v_sn, v_sh;
};

// Token b's K and V rows at position seq_len_b - 1 = (n - 1) * ps + kv_last_page_len[b] - 1 of
// sequence b's n listed pages: the append of a decode step (append_paged_kv_cache with
// batch_indices = b, positions = seq_len_b - 1), one block per sequence, VT-sized pieces.  That
// is the last page's slot kv_last_page_len - 1, or with kv_last_page_len 0 (the empty page the
// pool adds when a page fills) the previous page's last slot.  A sequence whose page list is
// empty or cut at num_indices, whose kv_last_page_len is outside [0, page_size], whose position
// is negative or whose page id is outside the pool gets nothing (the matrix-core kernel's
// fused append places and skips exactly the same tokens).
template <typename VT>
__global__ void append_last_kernel(AppendRows a, char* kc, char* vc, int64_t page_stride, int64_t num_pages,
                                   const int32_t* __restrict__ indptr, const int32_t* __restrict__ indices,
                                   int64_t num_indices, const int32_t* __restrict__ last, int32_t hkv,
                                   int32_t row_bytes, int32_t ps) {
  const int b = blockIdx.x;
  const int e0 = indptr[b], e1 = indptr[b + 1], lp = last[b];
  if (!(e0 >= 0 && e1 > e0 && (int64_t)e1 <= num_indices && lp >= 0 && lp <= ps)) return;
  const int at = (e1 - e0 - 1) * ps + lp - 1;
  if (at < 0) return;
  const int page = indices[e0 + at / ps];
  if (page < 0 || (int64_t)page >= num_pages) return;
  const int per = row_bytes / (int)sizeof(VT);
  const int64_t off = (int64_t)page * page_stride + (int64_t)(at % ps) * hkv * row_bytes;
  for (int x = threadIdx.x; x < 2 * hkv * per; x += blockDim.x) {
    const int kv = x / (hkv * per), r = x - kv * hkv * per, h = r / per, c = r - h * per;
    const char* src = kv ? (const char*)a.v + b * a.v_sn + h * a.v_sh : (const char*)a.k + b * a.k_sn + h * a.k_sh;
    char* dst = (kv ? vc : kc) + off + (int64_t)h * row_bytes;
    *reinterpret_cast<VT*>(dst + c * sizeof(VT)) = *reinterpret_cast<const VT*>(src + c * sizeof(VT));
  }
}

int launch_append_last(const AppendRows& a, int es, void* k_cache, void* v_cache, int64_t page_stride,
                       int64_t num_pages, const int32_t* indptr, const int32_t* indices, int64_t num_indices,
                       const int32_t* last, int32_t batch, int32_t hkv, int32_t d, int32_t ps, hipStream_t s) {
  AppendRows b = a;  // byte strides
  b.k_sn *= es, b.k_sh *= es, b.v_sn *= es, b.v_sh *= es;
  const int row = d * es;
  const int64_t pstride = page_stride * es;
  auto al = [&](int vec) {
    const uintptr_t m = (uintptr_t)a.k | (uintptr_t)a.v | (uintptr_t)k_cache | (uintptr_t)v_cache;
    const int64_t st = b.k_sn | b.k_sh | b.v_sn | b.v_sh | pstride | row;
    return m % vec == 0 && st % vec == 0;
  };
#define PKV_APPEND_LAST(VT)                                                                              \
  hipLaunchKernelGGL(append_last_kernel<VT>, dim3(batch), dim3(128), 0, s, b, (char*)k_cache, (char*)v_cache, \
                     pstride, num_pages, indptr, indices, num_indices, last, hkv, row, ps)
  if (al(16)) PKV_APPEND_LAST(uint4);
  else if (es == 4 || al(4)) PKV_APPEND_LAST(uint32_t);
  else PKV_APPEND_LAST(uint16_t);
#undef PKV_APPEND_LAST
  return (int)hipGetLastError();
}

int batch_decode(const void* q, int64_t q_stride_n, int64_t q_stride_h, const AppendRows* app, void* k_cache,
                 void* v_cache, int64_t page_stride, int64_t num_pages, const int32_t* kv_indptr,
                 const int32_t* kv_indices, int64_t num_indices, const int32_t* kv_last_page_len, int32_t batch,
                 int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size, float sm_scale,
                 int32_t num_ctas, void* workspace, int64_t workspace_bytes, void* out, int64_t o_stride_n,
                 int64_t o_stride_h, int32_t dtype, int32_t flags, void* stream) {
  if (batch <= 0 || num_kv_heads <= 0 || num_qo_heads <= 0 || num_ctas <= 0) return kBadArg;
  if (num_qo_heads % num_kv_heads) return kBadGroup;
  if (page_size <= 0) return kBadPageSize;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return kBadHeadDim;
  if (num_indices < 0 || num_pages < 0) return kBadArg;
  if (dtype != kF32 && dtype != kF16 && dtype != kBF16) return kBadDType;
  if (app && (!app->k || !app->v)) return kBadArg;
  if (!ws_args_ok(batch, num_qo_heads, head_dim, num_ctas, num_indices)) return kBadArg;
  const WsLayout L = ws_layout(batch, num_qo_heads, head_dim, num_ctas, num_indices, workspace_bytes);
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
  P.ml_stride = ml_slot_stride(num_qo_heads);
  P.sched_hdr = (const int32_t*)(ws + L.ghdr);
  P.sched = (const int32_t*)(ws + L.recs);
  P.sched_head = (const int32_t*)(ws + L.heads);
  P.sched_pref = (const int32_t*)(ws + L.precs);
  {
    std::lock_guard<std::mutex> lock(g_plan_mu);
    const auto it = g_plan_cascade.find(workspace);
    P.cascade = it != g_plan_cascade.end() && it->second;
  }
  P.slot_cap = (int32_t)L.slots;
  P.r_cap = (int32_t)L.rcap;
  P.num_ctas = num_ctas;
  P.dynamic = (flags & PKV_DECODE_DYNAMIC) != 0;
  const int es = dtype == kF32 ? 4 : 2;
  P.q_vec = ((uintptr_t)q % 16 == 0) && ((q_stride_n * es) % 16 == 0) && ((q_stride_h * es) % 16 == 0);
  P.o_vec = ((uintptr_t)out % 8 == 0) && ((o_stride_n * es) % 8 == 0) && ((o_stride_h * es) % 8 == 0);
  P.ak = P.av = nullptr;
  P.ak_sn = P.ak_sh = P.av_sn = P.av_sh = 0;
  hipStream_t s = (hipStream_t)stream;
  const int g = num_qo_heads / num_kv_heads;
  // The matrix-core kernel reads the schedule pkv_decode_plan wrote into this workspace.
  if ((flags & PKV_DECODE_PLANNED) && !(flags & PKV_DECODE_VALU) && P.q_vec && page_size == 16 &&
      decode_mfma_supported(dtype, head_dim, g, num_kv_heads, batch)) {
    if (app) {
      // The append rides in the decode kernel (the wave that attends a sequence's last page
      // writes the token there) for the fixed page order of the plan's ranges and 16-byte rows
      // (the page that receives the token is never part of a shared prefix: the plan keeps it
      // in the sequence's own pages); otherwise it is a launch of its own before the decode.
      const uintptr_t m = (uintptr_t)app->k | (uintptr_t)app->v;
      const int64_t st = (app->k_sn | app->k_sh | app->v_sn | app->v_sh) * es;
      if (!P.dynamic && m % 16 == 0 && st % 16 == 0) {
        P.ak = (const char*)app->k;
        P.av = (const char*)app->v;
        P.ak_sn = app->k_sn * es, P.ak_sh = app->k_sh * es, P.av_sn = app->v_sn * es, P.av_sh = app->v_sh * es;
      } else {
        const int rc = launch_append_last(*app, es, k_cache, v_cache, page_stride, num_pages, kv_indptr, kv_indices,
                                          num_indices, kv_last_page_len, batch, num_kv_heads, head_dim, page_size, s);
        if (rc) return rc;
      }
    }
    return decode_mfma_dispatch(P, dtype, head_dim, s);
  }
  if (app) {
    const int rc = launch_append_last(*app, es, k_cache, v_cache, page_stride, num_pages, kv_indptr, kv_indices,
                                      num_indices, kv_last_page_len, batch, num_kv_heads, head_dim, page_size, s);
    if (rc) return rc;
  }
  return decode_valu_dispatch(P, dtype, head_dim, s);
}

}  // namespace

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
  return batch_decode(q, q_stride_n, q_stride_h, nullptr, const_cast<void*>(k_cache), const_cast<void*>(v_cache),
                      page_stride, num_pages, kv_indptr, kv_indices, num_indices, kv_last_page_len, batch,
                      num_qo_heads, num_kv_heads, head_dim, page_size, sm_scale, num_ctas, workspace,
                      workspace_bytes, out, o_stride_n, o_stride_h, dtype, flags, stream);
}

extern "C" int pkv_batch_decode_append(const void* q, int64_t q_stride_n, int64_t q_stride_h,
                                       const void* append_key, int64_t k_stride_n, int64_t k_stride_h,
                                       const void* append_value, int64_t v_stride_n, int64_t v_stride_h,
                                       void* k_cache, void* v_cache, int64_t page_stride, int64_t num_pages,
                                       const int32_t* kv_indptr, const int32_t* kv_indices, int64_t num_indices,
                                       const int32_t* kv_last_page_len, int32_t batch, int32_t num_qo_heads,
                                       int32_t num_kv_heads, int32_t head_dim, int32_t page_size, float sm_scale,
                                       int32_t num_ctas, void* workspace, int64_t workspace_bytes, void* out,
                                       int64_t o_stride_n, int64_t o_stride_h, int32_t dtype, int32_t flags,
                                       void* stream) {
  const AppendRows app{append_key, k_stride_n, k_stride_h, append_value, v_stride_n, v_stride_h};
  return batch_decode(q, q_stride_n, q_stride_h, &app, k_cache, v_cache, page_stride, num_pages, kv_indptr,
                      kv_indices, num_indices, kv_last_page_len, batch, num_qo_heads, num_kv_heads, head_dim,
                      page_size, sm_scale, num_ctas, workspace, workspace_bytes, out, o_stride_n, o_stride_h, dtype,
                      flags, stream);
}

// ---- allocation-free variant: the workspace is a file-scope device array

namespace {

// Scratch for pkv_batch_decode_noalloc: counters, split partials and the schedule of one call.
// Every device the library runs on holds its own copy until the process ends.
constexpr size_t kNoAllocScratchBytes = (size_t)PKV_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
void* g_scratch[kMaxDevices] = {};
std::mutex g_scratch_mu;

// Device address of this device's `scratch`, looked up once per device with that device current
// (host code never passes the symbol itself to a kernel: on the host it is only a stand-in).
int scratch_for(int dev, void** out) {
  if (dev < 0 || dev >= kMaxDevices) return kBadArg;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return (int)e;
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return (int)e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) return (int)e;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return kOk;
}

}  // namespace

extern "C" int pkv_batch_decode_noalloc(const void* q, int64_t q_stride_n, int64_t q_stride_h,
                                        const void* k_cache, const void* v_cache, int64_t page_stride,
                                        int64_t num_pages, const int32_t* kv_indptr,
                                        const int32_t* kv_indices, int64_t num_indices,
                                        const int32_t* kv_last_page_len, int32_t batch,
                                        int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                        int32_t page_size, float sm_scale, int32_t num_ctas, void* out,
                                        int64_t o_stride_n, int64_t o_stride_h, int32_t dtype,
                                        void* stream) {
  if (batch <= 0 || num_kv_heads <= 0 || num_qo_heads <= 0 || num_ctas <= 0) return kBadArg;
  if (!ws_args_ok(batch, num_qo_heads, head_dim, num_ctas, num_indices)) return kBadArg;
  // sizes beyond the array are refused before anything is enqueued
  if (ws_layout(batch, num_qo_heads, head_dim, num_ctas, num_indices).total > kNoAllocScratchBytes)
    return kWorkspaceTooSmall;
  hipDevice_t dev = 0;
  hipError_t e = stream ? hipStreamGetDevice((hipStream_t)stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  void* ws = nullptr;
  int rc = scratch_for((int)dev, &ws);
  if (rc) return rc;
  const int64_t ws_bytes = (int64_t)kNoAllocScratchBytes;
  // The array keeps the previous call's contents: the split counters start every call at zero
  // (a fill kernel, not a memset node, so the call can also be captured).
  if ((rc = pkv_decode_workspace_init(ws, batch, stream))) return rc;
  int flags = 0;
  if (page_size == 16 && num_qo_heads % num_kv_heads == 0 &&
      decode_mfma_supported(dtype, head_dim, num_qo_heads / num_kv_heads, num_kv_heads, batch)) {
    if ((rc = pkv_decode_plan(kv_indptr, kv_indices, num_indices, kv_last_page_len, nullptr, batch, num_qo_heads,
                              num_kv_heads, head_dim, page_size, num_ctas, 0, ws, ws_bytes, stream)))
      return rc;
    flags = PKV_DECODE_PLANNED;
  }
  return pkv_batch_decode(q, q_stride_n, q_stride_h, k_cache, v_cache, page_stride, num_pages, kv_indptr,
                          kv_indices, num_indices, kv_last_page_len, batch, num_qo_heads, num_kv_heads,
                          head_dim, page_size, sm_scale, num_ctas, ws, ws_bytes, out, o_stride_n,
                          o_stride_h, dtype, flags, stream);
}
