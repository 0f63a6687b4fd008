// A streaming read of device memory, to measure the HBM read rate a launch of a given size
// and workgroup count reaches on this chip (the achievable bandwidth that the decode's bytes
// per second are set beside; the nominal 8 TB/s is the datasheet's).  No counterpart in the
// reference.
//
// Workgroup b (1024 threads) reads its contiguous slice of the buffer with 16-byte non-temporal
// loads, eight in flight per thread (128 KB per workgroup, so that one workgroup per CU is not
// starved by the memory latency), and folds what it read into one word per thread; a word that
// happens to equal a fixed constant is OR-ed into *sink (so the loads are not optimised away).
#include "common.h"
#include "../../include/pagedkv.h"

using namespace pkv;

namespace {

constexpr int kProbeThreads = 1024, kProbeUnroll = 8;
constexpr uint32_t kProbeMagic = 0x9E3779B9u;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                                    int64_t per16, uint32_t* sink) {
  const int64_t b0 = (int64_t)blockIdx.x * per16;
  const int64_t b1 = b0 + per16 < n16 ? b0 + per16 : n16;
  uint32_t acc = 0;
  for (int64_t i = b0 + threadIdx.x; i < b1; i += kProbeUnroll * kProbeThreads) {
    u32x4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) {
      const int64_t k = i + (int64_t)u * kProbeThreads;
      v[u] = k < b1 ? __builtin_nontemporal_load(src + k) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == kProbeMagic) atomicOr(sink, 1u);
}

}  // namespace

extern "C" int pkv_probe_stream_read(const void* src, int64_t bytes, int32_t blocks, uint32_t* sink,
                                     void* stream) {
  if (!src || !sink || bytes <= 0 || bytes % 16 || (uintptr_t)src % 16 || blocks <= 0) return kBadArg;
  const int64_t n16 = bytes / 16;
  const int64_t per16 = (n16 + blocks - 1) / blocks;
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(kProbeThreads), 0, (hipStream_t)stream,
                     reinterpret_cast<const u32x4*>(src), n16, per16, sink);
  return (int)hipGetLastError();
}
