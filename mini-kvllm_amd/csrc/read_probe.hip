// Streaming-read probe: the HBM read rate a plain kernel reaches on this GPU,
// the measured on-box ceiling that the decode kernels' read rate is set
// against (the 8 TB/s datasheet figure is not reached by any read stream).
// No reference counterpart: measurement only.
//
// Every lane reads 16-byte chunks with non-temporal loads (the decode's KV
// load type), up to kProbeUnroll of them in flight, grid-stride over the buffer; a
// wave folds what it read into one dword (XOR) written to its sink word, so
// the loads cannot be dropped.  Nothing else is written.
#include "mkv_device.hpp"

namespace mkv {
namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 16;

__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(const u32x4* __restrict__ p,
                                                                    int64_t n16,
                                                                    uint32_t* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * kProbeThreads;
  int64_t i = (int64_t)blockIdx.x * kProbeThreads + threadIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + (kProbeUnroll - 1) * stride < n16; i += kProbeUnroll * stride) {
    u32x4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u];
  }
  for (; i < n16; i += stride) acc ^= __builtin_nontemporal_load(p + i);
  uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x ^= (uint32_t)__shfl_xor((int)x, off);
  if ((threadIdx.x & 63) == 0) sink[(int64_t)blockIdx.x * (kProbeThreads / kWave) + (threadIdx.x >> 6)] = x;
}

}  // namespace
}  // namespace mkv

extern "C" size_t mkv_stream_read_probe_sink_words(int grid) {
  return grid > 0 ? (size_t)grid * (mkv::kProbeThreads / mkv::kWave) : 0;
}

extern "C" int mkv_stream_read_probe(const void* buf, int64_t bytes, uint32_t* sink, int grid,
                                     void* stream) {
  if (bytes < 0 || grid <= 0 || grid > (1 << 20)) return MKV_ERR_BAD_SHAPE;
  if (bytes % 16) return MKV_ERR_BAD_SHAPE;
  if (!buf || !sink) return MKV_ERR_NULL_POINTER;
  if (reinterpret_cast<uintptr_t>(buf) & 15u) return MKV_ERR_MISALIGNED;
  hipLaunchKernelGGL(mkv::stream_read_kernel, dim3((unsigned)grid), dim3(mkv::kProbeThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const mkv::u32x4*>(buf),
                     bytes / 16, sink);
  return (int)hipGetLastError();
}
