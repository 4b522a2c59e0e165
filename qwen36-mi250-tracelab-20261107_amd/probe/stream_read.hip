// Measurement probe, not part of the MoE path: a plain streaming read of device memory, the
// practical read ceiling that bench.py --hbm-ceiling sets beside the 8 TB/s peak.
//
// Each lane keeps 8 independent 16-byte loads in flight (consecutive lanes read consecutive
// 16 bytes, so a wave reads 1 KiB per load instruction); the grid strides over the buffer.
// The loaded words are folded into one value per lane that is stored only when it equals a
// value the data never gives, so the loads cannot be dropped.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 8;

__global__ __launch_bounds__(kThreads) void k_stream_read(const uint4* __restrict__ p,
                                                          long long n16, uint32_t* sink) {
  const long long step = (long long)gridDim.x * kThreads * kUnroll;
  long long i = (long long)blockIdx.x * kThreads * kUnroll + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (kUnroll - 1) * kThreads < n16; i += step) {
    uint4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = p[i + u * kThreads];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (int u = 0; u < kUnroll; ++u) {  // the last partial stride
    const long long j = i + u * kThreads;
    if (j < n16) {
      const uint4 v = p[j];
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  }
  if (acc == 0x9e3779b9u) sink[blockIdx.x * kThreads + threadIdx.x] = acc;
}

}  // namespace

// Reads `bytes` (a multiple of 16) from src with `blocks` workgroups of 256 lanes on
// `stream`; sink holds blocks * 256 uint32 (written only in the impossible case above).
// Returns 0, or 1 for bad arguments, 2 when the launch fails.
extern "C" int moe_probe_stream_read(const void* src, long long bytes, void* sink, int blocks,
                                     void* stream) {
  if (!src || !sink || bytes <= 0 || bytes % 16 || blocks <= 0) return 1;
  hipLaunchKernelGGL(k_stream_read, dim3(blocks), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint4*>(src),
                     bytes / 16, static_cast<uint32_t*>(sink));
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
