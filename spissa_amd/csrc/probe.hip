// probe.hip -- the streaming-read ceiling of the device: every 16-byte piece
// of a buffer read exactly once with non-temporal 128-bit loads, as the decode
// kernels read the KV cache, and nothing else. Its measured rate at the decode
// working-set sizes (one layer's 67 MB of K/V, and 1 GB) is the achievable
// bound the decode kernels are compared with, beside the HBM3E spec peak.
#include "internal.hpp"

namespace spissa {

namespace {
constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 8;  // 16-byte loads in flight per thread
}  // namespace

// Each thread reads kProbeUnroll pieces strided by the grid's thread count, so
// a wave's loads of one round are 1 KB contiguous; one round covers the buffer
// (the grid is sized for it). The sum lands in `sink` only if it equals a value
// it practically never takes, which keeps the loads without a store per thread.
__global__ __launch_bounds__(kProbeThreads) void hbm_read_kernel(const float4 *__restrict__ p, long n4,
                                                                  float *__restrict__ sink) {
  typedef __attribute__((ext_vector_type(4))) float f32x4v;
  const long stride = (long)gridDim.x * kProbeThreads;
  const long i0 = (long)blockIdx.x * kProbeThreads + threadIdx.x;
  f32x4v acc = {0.f, 0.f, 0.f, 0.f};
  f32x4v v[kProbeUnroll];
#pragma unroll
  for (int u = 0; u < kProbeUnroll; ++u) {
    const long i = i0 + u * stride;
    v[u] = i < n4 ? __builtin_nontemporal_load(reinterpret_cast<const f32x4v *>(p) + i) : f32x4v{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int u = 0; u < kProbeUnroll; ++u) acc += v[u];
  const float s = (acc.x + acc.y) + (acc.z + acc.w);
  if (s == 1.2345678e-30f) sink[0] = s;
}

hipError_t launch_hbm_read(hipStream_t st, const void *buf, size_t bytes, float *sink) {
  const long n4 = (long)(bytes / 16);
  if (n4 <= 0) return hipSuccess;
  const long per_block = (long)kProbeThreads * kProbeUnroll;
  const long blocks = (n4 + per_block - 1) / per_block;
  if (blocks > 0x7fffffffL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(hbm_read_kernel, dim3((unsigned)blocks), dim3(kProbeThreads), 0, st,
                     reinterpret_cast<const float4 *>(buf), n4, sink);
  return hipGetLastError();
}

}  // namespace spissa
