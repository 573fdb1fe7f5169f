// probe.hip -- two ceilings of the device, measured beside the spec peaks:
//  - the streaming read: every 16-byte piece of a buffer read exactly once
//    with non-temporal 128-bit loads, as the decode kernels read the KV
//    cache, and nothing else (at one layer's 67 MB of K/V and at 1 GB), the
//    achievable bound of the decode kernels;
//  - the dense bf16 MFMA rate: waves that issue independent
//    v_mfma_f32_32x32x16_bf16 from registers on non-trivial operands, two per
//    SIMD on every CU, with no memory traffic; what the chip sustains under
//    that load (clock and power limits included) bounds the prefill kernels.
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

namespace {
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
constexpr int kMfmaChains = 8;  // independent accumulators per wave
}  // namespace

// `rounds` x kMfmaChains MFMAs per wave; the operands are lane-dependent
// values of both signs (MFMA power depends on the data). The accumulators'
// sum lands in `sink` only if it equals a value it practically never takes.
__global__ __launch_bounds__(kProbeThreads, 2) void mfma_rate_kernel(int rounds, float *__restrict__ sink) {
  const int lane = threadIdx.x & 63;
  bf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(0.125f * (float)(((lane * 7 + i * 13 + blockIdx.x) % 17) - 8));
    b[i] = (__bf16)(0.0625f * (float)(((lane * 5 + i * 11 + threadIdx.x / 64) % 19) - 9));
  }
  f32x16 acc[kMfmaChains];
#pragma unroll
  for (int j = 0; j < kMfmaChains; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;
  for (int r = 0; r < rounds; ++r) {
#pragma unroll
    for (int j = 0; j < kMfmaChains; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < kMfmaChains; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[j][e];
  if (s == 1.2345678e-30f) sink[0] = s;
}

hipError_t launch_mfma_rate(hipStream_t st, int cus, int rounds, float *sink, double *flop) {
  if (rounds <= 0 || cus <= 0) return hipErrorInvalidValue;
  const long blocks = 2L * cus;  // two four-wave workgroups per CU: two waves per SIMD
  hipLaunchKernelGGL(mfma_rate_kernel, dim3((unsigned)blocks), dim3(kProbeThreads), 0, st, rounds, sink);
  *flop = (double)blocks * (kProbeThreads / 64) * rounds * kMfmaChains * 32.0 * 32.0 * 16.0 * 2.0;
  return hipGetLastError();
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
