// generic.hip -- f32 SIMT attention for any head_dim and query length
// (rotary.rs:335-415, plus the sliding-window extension). It serves head
// dimensions the tuned kernels do not instantiate and the f32 prefill
// precision. One 256-thread workgroup per (query position, query head) walks
// the visible keys in chunks of 256: each thread scores one key (sequential f32
// dot over head_dim), the chunk's max and sum are block-reduced, and threads
// then accumulate the output over head dimensions with an online softmax.
#include "internal.hpp"

namespace spissa {

namespace {
constexpr int kThreads = 256;
constexpr int kMaxDim = 1024;

__device__ __forceinline__ float block_max(float v, float *red) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < kThreads / 64; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}

__device__ __forceinline__ float block_sum(float v, float *red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < kThreads / 64; ++i) r += red[i];
  __syncthreads();
  return r;
}
}  // namespace

__global__ __launch_bounds__(kThreads) void generic_attention_kernel(const GenericArgs a) {
  constexpr float NEG_INF = -__builtin_inff();
  constexpr int PER = kMaxDim / kThreads;
  __shared__ float qs[kMaxDim];
  __shared__ float ps[kThreads];
  __shared__ float red[kThreads / 64];

  const int head = blockIdx.x % a.Hq;
  const int qpos = blockIdx.x / a.Hq;
  const int kvh = head / a.R;
  const int q_abs = a.P + qpos;
  const int D = a.D;
  const int kend = a.causal ? q_abs + 1 : a.P + a.S;
  const int kbeg = a.window > 0 ? max(0, q_abs - a.window + 1) : 0;
  const int tid = threadIdx.x;

  const float *qrow = a.q + ((long)qpos * a.Hq + head) * D;
  for (int d = tid; d < D; d += kThreads) qs[d] = qrow[d];
  __syncthreads();

  float m = NEG_INF, l = 0.0f;
  float o[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) o[u] = 0.0f;

  for (int c = kbeg; c < kend; c += kThreads) {
    const int j = c + tid;
    float s = NEG_INF;
    if (j < kend) {
      const float *krow = j < a.P ? a.cache_k + ((long)j * a.Hkv + kvh) * D
                                  : a.cur_k + ((long)(j - a.P) * a.Hkv + kvh) * D;
      float dot = 0.0f;
      for (int d = 0; d < D; ++d) dot = fmaf(qs[d], krow[d], dot);
      s = dot * a.scale;
    }
    const float tmax = block_max(s, red);
    const float mnew = fmaxf(m, tmax);
    const float msafe = mnew == NEG_INF ? 0.0f : mnew;
    const float alpha = expf(m - msafe);
    const float p = expf(s - msafe);
    ps[tid] = p;
    const float psum = block_sum(p, red);  // its barriers also publish ps[]
    l = l * alpha + psum;
    const int n = min(kThreads, kend - c);
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int d = tid + u * kThreads;
      if (d < D) {
        float acc = o[u] * alpha;
        for (int jj = 0; jj < n; ++jj) {
          const int key = c + jj;
          const float *vrow = key < a.P ? a.cache_v + ((long)key * a.Hkv + kvh) * D
                                        : a.cur_v + ((long)(key - a.P) * a.Hkv + kvh) * D;
          acc = fmaf(ps[jj], vrow[d], acc);
        }
        o[u] = acc;
      }
    }
    m = mnew;
    __syncthreads();
  }
  if (tid == 0 && !(l > 0.0f && l < __builtin_inff())) atomicOr(a.err, kDevErrSoftmaxDenominator);
  float *orow = a.out + ((long)qpos * a.Hq + head) * D;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int d = tid + u * kThreads;
    if (d < D) orow[d] = o[u] / l;
  }
}

hipError_t launch_generic(hipStream_t st, const GenericArgs &a) {
  if (a.D > kMaxDim) return hipErrorInvalidValue;
  const long blocks = (long)a.S * a.Hq;
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(generic_attention_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

}  // namespace spissa
