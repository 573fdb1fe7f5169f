// sampling.hip -- the greedy token choice over device logits:
// crates/spissa-runtime/src/ops.rs:309-324 sample_argmax and ops.rs:326-348
// sample_argmax_excluding.
//
// Both reference functions are sequential scans, and their results are
// reproduced exactly, NaN and signed-zero cases included:
//  - sample_argmax keeps element 0 and replaces it only by a strictly
//    greater value. A NaN never compares greater, so a NaN at index 0 is the
//    answer, and NaNs elsewhere are never chosen; otherwise the answer is the
//    first index of the largest non-NaN value (-0.0 and +0.0 tie, so the
//    earlier one wins).
//  - sample_argmax_excluding (0 <= excluded < n, n >= 2) skips `excluded`
//    and replaces the best unless `value <= best`. With no NaN that is again
//    the first maximum. A NaN always replaces, and the element after a NaN
//    always replaces it, so the answer is the first maximum among the
//    elements after the last NaN, or that NaN's index when none follows.
//
// Phase 1 (argmax_partial_kernel): workgroup b scans the contiguous range
// [b * per_block, (b + 1) * per_block) and writes the first maximum over its
// non-NaN, non-excluded elements and its last NaN index. Phase 2
// (argmax_final_kernel, one workgroup) combines the ranges in order; only the
// excluding form with a NaN present rescans the suffix after the last NaN.
#include <climits>

#include "internal.hpp"

namespace spissa {

namespace {

struct Best {
  float v;
  int i;  // INT_MAX: none yet
};

// Strictly greater, or equal at a smaller index; a NaN is never better.
__device__ __forceinline__ bool better(float v, int i, const Best &b) { return v > b.v || (v == b.v && i < b.i); }

__device__ __forceinline__ void take(Best &b, float v, int i) {
  if (better(v, i, b)) {
    b.v = v;
    b.i = i;
  }
}

__device__ __forceinline__ void see(Best &b, int &last_nan, float v, int i, int excl) {
  if (i == excl) return;
  if (v != v) last_nan = i > last_nan ? i : last_nan;
  take(b, v, i);
}

// Combines over the 256 threads of a workgroup; every thread receives it.
__device__ Best block_best(Best b, int &last_nan) {
  __shared__ float sv[4];
  __shared__ int si[4], sn[4];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(b.v, off);
    const int oi = __shfl_xor(b.i, off);
    const int on = __shfl_xor(last_nan, off);
    take(b, ov, oi);
    last_nan = on > last_nan ? on : last_nan;
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = b.v;
    si[wave] = b.i;
    sn[wave] = last_nan;
  }
  __syncthreads();
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    take(b, sv[w], si[w]);
    last_nan = sn[w] > last_nan ? sn[w] : last_nan;
  }
  __syncthreads();
  return b;
}

}  // namespace

// Grid: ceil(n / per_block) workgroups of 256 threads; per_block is a
// multiple of 1024. vec: x is 16-byte aligned.
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *__restrict__ x, int n, int excl,
                                                             int per_block, int vec,
                                                             ArgmaxPart *__restrict__ parts) {
  const int start = blockIdx.x * per_block;
  const int end = start + min(per_block, n - start);
  Best b{-INFINITY, INT_MAX};
  int last_nan = -1;
  for (int i = start + 4 * (int)threadIdx.x; i < end; i += 1024) {
    if (vec && i + 4 <= end) {
      const float4 q = *reinterpret_cast<const float4 *>(x + i);
      see(b, last_nan, q.x, i, excl);
      see(b, last_nan, q.y, i + 1, excl);
      see(b, last_nan, q.z, i + 2, excl);
      see(b, last_nan, q.w, i + 3, excl);
    } else {
      for (int j = i; j < min(i + 4, end); ++j) see(b, last_nan, x[j], j, excl);
    }
  }
  b = block_best(b, last_nan);
  if (threadIdx.x == 0) parts[blockIdx.x] = ArgmaxPart{b.v, b.i, last_nan, 0};
}

// One workgroup of 256 threads. excl < 0: sample_argmax; otherwise
// sample_argmax_excluding with 0 <= excl < n and n >= 2.
__global__ __launch_bounds__(256) void argmax_final_kernel(const float *__restrict__ x, int n, int excl,
                                                           const ArgmaxPart *__restrict__ parts, int nparts,
                                                           int *__restrict__ token) {
  Best b{-INFINITY, INT_MAX};
  int last_nan = -1;
  for (int p = threadIdx.x; p < nparts; p += 256) {
    const ArgmaxPart q = parts[p];
    take(b, q.v, q.i);
    last_nan = q.last_nan > last_nan ? q.last_nan : last_nan;
  }
  b = block_best(b, last_nan);
  int result;
  if (excl < 0) {
    // sample_argmax: element 0 is the starting best and a NaN there stays
    const float x0 = x[0];
    result = (x0 != x0) ? 0 : b.i;
  } else if (last_nan < 0) {
    result = b.i;
  } else {
    // first maximum after the last NaN, else the NaN itself
    Best s{-INFINITY, INT_MAX};
    int unused = -1;
    for (int i = last_nan + 1 + (int)threadIdx.x; i < n; i += 256)
      if (i != excl) take(s, x[i], i);
    s = block_best(s, unused);
    result = s.i == INT_MAX ? last_nan : s.i;
  }
  if (threadIdx.x == 0) *token = result;
}

hipError_t launch_argmax(hipStream_t st, const float *x, int n, int excl, ArgmaxPart *parts, int *token) {
  const long blocks = ((long)n + 1023) / 1024;
  const long per_block = 1024 * ((blocks + kArgmaxMaxParts - 1) / kArgmaxMaxParts);
  const int nparts = (int)(((long)n + per_block - 1) / per_block);
  const int vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(nparts), dim3(256), 0, st, x, n, excl, (int)per_block, vec,
                     parts);
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, st, x, n, excl, parts, nparts, token);
  return hipGetLastError();
}

}  // namespace spissa
