// decode.hip -- single-token f32 attention against the resident KV cache
// (rotary.rs:335-415 with query_len == 1), as split-K flash-decoding for gfx950.
//
// Work split. One workgroup (256 threads, 4 waves) owns a range of keys
// ("split") of one KV head for one sequence and serves RB query heads of that
// KV head's group, so each K/V row is read from HBM once per head block. A key
// row (D floats) is spread over LPR = D/8 lanes, each lane holding two float4
// (dims [4*sub, 4*sub+4) and [D/2 + 4*sub, ...)), so each load instruction
// moves contiguous 16*LPR-byte pieces of rows. A wave therefore streams 64/LPR
// rows at once, the workgroup NG = 4*64/LPR rows, and every lane keeps RPG rows
// of K and V in flight per iteration.
//
// Scores. The lane's 8-element partial dot is reduced over the row's LPR lanes
// with DPP (quad_perm, row_half_mirror, row_mirror) and the gfx950
// v_permlane16_swap / v_permlane32_swap exchanges: all-reduce, no LDS.
//
// Softmax. Each row group runs its own online softmax in the log2 domain
// (the scale 1/sqrt(D)*log2(e) is folded into q). Groups are merged through
// LDS at the end of the workgroup, splits are merged by a combine tree: the
// last-arriving workgroup of every kCombineFanIn siblings (atomic arrival
// counter) merges their partial (max, sum, output) entries, up to the root,
// which writes the normalised output. Counters reset themselves, so
// consecutive launches need no memset.
//
// Errors. A zero or non-finite softmax denominator (rotary.rs:560-564) sets a
// device error bit instead of aborting.
#include "internal.hpp"

namespace spissa {

namespace {

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xf, 0xf, false);
}

// Sum / max of v with the value of lane ^ 16 (v_permlane16_swap_b32).
__device__ __forceinline__ float swap16_sum(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap32_sum(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// All-reduce (sum) over aligned groups of LPR lanes.
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(LPR >= 2 && LPR <= 64 && (LPR & (LPR - 1)) == 0, "LPR");
  v += dpp<0xB1>(v);                              // lane ^ 1  (quad_perm [1,0,3,2])
  if constexpr (LPR >= 4) v += dpp<0x4E>(v);      // lane ^ 2  (quad_perm [2,3,0,1])
  if constexpr (LPR >= 8) v += dpp<0x141>(v);     // quad <-> quad (row_half_mirror)
  if constexpr (LPR >= 16) v += dpp<0x140>(v);    // 8 <-> 8 (row_mirror)
  if constexpr (LPR >= 32) v = swap16_sum(v);     // row <-> row
  if constexpr (LPR >= 64) v = swap32_sum(v);     // half <-> half
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

__device__ __forceinline__ float dot8(const float4 a0, const float4 a1, const float4 b0,
                                      const float4 b1) {
  float s = a0.x * b0.x;
  s = fmaf(a0.y, b0.y, s);
  s = fmaf(a0.z, b0.z, s);
  s = fmaf(a0.w, b0.w, s);
  s = fmaf(a1.x, b1.x, s);
  s = fmaf(a1.y, b1.y, s);
  s = fmaf(a1.z, b1.z, s);
  s = fmaf(a1.w, b1.w, s);
  return s;
}

__device__ __forceinline__ float4 scale4(float4 v, float s) {
  return make_float4(v.x * s, v.y * s, v.z * s, v.w * s);
}
__device__ __forceinline__ float4 fma4(float p, float4 v, float4 acc) {
  return make_float4(fmaf(p, v.x, acc.x), fmaf(p, v.y, acc.y), fmaf(p, v.z, acc.z),
                     fmaf(p, v.w, acc.w));
}

}  // namespace

int combine_tree_entries(int n) {
  int total = n;
  while (n > 1) {
    int groups = (n + kCombineFanIn - 1) / kCombineFanIn;
    if (groups > 1) total += groups;
    n = groups;
  }
  return total;
}

int combine_tree_counters(int n) {
  int total = 0;
  while (n > 1) {
    int groups = (n + kCombineFanIn - 1) / kCombineFanIn;
    total += groups;
    n = groups;
  }
  return total;
}

template <int D, int RB, int RPG>
__global__ __launch_bounds__(256) void decode_kernel(const DecodeArgs a) {
  constexpr int LPR = D / 8;
  constexpr int GPW = 64 / LPR;
  constexpr int NG = 4 * GPW;
  constexpr int HALF = D / 2;
  constexpr int ENTRY = RB * (D + 2);  // O[RB][D] then (max, sum)[RB]
  constexpr float NEG_INF = -__builtin_inff();

  __shared__ float red_o[NG][RB][D];
  __shared__ float red_m[NG][RB];
  __shared__ float red_l[NG][RB];
  __shared__ float fac[NG > kCombineFanIn ? NG : kCombineFanIn][RB];
  __shared__ float s_max[RB];
  __shared__ float s_sum[RB];
  __shared__ int s_last;

  const int split = blockIdx.x;
  const int hb = blockIdx.y % a.HB;
  const int h = blockIdx.y / a.HB;
  const int b = blockIdx.z;
  const int P = a.seq[b].past;
  const int kend = P + 1;
  const int kstart = a.window > 0 ? max(0, kend - a.window) : 0;
  const int nsplit = (kend - kstart + a.kps - 1) / a.kps;
  if (split >= nsplit) return;
  const int k0 = kstart + split * a.kps;
  const int k1 = min(kend, k0 + a.kps);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int sub = lane % LPR;
  const int grp = (tid >> 6) * GPW + lane / LPR;
  const int qh0 = h * a.R + hb * RB;

  float4 qv[RB][2];
  {
    const float *qb = a.q + ((long)b * a.Hq + qh0) * D;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      qv[r][0] = scale4(ld4(qb + r * D + 4 * sub), a.qscale);
      qv[r][1] = scale4(ld4(qb + r * D + HALF + 4 * sub), a.qscale);
    }
  }
  float m[RB], l[RB];
  float4 o[RB][2];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    m[r] = NEG_INF;
    l[r] = 0.0f;
    o[r][0] = make_float4(0.f, 0.f, 0.f, 0.f);
    o[r][1] = o[r][0];
  }

  const long row_stride = (long)a.Hkv * D;
  const float *kcache = a.seq[b].k;
  const float *vcache = a.seq[b].v;
  const float *knew = a.cur_k + ((long)b * a.Hkv + h) * D;
  const float *vnew = a.cur_v + ((long)b * a.Hkv + h) * D;

  for (int c = k0; c < k1; c += NG * RPG) {
    float4 kr[RPG][2], vr[RPG][2];
    bool valid[RPG];
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
      const int j = c + grp + i * NG;
      valid[i] = j < k1;
      if (valid[i]) {
        const float *kp = knew, *vp = vnew;
        if (j < P) {
          kp = kcache + (long)j * row_stride + (long)h * D;
          vp = vcache + (long)j * row_stride + (long)h * D;
        }
        kr[i][0] = ld4(kp + 4 * sub);
        kr[i][1] = ld4(kp + HALF + 4 * sub);
        vr[i][0] = ld4(vp + 4 * sub);
        vr[i][1] = ld4(vp + HALF + 4 * sub);
      } else {
        kr[i][0] = kr[i][1] = vr[i][0] = vr[i][1] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    float sc[RPG][RB];
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        float s = group_sum<LPR>(dot8(qv[r][0], qv[r][1], kr[i][0], kr[i][1]));
        sc[i][r] = valid[i] ? s : NEG_INF;
      }
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      float mx = m[r];
#pragma unroll
      for (int i = 0; i < RPG; ++i) mx = fmaxf(mx, sc[i][r]);
      const float ms = mx == NEG_INF ? 0.0f : mx;
      const float alpha = fast_exp2(m[r] - ms);
      l[r] *= alpha;
      o[r][0] = scale4(o[r][0], alpha);
      o[r][1] = scale4(o[r][1], alpha);
#pragma unroll
      for (int i = 0; i < RPG; ++i) {
        const float p = fast_exp2(sc[i][r] - ms);
        l[r] += p;
        o[r][0] = fma4(p, vr[i][0], o[r][0]);
        o[r][1] = fma4(p, vr[i][1], o[r][1]);
      }
      m[r] = mx;
    }
  }

  // ---- merge the NG row groups of this workgroup ----
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    *reinterpret_cast<float4 *>(&red_o[grp][r][4 * sub]) = o[r][0];
    *reinterpret_cast<float4 *>(&red_o[grp][r][HALF + 4 * sub]) = o[r][1];
    if (sub == 0) {
      red_m[grp][r] = m[r];
      red_l[grp][r] = l[r];
    }
  }
  __syncthreads();
  if (tid < RB) {
    float M = NEG_INF;
    for (int g = 0; g < NG; ++g) M = fmaxf(M, red_m[g][tid]);
    s_max[tid] = M;
  }
  __syncthreads();
  if (tid < NG * RB) {
    const int g = tid / RB, r = tid % RB;
    const float M = s_max[r];
    fac[g][r] = fast_exp2(red_m[g][r] - (M == NEG_INF ? 0.0f : M));
  }
  __syncthreads();
  if (tid < RB) {
    float L = 0.0f;
    for (int g = 0; g < NG; ++g) L += red_l[g][tid] * fac[g][tid];
    s_sum[tid] = L;
  }
  // Each thread owns outputs e = tid + 256*u of the RB*D block.
  constexpr int PER = (RB * D + 255) / 256;
  float acc[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int e = tid + 256 * u;
    float s = 0.0f;
    if (e < RB * D) {
      const int r = e / D, dim = e % D;
      for (int g = 0; g < NG; ++g) s += red_o[g][r][dim] * fac[g][r];
    }
    acc[u] = s;
  }
  __syncthreads();

  const long bhh = ((long)b * a.Hkv + h) * a.HB + hb;
  float *out = a.out + ((long)b * a.Hq + qh0) * D;

  auto finalize = [&]() {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int e = tid + 256 * u;
      if (e < RB * D) {
        const float L = s_sum[e / D];
        out[e] = acc[u] / L;
        if ((e % D) == 0 && !(L > 0.0f && L < __builtin_inff())) atomicOr(a.err, kDevErrSoftmaxDenominator);
      }
    }
  };

  if (nsplit == 1) {
    finalize();
    return;
  }

  float *ebase = a.partial + bhh * (long)a.max_entries * ENTRY;
  int *cbase = a.counters + bhh * a.max_counters;
  auto write_entry = [&](int slot) {
    float *ent = ebase + (long)slot * ENTRY;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int e = tid + 256 * u;
      if (e < RB * D) ent[e] = acc[u];
    }
    if (tid < RB) {
      ent[RB * D + 2 * tid] = s_max[tid];
      ent[RB * D + 2 * tid + 1] = s_sum[tid];
    }
  };

  int n = nsplit, idx = split, eoff = 0, coff = 0;
  write_entry(idx);
  while (n > 1) {
    const int groups = (n + kCombineFanIn - 1) / kCombineFanIn;
    const int g = idx / kCombineFanIn;
    const int first = g * kCombineFanIn;
    const int cnt = min(kCombineFanIn, n - first);
    __threadfence();
    __syncthreads();
    if (tid == 0) {
      const int old = atomicAdd(&cbase[coff + g], 1);
      s_last = (old == cnt - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    if (tid == 0) atomicExch(&cbase[coff + g], 0);
    const float *ents = ebase + (long)(eoff + first) * ENTRY;
    if (tid < RB) {
      float M = NEG_INF;
      for (int k = 0; k < cnt; ++k) M = fmaxf(M, ents[(long)k * ENTRY + RB * D + 2 * tid]);
      s_max[tid] = M;
    }
    __syncthreads();
    if (tid < cnt * RB) {
      const int k = tid / RB, r = tid % RB;
      const float M = s_max[r];
      fac[k][r] = fast_exp2(ents[(long)k * ENTRY + RB * D + 2 * r] - (M == NEG_INF ? 0.0f : M));
    }
    __syncthreads();
    if (tid < RB) {
      float L = 0.0f;
      for (int k = 0; k < cnt; ++k) L += ents[(long)k * ENTRY + RB * D + 2 * tid + 1] * fac[k][tid];
      s_sum[tid] = L;
    }
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int e = tid + 256 * u;
      float s = 0.0f;
      if (e < RB * D) {
        const int r = e / D;
        for (int k = 0; k < cnt; ++k) s += ents[(long)k * ENTRY + e] * fac[k][r];
      }
      acc[u] = s;
    }
    __syncthreads();
    if (groups == 1) {
      finalize();
      return;
    }
    eoff += n;
    coff += groups;
    idx = g;
    n = groups;
    write_entry(eoff + idx);
  }
}

namespace {
constexpr int kRowsPerGroup = 4;

template <int D, int RB>
hipError_t launch_one(hipStream_t st, const DecodeArgs &a, int max_splits) {
  dim3 grid((unsigned)max_splits, (unsigned)(a.Hkv * a.HB), (unsigned)a.B);
  hipLaunchKernelGGL((decode_kernel<D, RB, kRowsPerGroup>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

template <int D>
hipError_t launch_d(hipStream_t st, const DecodeArgs &a, int RB, int max_splits) {
  switch (RB) {
    case 1: return launch_one<D, 1>(st, a, max_splits);
    case 2: return launch_one<D, 2>(st, a, max_splits);
    case 3: return launch_one<D, 3>(st, a, max_splits);
    case 4: return launch_one<D, 4>(st, a, max_splits);
    default: return hipErrorInvalidValue;
  }
}
}  // namespace

bool decode_supported(int D, int R) { return (D == 64 || D == 128 || D == 256) && R >= 1; }

int decode_keys_per_split(int D, int RB, long total_rows, int max_keys) {
  (void)RB;
  const int chunk = 4 * (64 / (D / 8)) * kRowsPerGroup;  // keys one workgroup iteration covers
  static long target = [] {
    const char *env = getenv("SPISSA_DECODE_TARGET_WGS");
    long v = env ? atol(env) : 0;
    return v > 0 ? v : 2048L;
  }();
  long per = (total_rows + target - 1) / target;
  long iters = (per + chunk - 1) / chunk;
  if (iters < 1) iters = 1;
  long kps = iters * chunk;
  // Keep the combine tree shallow: at most kCombineFanIn^2 splits per (sequence, head).
  while ((max_keys + kps - 1) / kps > kCombineFanIn * kCombineFanIn) kps += chunk;
  return (int)kps;
}

hipError_t launch_decode(hipStream_t st, const DecodeArgs &a, int D, int RB, int max_splits) {
  switch (D) {
    case 64: return launch_d<64>(st, a, RB, max_splits);
    case 128: return launch_d<128>(st, a, RB, max_splits);
    case 256: return launch_d<256>(st, a, RB, max_splits);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace spissa
