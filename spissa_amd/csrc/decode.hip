// decode.hip -- single-token f32 attention against the resident KV cache
// (rotary.rs:335-415 with query_len == 1), as split-K flash-decoding for gfx950.
//
// Two kernels per launch:
//
// 1. decode_split_kernel covers the cached keys only. One workgroup
//    (256 threads, 4 waves) owns a range of cached keys ("split") of one KV
//    head for one sequence and serves RB query heads of that head's group, so
//    every K/V row is read from HBM once per head block. A key row (D floats)
//    is spread over LPR = D/8 lanes; a lane holds two float4 (dims
//    [4*sub, 4*sub+4) and [D/2 + 4*sub, ...)), so each load instruction of a
//    lane group moves a contiguous 16*LPR-byte piece of a row, and the lane's
//    two float4 are exactly rotate-half partners (RoPE of q is lane-local).
//    The 8-element partial dots are all-reduced over the row's LPR lanes with
//    DPP (quad_perm, row_half_mirror, row_mirror) and the gfx950
//    v_permlane16/32_swap exchanges; each row group runs an online softmax in
//    the log2 domain; the groups of a wave merge in registers (DPP row_ror:8,
//    permlane swaps), the four waves through one LDS exchange, and every
//    workgroup stores its partial (max, sum, unnormalised output).
//
// 2. decode_combine_kernel handles the new token itself (its optional RoPE,
//    its score and value), merges it with the splits' partials into the
//    normalised output, and optionally appends the new (rotated) key and
//    value to the cache row it occupies. The kernel boundary publishes the
//    partials across XCDs, so no in-kernel device-scope synchronisation is
//    needed, and a whole decode step of a layer (RoPE, attention, append) is
//    these two launches.
//
// Errors. A zero or non-finite softmax denominator (rotary.rs:560-564) sets a
// device error bit instead of aborting.
#include <cstdlib>

#include "internal.hpp"

namespace spissa {

namespace {

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xf, 0xf, false);
}

// Value of lane ^ 16 (v_permlane16_swap_b32) and of lane ^ 32 (v_permlane32_swap_b32).
__device__ __forceinline__ float xor16(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float xor32(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}
// Value of lane ^ 8 (DPP row_ror:8 within each 16-lane row).
__device__ __forceinline__ float xor8(float v) { return dpp<0x128>(v); }

template <int M>
__device__ __forceinline__ float lane_xor(float v) {
  if constexpr (M == 8) return xor8(v);
  else if constexpr (M == 16) return xor16(v);
  else return xor32(v);
}

// All-reduce (sum) over aligned groups of LPR lanes.
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(LPR >= 2 && LPR <= 64 && (LPR & (LPR - 1)) == 0, "LPR");
  v += dpp<0xB1>(v);                           // lane ^ 1  (quad_perm [1,0,3,2])
  if constexpr (LPR >= 4) v += dpp<0x4E>(v);   // lane ^ 2  (quad_perm [2,3,0,1])
  if constexpr (LPR >= 8) v += dpp<0x141>(v);  // quad <-> quad (row_half_mirror)
  if constexpr (LPR >= 16) v += dpp<0x140>(v); // 8 <-> 8 (row_mirror)
  if constexpr (LPR >= 32) v += xor16(v);      // row <-> row
  if constexpr (LPR >= 64) v += xor32(v);      // half <-> half
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
__device__ __forceinline__ float4 axpby4(float4 x, float a, float4 y, float b) {
  return make_float4(x.x * a + y.x * b, x.y * a + y.y * b, x.z * a + y.z * b, x.w * a + y.w * b);
}

constexpr float NEG_INF = -__builtin_inff();

__device__ __forceinline__ float safe_max(float m) { return m == NEG_INF ? 0.0f : m; }

// rotary.rs:467-481 on one (first, second) pair, each product rounded
// separately, so the result is bit-identical to the reference rotation.
__device__ __forceinline__ void rotate_pair(float &first, float &second, float c, float s) {
#pragma clang fp contract(off)
  const float a = first * c - second * s;
  const float b = second * c + first * s;
  first = a;
  second = b;
}

// Merges the online-softmax state of this lane with lane ^ M (same dims, other row group).
template <int RB, int M>
__device__ __forceinline__ void merge_with(float (&m)[RB], float (&l)[RB], float4 (&o)[RB][2]) {
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const float mp = lane_xor<M>(m[r]);
    const float lp = lane_xor<M>(l[r]);
    float4 op0, op1;
    op0.x = lane_xor<M>(o[r][0].x); op0.y = lane_xor<M>(o[r][0].y);
    op0.z = lane_xor<M>(o[r][0].z); op0.w = lane_xor<M>(o[r][0].w);
    op1.x = lane_xor<M>(o[r][1].x); op1.y = lane_xor<M>(o[r][1].y);
    op1.z = lane_xor<M>(o[r][1].z); op1.w = lane_xor<M>(o[r][1].w);
    const float mn = fmaxf(m[r], mp);
    const float ms = safe_max(mn);
    const float fa = fast_exp2(m[r] - ms), fb = fast_exp2(mp - ms);
    l[r] = l[r] * fa + lp * fb;
    o[r][0] = axpby4(o[r][0], fa, op0, fb);
    o[r][1] = axpby4(o[r][1], fa, op1, fb);
    m[r] = mn;
  }
}

}  // namespace

// At least 4 waves per SIMD (<= 128 VGPRs): four workgroups per CU stay resident.
template <int D, int RB, int RPG>
__global__ __launch_bounds__(256, 4) void decode_split_kernel(const DecodeArgs a) {
  constexpr int LPR = D / 8;
  constexpr int GPW = 64 / LPR;  // row groups per wave
  constexpr int NG = 4 * GPW;    // row groups per workgroup
  constexpr int HALF = D / 2;
  constexpr int ENTRY = RB * (D + 2);  // O[RB][D] then (max, sum)[RB]

  __shared__ float w_o[4][RB][D];
  __shared__ float w_ml[4][RB][2];

  // Head blocks are the fastest grid dimension: the workgroups that read the
  // same key rows (all KV heads of one split) are dispatched back to back.
  const int split = blockIdx.y;
  const int hb = blockIdx.x % a.HB;
  const int h = blockIdx.x / a.HB;
  const int b = blockIdx.z;
  const int P = a.seq[b].past;
  const int kstart = a.window > 0 ? max(0, P + 1 - a.window) : 0;
  const int nsplit = (P - kstart + a.kps - 1) / a.kps;  // cached keys only
  if (split >= nsplit) return;
  const int k0 = kstart + split * a.kps;
  const int k1 = min(P, k0 + a.kps);

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int sub = lane % LPR;
  const int grp = wave * GPW + lane / LPR;
  const int qh0 = h * a.R + hb * RB;

  const long row_stride = (long)a.Hkv * D;
  const float *kcache = a.seq[b].k + (long)h * D;
  const float *vcache = a.seq[b].v + (long)h * D;

  float4 qv[RB][2];
  {
    const float *qb = a.q + ((long)b * a.Hq + qh0) * D;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      qv[r][0] = ld4(qb + r * D + 4 * sub);
      qv[r][1] = ld4(qb + r * D + HALF + 4 * sub);
    }
    if (a.rope_cos) {
      const float4 c = ld4(a.rope_cos + (long)P * HALF + 4 * sub);
      const float4 sn = ld4(a.rope_sin + (long)P * HALF + 4 * sub);
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        rotate_pair(qv[r][0].x, qv[r][1].x, c.x, sn.x);
        rotate_pair(qv[r][0].y, qv[r][1].y, c.y, sn.y);
        rotate_pair(qv[r][0].z, qv[r][1].z, c.z, sn.z);
        rotate_pair(qv[r][0].w, qv[r][1].w, c.w, sn.w);
      }
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

  for (int c = k0; c < k1; c += NG * RPG) {
    float4 kr[RPG][2], vr[RPG][2];
    bool valid[RPG];
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
      const int j = c + grp + i * NG;
      valid[i] = j < k1;
      if (valid[i]) {
        const float *kp = kcache + (long)j * row_stride;
        const float *vp = vcache + (long)j * row_stride;
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
        const float s = group_sum<LPR>(dot8(qv[r][0], qv[r][1], kr[i][0], kr[i][1])) * a.qscale;
        sc[i][r] = valid[i] ? s : NEG_INF;
      }
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      float mx = m[r];
#pragma unroll
      for (int i = 0; i < RPG; ++i) mx = fmaxf(mx, sc[i][r]);
      const float ms = safe_max(mx);
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

  // ---- merge the row groups of each wave in registers ----
  if constexpr (GPW >= 8) merge_with<RB, 8>(m, l, o);
  if constexpr (GPW >= 4) merge_with<RB, 16>(m, l, o);
  if constexpr (GPW >= 2) merge_with<RB, 32>(m, l, o);
  // Lanes of row group 0 now hold the wave's state; merge the four waves in LDS.
  if (lane < LPR) {
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      *reinterpret_cast<float4 *>(&w_o[wave][r][4 * sub]) = o[r][0];
      *reinterpret_cast<float4 *>(&w_o[wave][r][HALF + 4 * sub]) = o[r][1];
      if (sub == 0) {
        w_ml[wave][r][0] = m[r];
        w_ml[wave][r][1] = l[r];
      }
    }
  }
  __syncthreads();

  const long bhh = ((long)b * a.Hkv + h) * a.HB + hb;
  float *dst = a.partial + (bhh * a.max_splits + split) * (long)ENTRY;
  for (int e = tid; e < RB * D; e += 256) {
    const int r = e / D;
    const float M = fmaxf(fmaxf(w_ml[0][r][0], w_ml[1][r][0]), fmaxf(w_ml[2][r][0], w_ml[3][r][0]));
    const float Ms = safe_max(M);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = fast_exp2(w_ml[w][r][0] - Ms);
      L += w_ml[w][r][1] * f;
      O += w_o[w][r][e % D] * f;
    }
    dst[e] = O;
    if ((e % D) == 0) {
      dst[RB * D + 2 * r] = M;
      dst[RB * D + 2 * r + 1] = L;
    }
  }
}

// Finishes the attention of one (sequence, KV head, head block): the new
// token's score and value, merged with the partials of every split of the
// cached keys, then the optional append of the new key and value.
// Grid: (RB*D / 64, Hkv*HB, B); 1024 threads = 64 consecutive outputs x 16
// split lanes. Each lane keeps an online (max, sum, output) over its splits
// with the loads of four splits in flight; the 16 lanes of every output are
// merged through LDS.
template <int D, int RB>
__global__ __launch_bounds__(1024) void decode_combine_kernel(const DecodeArgs a) {
  constexpr int HALF = D / 2;
  constexpr int ENTRY = RB * (D + 2);
  constexpr int OUTS = 64, SL = 16, UNROLL = 4;
  __shared__ float s_m[SL][OUTS], s_l[SL][OUTS], s_o[SL][OUTS];
  __shared__ float s_dot[RB * D / 64];
  __shared__ float s_new[RB];

  const int hb = blockIdx.y % a.HB;
  const int h = blockIdx.y / a.HB;
  const int b = blockIdx.z;
  const int P = a.seq[b].past;
  const int kstart = a.window > 0 ? max(0, P + 1 - a.window) : 0;
  const int nsplit = (P - kstart + a.kps - 1) / a.kps;
  const int tid = threadIdx.x;
  const int out = tid & (OUTS - 1);
  const int sl = tid / OUTS;
  const int e = blockIdx.x * OUTS + out;  // < RB*D: RB*D is a multiple of 64
  const int r = e / D;
  const int qh0 = h * a.R + hb * RB;
  const float *knew = a.cur_k + ((long)b * a.Hkv + h) * D;
  const float *vnew = a.cur_v + ((long)b * a.Hkv + h) * D;

  // ---- the new token: (rotated) q . (rotated) k for the RB query heads ----
  float kd = 0.0f;  // this thread's (rotated) key element, kept for the append
  if (tid < RB * D) {
    const int rr = tid / D, d = tid % D;
    const float *qrow = a.q + ((long)b * a.Hq + qh0 + rr) * D;
    float qd = qrow[d];
    kd = knew[d];
    if (a.rope_cos) {
      const int pair = d % HALF;
      const float c = a.rope_cos[(long)P * HALF + pair], sn = a.rope_sin[(long)P * HALF + pair];
      float q1 = qrow[pair], q2 = qrow[pair + HALF], k1 = knew[pair], k2 = knew[pair + HALF];
      rotate_pair(q1, q2, c, sn);
      rotate_pair(k1, k2, c, sn);
      qd = d < HALF ? q1 : q2;
      kd = d < HALF ? k1 : k2;
    }
    float prod = qd * kd;
    prod = group_sum<64>(prod);
    if ((tid & 63) == 0) s_dot[tid >> 6] = prod;
  }

  // ---- the cached keys: partials of the splits ----
  const long bhh = ((long)b * a.Hkv + h) * a.HB + hb;
  const float *ents = a.partial + bhh * a.max_splits * (long)ENTRY;
  float m = NEG_INF, l = 0.0f, o = 0.0f;
  for (int s0 = sl; s0 < nsplit; s0 += SL * UNROLL) {
    float ms[UNROLL], ls[UNROLL], os[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int s = s0 + u * SL;
      if (s < nsplit) {
        const float *ent = ents + (long)s * ENTRY;
        ms[u] = ent[RB * D + 2 * r];
        ls[u] = ent[RB * D + 2 * r + 1];
        os[u] = ent[e];
      } else {
        ms[u] = NEG_INF;
        ls[u] = 0.0f;
        os[u] = 0.0f;
      }
    }
    float mx = m;
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) mx = fmaxf(mx, ms[u]);
    const float mxs = safe_max(mx);
    const float f = fast_exp2(m - mxs);
    l *= f;
    o *= f;
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const float g = fast_exp2(ms[u] - mxs);
      l += ls[u] * g;
      o += os[u] * g;
    }
    m = mx;
  }
  s_m[sl][out] = m;
  s_l[sl][out] = l;
  s_o[sl][out] = o;
  __syncthreads();
  if (tid < RB) {
    float dot = 0.0f;
#pragma unroll
    for (int w = 0; w < D / 64; ++w) dot += s_dot[tid * (D / 64) + w];
    s_new[tid] = dot * a.qscale;
  }
  __syncthreads();
  if (sl == 0) {
    const float sn = s_new[r];
    float M = sn;
#pragma unroll
    for (int k = 0; k < SL; ++k) M = fmaxf(M, s_m[k][out]);
    const float Ms = safe_max(M);
    const float pn = fast_exp2(sn - Ms);
    float L = pn, O = pn * vnew[e % D];
#pragma unroll
    for (int k = 0; k < SL; ++k) {
      const float g = fast_exp2(s_m[k][out] - Ms);
      L += s_l[k][out] * g;
      O += s_o[k][out] * g;
    }
    a.out[((long)b * a.Hq + qh0) * D + e] = O / L;
    if ((e % D) == 0 && !(L > 0.0f && L < __builtin_inff())) atomicOr(a.err, kDevErrSoftmaxDenominator);
  }
  // ---- append the new (rotated) key and value at cache row P ----
  if (a.do_append && blockIdx.x == 0 && hb == 0 && tid < D) {
    const float vd = vnew[tid];
    a.app_k[b][(long)h * D + tid] = kd;
    a.app_v[b][(long)h * D + tid] = vd;
    if (a.app_kb[b]) {
      const long cap = a.app_cap[b];
      a.app_kb[b][((long)h * cap + P) * D + tid] = (bf16)kd;
      a.app_vt[b][((long)h * D + tid) * cap + P] = (bf16)vd;
    }
  }
}

namespace {
// Rows per lane group in flight: four, three for four query heads per block
// (keeps the split kernel within 128 VGPRs without spills).
constexpr int rows_per_group(int RB) { return RB >= 4 ? 3 : 4; }

template <int D, int RB>
hipError_t launch_one(hipStream_t st, const DecodeArgs &a) {
  if (a.max_splits > 0) {
    dim3 grid((unsigned)(a.Hkv * a.HB), (unsigned)a.max_splits, (unsigned)a.B);
    hipLaunchKernelGGL((decode_split_kernel<D, RB, rows_per_group(RB)>), grid, dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  dim3 cgrid((unsigned)(RB * D / 64), (unsigned)(a.Hkv * a.HB), (unsigned)a.B);
  hipLaunchKernelGGL((decode_combine_kernel<D, RB>), cgrid, dim3(1024), 0, st, a);
  return hipGetLastError();
}

template <int D>
hipError_t launch_d(hipStream_t st, const DecodeArgs &a, int RB) {
  switch (RB) {
    case 1: return launch_one<D, 1>(st, a);
    case 2: return launch_one<D, 2>(st, a);
    case 3: return launch_one<D, 3>(st, a);
    case 4: return launch_one<D, 4>(st, a);
    default: return hipErrorInvalidValue;
  }
}
}  // namespace

bool decode_supported(int D, int R) { return (D == 64 || D == 128 || D == 256) && R >= 1; }

int decode_keys_per_split(int D, int RB, long total_rows, int max_keys) {
  const int chunk = 4 * (64 / (D / 8)) * rows_per_group(RB);  // keys of one workgroup iteration
  static const long target = [] {
    const char *env = getenv("SPISSA_DECODE_TARGET_WGS");
    const long v = env ? atol(env) : 0;
    return v > 0 ? v : 1024L;
  }();
  const long per = (total_rows + target - 1) / target;
  long kps = ((per + chunk - 1) / chunk) * chunk;
  if (kps < chunk) kps = chunk;
  // Bound the partials the combine kernel reads per output.
  while ((max_keys + kps - 1) / kps > kMaxDecodeSplits) kps += chunk;
  return (int)kps;
}

hipError_t launch_decode(hipStream_t st, const DecodeArgs &a, int D, int RB) {
  switch (D) {
    case 64: return launch_d<64>(st, a, RB);
    case 128: return launch_d<128>(st, a, RB);
    case 256: return launch_d<256>(st, a, RB);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace spissa
