// decode.hip -- single-token f32 attention against the resident KV cache
// (rotary.rs:335-415 with query_len == 1), as split-K flash-decoding for gfx950.
//
// Two kernels per launch:
//
// 1. decode_split_kernel covers the keys. One workgroup
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
//    workgroup stores its partial (max, sum, unnormalised output). Split 0
//    of a sequence (dispatched first) also takes the new token: its key
//    (QK-normed and rotated in registers when those are fused) and value
//    join as one more row, and with the fused append that workgroup writes
//    them to cache row P, which no split reads.
//
// 2. decode_combine_kernel merges the splits' partials into the normalised
//    output. The kernel boundary publishes the partials across XCDs, so no
//    in-kernel device-scope synchronisation is needed, and a whole decode
//    step of a layer (RoPE, attention, append) is these two launches.
//
// Errors. A zero or non-finite softmax denominator (rotary.rs:560-564) sets a
// device error bit instead of aborting.
#include <algorithm>
#include <cstdlib>

#include "internal.hpp"

namespace spissa {

namespace {

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xf, 0xf, false);
}

// Source operand of a DPP add (all source lanes are valid for these controls,
// so `old` is never read; 0 lets the compiler fold it into v_add_f32_dpp).
template <int CTRL>
__device__ __forceinline__ float dpp0(float v) {
  return __builtin_amdgcn_update_dpp(0.0f, v, CTRL, 0xf, 0xf, false);
}

// Sum / max of v with the value of lane ^ 16 or lane ^ 32 (one permlane swap).
__device__ __forceinline__ float sum16(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum32(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max16(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max32(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// All-reduce (sum) over aligned groups of LPR lanes.
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(LPR >= 2 && LPR <= 64 && (LPR & (LPR - 1)) == 0, "LPR");
  v += dpp0<0xB1>(v);                           // lane ^ 1  (quad_perm [1,0,3,2])
  if constexpr (LPR >= 4) v += dpp0<0x4E>(v);   // lane ^ 2  (quad_perm [2,3,0,1])
  if constexpr (LPR >= 8) v += dpp0<0x141>(v);  // quad <-> quad (row_half_mirror)
  if constexpr (LPR >= 16) v += dpp0<0x140>(v); // 8 <-> 8 (row_mirror)
  if constexpr (LPR >= 32) v = sum16(v);        // row <-> row
  if constexpr (LPR >= 64) v = sum32(v);        // half <-> half
  return v;
}

// Max over the row groups of a wave (lanes l, l ^ LPR, l ^ 2 LPR, ...), for a
// value that is uniform within each group of LPR lanes.
template <int LPR>
__device__ __forceinline__ float groups_max(float v) {
  if constexpr (LPR <= 8) v = fmaxf(v, __builtin_amdgcn_update_dpp(v, v, 0x128, 0xf, 0xf, false));  // row_ror:8
  if constexpr (LPR <= 16) v = max16(v);
  if constexpr (LPR <= 32) v = max32(v);
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
// A cached K/V row is read once per step (by the head blocks of one KV head
// at about the same time): a non-temporal load, so the stream does not
// displace other cached lines (4-7% faster measured at batch 1).
__device__ __forceinline__ float4 ld4_stream(const char *p) {
  typedef __attribute__((ext_vector_type(4))) float f32x4v;
  const f32x4v q = __builtin_nontemporal_load(reinterpret_cast<const f32x4v *>(p));
  return make_float4(q.x, q.y, q.z, q.w);
}

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
__device__ __forceinline__ float4 mul4(float4 a, float4 b) {
  return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
}
__device__ __forceinline__ float4 fma4(float p, float4 v, float4 acc) {
  return make_float4(fmaf(p, v.x, acc.x), fmaf(p, v.y, acc.y), fmaf(p, v.z, acc.z),
                     fmaf(p, v.w, acc.w));
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

// The rotation of a lane's two float4 (dims [4s, 4s+4) and [D/2 + 4s, ...),
// rotate-half partners) by the table's cos/sin of those pairs.
__device__ __forceinline__ void rotate4(float4 &x0, float4 &x1, const float4 c, const float4 s) {
  rotate_pair(x0.x, x1.x, c.x, s.x);
  rotate_pair(x0.y, x1.y, c.y, s.y);
  rotate_pair(x0.z, x1.z, c.z, s.z);
  rotate_pair(x0.w, x1.w, c.w, s.w);
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

  __shared__ float red_o[NG][RB][D];
  __shared__ float red_l[NG][RB];
  __shared__ float wave_m[4][RB];
  __shared__ __attribute__((aligned(16))) float knorm_sq[D];  // squares of the new key (fused QK-norm)

  // Head blocks are the fastest grid dimension: the workgroups that read the
  // same key rows (all KV heads of one split) are dispatched back to back.
  const int split = blockIdx.y;
  const int hb = blockIdx.x % a.HB;
  const int h = blockIdx.x / a.HB;
  const int b = blockIdx.z;
  const int P = a.seq[b].past;
  const int kstart = a.window > 0 ? max(0, P + 1 - a.window) : 0;
  // The cached keys in splits of kps. The new token has a split of its own,
  // split 0, dispatched first (tok_split; the cached splits are then 1..),
  // or is taken by cached split 0 (one split with no cached key when there
  // are none).
  const int ncached = (P - kstart + a.kps - 1) / a.kps;
  const int nsplit = a.tok_split ? ncached + 1 : max(1, ncached);
  if (split >= nsplit) return;
  const int cs = a.tok_split ? split - 1 : split;  // cached split index (-1: the token's own)
  const int k0 = cs < 0 ? P : kstart + cs * a.kps;
  const int k1 = min(P, k0 + a.kps);

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int sub = lane % LPR;
  const int grp = wave * GPW + lane / LPR;
  const int qh0 = h * a.R + hb * RB;

  // K/V rows are addressed as 32-bit byte offsets from the (uniform, SGPR)
  // cache base -- the host keeps cache buffers under 4 GiB for this kernel --
  // so a row costs one VGPR of address (shared by K and V) instead of four.
  const unsigned row_bytes = (unsigned)(a.Hkv * D * 4);
  const char *kcache = reinterpret_cast<const char *>(a.seq[b].k);
  const char *vcache = reinterpret_cast<const char *>(a.seq[b].v);
  const unsigned lane_off = (unsigned)((h * D + 4 * sub) * 4);

  float4 kr[RPG][2], vr[RPG][2];
  bool valid[RPG];
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
      const int j = c + grp + i * NG;
      valid[i] = j < k1;
      if (valid[i]) {
        const unsigned off = (unsigned)j * row_bytes + lane_off;
        kr[i][0] = ld4_stream(kcache + off);
        kr[i][1] = ld4_stream(kcache + off + HALF * 4);
        vr[i][0] = ld4_stream(vcache + off);
        vr[i][1] = ld4_stream(vcache + off + HALF * 4);
      } else {
        kr[i][0] = kr[i][1] = vr[i][0] = vr[i][1] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };
  // The first chunk's K/V loads go out before q and the RoPE table: the loads
  // return in order, so q is ready when the K/V rows are, at no extra latency.
  load_chunk(k0);

  float4 qv[RB][2];
  {
    const float *qb = a.q + ((long)b * a.Hq + qh0) * D;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      qv[r][0] = ld4(qb + r * D + 4 * sub);
      qv[r][1] = ld4(qb + r * D + HALF + 4 * sub);
    }
    if (a.q_norm) {
      // Gemma QK-norm of q. The sum of squares is a tree over the row's lanes
      // (q only enters the scores, which are compared within tolerance; the
      // appended key below keeps the reference's sequential sum).
      const float4 w0 = ld4(a.q_norm + 4 * sub), w1 = ld4(a.q_norm + HALF + 4 * sub);
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const float ss = group_sum<LPR>(dot8(qv[r][0], qv[r][1], qv[r][0], qv[r][1]));
        const float inv = 1.0f / sqrtf(ss / (float)D + a.norm_eps);
        qv[r][0] = mul4(scale4(qv[r][0], inv), w0);
        qv[r][1] = mul4(scale4(qv[r][1], inv), w1);
      }
    }
    if (a.rope_cos) {
      const float4 c = ld4(a.rope_cos + (long)P * HALF + 4 * sub);
      const float4 sn = ld4(a.rope_sin + (long)P * HALF + 4 * sub);
#pragma unroll
      for (int r = 0; r < RB; ++r) rotate4(qv[r][0], qv[r][1], c, sn);
    }
    if (a.q_norm) {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        qv[r][0] = scale4(qv[r][0], a.q_prescale);
        qv[r][1] = scale4(qv[r][1], a.q_prescale);
      }
    }
  }
  // Online softmax with one running maximum per head shared by the whole wave
  // (log2 domain), so the row groups' sums and outputs add without rescaling.
  float m[RB], l[RB];
  float4 o[RB][2];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    m[r] = NEG_INF;
    l[r] = 0.0f;
    o[r][0] = make_float4(0.f, 0.f, 0.f, 0.f);
    o[r][1] = o[r][0];
  }
  const float qs = a.qscale;

  for (int c = k0; c < k1; c += NG * RPG) {
    if (c != k0) load_chunk(c);
    float d[RPG][RB];
#pragma unroll
    for (int i = 0; i < RPG; ++i)
#pragma unroll
      for (int r = 0; r < RB; ++r) d[i][r] = group_sum<LPR>(dot8(qv[r][0], qv[r][1], kr[i][0], kr[i][1]));
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      float cm = NEG_INF;
#pragma unroll
      for (int i = 0; i < RPG; ++i) cm = valid[i] ? fmaxf(cm, d[i][r]) : cm;
      cm = groups_max<LPR>(cm);
      const float mnew = fmaxf(m[r], cm * qs);
      const float ms = safe_max(mnew);
      const float alpha = fast_exp2(m[r] - ms);
      l[r] *= alpha;
      o[r][0] = scale4(o[r][0], alpha);
      o[r][1] = scale4(o[r][1], alpha);
#pragma unroll
      for (int i = 0; i < RPG; ++i) {
        const float p = valid[i] ? fast_exp2(fmaf(d[i][r], qs, -ms)) : 0.0f;
        l[r] += p;
        o[r][0] = fma4(p, vr[i][0], o[r][0]);
        o[r][1] = fma4(p, vr[i][1], o[r][1]);
      }
      m[r] = mnew;
    }
  }

  // ---- the new token (key P), in its own split or in split 0: wave 0 adds
  // it as one more row.
  // Every row group of the wave loads the same row, so its scores are
  // uniform and only group 0 adds the value. ----
  if ((a.tok_split ? cs < 0 : cs == 0) && wave == 0) {  // the token's own split, or cached split 0
    const long row = ((long)b * a.Hkv + h) * D;
    float4 kn0 = ld4(a.cur_k + row + 4 * sub), kn1 = ld4(a.cur_k + row + HALF + 4 * sub);
    const float4 vn0 = ld4(a.cur_v + row + 4 * sub), vn1 = ld4(a.cur_v + row + HALF + 4 * sub);
    const bool first = lane < LPR;
    if (a.k_norm) {
      // ops.rs:159-179 on the key row, bit for bit: the squares in index
      // order through LDS, summed sequentially by lane 0, then x * inv * w.
      if (first) {
        *reinterpret_cast<float4 *>(&knorm_sq[4 * sub]) = mul4(kn0, kn0);
        *reinterpret_cast<float4 *>(&knorm_sq[HALF + 4 * sub]) = mul4(kn1, kn1);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      float inv = 0.0f;
      if (lane == 0) {
        // The chain reads D/16 squares ahead of the ones it adds, so the LDS
        // latency overlaps the adds (the same order of additions; the read
        // ahead scales with D so that head_dim 64 stays within 128 VGPRs).
        constexpr int CH = D / 64, NIT = D / (4 * CH);
        const float4 *sq4 = reinterpret_cast<const float4 *>(knorm_sq);
        float4 cur[CH], nxt[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j) cur[j] = sq4[j];
        float acc = 0.0f;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
          if (it + 1 < NIT) {
#pragma unroll
            for (int j = 0; j < CH; ++j) nxt[j] = sq4[CH * (it + 1) + j];
          }
#pragma unroll
          for (int j = 0; j < CH; ++j) {
            acc += cur[j].x;
            acc += cur[j].y;
            acc += cur[j].z;
            acc += cur[j].w;
          }
#pragma unroll
          for (int j = 0; j < CH; ++j) cur[j] = nxt[j];
        }
        inv = 1.0f / sqrtf(acc / (float)D + a.norm_eps);
      }
      inv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv), 0));
      kn0 = mul4(scale4(kn0, inv), ld4(a.k_norm + 4 * sub));
      kn1 = mul4(scale4(kn1, inv), ld4(a.k_norm + HALF + 4 * sub));
    }
    if (a.rope_cos)
      rotate4(kn0, kn1, ld4(a.rope_cos + (long)P * HALF + 4 * sub), ld4(a.rope_sin + (long)P * HALF + 4 * sub));
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const float dn = group_sum<LPR>(dot8(qv[r][0], qv[r][1], kn0, kn1)) * qs;
      const float mnew = fmaxf(m[r], dn);
      const float ms = safe_max(mnew);
      const float alpha = fast_exp2(m[r] - ms);
      const float p = first ? fast_exp2(dn - ms) : 0.0f;
      l[r] = fmaf(l[r], alpha, p);
      o[r][0] = fma4(p, vn0, scale4(o[r][0], alpha));
      o[r][1] = fma4(p, vn1, scale4(o[r][1], alpha));
      m[r] = mnew;
    }
    // append the rotated key and the value at cache row P (f32 rows, and the
    // bf16 prefill operands when the cache has them)
    if (a.do_append && hb == 0 && first) {
      float *kd = a.app_k[b] + (long)h * D, *vd = a.app_v[b] + (long)h * D;
      *reinterpret_cast<float4 *>(kd + 4 * sub) = kn0;
      *reinterpret_cast<float4 *>(kd + HALF + 4 * sub) = kn1;
      *reinterpret_cast<float4 *>(vd + 4 * sub) = vn0;
      *reinterpret_cast<float4 *>(vd + HALF + 4 * sub) = vn1;
      if (a.app_kb[b]) {
        const long cap = a.app_cap[b];
        bf16 *kb = a.app_kb[b] + ((long)h * cap + P) * D;
        bf16 *vt = a.app_vt[b] + (long)h * D * cap + vt_key_slot(P);
        const float kk[8] = {kn0.x, kn0.y, kn0.z, kn0.w, kn1.x, kn1.y, kn1.z, kn1.w};
        const float vv[8] = {vn0.x, vn0.y, vn0.z, vn0.w, vn1.x, vn1.y, vn1.z, vn1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int dim = (i < 4 ? 0 : HALF) + 4 * sub + (i & 3);
          kb[dim] = (bf16)kk[i];
          vt[(long)dim * cap] = (bf16)vv[i];
        }
      }
    }
  }

  // ---- merge: the groups of a wave share m, the four waves are rescaled ----
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    *reinterpret_cast<float4 *>(&red_o[grp][r][4 * sub]) = o[r][0];
    *reinterpret_cast<float4 *>(&red_o[grp][r][HALF + 4 * sub]) = o[r][1];
    if (sub == 0) red_l[grp][r] = l[r];
    if (lane == 0) wave_m[wave][r] = m[r];
  }
  __syncthreads();

  const long bhh = ((long)b * a.Hkv + h) * a.HB + hb;
  float *dst = a.partial + (bhh * a.max_splits + split) * (long)ENTRY;
  for (int e = tid; e < RB * D; e += 256) {
    const int r = e / D, dim = e % D;
    const float M = fmaxf(fmaxf(wave_m[0][r], wave_m[1][r]), fmaxf(wave_m[2][r], wave_m[3][r]));
    const float Ms = safe_max(M);
    float O = 0.0f, L = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      float ow = 0.0f, lw = 0.0f;
#pragma unroll
      for (int g = 0; g < GPW; ++g) {
        ow += red_o[w * GPW + g][r][dim];
        lw += red_l[w * GPW + g][r];
      }
      const float f = fast_exp2(wave_m[w][r] - Ms);
      O = fmaf(ow, f, O);
      L = fmaf(lw, f, L);
    }
    dst[e] = O;
    if (dim == 0) {
      dst[RB * D + 2 * r] = M;
      dst[RB * D + 2 * r + 1] = L;
    }
  }
}

// Finishes the attention of one (sequence, KV head, head block): merges the
// partials of every split (split 0 holds the new token) into O / L.
// Grid: (Hkv*HB, RB*D / OUTS, B), the head blocks fastest as in the split
// kernel: consecutive workgroups go to consecutive XCDs, so the combine of a
// head runs on the XCD whose workgroups wrote that head's partials (measured
// 4% faster per batch-1 layer at 8192 keys). NT threads = OUTS consecutive
// outputs x SL split lanes: 16 x 16 in 256-thread workgroups, or 16 x 64 in
// 1024-thread ones when there are many splits (256 threads for 16 lanes
// measured 3-4% faster per batch-1 layer than 1024, and 64 or 128 threads
// slower). Each lane keeps an online (max, sum, output) over its splits with
// the loads of eight splits in flight; the SL lanes of every output are
// merged through LDS.
template <int D, int RB, int SL, int NT>
__global__ __launch_bounds__(NT) void decode_combine_kernel(const DecodeArgs a) {
  constexpr int ENTRY = RB * (D + 2);
  constexpr int OUTS = NT / SL, UNROLL = 8;  // one load round up to SL * 8 splits
  __shared__ float s_m[SL][OUTS], s_l[SL][OUTS], s_o[SL][OUTS];

  const int hb = blockIdx.x % a.HB;
  const int h = blockIdx.x / a.HB;
  const int b = blockIdx.z;
  const int P = a.seq[b].past;
  const int kstart = a.window > 0 ? max(0, P + 1 - a.window) : 0;
  const int ncached = (P - kstart + a.kps - 1) / a.kps;
  const int nsplit = a.tok_split ? ncached + 1 : max(1, ncached);
  const int tid = threadIdx.x;
  const int out = tid & (OUTS - 1);
  const int sl = tid / OUTS;
  const int e = blockIdx.y * OUTS + out;  // < RB*D: RB*D is a multiple of OUTS
  const int r = e / D;
  const int qh0 = h * a.R + hb * RB;

  const long bhh = ((long)b * a.Hkv + h) * a.HB + hb;
  const float *ents = a.partial + bhh * a.max_splits * (long)ENTRY;
  float ms[UNROLL], ls[UNROLL], os[UNROLL];
  auto load_batch = [&](int s0) {
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
  };

  float m = NEG_INF, l = 0.0f, o = 0.0f;
  for (int s0 = sl; s0 < nsplit; s0 += SL * UNROLL) {
    load_batch(s0);
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
  if (sl == 0) {
    float M = NEG_INF;
#pragma unroll
    for (int k = 0; k < SL; ++k) M = fmaxf(M, s_m[k][out]);
    const float Ms = safe_max(M);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int k = 0; k < SL; ++k) {
      const float g = fast_exp2(s_m[k][out] - Ms);
      L += s_l[k][out] * g;
      O += s_o[k][out] * g;
    }
    a.out[((long)b * a.Hq + qh0) * D + e] = O / L;
    if ((e % D) == 0 && !(L > 0.0f && L < __builtin_inff())) atomicOr(a.err, kDevErrSoftmaxDenominator);
  }
}

namespace {
// Rows per lane group in flight: three (two for four query heads per block)
// keep the split kernel within 128 VGPRs without spills, so four workgroups
// stay resident per CU.
constexpr int rows_per_group(int RB) { return RB >= 4 ? 2 : 3; }

// Above this many splits the combine gives each output 64 split lanes.
constexpr int kCombineWideSplits = 128;

template <int D, int RB>
hipError_t launch_one(hipStream_t st, const DecodeArgs &a) {
  if (a.max_splits < 1) return hipErrorInvalidValue;  // the new token needs a split
  {
    dim3 grid((unsigned)(a.Hkv * a.HB), (unsigned)a.max_splits, (unsigned)a.B);
    if (a.kps < 4 * (64 / (D / 8)) * rows_per_group(RB))  // small layers: one row per group
      hipLaunchKernelGGL((decode_split_kernel<D, RB, 1>), grid, dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((decode_split_kernel<D, RB, rows_per_group(RB)>), grid, dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (a.max_splits > kCombineWideSplits) {
    dim3 cgrid((unsigned)(a.Hkv * a.HB), (unsigned)(RB * D / 16), (unsigned)a.B);
    hipLaunchKernelGGL((decode_combine_kernel<D, RB, 64, 1024>), cgrid, dim3(1024), 0, st, a);
  } else {
    dim3 cgrid((unsigned)(a.Hkv * a.HB), (unsigned)(RB * D / 16), (unsigned)a.B);
    hipLaunchKernelGGL((decode_combine_kernel<D, RB, 16, 256>), cgrid, dim3(256), 0, st, a);
  }
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

int decode_keys_per_split(int D, int RB, const int *keys, int nseq, long heads, int split_cap) {
  const int chunk = 4 * (64 / (D / 8)) * rows_per_group(RB);  // keys of one workgroup iteration
  long total_rows = 0;
  int max_keys = 1;
  for (int b = 0; b < nseq; ++b) {
    total_rows += (long)keys[b] * heads;
    max_keys = std::max(max_keys, keys[b]);
  }
  // Workgroups with work at kps keys per split (the others of the grid exit
  // at once).
  auto active = [&](long kps) {
    long n = 0;
    for (int b = 0; b < nseq; ++b) n += heads * ((keys[b] + kps - 1) / kps);
    return n;
  };
  // The fewest iterations per workgroup that keep the grid within
  // kDecodeGridWorkgroups, at the longest split that count allows: at a fixed
  // iteration count fewer workgroups ran faster (Llama-3.2-3B at 8192 keys,
  // three iterations: 600 / 520 / 464 workgroups, 18.8 / 17.2 / 16.3 us).
  constexpr long target = kDecodeGridWorkgroups;
  const long per = (total_rows + target - 1) / target;
  long kps = ((per + chunk - 1) / chunk) * chunk;
  if (kps < chunk) kps = chunk;
  // Splits round up per sequence, which can take the workgroups with work past
  // the target (batch 3 at 8192 keys: 24 groups x 22 splits = 528): whole
  // iterations more per split until they fit.
  while (active(kps) > target && kps < max_keys) kps += chunk;
  // Small layers (fewer keys per workgroup than one iteration's worth): one
  // row per lane group, so the grid has twice or three times the workgroups
  // (Llama-3.2-1B at 512 keys: 7.38 -> 6.99 us per layer), unless that takes
  // the combine past its narrow form (Gemma-3-4B's W1024 layer at 128 splits:
  // 7.7 -> 9.6 us).
  if (per < chunk) {
    const long small = std::max<long>(chunk / rows_per_group(RB), per);
    if ((max_keys + small - 1) / small < kCombineWideSplits) kps = small;
  }
  // Bound the partials the combine kernel reads per output (and the caller's
  // partial buffer).
  const long cap = std::max(1, std::min(split_cap, kMaxDecodeSplits));
  if ((max_keys + kps - 1) / kps > cap) {
    const long need = (max_keys + cap - 1) / cap;
    kps = ((need + chunk - 1) / chunk) * chunk;
  }
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
