// prefill.hip -- causal GQA prefill for head_dim 256 (rotary.rs:335-415 with
// query_len > 1, including chunked prefill against a cache and the
// sliding-window extension) as a bf16-MFMA flash-attention kernel for gfx950,
// and the prefill launcher (head_dim 64 and 128 run prefill_wide.hip). Inputs and outputs are
// f32; Q is rounded to bf16 in registers, K and V are read from bf16 copies
// (the cache's bf16 shadow for keys already cached, a staging buffer for the
// rest); scores, softmax state and the output accumulate in f32.
//
// Tiling. A workgroup owns NPB blocks of 32 query positions for RB query
// heads of one KV head (NW = RB*NPB waves, one 32-query block of one head per
// wave), so every K/V tile staged in LDS serves all RB heads of the group.
// Per key tile of BN keys a wave computes
//   S^T = K Q^T   with v_mfma_f32_32x32x16_bf16 (A = K rows from LDS, B = Q in
//                 registers); the accumulator layout puts one query per lane
//                 (lane & 31) and 16 of its keys per lane, so the row max and
//                 sum are lane-local plus one v_permlane32_swap;
//   O^T += V^T P^T with the same instruction (A = V^T from the transposed LDS
//                 tile, B = P^T straight from the score registers: the key
//                 order of the contraction is permuted consistently on both
//                 operands, so no register shuffle is needed).
// The online softmax runs in the log2 domain with v_exp_f32.
// Workgroups are issued longest (last query tile) first for causal balance.
#include "internal.hpp"

namespace spissa {

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float xor32_max(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ u32x2 kreg_lo(u32x4 v) { return __builtin_shufflevector(v, v, 0, 1); }
__device__ __forceinline__ u32x2 kreg_hi(u32x4 v) { return __builtin_shufflevector(v, v, 2, 3); }

__device__ __forceinline__ bf16x8 cat(bf16x4 a, bf16x4 b) {
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

}  // namespace

// Two waves per SIMD up to head_dim 128; head_dim 256 (O alone is 128
// accumulators per lane) takes one wave per SIMD with the full register file.
template <int D, int RB, int NPB, int BN>
__global__ __launch_bounds__(RB *NPB * 64, D >= 256 ? 1 : 2) void prefill_kernel(const PrefillArgs a) {
  constexpr int NW = RB * NPB;
  constexpr int NT = NW * 64;
  constexpr int KS = D + 8;   // K tile row stride (bf16), padded against LDS bank conflicts
  constexpr int VS = BN + 4;  // V^T tile row stride (bf16)
  constexpr int WGQ = NPB * 32;
  constexpr int DB = D / 32;  // 32-dim output blocks
  constexpr int KB = BN / 32; // 32-key score blocks
  constexpr float NEG_INF = -__builtin_inff();

  __shared__ __attribute__((aligned(16))) bf16 Ks[BN * KS];
  __shared__ __attribute__((aligned(16))) bf16 Vs[D * VS];

  const int HB = a.R / RB;
  int bid = blockIdx.x;
  const int hh = bid % (a.Hkv * HB);
  bid /= (a.Hkv * HB);
  const int split = bid % a.splits;
  bid /= a.splits;
  const int qt = a.n_qblocks - 1 - bid;  // longest rows first
  const int h = hh / HB, hb = hh % HB;
  // The wave index is uniform: readfirstlane keeps it (and all that derives
  // from it) in scalar registers and wave-level branches uniform.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int r = wave % RB, pb = wave / RB;
  const int head = h * a.R + hb * RB + r;
  const int p0 = qt * WGQ;
  const int wp0 = p0 + pb * 32;
  const int lq = lane & 31, hl = lane >> 5;
  const int my_pos = wp0 + lq;
  const bool pos_ok = my_pos < a.S;
  const int q_abs = a.P + my_pos;
  const int key_total = a.P + a.S;

  int key_end = key_total;
  if (a.causal) key_end = min(key_total, a.P + min(a.S, p0 + WGQ));
  int key_begin = 0;
  if (a.window > 0) key_begin = max(0, a.P + p0 - a.window + 1);
  int t_begin = key_begin / BN;
  int t_end = (key_end + BN - 1) / BN;
  if (a.splits > 1) {  // this split's share of the tiles (empty: m = -inf, l = 0)
    t_begin += split * a.tps;
    t_end = min(t_end, t_begin + a.tps);
  }

  // Q as the B operand of S^T = K Q^T: lane holds query lq, dims 16t + 8hl + [0,8).
  bf16x8 qf[D / 16];
  {
    const int pos = min(my_pos, a.S - 1);
    const float *qp = a.q + ((long)pos * a.Hq + head) * D + 8 * hl;
#pragma unroll
    for (int t = 0; t < D / 16; ++t) {
      const float4 x0 = *reinterpret_cast<const float4 *>(qp + 16 * t);
      const float4 x1 = *reinterpret_cast<const float4 *>(qp + 16 * t + 4);
      bf16x8 v;
      v[0] = (bf16)x0.x; v[1] = (bf16)x0.y; v[2] = (bf16)x0.z; v[3] = (bf16)x0.w;
      v[4] = (bf16)x1.x; v[5] = (bf16)x1.y; v[6] = (bf16)x1.z; v[7] = (bf16)x1.w;
      qf[t] = v;
    }
  }

  f32x16 oacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int i = 0; i < 16; ++i) oacc[d][i] = 0.0f;
  // Running max m is kept in the scaled log2 domain; scores stay raw and the
  // scale is folded into the exp2 argument.
  float m = NEG_INF, l = 0.0f;
  const float c = a.qk_scale_log2;

  const int wave_min_q = a.P + wp0;
  const int wave_max_q = a.P + min(wp0 + 31, a.S - 1);
  const bool wave_live = wp0 < a.S;

  // Per-thread staging slots, fixed for the whole loop: K chunk (row, 8 dims)
  // and V^T chunk (dim, 8 keys) offsets inside a tile and inside LDS.
  constexpr int KCH = BN * (D / 8) / NT;  // 16-byte K chunks per thread per tile
  constexpr int VCH = D * (BN / 8) / NT;  // 16-byte V^T chunks per thread per tile
  static_assert(KCH * NT == BN * (D / 8) && VCH * NT == D * (BN / 8), "tile/thread mismatch");
  int k_row[KCH], k_lds[KCH], v_dim[VCH], v_kc[VCH], v_lds[VCH];
#pragma unroll
  for (int u = 0; u < KCH; ++u) {
    const int cc = threadIdx.x + u * NT;
    k_row[u] = cc / (D / 8);
    const int col = (cc % (D / 8)) * 8;
    k_lds[u] = k_row[u] * KS + col;
    k_row[u] = k_row[u] * D + col;  // element offset of the chunk inside a tile of D-wide rows
  }
#pragma unroll
  for (int u = 0; u < VCH; ++u) {
    const int cc = threadIdx.x + u * NT;
    v_dim[u] = cc / (BN / 8);
    v_kc[u] = (cc % (BN / 8)) * 8;
    v_lds[u] = v_dim[u] * VS + v_kc[u];
  }
  const bf16 *kb_c = a.kb_cache + (long)h * a.cap_cache * D;
  const bf16 *kb_s = a.kb_stage + (long)h * a.cap_stage * D;
  const bf16 *vt_c = a.vt_cache + (long)h * D * a.cap_cache;
  const bf16 *vt_s = a.vt_stage + (long)h * D * a.cap_stage;

  // The next tile's K / V^T chunks are loaded into registers while the
  // current tile is computed (register double buffering). Tiles never straddle
  // the cache / staging boundary P8 (a multiple of the tile width), so the
  // source buffer is a uniform choice per tile. Iteration t_begin - 1 only
  // loads the first tile.
  u32x4 kreg[KCH], vreg[VCH];
  for (int t = t_begin - 1; t < t_end; ++t) {
    const int kt0 = t * BN;
    if (t >= t_begin) {
      __syncthreads();  // every wave is done with the previous tile
#pragma unroll
      for (int u = 0; u < KCH; ++u) *reinterpret_cast<u32x4 *>(&Ks[k_lds[u]]) = kreg[u];
#pragma unroll
      for (int u = 0; u < VCH; ++u) {
        *reinterpret_cast<u32x2 *>(&Vs[v_lds[u]]) = kreg_lo(vreg[u]);
        *reinterpret_cast<u32x2 *>(&Vs[v_lds[u] + 4]) = kreg_hi(vreg[u]);
      }
      __syncthreads();
    }
    if (t + 1 < t_end) {
      const int nk = kt0 + BN;
      const bool from_cache = nk < a.P8;
      const bf16 *kt = from_cache ? kb_c + (long)nk * D : kb_s + (long)(nk - a.P8) * D;
      const bf16 *vt = from_cache ? vt_c + nk : vt_s + (nk - a.P8);
      const long vstride = from_cache ? a.cap_cache : a.cap_stage;
#pragma unroll
      for (int u = 0; u < KCH; ++u) kreg[u] = *reinterpret_cast<const u32x4 *>(kt + k_row[u]);
#pragma unroll
      for (int u = 0; u < VCH; ++u)
        vreg[u] = *reinterpret_cast<const u32x4 *>(vt + (long)v_dim[u] * vstride + v_kc[u]);
    }
    if (t < t_begin) continue;

    const bool active = wave_live && !(a.causal && kt0 > wave_max_q) &&
                        !(a.window > 0 && kt0 + BN - 1 + a.window <= wave_min_q);
    if (!active) continue;

    // ---- S^T = K Q^T (raw scores) ----
    f32x16 sacc[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) sacc[kb][i] = 0.0f;
#pragma unroll
      for (int tt = 0; tt < D / 16; ++tt) {
        const bf16x8 ka =
            *reinterpret_cast<const bf16x8 *>(&Ks[(kb * 32 + lq) * KS + 16 * tt + 8 * hl]);
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[tt], sacc[kb], 0, 0, 0);
      }
    }

    // ---- mask (diagonal and tail tiles only), tile max ----
    const bool need_mask = (a.causal && kt0 + BN - 1 > wave_min_q) ||
                           (a.window > 0 && kt0 + a.window <= wave_max_q) ||
                           (kt0 + BN > key_total);
    // Masked scores go to a copy: writing -inf in place into the MFMA
    // accumulator registers gave wrong results on masked tiles.
    float sc[KB][16];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float v = sacc[kb][i];
        if (need_mask) {
          const int key = kt0 + kb * 32 + 8 * (i >> 2) + 4 * hl + (i & 3);
          const bool masked = (a.causal && key > q_abs) ||
                              (a.window > 0 && key + a.window <= q_abs) || key >= key_total;
          if (masked) v = NEG_INF;
        }
        sc[kb][i] = v;
      }
    float tmax = NEG_INF;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int i = 0; i < 16; i += 2) tmax = fmaxf(tmax, fmaxf(sc[kb][i], sc[kb][i + 1]));
    tmax = xor32_max(tmax) * c;

    // ---- online softmax; rescale O only when some row's maximum grew ----
    const float mnew = fmaxf(m, tmax);
    const float ms = mnew == NEG_INF ? 0.0f : mnew;
    if (__ballot(mnew > m)) {
      const float alpha = fast_exp2(m - ms);
      l *= alpha;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[d][i] *= alpha;
    }
    m = mnew;

    // ---- O^T += V^T P^T ----
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      bf16x8 pa, pb;
      float ls = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float p0v = fast_exp2(fmaf(sc[kb][i], c, -ms));
        const float p1v = fast_exp2(fmaf(sc[kb][i + 8], c, -ms));
        ls += p0v + p1v;
        pa[i] = (bf16)p0v;
        pb[i] = (bf16)p1v;
      }
      l += ls;
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        // V^T rows hold keys in vt_key_slot order: this lane's 8 keys of each
        // 16-key step are contiguous.
        const bf16 *vrow = &Vs[(d * 32 + lq) * VS + kb * 32 + 8 * hl];
        const bf16x8 va = cat(*reinterpret_cast<const bf16x4 *>(vrow),
                              *reinterpret_cast<const bf16x4 *>(vrow + 4));
        oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pa, oacc[d], 0, 0, 0);
        const bf16x8 vb = cat(*reinterpret_cast<const bf16x4 *>(vrow + 16),
                              *reinterpret_cast<const bf16x4 *>(vrow + 20));
        oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vb, pb, oacc[d], 0, 0, 0);
      }
    }
  }

  const float lt = xor32_sum(l);
  if (a.splits > 1) {  // unnormalised O and (m, l) of this key split
    if (pos_ok) {
      const long row = ((long)split * a.S + my_pos) * a.Hq + head;
      float *op = a.part_o + row * D + 4 * hl;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<float4 *>(op + d * 32 + 8 * g) =
              make_float4(oacc[d][4 * g], oacc[d][4 * g + 1], oacc[d][4 * g + 2], oacc[d][4 * g + 3]);
      if (hl == 0) {
        a.part_ml[row * 2] = m;
        a.part_ml[row * 2 + 1] = lt;
      }
    }
    return;
  }

  // ---- epilogue: O = O^T / l ----
  if (pos_ok) {
    if (hl == 0 && !(lt > 0.0f && lt < __builtin_inff())) atomicOr(a.err, kDevErrSoftmaxDenominator);
    const float inv = 1.0f / lt;
    float *op = a.out + ((long)my_pos * a.Hq + head) * D + 4 * hl;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float4 v = make_float4(oacc[d][4 * g] * inv, oacc[d][4 * g + 1] * inv,
                               oacc[d][4 * g + 2] * inv, oacc[d][4 * g + 3] * inv);
        *reinterpret_cast<float4 *>(op + d * 32 + 8 * g) = v;
      }
    }
  }
}

namespace {

template <int D, int RB, int NPB>
hipError_t launch_cfg(hipStream_t st, PrefillArgs a) {
  constexpr int BN = D >= 256 ? 32 : 64;
  constexpr int WGQ = NPB * 32;
  a.n_qblocks = (a.S + WGQ - 1) / WGQ;
  const long blocks = (long)a.n_qblocks * a.splits * a.Hkv * (a.R / RB);
  hipLaunchKernelGGL((prefill_kernel<D, RB, NPB, BN>), dim3((unsigned)blocks), dim3(RB * NPB * 64),
                     0, st, a);
  return hipGetLastError();
}

// Four waves per workgroup (one per SIMD): four query heads of a KV group
// with one 32-position block, two heads with two blocks, or one head with four
// blocks (also for groups of three or five heads).
template <int D>
hipError_t launch_d(hipStream_t st, const PrefillArgs &a) {
  if (a.R % 4 == 0) return launch_cfg<D, 4, 1>(st, a);
  if (a.R % 2 == 0) return launch_cfg<D, 2, 2>(st, a);
  return launch_cfg<D, 1, 4>(st, a);
}

}  // namespace

bool prefill_supported(int D) { return D == 64 || D == 128 || D == 256; }

// Both kernels launch four-wave workgroups of 32 queries per wave: four heads
// x 32 queries, two heads x 64, or one head x 128 (launch_d here and in
// prefill_wide.hip).
int prefill_wg_queries(const PrefillArgs &a, int) { return a.R % 4 == 0 ? 32 : a.R % 2 == 0 ? 64 : 128; }
int prefill_wgs_per_cu(int D) { return D >= 256 ? 1 : 2; }
int prefill_tile_keys(int D) { return D >= 256 ? 32 : 64; }

long prefill_base_workgroups(const PrefillArgs &a, int D) {
  const int wgq = prefill_wg_queries(a, D);
  const int rb = 128 / wgq;
  return (long)((a.S + wgq - 1) / wgq) * a.Hkv * (a.R / rb);
}

// Merges key splits: per (query row, head), M = max m_j, then
// O = sum_j O_j 2^(m_j - M), L = sum_j l_j 2^(m_j - M), out = O / L. Splits
// that saw no key of the row (m_j = -inf) contribute nothing. One workgroup of
// D threads per (row, head): the (m, l) pairs of all splits are loaded once
// into LDS by parallel threads, then every thread accumulates its output
// element over the splits with independent loads. The error bit is set for an
// invalid L, as the unsplit kernels do (rotary.rs:560-564).
constexpr int kMaxPrefillSplits = 256;

__global__ __launch_bounds__(256) void prefill_combine_kernel(const PrefillArgs a, int D) {
  __shared__ float s_g[kMaxPrefillSplits];  // weight 2^(m_j - M) (0 for empty splits)
  __shared__ float s_l[kMaxPrefillSplits];
  __shared__ float s_red[256];
  const long row = blockIdx.x;  // pos * Hq + head
  const int d = threadIdx.x;
  const long stride = (long)a.S * a.Hq;
  float mj = -__builtin_inff(), lj = 0.0f;
  for (int j = d; j < a.splits; j += blockDim.x) {  // splits <= kMaxPrefillSplits <= blockDim in practice
    mj = a.part_ml[(j * stride + row) * 2];
    lj = a.part_ml[(j * stride + row) * 2 + 1];
  }
  s_red[d] = mj;
  __syncthreads();
  for (int w = blockDim.x / 2; w > 0; w >>= 1) {
    if (d < w) s_red[d] = fmaxf(s_red[d], s_red[d + w]);
    __syncthreads();
  }
  const float M = s_red[0];
  const float Ms = M == -__builtin_inff() ? 0.0f : M;
  if (d < a.splits) {
    s_g[d] = mj == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(mj - Ms);
    s_l[d] = lj;
  }
  __syncthreads();
  float L = 0.0f, O = 0.0f;
  const float *po = a.part_o + row * D + d;
  int j = 0;
  for (; j + 4 <= a.splits; j += 4) {  // four independent loads in flight
    const float o0 = po[(j + 0) * stride * D], o1 = po[(j + 1) * stride * D];
    const float o2 = po[(j + 2) * stride * D], o3 = po[(j + 3) * stride * D];
    O = fmaf(o0, s_g[j], O);
    O = fmaf(o1, s_g[j + 1], O);
    O = fmaf(o2, s_g[j + 2], O);
    O = fmaf(o3, s_g[j + 3], O);
  }
  for (; j < a.splits; ++j) O = fmaf(po[j * stride * D], s_g[j], O);
  for (int k = 0; k < a.splits; ++k) L = fmaf(s_l[k], s_g[k], L);
  a.out[row * D + d] = O / L;
  if (d == 0 && !(__float_as_uint(L) - 1u < 0x7f7fffffu)) atomicOr(a.err, kDevErrSoftmaxDenominator);
}

hipError_t launch_prefill_combine(hipStream_t st, const PrefillArgs &a, int D) {
  if (a.splits <= 1) return hipSuccess;
  if (a.splits > kMaxPrefillSplits || a.splits > D) return hipErrorInvalidValue;
  hipLaunchKernelGGL(prefill_combine_kernel, dim3((unsigned)((long)a.S * a.Hq)), dim3(D), 0, st, a, D);
  return hipGetLastError();
}

hipError_t launch_prefill(hipStream_t st, const PrefillArgs &a, int D) {
  switch (D) {
    case 64:
    case 128: return launch_prefill_wide(st, a, D);
    case 256: return launch_d<256>(st, a);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace spissa
