// prefill.hip -- causal GQA prefill for head_dim 64, 128 and 256
// (rotary.rs:335-415 with query_len > 1, including chunked prefill against a
// cache and the sliding-window extension) as a bf16-MFMA flash-attention
// kernel for gfx950. Inputs and outputs are f32; Q is rounded to bf16 in
// registers, K and V are read from bf16 copies (the cache's bf16 shadow for
// tiles below P8, the staging buffer for the rest); scores, softmax state and
// the output accumulate in f32.
//
// Work split. At head_dim 64 and 128 (prefill_kernel) each wave owns QB
// 32-query blocks of one query head (QB = 1 in the launched configurations),
// and the four waves of a workgroup share one KV head: four heads of a group,
// two heads with two blocks each, or one head with four blocks; two waves run
// per SIMD (at most 256 VGPRs each). Head_dim 256 (prefill_q16_kernel, after
// prefill_kernel) gives each wave 16 queries on 16x16x32 MFMAs, 32-key tiles.
// Key splits (PrefillArgs::splits > 1) add workgroups over the key range for
// grids too small to fill the GPU (short chunks over long caches, few heads);
// prefill_combine_kernel merges their partial results.
//
// Per key tile of BN keys and per query block a wave computes
//   S^T = K Q^T   v_mfma_f32_32x32x16_bf16, A = K rows from LDS, B = Q^T in
//                 registers; the accumulator puts one query per lane (lane &
//                 31) and 16 of its keys per lane, so row max and sum are
//                 lane-local plus one v_permlane32_swap;
//   O^T += V^T P^T  A = V^T from LDS, B = P^T straight from the score
//                 registers (keys of the V^T operand are stored in
//                 vt_key_slot order, so each lane's 8 keys are 16 contiguous
//                 bytes).
// Copies. K and V^T tiles go global -> LDS with global_load_lds_dwordx4 (no
// staging registers) into two alternating buffers each. The loop is
// software-pipelined one tile deep. In step t the copies of K(t+2) and V(t+1)
// are in flight while
//   part A: the exponentials of tile t run on the VALU next to the MFMAs of
//           S(t+1) = K(t+1) Q^T;
//   part B: O^T += V(t)^T P(t)^T runs on the MFMAs (at head_dim 64 next to
//           the row maxima of tile t+1, which fix the exponent reference of
//           step t+1);
// then the (rare) rescale of O and one barrier. The compiler interleaves the
// VALU and MFMA work of each part freely.
// Scores. Q is rounded to bf16 after scaling by softmax scale * log2(e), and
// the score MFMAs start from minus the row's exponent reference, so the
// accumulators hold (scaled score - reference) and feed the exponentials
// directly. Masked tiles (causal diagonal, window edge, keys past the end)
// start at -inf for the hidden keys instead, so the MFMAs yield -inf there
// and the maxima and exponentials need no per-element selects.
// Tiles are unpadded; the 16-byte chunks of each row are XOR-swizzled within
// the row by swz(row), chosen so that the 8 consecutive rows one LDS read
// serves together (same chunk index) hit 8 distinct 16-byte bank groups:
//   K tile   [BN keys][D]: chunk c of key row r at byte r*2D  + 16*(c ^ swz(r))
//   V^T tile [D][BN keys]: chunk c of dim row d at byte d*2BN + 16*(c ^ swz(d))
// Softmax. The exponent reference m of a row is raised rarely: at head_dim
// 64 when the next tile's row maximum exceeds it by more than 8 (log2
// domain); at head_dim 128 and 256 only when a tile's probabilities sum past
// 2^16 (or the row has seen no key yet), which drops the per-tile row
// maximum. O and the sum share m, so O / sum is exact softmax arithmetic.
// Row sums add the bf16 probabilities that the PV MFMAs use.
// This file is compiled with MFMA results in VGPRs (-amdgpu-mfma-vgpr-form):
// the score accumulators feed VALU code directly instead of round-tripping
// through AGPRs.
#include <algorithm>
#include <type_traits>

#include "internal.hpp"

namespace spissa {

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((address_space(3))) void lds_void;

constexpr float NEG_INF = -__builtin_inff();
// Eager raising (head_dim 64): the largest growth of a row maximum
// (log2 domain) absorbed without rescaling, checked on every tile.
constexpr float kRescaleSlack = 8.0f;
// Lazy raising (head_dim 128 and 256): a lane's sum of one tile's probabilities above
// which its row's exponent reference is raised (the probabilities then stay
// far from f32 and bf16 overflow, and O keeps full relative precision).
constexpr float kRaiseSum = 65536.0f;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// NaN-propagating maximum (v_maximum_f32): no input canonicalisation, and a
// NaN score reaches the denominator check.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

__device__ __forceinline__ float xor32_max(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Copies 16 bytes per lane from src into LDS at lds_base + 16 * lane.
__device__ __forceinline__ void dma16(const char *src, char *lds_base) {
  __builtin_amdgcn_global_load_lds(src, (lds_void *)lds_base, 16, 0, 0);
}

// dma16 issued as inline assembly. The compiler then tracks no copy into LDS
// and inserts no wait of its own before LDS reads (it cannot tell which stage a
// copy fills once control flow merges); the kernel waits for exactly the
// copies it reads with wait_copies_upto. The compiler's own vmcnt waits for
// its loads stay correct: copies complete in issue order, and copies it does
// not count only make a wait for an earlier load stricter.
// base is wave-uniform (an SGPR pair), off the lane's byte offset from it.
__device__ __forceinline__ void dma16_untracked(const char *base, unsigned off, char *lds_base) {
  const unsigned lds = (unsigned)(uintptr_t)(lds_void *)lds_base;
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}

// Waits for this wave's outstanding global -> LDS copies.
__device__ __forceinline__ void wait_copies() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt and lgkmcnt unconstrained
}

// Workgroup barrier that orders LDS accesses but, unlike __syncthreads(), lets
// this wave's global -> LDS copies stay in flight (the workgroup fence there
// waits for all of them). The caller waits for the copies the next step reads
// (wait_copies, wait_copies_upto); lgkmcnt(0) retires this wave's LDS reads
// before another wave's copy may overwrite what they read.
__device__ __forceinline__ void copies_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Waits until at most n of this wave's global -> LDS copies are outstanding
// (they complete in issue order). n is wave-uniform; the wait uses the largest
// multiple of STEP not above n or MAX.
template <int MAX, int STEP>
__device__ __forceinline__ void wait_copies_upto(int n) {
  static_assert(MAX < 64, "vmcnt holds 6 bits");
  if constexpr (MAX <= 0) {
    wait_copies();
  } else {
    if (n >= MAX) {
      __builtin_amdgcn_s_waitcnt(0x0F70 | (MAX & 15) | ((MAX >> 4) << 14));
      return;
    }
    wait_copies_upto<MAX - STEP, STEP>(n);
  }
}

// XOR swizzle of a row of NC 16-byte chunks (NC = 4, 8, 16 or 32), staying below
// NC. For a fixed chunk index, any 8 aligned consecutive rows land in 8
// distinct 16-byte groups modulo 128 bytes and any 16 aligned consecutive rows
// in 16 distinct groups modulo 256 bytes, so an LDS read is conflict-free
// whether the hardware serves 8 lanes per 128 bytes or 16 lanes per 256. The
// swizzle of row 32 b + l does not depend on b.
template <int NC>
__device__ __forceinline__ constexpr int swz(int row) {
  static_assert(NC == 4 || NC == 8 || NC == 16 || NC == 32, "row width");
  return NC >= 16 ? (row & 15) : NC == 8 ? ((row ^ ((row >> 3) & 1)) & 7) : (((row >> 1) ^ (row >> 2)) & 3);
}

template <int D, int BN, int NW>
struct Geom {
  static constexpr int KBYTES = BN * D * 2;
  static constexpr int VBYTES = D * BN * 2;
  static constexpr int KDMA = KBYTES / 1024 / NW;  // K copies per wave per tile
  static constexpr int VDMA = VBYTES / 1024 / NW;  // V^T copies per wave per tile
  static constexpr int DT = D / 16;                // 16-dim steps of S^T = K Q^T
  static constexpr int KB = BN / 32;               // 32-key score blocks
  static constexpr int KS = BN / 16;               // 16-key steps of O^T += V^T P^T
  static constexpr int DB = D / 32;                // 32-dim output blocks
  static constexpr int KNC = D / 8;                // 16-byte chunks per K row
  static constexpr int VNC = BN / 8;               // 16-byte chunks per V^T row
  static_assert(KDMA * NW * 1024 == KBYTES && VDMA * NW * 1024 == VBYTES, "tile/wave split");
};

// S^T of one key tile for the wave's QB query blocks over the 16-dim steps
// [T0, T1), accumulated onto s (which the first step finds holding minus the
// row's exponent reference, or -inf for a masked tile's hidden keys); kbuf is
// the K tile in LDS.
template <int D, int BN, int QB, int T0, int T1, int NT>
__device__ __forceinline__ void score_tile(f32x16 (&s)[QB][BN / 32], const char *kbuf, const unsigned (&k_rd)[NT],
                                           const bf16x8 (&qf)[QB][NT]) {
  constexpr int KB = BN / 32;
#pragma unroll
  for (int tt = T0; tt < T1; ++tt)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const bf16x8 kf = *reinterpret_cast<const bf16x8 *>(kbuf + kb * 64 * D + k_rd[tt]);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
        s[qb][kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[qb][tt], s[qb][kb], 0, 0, 0);
    }
}

// Sum of the eight bf16 probabilities of p (v_dot2c_f32_bf16 against 1.0 pairs).
__device__ __forceinline__ float sum_bf16x8(const bf16x8 p) {
  typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  float s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p, p, 0, 1), one, 0.0f, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p, p, 2, 3), one, s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p, p, 4, 5), one, s, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(p, p, 6, 7), one, s, false);
}

}  // namespace

// Head_dim 64 and 128. QB query blocks of 32 per wave (1 in the launched
// shapes); two waves per SIMD (the second __launch_bounds__ argument is the
// minimum waves per SIMD: at most 256 VGPRs each). KSP waves share each
// query block's key tiles (wave pairs: tile 2T + kh of super-tile T goes to
// wave kh of the pair).
template <int D, int RB, int NPB, int BN, int QB, int KSP>
__global__ __launch_bounds__(RB *NPB *KSP * 64, 2) void prefill_kernel(const PrefillArgs a) {
  static_assert(D <= 128, "head_dim 256 runs prefill_q16_kernel");
  static_assert(KSP == 1 || KSP == 2, "one wave or a wave pair per query block");
  constexpr int NW = RB * NPB * KSP;
  constexpr int WQ = QB * 32;  // queries per wave
  constexpr int WGQ = NPB * WQ;
  using G = Geom<D, BN, NW>;
  // Exponent reference raised lazily (from the tile's probability sums) or
  // eagerly (from every next tile's row maxima): lazily measured 2-3% faster
  // at head_dim 128, eagerly 4-5% faster at 64.
  constexpr bool LAZY = D == 128;
  constexpr int DT = G::DT, KB = G::KB, KS = G::KS, DB = G::DB;

  // Four separate LDS objects (not one array): the compiler then knows that
  // copies into one buffer do not alias reads of another and does not wait
  // for the copies before every LDS read.
  // (With wave pairs each buffer holds the KSP tiles of a super-tile.)
  __shared__ __attribute__((aligned(1024))) char k_lds0[KSP * G::KBYTES];
  __shared__ __attribute__((aligned(1024))) char k_lds1[KSP * G::KBYTES];
  __shared__ __attribute__((aligned(1024))) char v_lds0[KSP * G::VBYTES];
  __shared__ __attribute__((aligned(1024))) char v_lds1[KSP * G::VBYTES];

  const int HB = a.R / RB;
  int h, hb, split, qt;
  if (a.xcd_group == 1) {
    // Workgroup ids 8 apart run on one XCD. The HB * n_qblocks workgroups
    // that read the same keys (one KV head, one split) get ids
    // lo + 8 * (g + G * hi), unit = 8 * hi + lo, so that they share that
    // XCD's L2 instead of each fetching the keys from HBM.
    const int G = HB * a.n_qblocks;
    const int lo = (int)(blockIdx.x & 7), rest = (int)(blockIdx.x >> 3);
    const int g = rest % G, unit = (rest / G) * 8 + lo;
    if (unit >= a.Hkv * a.splits) return;  // padding up to a multiple of 8 units
    h = unit % a.Hkv;
    split = unit / a.Hkv;
    hb = g % HB;
    qt = a.n_qblocks - 1 - g / HB;
  } else {
    int bid = blockIdx.x;
    if (a.xcd_group == 2) {  // ids of one XCD (equal mod 8) take a contiguous run
      bid = (int)(blockIdx.x & 7) * (int)(gridDim.x >> 3) + (int)(blockIdx.x >> 3);
      if (bid >= a.n_qblocks * HB * a.Hkv * a.splits) return;  // padding to a multiple of 8
    }
    const int hh = bid % (a.Hkv * HB);
    bid /= (a.Hkv * HB);
    split = bid % a.splits;
    bid /= a.splits;
    qt = a.n_qblocks - 1 - bid;  // longest rows first
    h = hh / HB;
    hb = hh % HB;
  }
  // The wave index is uniform: readfirstlane keeps it (and all that derives
  // from it) in scalar registers and wave-level branches uniform.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int kh = wave % KSP, wq = wave / KSP;  // tile parity within the pair; the pair
  const int r = wq % RB, pb = wq / RB;
  const int head = h * a.R + hb * RB + r;
  const int p0 = qt * WGQ;
  const int wp0 = p0 + pb * WQ;
  const int lq = lane & 31, hl = lane >> 5;
  const int key_total = a.P + a.S;

  int key_end = key_total;
  if (a.causal) key_end = min(key_total, a.P + min(a.S, p0 + WGQ));
  int key_begin = 0;
  if (a.window > 0) key_begin = max(0, a.P + p0 - a.window + 1);
  int t_begin = key_begin / BN;
  int t_end = (key_end + BN - 1) / BN;
  if (a.splits > 1) {  // this split's share of the workgroup's tiles
    t_begin += split * a.tps;
    t_end = min(t_end, t_begin + a.tps);
  }
  if (t_begin >= t_end) {  // this split sees none of the workgroup's keys (uniform exit)
    const int pos = wp0 + lane;
    if (kh == 0 && lane < WQ && pos < a.S) {
      float *ml = a.part_ml + (((long)split * a.S + pos) * a.Hq + head) * 2;
      ml[0] = -__builtin_inff();
      ml[1] = 0.0f;
    }
    return;
  }
  // Super-tiles of KSP tiles: T covers tiles [KSP*T, KSP*T + KSP). Wave kh of
  // a pair scores tile KSP*T + kh; a tile outside [t_begin, t_end) is hidden
  // from it.
  const int T_begin = t_begin / KSP, T_end = (t_end + KSP - 1) / KSP;

  // Q^T (B operand): lane holds query lq of block qb, dims 16t + 8hl + [0,8).
  // Q carries the softmax scale times log2(e), so the scores come out of the
  // MFMAs in the log2 domain.
  // (Loaded in the prologue, after the first copies are issued, so that the
  // two memory latencies overlap.)
  bf16x8 qf[QB][DT];
  auto load_q = [&]() {
    const float c = a.qk_scale_log2;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int pos = min(wp0 + 32 * qb + lq, a.S - 1);
      if (a.qb) {  // already scaled and rounded (the fused prefill step)
        const bf16 *qp = a.qb + ((long)pos * a.Hq + head) * D + 8 * hl;
#pragma unroll
        for (int t = 0; t < DT; ++t) qf[qb][t] = *reinterpret_cast<const bf16x8 *>(qp + 16 * t);
        continue;
      }
      const float *qp = a.q + ((long)pos * a.Hq + head) * D + 8 * hl;
      float x[DT][8];
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        *reinterpret_cast<float4 *>(&x[t][0]) = *reinterpret_cast<const float4 *>(qp + 16 * t);
        *reinterpret_cast<float4 *>(&x[t][4]) = *reinterpret_cast<const float4 *>(qp + 16 * t + 4);
      }
      if (a.q_cos) {
        // Rotate-half pairs (d, d + D/2) sit in one lane: dims 16t + 8hl + j
        // and 16(t + DT/2) + 8hl + j. Each product is rounded apart
        // (rotary.rs:467-481), as the append pass computes it.
#pragma clang fp contract(off)
        const float *cp = a.q_cos + (long)(a.P + pos) * (D / 2) + 8 * hl;
        const float *sp = a.q_sin + (long)(a.P + pos) * (D / 2) + 8 * hl;
#pragma unroll
        for (int t = 0; t < DT / 2; ++t) {
          float cs[8], sn[8];
          *reinterpret_cast<float4 *>(&cs[0]) = *reinterpret_cast<const float4 *>(cp + 16 * t);
          *reinterpret_cast<float4 *>(&cs[4]) = *reinterpret_cast<const float4 *>(cp + 16 * t + 4);
          *reinterpret_cast<float4 *>(&sn[0]) = *reinterpret_cast<const float4 *>(sp + 16 * t);
          *reinterpret_cast<float4 *>(&sn[4]) = *reinterpret_cast<const float4 *>(sp + 16 * t + 4);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float first = x[t][j], second = x[t + DT / 2][j];
            x[t][j] = first * cs[j] - second * sn[j];
            x[t + DT / 2][j] = second * cs[j] + first * sn[j];
          }
        }
      }
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        bf16x8 v;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (bf16)(x[t][j] * c);
        qf[qb][t] = v;
      }
    }
  };
  f32x16 oacc[QB][DB];
  float m[QB], l[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int i = 0; i < 16; ++i) oacc[qb][d][i] = 0.0f;
    m[qb] = NEG_INF;
    l[qb] = 0.0f;
  }

  // LDS byte offsets of this lane's fragments (key block 0 / dim block 0).
  // (Rows of a fragment are 32 * block + lq, and 32 * block leaves swz unchanged.)
  unsigned k_rd[DT], v_rd[KS];
#pragma unroll
  for (int t = 0; t < DT; ++t) k_rd[t] = lq * 2 * D + 16 * ((2 * t + hl) ^ swz<G::KNC>(lq));
#pragma unroll
  for (int t = 0; t < KS; ++t) v_rd[t] = lq * 2 * BN + 16 * ((2 * t + hl) ^ swz<G::VNC>(lq));

  // Source of this lane's copies: copy j of the wave fills LDS bytes
  // [(wave + j*NW) * 1024, +1024) of a tile; lane l writes its 16 bytes at
  // +16 l, i.e. position p of K row `row` (V^T: dim row d), which holds chunk
  // p ^ swz(row) of that row. Every source chunk lies inside the tile's row.
  // The offsets are recomputed per copy (a few VALU operations) rather than
  // held in registers across the loop.
  auto k_src = [&](int j) {
    const int byte = (wave + j * NW) * 1024 + lane * 16;
    const int row = byte / (2 * D), p = (byte % (2 * D)) / 16;
    return (unsigned)(row * D + 8 * (p ^ swz<G::KNC>(row))) * 2u;
  };
  auto v_src = [&](int j, unsigned stride) {
    const int byte = (wave + j * NW) * 1024 + lane * 16;
    const int d = byte / (2 * BN), p = (byte % (2 * BN)) / 16;
    return ((unsigned)d * stride + (unsigned)(8 * (p ^ swz<G::VNC>(d)))) * 2u;
  };
  const char *kb_c = reinterpret_cast<const char *>(a.kb_cache + (long)h * a.cap_cache * D);
  const char *kb_s = reinterpret_cast<const char *>(a.kb_stage + (long)h * a.cap_stage * D);
  const char *vt_c = reinterpret_cast<const char *>(a.vt_cache + (long)h * D * a.cap_cache);
  const char *vt_s = reinterpret_cast<const char *>(a.vt_stage + (long)h * D * a.cap_stage);
  // V^T row strides held in scalar registers (otherwise reloaded from the
  // kernel arguments, with a wait, on every step)
  const unsigned vt_stride_c = __builtin_amdgcn_readfirstlane((unsigned)a.cap_cache);
  const unsigned vt_stride_s = __builtin_amdgcn_readfirstlane((unsigned)a.cap_stage);

  // Tiles below P8 come from the cache shadow, the others from staging (P8 is
  // a multiple of the tile width, so the choice is uniform per tile).
  // (A super-tile's tiles past the range's last are copied as that last one:
  // in bounds, and hidden from the wave that takes them.)
  auto copy_k = [&](int T, char *dst) {
#pragma unroll
    for (int i = 0; i < KSP; ++i) {
      const int nk = (KSP == 1 ? T : min(KSP * T + i, t_end - 1)) * BN;
      const char *src = nk < a.P8 ? kb_c + (long)nk * D * 2 : kb_s + (long)(nk - a.P8) * D * 2;
#pragma unroll
      for (int j = 0; j < G::KDMA; ++j)
        dma16_untracked(src, k_src(j), dst + i * G::KBYTES + (wave + j * NW) * 1024);
    }
  };
  auto copy_v = [&](int T, char *dst) {
#pragma unroll
    for (int i = 0; i < KSP; ++i) {
      const int nk = (KSP == 1 ? T : min(KSP * T + i, t_end - 1)) * BN;
      const bool cached = nk < a.P8;
      const char *src = cached ? vt_c + (long)nk * 2 : vt_s + (long)(nk - a.P8) * 2;
      const unsigned stride = cached ? vt_stride_c : vt_stride_s;
#pragma unroll
      for (int j = 0; j < G::VDMA; ++j)
        dma16_untracked(src, v_src(j, stride), dst + i * G::VBYTES + (wave + j * NW) * 1024);
    }
  };

  // Visible keys [vis_lo, vis_hi] of this lane's two queries.
  int vis_lo[QB], vis_hi[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int q_abs = a.P + wp0 + 32 * qb + lq;
    vis_hi[qb] = a.causal ? min(q_abs, key_total - 1) : key_total - 1;
    vis_lo[qb] = a.window > 0 ? q_abs - a.window + 1 : 0;
  }
  const int wave_min_q = a.P + wp0;
  const int wave_max_q = a.P + min(wp0 + WQ - 1, a.S - 1);

  // Whether tile t needs a mask (uniform): the causal diagonal, the window's
  // lower edge, or keys past the end.
  auto tile_masked = [&](int t) {
    const int kt0 = t * BN;
    return (a.causal && kt0 + BN - 1 > wave_min_q) || (a.window > 0 && kt0 + a.window <= wave_max_q) ||
           (kt0 + BN > key_total);
  };
  // Exponent reference per row: exponentials of a tile are taken against ms
  // (m, or 0 while m = -inf); m rises by more than kRescaleSlack (eager) or
  // when a tile's probabilities sum past kRaiseSum (lazy). The
  // score MFMAs start from -ms, so a score accumulator holds
  // (scaled score - ms) and its exponential needs no subtraction.
  float ms[QB];
  // The score accumulators start at -ms, written into them before the first
  // MFMA (a block of -ms kept in 16 VGPRs across steps left no room for the
  // LDS reads that the step's schedule runs ahead, at 243 of 256). A masked
  // tile's accumulators start at -inf for the keys a row does not see, so the
  // MFMAs produce -inf there and the maxima and exponentials need no selects.
  // Score element i of block kb is key kb*32 + 8(i/4) + 4hl + i%4 of its tile.
  // (Keys beyond the last one are zero padding, so -inf + finite stays -inf.)
  // This issues the first 16-dim step of S(t), t = KSP*T + kh, from the
  // wave's tile of the super-tile in kbuf; score_tile<..., 1, DT> adds the
  // rest.
  auto score_first = [&](f32x16 (&s)[QB][KB], const char *kbuf, int T) {
    const int t = KSP * T + kh;
    if (KSP > 1 && (t < t_begin || t >= t_end)) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) s[qb][kb][i] = NEG_INF;
    } else if (tile_masked(t)) {
      const int kt0 = t * BN;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const int lo = vis_lo[qb] - kt0 - 4 * hl, hi = vis_hi[qb] - kt0 - 4 * hl;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int kk = kb * 32 + 8 * (i >> 2) + (i & 3);
            s[qb][kb][i] = (kk < lo || kk > hi) ? NEG_INF : -ms[qb];
          }
      }
    } else {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) s[qb][kb][i] = -ms[qb];
    }
    score_tile<D, BN, QB, 0, 1>(s, kbuf + kh * G::KBYTES, k_rd, qf);
  };
  // Row maxima of a score tile (log2 domain, the reference added back).
  auto row_max = [&](const f32x16 (&s)[QB][KB], float (&mx)[QB]) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float v = s[qb][0][0];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) v = vmax(v, s[qb][kb][i]);
      mx[qb] = xor32_max(v) + ms[qb];
    }
  };

  // One pipelined step on (super-)tile t (scores in `cur`, exponent
  // reference ms already covering tile t, O and l already scaled to it):
  //   copies of K(t+2) and V(t+1) go out;
  //   part A: the probabilities of tile t on the VALU next to the MFMAs of
  //     S(t+1) = K(t+1) Q^T (unconditional: on the last tile it reads a
  //     stale buffer and its result is ignored);
  //   part B: O^T += V(t)^T P(t)^T on the MFMAs next to the row maxima of
  //     tile t+1, which set the exponent reference of the next step;
  //   the (rare) rescale of O, after the PV MFMAs; one barrier.
  // O selects the buffers; a wave reads its own tile of each super-tile.
  auto step = [&](auto O_, int t, f32x16 (&cur)[QB][KB], f32x16 (&nxt)[QB][KB]) {
    constexpr int O = decltype(O_)::value;
    char *const k_this = O ? k_lds1 : k_lds0;  // receives K(t+2)
    char *const k_next = O ? k_lds0 : k_lds1;  // holds K(t+1)
    char *const v_this = O ? v_lds1 : v_lds0;  // holds V(t)
    char *const v_next = O ? v_lds0 : v_lds1;  // receives V(t+1)
    const char *const k_mine = k_next + kh * G::KBYTES;
    const char *const v_mine = v_this + kh * G::VBYTES;
    if (t + 2 < T_end) copy_k(t + 2, k_this);
    if (t + 1 < T_end) copy_v(t + 1, v_next);
    score_first(nxt, k_next, t + 1);

    // Part A.
    float psum[QB];
    bf16x8 pf[QB][KS];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        bf16x8 p;
#pragma unroll
        for (int j = 0; j < 8; ++j) p[j] = (bf16)fast_exp2(cur[qb][ks >> 1][8 * (ks & 1) + j]);
        // The row sum adds the bf16 probabilities the PV MFMAs use, one chain
        // per 16-key step.
        const float s8 = sum_bf16x8(p);
        psum[qb] = ks == 0 ? s8 : psum[qb] + s8;
        pf[qb][ks] = p;
      }
    }
    score_tile<D, BN, QB, 1, DT>(nxt, k_mine, k_rd, qf);
    if constexpr (QB == 1) {
      // Schedule of part A: three K fragments read ahead of the score MFMAs,
      // then per MFMA one more read and up to eight VALU operations of the
      // exponentials. Left to itself the compiler reads one fragment ahead
      // here and two in part B, and the MFMAs wait on LDS: with both
      // schedules the 4096-token causal layer (the reference-order call)
      // went from 121.7 to 118.4 us on one box.
      constexpr int NM = KB * (DT - 1);
      __builtin_amdgcn_sched_group_barrier(0x100, 3, 1);  // DS reads
#pragma unroll
      for (int i = 0; i < NM - 3; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);  // DS read
        __builtin_amdgcn_sched_group_barrier(0x002, 8, 1);  // VALU
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 3, 1);
    }

    if constexpr (LAZY) {
    // The exponent reference is raised lazily: only a row whose probabilities
    // grew large (a lane's sum above 2^16, i.e. scores well above the
    // reference) or that has seen no key yet takes the exact maximum of tile
    // t, rescales O and its sum, recomputes the tile's probabilities and
    // shifts S(t+1), which started from the old reference. No per-tile row
    // maximum is needed otherwise.
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const bool hot = (psum[qb] > kRaiseSum) | (m[qb] == NEG_INF);
      if (__ballot(hot)) {
        float v = cur[qb][0][0];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) v = vmax(v, cur[qb][kb][i]);
        const float mx = xor32_max(v) + ms[qb];  // tile t's maximum (log2 domain)
        const float mnew = mx > m[qb] ? mx : m[qb];
        const float msn = mnew == NEG_INF ? 0.0f : mnew;
        const float shift = msn - ms[qb];
        // (from m, not ms: a row that has seen no key has m = -inf, ms = 0,
        // nothing accumulated, and must scale by 0, not 2^-shift)
        const float alpha = fast_exp2(m[qb] - msn);
        l[qb] *= alpha;
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
          for (int i = 0; i < 16; ++i) oacc[qb][d][i] *= alpha;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          bf16x8 pp;
#pragma unroll
          for (int j = 0; j < 8; ++j) pp[j] = (bf16)fast_exp2(cur[qb][ks >> 1][8 * (ks & 1) + j] - shift);
          const float s8 = sum_bf16x8(pp);
          psum[qb] = ks == 0 ? s8 : psum[qb] + s8;
          pf[qb][ks] = pp;
        }
        // S(t+1) was biased by the old reference
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) nxt[qb][kb][i] -= shift;
        m[qb] = mnew;
        ms[qb] = msn;
      }
      l[qb] += psum[qb];
    }

    } else {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) l[qb] += psum[qb];
    }

    // Part B.
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        const bf16x8 vf = *reinterpret_cast<const bf16x8 *>(v_mine + d * 64 * BN + v_rd[ks]);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          oacc[qb][d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[qb][ks], oacc[qb][d], 0, 0, 0);
      }
    if constexpr (QB == 1) {
      // Schedule of part B: four V^T fragments read ahead of the PV MFMAs,
      // then one read per MFMA (the default reads two ahead, and with no VALU
      // work in this part every pair of MFMAs waits on LDS).
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // DS reads
#pragma unroll
      for (int i = 0; i < KS * DB - 4; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    }
    if constexpr (!LAZY) {
    const bool has_next = t + 1 < T_end;
    float mx[QB], alpha[QB], shift[QB];
    bool raise[QB];
    row_max(nxt, mx);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      raise[qb] = (mx[qb] > m[qb] + kRescaleSlack) & has_next;  // no short-circuit branch
      const float mnew = raise[qb] ? mx[qb] : m[qb];
      const float msn = mnew == NEG_INF ? 0.0f : mnew;
      alpha[qb] = fast_exp2(m[qb] - msn);
      shift[qb] = msn - ms[qb];  // 0 unless this row's reference rises
      l[qb] *= alpha[qb];
      m[qb] = mnew;
      ms[qb] = msn;
      // Keeps the row sum here, among the MFMAs: otherwise it is sunk past the
      // rescale branch and holds the tile's probabilities live until then.
      asm volatile("" : "+v"(l[qb]));
    }
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
      if (__ballot(raise[qb])) {
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
          for (int i = 0; i < 16; ++i) oacc[qb][d][i] *= alpha[qb];
        // S(t+1) was biased by the old reference
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) nxt[qb][kb][i] -= shift[qb];
      }
    }
    wait_copies();
    copies_barrier();
  };

  // Prologue: K(t0), V(t0), K(t0+1) copied; S(t0) and its row maxima.
  f32x16 sa[QB][KB], sb[QB][KB];
  copy_k(T_begin, k_lds0);
  copy_v(T_begin, v_lds0);
  if (T_begin + 1 < T_end) copy_k(T_begin + 1, k_lds1);
  load_q();
  wait_copies();
  copies_barrier();
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) ms[qb] = 0.0f;
  score_first(sa, k_lds0, T_begin);
  score_tile<D, BN, QB, 1, DT>(sa, k_lds0 + kh * G::KBYTES, k_rd, qf);
  {
    float mx[QB];
    row_max(sa, mx);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      m[qb] = mx[qb];
      ms[qb] = mx[qb] == NEG_INF ? 0.0f : mx[qb];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) sa[qb][kb][i] -= ms[qb];
    }
  }
  copies_barrier();  // every wave is done with K(t0) before K(t0+2) lands in its buffer

  for (int t = T_begin; t < T_end; t += 2) {
    step(std::integral_constant<int, 0>(), t, sa, sb);
    if (t + 1 < T_end) step(std::integral_constant<int, 1>(), t + 1, sb, sa);
  }

  if constexpr (KSP == 2) {
    // The pair's odd wave hands (O, m, l) of its tiles to the even wave
    // through LDS (the K buffers: the last step's barrier has passed every
    // read of them, and no copy is in flight), which merges them onto its own
    // against the larger maximum; m = -inf (no key seen) contributes nothing.
    // Layout [value][lane], one float per lane per value.
    constexpr int NX = QB * (DB * 16 + 2);
    static_assert(NX * 64 * 4 <= KSP * G::KBYTES && RB * NPB <= 2, "pair exchange fits one K buffer per pair");
    float *xch = reinterpret_cast<float *>(wq == 0 ? k_lds0 : k_lds1) + lane;
    if (kh == 1) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
          for (int i = 0; i < 16; ++i) xch[((qb * DB + d) * 16 + i) * 64] = oacc[qb][d][i];
        xch[(QB * DB * 16 + 2 * qb) * 64] = m[qb];
        xch[(QB * DB * 16 + 2 * qb + 1) * 64] = l[qb];
      }
    }
    __syncthreads();
    if (kh == 1) return;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const float m1 = xch[(QB * DB * 16 + 2 * qb) * 64], l1 = xch[(QB * DB * 16 + 2 * qb + 1) * 64];
      const float M = m[qb] > m1 ? m[qb] : m1;
      const float f0 = m[qb] == NEG_INF ? 0.0f : fast_exp2(m[qb] - M);
      const float f1 = m1 == NEG_INF ? 0.0f : fast_exp2(m1 - M);
      l[qb] = l[qb] * f0 + l1 * f1;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[qb][d][i] = oacc[qb][d][i] * f0 + xch[((qb * DB + d) * 16 + i) * 64] * f1;
      m[qb] = M;
    }
  }

  if (a.splits > 1) {  // unnormalised O and (m, l) of this key split
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int pos = wp0 + 32 * qb + lq;
      const float lt = xor32_sum(l[qb]);
      if (pos < a.S) {
        const long row = ((long)split * a.S + pos) * a.Hq + head;
        float *op = a.part_o + row * D + 4 * hl;
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            *reinterpret_cast<float4 *>(op + d * 32 + 8 * g) =
                make_float4(oacc[qb][d][4 * g], oacc[qb][d][4 * g + 1], oacc[qb][d][4 * g + 2], oacc[qb][d][4 * g + 3]);
        if (hl == 0) {
          a.part_ml[row * 2] = m[qb];
          a.part_ml[row * 2 + 1] = lt;
        }
      }
    }
    return;
  }

  // ---- epilogue: O = O^T / l ----
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int pos = wp0 + 32 * qb + lq;
    const float lt = xor32_sum(l[qb]);
    if (pos < a.S) {
      // positive, finite and non-zero, tested on the bits (NaN fails it)
      if (hl == 0 && !(__float_as_uint(lt) - 1u < 0x7f7fffffu))
        atomicOr(a.err, kDevErrSoftmaxDenominator);
      const float inv = 1.0f / lt;
      float *op = a.out + ((long)pos * a.Hq + head) * D + 4 * hl;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float4 v = make_float4(oacc[qb][d][4 * g] * inv, oacc[qb][d][4 * g + 1] * inv,
                                 oacc[qb][d][4 * g + 2] * inv, oacc[qb][d][4 * g + 3] * inv);
          *reinterpret_cast<float4 *>(op + d * 32 + 8 * g) = v;
        }
    }
  }
}


// ---- 16-query waves (v_mfma_f32_16x16x32_bf16) ----
namespace {
typedef __attribute__((ext_vector_type(4))) float f32x4q;

// Swizzle of the K tile rows read by 16-query waves: one score block reads key
// rows {0..7, 16..23} (+8, +32 j) of the tile, and the 16 lanes one LDS read
// serves take one chunk index of each: bits 0-2 and 4 of the row give 16
// distinct chunks (8 distinct among any 8 aligned lanes).
__device__ __forceinline__ constexpr int swz_k16(int row) { return (row & 7) | ((row >> 1) & 8); }

// Key (within the tile) of row rho of 16-key score block b. Blocks 2j and 2j+1
// cover keys [32j, 32j+32) so that lane group g (lanes 16g..16g+15) holds in
// its four elements of block 2j, then of block 2j+1, the eight keys of V^T
// slots 32j + 8g + [0, 8) in vt_key_slot order: P^T feeds the B operand of the
// PV MFMA with no shuffle.
__device__ __forceinline__ constexpr int key16(int b, int rho) {
  return 32 * (b >> 1) + (rho < 8 ? rho : rho + 8) + 8 * (b & 1);
}

__device__ __forceinline__ float xor16_max(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
}  // namespace

// The head_dim-256 prefill: waves of 16 queries on v_mfma_f32_16x16x32_bf16.
// A wave holds the whole head dim of its 16 queries (O^T 64 VGPRs, Q^T 32), so
// no O split or score exchange between waves is needed. RB heads x NPB blocks
// of 16 queries per workgroup, BN-key tiles, the masks and key splits of
// prefill_kernel, lazy exponent reference. NST K and V^T stages of LDS: two
// (two workgroups per CU) with the step order of prefill_kernel, or four (one
// per CU) with DEEP, a software-pipelined step (fragment reads ahead of the
// MFMAs, copies spread among them) for a lone wave per SIMD.
//   S^T = K Q^T   A = 16 key rows x 32 dims from LDS (rows key16(b, lane %
//                 16)), B = Q^T in registers; lane l holds keys key16(b,
//                 4 (l / 16) + i) of query l % 16;
//   O^T += V^T P^T  A = 16 dim rows x 32 V^T slots from LDS, B = P^T from
//                 the score registers (key16 makes them the slots' keys).
template <int D, int RB, int NPB, int BN, int NST, bool DEEP>
__global__ __launch_bounds__(RB *NPB * 64, NST > 2 ? 1 : 2) void prefill_q16_kernel(const PrefillArgs a) {
  static_assert(NST == 2 || NST == 4, "the step loop alternates two score buffers over NST stages");
  constexpr int NW = RB * NPB;
  constexpr int WGQ = NPB * 16;
  using G = Geom<D, BN, NW>;
  constexpr int DT = D / 32;   // 32-dim steps of S^T = K Q^T
  constexpr int KB = BN / 16;  // 16-key score blocks
  constexpr int KS = BN / 32;  // 32-key steps of O^T += V^T P^T
  constexpr int DB = D / 16;   // 16-dim output blocks
  static_assert(D >= 128 && D / 8 >= 16, "swz_k16 needs 16 chunks per K row");

  // One named array per stage: the compiler then sees that a read of one stage
  // does not alias the copies into another and waits for no copy before it.
  constexpr int KB2 = NST > 2 ? G::KBYTES : 16, VB2 = NST > 2 ? G::VBYTES : 16;
  __shared__ __attribute__((aligned(1024))) char k_lds0[G::KBYTES];
  __shared__ __attribute__((aligned(1024))) char k_lds1[G::KBYTES];
  __shared__ __attribute__((aligned(1024))) char k_lds2[KB2];
  __shared__ __attribute__((aligned(1024))) char k_lds3[KB2];
  __shared__ __attribute__((aligned(1024))) char v_lds0[G::VBYTES];
  __shared__ __attribute__((aligned(1024))) char v_lds1[G::VBYTES];
  __shared__ __attribute__((aligned(1024))) char v_lds2[VB2];
  __shared__ __attribute__((aligned(1024))) char v_lds3[VB2];
  auto k_lds = [&](auto I_) -> char * {
    constexpr int I = decltype(I_)::value % NST;
    if constexpr (I == 0) return k_lds0;
    else if constexpr (I == 1) return k_lds1;
    else if constexpr (I == 2) return k_lds2;
    else return k_lds3;
  };
  auto v_lds = [&](auto I_) -> char * {
    constexpr int I = decltype(I_)::value % NST;
    if constexpr (I == 0) return v_lds0;
    else if constexpr (I == 1) return v_lds1;
    else if constexpr (I == 2) return v_lds2;
    else return v_lds3;
  };
  using I0 = std::integral_constant<int, 0>;

  const int HB = a.R / RB;
  int h, hb, split, qt;
  if (a.xcd_group == 1) {
    const int Gq = HB * a.n_qblocks;
    const int lo = (int)(blockIdx.x & 7), rest = (int)(blockIdx.x >> 3);
    const int gg = rest % Gq, unit = (rest / Gq) * 8 + lo;
    if (unit >= a.Hkv * a.splits) return;
    h = unit % a.Hkv;
    split = unit / a.Hkv;
    hb = gg % HB;
    qt = a.n_qblocks - 1 - gg / HB;
  } else {
    int bid = blockIdx.x;
    if (a.xcd_group == 2) {
      bid = (int)(blockIdx.x & 7) * (int)(gridDim.x >> 3) + (int)(blockIdx.x >> 3);
      if (bid >= a.n_qblocks * HB * a.Hkv * a.splits) return;
    }
    const int hh = bid % (a.Hkv * HB);
    bid /= (a.Hkv * HB);
    split = bid % a.splits;
    bid /= a.splits;
    qt = a.n_qblocks - 1 - bid;
    h = hh / HB;
    hb = hh % HB;
  }
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int r = wave % RB, pb = wave / RB;
  const int head = h * a.R + hb * RB + r;
  const int p0 = qt * WGQ;
  const int wp0 = p0 + pb * 16;
  const int lq = lane & 15, g = lane >> 4;
  const int key_total = a.P + a.S;

  int key_end = key_total;
  if (a.causal) key_end = min(key_total, a.P + min(a.S, p0 + WGQ));
  int key_begin = 0;
  if (a.window > 0) key_begin = max(0, a.P + p0 - a.window + 1);
  int t_begin = key_begin / BN;
  int t_end = (key_end + BN - 1) / BN;
  if (a.splits > 1) {
    t_begin += split * a.tps;
    t_end = min(t_end, t_begin + a.tps);
  }
  if (t_begin >= t_end) {
    const int pos = wp0 + lane;
    if (lane < 16 && pos < a.S) {
      float *ml = a.part_ml + (((long)split * a.S + pos) * a.Hq + head) * 2;
      ml[0] = -__builtin_inff();
      ml[1] = 0.0f;
    }
    return;
  }

  // Q^T (B operand): lane holds query lq, dims 32t + 8g + [0, 8), carrying the
  // softmax scale times log2(e).
  bf16x8 qf[DT];
  {
    const int pos = min(wp0 + lq, a.S - 1);
    if (a.qb) {
      const bf16 *qp = a.qb + ((long)pos * a.Hq + head) * D + 8 * g;
#pragma unroll
      for (int t = 0; t < DT; ++t) qf[t] = *reinterpret_cast<const bf16x8 *>(qp + 32 * t);
    } else {
      const float c = a.qk_scale_log2;
      const float *qp = a.q + ((long)pos * a.Hq + head) * D + 8 * g;
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const float4 x0 = *reinterpret_cast<const float4 *>(qp + 32 * t);
        const float4 x1 = *reinterpret_cast<const float4 *>(qp + 32 * t + 4);
        bf16x8 v;
        v[0] = (bf16)(x0.x * c); v[1] = (bf16)(x0.y * c); v[2] = (bf16)(x0.z * c); v[3] = (bf16)(x0.w * c);
        v[4] = (bf16)(x1.x * c); v[5] = (bf16)(x1.y * c); v[6] = (bf16)(x1.z * c); v[7] = (bf16)(x1.w * c);
        qf[t] = v;
      }
    }
  }
  f32x4q o[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) o[d] = f32x4q{0.0f, 0.0f, 0.0f, 0.0f};
  float m = NEG_INF, l = 0.0f, ms = 0.0f;
  f32x4q bias = f32x4q{0.0f, 0.0f, 0.0f, 0.0f};

  // LDS read offsets. K block b, dim step t: row key16(b, lq), chunk
  // (4t + g) ^ swz_k16(row) = offset kbase[b] ^ (t << 6).
  unsigned kbase[KB];
#pragma unroll
  for (int b = 0; b < KB; ++b) {
    const int row = key16(b, lq), sw = swz_k16(row);
    kbase[b] = (unsigned)(row * 2 * D + 16 * (g ^ (sw & 3)) + 64 * (sw >> 2));
  }
  // V^T dim block db, 32-key step s: row 16 db + lq, chunk (4s + g) ^ swz(row)
  // (swz of the V^T tile depends on the row's low four bits only).
  unsigned vbase;
  {
    const int sv = swz<G::VNC>(lq);
    vbase = (unsigned)(lq * 2 * BN + 16 * (g ^ (sv & 3)) + 64 * (sv >> 2));
  }

  // Copies: copy j of the wave fills LDS bytes [(wave + j*NW) * 1024, +1024).
  auto k_src = [&](int j) {
    const int byte = (wave + j * NW) * 1024 + lane * 16;
    const int row = byte / (2 * D), p = (byte % (2 * D)) / 16;
    return (unsigned)(row * D + 8 * (p ^ swz_k16(row))) * 2u;
  };
  auto v_src = [&](int j, unsigned stride) {
    const int byte = (wave + j * NW) * 1024 + lane * 16;
    const int d = byte / (2 * BN), p = (byte % (2 * BN)) / 16;
    return ((unsigned)d * stride + (unsigned)(8 * (p ^ swz<G::VNC>(d)))) * 2u;
  };
  const char *kb_c = reinterpret_cast<const char *>(a.kb_cache + (long)h * a.cap_cache * D);
  const char *kb_s = reinterpret_cast<const char *>(a.kb_stage + (long)h * a.cap_stage * D);
  const char *vt_c = reinterpret_cast<const char *>(a.vt_cache + (long)h * D * a.cap_cache);
  const char *vt_s = reinterpret_cast<const char *>(a.vt_stage + (long)h * D * a.cap_stage);
  const unsigned vt_stride_c = __builtin_amdgcn_readfirstlane((unsigned)a.cap_cache);
  const unsigned vt_stride_s = __builtin_amdgcn_readfirstlane((unsigned)a.cap_stage);
  auto copy_k = [&](int t, char *dst) {
    const int nk = t * BN;
    const char *src = nk < a.P8 ? kb_c + (long)nk * D * 2 : kb_s + (long)(nk - a.P8) * D * 2;
#pragma unroll
    for (int j = 0; j < G::KDMA; ++j) dma16_untracked(src, k_src(j), dst + (wave + j * NW) * 1024);
  };
  auto copy_v = [&](int t, char *dst) {
    const int nk = t * BN;
    const bool cached = nk < a.P8;
    const char *src = cached ? vt_c + (long)nk * 2 : vt_s + (long)(nk - a.P8) * 2;
    const unsigned stride = cached ? vt_stride_c : vt_stride_s;
#pragma unroll
    for (int j = 0; j < G::VDMA; ++j) dma16_untracked(src, v_src(j, stride), dst + (wave + j * NW) * 1024);
  };
  // Copy j (of KDMA + VDMA) of this wave's share of K(tk) and V(tv).
  auto copy_kv1 = [&](int tk, char *kdst, int tv, char *vdst, int j) {
    if (j < G::KDMA) {
      const int nk = tk * BN;
      const char *src = nk < a.P8 ? kb_c + (long)nk * D * 2 : kb_s + (long)(nk - a.P8) * D * 2;
      dma16_untracked(src, k_src(j), kdst + (wave + j * NW) * 1024);
    } else {
      const int nk = tv * BN;
      const bool cached = nk < a.P8;
      const char *src = cached ? vt_c + (long)nk * 2 : vt_s + (long)(nk - a.P8) * 2;
      const unsigned stride = cached ? vt_stride_c : vt_stride_s;
      dma16_untracked(src, v_src(j - G::KDMA, stride), vdst + (wave + (j - G::KDMA) * NW) * 1024);
    }
  };

  const int q_abs = a.P + wp0 + lq;
  const int vis_hi = a.causal ? min(q_abs, key_total - 1) : key_total - 1;
  const int vis_lo = a.window > 0 ? q_abs - a.window + 1 : 0;
  const int wave_min_q = a.P + wp0;
  const int wave_max_q = a.P + min(wp0 + 15, a.S - 1);
  const int gk = 4 * g + 8 * (g >> 1);  // key16(b, 4g + i) = 32 (b >> 1) + 8 (b & 1) + i + gk
  auto tile_masked = [&](int t) {
    const int kt0 = t * BN;
    return (a.causal && kt0 + BN - 1 > wave_min_q) || (a.window > 0 && kt0 + a.window <= wave_max_q) ||
           (kt0 + BN > key_total);
  };
  // S^T of tile t into s (scaled score minus ms; -inf where masked): the
  // accumulators' start values, then the MFMAs.
  auto score_init = [&](f32x4q (&s)[KB], int t) {
    if (tile_masked(t)) {
      const int kt0 = t * BN;
      const int lo = vis_lo - kt0 - gk, hi = vis_hi - kt0 - gk;
#pragma unroll
      for (int b = 0; b < KB; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kk = 32 * (b >> 1) + 8 * (b & 1) + i;
          s[b][i] = (kk < lo || kk > hi) ? NEG_INF : -ms;
        }
    } else {
#pragma unroll
      for (int b = 0; b < KB; ++b) s[b] = bias;
    }
  };
  // Fragment i of the K tile (dim step i / KB, block i % KB) and of the V^T
  // tile (32-key step i / DB, dim block i % DB).
  auto read_k = [&](const char *kbuf, int i) {
    return *reinterpret_cast<const bf16x8 *>(kbuf + (kbase[i % KB] ^ (unsigned)((i / KB) << 6)));
  };
  auto read_v = [&](const char *vbuf, int i) {
    return *reinterpret_cast<const bf16x8 *>(vbuf + ((vbase ^ (unsigned)((i / DB) << 6)) + (i % DB) * 16 * 2 * BN));
  };
  auto score = [&](f32x4q (&s)[KB], const char *kbuf, int t) {
    score_init(s, t);
#pragma unroll
    for (int i = 0; i < DT * KB; ++i)
      s[i % KB] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(read_k(kbuf, i), qf[i / KB], s[i % KB], 0, 0, 0);
    if constexpr (!DEEP) {
      // Four K fragments read ahead of the score MFMAs, and the exponentials
      // of the step spread among them; the PV loop below reads four V^T
      // fragments ahead too. Left to itself the compiler reads one fragment
      // ahead and every 16-cycle MFMA waits on LDS (Gemma-3-1B's global 4096
      // layer: 95.7 against 87.2 us; three ahead 89, six 89).
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 2);  // DS reads
#pragma unroll
      for (int i = 0; i < DT * KB - 4; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 2);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 2);  // DS read
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 2);  // VALU
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 2);
    }
  };

  // K(j) and V(j) live in stage (j - t_begin) % NST. Step t copies K(t + NST)
  // into K(t)'s stage (its scores were taken one step earlier) and V(t + NST -
  // 1) into V(t - 1)'s stage, and needs K(t + 1) and V(t) landed; at its end it
  // waits for K(t + 2) and V(t + 1) only. In copy order the pairs are K(t0),
  // then (K(t0 + k), V(t0 + k - 1)) for k = 1, 2, ...; pending(t, k0, k1) counts
  // this wave's copies in pairs (K(t + k), V(t + k - 1)), k0 <= k <= k1.
  static_assert(G::KDMA == G::VDMA, "pending() counts K and V copies in equal groups");
  // Deep steps: software-pipelined, PF fragment pairs read ahead (4, 6 and 8
  // measured alike).
  constexpr int PF = 4;
  static_assert(!DEEP || DT * KB == KS * DB, "deep steps pair K and V fragments");
  auto pending = [&](int t, int k0, int k1) {
    int n = 0;
#pragma unroll
    for (int k = k0; k <= k1; ++k) n += (t + k < t_end ? G::KDMA : 0) + (t + k - 1 < t_end ? G::VDMA : 0);
    return n;
  };
  auto step = [&](auto Ph_, int t, f32x4q (&cur)[KB], f32x4q (&nxt)[KB]) {
    constexpr int Ph = decltype(Ph_)::value;  // (t - t_begin) % NST
    char *const k_next = k_lds(std::integral_constant<int, Ph + 1>());  // holds K(t+1)
    char *const v_this = v_lds(Ph_);                                    // holds V(t)
    // (the scores of tile t + 1 read a stale buffer on the last tile; ignored)
    constexpr int NF = DT * KB;  // fragments of each kind per step
    bf16x8 kf[DEEP ? NF : 1], vf[DEEP ? NF : 1];
    if constexpr (DEEP) {
      // Software pipeline for one wave per SIMD: fragment reads run PF pairs
      // ahead of their MFMAs and the step's copies are spread over the MFMAs,
      // so the LDS, the copy path and the matrix unit work at the same time.
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        kf[i] = read_k(k_next, i);
        vf[i] = read_v(v_this, i);
      }
    } else {
      if (t + NST < t_end) copy_k(t + NST, k_lds(Ph_));
      if (t + NST - 1 < t_end) copy_v(t + NST - 1, v_lds(std::integral_constant<int, Ph + NST - 1>()));
      score(nxt, k_next, t + 1);
    }

    // probabilities of tile t, P^T for the PV B operand
    bf16x8 pf[KS];
    float psum = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      bf16x8 p;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = (bf16)fast_exp2(cur[2 * s][i]);
        p[4 + i] = (bf16)fast_exp2(cur[2 * s + 1][i]);
      }
      psum += sum_bf16x8(p);
      pf[s] = p;
    }
    const bool hot = (psum > kRaiseSum) | (m == NEG_INF);
    if (__ballot(hot)) {
      float v = cur[0][0];
#pragma unroll
      for (int b = 0; b < KB; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) v = vmax(v, cur[b][i]);
      const float mx = xor32_max(xor16_max(v)) + ms;
      const float mnew = mx > m ? mx : m;
      const float msn = mnew == NEG_INF ? 0.0f : mnew;
      const float shift = msn - ms;
      const float alpha = fast_exp2(m - msn);  // 0 for a row that has seen no key
      l *= alpha;
#pragma unroll
      for (int d = 0; d < DB; ++d) o[d] *= alpha;
      psum = 0.0f;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        bf16x8 p;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[i] = (bf16)fast_exp2(cur[2 * s][i] - shift);
          p[4 + i] = (bf16)fast_exp2(cur[2 * s + 1][i] - shift);
        }
        psum += sum_bf16x8(p);
        pf[s] = p;
      }
      if constexpr (!DEEP) {
#pragma unroll
        for (int b = 0; b < KB; ++b) nxt[b] -= shift;
      }
      bias = f32x4q{-msn, -msn, -msn, -msn};
      m = mnew;
      ms = msn;
    }
    l += psum;
    if constexpr (DEEP) {
      score_init(nxt, t + 1);  // (after the reference update: no shift of nxt needed)
      // Every step copies K(t + NST) and V(t + NST - 1), clamped to the last
      // tile past the range (into stages no later step reads), so the waits
      // count a fixed number of copies.
      const int tk = min(t + NST, t_end - 1), tv = min(t + NST - 1, t_end - 1);
      char *const kdst = k_lds(Ph_);
      char *const vdst = v_lds(std::integral_constant<int, Ph + NST - 1>());
      constexpr int NC = G::KDMA + G::VDMA;
      static_assert(NF % NC == 0, "copies spread evenly over the MFMA pairs");
#pragma unroll
      for (int i = 0; i < NF; ++i) {
        nxt[i % KB] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[i], qf[i / KB], nxt[i % KB], 0, 0, 0);
        o[i % DB] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[i], pf[i / DB], o[i % DB], 0, 0, 0);
        if (i + PF < NF) {
          kf[i + PF] = read_k(k_next, i + PF);
          vf[i + PF] = read_v(v_this, i + PF);
        }
        if (i % (NF / NC) == NF / NC - 1) copy_kv1(tk, kdst, tv, vdst, i / (NF / NC));
      }
    } else {
#pragma unroll
      for (int i = 0; i < KS * DB; ++i)
        o[i % DB] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(read_v(v_this, i), pf[i / DB], o[i % DB], 0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 3);  // DS reads
#pragma unroll
      for (int i = 0; i < KS * DB - 4; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 3);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 3);  // DS read
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 3);
    }
    if constexpr (DEEP) wait_copies_upto<(NST - 2) * 2 * G::KDMA, G::KDMA>((NST - 2) * 2 * G::KDMA);
    else wait_copies_upto<(NST - 2) * 2 * G::KDMA, G::KDMA>(pending(t, 3, NST));
    copies_barrier();
  };

  // Prologue: K(t0) .. K(t0 + NST - 1), V(t0) .. V(t0 + NST - 2); S(t0).
  f32x4q sa[KB], sb[KB];
  copy_k(t_begin, k_lds(I0()));
  auto prologue_pair = [&](auto K_) {
    constexpr int k = decltype(K_)::value;
    if constexpr (k < NST) {
      if constexpr (DEEP) {  // (clamped as in the steps)
        copy_k(min(t_begin + k, t_end - 1), k_lds(K_));
        copy_v(min(t_begin + k - 1, t_end - 1), v_lds(std::integral_constant<int, k - 1>()));
      } else {
        if (t_begin + k < t_end) copy_k(t_begin + k, k_lds(K_));
        if (t_begin + k - 1 < t_end) copy_v(t_begin + k - 1, v_lds(std::integral_constant<int, k - 1>()));
      }
    }
  };
  prologue_pair(std::integral_constant<int, 1>());
  prologue_pair(std::integral_constant<int, 2>());
  prologue_pair(std::integral_constant<int, 3>());
  wait_copies_upto<(NST - 1) * 2 * G::KDMA, G::KDMA>(DEEP ? (NST - 1) * 2 * G::KDMA : pending(t_begin, 1, NST - 1));
  copies_barrier();
  score(sa, k_lds(I0()), t_begin);
  wait_copies_upto<(NST - 2) * 2 * G::KDMA, G::KDMA>(DEEP ? (NST - 2) * 2 * G::KDMA : pending(t_begin, 2, NST - 1));
  copies_barrier();  // K(t0+1) and V(t0) landed; every wave is done with K(t0) before K(t0+NST) lands there

  for (int t = t_begin; t < t_end; t += NST) {
    step(std::integral_constant<int, 0>(), t, sa, sb);
    if (t + 1 < t_end) step(std::integral_constant<int, 1>(), t + 1, sb, sa);
    if constexpr (NST == 4) {
      if (t + 2 < t_end) step(std::integral_constant<int, 2>(), t + 2, sa, sb);
      if (t + 3 < t_end) step(std::integral_constant<int, 3>(), t + 3, sb, sa);
    }
  }

  const float lt = xor32_sum(xor16_sum(l));
  const int pos = wp0 + lq;
  if (a.splits > 1) {
    if (pos < a.S) {
      const long row = ((long)split * a.S + pos) * a.Hq + head;
      float *op = a.part_o + row * D + 4 * g;
#pragma unroll
      for (int d = 0; d < DB; ++d)
        *reinterpret_cast<float4 *>(op + 16 * d) = make_float4(o[d][0], o[d][1], o[d][2], o[d][3]);
      if (g == 0) {
        a.part_ml[row * 2] = m;
        a.part_ml[row * 2 + 1] = lt;
      }
    }
    return;
  }
  if (pos < a.S) {
    if (g == 0 && !(__float_as_uint(lt) - 1u < 0x7f7fffffu)) atomicOr(a.err, kDevErrSoftmaxDenominator);
    const float inv = 1.0f / lt;
    float *op = a.out + ((long)pos * a.Hq + head) * D + 4 * g;
#pragma unroll
    for (int d = 0; d < DB; ++d)
      *reinterpret_cast<float4 *>(op + 16 * d) = make_float4(o[d][0] * inv, o[d][1] * inv, o[d][2] * inv, o[d][3] * inv);
  }
}

namespace {

template <int D, int RB, int NPB, int BN, int NST, bool DEEP>
hipError_t launch_q16(hipStream_t st, PrefillArgs a) {
  constexpr int WGQ = NPB * 16;
  a.n_qblocks = (a.S + WGQ - 1) / WGQ;
  const long blocks = prefill_grid_workgroups(a.n_qblocks, a.R / RB, a.Hkv, a.splits, a.xcd_group);
  hipLaunchKernelGGL((prefill_q16_kernel<D, RB, NPB, BN, NST, DEEP>), dim3((unsigned)blocks), dim3(RB * NPB * 64), 0,
                     st, a);
  return hipGetLastError();
}

template <int D, int RB, int NPB, int BN, int QB, int KSP>
hipError_t launch_shape(hipStream_t st, PrefillArgs a) {
  constexpr int WGQ = NPB * QB * 32;
  a.n_qblocks = (a.S + WGQ - 1) / WGQ;
  const long blocks = prefill_grid_workgroups(a.n_qblocks, a.R / RB, a.Hkv, a.splits, a.xcd_group);
  hipLaunchKernelGGL((prefill_kernel<D, RB, NPB, BN, QB, KSP>), dim3((unsigned)blocks), dim3(RB * NPB * KSP * 64),
                     0, st, a);
  return hipGetLastError();
}

// Four-wave workgroups of 32 queries per wave, 64-key tiles, two waves per
// SIMD: four heads of the KV group, two heads with two blocks, or one head
// with four blocks. (64 queries per wave halves the LDS fragment reads per
// MFMA but, at head_dim 128, needs more than 256 VGPRs and measured slower;
// at head_dim 64 it halves the workgroup count, which a 2048-token prefill
// cannot afford.)
// Wave pairs (head_dim 64, prefill_wave_pairs): two heads, or one head with
// two blocks, each block's key tiles split between the two waves of a pair.
template <int D>
hipError_t launch_r(hipStream_t st, const PrefillArgs &a) {
  constexpr int BN = 64;
  if constexpr (D == 64) {
    if (a.ksp == 2) {
      if (a.R % 2 == 0) return launch_shape<D, 2, 1, BN, 1, 2>(st, a);
      return launch_shape<D, 1, 2, BN, 1, 2>(st, a);
    }
  }
  if (a.R % 4 == 0) return launch_shape<D, 4, 1, BN, 1, 1>(st, a);
  if (a.R % 2 == 0) return launch_shape<D, 2, 2, BN, 1, 1>(st, a);
  return launch_shape<D, 1, 4, BN, 1, 1>(st, a);
}

// head_dim 256: four waves of 16 queries, 32-key tiles: four heads, two heads
// with two blocks, or one head with four blocks.
template <int D, int NST, bool DEEP>
hipError_t launch_r16n(hipStream_t st, const PrefillArgs &a) {
  constexpr int BN = 32;
  if (a.R % 4 == 0) return launch_q16<D, 4, 1, BN, NST, DEEP>(st, a);
  if (a.R % 2 == 0) return launch_q16<D, 2, 2, BN, NST, DEEP>(st, a);
  return launch_q16<D, 1, 4, BN, NST, DEEP>(st, a);
}
// Windowed layers (one workgroup per CU at Gemma-3-1B's 4096 tokens): four
// stages and the software-pipelined step. Full causal layers: two stages and
// two workgroups per CU, where the pipelined step measured slower.
template <int D>
hipError_t launch_r16(hipStream_t st, const PrefillArgs &a) {
  if (a.window > 0) return launch_r16n<D, 4, true>(st, a);
  return launch_r16n<D, 2, false>(st, a);
}

template <int D>
hipError_t launch_d(hipStream_t st, const PrefillArgs &a) {
  if constexpr (D >= 256) return launch_r16<D>(st, a);
  else return launch_r<D>(st, a);
}

}  // namespace


bool prefill_supported(int D) { return D == 64 || D == 128 || D == 256; }

// Workgroups of four waves (launch_r, launch_r16 above): four heads, two
// heads with two query blocks, or one head with four blocks; a wave's block is
// 32 queries (16 at head_dim 256), so a workgroup covers 128 query rows (64).
// With wave pairs (a.ksp == 2) two waves share a block: two heads, or one
// head with two blocks.
int prefill_wg_heads(const PrefillArgs &a, int) {
  if (a.ksp == 2) return a.R % 2 == 0 ? 2 : 1;
  return a.R % 4 == 0 ? 4 : a.R % 2 == 0 ? 2 : 1;
}
int prefill_wg_queries(const PrefillArgs &a, int D) {
  return (D >= 256 ? 64 : 128) / (prefill_wg_heads(a, D) * (a.ksp == 2 ? 2 : 1));
}
// Wave pairs for causal head_dim-64 prompts (fewer cached keys than
// queries) whose paired grid still fits one round of workgroup slots: there
// the longest query blocks' tile chain sets the launch time, and a pair
// halves it. A pair's workgroup covers half the heads, so each K/V tile copy
// serves half the waves: with a second round of workgroups that costs more
// than the chain saves. Llama-3.2-1B (32/8 heads) prompts, reference-order
// call per layer: 1024 tokens 24.2 -> 21.2 us, 512 15.5 -> 13.9 us, 256
// 12.0 -> 11.0 us; 2048 tokens (two rounds paired) 42.9 against 46.1 us.
int prefill_wave_pairs(const PrefillArgs &a, int D, long slots) {
  if (D != 64 || !a.causal || a.window > 0 || a.S < 2 * 64 || a.P >= a.S) return 1;
  PrefillArgs b = a;
  b.ksp = 1;
  return 2 * prefill_base_workgroups(b, D) <= slots ? 2 : 1;
}
// Windowed head_dim-256 layers run the four-stage kernel (128 KB of LDS).
int prefill_wgs_per_cu(const PrefillArgs &a, int D) { return D >= 256 && a.window > 0 ? 1 : 2; }
int prefill_tile_keys(int D) { return D >= 256 ? 32 : 64; }  // BN of launch_d

long prefill_base_workgroups(const PrefillArgs &a, int D) {
  const int wgq = prefill_wg_queries(a, D);
  return (long)((a.S + wgq - 1) / wgq) * a.Hkv * (a.R / prefill_wg_heads(a, D));
}

long prefill_grid_workgroups(long n_qblocks, long head_blocks, long Hkv, long splits, int xcd_group) {
  const long n = n_qblocks * head_blocks * Hkv * splits;
  if (xcd_group == 2) return (n + 7) / 8 * 8;
  if (!xcd_group) return n;
  const long units = (Hkv * splits + 7) / 8 * 8;
  return units * head_blocks * n_qblocks;
}

int prefill_use_xcd_group(const PrefillArgs &a, int D) {
  const int wgq = prefill_wg_queries(a, D);
  const long G = (long)(a.R / prefill_wg_heads(a, D)) * ((a.S + wgq - 1) / wgq);
  if (a.splits > 1 && (long)a.Hkv * a.splits >= 8 && G > 1) return 1;
  // Unsplit windowed layers of at least two workgroups per XCD: a contiguous
  // run of query blocks per XCD, whose windows overlap in that XCD's L2
  // (round-robin ids make every XCD fetch nearly all of the keys).
  if (a.splits == 1 && a.window > 0 && G * a.Hkv >= 16) return 2;
  return 0;
}

// The largest t_end - t_begin of prefill_kernel over its query blocks, with
// the kernel's own range arithmetic: causal blocks end at their last query,
// non-causal ones at the last key; a window starts each block at its first
// query's window.
long prefill_max_tile_span(const PrefillArgs &a, int D) {
  const long wgq = prefill_wg_queries(a, D), bn = prefill_tile_keys(D);
  const long key_total = (long)a.P + a.S;
  const long nq = (a.S + wgq - 1) / wgq;
  long span = 0;
  for (long qt = 0; qt < nq; ++qt) {
    const long p0 = qt * wgq;
    long key_end = key_total;
    if (a.causal) key_end = std::min(key_total, (long)a.P + std::min((long)a.S, p0 + wgq));
    long key_begin = 0;
    if (a.window > 0) key_begin = std::max(0L, (long)a.P + p0 - a.window + 1);
    span = std::max(span, (key_end + bn - 1) / bn - key_begin / bn);
  }
  return span;
}

// Merges key splits: per (query row, head), M = max m_j, then
// O = sum_j O_j 2^(m_j - M), L = sum_j l_j 2^(m_j - M), out = O / L. Splits
// that saw no key of the row (m_j = -inf; their O was never written) are
// skipped. WPR waves share
// a row (WPR = 1: four rows per workgroup; WPR = 4: one): lane l holds the
// row's elements [l * D/64, (l + 1) * D/64), the lanes find M together, and
// wave w sums splits w, w + WPR, ... in order, reading each split's (m, l)
// pair on every lane (one line per split). With WPR = 4 the four partial sums
// meet in LDS, in wave order. The error bit is set for an invalid L, as the
// unsplit kernels do (rotary.rs:560-564).
constexpr int kMaxPrefillSplits = 256;
// Above this many splits a row gets a whole workgroup.
constexpr int kCombineWaveSplits = 8;

template <int E>
__device__ __forceinline__ void load_e(const float *p, float (&v)[E]) {
  if constexpr (E == 4) {
    const float4 q = *reinterpret_cast<const float4 *>(p);
    v[0] = q.x, v[1] = q.y, v[2] = q.z, v[3] = q.w;
  } else if constexpr (E == 2) {
    const float2 q = *reinterpret_cast<const float2 *>(p);
    v[0] = q.x, v[1] = q.y;
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = p[e];
  }
}

template <int D, int WPR>
__global__ __launch_bounds__(256) void prefill_combine_kernel(const PrefillArgs a) {
  constexpr int E = D / 64;
  __shared__ float s_o[WPR > 1 ? WPR : 1][64][E];
  __shared__ float s_l[WPR > 1 ? WPR : 1];
  const long rows = (long)a.S * a.Hq;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * (4 / WPR) + wave / WPR;  // pos * Hq + head
  const int sub = wave % WPR;
  if (WPR == 1 && row >= rows) return;  // whole waves; with WPR > 1 the grid is exact
  const float *ml = a.part_ml + row * 2;  // split j at ml[j * rows * 2]
  float M = -__builtin_inff();
  for (int j = lane; j < a.splits; j += 64) M = fmaxf(M, ml[j * rows * 2]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
  const float Ms = M == -__builtin_inff() ? 0.0f : M;
  float L = 0.0f, O[E];
#pragma unroll
  for (int e = 0; e < E; ++e) O[e] = 0.0f;
  const float *po = a.part_o + row * D + lane * E;
#pragma unroll 8
  for (int j = sub; j < a.splits; j += WPR) {
    const float mj = ml[j * rows * 2], lj = ml[j * rows * 2 + 1];
    // a split that saw none of the row's keys wrote no O: skip it (uniform)
    if (mj == -__builtin_inff()) continue;
    const float g = __builtin_amdgcn_exp2f(mj - Ms);
    float o[E];
    load_e<E>(po + j * rows * D, o);
#pragma unroll
    for (int e = 0; e < E; ++e) O[e] = fmaf(o[e], g, O[e]);
    L = fmaf(lj, g, L);
  }
  if constexpr (WPR > 1) {
#pragma unroll
    for (int e = 0; e < E; ++e) s_o[sub][lane][e] = O[e];
    if (lane == 0) s_l[sub] = L;
    __syncthreads();
    if (sub != 0) return;
#pragma unroll
    for (int w = 1; w < WPR; ++w) {
#pragma unroll
      for (int e = 0; e < E; ++e) O[e] += s_o[w][lane][e];
      L += s_l[w];
    }
  }
  float *dst = a.out + row * D + lane * E;
#pragma unroll
  for (int e = 0; e < E; ++e) dst[e] = O[e] / L;
  if (lane == 0 && !(__float_as_uint(L) - 1u < 0x7f7fffffu)) atomicOr(a.err, kDevErrSoftmaxDenominator);
}

template <int D>
hipError_t launch_combine_d(hipStream_t st, const PrefillArgs &a) {
  const long rows = (long)a.S * a.Hq;
  if (a.splits > kCombineWaveSplits) {
    hipLaunchKernelGGL((prefill_combine_kernel<D, 4>), dim3((unsigned)rows), dim3(256), 0, st, a);
  } else {
    hipLaunchKernelGGL((prefill_combine_kernel<D, 1>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

hipError_t launch_prefill_combine(hipStream_t st, const PrefillArgs &a, int D) {
  if (a.splits <= 1) return hipSuccess;
  if (a.splits > kMaxPrefillSplits) return hipErrorInvalidValue;
  switch (D) {
    case 64: return launch_combine_d<64>(st, a);
    case 128: return launch_combine_d<128>(st, a);
    case 256: return launch_combine_d<256>(st, a);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_prefill(hipStream_t st, const PrefillArgs &a, int D) {
  switch (D) {
    case 64: return launch_d<64>(st, a);
    case 128: return launch_d<128>(st, a);
    case 256: return launch_d<256>(st, a);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace spissa
