// linear.hip -- the projections on either side of the attention path:
// out[M, N] = x[M, K] x W[N, K]^T + bias[N] with f32 activations and output
// and the weight resident in HBM as bf16, f16 or f32
// (crates/spissa-runtime/src/streaming/linear.rs:269-576,
// streaming_tile_linear_from_model, whose exact default accumulates each
// output as bias + a sequential f32 dot: streaming/kernels_raw16.rs:532-600,
// streaming/mod.rs:311-320; the plain form is ops.rs:62-105 linear).
//
// Four kernels:
//  - linear_gemv_kernel (M <= 4 tokens, the decode projections): bound by the
//    weight bytes. A wave owns two weight rows; each lane streams 16-byte
//    pieces of them (8 bf16/f16 or 4 f32 weights) with the matching
//    activations from the cache, accumulates in f32, and the wave sums its
//    lanes with DPP and permlane exchanges.
//  - linear_skinny_kernel (bf16 weights, 5 <= M <= 64, K % 128 == 0: batched
//    decode): weight fragments straight from HBM into 16x16x32 MFMAs, the
//    activations split as below, K split over the workgroup's four waves.
//  - linear_gemm_kernel (bf16 weights, M > 64, K % 32 == 0: prefill): MFMA
//    v_mfma_f32_32x32x16_bf16 on 128 x 256 or 256 x 320 output tiles, 32-deep
//    k tiles in LDS (weights copied global -> LDS with global_load_lds_dwordx4,
//    activations converted in registers). Each f32 activation is split into
//    bf16 hi = rne(x) and lo = rne(x - hi), and both halves meet the bf16
//    weight: the products are exact in f32 and the residual of the split is
//    below 2^-16 |x|, so the result carries f32-level error rather than bf16.
//  - linear_generic_kernel (everything else): one thread per output, the
//    reference's sequential f32 sum from the bias with separately rounded
//    products, so its results equal the reference's linear bit for bit.
#include <type_traits>

#include "internal.hpp"

namespace spissa {

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4;
typedef __attribute__((address_space(3))) void lds_void;

// 16 bytes of weights -> f32 (exact for every dtype).
template <typename WT>
struct WChunk;
template <>
struct WChunk<float> {
  static constexpr int N = 4;
  __device__ static void get(const uint4 r, float (&f)[4]) {
    f[0] = __uint_as_float(r.x);
    f[1] = __uint_as_float(r.y);
    f[2] = __uint_as_float(r.z);
    f[3] = __uint_as_float(r.w);
  }
};
template <>
struct WChunk<__bf16> {
  static constexpr int N = 8;
  __device__ static void get(const uint4 r, float (&f)[8]) {
    const unsigned u[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(u[i] << 16);
      f[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    }
  }
};
template <>
struct WChunk<_Float16> {
  static constexpr int N = 8;
  __device__ static void get(const uint4 r, float (&f)[8]) {
    const unsigned u[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = (float)__builtin_bit_cast(_Float16, (unsigned short)(u[i] & 0xffffu));
      f[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (unsigned short)(u[i] >> 16));
    }
  }
};

template <int CTRL>
__device__ __forceinline__ float dpp0(float v) {
  return __builtin_amdgcn_update_dpp(0.0f, v, CTRL, 0xf, 0xf, false);
}

// Sum over the 64 lanes of a wave (every lane receives it).
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp0<0xB1>(v);   // lane ^ 1
  v += dpp0<0x4E>(v);   // lane ^ 2
  v += dpp0<0x141>(v);  // row_half_mirror
  v += dpp0<0x140>(v);  // row_mirror
  auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
  auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

constexpr int kGemvRowsPerWave = 2;

}  // namespace

// The rows of workgroup `block`: 4 * kGemvRowsPerWave of them. K is a
// multiple of the chunk width (8 for 16-bit weights, 4 for f32).
template <typename WT, int NB>
__device__ __forceinline__ void gemv_rows(const LinearArgs &a, int block) {
  using C = WChunk<WT>;
  constexpr int EPC = C::N, RW = kGemvRowsPerWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int r0 = (block * 4 + wave) * RW;
  if (r0 >= a.N) return;  // uniform per wave
  const int nch = a.K / EPC;
  const char *wb = reinterpret_cast<const char *>(a.w);
  long roff[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i) roff[i] = (long)min(r0 + i, a.N - 1) * a.K * (long)sizeof(WT);

  float acc[RW][NB], ss[NB];
#pragma unroll
  for (int t = 0; t < NB; ++t) {
    ss[t] = 0.0f;
#pragma unroll
    for (int i = 0; i < RW; ++i) acc[i][t] = 0.0f;
  }
  const float *nw = a.norm_w;  // (uniform)

#pragma unroll 2
  for (int c = lane; c < nch; c += 64) {
    uint4 raw[RW];
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      // each weight byte is read once per call: the non-temporal hint keeps
      // the stream from displacing cached lines (5-8% faster measured)
      const u32x4 q = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wb + roff[i] + (long)c * 16));
      raw[i] = make_uint4(q.x, q.y, q.z, q.w);
    }
    float xv[NB][EPC];
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      const float *xp = a.x + (long)t * a.K + (long)c * EPC;
#pragma unroll
      for (int j = 0; j < EPC; j += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(xp + j);
        xv[t][j] = v.x;
        xv[t][j + 1] = v.y;
        xv[t][j + 2] = v.z;
        xv[t][j + 3] = v.w;
      }
    }
    if (nw) {  // folded RMSNorm: sum of squares, then x * w
      float g[EPC];
#pragma unroll
      for (int j = 0; j < EPC; j += 4) *reinterpret_cast<float4 *>(&g[j]) = *reinterpret_cast<const float4 *>(nw + (long)c * EPC + j);
#pragma unroll
      for (int t = 0; t < NB; ++t)
#pragma unroll
        for (int j = 0; j < EPC; ++j) {
          ss[t] = fmaf(xv[t][j], xv[t][j], ss[t]);
          xv[t][j] *= g[j];
        }
    }
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      float wf[EPC];
      C::get(raw[i], wf);
#pragma unroll
      for (int t = 0; t < NB; ++t)
#pragma unroll
        for (int j = 0; j < EPC; ++j) acc[i][t] = fmaf(wf[j], xv[t][j], acc[i][t]);
    }
  }
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int t = 0; t < NB; ++t) acc[i][t] = wave_sum(acc[i][t]);
  if (nw) {
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      const float inv = 1.0f / sqrtf(wave_sum(ss[t]) / (float)a.K + a.norm_eps);
#pragma unroll
      for (int i = 0; i < RW; ++i) acc[i][t] *= inv;
    }
  }
  if (lane < RW * NB) {
    const int i = lane / NB, t = lane % NB;
    const int r = r0 + i;
    float v = 0.0f;
#pragma unroll
    for (int ii = 0; ii < RW; ++ii)
#pragma unroll
      for (int tt = 0; tt < NB; ++tt) v = (ii == i && tt == t) ? acc[ii][tt] : v;
    if (r < a.N) a.out[(long)t * a.N + r] = (a.bias ? a.bias[r] : 0.0f) + v;
  }
}


// Grid: ceil(N / (4 * kGemvRowsPerWave)) workgroups of 256 threads.
template <typename WT, int NB>
__global__ __launch_bounds__(256) void linear_gemv_kernel(const LinearArgs a) {
  gemv_rows<WT, NB>(a, blockIdx.x);
}

// Several projections of the same input in one launch (the q, k and v
// weights of a layer). Workgroup b belongs to the first segment whose
// cumulative workgroup count exceeds b; within it, the rows and arithmetic
// are those of linear_gemv_kernel, so the results are identical.
template <typename WT, int NB>
__global__ __launch_bounds__(256) void linear_gemv_multi_kernel(const LinearSegments m) {
  int b = blockIdx.x, seg = 0;
  while (seg + 1 < m.n && b >= m.blocks[seg]) b -= m.blocks[seg++];
  gemv_rows<WT, NB>(seg == 0 ? m.seg[0] : seg == 1 ? m.seg[1] : m.seg[2], b);
}

namespace {
constexpr int kBK = 32;              // GEMM k tile
constexpr int kRowBytes = kBK * 2;  // one bf16 tile row: 64 bytes, four 16-byte chunks

// Chunk swizzle of a 64-byte LDS row: any 8 aligned consecutive rows reading
// the same chunk hit 8 distinct 16-byte groups modulo 128 bytes.
__device__ __forceinline__ int swz4(int row) { return ((row >> 1) ^ (row >> 2)) & 3; }

typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

// (rne(a), rne(b)) as bf16 bits, a in the low half.
__device__ __forceinline__ unsigned bf16x2_rne(float a, float b) {
  return __builtin_bit_cast(unsigned, __builtin_convertvector((f32x2){a, b}, bf16x2));
}

// 16 bytes per lane global -> LDS (global_load_lds_dwordx4); the LDS address
// is the wave's base, lane l's bytes land at +16 l.
__device__ __forceinline__ void copy16_to_lds(const char *src, char *dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void *)dst, 16, 0, 0);
}
// s_waitcnt vmcnt(N) (N < 16; the other counters unconstrained).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}
}  // namespace

// Grid: ceil(M / BM) * ceil(N / BN) workgroups of 512 threads (WM x WN waves,
// each (BM / WM) x (BN / WN) outputs in 32 x 32 blocks). K % 32 == 0. Rows
// past M or N are read clamped and not stored. Two tile shapes
// (linear_gemm_shape picks one per call):
//   128 x 256, 2 x 4 waves of 64 x 64: 64 KB of LDS and at most 128 VGPRs, so
//     two workgroups share a CU (four waves per SIMD);
//   256 x 320, 4 x 2 waves of 64 x 160: 104 KB of LDS, one workgroup per CU
//     (two waves per SIMD), for grids whose 128 x 256 tiles would leave a
//     second round of slots mostly empty.
// Pipeline, per 32-deep k tile t: the weight tile is copied into one of two
// LDS buffers one step ahead (issued in step t-1), and the activations are
// loaded into registers two steps ahead (issued in step t-2, split and written
// to one of two LDS buffers at the start of step t-1). Step t writes the
// activations of tile t+1, copies the weights of tile t+1, loads the
// activations of tile t+2, runs the MFMAs of tile t, then waits for
// everything but the activation loads it just issued.
// Measured on the 4096 x 5120 x 3072 projection: 284 us with 128 x 256 tiles,
// 242-250 us with 256 x 320 ones (MFMA busy 53% under the profiler, no LDS
// bank conflicts); 128 x 128 tiles of four waves took 292 us with this
// pipeline (three workgroups per CU) and 342 us with a third weight buffer two
// steps ahead (two per CU). Reading a step's first fragments before its
// copies, and an XCD-grouped tile order (each XCD a 4 x 8 block of tiles:
// 424 MB fetched beyond L2 for 81 MB of operands otherwise), measured within
// noise.
template <int BM, int BN, int WM, int WN, int MINWG>
__global__ __launch_bounds__(WM * WN * 64, MINWG) void linear_gemm_kernel(const LinearArgs a) {
  static_assert(WM * WN == 8, "eight waves");
  constexpr int TM = BM / WM, TN = BN / WN;  // the wave's outputs
  constexpr int BI = TM / 32, BJ = TN / 32;  // its 32 x 32 blocks
  static_assert(BI * 32 == TM && BJ * 32 == TN, "32 x 32 blocks");
  constexpr int WCOPIES = BN * kRowBytes / 1024;  // 1 KB weight copies per k tile
  constexpr int WCW = (WCOPIES + 7) / 8;          // per wave (the last round partial)
  constexpr int XR = BM / 128;                    // activation rows per thread
  static_assert(XR * 128 == BM && WCOPIES * 1024 == BN * kRowBytes, "tile shape");
  __shared__ __attribute__((aligned(1024))) char w_lds0[BN * kRowBytes];
  __shared__ __attribute__((aligned(1024))) char w_lds1[BN * kRowBytes];
  __shared__ __attribute__((aligned(1024))) char xh_lds0[BM * kRowBytes];
  __shared__ __attribute__((aligned(1024))) char xh_lds1[BM * kRowBytes];
  __shared__ __attribute__((aligned(1024))) char xl_lds0[BM * kRowBytes];
  __shared__ __attribute__((aligned(1024))) char xl_lds1[BM * kRowBytes];

  const int tiles_n = (a.N + BN - 1) / BN;
  const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wm = wave / WN, wn = wave % WN;  // the wave's TM x TN block
  const int lr = lane & 31, hl = lane >> 5;
  const int nk = a.K / kBK;

  // Weight copies: copy c = wave + 8 j fills LDS bytes [c * 1024, +1024);
  // lane l's 16 bytes land at +16 l, i.e. row R = byte / 64, position p, which
  // holds chunk p ^ swz4(R).
  const char *wg = reinterpret_cast<const char *>(a.w);
  long w_src[WCW];
#pragma unroll
  for (int j = 0; j < WCW; ++j) {
    const int c = min(wave + 8 * j, WCOPIES - 1);
    const int byte = c * 1024 + lane * 16;
    const int row = byte / kRowBytes, p = (byte % kRowBytes) / 16;
    const int n = min(n0 + row, a.N - 1);
    w_src[j] = (long)n * a.K * 2 + 16 * (p ^ swz4(row));
  }
  auto copy_w = [&](int kt, char *dst) {
#pragma unroll
    for (int j = 0; j < WCW; ++j)
      if (wave + 8 * j < WCOPIES) copy16_to_lds(wg + w_src[j] + (long)kt * kBK * 2, dst + (wave + 8 * j) * 1024);
  };
  // Activations: thread t loads rows t / 4 + 128 i, columns 8 (t % 4) + [0, 8)
  // of the k tile, splits them and writes 16 bytes of hi and of lo (chunk
  // t % 4 of the row).
  const int xr = tid >> 2, xc = tid & 3;
  const float *xg[XR];
#pragma unroll
  for (int i = 0; i < XR; ++i) xg[i] = a.x + (long)min(m0 + xr + 128 * i, a.M - 1) * a.K + 8 * xc;
  auto load_x = [&](int kt, float4 (&xv)[XR][2]) {
#pragma unroll
    for (int i = 0; i < XR; ++i)
#pragma unroll
      for (int e = 0; e < 2; ++e) xv[i][e] = *reinterpret_cast<const float4 *>(xg[i] + (long)kt * kBK + 4 * e);
  };
  auto store_x = [&](const float4 (&xv)[XR][2], char *hi, char *lo) {
#pragma unroll
    for (int r = 0; r < XR; ++r) {
      const float f[8] = {xv[r][0].x, xv[r][0].y, xv[r][0].z, xv[r][0].w, xv[r][1].x, xv[r][1].y, xv[r][1].z, xv[r][1].w};
      unsigned h[4], l[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // one v_cvt_pk_bf16_f32 per pair (round to nearest even), for hi and for lo
        h[i] = bf16x2_rne(f[2 * i], f[2 * i + 1]);
        const float r0 = f[2 * i] - __uint_as_float(h[i] << 16);
        const float r1 = f[2 * i + 1] - __uint_as_float(h[i] & 0xffff0000u);
        l[i] = bf16x2_rne(r0, r1);
      }
      const int row = xr + 128 * r;
      const int off = row * kRowBytes + 16 * (xc ^ swz4(row));
      *reinterpret_cast<uint4 *>(hi + off) = make_uint4(h[0], h[1], h[2], h[3]);
      *reinterpret_cast<uint4 *>(lo + off) = make_uint4(l[0], l[1], l[2], l[3]);
    }
  };

  // Fragment offsets: block b of the wave's block, 16-deep k step s: row
  // 32 b + lr of it, chunk 2 s + hl (TM, TN and 32 b are multiples of 32 and
  // leave swz4 unchanged).
  unsigned a_rd[BI][2], b_rd[BJ][2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
#pragma unroll
    for (int b = 0; b < BI; ++b) {
      const int ra = wm * TM + 32 * b + lr;
      a_rd[b][s] = ra * kRowBytes + 16 * ((2 * s + hl) ^ swz4(ra));
    }
#pragma unroll
    for (int b = 0; b < BJ; ++b) {
      const int rb = wn * TN + 32 * b + lr;
      b_rd[b][s] = rb * kRowBytes + 16 * ((2 * s + hl) ^ swz4(rb));
    }
  }

  f32x16 acc[BI][BJ];
#pragma unroll
  for (int i = 0; i < BI; ++i)
#pragma unroll
    for (int j = 0; j < BJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  auto compute = [&](const char *wl, const char *xh, const char *xl) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      bf16x8 fa_h[BI], fa_l[BI], fb[BJ];
#pragma unroll
      for (int b = 0; b < BI; ++b) {
        fa_h[b] = *reinterpret_cast<const bf16x8 *>(xh + a_rd[b][s]);
        fa_l[b] = *reinterpret_cast<const bf16x8 *>(xl + a_rd[b][s]);
      }
#pragma unroll
      for (int b = 0; b < BJ; ++b) fb[b] = *reinterpret_cast<const bf16x8 *>(wl + b_rd[b][s]);
#pragma unroll
      for (int i = 0; i < BI; ++i)
#pragma unroll
        for (int j = 0; j < BJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa_h[i], fb[j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < BI; ++i)
#pragma unroll
        for (int j = 0; j < BJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa_l[i], fb[j], acc[i][j], 0, 0, 0);
    }
  };

  // One step on tile t; B selects the buffers (t % 2 computes, (t+1) % 2
  // receives): the weights of tile t+1 are copied one step ahead, the
  // activations loaded two ahead and written one ahead.
  auto step = [&](auto B_, int t, float4 (&xnext)[XR][2]) {
    constexpr int B = decltype(B_)::value;
    char *const w_cur = B ? w_lds1 : w_lds0, *const w_fill = B ? w_lds0 : w_lds1;
    char *const xh_cur = B ? xh_lds1 : xh_lds0, *const xl_cur = B ? xl_lds1 : xl_lds0;
    char *const xh_fill = B ? xh_lds0 : xh_lds1, *const xl_fill = B ? xl_lds0 : xl_lds1;
    if (t + 1 < nk) {
      store_x(xnext, xh_fill, xl_fill);
      copy_w(t + 1, w_fill);
    }
    const bool more = t + 2 < nk;
    if (more) load_x(t + 2, xnext);
    compute(w_cur, xh_cur, xl_cur);
    // everything but this step's activation loads is done
    if (more) wait_vmcnt<2 * XR>();
    else wait_vmcnt<0>();
    __syncthreads();
  };

  // Prologue: weights of tile 0 copied, activations of tile 0 in LDS, tile
  // 1's in registers.
  float4 xv[XR][2];
  copy_w(0, w_lds0);
  load_x(0, xv);
  store_x(xv, xh_lds0, xl_lds0);
  if (nk > 1) load_x(1, xv);
  wait_vmcnt<0>();
  __syncthreads();

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  int t = 0;
  for (; t + 2 <= nk; t += 2) {
    step(I0(), t, xv);
    step(I1(), t + 1, xv);
  }
  if (t < nk) step(I0(), t, xv);

  // Accumulator layout: element e of lane l is row 8 (e / 4) + 4 hl + e % 4,
  // column lr of its 32 x 32 block.
#pragma unroll
  for (int j = 0; j < BJ; ++j) {
    const int n = n0 + wn * TN + 32 * j + lr;
    if (n >= a.N) continue;
    const float bn = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < BI; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * TM + 32 * i + 8 * (e >> 2) + 4 * hl + (e & 3);
        if (m < a.M) a.out[(long)m * a.N + n] = bn + acc[i][j][e];
      }
  }
}

namespace {
typedef __attribute__((ext_vector_type(4))) float f32x4;
constexpr int kSkinnyRows = 16;  // weight rows (output features) per workgroup
}  // namespace

// Grid: ceil(N / 16) workgroups of 256 threads, for 5..64 tokens (MB blocks
// of 16), bf16 weights, K % 128 == 0. Wave w covers k in [w K/4, (w+1) K/4).
// Per 32-deep k step a lane loads 16 bytes of one weight row (the A operand
// of v_mfma_f32_16x16x32_bf16: row lane % 16, k 8 (lane / 16) + [0, 8)) straight
// from HBM, and 8 activations of one token (the B operand) from the cache,
// split into bf16 hi and lo; both meet the weights. The four waves' partial
// sums are added through LDS.
template <int MB>
__global__ __launch_bounds__(256) void linear_skinny_kernel(const LinearArgs a) {
  __shared__ f32x4 part[4][MB][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n0 = blockIdx.x * kSkinnyRows;
  const int r = lane & 15, kq = lane >> 4;  // operand row/column, k quarter (8 of 32)
  const int kw = a.K / 4;
  const int k_begin = wave * kw, k_end = k_begin + kw;
  const char *wrow = reinterpret_cast<const char *>(a.w) + (long)min(n0 + r, a.N - 1) * a.K * 2;
  const float *xrow[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) xrow[b] = a.x + (long)min(16 * b + r, a.M - 1) * a.K;

  f32x4 acc[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) acc[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  auto step = [&](int kk) {
    const bf16x8 wf = *reinterpret_cast<const bf16x8 *>(wrow + (long)(kk + 8 * kq) * 2);
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const float4 x0 = *reinterpret_cast<const float4 *>(xrow[b] + kk + 8 * kq);
      const float4 x1 = *reinterpret_cast<const float4 *>(xrow[b] + kk + 8 * kq + 4);
      const float f[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      unsigned h[4], l[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        h[i] = bf16x2_rne(f[2 * i], f[2 * i + 1]);
        l[i] = bf16x2_rne(f[2 * i] - __uint_as_float(h[i] << 16), f[2 * i + 1] - __uint_as_float(h[i] & 0xffff0000u));
      }
      const bf16x8 xh = __builtin_bit_cast(bf16x8, make_uint4(h[0], h[1], h[2], h[3]));
      const bf16x8 xl = __builtin_bit_cast(bf16x8, make_uint4(l[0], l[1], l[2], l[3]));
      acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf, xh, acc[b], 0, 0, 0);
      acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf, xl, acc[b], 0, 0, 0);
    }
  };
  constexpr int U = MB <= 2 ? 8 : 4;  // k steps in flight (registers allowing)
  int kk = k_begin;
  for (; kk + 32 * U <= k_end; kk += 32 * U) {
#pragma unroll
    for (int u = 0; u < U; ++u) step(kk + 32 * u);
  }
  for (; kk < k_end; kk += 32) step(kk);

#pragma unroll
  for (int b = 0; b < MB; ++b) part[wave][b][lane] = acc[b];
  __syncthreads();
  // D layout: element e of lane l is row (weight) 4 (l / 16) + e, column
  // (token) l % 16 of its block. Thread t < 64 * MB finishes block t / 64.
  if (threadIdx.x < 64 * MB) {
    const int b = threadIdx.x >> 6, l = threadIdx.x & 63;
    const f32x4 s = part[0][b][l] + part[1][b][l] + part[2][b][l] + part[3][b][l];
    const int t = 16 * b + (l & 15);
    if (t < a.M) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int n = n0 + 4 * (l >> 4) + e;
        if (n < a.N) a.out[(long)t * a.N + n] = (a.bias ? a.bias[n] : 0.0f) + s[e];
      }
    }
  }
}

// One thread per output: the sum starts at the bias and adds x[m][k] * w[n][k]
// in index order, each product rounded first (ops.rs:94-103; also the exact
// batch-1 row-block loop of streaming/kernels_raw16.rs:640-672).
template <typename WT>
__global__ __launch_bounds__(256) void linear_generic_kernel(const LinearArgs a) {
#pragma clang fp contract(off)
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)a.M * a.N) return;
  const int m = (int)(idx / a.N), n = (int)(idx % a.N);
  const WT *w = reinterpret_cast<const WT *>(a.w) + (long)n * a.K;
  const float *x = a.x + (long)m * a.K;
  float sum = a.bias ? a.bias[n] : 0.0f;
  for (int k = 0; k < a.K; ++k) {
    float wf;
    if constexpr (sizeof(WT) == 4) wf = (float)w[k];
    else if constexpr (__is_same(WT, __bf16)) wf = __uint_as_float((unsigned)__builtin_bit_cast(unsigned short, w[k]) << 16);
    else wf = (float)w[k];
    const float p = x[k] * wf;
    sum = sum + p;
  }
  a.out[idx] = sum;
}

namespace {
template <typename WT>
hipError_t launch_gemv(hipStream_t st, const LinearArgs &a) {
  const unsigned grid = (unsigned)((a.N + 4 * kGemvRowsPerWave - 1) / (4 * kGemvRowsPerWave));
  switch (a.M) {
    case 1: hipLaunchKernelGGL((linear_gemv_kernel<WT, 1>), dim3(grid), dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL((linear_gemv_kernel<WT, 2>), dim3(grid), dim3(256), 0, st, a); break;
    case 3: hipLaunchKernelGGL((linear_gemv_kernel<WT, 3>), dim3(grid), dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL((linear_gemv_kernel<WT, 4>), dim3(grid), dim3(256), 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
template <typename WT>
hipError_t launch_gemv_multi(hipStream_t st, const LinearSegments &m) {
  long total = 0;
  for (int i = 0; i < m.n; ++i) total += m.blocks[i];
  switch (m.seg[0].M) {
    case 1: hipLaunchKernelGGL((linear_gemv_multi_kernel<WT, 1>), dim3((unsigned)total), dim3(256), 0, st, m); break;
    case 2: hipLaunchKernelGGL((linear_gemv_multi_kernel<WT, 2>), dim3((unsigned)total), dim3(256), 0, st, m); break;
    case 3: hipLaunchKernelGGL((linear_gemv_multi_kernel<WT, 3>), dim3((unsigned)total), dim3(256), 0, st, m); break;
    case 4: hipLaunchKernelGGL((linear_gemv_multi_kernel<WT, 4>), dim3((unsigned)total), dim3(256), 0, st, m); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
template <typename WT>
hipError_t launch_generic_linear(hipStream_t st, const LinearArgs &a) {
  const long n = (long)a.M * a.N;
  hipLaunchKernelGGL((linear_generic_kernel<WT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a);
  return hipGetLastError();
}
template <int BM, int BN, int WM, int WN, int MINWG>
hipError_t launch_gemm(hipStream_t st, const LinearArgs &a) {
  const long grid = (long)((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  hipLaunchKernelGGL((linear_gemm_kernel<BM, BN, WM, WN, MINWG>), dim3((unsigned)grid), dim3(512), 0, st, a);
  return hipGetLastError();
}
template <typename WT>
hipError_t launch_typed(hipStream_t st, const LinearArgs &a, int path) {
  if (path == kLinearGemv) return launch_gemv<WT>(st, a);
  return launch_generic_linear<WT>(st, a);
}
}  // namespace

int linear_path(int dtype, long M, long K) {
  const int epc = dtype == SPISSA_DTYPE_F32 ? 4 : 8;
  if (dtype == SPISSA_DTYPE_BF16 && M > 4 && M <= 64 && K % 128 == 0) return kLinearSkinny;
  if (dtype == SPISSA_DTYPE_BF16 && M > 4 && K % kBK == 0) return kLinearGemm;
  if (M <= 4 && K % epc == 0) return kLinearGemv;
  return kLinearGeneric;
}

hipError_t launch_linear_multi(hipStream_t st, const LinearArgs *segs, int n) {
  if (n < 1 || n > kMaxLinearSegments) return hipErrorInvalidValue;
  LinearSegments m{};
  m.n = n;
  for (int i = 0; i < n; ++i) {
    const LinearArgs &a = segs[i];
    // one launch only when every segment takes the GEMV with the same input shape
    if (a.M != segs[0].M || a.K != segs[0].K || a.dtype != segs[0].dtype || a.x != segs[0].x || a.N <= 0 ||
        linear_path(a.dtype, a.M, a.K) != kLinearGemv) {
      for (int j = 0; j < n; ++j) {
        const hipError_t e = launch_linear(st, segs[j], linear_path(segs[j].dtype, segs[j].M, segs[j].K));
        if (e != hipSuccess) return e;
      }
      return hipSuccess;
    }
    m.seg[i] = a;
    m.blocks[i] = (a.N + 4 * kGemvRowsPerWave - 1) / (4 * kGemvRowsPerWave);
  }
  switch (segs[0].dtype) {
    case SPISSA_DTYPE_F32: return launch_gemv_multi<float>(st, m);
    case SPISSA_DTYPE_BF16: return launch_gemv_multi<__bf16>(st, m);
    case SPISSA_DTYPE_F16: return launch_gemv_multi<_Float16>(st, m);
    default: return hipErrorInvalidValue;
  }
}

// The 256 x 320 tiles when their rounds of one workgroup per CU, each tile
// 2.5 times the work of a 128 x 256 one at the same rate per CU, take less
// time than the 128 x 256 tiles' rounds of two per CU (4096 x 5120: 640
// tiles of 128 x 256, a second round a quarter full, against 256 wide tiles
// in one round).
static bool linear_gemm_wide(long M, long N, int cus) {
  const long c = cus > 0 ? cus : 256;
  const long small = ((M + 127) / 128) * ((N + 255) / 256), wide = ((M + 255) / 256) * ((N + 319) / 320);
  const long rounds_small = (small + 2 * c - 1) / (2 * c), rounds_wide = (wide + c - 1) / c;
  return 5 * rounds_wide < 4 * rounds_small;
}

hipError_t launch_linear(hipStream_t st, const LinearArgs &a, int path) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (a.norm_w && path != kLinearGemv) return hipErrorInvalidValue;  // the folded norm is the GEMV's
  if (path == kLinearSkinny) {
    if (a.dtype != SPISSA_DTYPE_BF16 || a.K % 128 != 0 || a.M > 64) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((a.N + kSkinnyRows - 1) / kSkinnyRows));
    switch ((a.M + 15) / 16) {
      case 1: hipLaunchKernelGGL(linear_skinny_kernel<1>, grid, dim3(256), 0, st, a); break;
      case 2: hipLaunchKernelGGL(linear_skinny_kernel<2>, grid, dim3(256), 0, st, a); break;
      case 3: hipLaunchKernelGGL(linear_skinny_kernel<3>, grid, dim3(256), 0, st, a); break;
      default: hipLaunchKernelGGL(linear_skinny_kernel<4>, grid, dim3(256), 0, st, a); break;
    }
    return hipGetLastError();
  }
  if (path == kLinearGemm) {
    if (a.dtype != SPISSA_DTYPE_BF16 || a.K % kBK != 0) return hipErrorInvalidValue;
    return linear_gemm_wide(a.M, a.N, a.cus) ? launch_gemm<256, 320, 4, 2, 1>(st, a)
                                              : launch_gemm<128, 256, 2, 4, 2>(st, a);
  }
  switch (a.dtype) {
    case SPISSA_DTYPE_F32: return launch_typed<float>(st, a, path);
    case SPISSA_DTYPE_BF16: return launch_typed<__bf16>(st, a, path);
    case SPISSA_DTYPE_F16: return launch_typed<_Float16>(st, a, path);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace spissa
