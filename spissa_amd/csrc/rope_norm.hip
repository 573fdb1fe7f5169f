// rope_norm.hip -- RoPE application, RMSNorm (Gemma QK-norm), the fused Gemma
// Q/K prologue, and the f32 -> bf16 K / transposed-V staging used by prefill.
//
// RoPE and RMSNorm here are bit-identical to the Rust reference: cos/sin come
// from a table computed on the host with the reference's own per-(position,
// pair) formula and glibc libm, every multiply and add is rounded separately
// (contraction off), and hipcc's default f32 division and sqrt are correctly
// rounded.
#include <algorithm>

#include "internal.hpp"

namespace spissa {

// rotary.rs:467-481 rotate_neox_pair, applied to every (row, pair) in parallel.
// Rows are S * (qh + kh): for each position, qh query rows then kh key rows.
__global__ void rope_apply_kernel(const float *__restrict__ cos_tab,
                                  const float *__restrict__ sin_tab, long tab_stride,
                                  float *__restrict__ q, float *__restrict__ k, long S, int qh,
                                  int kh, int D, int half) {
#pragma clang fp contract(off)
  long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  long rows = S * (qh + kh);
  if (t >= rows * half) return;
  long row = t / half;
  int pair = (int)(t - row * half);
  long pos = row / (qh + kh);
  int hh = (int)(row - pos * (qh + kh));
  float *base = hh < qh ? q + (pos * qh + hh) * (long)D : k + (pos * kh + (hh - qh)) * (long)D;
  float c = cos_tab[pos * tab_stride + pair];
  float s = sin_tab[pos * tab_stride + pair];
  float first = base[pair];
  float second = base[pair + half];
  base[pair] = first * c - second * s;
  base[pair + half] = second * c + first * s;
}

// ops.rs:159-179 rms_norm: one thread per row, sequential sum of squares.
__global__ void rms_norm_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                long rows, int cols, float eps, float *__restrict__ out) {
#pragma clang fp contract(off)
  long r = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const float *row = x + r * cols;
  float acc = 0.0f;
  for (int c = 0; c < cols; ++c) acc += row[c] * row[c];
  float mean_square = acc / (float)cols;
  float inv_rms = 1.0f / sqrtf(mean_square + eps);
  float *o = out + r * cols;
  for (int c = 0; c < cols; ++c) o[c] = row[c] * inv_rms * w[c];
}

// The same sum for wide rows: one workgroup per row stages the row in LDS
// with coalesced loads, lane 0 of wave 0 adds the squares in index order
// (bit-identical to the one-thread-per-row kernel), and every thread then
// scales its share of the row. Rows of up to kNormRowMax floats.
constexpr int kNormRowMax = 8192;
__global__ __launch_bounds__(256) void rms_norm_row_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                           int cols, float eps, float *__restrict__ out) {
#pragma clang fp contract(off)
  __shared__ float row_s[kNormRowMax];
  __shared__ float inv_s;
  const float *row = x + (long)blockIdx.x * cols;
  for (int c = threadIdx.x; c < cols; c += 256) row_s[c] = row[c];
  __syncthreads();
  if (threadIdx.x == 0) {
    float acc = 0.0f;
    for (int c = 0; c < cols; ++c) acc += row_s[c] * row_s[c];
    float mean_square = acc / (float)cols;
    inv_s = 1.0f / sqrtf(mean_square + eps);
  }
  __syncthreads();
  const float inv_rms = inv_s;
  float *o = out + (long)blockIdx.x * cols;
  for (int c = threadIdx.x; c < cols; c += 256) o[c] = row_s[c] * inv_rms * w[c];
}

// RMSNorm with a tree-reduced sum of squares, for the attention sublayer's
// input and post-attention norms (one workgroup per row): results differ
// from the sequential sum by rounding only (relative 1e-7), at the cost of a
// launch instead of a serial chain of `cols` additions.
__global__ __launch_bounds__(256) void rms_norm_tree_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                            int cols, float eps, float *__restrict__ out) {
  __shared__ float part[4];
  const float *row = x + (long)blockIdx.x * cols;
  float *o = out + (long)blockIdx.x * cols;
  // 16-byte pieces when the rows allow it, four loads in flight per thread
  const bool vec = (cols & 3) == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                                        reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  float acc = 0.0f;
  if (vec) {
    const float4 *r4 = reinterpret_cast<const float4 *>(row);
#pragma unroll 4
    for (int c = threadIdx.x; c < (cols >> 2); c += 256) {
      const float4 v = r4[c];
      acc = fmaf(v.x, v.x, acc);
      acc = fmaf(v.y, v.y, acc);
      acc = fmaf(v.z, v.z, acc);
      acc = fmaf(v.w, v.w, acc);
    }
  } else {
#pragma unroll 4
    for (int c = threadIdx.x; c < cols; c += 256) acc = fmaf(row[c], row[c], acc);
  }
  for (int d = 32; d > 0; d >>= 1) acc += __shfl_xor(acc, d, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  const float total = (part[0] + part[1]) + (part[2] + part[3]);
  const float inv_rms = 1.0f / sqrtf(total / (float)cols + eps);
  if (vec) {
    const float4 *r4 = reinterpret_cast<const float4 *>(row);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    float4 *o4 = reinterpret_cast<float4 *>(o);
#pragma unroll 4
    for (int c = threadIdx.x; c < (cols >> 2); c += 256) {
      const float4 v = r4[c], g = w4[c];
      o4[c] = make_float4(v.x * inv_rms * g.x, v.y * inv_rms * g.y, v.z * inv_rms * g.z, v.w * inv_rms * g.w);
    }
  } else {
    for (int c = threadIdx.x; c < cols; c += 256) o[c] = row[c] * inv_rms * w[c];
  }
}

// models/gemma/generate.rs:230-278 for one row of q or k: rms_norm, Gemma
// rotate-half with the layer's table, then (q rows only) the prescale.
__global__ void gemma_prologue_kernel(const float *__restrict__ cos_tab,
                                      const float *__restrict__ sin_tab, long tab_stride,
                                      float *__restrict__ q, float *__restrict__ k, long S, int qh,
                                      int kh, int D, int half, const float *__restrict__ qn,
                                      const float *__restrict__ kn, float eps, float prescale) {
#pragma clang fp contract(off)
  long row = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= S * (qh + kh)) return;
  long pos = row / (qh + kh);
  int hh = (int)(row - pos * (qh + kh));
  bool is_q = hh < qh;
  float *x = is_q ? q + (pos * qh + hh) * (long)D : k + (pos * kh + (hh - qh)) * (long)D;
  const float *w = is_q ? qn : kn;
  float acc = 0.0f;
  for (int c = 0; c < D; ++c) acc += x[c] * x[c];
  float mean_square = acc / (float)D;
  float inv_rms = 1.0f / sqrtf(mean_square + eps);
  const float *ct = cos_tab + pos * tab_stride;
  const float *st = sin_tab + pos * tab_stride;
  for (int p = 0; p < half; ++p) {
    float first = x[p] * inv_rms * w[p];
    float second = x[p + half] * inv_rms * w[p + half];
    float c = ct[p], s = st[p];
    float a = first * c - second * s;
    float b = second * c + first * s;
    if (is_q) {
      a *= prescale;
      b *= prescale;
    }
    x[p] = a;
    x[p + half] = b;
  }
  for (int c = 2 * half; c < D; ++c) {
    float v = x[c] * inv_rms * w[c];
    if (is_q) v *= prescale;
    x[c] = v;
  }
}

// The same prologue with one wave per row, for D = 64, 128 or 256: lane l
// holds elements [l * D/64, (l + 1) * D/64) of the row, so every load and
// store is coalesced, and its rotate-half partners sit in lane l ^ 32. The
// squares go through LDS and lane 0 adds them in index order, so the sum is
// the reference's sequential one, bit for bit (ops.rs:159-179); the norm,
// rotation and prescale then run on all lanes. Four rows per workgroup.
template <int D>
__global__ __launch_bounds__(256) void gemma_prologue_wave_kernel(
    const float *__restrict__ cos_tab, const float *__restrict__ sin_tab, long tab_stride, float *__restrict__ q,
    float *__restrict__ k, long S, int qh, int kh, const float *__restrict__ qn, const float *__restrict__ kn,
    float eps, float prescale) {
#pragma clang fp contract(off)
  constexpr int E = D / 64, HALF = D / 2;
  __shared__ float sq[4][D];
  __shared__ float inv_s[4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + wave;
  const bool live = row < S * (qh + kh);
  long pos = 0;
  bool is_q = false;
  float *x = nullptr;
  const float *w = nullptr;
  float v[E];
  if (live) {
    pos = row / (qh + kh);
    const int hh = (int)(row - pos * (qh + kh));
    is_q = hh < qh;
    x = is_q ? q + (pos * qh + hh) * (long)D : k + (pos * kh + (hh - qh)) * (long)D;
    w = is_q ? qn : kn;
#pragma unroll
    for (int j = 0; j < E; ++j) {
      v[j] = x[lane * E + j];
      sq[wave][lane * E + j] = v[j] * v[j];
    }
  }
  __syncthreads();
  if (live && lane == 0) {
    float acc = 0.0f;
    for (int c = 0; c < D; ++c) acc += sq[wave][c];
    const float mean_square = acc / (float)D;
    inv_s[wave] = 1.0f / sqrtf(mean_square + eps);
  }
  __syncthreads();
  if (!live) return;
  const float inv_rms = inv_s[wave];
  float nv[E];
#pragma unroll
  for (int j = 0; j < E; ++j) nv[j] = v[j] * inv_rms * w[lane * E + j];
  // rotate-half: lanes < 32 hold first halves (pairs p = lane*E + j), lanes
  // >= 32 the second halves of the same pairs
  const bool lo = lane < 32;
  const int p0 = (lane & 31) * E;
  const float *ct = cos_tab + pos * tab_stride + p0;
  const float *st = sin_tab + pos * tab_stride + p0;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(nv[j]), __float_as_uint(nv[j]), false, false);
    const float partner = __uint_as_float(lo ? r[1] : r[0]);
    const float first = lo ? nv[j] : partner, second = lo ? partner : nv[j];
    const float c = ct[j], s = st[j];
    float o = lo ? first * c - second * s : second * c + first * s;
    if (is_q) o *= prescale;
    x[lane * E + j] = o;
  }
  static_assert(HALF == 32 * E, "rotate-half partners are 32 lanes apart");
}

// Converts n rows of K and V ([n, H, D] f32) to the prefill operand layouts:
// kb [H, cap, D] bf16 (head-major K) and vt [H, D, cap] bf16 (transposed V,
// key p stored at slot vt_key_slot(p)), at buffer positions dst_first + i.
// Rows with n <= i < n_pad are written as zeros so padded key tiles read
// finite data; buffer positions outside [dst_first, dst_first + n_pad) are
// left untouched.
// A block owns the 64 buffer positions [P0, P0 + 64), P0 a multiple of 64 (so
// the slot permutation, which stays inside aligned groups of 16, stays inside
// the block), and 64 dims [d0, d0 + 64) of one head. K rows are converted 8
// dims per thread with 16-byte loads and stores; V rows go through an LDS
// tile, from which each thread writes 8 consecutive slots of one V^T row as
// one 16-byte store.
// Grid: (blocks over positions, H, D / 64), 256 threads.
__global__ __launch_bounds__(256) void stage_bf16_kernel(const float *__restrict__ k_rows,
                                                         const float *__restrict__ v_rows, long n, long n_pad,
                                                         int H, int D, bf16 *__restrict__ kb,
                                                         bf16 *__restrict__ vt, long dst_first, long cap) {
  typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
  __shared__ float tile[64][65];  // V[position][dim] of the block, padded against bank conflicts
  const int h = blockIdx.y, d0 = 64 * blockIdx.z;
  const long P0 = (dst_first & ~63L) + 64L * blockIdx.x;
  const long lo = dst_first, hi = dst_first + n_pad;  // positions this call writes

  // K rows (and V rows into LDS): position P0 + r holds source row i = P0 + r - dst_first.
  // Both of a thread's rows are loaded before either is converted, so all
  // eight 16-byte loads are in flight together.
  float4 src[2][4];
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int w = threadIdx.x + 256 * it;
    const int r = w >> 3, cc = w & 7;
    const long pos = P0 + r, i = pos - dst_first;
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    src[it][0] = src[it][1] = src[it][2] = src[it][3] = z;
    if (pos >= lo && pos < hi && i < n) {
      const long base = (i * H + h) * (long)D + d0 + 8 * cc;
      src[it][0] = *reinterpret_cast<const float4 *>(k_rows + base);
      src[it][1] = *reinterpret_cast<const float4 *>(k_rows + base + 4);
      src[it][2] = *reinterpret_cast<const float4 *>(v_rows + base);
      src[it][3] = *reinterpret_cast<const float4 *>(v_rows + base + 4);
    }
  }
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int w = threadIdx.x + 256 * it;
    const int r = w >> 3, cc = w & 7;
    const long pos = P0 + r;
    if (pos < lo || pos >= hi) continue;
    const float4 k0 = src[it][0], k1 = src[it][1], v0 = src[it][2], v1 = src[it][3];
    bf16x8 kv;
    kv[0] = (bf16)k0.x; kv[1] = (bf16)k0.y; kv[2] = (bf16)k0.z; kv[3] = (bf16)k0.w;
    kv[4] = (bf16)k1.x; kv[5] = (bf16)k1.y; kv[6] = (bf16)k1.z; kv[7] = (bf16)k1.w;
    *reinterpret_cast<bf16x8 *>(kb + ((long)h * cap + pos) * D + d0 + 8 * cc) = kv;
    float *t = &tile[r][8 * cc];
    t[0] = v0.x; t[1] = v0.y; t[2] = v0.z; t[3] = v0.w;
    t[4] = v1.x; t[5] = v1.y; t[6] = v1.z; t[7] = v1.w;
  }
  __syncthreads();

  // V^T: row d0 + dd, slots [P0 + 8c, P0 + 8c + 8); slot s holds the key at
  // position vt_key_slot(s), which lies in the same aligned 16-group.
  for (int w = threadIdx.x; w < 64 * 8; w += 256) {
    const int dd = w >> 3, c = w & 7;
    const long s0 = P0 + 8 * c;
    bf16 *dst = vt + ((long)h * D + d0 + dd) * cap;
    const long g0 = s0 & ~15L;  // the aligned 16-group whose keys these slots hold
    if (g0 >= lo && g0 + 16 <= hi) {
      bf16x8 vv;
#pragma unroll
      for (int j = 0; j < 8; ++j) vv[j] = (bf16)tile[vt_key_slot(s0 + j) - P0][dd];
      *reinterpret_cast<bf16x8 *>(dst + s0) = vv;
    } else {
      for (int j = 0; j < 8; ++j) {
        const long sl = s0 + j, key = vt_key_slot(sl);
        if (key >= lo && key < hi) dst[sl] = (bf16)tile[key - P0][dd];
      }
    }
  }
}

// The append and operand staging of a fused prefill step, in one pass over
// the chunk's rows: the RoPE of rotary.rs:75-125 / 137-186 (optional, table
// rows are absolute positions), then KvCache::append (rotary.rs:226-256).
//   K/V blocks (blockIdx.y < H): cache position P + i receives row i of the
//     chunk: the rotated key and the value in the f32 rows, the bf16 key in
//     the shadow K [H, cap, D] and the bf16 value at slot vt_key_slot(pos) of
//     the shadow V^T [H, D, cap]; shadow positions [P + S, pad_end) are zeroed
//     so the last key tile the prefill kernel reads is finite.
//   Q blocks (blockIdx.y >= H): query row i, rotated at position P + i,
//     times qscale, rounded to bf16 into qb [S, Hq, D] -- the prefill
//     kernel's Q operand, the same bits it would form from the rotated f32 row.
// 1 / sqrt(mean(x^2) + eps) of a row of D floats held by a quad of lanes
// (lane c of the quad holds dims 32z + 8c + [0, 8) and D/2 + 32z + 8c + [0, 8)
// for every z), with the sum of squares taken in index order as
// ops.rs:159-179 takes it: the running sum visits the lanes in dim order,
// eight rounded squares at a time, passed on with a quad rotation (DPP).
template <int D>
__device__ __forceinline__ float quad_inv_rms(const float *row, int c, float eps) {
#pragma clang fp contract(off)
  constexpr int HALF = D / 2, G = HALF / 32;
  float4 x[2][G][2];
#pragma unroll
  for (int part = 0; part < 2; ++part)
#pragma unroll
    for (int z = 0; z < G; ++z) {
      x[part][z][0] = *reinterpret_cast<const float4 *>(row + part * HALF + 32 * z + 8 * c);
      x[part][z][1] = *reinterpret_cast<const float4 *>(row + part * HALF + 32 * z + 8 * c + 4);
    }
  float acc = 0.0f;
#pragma unroll
  for (int part = 0; part < 2; ++part)
#pragma unroll
    for (int z = 0; z < G; ++z) {
      const float *v = reinterpret_cast<const float *>(x[part][z]);
#pragma unroll
      for (int turn = 0; turn < 4; ++turn) {
        float t = acc;
#pragma unroll
        for (int j = 0; j < 8; ++j) t = t + v[j] * v[j];
        acc = c == turn ? t : acc;
        // lane c takes lane c - 1's sum (quad_perm [3, 0, 1, 2])
        acc = __builtin_amdgcn_update_dpp(acc, acc, 0x93, 0xf, 0xf, false);
      }
    }
  // lane 0 of the quad holds the total; every lane takes it (quad_perm [0, 0, 0, 0])
  acc = __builtin_amdgcn_update_dpp(acc, acc, 0x00, 0xf, 0xf, false);
  const float mean_square = acc / (float)D;
  return 1.0f / sqrtf(mean_square + eps);
}

// A block owns 64 positions and the 32 rotary pairs [32z, 32z + 32) of one
// head, i.e. dims [32z, +32) and [D/2 + 32z, +32); thread t holds position
// t / 4 and the eight pairs 8(t % 4) .. +7 of that range: a float4 pair of
// each half. Values pass through an LDS tile for the V^T stores.
// Grid: (position blocks, H + Hq, D / 64), 256 threads. NORM_D: 0, or the
// head dim with the Gemma QK-norm folded in (each quad of lanes first takes
// its full row's 1/rms).
template <int NORM_D>
__global__ __launch_bounds__(256) void prefill_append_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ cos_tab, const float *__restrict__ sin_tab, long P, long S, int H, int Hq, int D,
    float *__restrict__ cache_k, float *__restrict__ cache_v, bf16 *__restrict__ kb, bf16 *__restrict__ vt,
    long cap, long pad_end, bf16 *__restrict__ qb, float qscale, const PrefillNorm nrm) {
#pragma clang fp contract(off)
  typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
  __shared__ float tile[64][65];  // V[position][lo 32 | hi 32 dims], padded against bank conflicts
  const int half = D / 2;
  const int r = threadIdx.x >> 2, c = threadIdx.x & 3;
  const int p0 = 32 * blockIdx.z + 8 * c;  // first pair of this thread
  const bool kv = (int)blockIdx.y < H;

  auto rotate = [&](float4 (&lo)[2], float4 (&hi)[2], long pos) {
    if (!cos_tab) return;
    const float *cp = cos_tab + pos * half + p0, *sp = sin_tab + pos * half + p0;
    float *a = reinterpret_cast<float *>(lo), *b = reinterpret_cast<float *>(hi);
    float cs[8], sn[8];
    *reinterpret_cast<float4 *>(cs) = *reinterpret_cast<const float4 *>(cp);
    *reinterpret_cast<float4 *>(cs + 4) = *reinterpret_cast<const float4 *>(cp + 4);
    *reinterpret_cast<float4 *>(sn) = *reinterpret_cast<const float4 *>(sp);
    *reinterpret_cast<float4 *>(sn + 4) = *reinterpret_cast<const float4 *>(sp + 4);
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // rotate_neox_pair (rotary.rs:467-481)
      const float first = a[j], second = b[j];
      a[j] = first * cs[j] - second * sn[j];
      b[j] = second * cs[j] + first * sn[j];
    }
  };
  auto to_bf16 = [](const float4 (&x)[2], float s) {
    const float *f = reinterpret_cast<const float *>(x);
    bf16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = (bf16)(f[j] * s);
    return o;
  };
  auto load2 = [](const float *p, float4 (&x)[2]) {
    x[0] = *reinterpret_cast<const float4 *>(p);
    x[1] = *reinterpret_cast<const float4 *>(p + 4);
  };
  auto store2 = [](float *p, const float4 (&x)[2]) {
    *reinterpret_cast<float4 *>(p) = x[0];
    *reinterpret_cast<float4 *>(p + 4) = x[1];
  };
  auto row_inv = [&](const float *row) {
    if constexpr (NORM_D > 0) return quad_inv_rms<NORM_D>(row, c, nrm.eps);
    return 1.0f;
  };
  // Gemma QK-norm of a row's eight pairs: (x * inv) * w, as the prologue.
  auto norm = [&](float4 (&lo)[2], float4 (&hi)[2], float inv, const float *w) {
    float4 wl[2], wh[2];
    load2(w + p0, wl);
    load2(w + half + p0, wh);
    float *a = reinterpret_cast<float *>(lo), *b = reinterpret_cast<float *>(hi);
    const float *x = reinterpret_cast<const float *>(wl), *y = reinterpret_cast<const float *>(wh);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      a[j] = a[j] * inv * x[j];
      b[j] = b[j] * inv * y[j];
    }
  };

  if (!kv) {
    const int hq = blockIdx.y - H;
    const long i = 64L * blockIdx.x + r;
    if (i >= S) return;
    const float *src = q + (i * Hq + hq) * (long)D;
    float4 lo[2], hi[2];
    load2(src + p0, lo);
    load2(src + half + p0, hi);
    if (NORM_D) norm(lo, hi, row_inv(src), nrm.q_norm);
    rotate(lo, hi, P + i);
    if (NORM_D) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        lo[j] = make_float4(lo[j].x * nrm.q_prescale, lo[j].y * nrm.q_prescale, lo[j].z * nrm.q_prescale,
                            lo[j].w * nrm.q_prescale);
        hi[j] = make_float4(hi[j].x * nrm.q_prescale, hi[j].y * nrm.q_prescale, hi[j].z * nrm.q_prescale,
                            hi[j].w * nrm.q_prescale);
      }
    }
    bf16 *dst = qb + (i * Hq + hq) * (long)D;
    *reinterpret_cast<bf16x8 *>(dst + p0) = to_bf16(lo, qscale);
    *reinterpret_cast<bf16x8 *>(dst + half + p0) = to_bf16(hi, qscale);
    return;
  }

  const int h = blockIdx.y;
  const long P0 = (P & ~63L) + 64L * blockIdx.x;
  const long pos = P0 + r;
  float4 klo[2], khi[2], vlo[2], vhi[2];
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
  klo[0] = klo[1] = khi[0] = khi[1] = vlo[0] = vlo[1] = vhi[0] = vhi[1] = z;
  const bool row = pos >= P && pos < P + S;
  if (row) {
    const long i = pos - P;
    const float *ks = k + (i * H + h) * (long)D, *vs = v + (i * H + h) * (long)D;
    load2(ks + p0, klo);
    load2(ks + half + p0, khi);
    load2(vs + p0, vlo);
    load2(vs + half + p0, vhi);
    if (NORM_D) norm(klo, khi, row_inv(ks), nrm.k_norm);
    rotate(klo, khi, pos);
    float *ck = cache_k + (pos * H + h) * (long)D, *cv = cache_v + (pos * H + h) * (long)D;
    store2(ck + p0, klo);
    store2(ck + half + p0, khi);
    store2(cv + p0, vlo);
    store2(cv + half + p0, vhi);
  }
  if (pos >= P && pos < pad_end) {  // the chunk's rows, then zero padding
    bf16 *dk = kb + ((long)h * cap + pos) * D;
    *reinterpret_cast<bf16x8 *>(dk + p0) = to_bf16(klo, 1.0f);
    *reinterpret_cast<bf16x8 *>(dk + half + p0) = to_bf16(khi, 1.0f);
  }
  {
    float *t = &tile[r][8 * c];
    const float *a = reinterpret_cast<const float *>(vlo), *b = reinterpret_cast<const float *>(vhi);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      t[j] = a[j];
      t[32 + j] = b[j];
    }
  }
  __syncthreads();
  // V^T: 64 dim rows (lo 32, hi 32) x 64 slots, eight slots per store.
  for (int w = threadIdx.x; w < 64 * 8; w += 256) {
    const int dd = w >> 3, c8 = w & 7;
    const int dim = dd < 32 ? 32 * blockIdx.z + dd : half + 32 * blockIdx.z + (dd - 32);
    const long s0 = P0 + 8 * c8;
    bf16 *dst = vt + ((long)h * D + dim) * cap;
    const long g0 = s0 & ~15L;  // the aligned 16-key group these slots hold
    if (g0 >= P && g0 + 16 <= pad_end) {
      bf16x8 vv;
#pragma unroll
      for (int j = 0; j < 8; ++j) vv[j] = (bf16)tile[vt_key_slot(s0 + j) - P0][dd];
      *reinterpret_cast<bf16x8 *>(dst + s0) = vv;
    } else {
      for (int j = 0; j < 8; ++j) {
        const long sl = s0 + j, key = vt_key_slot(sl);
        if (key >= P && key < pad_end) dst[sl] = (bf16)tile[key - P0][dd];
      }
    }
  }
}

static inline unsigned blocks_for(long n, int per) { return (unsigned)((n + per - 1) / per); }

hipError_t launch_prefill_append(hipStream_t st, const float *q, const float *k, const float *v,
                                 const float *cos_tab, const float *sin_tab, size_t P, size_t S, size_t H,
                                 size_t Hq, size_t D, float *cache_k, float *cache_v, bf16 *kb, bf16 *vt,
                                 size_t cap, bf16 *qb, float qscale, const PrefillNorm *norm) {
  if (S == 0) return hipSuccess;
  const long pad_end = ((long)(P + S) + 63) & ~63L;
  if (D % 64 != 0 || cap % 64 != 0 || pad_end > (long)cap) return hipErrorInvalidValue;
  const long kv_blocks = (pad_end - ((long)P & ~63L)) / 64, q_blocks = qb ? ((long)S + 63) / 64 : 0;
  // (No qb: the attention rotates and scales q itself; only the K/V rows.)
  dim3 grid((unsigned)std::max(kv_blocks, q_blocks), (unsigned)(H + (qb ? Hq : 0)), (unsigned)(D / 64));
  const PrefillNorm none{};
  auto kern = prefill_append_kernel<0>;
  if (norm) {
    if (D != 64 && D != 128 && D != 256) return hipErrorInvalidValue;
    kern = D == 64 ? prefill_append_kernel<64> : D == 128 ? prefill_append_kernel<128> : prefill_append_kernel<256>;
  }
  hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, q, k, v, cos_tab, sin_tab, (long)P, (long)S, (int)H, (int)Hq,
                     (int)D, cache_k, cache_v, kb, vt, (long)cap, pad_end, qb, qscale, norm ? *norm : none);
  return hipGetLastError();
}

hipError_t launch_rope_apply(hipStream_t st, const float *cos_tab, const float *sin_tab,
                             size_t tab_stride, float *q, float *k, size_t S, size_t qh,
                             size_t kh, size_t D, size_t half) {
  long total = (long)S * (long)(qh + kh) * (long)half;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(rope_apply_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, st, cos_tab,
                     sin_tab, (long)tab_stride, q, k, (long)S, (int)qh, (int)kh, (int)D, (int)half);
  return hipGetLastError();
}

hipError_t launch_rms_norm(hipStream_t st, const float *x, const float *w, size_t rows,
                           size_t cols, float eps, float *out) {
  if (rows == 0) return hipSuccess;
  // wide rows: a workgroup per row, so loads are coalesced and never serial
  if (cols >= 512 && cols <= (size_t)kNormRowMax)
    hipLaunchKernelGGL(rms_norm_row_kernel, dim3((unsigned)rows), dim3(256), 0, st, x, w, (int)cols, eps, out);
  else
    hipLaunchKernelGGL(rms_norm_kernel, dim3(blocks_for((long)rows, 64)), dim3(64), 0, st, x, w,
                       (long)rows, (int)cols, eps, out);
  return hipGetLastError();
}

hipError_t launch_rms_norm_tree(hipStream_t st, const float *x, const float *w, size_t rows, size_t cols,
                                float eps, float *out) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(rms_norm_tree_kernel, dim3((unsigned)rows), dim3(256), 0, st, x, w, (int)cols, eps, out);
  return hipGetLastError();
}

hipError_t launch_gemma_prologue(hipStream_t st, const float *cos_tab, const float *sin_tab,
                                 size_t tab_stride, float *q, float *k, size_t S, size_t qh,
                                 size_t kh, size_t D, size_t half, const float *qn,
                                 const float *kn, float eps, float prescale) {
  long rows = (long)S * (long)(qh + kh);
  if (rows == 0) return hipSuccess;
  if (2 * half == D && (D == 64 || D == 128 || D == 256)) {  // one wave per row, coalesced
    auto kern = D == 64 ? gemma_prologue_wave_kernel<64>
                : D == 128 ? gemma_prologue_wave_kernel<128> : gemma_prologue_wave_kernel<256>;
    hipLaunchKernelGGL(kern, dim3(blocks_for(rows, 4)), dim3(256), 0, st, cos_tab, sin_tab, (long)tab_stride, q, k,
                       (long)S, (int)qh, (int)kh, qn, kn, eps, prescale);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(gemma_prologue_kernel, dim3(blocks_for(rows, 64)), dim3(64), 0, st, cos_tab,
                     sin_tab, (long)tab_stride, q, k, (long)S, (int)qh, (int)kh, (int)D, (int)half,
                     qn, kn, eps, prescale);
  return hipGetLastError();
}

hipError_t launch_stage_bf16(hipStream_t st, const float *k_rows, const float *v_rows, size_t n,
                             size_t n_pad_rows, size_t H, size_t D, bf16 *kb, bf16 *vt,
                             size_t dst_first, size_t dst_cap) {
  long n_pad = (long)n_pad_rows;
  if (n_pad <= 0) return hipSuccess;
  if ((long)dst_first + n_pad > (long)dst_cap || n_pad < (long)n || D % 64 != 0 || dst_cap % 64 != 0)
    return hipErrorInvalidValue;
  const long first_block = (long)dst_first & ~63L, last = (long)dst_first + n_pad;
  dim3 grid(blocks_for(last - first_block, 64), (unsigned)H, (unsigned)(D / 64));
  hipLaunchKernelGGL(stage_bf16_kernel, grid, dim3(256), 0, st, k_rows, v_rows, (long)n, n_pad,
                     (int)H, (int)D, kb, vt, (long)dst_first, (long)dst_cap);
  return hipGetLastError();
}

}  // namespace spissa
