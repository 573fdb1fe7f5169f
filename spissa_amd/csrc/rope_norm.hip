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
// Each quad of lanes owns one whole row of D floats; workgroups take RPW
// rows of one tensor and head:
//   K blocks (blockIdx.y < H): cache position P + i receives the rotated key
//     row i of the chunk in the f32 rows and in bf16 in the shadow K
//     [H, cap, D]; shadow positions [P + S, pad_end) are zeroed so the last
//     key tile the prefill kernel reads is finite.
//   V blocks (H <= blockIdx.y < 2H): the value row in the f32 rows, and in
//     bf16 at slot vt_key_slot(pos) of the shadow V^T [H, D, cap] (through
//     an LDS tile), zeros for the padding positions.
//   Q blocks (blockIdx.y >= 2H): query row i, rotated at position P + i,
//     times qscale, rounded to bf16 into qb [S, Hq, D] -- the prefill
//     kernel's Q operand, the same bits it would form from the rotated f32 row.
// Lane c of a quad holds dims 32z + 16e + 4c + [0, 4) of each half (z < D/64,
// e < 2): the quad covers 64 contiguous bytes of a row per access, and rotary
// pair p = (p, D/2 + p) sits in one lane.
// With NORM the Gemma QK-norm (ops.rs:159-179, as models/gemma/generate.rs:
// 232-245 calls it) comes first: the row's sum of squares in index order,
// four rounded squares at a time, the running sum passed from lane to lane
// of the quad by a DPP rotation; then x * inv * w.
// Grid: (position blocks of RPW, 2H + Hq (Hq only with qb)), 4 * RPW threads.
template <int D>
__device__ __forceinline__ float quad_inv_rms(const float4 (&x)[2][D / 64][2], int c, float eps) {
#pragma clang fp contract(off)
  constexpr int G = D / 64;
  float acc = 0.0f;
#pragma unroll
  for (int part = 0; part < 2; ++part)
#pragma unroll
    for (int z = 0; z < G; ++z)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float *v = reinterpret_cast<const float *>(&x[part][z][e]);
#pragma unroll
        for (int turn = 0; turn < 4; ++turn) {
          float t = acc;
#pragma unroll
          for (int j = 0; j < 4; ++j) t = t + v[j] * v[j];
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

template <int D, bool NORM, int RPW>
__global__ __launch_bounds__(RPW * 4) void prefill_append_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ cos_tab, const float *__restrict__ sin_tab, long P, long S, int H, int Hq,
    float *__restrict__ cache_k, float *__restrict__ cache_v, bf16 *__restrict__ kb, bf16 *__restrict__ vt,
    long cap, long pad_end, bf16 *__restrict__ qb, float qscale, const PrefillNorm nrm) {
#pragma clang fp contract(off)
  typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
  typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
  constexpr int HALF = D / 2, G = D / 64;
  __shared__ bf16 tile[RPW][D + 8];  // V[position][dim] of the block, padded
  const int r = threadIdx.x >> 2, c = threadIdx.x & 3;
  float4 x[2][G][2];  // [half][z][e]
  auto off = [&](int z, int e) { return 32 * z + 16 * e + 4 * c; };
  auto load_row = [&](const float *row) {
#pragma unroll
    for (int part = 0; part < 2; ++part)
#pragma unroll
      for (int z = 0; z < G; ++z)
#pragma unroll
        for (int e = 0; e < 2; ++e) x[part][z][e] = *reinterpret_cast<const float4 *>(row + part * HALF + off(z, e));
  };
  auto load8 = [&](const float *p, int z, float (&o)[8]) {
    *reinterpret_cast<float4 *>(o) = *reinterpret_cast<const float4 *>(p + off(z, 0));
    *reinterpret_cast<float4 *>(o + 4) = *reinterpret_cast<const float4 *>(p + off(z, 1));
  };
  // QK-norm (with NORM) and rotate_neox_pair (rotary.rs:467-481) at `pos`.
  // The 16-row form (short chunks: latency-bound, few waves) loads every
  // chunk's weights and table rows before the sum of squares, so their
  // latency runs beside it (Gemma-3-4B chunk of 128 on 16384: 1.044 -> 0.992
  // ms over 34 layers); the 64-row form loads them chunk by chunk after it,
  // keeping the registers for residency (the same early loads took Gemma-3-1B's
  // 4096-token prefill from 1.10-1.12 to 1.14 ms).
  constexpr bool EARLY = RPW < 64;
  auto norm_rotate = [&](const float *w, long pos) {
    float wl[EARLY ? G : 1][8], wh[EARLY ? G : 1][8], cs[EARLY ? G : 1][8], sn[EARLY ? G : 1][8];
    auto load_chunk = [&](int z, int i) {
      if constexpr (NORM) {
        load8(w, z, wl[i]);
        load8(w + HALF, z, wh[i]);
      }
      if (cos_tab) {
        load8(cos_tab + pos * HALF, z, cs[i]);
        load8(sin_tab + pos * HALF, z, sn[i]);
      }
    };
    if constexpr (EARLY) {
#pragma unroll
      for (int z = 0; z < G; ++z) load_chunk(z, z);
    }
    float inv = 1.0f;
    if constexpr (NORM) inv = quad_inv_rms<D>(x, c, nrm.eps);
#pragma unroll
    for (int z = 0; z < G; ++z) {
      const int i = EARLY ? z : 0;
      if constexpr (!EARLY) load_chunk(z, 0);
      float *a = reinterpret_cast<float *>(x[0][z]), *b = reinterpret_cast<float *>(x[1][z]);
      if constexpr (NORM) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          a[j] = a[j] * inv * wl[i][j];
          b[j] = b[j] * inv * wh[i][j];
        }
      }
      if (cos_tab) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float first = a[j], second = b[j];
          a[j] = first * cs[i][j] - second * sn[i][j];
          b[j] = second * cs[i][j] + first * sn[i][j];
        }
      }
    }
  };
  auto store_bf16 = [&](bf16 *dst, float s) {
#pragma unroll
    for (int part = 0; part < 2; ++part)
#pragma unroll
      for (int z = 0; z < G; ++z)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float4 f = x[part][z][e];
          bf16x4 o;
          o[0] = (bf16)(f.x * s); o[1] = (bf16)(f.y * s); o[2] = (bf16)(f.z * s); o[3] = (bf16)(f.w * s);
          *reinterpret_cast<bf16x4 *>(dst + part * HALF + off(z, e)) = o;
        }
  };
  auto store_f32 = [&](float *dst) {
#pragma unroll
    for (int part = 0; part < 2; ++part)
#pragma unroll
      for (int z = 0; z < G; ++z)
#pragma unroll
        for (int e = 0; e < 2; ++e) *reinterpret_cast<float4 *>(dst + part * HALF + off(z, e)) = x[part][z][e];
  };

  const int y = blockIdx.y;
  if (y >= 2 * H) {
    const int hq = y - 2 * H;
    const long i = (long)RPW * blockIdx.x + r;
    if (i >= S) return;
    load_row(q + (i * Hq + hq) * (long)D);
    norm_rotate(nrm.q_norm, P + i);
    if constexpr (NORM) {
#pragma unroll
      for (int part = 0; part < 2; ++part)
#pragma unroll
        for (int z = 0; z < G; ++z)
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            float4 &t = x[part][z][e];
            t = make_float4(t.x * nrm.q_prescale, t.y * nrm.q_prescale, t.z * nrm.q_prescale, t.w * nrm.q_prescale);
          }
    }
    store_bf16(qb + (i * Hq + hq) * (long)D, qscale);
    return;
  }
  const bool is_k = y < H;
  const int h = is_k ? y : y - H;
  const long P0 = (P & ~(long)(RPW - 1)) + (long)RPW * blockIdx.x;
  const long pos = P0 + r;
  const bool row = pos >= P && pos < P + S;
  if (row) {
    load_row((is_k ? k : v) + ((pos - P) * H + h) * (long)D);
  } else {
#pragma unroll
    for (int part = 0; part < 2; ++part)
#pragma unroll
      for (int z = 0; z < G; ++z) x[part][z][0] = x[part][z][1] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (is_k) {
    if (row) {
      norm_rotate(nrm.k_norm, pos);
      store_f32(cache_k + (pos * H + h) * (long)D);
    }
    if (pos >= P && pos < pad_end) store_bf16(kb + ((long)h * cap + pos) * D, 1.0f);  // the rows, then zeros
    return;
  }
  if (row) store_f32(cache_v + (pos * H + h) * (long)D);
#pragma unroll
  for (int part = 0; part < 2; ++part)
#pragma unroll
    for (int z = 0; z < G; ++z)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float4 f = x[part][z][e];
        bf16x4 o;
        o[0] = (bf16)f.x; o[1] = (bf16)f.y; o[2] = (bf16)f.z; o[3] = (bf16)f.w;
        *reinterpret_cast<bf16x4 *>(&tile[r][part * HALF + off(z, e)]) = o;
      }
  __syncthreads();
  // V^T: D dim rows x RPW slots, eight slots per store; slot s holds the key
  // at position vt_key_slot(s), which lies in the same aligned 16-group.
  constexpr int SG = RPW / 8;
  for (int w = threadIdx.x; w < D * SG; w += RPW * 4) {
    const int dd = w / SG, c8 = w % SG;
    const long s0 = P0 + 8 * c8;
    bf16 *dst = vt + ((long)h * D + dd) * cap;
    const long g0 = s0 & ~15L;  // the aligned 16-key group these slots hold
    if (g0 >= P && g0 + 16 <= pad_end) {
      bf16x8 vv;
#pragma unroll
      for (int j = 0; j < 8; ++j) vv[j] = tile[vt_key_slot(s0 + j) - P0][dd];
      *reinterpret_cast<bf16x8 *>(dst + s0) = vv;
    } else {
      for (int j = 0; j < 8; ++j) {
        const long sl = s0 + j, key = vt_key_slot(sl);
        if (key >= P && key < pad_end) dst[sl] = tile[key - P0][dd];
      }
    }
  }
}

static inline unsigned blocks_for(long n, int per) { return (unsigned)((n + per - 1) / per); }

template <int D, bool NORM, int RPW>
static hipError_t launch_append_rows(hipStream_t st, const float *q, const float *k, const float *v,
                                     const float *cos_tab, const float *sin_tab, long P, long S, int H, int Hq,
                                     float *cache_k, float *cache_v, bf16 *kb, bf16 *vt, long cap, long pad_end,
                                     bf16 *qb, float qscale, const PrefillNorm &nrm) {
  const long kv_blocks = (pad_end - (P & ~(long)(RPW - 1))) / RPW, q_blocks = qb ? (S + RPW - 1) / RPW : 0;
  dim3 grid((unsigned)std::max(kv_blocks, q_blocks), (unsigned)(2 * H + (qb ? Hq : 0)));
  hipLaunchKernelGGL((prefill_append_kernel<D, NORM, RPW>), grid, dim3(4 * RPW), 0, st, q, k, v, cos_tab, sin_tab, P,
                     S, H, Hq, cache_k, cache_v, kb, vt, cap, pad_end, qb, qscale, nrm);
  return hipGetLastError();
}

template <int D, bool NORM>
static hipError_t launch_append_d(hipStream_t st, const float *q, const float *k, const float *v,
                                  const float *cos_tab, const float *sin_tab, long P, long S, int H, int Hq,
                                  float *cache_k, float *cache_v, bf16 *kb, bf16 *vt, long cap, long pad_end,
                                  bf16 *qb, float qscale, const PrefillNorm &nrm) {
  // 64-row workgroups when they give every CU one (Llama-3.2-3B 4096 rows:
  // 1024; Gemma-3-1B: 384), else 16-row ones (one wave each) for more
  // workgroups on short chunks.
  const long blocks64 = (pad_end - (P & ~63L)) / 64 * (2 * H + (qb ? Hq : 0));
  if (blocks64 >= 256)
    return launch_append_rows<D, NORM, 64>(st, q, k, v, cos_tab, sin_tab, P, S, H, Hq, cache_k, cache_v, kb, vt, cap,
                                           pad_end, qb, qscale, nrm);
  return launch_append_rows<D, NORM, 16>(st, q, k, v, cos_tab, sin_tab, P, S, H, Hq, cache_k, cache_v, kb, vt, cap,
                                         pad_end, qb, qscale, nrm);
}

hipError_t launch_prefill_append(hipStream_t st, const float *q, const float *k, const float *v,
                                 const float *cos_tab, const float *sin_tab, size_t P, size_t S, size_t H,
                                 size_t Hq, size_t D, float *cache_k, float *cache_v, bf16 *kb, bf16 *vt,
                                 size_t cap, bf16 *qb, float qscale, const PrefillNorm *norm) {
  if (S == 0) return hipSuccess;
  const long pad_end = ((long)(P + S) + 63) & ~63L;
  if ((D != 64 && D != 128 && D != 256) || cap % 64 != 0 || pad_end > (long)cap) return hipErrorInvalidValue;
  // (No qb: the attention rotates and scales q itself; only the K/V rows.)
  const PrefillNorm nrm = norm ? *norm : PrefillNorm{};
#define SPISSA_APPEND_D(DD)                                                                                          \
  if (D == DD)                                                                                                       \
    return norm ? launch_append_d<DD, true>(st, q, k, v, cos_tab, sin_tab, (long)P, (long)S, (int)H, (int)Hq, cache_k, \
                                            cache_v, kb, vt, (long)cap, pad_end, qb, qscale, nrm)                    \
                : launch_append_d<DD, false>(st, q, k, v, cos_tab, sin_tab, (long)P, (long)S, (int)H, (int)Hq, cache_k, \
                                             cache_v, kb, vt, (long)cap, pad_end, qb, qscale, nrm);
  SPISSA_APPEND_D(64)
  SPISSA_APPEND_D(128)
  SPISSA_APPEND_D(256)
#undef SPISSA_APPEND_D
  return hipErrorInvalidValue;
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
