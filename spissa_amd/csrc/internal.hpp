// internal.hpp -- shared types and kernel launchers of the gfx950 attention path.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>

#include <cstddef>
#include <cstdint>

#include "../../include/spissa_hip.h"

namespace spissa {

typedef __bf16 bf16;

// Device-side error bits reported through spissa_session_sync().
enum : int { kDevErrSoftmaxDenominator = 1 };

// Largest batch a single decode launch carries in its kernel arguments.
constexpr int kMaxDecodeBatch = 16;
// Most key splits of one (sequence, KV head) the decode combine reads.
constexpr int kMaxDecodeSplits = 512;
// Most workgroups a decode launch aims at, token splits included: two per CU
// on 256 CUs. Split-kernel grids a few workgroups past it ran far slower than
// grids just under it (Gemma-3-4B's global layer at 16512 keys: 520 against
// 464 workgroups, 34.5 against 27.4 us per layer), and grids of 3-4 per CU
// (Llama-3.2-3B at 8192 keys, 696 workgroups: 17.3 us) slower than 2 (464:
// 16.3 us).
constexpr int kDecodeGridWorkgroups = 512;
// Prefill key tiles are at most this wide; the staging buffer starts at a
// multiple of it.
constexpr int kPrefillTileAlign = 64;

// Key order of the transposed bf16 V operand (the cache shadow's vt and the
// prefill staging buffer): inside every group of 16 keys, keys 4-7 and 8-11
// trade places, so that the 8 keys one MFMA lane contributes to a 16-key step
// of O^T += V^T P^T (keys 0-3 and 8-11, or 4-7 and 12-15, as the score
// accumulator holds them) are 16 contiguous bytes. The map is its own inverse.
__host__ __device__ constexpr long vt_key_slot(long key) {
  return (key & ~12L) | ((key & 4) << 1) | ((key & 8) >> 1);
}

struct SeqDesc {
  const float *k;  // cache keys   [max_seq, Hkv, D] (may be null when past == 0)
  const float *v;  // cache values [max_seq, Hkv, D]
  int past;        // cached tokens
  int pad;
};

struct DecodeArgs {
  float *q;            // [B, Hq, D]; read only (rotated in registers when rope_cos is set)
  float *cur_k;        // [B, Hkv, D]: the new token's key; read only
  const float *cur_v;  // [B, Hkv, D]
  float *out;          // [B, Hq, D]
  float *partial;      // [B, Hkv, HB, max_splits] entries of RB*(D+2) floats
  int *err;            // device error bits
  // Fused RoPE (rotate-half over the whole head, D/2 pairs): table rows are
  // absolute positions; the new token of sequence b sits at position seq[b].past.
  const float *rope_cos;  // [positions, D/2] or null (no RoPE)
  const float *rope_sin;
  // Fused append: cache rows seq[b].past receive the (rotated) new key and value.
  float *app_k[kMaxDecodeBatch];
  float *app_v[kMaxDecodeBatch];
  // bf16 prefill shadow of the cache (null when the cache has none): the
  // appended row also goes to kb [Hkv, cap, D] and vt [Hkv, D, cap].
  bf16 *app_kb[kMaxDecodeBatch];
  bf16 *app_vt[kMaxDecodeBatch];
  long app_cap[kMaxDecodeBatch];
  int do_append;
  // Fused Gemma QK-norm (models/gemma/generate.rs:232-275), null: none. q and
  // the new key are RMS-normed with these [D] weights before RoPE, and q is
  // multiplied by q_prescale after it.
  const float *q_norm;
  const float *k_norm;
  float norm_eps, q_prescale;
  int B, Hq, Hkv, R, HB;  // R = Hq/Hkv, HB = head blocks per kv head
  int window;
  int kps;             // cached keys per split
  int max_splits;      // splits of the longest sequence in the launch (with the token's own)
  // 1: split 0 is the new token's own split, dispatched first, and the cached
  // keys' splits are 1..max_splits-1 (the token's latency -- loads, QK-norm,
  // RoPE, append -- then overlaps the streaming splits); 0: cached split 0
  // takes the token after its cached rows.
  int tok_split;
  float qscale;        // softmax scale * log2(e), applied to the scores
  SeqDesc seq[kMaxDecodeBatch];
};

// Linear projection out[M, N] = x[M, K] x W[N, K]^T + bias (linear.hip).
struct LinearArgs {
  const void *w;       // [N, K] row-major, dtype
  const float *x;      // [M, K]
  const float *bias;   // [N] or null
  float *out;          // [M, N]
  int M, N, K;
  int dtype;           // spissa_dtype
  // GEMV path only: when set, each x row is RMS-normed with these [K]
  // weights first (ops.rs:159-179 up to rounding: the sum of squares rides
  // the dot-product loop and 1/rms scales the finished sums).
  const float *norm_w;
  float norm_eps;
  int cus;  // compute units of the device (sizes the GEMM's tiles; 0: 256)
};
enum { kLinearGemv = 0, kLinearGemm = 1, kLinearGeneric = 2, kLinearSkinny = 3 };

struct PrefillArgs {
  const float *q;     // [S, Hq, D] f32
  // Or, when set, Q already scaled by qk_scale_log2 and rounded to bf16
  // [S, Hq, D] (the fused prefill step's staging); q is then unused.
  const bf16 *qb;
  // With q (f32): when set, the RoPE tables [position][D/2] q is rotated by
  // at load, query i at position P + i (rotate-half, each product rounded
  // apart, as the append pass rotates it), before the scale.
  const float *q_cos, *q_sin;
  float *out;         // [S, Hq, D] f32
  // bf16 K/V for keys [0, P8) come from the cache shadow, keys [P8, P+S) from
  // the staging buffer; P8 is a multiple of kPrefillTileAlign, so no key tile
  // straddles the two.
  const bf16 *kb_cache;  // [Hkv, cap_cache, D]
  const bf16 *vt_cache;  // [Hkv, D, cap_cache], keys in vt_key_slot order
  const bf16 *kb_stage;  // [Hkv, cap_stage, D], key 0 of the buffer is absolute key P8
  const bf16 *vt_stage;  // [Hkv, D, cap_stage], keys in vt_key_slot order
  long cap_cache, cap_stage;
  int P, P8, S, Hq, Hkv, R;
  int causal, window;
  int *err;
  float qk_scale_log2;  // softmax scale * log2(e), applied to the f32 scores
  int n_qblocks;        // query blocks of one workgroup (set by the launcher)
  // Key splits (flash-decoding for short chunks over long caches): with
  // splits > 1, split j of a workgroup covers key tiles [j*tps, (j+1)*tps) of
  // the workgroup's visible tile range and writes its unnormalised O and
  // (m, l) per query row to part_o [splits][S][Hq][D] and part_ml
  // [splits][S][Hq][2] (m in the scaled log2 domain, -inf when the row saw no
  // key); launch_prefill_combine merges them. splits == 1 writes `out`.
  int splits, tps;
  float *part_o, *part_ml;
  // 1 (with key splits): the workgroups that read one KV head's split (its
  // head blocks and query blocks) are given ids 8 apart, so they run on one
  // XCD and share its L2 (the grid is padded to a multiple of 8 units).
  // 2 (unsplit windowed layers): the ids of one XCD take a contiguous run of
  // the workgroup order (the grid is padded to a multiple of 8).
  // prefill_use_xcd_group decides.
  int xcd_group;
  // Waves per query block that share its key tiles (1 or 2): with 2, the two
  // waves of a pair take alternate 64-key tiles of the same queries and merge
  // their (m, l, O) through LDS at the end, halving the longest causal
  // blocks' serial tile chain. prefill_wave_pairs decides.
  int ksp;
};

// Workgroup slots per CU and key-tile width of the prefill kernels, and the
// queries per workgroup, for choosing key splits.
int prefill_wgs_per_cu(const PrefillArgs &a, int D);
int prefill_tile_keys(int D);
int prefill_wg_queries(const PrefillArgs &a, int D);
int prefill_wg_heads(const PrefillArgs &a, int D);  // query heads per workgroup
// Workgroups one (unsplit) prefill launch would have.
long prefill_base_workgroups(const PrefillArgs &a, int D);
// Most key tiles one (unsplit) prefill workgroup visits.
long prefill_max_tile_span(const PrefillArgs &a, int D);
// Workgroups of a prefill launch of n_qblocks x head_blocks x Hkv x splits
// (grouped by XCD: units of one KV head and split padded to a multiple of 8).
long prefill_grid_workgroups(long n_qblocks, long head_blocks, long Hkv, long splits, int xcd_group);
int prefill_use_xcd_group(const PrefillArgs &a, int D);
int prefill_wave_pairs(const PrefillArgs &a, int D, long slots);

struct GenericArgs {
  const float *q;  // [S, Hq, D]
  const float *cur_k, *cur_v;  // [S, Hkv, D]
  const float *cache_k, *cache_v;  // [*, Hkv, D]
  float *out;
  int *err;
  int S, P, Hq, Hkv, D, R, causal, window;
  float scale;
};

// ---- launchers (each returns the launch error) ----
hipError_t launch_rope_apply(hipStream_t st, const float *cos_tab, const float *sin_tab,
                             size_t tab_stride, float *q, float *k, size_t S, size_t qh,
                             size_t kh, size_t D, size_t half);
hipError_t launch_rms_norm(hipStream_t st, const float *x, const float *w, size_t rows,
                           size_t cols, float eps, float *out);
// Tree-reduced RMSNorm (not the reference's summation order; rounding-level
// differences), one workgroup per row: the sublayer's wide norms.
hipError_t launch_rms_norm_tree(hipStream_t st, const float *x, const float *w, size_t rows, size_t cols,
                                float eps, float *out);
hipError_t launch_gemma_prologue(hipStream_t st, const float *cos_tab, const float *sin_tab,
                                 size_t tab_stride, float *q, float *k, size_t S, size_t qh,
                                 size_t kh, size_t D, size_t half, const float *qn,
                                 const float *kn, float eps, float prescale);
// The append half of a fused prefill step: rows [0, S) of k/v (optionally
// rotated with cos/sin rows at positions P + i) into cache rows [P, P + S)
// and the bf16 shadow (zeros up to the next multiple of 64), and, when qb is
// set, q rotated, scaled by qscale and rounded into qb [S, Hq, D] bf16.
// D % 64 == 0.
// Fused Gemma QK-norm of the prefill step's append (null q_norm: none): q
// and k rows are RMS-normed with the [D] weights before RoPE (the sum of
// squares in index order, ops.rs:159-179), and q is multiplied by q_prescale
// after it (models/gemma/generate.rs:232-275).
struct PrefillNorm {
  const float *q_norm, *k_norm;  // [D]
  float eps, q_prescale;
};
hipError_t launch_prefill_append(hipStream_t st, const float *q, const float *k, const float *v,
                                 const float *cos_tab, const float *sin_tab, size_t P, size_t S, size_t H,
                                 size_t Hq, size_t D, float *cache_k, float *cache_v, bf16 *kb, bf16 *vt,
                                 size_t cap, bf16 *qb, float qscale, const PrefillNorm *norm = nullptr);
// Writes rows [0, n) and zero rows [n, n_pad) at buffer positions dst_first + i.
hipError_t launch_stage_bf16(hipStream_t st, const float *k_rows, const float *v_rows, size_t n,
                             size_t n_pad, size_t H, size_t D, bf16 *kb, bf16 *vt,
                             size_t dst_first, size_t dst_cap);
hipError_t launch_decode(hipStream_t st, const DecodeArgs &a, int D, int RB);
// Streaming-read probe: reads bytes (a multiple of 16, 16-byte aligned) of buf once.
// The dense bf16 MFMA ceiling: rounds x 8 MFMAs on each of 8 waves per CU;
// *flop receives the launch's FLOP count.
hipError_t launch_mfma_rate(hipStream_t st, int cus, int rounds, float *sink, double *flop);
hipError_t launch_hbm_read(hipStream_t st, const void *buf, size_t bytes, float *sink);
hipError_t launch_prefill(hipStream_t st, const PrefillArgs &a, int D);
// Merges the key splits of a split prefill into `out` (and the error flag).
hipError_t launch_prefill_combine(hipStream_t st, const PrefillArgs &a, int D);
hipError_t launch_generic(hipStream_t st, const GenericArgs &a);
// Kernel choice for a linear projection (kLinearGemv for M <= 4; for bf16
// weights kLinearSkinny for M <= 64 with K % 128 == 0, kLinearGemm for larger M
// with K % 32 == 0; else kLinearGeneric), and its launch. The vector paths also need 16-byte aligned x and weight rows.
int linear_path(int dtype, long M, long K);
hipError_t launch_linear(hipStream_t st, const LinearArgs &a, int path);
// Projections of one input [M, K] by several weights in one GEMV launch when
// every segment takes the GEMV path with the same M, K, dtype and x (16-byte
// aligned); otherwise one launch each.
constexpr int kMaxLinearSegments = 3;
struct LinearSegments {
  LinearArgs seg[kMaxLinearSegments];
  int blocks[kMaxLinearSegments];  // workgroups of each segment
  int n;
};
hipError_t launch_linear_multi(hipStream_t st, const LinearArgs *segs, int n);

// Greedy token choice: one partial per contiguous range of the logits.
struct ArgmaxPart {
  float v;       // first maximum of the range's non-NaN, non-excluded values
  int i;         // its index (INT_MAX: the range has none)
  int last_nan;  // last NaN index of the range (-1: none)
  int pad;
};
constexpr int kArgmaxMaxParts = 1024;  // partials one launch writes at most
// token[0] = sample_argmax(x[0..n)) for excl < 0, else
// sample_argmax_excluding(x, excl) with 0 <= excl < n and n >= 2;
// n <= INT32_MAX - 1024.
hipError_t launch_argmax(hipStream_t st, const float *x, int n, int excl, ArgmaxPart *parts, int *token);

// Keys per split of a decode launch: keys[b] = visible cached keys of
// sequence b (nseq of them), heads = (KV head, head block) pairs per
// sequence; the longest range gets at most split_cap splits (and never more
// than kMaxDecodeSplits).
int decode_keys_per_split(int D, int RB, const int *keys, int nseq, long heads, int split_cap);
bool decode_supported(int D, int R);
bool prefill_supported(int D);

}  // namespace spissa
