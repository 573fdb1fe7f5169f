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
// Fan-in of the split-K combine tree.
constexpr int kCombineFanIn = 16;

struct SeqDesc {
  const float *k;  // cache keys   [max_seq, Hkv, D] (may be null when past == 0)
  const float *v;  // cache values [max_seq, Hkv, D]
  int past;        // cached tokens
  int pad;
};

struct DecodeArgs {
  const float *q;      // [B, Hq, D]
  const float *cur_k;  // [B, Hkv, D]: the new token's key
  const float *cur_v;
  float *out;          // [B, Hq, D]
  float *partial;      // combine-tree entries
  int *counters;       // combine-tree arrival counters (zero between launches)
  int *err;            // device error bits
  int B, Hq, Hkv, R, HB;  // R = Hq/Hkv, HB = head blocks per kv head
  int window;
  int kps;             // keys per split
  int max_entries;     // combine-tree entries per (b, h, hb) for the largest split count
  int max_counters;    // combine-tree counters per (b, h, hb)
  float qscale;        // softmax scale * log2(e), folded into q
  SeqDesc seq[kMaxDecodeBatch];
};

struct PrefillArgs {
  const float *q;     // [S, Hq, D] f32
  float *out;         // [S, Hq, D] f32
  // bf16 K/V for keys [0, P8) come from the cache shadow, keys [P8, P+S) from the staging buffer.
  const bf16 *kb_cache;  // [Hkv, cap_cache, D]
  const bf16 *vt_cache;  // [Hkv, D, cap_cache]
  const bf16 *kb_stage;  // [Hkv, cap_stage, D], key 0 of the buffer is absolute key P8
  const bf16 *vt_stage;  // [Hkv, D, cap_stage]
  long cap_cache, cap_stage;
  int P, P8, S, Hq, Hkv, R;
  int causal, window;
  int *err;
  float qk_scale_log2;  // softmax scale * log2(e), applied to the f32 scores
  int n_qblocks;        // query blocks of 32 positions
};

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
hipError_t launch_gemma_prologue(hipStream_t st, const float *cos_tab, const float *sin_tab,
                                 size_t tab_stride, float *q, float *k, size_t S, size_t qh,
                                 size_t kh, size_t D, size_t half, const float *qn,
                                 const float *kn, float eps, float prescale);
// Writes rows [0, n) and zero rows [n, n_pad) at buffer positions dst_first + i.
hipError_t launch_stage_bf16(hipStream_t st, const float *k_rows, const float *v_rows, size_t n,
                             size_t n_pad, size_t H, size_t D, bf16 *kb, bf16 *vt,
                             size_t dst_first, size_t dst_cap);
hipError_t launch_decode(hipStream_t st, const DecodeArgs &a, int D, int RB, int max_splits);
hipError_t launch_prefill(hipStream_t st, const PrefillArgs &a, int D);
hipError_t launch_generic(hipStream_t st, const GenericArgs &a);

// Keys per split chosen for a decode launch.
int decode_keys_per_split(int D, int RB, long total_keys_times_heads, int max_keys);
// Entries / counters of the combine tree for nsplit leaves.
int combine_tree_entries(int nsplit);
int combine_tree_counters(int nsplit);
bool decode_supported(int D, int R);
bool prefill_supported(int D);

}  // namespace spissa
