// Launch plumbing for the decode attention and SwiGLU kernels (decode.hip).
#pragma once
#include "common.h"
#include "lm_head_launch.h"

namespace fx {

// Per-head q/k RMSNorm + RoPE folded into the attention (q is then the raw
// projection); k_raw null: q is already normalised and rotated and the caches
// already hold position pos.
struct AttnPre {
  const uint16_t* k_raw;     // [Hk, D] raw key projection of position pos
  const uint16_t* v_raw;     // [Hk, D] value of position pos
  const uint16_t* q_weight;  // [D] q_norm weight
  const uint16_t* k_weight;  // [D] k_norm weight
  const uint16_t* cos;       // [D] RoPE row of position pos
  const uint16_t* sin;
  float eps;
  int rope_mode;             // 1 stock, 2 fused (addcmul)
};

struct AttnArgs {
  const uint16_t* q;   // [Hq, D]
  const uint16_t* k;   // [Hk, Lmax, D]
  const uint16_t* v;   // [Hk, Lmax, D]
  float* partial;      // [Hq, splits, D] split outputs, then [Hq, splits, 2] their (max, sum)
  uint16_t* out;       // [Hq, D]
  const int16_t* out_index;  // null: out in head order; else value i goes to out[out_index[i]]
  int Hq, Hk, Lmax, pos;
  int kpt, splits;     // keys per thread (1, 2, 4); splits = ceil((pos + 1) / (keys per workgroup))
  int groups;          // query-head groups of 256 threads per split workgroup (1, 2, 4)
  float scale;
  AttnPre pre;
};

// One split writes the output directly; more write partials that a second
// kernel (one workgroup per query head) combines.  A last-arriving-workgroup
// combine inside the split kernel measured slower at every decode length: its
// store wait, arrival atomic and coherent reloads form three dependent memory
// round trips on one workgroup (9.55 vs 7.46 us at 544 keys, 10.3 vs 7.5 us at
// 512, Qwen3-8B heads with q/k norm and RoPE), more than the second launch.  A
// single-pass kernel (one 512-thread workgroup per query head over all keys,
// every load issued up front, no partials) is faster only while the cache is
// hot (4.9 us in a loop over one layer's cache): in the 36-layer decode graph,
// where each layer's cache comes from HBM, its 32 workgroups stream 278 KB each
// at ~30 GB/s per CU and the step took 1.513 against 1.441 ms per token.

// Keys one attention workgroup covers: 256 / (D / 8) key rows times keys per thread.
inline int attn_keys_per_block(int head_dim, int kpt) { return 256 / (head_dim / 8) * kpt; }

bool launch_decode_attention(int dt, int head_dim, const AttnArgs& a, hipStream_t s);
bool launch_silu_mul(int dt, const uint16_t* gate, const uint16_t* up, uint16_t* out, int n,
                     hipStream_t s);
// Embedding row of *token + its 16-element tile sums of squares; out_index set:
// element i also goes to sorted_out[out_index[i]]; merge.prediction set: also the
// argmax merge of merge.part_val / part_idx (merge.blocks of them).
bool launch_decode_embed(int dt, const long long* token, const uint16_t* table, int vocab, int hidden,
                         uint16_t* out, float* tile_sumsq, const int16_t* out_index, uint16_t* sorted_out,
                         const LmHeadArgs& merge, hipStream_t s);

}  // namespace fx
