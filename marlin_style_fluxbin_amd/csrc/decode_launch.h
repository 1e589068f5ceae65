// Launch plumbing for the decode attention and SwiGLU kernels (decode.hip).
#pragma once
#include "common.h"

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
  float* partial;      // [Hq, splits, D + 2]
  unsigned* arrivals;  // [Hk] arrival counters (zero between calls)
  uint16_t* out;       // [Hq, D]
  int Hq, Hk, Lmax, pos;
  int kpt, splits;     // keys per thread (1, 2, 4); splits = ceil((pos + 1) / (keys per workgroup))
  int combine;         // kAttnDirect, kAttnLastArrival or kAttnCombineKernel
  float scale;
  AttnPre pre;
};

// How the per-split partials become the output: one split writes it directly;
// up to kAttnInlineSplits splits (with at most 256 (head, split) pairs and
// 256 * kAttnInlineOutputs output values per KV head) are combined by the last
// workgroup of the KV head to finish, in one load round; more go through the
// separate combine kernel.
enum : int { kAttnDirect = 0, kAttnLastArrival = 1, kAttnCombineKernel = 2 };
constexpr int kAttnInlineSplits = 16;
constexpr int kAttnInlineOutputs = 4;

// Keys one attention workgroup covers: 256 / (D / 8) key rows times keys per thread.
inline int attn_keys_per_block(int head_dim, int kpt) { return 256 / (head_dim / 8) * kpt; }

bool launch_decode_attention(int dt, int head_dim, const AttnArgs& a, hipStream_t s);
bool launch_silu_mul(int dt, const uint16_t* gate, const uint16_t* up, uint16_t* out, int n,
                     hipStream_t s);

}  // namespace fx
