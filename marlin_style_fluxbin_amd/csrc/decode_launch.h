// Launch plumbing for the decode attention and SwiGLU kernels (decode.hip).
#pragma once
#include "common.h"

namespace fx {

struct AttnArgs {
  const uint16_t* q;   // [Hq, D]
  const uint16_t* k;   // [Hk, Lmax, D]
  const uint16_t* v;   // [Hk, Lmax, D]
  float* partial;      // [Hq, splits, D + 2]
  uint16_t* out;       // [Hq, D]
  int Hq, Hk, Lmax, pos;
  int kpt, splits;     // keys per thread (1, 2, 4); splits = ceil((pos + 1) / (keys per workgroup))
  float scale;
};

// Keys one attention workgroup covers: 256 / (D / 8) key rows times keys per thread.
inline int attn_keys_per_block(int head_dim, int kpt) { return 256 / (head_dim / 8) * kpt; }

bool launch_decode_attention(int dt, int head_dim, const AttnArgs& a, hipStream_t s);
bool launch_silu_mul(int dt, const uint16_t* gate, const uint16_t* up, uint16_t* out, int n,
                     hipStream_t s);

}  // namespace fx
