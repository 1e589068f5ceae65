// Launch plumbing for the decode LM head with the final RMSNorm and the greedy
// argmax folded in (lm_head.hip).
#pragma once
#include "common.h"

namespace fx {

constexpr int kLmWaves = 4;             // waves per workgroup (256 threads)
constexpr int kLmMaxChunks = 16;        // hidden <= 16 * 512
constexpr int kLmMaxBlocks = 4096;      // workgroups (argmax partials) per launch
constexpr int kLmRowsInFlight = 1;      // weight rows a wave loads before its first dot product
constexpr size_t kLmCounterBytes = 256; // reserved head of the workspace (kept for the ABI's size)

struct LmHeadArgs {
  const uint16_t* x;       // [K] hidden state (normalised here when norm_w is set)
  const uint16_t* norm_w;  // [K] final RMSNorm weight, or null: x is already normalised
  float eps;
  const uint16_t* w;       // [V, K] LM-head weight, row-major
  uint16_t* logits;        // [V]
  long long* prediction;   // [1] argmax of the rounded logits (first index of the maximum)
  unsigned* arrival;       // workspace head (unused), then the partials
  float* part_val;         // [blocks]
  int* part_idx;           // [blocks]
  int V, K, blocks;
};

bool launch_lm_head_argmax(int dt, const LmHeadArgs& a, hipStream_t s);
// The streaming kernel alone (logits and per-workgroup maxima; no prediction).
bool launch_lm_head_partials(int dt, const LmHeadArgs& a, hipStream_t s);
// The merge alone: the best of a.blocks partials -> *a.prediction.
void launch_lm_head_merge(const LmHeadArgs& a, hipStream_t s);

#ifdef __HIPCC__
// (v, i) ranks above (u, j): NaN above every number (the first NaN wins),
// otherwise the larger value, ties to the lower index.  A strict total order
// over distinct indices, so merges in any order give the same winner.
__device__ __forceinline__ bool ranks_above(float v, int i, float u, int j) {
  const bool vn = v != v, un = u != u;
  if (vn || un) return vn && (!un || i < j);
  return v > u || (v == u && i < j);
}

// One workgroup of kLmWaves waves: the best of `blocks` (value, index) partials
// under ranks_above -> *prediction (thread 0 writes).  Every thread calls it.
__device__ __forceinline__ void merge_argmax_partials(const float* part_val, const int* part_idx, int blocks,
                                                      long long* prediction) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  float v = -INFINITY;
  int i = 0x7fffffff;
  for (int b = t; b < blocks; b += 64 * kLmWaves) {
    const float pv = part_val[b];
    const int pi = part_idx[b];
    if (ranks_above(pv, pi, v, i)) {
      v = pv;
      i = pi;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o, 64);
    const int oi = __shfl_xor(i, o, 64);
    if (ranks_above(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
  __shared__ float wv[kLmWaves];
  __shared__ int wi[kLmWaves];
  if (lane == 0) {
    wv[wave] = v;
    wi[wave] = i;
  }
  __syncthreads();
  if (t == 0) {
    for (int w = 1; w < kLmWaves; ++w)
      if (ranks_above(wv[w], wi[w], v, i)) {
        v = wv[w];
        i = wi[w];
      }
    *prediction = i;
  }
}
#endif

}  // namespace fx
