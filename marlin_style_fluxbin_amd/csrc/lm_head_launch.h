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

}  // namespace fx
