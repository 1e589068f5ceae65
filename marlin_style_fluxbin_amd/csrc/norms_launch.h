// Launch plumbing for the RMSNorm / per-head norm + RoPE kernels (norms.hip).
#pragma once
#include "common.h"

namespace fx {

enum : int { kRopeNone = 0, kRopeStock = 1, kRopeFused = 2 };

constexpr int kMaxHeadTensors = 4;

// One tensor of [batch, heads, seq, head_dim] rows (element strides; head_dim
// is contiguous).  weight null: no RMSNorm; rope 0: RoPE not applied (a
// strided copy, e.g. v into a KV cache).
struct HeadTensor {
  const void* in;
  void* out;
  const void* weight;
  long long in_stride[3];   // batch, head, position
  long long out_stride[3];
  int heads;
  int rope;
};

struct HeadNormRopeArgs {
  HeadTensor t[kMaxHeadTensors];
  int rows[kMaxHeadTensors];  // batch * heads * seq per tensor
  int ntensors;
  int seq, head_dim;
  const void* cos;            // [.., head_dim] rows, element strides cs_stride
  const void* sin;
  long long cs_stride[2];     // batch, position
  const int* position;        // optional device scalar: cos/sin row offset position[0]
  float eps;
  int rope_mode;              // kRopeNone / kRopeStock / kRopeFused
};

bool launch_rmsnorm(int dt, const uint16_t* x, const uint16_t* residual, const uint16_t* weight,
                    uint16_t* out, uint16_t* residual_out, int rows, int hidden, float eps,
                    hipStream_t s);
bool launch_head_norm_rope(int dt, const HeadNormRopeArgs& a, hipStream_t s);

}  // namespace fx
