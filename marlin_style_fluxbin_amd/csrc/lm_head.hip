// Batch-1 LM head of the greedy decode step for gfx950, with the final RMSNorm
// and the argmax folded in: the reference's decode step ends in the model's
// final norm, `lm_head` and `logits.argmax(-1, keepdim=True)`
// (static_decode.py:67-76; HF Qwen3ForCausalLM with logits_to_keep=1).
//
//   x      = round(w_norm * round(h * rsqrt(mean(h^2) + eps)))   (Qwen3RMSNorm)
//   logits = round(W x)          W [V, K] row-major, fp32 accumulation
//   pred   = argmax(logits)      over the rounded logits, first index of the
//                                maximum, NaN above every number (torch.argmax)
//
// HBM-bound: the weight (V K 2 bytes, 1.24 GB for Qwen3-8B) is streamed once per
// token with non-temporal loads; everything else is a few KB.
#include "common.h"
#include "lm_head_launch.h"

#include <climits>

namespace fx {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// a.lo * b.lo + a.hi * b.hi + c in fp32 (v_dot2c_f32_bf16 / v_dot2c_f32_f16)
template <int DT>
__device__ __forceinline__ float dot2(unsigned a, unsigned b, float c) {
  if constexpr (DT == kBF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                           false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c, false);
}

// grid `blocks` workgroups of 4 waves; wave w of the grid takes the row groups
// (RPI p .. RPI p + RPI - 1), p = w, w + waves, ... (neighbouring waves stream
// neighbouring rows).  Lane l holds elements [8 (64 c + l), +8) of the activation
// for each 512-element chunk c, so a weight row is NC loads of 16 B per lane,
// coalesced, and a wave keeps RPI rows (RPI * 8 KB at K = 4096) in flight.
// Every wave normalises the activation itself (the RMSNorm batch order of
// rmsnorm_kernel: per-chunk wave totals added in chunk order; bit-identical
// normalised values).  Each wave keeps its running argmax; the workgroup's
// best goes to the workspace with plain stores, and lm_head_merge_kernel -- the
// next launch on the stream, so the kernel boundary orders every block's stores
// before its loads -- merges them and writes the prediction.  (Merging inside this
// launch needs a device-scope release per block, which writes back the block's
// XCD L2: 191.5 -> 207.1 us per call at 151936 x 4096.)  A row's logit does not
// depend on RPI or the grid: each row is one wave's two dot2 chains and one
// wave total.
template <int DT, int NC, bool NORM, int RPI>
__global__ __launch_bounds__(256) void lm_head_argmax_kernel(LmHeadArgs a) {
  asm volatile("" ::"s"(a.x), "s"(a.norm_w), "s"(a.eps), "s"(a.w), "s"(a.logits), "s"(a.part_val),
               "s"(a.part_idx), "s"(a.V));
  constexpr int K = NC * 512;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;

  u32x4_t xv[NC];
  {
    const u32x4_t* xp = reinterpret_cast<const u32x4_t*>(a.x) + lane;
#pragma unroll
    for (int c = 0; c < NC; ++c) xv[c] = xp[64 * c];
  }
  if constexpr (NORM) {
    const u32x4_t* wp = reinterpret_cast<const u32x4_t*>(a.norm_w) + lane;
    u32x4_t wv[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) wv[c] = wp[64 * c];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) ss += wave_total(sum_sq8<DT>(xv[c]));
    const float inv = rsqrtf(ss / float(K) + a.eps);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float n0 = round_to<DT>(to_f32<DT>(uint16_t(xv[c][w])) * inv);
        const float n1 = round_to<DT>(to_f32<DT>(uint16_t(xv[c][w] >> 16)) * inv);
        const float y0 = to_f32<DT>(uint16_t(wv[c][w])) * n0;
        const float y1 = to_f32<DT>(uint16_t(wv[c][w] >> 16)) * n1;
        xv[c][w] = unsigned(from_f32<DT>(y0)) | (unsigned(from_f32<DT>(y1)) << 16);
      }
    }
  }

  float best = -INFINITY;
  int best_i = INT_MAX;
  const int waves = gridDim.x * kLmWaves, groups = (a.V + RPI - 1) / RPI;
  for (int p = blockIdx.x * kLmWaves + wave; p < groups; p += waves) {
    int r[RPI];
    u32x4_t b[RPI][NC];
#pragma unroll
    for (int j = 0; j < RPI; ++j) {
      r[j] = min(RPI * p + j, a.V - 1);  // the last group of a ragged V re-reads row V - 1
      const u32x4_t* wr = reinterpret_cast<const u32x4_t*>(a.w + size_t(r[j]) * K) + lane;
#pragma unroll
      for (int c = 0; c < NC; ++c) b[j][c] = __builtin_nontemporal_load(wr + 64 * c);
    }
    __builtin_amdgcn_sched_barrier(0);  // every row's loads in flight before the first use
    float sacc[RPI][2];
#pragma unroll
    for (int j = 0; j < RPI; ++j) sacc[j][0] = sacc[j][1] = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int j = 0; j < RPI; ++j) sacc[j][w & 1] = dot2<DT>(b[j][c][w], xv[c][w], sacc[j][w & 1]);
#pragma unroll
    for (int j = 0; j < RPI; ++j) {
      const float y = round_to<DT>(wave_total(sacc[j][0] + sacc[j][1]));
      const bool fresh = j == 0 || r[j] != r[j - 1];
      if (lane == j && fresh) a.logits[r[j]] = from_f32<DT>(y);
      if (fresh && ranks_above(y, r[j], best, best_i)) {
        best = y;
        best_i = r[j];
      }
    }
  }

  __shared__ float wbest[kLmWaves];
  __shared__ int wbest_i[kLmWaves];
  if (lane == 0) {
    wbest[wave] = best;
    wbest_i[wave] = best_i;
  }
  __syncthreads();
  if (t == 0) {
    float v = wbest[0];
    int i = wbest_i[0];
#pragma unroll
    for (int w = 1; w < kLmWaves; ++w)
      if (ranks_above(wbest[w], wbest_i[w], v, i)) {
        v = wbest[w];
        i = wbest_i[w];
      }
    a.part_val[blockIdx.x] = v;
    a.part_idx[blockIdx.x] = i;
  }
}

// One workgroup: the best of the `blocks` partials under ranks_above (a strict
// total order, so the result does not depend on the merge order) -> *prediction.
__global__ __launch_bounds__(256) void lm_head_merge_kernel(const float* part_val, const int* part_idx, int blocks,
                                                            long long* prediction) {
  merge_argmax_partials(part_val, part_idx, blocks, prediction);
}

template <int DT, int NC>
bool lm_dispatch(int nc, const LmHeadArgs& a, hipStream_t s) {
  if constexpr (NC > kLmMaxChunks) {
    return false;
  } else {
    if (nc != NC) return lm_dispatch<DT, NC + 1>(nc, a, s);
    if (a.norm_w)
      hipLaunchKernelGGL((lm_head_argmax_kernel<DT, NC, true, kLmRowsInFlight>), dim3(a.blocks), dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((lm_head_argmax_kernel<DT, NC, false, kLmRowsInFlight>), dim3(a.blocks), dim3(256), 0, s,
                         a);
    return true;
  }
}

bool launch_lm_head_partials(int dt, const LmHeadArgs& a, hipStream_t s) {
  if (a.K % 512 != 0) return false;
  if (dt == kBF16) return lm_dispatch<kBF16, 1>(a.K / 512, a, s);
  if (dt == kF16) return lm_dispatch<kF16, 1>(a.K / 512, a, s);
  return false;
}

void launch_lm_head_merge(const LmHeadArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(lm_head_merge_kernel, dim3(1), dim3(256), 0, s, a.part_val, a.part_idx, a.blocks,
                     a.prediction);
}

bool launch_lm_head_argmax(int dt, const LmHeadArgs& a, hipStream_t s) {
  if (!launch_lm_head_partials(dt, a, s)) return false;
  launch_lm_head_merge(a, s);
  return true;
}

}  // namespace fx
