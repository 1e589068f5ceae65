// W3 g128 planar GEMV for gfx950, activation lookup tables in LDS.
//
// Payload (the reference's planar layout, gptq_deployment.py:199-227):
//   planes  uint8 [G,3,O,16]  bit p of the codes of sorted columns 128g+8c+j of
//                             row o is bit j of planes[g,p,o,c]; plane 2 inverted
//   scales  bf16|fp16 [G,O]
//   zeros   uint8 [G,O] or null (null: zero = 4, the reference's fixed point)
//   perm    int16 [K] or null (sorted column s reads x[perm[s]])
// y[m,o] = sum_g s[g,o] * sum_{k in g} (q[k,o] - z[g,o]) * x[m, perm[k]]
//
// Work split: a 256-thread workgroup owns 256*RPT consecutive output rows and
// one contiguous range of groups (a K split).  Per group it builds, for each of
// the M activation rows, 16 unsigned 256-entry fp32 subset-sum tables (one per
// 8-column chunk; reference csrc/lut8_unsigned.cuh:13-27 computes the same
// table values) and each thread evaluates its rows with 48 table reads per
// group: a0 + 2 a1 - 4 a2 + (4 - z) * sum(x), times the scale.
// K splits are reduced inside the same launch: every workgroup writes its fp32
// partial rows, and the last workgroup of a row tile to arrive (device-scope
// counter) sums the partials in split order and writes the output, so the
// result does not depend on arrival order.
#include "common.h"

namespace fx {

constexpr int kLutThreads = 256;

enum : int { kModeDirect = 0, kModePartial = 1, kModeFused = 2 };

template <int SDT>
__device__ __forceinline__ float load_scale(const uint16_t* scales, size_t index) {
  return to_f32<SDT>(scales[index]);
}

// One byte of a 128-bit plane row, as a float index into a 256-entry table.
__device__ __forceinline__ unsigned plane_byte(const uint4& w, int c) {
  const unsigned word = (c < 4) ? w.x : (c < 8) ? w.y : (c < 12) ? w.z : w.w;
  return (word >> (8 * (c & 3))) & 0xffu;
}

template <int M, int RPT, int XDT, int SDT, bool DECODED>
__global__ __launch_bounds__(kLutThreads) void w3_lut_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ planes,
    const uint16_t* __restrict__ scales, const uint8_t* __restrict__ zeros,
    const int16_t* __restrict__ perm, float* __restrict__ partial,
    unsigned* __restrict__ counters, uint16_t* __restrict__ out, int O, int G,
    int gps, int splits, int mode) {
  __shared__ float lut[M][16][256];
  __shared__ float chunk_sum[M][16];
  __shared__ int last_flag;

  const int t = threadIdx.x;
  const int K = G * 128;
  const int row0 = int(blockIdx.x) * (kLutThreads * RPT);
  const int split = int(blockIdx.y);
  const int g_begin = split * gps;
  const int g_end = min(G, g_begin + gps);

  // table builder role: table (chunk) = t / 16, entries 16*part .. 16*part+15
  const int table = t >> 4;
  const int part = t & 15;

  float acc[M][RPT];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RPT; ++r) acc[m][r] = 0.f;

  for (int g = g_begin; g < g_end; ++g) {
    // Issue this group's plane loads first so they are in flight while the
    // tables are built.
    uint4 w[RPT][3];
    float scale[RPT];
    float zshift[RPT];
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      const int o = row0 + r * kLutThreads + t;
      if (o < O) {
#pragma unroll
        for (int p = 0; p < 3; ++p)
          w[r][p] = *reinterpret_cast<const uint4*>(planes + ((size_t(g) * 3 + p) * O + o) * 16);
        scale[r] = load_scale<SDT>(scales, size_t(g) * O + o);
        zshift[r] = zeros ? float(4 - int(zeros[size_t(g) * O + o])) : 0.f;
      } else {
#pragma unroll
        for (int p = 0; p < 3; ++p) w[r][p] = make_uint4(0u, 0u, 0u, 0u);
        scale[r] = 0.f;
        zshift[r] = 0.f;
      }
    }

    // Build the M x 16 tables of this group.
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int k = g * 128 + table * 8 + j;
        const int src = perm ? int(perm[k]) : k;
        v[j] = to_f32<XDT>(x[size_t(m) * K + src]);
      }
      float low[16];
      low[0] = 0.f;
      low[1] = v[0];
      low[2] = v[1];
      low[3] = v[0] + v[1];
#pragma unroll
      for (int i = 0; i < 4; ++i) low[4 + i] = low[i] + v[2];
#pragma unroll
      for (int i = 0; i < 8; ++i) low[8 + i] = low[i] + v[3];
      float base = 0.f;
      if (part & 1) base += v[4];
      if (part & 2) base += v[5];
      if (part & 4) base += v[6];
      if (part & 8) base += v[7];
      float4* dst = reinterpret_cast<float4*>(&lut[m][table][part * 16]);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        dst[q] = make_float4(base + low[4 * q], base + low[4 * q + 1], base + low[4 * q + 2],
                             base + low[4 * q + 3]);
      if (part == 15) chunk_sum[m][table] = base + low[15];
    }
    __syncthreads();

    float group_sum[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < 16; ++c) s += chunk_sum[m][c];
      group_sum[m] = s;
    }

#pragma unroll
    for (int r = 0; r < RPT; ++r) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, corr = 0.f;
#pragma unroll
        for (int c = 0; c < 16; ++c) {
          const unsigned b0 = plane_byte(w[r][0], c);
          const unsigned b1 = plane_byte(w[r][1], c);
          const unsigned b2 = plane_byte(w[r][2], c);
          a0 += lut[m][c][b0];
          a1 += lut[m][c][b1];
          a2 += lut[m][c][b2];
          if constexpr (DECODED) {
            // signed code +3 is q=7 (stored bits 1,1,0); -3 is q=1 (1,0,1)
            const unsigned plus = b0 & b1 & (~b2 & 0xffu);
            const unsigned minus = b0 & (~b1 & 0xffu) & b2;
            corr += lut[m][c][plus] - lut[m][c][minus];
          }
        }
        float dot = (a0 + 2.f * a1) - 4.f * a2;
        dot += zshift[r] * group_sum[m];
        float value = dot * scale[r];
        if constexpr (DECODED) {
          const float three = 3.f * scale[r];
          value += corr * (round_to<kBF16>(three) - three);
        }
        acc[m][r] += value;
      }
    }
    __syncthreads();  // readers done before the next group's tables overwrite
  }

  if (mode == kModeDirect) {
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      const int o = row0 + r * kLutThreads + t;
      if (o < O)
#pragma unroll
        for (int m = 0; m < M; ++m) out[size_t(m) * O + o] = from_f32<XDT>(acc[m][r]);
    }
    return;
  }

#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int o = row0 + r * kLutThreads + t;
    if (o < O)
#pragma unroll
      for (int m = 0; m < M; ++m) partial[(size_t(split) * M + m) * O + o] = acc[m][r];
  }
  if (mode == kModePartial) return;

  // Fused reduction: publish this split, count arrivals per row tile.
  __threadfence();
  __syncthreads();
  if (t == 0) {
    const unsigned previous = atomicAdd(&counters[blockIdx.x], 1u);
    last_flag = (previous == unsigned(splits - 1)) ? 1 : 0;
  }
  __syncthreads();
  if (!last_flag) return;
  __threadfence();
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int o = row0 + r * kLutThreads + t;
    if (o < O) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float total = 0.f;
        for (int s = 0; s < splits; ++s)
          total += __builtin_nontemporal_load(&partial[(size_t(s) * M + m) * O + o]);
        out[size_t(m) * O + o] = from_f32<XDT>(total);
      }
    }
  }
  if (t == 0) counters[blockIdx.x] = 0u;  // ready for the next launch
}

// out[m,o] = sum over splits of partial[s,m,o], sequential in s
// (reference csrc/w3_lut.cu:141-150).
template <int XDT>
__global__ __launch_bounds__(256) void w3_finish_kernel(const float* __restrict__ partial,
                                                        uint16_t* __restrict__ out, int MO,
                                                        int splits) {
  const int i = int(blockIdx.x) * 256 + threadIdx.x;
  if (i >= MO) return;
  float total = 0.f;
  for (int s = 0; s < splits; ++s) total += partial[size_t(s) * MO + i];
  out[i] = from_f32<XDT>(total);
}

// Dequantize to a dense [O,K] weight with the reference's rounding points
// (restore_planar_w3, gptq_deployment.py:247-260): round_scale_dtype(s*(q-z)),
// then round to the weight dtype.  One thread per (group, row).
template <int SDT, int WDT>
__global__ __launch_bounds__(256) void w3_restore_kernel(
    const uint8_t* __restrict__ planes, const uint16_t* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const int16_t* __restrict__ perm,
    uint16_t* __restrict__ weight, int O, int G) {
  const int idx = int(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= O * G) return;
  const int g = idx / O, o = idx % O;
  const int K = G * 128;
  uint4 w[3];
#pragma unroll
  for (int p = 0; p < 3; ++p)
    w[p] = *reinterpret_cast<const uint4*>(planes + ((size_t(g) * 3 + p) * O + o) * 16);
  const float s = to_f32<SDT>(scales[size_t(g) * O + o]);
  const int z = zeros ? int(zeros[size_t(g) * O + o]) : 4;
  for (int c = 0; c < 16; ++c) {
    const unsigned b0 = plane_byte(w[0], c), b1 = plane_byte(w[1], c), b2 = plane_byte(w[2], c);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int q = int((b0 >> j) & 1u) | (int((b1 >> j) & 1u) << 1) | ((1 - int((b2 >> j) & 1u)) << 2);
      const float product = round_to<SDT>(s * float(q - z));
      const int sorted = g * 128 + c * 8 + j;
      const int col = perm ? int(perm[sorted]) : sorted;
      weight[size_t(o) * K + col] = from_f32<WDT>(product);
    }
  }
}

}  // namespace fx
