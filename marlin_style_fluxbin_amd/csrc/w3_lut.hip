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
// With one K split the workgroup writes the output; otherwise it writes fp32
// partial rows partial[split, m, o] that w3_finish_kernel sums in split order
// (the reference's inline_main + finish contract, csrc/w3_lut.cu:141-189).
#include "common.h"

namespace fx {

constexpr int kLutThreads = 256;

enum : int { kModeDirect = 0, kModePartial = 1 };

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
    uint16_t* __restrict__ out, int O, int G, int gps, int mode) {
  __shared__ float lut[M][16][256];
  __shared__ float chunk_sum[M][16];

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
      // decoded_bf16: byte masks of the columns whose signed code is +3 / -3,
      // i.e. q = z + 3 / q = z - 3.  Stored bits of code q are (q0, q1, 1 - q2);
      // a column matches when every stored bit equals the code's bit, so the
      // mask is AND_p (byte_p XOR flip_p) with flip_p = 0xff where the code's
      // stored bit is 0.
      unsigned plus_flip[3] = {0u, 0u, 0u}, minus_flip[3] = {0u, 0u, 0u};
      unsigned plus_keep = 0u, minus_keep = 0u;
      if constexpr (DECODED) {
        const int z = 4 - int(zshift[r]);
        const int plus_code = z + 3, minus_code = z - 3;
        plus_keep = (plus_code <= 7) ? 0xffu : 0u;
        minus_keep = (minus_code >= 0) ? 0xffu : 0u;
#pragma unroll
        for (int p = 0; p < 3; ++p) {
          const int pb = (plus_code >> p) & 1, mb = (minus_code >> p) & 1;
          const int pstored = (p == 2) ? 1 - pb : pb;
          const int mstored = (p == 2) ? 1 - mb : mb;
          plus_flip[p] = pstored ? 0u : 0xffu;
          minus_flip[p] = mstored ? 0u : 0xffu;
        }
      }
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
            const unsigned plus =
                (b0 ^ plus_flip[0]) & (b1 ^ plus_flip[1]) & (b2 ^ plus_flip[2]) & plus_keep;
            const unsigned minus =
                (b0 ^ minus_flip[0]) & (b1 ^ minus_flip[1]) & (b2 ^ minus_flip[2]) & minus_keep;
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
#pragma unroll 8
  for (int s = 0; s < splits; ++s) total += partial[size_t(s) * MO + i];
  out[i] = from_f32<XDT>(total);
}

// Dequantize to a dense [O,K] weight with the reference's rounding points
// (restore_planar_w3, gptq_deployment.py:247-260): round_scale_dtype(s*(q-z)),
// then round to the weight dtype.  Sorted column s = 128g+8c+j of row o lands
// at weight[o, perm[s]].
//
// The eight values of byte c of a row's three plane vectors (sorted columns
// 128g+8c .. 128g+8c+7), two per word in column order.
template <int SDT, int WDT>
__device__ __forceinline__ void restore_eight(unsigned b0, unsigned b1, unsigned b2, float s, int z,
                                              unsigned (&pair)[4]) {
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    unsigned two = 0;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int b = j + e;
      const int q = int((b0 >> b) & 1u) | (int((b1 >> b) & 1u) << 1) | ((1 - int((b2 >> b) & 1u)) << 2);
      two |= unsigned(from_f32<WDT>(round_to<SDT>(s * float(q - z)))) << (16 * e);
    }
    pair[j >> 1] = two;
  }
}

// Identity order.  A workgroup owns 16 rows and kRestoreGroups consecutive
// groups (consecutive workgroups: the next groups of the same rows); per group
// lane c of a row's 16 lanes expands byte c of the row's plane vectors and
// writes its eight columns as one 16-byte store (element stores when the
// weight is not 16-byte aligned), so the 16 lanes of a row store the group's
// 256 bytes of that row together.
constexpr int kRestoreGroups = 2;

template <int SDT, int WDT>
__global__ __launch_bounds__(256) void w3_restore_kernel(
    const uint8_t* __restrict__ planes, const uint16_t* __restrict__ scales,
    const uint8_t* __restrict__ zeros, uint16_t* __restrict__ weight, int O, int G, int weight16) {
  const unsigned group_blocks = unsigned((G + kRestoreGroups - 1) / kRestoreGroups);
  const int g0 = int(blockIdx.x % group_blocks) * kRestoreGroups;
  const int o = int(blockIdx.x / group_blocks) * 16 + int(threadIdx.x >> 4);
  const int c = int(threadIdx.x & 15u);
  if (o >= O) return;
  const size_t plane = size_t(O) * 16;
  uint16_t* row = weight + size_t(o) * G * 128;
#pragma unroll
  for (int i = 0; i < kRestoreGroups; ++i) {
    const int g = g0 + i;
    if (g >= G) break;
    const size_t at = size_t(g) * 3 * plane + size_t(o) * 16 + c;
    unsigned pair[4];
    restore_eight<SDT, WDT>(planes[at], planes[at + plane], planes[at + 2 * plane],
                            to_f32<SDT>(scales[size_t(g) * O + o]),
                            zeros ? int(zeros[size_t(g) * O + o]) : 4, pair);
    uint16_t* dst = row + g * 128 + c * 8;
    if (weight16) {
      *reinterpret_cast<uint4*>(dst) = make_uint4(pair[0], pair[1], pair[2], pair[3]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) dst[j] = uint16_t(pair[j >> 1] >> (16 * (j & 1)));
    }
  }
}

// With a column permutation.  A workgroup stages `rows_per_block` whole rows
// in LDS (rows_per_block * K * 2 bytes, zeroed first), scatters each expanded
// value to its permuted column there, and then writes the rows out in order
// with 16-byte stores, so a scattered permutation costs LDS scatter and not
// scattered HBM stores.  Entries outside [0, K) are skipped; a column no entry
// names stays zero.  The eight entries of a lane are one 16-byte load when perm
// is 16-byte aligned.
constexpr int kRestoreStageThreads = 512;
constexpr int kRestoreStageBytes = 32768;  // rows_per_block = max(1, this / (2K))

template <int SDT, int WDT>
__global__ __launch_bounds__(kRestoreStageThreads) void w3_restore_permuted_kernel(
    const uint8_t* __restrict__ planes, const uint16_t* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const int16_t* __restrict__ perm,
    uint16_t* __restrict__ weight, int O, int G, int rows_per_block, int weight16, int perm16) {
  extern __shared__ uint4 stage_vec[];
  uint16_t* stage = reinterpret_cast<uint16_t*>(stage_vec);
  const int K = G * 128;
  const int o0 = int(blockIdx.x) * rows_per_block;
  const int rows = min(rows_per_block, O - o0);
  const int vecs = rows * K / 8;
  for (int i = threadIdx.x; i < vecs; i += kRestoreStageThreads) stage_vec[i] = make_uint4(0, 0, 0, 0);
  __syncthreads();
  const size_t plane = size_t(O) * 16;
  // items (g, r, c): 16 consecutive lanes read one row's 16 plane bytes
  const int items = G * rows * 16;
  for (int it = threadIdx.x; it < items; it += kRestoreStageThreads) {
    const int c = it & 15;
    const int r = (it >> 4) % rows;
    const int g = (it >> 4) / rows;
    const int o = o0 + r;
    const size_t at = size_t(g) * 3 * plane + size_t(o) * 16 + c;
    unsigned pair[4];
    restore_eight<SDT, WDT>(planes[at], planes[at + plane], planes[at + 2 * plane],
                            to_f32<SDT>(scales[size_t(g) * O + o]),
                            zeros ? int(zeros[size_t(g) * O + o]) : 4, pair);
    const int sorted = g * 128 + c * 8;
    unsigned cols[4];  // perm[sorted .. sorted+7], two per word
    if (perm16) {
      const uint4 p = *reinterpret_cast<const uint4*>(perm + sorted);
      cols[0] = p.x, cols[1] = p.y, cols[2] = p.z, cols[3] = p.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        cols[j] = unsigned(uint16_t(perm[sorted + 2 * j])) | (unsigned(uint16_t(perm[sorted + 2 * j + 1])) << 16);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int col = int(int16_t(cols[j >> 1] >> (16 * (j & 1))));
      if (unsigned(col) < unsigned(K)) stage[r * K + col] = uint16_t(pair[j >> 1] >> (16 * (j & 1)));
    }
  }
  __syncthreads();
  uint16_t* dst = weight + size_t(o0) * K;
  if (weight16) {
    uint4* dst_vec = reinterpret_cast<uint4*>(dst);
    for (int i = threadIdx.x; i < vecs; i += kRestoreStageThreads) dst_vec[i] = stage_vec[i];
  } else {
    for (int i = threadIdx.x; i < rows * K; i += kRestoreStageThreads) dst[i] = stage[i];
  }
}

}  // namespace fx
