// W3 g128 planar GEMV for gfx950 on the matrix cores: codes are dequantized in
// registers into bf16 MFMA operands and multiplied against exact bf16
// activations with fp32 accumulation.
//
// Why not table lookups: a 256-entry activation table indexed by weight bytes
// makes every lookup a data-dependent LDS read, and on gfx950 those serialise
// on LDS banks (measured ~17 cycles per wave-wide lookup), which caps the
// table kernel far below HBM speed.  Here each weight costs ~1.3 VALU ops and
// the multiply-accumulate runs on MFMA.
//
// Operand encoding (v_mfma_f32_16x16x32_bf16; lane l holds A[l%16][8(l/16)+j],
// B[8(l/16)+j][l%16], D[4(l/16)+j][l%16]):
// * A (weights): per 32-column word w of a plane row, the three plane words
//   P0, P1, ~P2 are merged into four nibble-packed words T_s (s = 0..3) whose
//   nibble n holds the unsigned code q of sorted column 32w + 4n + s.  Masking
//   T_s with 0x000F000F / 0x00F000F0 (and the same after >> 8) yields bf16
//   pairs whose bit pattern is q or 16q: exact bf16 subnormals q * 2^-133 and
//   q * 2^-129.  Slot j of the 8-element operand holds nibble n_j =
//   {0,4,2,6,1,5,3,7}[j], weighted 1 (j < 4) or 16 (j >= 4).
// * B (activations): x * 2^E_m / weight_j, exact in the activation's own type
//   (power-of-two scale), E_m chosen per activation row from max|x| so products
//   are normal fp32.  fp16 activations use the fp16 MFMA with fp16 subnormal
//   codes (q * 2^-24) the same way.
// * Columns: one MFMA chain covers 4 groups at once; k-block b of the
//   instruction carries group 4i+b and column c = b + 4m only sees k-block b,
//   so D[row][b + 4m] is the group's dot product for activation row m.
// y[m,o] = sum_g s[g,o] * (D * 2^(133-E_m) - z[g,o] * sum_{k in g} x[m,k]).
//
// x is first packed by w3_xprep_kernel into the B layout ([G][16 steps][MB][8]
// bf16), its per-group sums and the 2^(133-E_m) factors; the GEMV workgroup
// copies its K slice of that into LDS.  K is split across the waves of a
// workgroup (reduced through LDS) and optionally across workgroups (fp32
// partials reduced by w3_finish_kernel, stream-ordered, no device-scope fences).
#pragma once
#include "common.h"

namespace fx {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMfmaMaxRows = 4;  // activation rows per launch (columns b + 4m)

// The A operand's bit pattern q (or 16q) is a subnormal of the operand type:
// q * 2^-133 in bf16, q * 2^-24 in fp16.
template <int XDT>
constexpr int subnormal_exponent() { return XDT == kBF16 ? 133 : 24; }

// Exponent offset E so that max|x| * 2^E sits near 2^100 (bf16) or 2^14 (fp16):
// B stays finite in its type and the products with the subnormal codes are
// normal fp32 numbers.
template <int XDT>
__device__ __forceinline__ int choose_exponent(float max_abs) {
  if (!(max_abs > 0.f)) return 0;
  int e;
  frexpf(max_abs, &e);  // max_abs in [2^(e-1), 2^e)
  return (XDT == kBF16 ? 100 : 14) - e;
}

// x [MB, K] -> xs bf16 [G][16][MB][8], sx f32 [G][MB], fe int [MB] (= 133 - E_m).
// One workgroup of 256 threads per activation row m.
template <int XDT>
__global__ __launch_bounds__(256) void w3_xprep_kernel(const uint16_t* __restrict__ x,
                                                       const int16_t* __restrict__ perm,
                                                       uint16_t* __restrict__ xs,
                                                       float* __restrict__ sx,
                                                       int* __restrict__ fe, int K, int MB) {
  __shared__ float wmax[4];
  __shared__ float half_sum[2][4];
  const int m = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const uint16_t* xr = x + size_t(m) * K;

  float local = 0.f;
  for (int k = t; k < K; k += 256) local = fmaxf(local, fabsf(to_f32<XDT>(xr[k])));
  local = wave_max(local);
  if (lane == 0) wmax[wave] = local;
  __syncthreads();
  const float mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const int E = choose_exponent<XDT>(mx);
  if (t == 0) fe[m] = subnormal_exponent<XDT>() - E;

  // sorted position k = 256 i + t; a group (128 positions) is two waves
  for (int base = 0; base < K; base += 256) {
    const int k = base + t;
    float v = 0.f;
    if (k < K) {
      v = to_f32<XDT>(xr[perm ? int(perm[k]) : k]);
      const int g = k >> 7, kl = k & 127;
      const int w = kl >> 5, n = (kl & 31) >> 2, s = kl & 3;
      const int step = 4 * w + s;
      // nibble n -> slot j: even n -> j = n/2 mapped {0,4,2,6}->{0,1,2,3}; odd -> {1,5,3,7}->{4,5,6,7}
      const int j = (n & 1) ? (4 + ((n >> 2) & 1) + ((n >> 1) & 1) * 2)
                            : (((n >> 2) & 1) + ((n >> 1) & 1) * 2);
      // exact: power-of-two scaling of a bf16/fp16 value (ldexp handles the range)
      const float scaled = ldexpf(v, (n & 1) ? E - 4 : E);
      xs[((size_t(g) * 16 + step) * MB + m) * 8 + j] = from_f32<XDT>(scaled);
    }
    const float part = wave_sum(v);
    if (lane == 0) half_sum[wave >> 1][wave & 1] = part;
    __syncthreads();
    if (t < 2) {
      const int g = (base >> 7) + t;
      if (g * 128 < K) sx[size_t(g) * MB + m] = half_sum[t][0] + half_sum[t][1];
    }
    __syncthreads();
  }
}

// Build the four bf16x8 A operands of one plane word (32 columns, steps s = 0..3).
__device__ __forceinline__ void dequant_word(unsigned p0, unsigned p1, unsigned p2, u32x4_t a[4]) {
  const unsigned M = 0x11111111u;
  const unsigned q2 = ~p2;  // stored plane 2 is inverted
  unsigned tw[4];
  tw[0] = (p0 & M) | ((p1 << 1) & (M << 1)) | ((q2 << 2) & (M << 2));
  tw[1] = ((p0 >> 1) & M) | (p1 & (M << 1)) | ((q2 << 1) & (M << 2));
  tw[2] = ((p0 >> 2) & M) | ((p1 >> 1) & (M << 1)) | (q2 & (M << 2));
  tw[3] = ((p0 >> 3) & M) | ((p1 >> 2) & (M << 1)) | ((q2 >> 1) & (M << 2));
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const unsigned t = tw[s], th = t >> 8;
    a[s].x = t & 0x000F000Fu;
    a[s].y = th & 0x000F000Fu;
    a[s].z = t & 0x00F000F0u;
    a[s].w = th & 0x00F000F0u;
  }
}

template <int SDT>
__device__ __forceinline__ float scale_at(const uint16_t* scales, size_t idx) {
  return to_f32<SDT>(scales[idx]);
}

// grid (ceil(O / (16*TR)), splits); block NW*64.  Workgroup: rows
// [16*TR*bx, +16*TR), groups [gps*split, +gps) with gps a multiple of 4.
template <int NW, int TR, int MB, int XDT, int SDT>
__global__ __launch_bounds__(NW * 64) void w3_mfma_kernel(
    const uint8_t* __restrict__ planes, const uint16_t* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const uint16_t* __restrict__ xs,
    const float* __restrict__ sx, const int* __restrict__ fe, float* __restrict__ partial,
    uint16_t* __restrict__ out, int O, int G, int gps) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int split = blockIdx.y;
  const int g0 = split * gps;
  const int g1 = min(G, g0 + gps);
  const int ng = g1 - g0;
  const int nbatch = (ng + 3) >> 2;
  const int row0 = blockIdx.x * (16 * TR);

  // LDS: [ng][16][MB] 16-byte B chunks, then a zero chunk, then sums, then the reduction buffer.
  u32x4_t* xs_lds = reinterpret_cast<u32x4_t*>(smem);
  const int nchunk = ng * 16 * MB;
  u32x4_t* zero_chunk = xs_lds + nchunk;
  float* sx_lds = reinterpret_cast<float*>(zero_chunk + 1);
  float* red = sx_lds + ((ng * MB + 3) & ~3);

  const u32x4_t* xs_g = reinterpret_cast<const u32x4_t*>(xs) + size_t(g0) * 16 * MB;
  for (int i = t; i < nchunk; i += NW * 64) xs_lds[i] = xs_g[i];
  if (t == 0) *zero_chunk = u32x4_t{0u, 0u, 0u, 0u};
  for (int i = t; i < ng * MB; i += NW * 64) sx_lds[i] = sx[size_t(g0) * MB + i];
  int fev[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) fev[m] = fe[m];
  __syncthreads();

  const int r = lane & 15;        // A role: row within tile
  const int kb = lane >> 4;       // A role: k-block = group slot; D role: row block
  const int c = lane & 15;        // B / D role: column
  const int cslot = c & 3, cm = c >> 2;
  const bool b_active = (cslot == kb) && (cm < MB);

  float acc[TR][4];
#pragma unroll
  for (int tr = 0; tr < TR; ++tr)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[tr][j] = 0.f;

  for (int batch = wave; batch < nbatch; batch += NW) {
    const int gb = g0 + 4 * batch;
    const int ga = gb + kb;  // this lane's group for the A operand
#pragma unroll
    for (int tr = 0; tr < TR; ++tr) {
      const int row = row0 + 16 * tr + r;
      uint4 w[3];
      if (row < O && ga < g1) {
#pragma unroll
        for (int p = 0; p < 3; ++p)
          w[p] = *reinterpret_cast<const uint4*>(planes + ((size_t(ga) * 3 + p) * O + row) * 16);
      } else {
        w[0] = make_uint4(0u, 0u, 0u, 0u);
        w[1] = make_uint4(0u, 0u, 0u, 0u);
        w[2] = make_uint4(~0u, ~0u, ~0u, ~0u);  // inverted plane: all-ones encodes q = 0
      }
      // epilogue operands for this lane's D rows (4 kb + j) and column group gb + cslot
      const int ge = gb + cslot;
      const int erow = row0 + 16 * tr + 4 * kb;
      float se[4], ze[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool ok = (erow + j < O) && (ge < g1) && (cm < MB);
        se[j] = ok ? scale_at<SDT>(scales, size_t(ge) * O + erow + j) : 0.f;
        ze[j] = ok ? (zeros ? float(zeros[size_t(ge) * O + erow + j]) : 4.f) : 0.f;
      }

      f32x4_t d = {0.f, 0.f, 0.f, 0.f};
      const int gl = ga - g0;  // local group of the B chunk this lane supplies
      const u32x4_t* bsrc = b_active && ga < g1 ? xs_lds + (size_t(gl) * 16) * MB + cm : zero_chunk;
      const int bstride = (b_active && ga < g1) ? MB : 0;
      const unsigned* w0 = reinterpret_cast<const unsigned*>(&w[0]);
      const unsigned* w1 = reinterpret_cast<const unsigned*>(&w[1]);
      const unsigned* w2 = reinterpret_cast<const unsigned*>(&w[2]);
#pragma unroll
      for (int word = 0; word < 4; ++word) {
        u32x4_t a[4];
        dequant_word(w0[word], w1[word], w2[word], a);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const u32x4_t b = bsrc[(4 * word + s) * bstride];
          if constexpr (XDT == kBF16)
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a[s]),
                                                        __builtin_bit_cast(bf16x8_t, b), d, 0, 0, 0);
          else
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a[s]),
                                                       __builtin_bit_cast(f16x8_t, b), d, 0, 0, 0);
        }
      }
      if (cm < MB && ge < g1) {
        const int f = fev[cm];
        const float sxv = sx_lds[(ge - g0) * MB + cm];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[tr][j] += se[j] * (ldexpf(d[j], f) - ze[j] * sxv);
      }
    }
  }

  // sum the four group slots of each activation row (lanes c = 4m .. 4m+3)
#pragma unroll
  for (int tr = 0; tr < TR; ++tr)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v = acc[tr][j];
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      acc[tr][j] = v;
    }
  // cross-wave reduction: red[wave][tr][row 0..15][m]
  if (cslot == 0 && cm < MB) {
#pragma unroll
    for (int tr = 0; tr < TR; ++tr)
#pragma unroll
      for (int j = 0; j < 4; ++j) red[((wave * TR + tr) * 16 + 4 * kb + j) * MB + cm] = acc[tr][j];
  }
  __syncthreads();
  for (int i = t; i < TR * 16 * MB; i += NW * 64) {
    float total = 0.f;
#pragma unroll
    for (int wv = 0; wv < NW; ++wv) total += red[wv * TR * 16 * MB + i];
    const int m = i % MB;
    const int row = row0 + i / MB;
    if (row < O) {
      if (partial)
        partial[(size_t(split) * MB + m) * O + row] = total;
      else
        out[size_t(m) * O + row] = from_f32<XDT>(total);
    }
  }
}

}  // namespace fx
