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
//   T_s with 0x00070007 / 0x00700070 (and the same after >> 8) yields bf16
//   pairs whose bit pattern is q or 16q: exact bf16 subnormals q * 2^-133 and
//   q * 2^-129.  Slot j of the 8-element operand holds nibble n_j =
//   {0,4,2,6,1,5,3,7}[j], weighted 1 (j < 4) or 16 (j >= 4).
// * B (activations): x * 2^E / weight_j, exact in the activation's own type
//   (power-of-two scale), E chosen per (group, activation row) from max|x| so
//   products are normal fp32.  fp16 activations use the fp16 MFMA with fp16 subnormal
//   codes (q * 2^-24) the same way.
// * Columns: one MFMA chain covers 4 groups at once; k-block b of the
//   instruction carries group 4i+b and column c = b + 4m only sees k-block b,
//   so D[row][b + 4m] is the group's dot product for activation row m.
// y[m,o] = sum_g s[g,o] * (D * 2^(133-E) - z[g,o] * sum_{k in g} x[m,k]).
//
// x is first packed by w3_xprep_kernel (one wave per group, one pass) into the
// B layout ([G][16 steps][MB][8]), per-group sums and exponents.  Each wave
// stages one batch's B slice in its own LDS region (no workgroup barrier) and
// prefetches the next batch.  K is split across the waves of a workgroup
// (reduced through LDS) and optionally across workgroups (fp32 partials reduced
// by w3_finish_kernel, stream-ordered, no device-scope fences).
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

// x [MB, K] -> xs [Gp][16][MB][8] (B operands in the activation's type),
// sx f32 [Gp][MB] (sum of the group's x), fe int [Gp][MB] (subnormal exponent - E),
// with Gp = G rounded up to a multiple of 4 (the padding groups are zero).
// One wave per (group, activation row); E is chosen per group from its max|x|.
template <int XDT>
__global__ __launch_bounds__(256) void w3_xprep_kernel(const uint16_t* __restrict__ x,
                                                       const int16_t* __restrict__ perm,
                                                       uint16_t* __restrict__ xs,
                                                       float* __restrict__ sx,
                                                       int* __restrict__ fe, int K, int MB) {
  const int lane = threadIdx.x & 63;
  const int g = blockIdx.x * 4 + (threadIdx.x >> 6);  // groups padded to a multiple of 4
  const int m = blockIdx.y;
  const bool real = g * 128 < K;                       // padding groups get zeros
  const uint16_t* xr = x + size_t(m) * K;
  float v[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int k = g * 128 + h * 64 + lane;
    v[h] = real ? to_f32<XDT>(xr[perm ? int(perm[k]) : k]) : 0.f;
  }
  const float mx = wave_max(fmaxf(fabsf(v[0]), fabsf(v[1])));
  const float total = wave_sum(v[0] + v[1]);
  const int E = choose_exponent<XDT>(mx);
  if (lane == 0) {
    sx[size_t(g) * MB + m] = total;
    fe[size_t(g) * MB + m] = subnormal_exponent<XDT>() - E;
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int kl = h * 64 + lane;
    const int w = kl >> 5, n = (kl & 31) >> 2, s = kl & 3;
    const int step = 4 * w + s;
    // nibble n -> operand slot: {0,4,2,6} -> 0..3 (weight 1), {1,5,3,7} -> 4..7 (weight 16)
    const int j = (n & 1) ? (4 + ((n >> 2) & 1) + ((n >> 1) & 1) * 2)
                          : (((n >> 2) & 1) + ((n >> 1) & 1) * 2);
    // exact: power-of-two scaling of a bf16/fp16 value (ldexp handles the range)
    const float scaled = ldexpf(v[h], (n & 1) ? E - 4 : E);
    xs[((size_t(g) * 16 + step) * MB + m) * 8 + j] = from_f32<XDT>(scaled);
  }
}

// Build the four 8-element A operands of one plane word (32 columns, steps s = 0..3).
// T_s keeps the code of column 4n + s in bits 4n..4n+2 of nibble n (bit 4n+3 is
// don't-care, masked off below): bitfield inserts take bit 4n from P0, 4n+1
// from P1 and the remaining bits from the un-inverted plane 2.
__device__ __forceinline__ unsigned bitfield_insert(unsigned mask, unsigned a, unsigned b) {
  return (a & mask) | (b & ~mask);  // v_bfi_b32
}

__device__ __forceinline__ void dequant_word(unsigned p0, unsigned p1, unsigned p2, u32x4_t a[4]) {
  const unsigned M0 = 0x11111111u, M1 = 0x22222222u;
  const unsigned q2 = ~p2;  // stored plane 2 is inverted
  unsigned tw[4];
  tw[0] = bitfield_insert(M0, p0, bitfield_insert(M1, p1 << 1, q2 << 2));
  tw[1] = bitfield_insert(M0, p0 >> 1, bitfield_insert(M1, p1, q2 << 1));
  tw[2] = bitfield_insert(M0, p0 >> 2, bitfield_insert(M1, p1 >> 1, q2));
  tw[3] = bitfield_insert(M0, p0 >> 3, bitfield_insert(M1, p1 >> 2, q2 >> 1));
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const unsigned t = tw[s], th = t >> 8;
    a[s].x = t & 0x00070007u;
    a[s].y = th & 0x00070007u;
    a[s].z = t & 0x00700070u;
    a[s].w = th & 0x00700070u;
  }
}

template <int SDT>
__device__ __forceinline__ float scale_at(const uint16_t* scales, size_t idx) {
  return to_f32<SDT>(scales[idx]);
}

// Buffer resource over [base, base + bytes): loads at offsets past the end
// return zero instead of touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_resource(const void* base, size_t bytes) {
  const int records = bytes > 0x7fffffffu ? 0x7fffffff : int(bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), short(0), records, 0x00020000);
}

__device__ __forceinline__ u32x4_t load_b128(__amdgpu_buffer_rsrc_t r, int offset, int soffset) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, offset, soffset, 0));
}

// Everything one wave loads for one batch, kept as raw bits: this lane's plane
// row, its share of the batch's B slice, and the epilogue's scales, zero-points,
// sums and exponents.  Nothing loaded is used before consume(), so the
// prefetched batches stay in flight.
template <int MB>
struct BatchLoads {
  u32x4_t w[3];
  u32x4_t b[MB];
  unsigned s[4];   // scales of rows erow..erow+3 (vector path: s[0], s[1] hold pairs)
  unsigned z[4];   // zero-points (vector path: z[0] holds four)
  float sxv;
  int fev;
};

// grid (ceil(O / 16), splits); block NW*64.  Workgroup: rows [16 bx, +16),
// groups [gps*split, +gps) with gps a multiple of 4.  Wave w takes batches
// w, w + NW, ... of its split and keeps PD of them in flight: their loads are
// issued before the oldest one is dequantized and multiplied.  Rows past O and
// groups past G need no masking of the A operand: padded groups have B = 0 and
// rows past O get scale 0 and are never stored.
template <int NW, int PD, int MB, int XDT, int SDT>
__global__ __launch_bounds__(NW * 64) void w3_mfma_kernel(
    const uint8_t* __restrict__ planes, const uint16_t* __restrict__ scales,
    const uint8_t* __restrict__ zeros, const uint16_t* __restrict__ xs,
    const float* __restrict__ sx, const int* __restrict__ fe, float* __restrict__ partial,
    uint16_t* __restrict__ out, int O, int G, int gps) {
  __shared__ u32x4_t bstage[NW][64 * MB + 1];  // per-wave B slice of one batch + zero chunk
  __shared__ float red[NW][16 * MB];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int split = blockIdx.y;
  const int g0 = split * gps;
  const int g1 = min(G, g0 + gps);
  const int nbatch = (g1 - g0 + 3) >> 2;
  const int row0 = blockIdx.x * 16;
  const int Gp = (G + 3) & ~3;
  // four consecutive scales / zero-points of a row block are one aligned load
  const bool vec = (O & 3) == 0;
  const bool has_zeros = zeros != nullptr;

  const auto rp = buffer_resource(planes, size_t(G) * 3 * O * 16);
  const auto rs = buffer_resource(scales, size_t(G) * O * 2);
  const auto rz = buffer_resource(has_zeros ? (const void*)zeros : (const void*)scales,
                                  has_zeros ? size_t(G) * O : 0);
  const auto rx = buffer_resource(xs, size_t(Gp) * 256 * MB);
  const auto rsx = buffer_resource(sx, size_t(Gp) * MB * 4);
  const auto rfe = buffer_resource(fe, size_t(Gp) * MB * 4);

  const int r = lane & 15;    // A role: row within tile
  const int kb = lane >> 4;   // A role: k-block = group slot; D role: row block
  const int c = lane & 15;    // B / D role: column
  const int cslot = c & 3, cm = c >> 2;
  const bool b_active = (cslot == kb) && (cm < MB);
  u32x4_t* my_stage = bstage[wave];
  if (lane == 0) my_stage[64 * MB] = u32x4_t{0u, 0u, 0u, 0u};
  const u32x4_t* bsrc = b_active ? my_stage + kb * 16 * MB + cm : my_stage + 64 * MB;
  const int bstride = b_active ? MB : 0;
  const int row = row0 + r;
  const int erow = row0 + 4 * kb;
  const int plane_stride = O * 16;
  const int cmc = cm < MB ? cm : 0;

  auto issue = [&](int batch, BatchLoads<MB>& L) {
    const int gb = g0 + 4 * batch;
    const int poff = ((gb + kb) * 3 * O + row) * 16;  // past the end -> zeros
    L.w[0] = load_b128(rp, poff, 0);
    L.w[1] = load_b128(rp, poff, plane_stride);
    L.w[2] = load_b128(rp, poff, 2 * plane_stride);
#pragma unroll
    for (int i = 0; i < MB; ++i) L.b[i] = load_b128(rx, ((gb * 16 * MB) + i * 64 + lane) * 16, 0);
    const int ge = gb + cslot;
    const int eoff = ge * O + erow;
    if (vec) {
      const uint2 s4 = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, eoff * 2, 0, 0));
      L.s[0] = s4.x;
      L.s[1] = s4.y;
      L.z[0] = __builtin_amdgcn_raw_buffer_load_b32(rz, eoff, 0, 0);
    } else {  // odd O (tests, tiny layers): element loads
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        L.s[j] = __builtin_amdgcn_raw_buffer_load_b16(rs, (eoff + j) * 2, 0, 0);
        L.z[j] = __builtin_amdgcn_raw_buffer_load_b8(rz, eoff + j, 0, 0);
      }
    }
    L.sxv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsx, (ge * MB + cmc) * 4, 0, 0));
    L.fev = int(__builtin_amdgcn_raw_buffer_load_b32(rfe, (ge * MB + cmc) * 4, 0, 0));
  };

  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  int cur_batch = 0;
  auto consume = [&](const BatchLoads<MB>& L) {
#pragma unroll
    for (int i = 0; i < MB; ++i) my_stage[i * 64 + lane] = L.b[i];
    f32x4_t d = {0.f, 0.f, 0.f, 0.f};
    const unsigned w0[4] = {L.w[0].x, L.w[0].y, L.w[0].z, L.w[0].w};
    const unsigned w1[4] = {L.w[1].x, L.w[1].y, L.w[1].z, L.w[1].w};
    const unsigned w2[4] = {L.w[2].x, L.w[2].y, L.w[2].z, L.w[2].w};
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
    const int ge = g0 + 4 * cur_batch + cslot;
    const bool e_ok = (cm < MB) && (ge < g1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const unsigned sb = vec ? ((j & 1) ? (L.s[j >> 1] >> 16) : (L.s[j >> 1] & 0xffffu)) : L.s[j];
      const unsigned zb = !has_zeros ? 4u : (vec ? (L.z[0] >> (8 * j)) & 0xffu : L.z[j]);
      const bool ok = e_ok && (erow + j < O);
      const float se = ok ? to_f32<SDT>(uint16_t(sb)) : 0.f;
      acc[j] += se * (ldexpf(d[j], L.fev) - float(zb) * L.sxv);
    }
  };

  // my batches: wave, wave + NW, ...; the i-th is batch wave + i*NW
  const int mine = wave < nbatch ? (nbatch - wave + NW - 1) / NW : 0;
  BatchLoads<MB> ring[PD];
#pragma unroll
  for (int i = 0; i < PD; ++i)
    if (i < mine) issue(wave + i * NW, ring[i]);
  for (int base = 0; base < mine; base += PD) {
#pragma unroll
    for (int i = 0; i < PD; ++i) {
      if (base + i < mine) {
        cur_batch = wave + (base + i) * NW;
        consume(ring[i]);
        if (base + i + PD < mine) issue(wave + (base + i + PD) * NW, ring[i]);
      }
    }
  }

  // sum the four group slots of each activation row (lanes c = 4m .. 4m+3)
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v = acc[j];
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    acc[j] = v;
  }
  if (cslot == 0 && cm < MB) {
#pragma unroll
    for (int j = 0; j < 4; ++j) red[wave][(4 * kb + j) * MB + cm] = acc[j];
  }
  __syncthreads();
  for (int i = t; i < 16 * MB; i += NW * 64) {
    float total = 0.f;
#pragma unroll
    for (int wv = 0; wv < NW; ++wv) total += red[wv][i];
    const int m = i % MB;
    const int orow = row0 + i / MB;
    if (orow < O) {
      if (partial)
        partial[(size_t(split) * MB + m) * O + orow] = total;
      else
        out[size_t(m) * O + orow] = from_f32<XDT>(total);
    }
  }
}

}  // namespace fx
