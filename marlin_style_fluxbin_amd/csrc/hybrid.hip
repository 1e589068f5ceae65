// Hybrid g128/s8 two-base GEMV for gfx950 on the integer matrix cores (batch 1),
// over the reference's planar deployment layout (deployment.py:59-103).
//
// Per 128-column group g and base b the weight is sign * rows[g,o,b] * cols[g,k,b],
// plus an 8-column two-base refinement with its own row and column scales.  As
// in the rank-one kernel (two_base.hip), sign bits become int8 MFMA operands and
// activations become 16-bit fixed-point integers split into two int8 digits, but
// every group keeps its own accumulator column because its row scale differs:
//
// * A (main): word_v >> i & 0x01010101 holds, as int8 0/1, the bits of columns
//   8 (4v + q) + i for bytes q = 0..3 of word v (the layout's bit j of byte c is
//   column 8c + j), so bit position i of a 16-byte plane row is one operand with
//   element e covering column 8e + i.  A (refinement): the 8 bits of the
//   refinement byte spread to bytes by a multiply ((n * 0x204081) & 0x01010101).
// * B: D column c < 8 is (group slot c >> 1, digit c & 1) of the main product,
//   c >= 8 the same for the refinement; an operand is non-zero only in the lanes
//   of its own column and k-block (the others read a shared zero block).
// * Activations u_b = x * cols[.., b] are rounded to v = rint(u_b 2^F) with F per
//   (group, base) -- |v| <= 2^14 over the group's 128 columns -- and split into
//   digits 256 hi + lo.  Every D column holds one group, so each column is folded
//   with its own 2^-F: an outlier coarsens only its own group, whose row scale
//   multiplies it anyway.  Per batch the int32 products are folded:
//   acc += rows[g,o,b] (2 S - U_g,b) 2^-F_g,b with S the weighted digit sum and U
//   the exact sum of the same v; the refinement the same with its own scales and
//   exponents.  A refinement index outside [0, 128) makes the output NaN (its U
//   is NaN), as the reference's lookup does.
//
// Several layouts that read the same x (q|k|v, gate|up) can run as one launch:
// their row-side arrays concatenated along O, their column-side arrays (column
// scales, refinement indices and refinement column scales) one per segment; a
// workgroup takes its segment's from the segment table.  Every row is computed
// as in a launch of its own layout.
//
// Work split as in the rank-one kernel: a workgroup owns NT 16-row tiles and a K
// range; wave w stages batches w, w + NW, ... (one 8-column unit per lane and
// base, the refinement columns one per lane); after one barrier wave (tile,
// kpart) multiplies its batches; the K parts meet in LDS.
#include "common.h"
#include "two_base_launch.h"

namespace fx {

typedef int hy_i32x4_t __attribute__((ext_vector_type(4)));

constexpr float kHyMagic = 12583040.0f;  // 1.5 * 2^23 + 128: low 16 bits of the sum are v + 128
constexpr int kHyMaxUnits = 4;           // staged batches per wave
// The K reduction always runs in the order of eight K parts: batch b of a split
// feeds virtual part b % 8, each part accumulates its batches in order, and the
// eight part sums are added in part order.  A plan with NK < 8 waves per tile
// keeps 8 / NK accumulator sets per wave, so every plan (tiles, K parts) with the
// same number of K splits gives the same bits, and a fused q|k|v launch matches
// the separate projections whatever tiling each one picks.  Different K-split
// counts (narrow modules at long K) sum the splits' fp32 partials in another
// order.
constexpr int kHyVirtualParts = 8;

__device__ __forceinline__ int hy_exponent(float max_abs) {
  if (!(max_abs > 0.f)) return 0;
  int e;
  frexpf(max_abs, &e);
  return min(14 - e, 126);  // max_abs * 2^F in [2^13, 2^14) unless max_abs < 2^-112
}

// Refinement byte -> int8 0/1 elements 0..7 (four per word).
__device__ __forceinline__ u32x4_t refine_operand(unsigned byte) {
  return u32x4_t{((byte & 15u) * 0x204081u) & 0x01010101u, (((byte >> 4) & 15u) * 0x204081u) & 0x01010101u,
                 0u, 0u};
}

template <int NT, int NK, int XDT, int PRO>
__global__ __launch_bounds__(NT * NK * 64) void hybrid_kernel(HybridArgs a) {
  constexpr bool NORMIN = PRO == kHyProNorm, SWIGLU = PRO == kHyProSwiglu;
  constexpr int NW = NT * NK;
  extern __shared__ u32x4_t hy_dyn[];
  __shared__ u32x4_t zero16;
  __shared__ float fsc[kHybridMaxBatches][4][2];   // 2^-F per (batch, group slot, base)
  __shared__ float fref[kHybridMaxBatches][4][2];  // the same for the refinement operands
  __shared__ float ug[kHybridMaxBatches][4][2];    // U per (batch, group slot, base)
  __shared__ float vg[kHybridMaxBatches][4][2];    // refinement U per (batch, slot, base)
  __shared__ float red[kHyVirtualParts][16 * NT];
  static_assert(kHyVirtualParts % NK == 0, "K parts must divide the virtual parts");
  constexpr int VS = kHyVirtualParts / NK;  // accumulator sets per wave
  // one scalar-load round for every argument, before any branch
  asm volatile("" ::"s"(a.x), "s"(a.codes), "s"(a.rows), "s"(a.cols), "s"(a.idx), "s"(a.scodes), "s"(a.srows),
               "s"(a.scols), "s"(a.partial), "s"(a.out), "s"(a.O), "s"(a.G), "s"(a.gps), "s"(a.row_blocks),
               "s"(a.nseg));
  asm volatile("" ::"s"(a.seg_start[1]), "s"(a.seg_start[2]), "s"(a.seg_start[3]), "s"(a.seg_cols[1]),
               "s"(a.seg_cols[2]), "s"(a.seg_cols[3]), "s"(a.seg_idx[1]), "s"(a.seg_idx[2]), "s"(a.seg_idx[3]),
               "s"(a.seg_scols[1]), "s"(a.seg_scols[2]), "s"(a.seg_scols[3]));
  const int t = threadIdx.x, lane = t & 63, wave = wave_index();
  const int O = a.O, G = a.G, K = G * 128;
  const int split = blockIdx.y;
  const int row0 = xcd_local_index8(blockIdx.x, a.row_blocks) * (16 * NT);
  // the workgroup's segment: scalar selects over the segment table (no indexing
  // into the argument array, which would be a second scalar load round)
  const float* cols = a.cols;
  const int16_t* idxp = a.idx;
  const float* scols = a.scols;
#pragma unroll
  for (int s = 1; s < kHybridMaxSegments; ++s) {
    if (s < a.nseg && row0 >= a.seg_start[s]) {
      cols = a.seg_cols[s];
      idxp = a.seg_idx[s];
      scols = a.seg_scols[s];
    }
  }
  const int g0 = split * a.gps;
  const int g1 = min(G, g0 + a.gps);
  const int nbatch = (g1 - g0 + 3) >> 2;
  const int maxb = a.gps / 4;
  uint8_t* mslot = reinterpret_cast<uint8_t*>(hy_dyn);          // [batch][base][pos][slot][digit][16]
  uint8_t* rslot = mslot + size_t(maxb) * 2048;                 // [batch][base][slot][digit][16]
  u32x4_t* xs = reinterpret_cast<u32x4_t*>(rslot + size_t(maxb) * 256);  // [batch][64 units]

  const auto rx = buffer_resource(a.x, size_t(SWIGLU ? 2 : 1) * K * 2);
  const auto rcol = buffer_resource(cols, size_t(G) * 128 * 2 * 4);
  const auto ridx = buffer_resource(idxp, size_t(G) * 8 * 2);
  const auto rscol = buffer_resource(scols, size_t(G) * 8 * 2 * 4);
  const auto rp = buffer_resource(a.codes, size_t(G) * O * 32);
  const auto rsp = buffer_resource(a.scodes, size_t(G) * O * 2);
  const auto rrow = buffer_resource(a.rows, size_t(G) * O * 2 * 4);
  const auto rsrow = buffer_resource(a.srows, size_t(G) * O * 2 * 4);
  const int r = lane & 15, kb = lane >> 4, c = lane & 15;

  // ---- loads in consumption order (raw bits; nothing waits until all are issued):
  // NORMIN first the tile partials of h (each wave reduces them itself, in a
  // fixed order: lane l adds partials l, l + 64, ..., then the wave total)
  float pp[kMaxNormPartialsPerLane];
  if constexpr (NORMIN) {
    const auto rpp = buffer_resource(a.res.pro_partial, size_t(a.res.pro_n) * 4);
#pragma unroll
    for (int k = 0; k < kMaxNormPartialsPerLane; ++k) {
      const int i = lane + 64 * k;
      pp[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rpp, i < a.res.pro_n ? i * 4 : kOutOfRange, 0, 0));
    }
  }
  const auto rwn = buffer_resource(NORMIN ? (const void*)a.res.pro_weight : (const void*)a.x, NORMIN ? size_t(K) * 2 : 0);
  const int staged = wave < nbatch ? (nbatch - wave + NW - 1) / NW : 0;
  u32x4_t sx[kHyMaxUnits], sc[kHyMaxUnits][4], swn[kHyMaxUnits], sup[kHyMaxUnits];
  unsigned sidx[kHyMaxUnits], sscol[kHyMaxUnits];
#pragma unroll
  for (int q = 0; q < kHyMaxUnits; ++q) {
    const int g = g0 + 4 * (wave + q * NW) + kb;
    const bool real = q < staged && g < g1;
    const int col = g * 128 + 8 * r;
    sx[q] = load_b128(rx, real ? col * 2 : kOutOfRange, 0);
    if constexpr (NORMIN) swn[q] = load_b128(rwn, real ? col * 2 : kOutOfRange, 0);
    if constexpr (SWIGLU) sup[q] = load_b128(rx, real ? (K + col) * 2 : kOutOfRange, 0);
#pragma unroll
    for (int h = 0; h < 4; ++h) sc[q][h] = load_b128(rcol, real ? (col * 2 + 4 * h) * 4 : kOutOfRange, 0);
    sidx[q] = __builtin_amdgcn_raw_buffer_load_b16(ridx, real ? (g * 8 + (r & 7)) * 2 : kOutOfRange, 0, 0);
    sscol[q] = __builtin_amdgcn_raw_buffer_load_b32(rscol, real ? ((g * 8 + (r & 7)) * 2 + (r >> 3)) * 4 : kOutOfRange, 0, 0);
  }
  const int tile = wave % NT, kpart = wave / NT;
  const int prow = row0 + 16 * tile + r;          // A role row
  const int drow = row0 + 16 * tile + 4 * kb;     // D role: rows drow .. drow + 3
  const bool is_ref = c >= 8;
  const int dslot = (c & 7) >> 1, digit = c & 1;
  const int mine = kpart < nbatch ? (nbatch - kpart + NK - 1) / NK : 0;
  u32x4_t w0, w1, rv0, rv1;
  unsigned sb;
  auto issue = [&](int i) __attribute__((always_inline)) {
    const int bt = kpart + i * NK;
    const int g = g0 + 4 * bt + kb;
    const int poff = (g * O + prow) * 32;  // past the end -> zeros
    w0 = load_b128_stream(rp, poff, 0);
    w1 = load_b128_stream(rp, poff + 16, 0);
    sb = __builtin_amdgcn_raw_buffer_load_b16(rsp, (g * O + prow) * 2, 0, 0);
    // row scales of D rows drow .. +3 for this lane's group slot, both bases
    const int gd = g0 + 4 * bt + dslot;
    // the lane picks the refinement or the main row scales: both descriptors
    // stay scalar (one of the two loads out of range returns zeros), where a
    // per-lane choice of descriptor cost a waterfall loop around each load
    const int roff = (gd * O + drow) * 8;
    const int moff = is_ref ? kOutOfRange : roff, soff = is_ref ? roff : kOutOfRange;
    rv0 = load_b128(rrow, moff, 0) | load_b128(rsrow, soff, 0);
    rv1 = load_b128(rrow, moff == kOutOfRange ? kOutOfRange : moff + 16, 0) |
          load_b128(rsrow, soff == kOutOfRange ? kOutOfRange : soff + 16, 0);
  };
  if (mine > 0) issue(0);

  // ---- staging: wave w stages batches w, w + NW, ...
  if (t == 0) zero16 = u32x4_t{0u, 0u, 0u, 0u};
  float norm_inv = 1.f;
  if constexpr (NORMIN) {
    float total = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxNormPartialsPerLane; ++k) total += pp[k];
    norm_inv = rsqrtf(wave_total(total) / float(K) + a.res.pro_eps);
  }
#pragma unroll
  for (int q = 0; q < kHyMaxUnits; ++q) {
    if (q < staged) {
      const int bt = wave + q * NW;
      float xv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) xv[j] = to_f32<XDT>(uint16_t(sx[q][j >> 1] >> (16 * (j & 1))));
      if constexpr (NORMIN || SWIGLU) {  // the activation the GEMV reads, staged for the refinement too
        u32x4_t nb;
#pragma unroll
        for (int j = 0; j < 8; j += 2) {  // element pairs: one packed convert per rounding
          float a, b;
          if constexpr (NORMIN) {  // Qwen3RMSNorm: round(w * round(h * inv))
            a = xv[j] * norm_inv;
            b = xv[j + 1] * norm_inv;
            round_pair<XDT>(a, b);
            a *= to_f32<XDT>(uint16_t(swn[q][j >> 1]));
            b *= to_f32<XDT>(uint16_t(swn[q][j >> 1] >> 16));
          } else {  // Qwen3MLP: round(round(silu(gate)) * up), silu(g) = g / (1 + e^-g)
            a = xv[j] / (1.f + __expf(-xv[j]));
            b = xv[j + 1] / (1.f + __expf(-xv[j + 1]));
            round_pair<XDT>(a, b);
            a *= to_f32<XDT>(uint16_t(sup[q][j >> 1]));
            b *= to_f32<XDT>(uint16_t(sup[q][j >> 1] >> 16));
          }
          nb[j >> 1] = round_pair_bits<XDT>(a, b);
          xv[j] = a;
          xv[j + 1] = b;
        }
        xs[bt * 64 + lane] = nb;
      } else {
        xs[bt * 64 + lane] = sx[q];
      }
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        float u[8], mx = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          // cols[g][8r + j][b]: float 2 j + b of the lane's 16
          u[j] = xv[j] * __uint_as_float(sc[q][(2 * j + b) >> 2][(2 * j + b) & 3]);
          mx = fmaxf(mx, fabsf(u[j]));
        }
        const int F = hy_exponent(row16_max(mx));  // the group's 16 lanes
        const float scale = ldexpf(1.f, F);
        int vsum = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const unsigned wv = __float_as_uint(fmaf(u[j], scale, kHyMagic));  // low 16 bits: v + 128
          vsum += int(int16_t(uint16_t(wv))) - 128;
          // column 8r + j: position j, element r
          uint8_t* dst = mslot + ((((bt * 2 + b) * 8 + j) * 4 + kb) * 2) * 16 + r;
          dst[0] = uint8_t(wv >> 8);          // hi digit
          dst[16] = uint8_t(wv ^ 0x80u);      // lo digit
        }
        const float us = row16_sum(float(vsum));  // group slot kb; |sum| < 2^22: exact
        if (r == 0) {
          ug[bt][kb][b] = ldexpf(us, -F);
          fsc[bt][kb][b] = ldexpf(1.f, -F);
        }
      }
      __builtin_amdgcn_wave_barrier();  // xs of this batch written by this wave
      // refinement: lane (kb, r) takes column idx[g][r & 7] of base r >> 3
      const int j = r & 7, b = r >> 3;
      const int index = int(int16_t(uint16_t(sidx[q])));
      const bool bad_index = index < 0 || index > 127;
      const int cc = index & 127;  // the read stays inside the group; a bad index poisons U below
      const uint16_t* xs16 = reinterpret_cast<const uint16_t*>(xs + bt * 64 + kb * 16);
      const float v = to_f32<XDT>(xs16[cc]) * __uint_as_float(sscol[q]);
      float m8 = fabsf(v);  // max over the 8 lanes of this (group, base)
      m8 = fmaxf(m8, dpp_move<kDppXor1>(m8));
      m8 = fmaxf(m8, dpp_move<kDppXor2>(m8));
      m8 = fmaxf(m8, dpp_move<kDppHalfMirror>(m8));
      const int F = hy_exponent(m8);
      const unsigned wv = __float_as_uint(fmaf(v, ldexpf(1.f, F), kHyMagic));
      uint8_t* dst = rslot + (((bt * 2 + b) * 4 + kb) * 2) * 16 + j;
      dst[0] = uint8_t(wv >> 8);
      dst[16] = uint8_t(wv ^ 0x80u);
      float vs = bad_index ? __builtin_nanf("") : float(int(int16_t(uint16_t(wv))) - 128);
      vs += dpp_move<kDppXor1>(vs);
      vs += dpp_move<kDppXor2>(vs);
      vs += dpp_move<kDppHalfMirror>(vs);  // lanes j and 7 - j: completes the 8-lane sum
      if (j == 0) {
        vg[bt][kb][b] = ldexpf(vs, -F);
        fref[bt][kb][b] = ldexpf(1.f, -F);
      }
    }
  }
  __syncthreads();

  // ---- main loop: eight bit positions + the refinement per batch and base.
  // Batch i of this wave (virtual part kpart + NK (i % VS)) accumulates into
  // acc[0]; with VS > 1 the sets rotate after every batch (register moves), so
  // after `mine` batches set p holds virtual part kpart + NK ((p + mine) % VS).
  float acc[VS][4];
#pragma unroll
  for (int v = 0; v < VS; ++v)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[v][j] = 0.f;
  const u32x4_t* zp = &zero16;
  const bool main_lane = !is_ref && dslot == kb;
  const bool ref_lane = is_ref && dslot == kb;
  const float dw = digit ? 1.f : 256.f;
  for (int i = 0; i < mine; ++i) {
    const int bt = kpart + i * NK;
    const u32x4_t p0 = w0, p1 = w1, r0 = rv0, r1 = rv1;
    const unsigned sbv = sb;
    if (i + 1 < mine) issue(i + 1);
    hy_i32x4_t d0 = {0, 0, 0, 0}, d1 = {0, 0, 0, 0};
#pragma unroll
    for (int pos = 0; pos < 8; ++pos) {
      const u32x4_t* b0p = main_lane ? reinterpret_cast<const u32x4_t*>(mslot + ((((bt * 2 + 0) * 8 + pos) * 4 + kb) * 2 + digit) * 16) : zp;
      const u32x4_t* b1p = main_lane ? reinterpret_cast<const u32x4_t*>(mslot + ((((bt * 2 + 1) * 8 + pos) * 4 + kb) * 2 + digit) * 16) : zp;
      const u32x4_t bop0 = *b0p, bop1 = *b1p;
      const u32x4_t a0{(p0.x >> pos) & 0x01010101u, (p0.y >> pos) & 0x01010101u, (p0.z >> pos) & 0x01010101u,
                       (p0.w >> pos) & 0x01010101u};
      const u32x4_t a1{(p1.x >> pos) & 0x01010101u, (p1.y >> pos) & 0x01010101u, (p1.z >> pos) & 0x01010101u,
                       (p1.w >> pos) & 0x01010101u};
      d0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(hy_i32x4_t, a0), __builtin_bit_cast(hy_i32x4_t, bop0), d0, 0, 0, 0);
      d1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(hy_i32x4_t, a1), __builtin_bit_cast(hy_i32x4_t, bop1), d1, 0, 0, 0);
    }
    {
      const u32x4_t* b0p = ref_lane ? reinterpret_cast<const u32x4_t*>(rslot + (((bt * 2 + 0) * 4 + kb) * 2 + digit) * 16) : zp;
      const u32x4_t* b1p = ref_lane ? reinterpret_cast<const u32x4_t*>(rslot + (((bt * 2 + 1) * 4 + kb) * 2 + digit) * 16) : zp;
      const u32x4_t bop0 = *b0p, bop1 = *b1p;
      d0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(hy_i32x4_t, refine_operand(sbv & 0xffu)),
                                                __builtin_bit_cast(hy_i32x4_t, bop0), d0, 0, 0, 0);
      d1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(hy_i32x4_t, refine_operand((sbv >> 8) & 0xffu)),
                                                __builtin_bit_cast(hy_i32x4_t, bop1), d1, 0, 0, 0);
    }
    // fold: this lane's column is (group slot, digit) of the main or the refinement product
    const float s0 = dw * (is_ref ? fref[bt][dslot][0] : fsc[bt][dslot][0]);
    const float s1 = dw * (is_ref ? fref[bt][dslot][1] : fsc[bt][dslot][1]);
    const float u0 = digit ? 0.f : (is_ref ? vg[bt][dslot][0] : ug[bt][dslot][0]);
    const float u1 = digit ? 0.f : (is_ref ? vg[bt][dslot][1] : ug[bt][dslot][1]);
    // rv: rows drow + j, base b at float 2 j + b
    const float rs[8] = {__uint_as_float(r0.x), __uint_as_float(r0.y), __uint_as_float(r0.z), __uint_as_float(r0.w),
                         __uint_as_float(r1.x), __uint_as_float(r1.y), __uint_as_float(r1.z), __uint_as_float(r1.w)};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[0][j] = fmaf(rs[2 * j], fmaf(2.f * float(d0[j]), s0, -u0), acc[0][j]);
      acc[0][j] = fmaf(rs[2 * j + 1], fmaf(2.f * float(d1[j]), s1, -u1), acc[0][j]);
    }
    if constexpr (VS > 1) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float first = acc[0][j];
#pragma unroll
        for (int v = 0; v + 1 < VS; ++v) acc[v][j] = acc[v + 1][j];
        acc[VS - 1][j] = first;
      }
    }
  }

  // ---- rows 4 kb + j: sum over the 16 columns of the quad, then over the
  // virtual K parts in order
#pragma unroll
  for (int v = 0; v < VS; ++v) {
    const int part = kpart + NK * ((v + mine) % VS);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float s = row16_sum(acc[v][j]);
      if (c == 0) red[part][16 * tile + 4 * kb + j] = s;
    }
  }
  __syncthreads();
  const int orow = row0 + t;
  if (a.res.ep_residual) {
    // one K split: out = round(residual + round(y)) for the workgroup's rows and,
    // per 16-row tile (16 consecutive lanes), the sum of out^2 (DPP row sum)
    if (t < (16 * NT + 63) / 64 * 64) {
      float h2 = 0.f;
      if (t < 16 * NT && orow < O) {
        float y = 0.f;
#pragma unroll
        for (int q = 0; q < kHyVirtualParts; ++q) y += red[q][t];
        const float h = round_to<XDT>(to_f32<XDT>(a.res.ep_residual[orow]) + round_to<XDT>(y));
        a.out[orow] = from_f32<XDT>(h);
        h2 = h * h;
      }
      h2 = row16_sum(h2);
      if ((t & 15) == 0 && t < 16 * NT && orow < O) a.res.ep_partial[orow / 16] = h2;
    }
    return;
  }
  if (t < 16 * NT && orow < O) {
    float y = 0.f;
#pragma unroll
    for (int q = 0; q < kHyVirtualParts; ++q) y += red[q][t];
    if (a.partial)
      a.partial[size_t(split) * O + orow] = y;
    else
      a.out[orow] = from_f32<XDT>(y);
  }
}

// Dynamic LDS beyond the default 64 KB must be allowed per kernel, once.
template <int NT, int NK, int XDT, int PRO>
bool hybrid_launch(const HybridArgs& a, dim3 grid, hipStream_t s) {
  static const bool allowed =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&hybrid_kernel<NT, NK, XDT, PRO>),
                          hipFuncAttributeMaxDynamicSharedMemorySize,
                          int(hybrid_lds_bytes(4 * kHybridMaxBatches))) == hipSuccess;
  if (!allowed) return false;
  hipLaunchKernelGGL((hybrid_kernel<NT, NK, XDT, PRO>), grid, dim3(NT * NK * 64), hybrid_lds_bytes(a.gps), s, a);
  return true;
}

template <int NT, int NK, int XDT>
bool hybrid_for_prologue(int pro, const HybridArgs& a, dim3 grid, hipStream_t s) {
  if (pro == kHyProPlain) return hybrid_launch<NT, NK, XDT, kHyProPlain>(a, grid, s);
  if (pro == kHyProNorm) return hybrid_launch<NT, NK, XDT, kHyProNorm>(a, grid, s);
  if (pro == kHyProSwiglu) return hybrid_launch<NT, NK, XDT, kHyProSwiglu>(a, grid, s);
  return false;
}

template <int NT, int NK>
bool hybrid_for_dtype(int xdt, int pro, const HybridArgs& a, dim3 grid, hipStream_t s) {
  if (xdt == kBF16) return hybrid_for_prologue<NT, NK, kBF16>(pro, a, grid, s);
  if (xdt == kF16) return hybrid_for_prologue<NT, NK, kF16>(pro, a, grid, s);
  return false;
}

bool dispatch_hybrid(int xdt, int tiles, int kparts, int pro, const HybridArgs& a, dim3 grid, hipStream_t s) {
  if (tiles == 1 && kparts == 4) return hybrid_for_dtype<1, 4>(xdt, pro, a, grid, s);
  if (tiles == 1 && kparts == 8) return hybrid_for_dtype<1, 8>(xdt, pro, a, grid, s);
  if (tiles == 2 && kparts == 4) return hybrid_for_dtype<2, 4>(xdt, pro, a, grid, s);
  if (tiles == 3 && kparts == 4) return hybrid_for_dtype<3, 4>(xdt, pro, a, grid, s);
  if (tiles == 4 && kparts == 2) return hybrid_for_dtype<4, 2>(xdt, pro, a, grid, s);
  if (tiles == 5 && kparts == 2) return hybrid_for_dtype<5, 2>(xdt, pro, a, grid, s);
  if (tiles == 6 && kparts == 2) return hybrid_for_dtype<6, 2>(xdt, pro, a, grid, s);
  return false;
}

}  // namespace fx
