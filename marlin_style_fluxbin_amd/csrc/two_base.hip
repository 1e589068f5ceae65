// Two-base binary-basis GEMV for gfx950 on the integer matrix cores (batch 1).
//
// Rank-one format (two_base_launch.h): each weight is one sign bit in each of
// two bases, so the dot products are  S_b[o] = sum_{k: bit_b[o,k] = 1} u[k]  with
// u = t_c * x, and  B_b . u = 2 S_b - U  where U = sum_k u[k].
//
// Why matrix cores and not the reference's 256-entry subset-sum tables: a table
// lookup is a data-dependent LDS read per 8 weights per row, and those serialise
// on LDS banks.  Here one bitwise AND turns four sign bits into four int8 operand
// elements of v_mfma_i32_16x16x64_i8 (A and B element e of lane block l/16 are
// multiplied together; D[4(l/16)+j][l%16] lands in lane l), and the
// multiply-accumulate is exact integer arithmetic.
//
// * Sign layout: the 16 bytes of a (group, row, base) hold column k of the group
//   at bit k >> 4 of byte k & 15, so  word_v & (0x01010101 << i)  (word v = bytes
//   4v .. 4v+3) is the int8 quadruple bit * 2^i of columns 16 i + 4 v .. +3 (i = 7
//   reads as -128 * bit).  Bit position i of the four words is one A operand
//   covering the 16 consecutive columns 16 i .. 16 i + 15 of one group per k-block.
// * Activations: u is rounded to a 16-bit fixed-point integer v = rint(u 2^F), F
//   per batch from max|u| over its 512 columns so |v| <= 2^14, and split into int8
//   digits v = 256 hi + lo, lo = the signed low byte.  Rounding is one FMA with a
//   magic constant (the integer lands in the low mantissa bits), the digits are
//   bytes 0 and 1 of that word.
// * Columns: the operand of bit position i is non-zero only in D columns 2i (hi)
//   and 2i+1 (lo), so one int32 accumulator per base gathers all eight positions
//   and both digits of a batch; column c is worth 2^-i (x256 for hi), negated for
//   i = 7, and 2^-F of its batch.  Zero lanes of an operand read a shared zero
//   block (LDS broadcast).
// * U is the exact integer sum of the same v, so 2 S - U is the signed sum of
//   exactly the values the matrix cores used.
//
// Work split: a workgroup owns NT 16-row tiles and a K range of gps groups
// (batches of four groups, 512 columns).  Wave w stages batches w, w + NW, ...
// into LDS (one 8-column unit per lane, no workgroup-wide reduction); after one
// barrier wave w multiplies tile w % NT against batches w / NT, + NK, ... with PD
// batches of sign loads in flight, issued before anything waits, so HBM latency
// hides behind the staging.  The NK partial sums of a tile meet in LDS (second
// barrier); K splits over workgroups go through fp32 partials summed by the
// finish kernel.  Workgroups are few and tall on purpose: the dispatcher starts
// roughly one workgroup per 2.7 ns, so a grid of ~one workgroup per CU starts in
// under a microsecond.
#include "common.h"
#include "two_base_launch.h"

namespace fx {

typedef int tb_i32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTbMaxUnits = kRankOneMaxUnits;
// v + 128 + 1.5 * 2^23: the sum's low 16 bits are v + 128 for |v| < 2^22
constexpr float kTbMagic = 12583040.0f;

template <int XDT>
__device__ __forceinline__ void load_products(u32x4_t xv, u32x4_t tv, float u[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const unsigned xw = xv[j >> 1] >> (16 * (j & 1));
    const unsigned tw = tv[j >> 1] >> (16 * (j & 1));
    u[j] = to_f32<XDT>(uint16_t(xw)) * f16_bits_to_f32(uint16_t(tw));
  }
}

template <int NT, int NK, int PD, int XDT>
__global__ __launch_bounds__(NT * NK * 64) void rank_one_kernel(RankOneArgs a) {
  constexpr int NW = NT * NK;
  // dynamic LDS, per batch: digit operands [position][k-block][hi, lo] (16 B
  // each, 1 KB) and the batch's activations in staging order (1 KB)
  extern __shared__ u32x4_t tb_dyn[];
  __shared__ u32x4_t zero16;
  __shared__ float bscale[kRankOneMaxBatches];  // 2^-F of each batch
  __shared__ float bsum[kRankOneMaxBatches];    // U of each batch (real units)
  __shared__ float red[NK][16 * NT][2];
  __shared__ float sal_sum[16 * NT];
  // one scalar-load round for every argument, before any branch
  asm volatile("" ::"s"(a.x), "s"(a.planes), "s"(a.coef), "s"(a.srow), "s"(a.tcol), "s"(a.sal), "s"(a.sal_idx),
               "s"(a.partial), "s"(a.out), "s"(a.O), "s"(a.G), "s"(a.S), "s"(a.gps), "s"(a.row_blocks));
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int O = a.O, G = a.G, K = G * 128;
  const int split = blockIdx.y;
  const int row0 = xcd_local_index8(blockIdx.x, a.row_blocks) * (16 * NT);
  const int g0 = split * a.gps;
  const int g1 = min(G, g0 + a.gps);
  const int nbatch = (g1 - g0 + 3) >> 2;
  u32x4_t* slots = tb_dyn;                        // [batch][8][4][2]
  u32x4_t* xs = tb_dyn + size_t(a.gps / 4) * 64;  // [batch][64 units]

  const auto rp = buffer_resource(a.planes, size_t(G) * O * 32);
  const auto rx = buffer_resource(a.x, size_t(K) * 2);
  const auto rt = buffer_resource(a.tcol, size_t(K) * 2);
  const int r = lane & 15;   // A role: row in tile; staging role: 8-column chunk
  const int kb = lane >> 4;  // k-block = group slot; D role: row quad
  const int c = lane & 15;   // B / D role: column = 2 * position + digit

  // ---- loads, in the order they are consumed (vector loads return in order)
  // 1. staging: wave w stages batches w, w + NW, ...; lane (kb, r) takes columns
  //    8r .. 8r+7 of group 4 batch + kb
  const int staged = wave < nbatch ? (nbatch - wave + NW - 1) / NW : 0;
  u32x4_t sx[kTbMaxUnits], st[kTbMaxUnits];
#pragma unroll
  for (int q = 0; q < kTbMaxUnits; ++q) {
    const int g = g0 + 4 * (wave + q * NW) + kb;
    const bool real = q < staged && g < g1;
    const int col = g * 128 + 8 * r;
    sx[q] = load_b128(rx, real ? col * 2 : kOutOfRange, 0);
    st[q] = load_b128(rt, real ? col * 2 : kOutOfRange, 0);
  }
  // 2. salient columns: each K split adds those inside its range, 16 lanes per
  //    row taking columns j0 and j0 + 16; x[idx] is read from LDS after staging.
  //    Raw bits only (no arithmetic on loaded values before every load is issued:
  //    a use here would make the wave wait for all earlier loads).
  const bool salient = a.S > 0;
  const int srl = t >> 4, sj0 = t & 15;
  const int srow_s = row0 + srl;
  const bool sal_row = salient && srl < 16 * NT && srow_s < O;
  const auto rsi = buffer_resource(a.sal_idx, size_t(a.S) * 4);
  const auto rsv = buffer_resource(a.sal, size_t(O) * a.S * 2);
  unsigned sidx_raw[2], sval_raw[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int j = sj0 + 16 * q;
    const bool ok = sal_row && j < a.S;
    sidx_raw[q] = __builtin_amdgcn_raw_buffer_load_b32(rsi, ok ? j * 4 : kOutOfRange, 0, 0);
    sval_raw[q] = __builtin_amdgcn_raw_buffer_load_b16(rsv, ok ? (srow_s * a.S + j) * 2 : kOutOfRange, 0, 0);
  }
  // 3. sign planes: wave (tile, kpart) takes batches kpart, kpart + NK, ..., the
  //    first PD of them in flight before anything waits
  const int tile = wave % NT, kpart = wave / NT;
  const int prow = row0 + 16 * tile + r;
  const int mine = kpart < nbatch ? (nbatch - kpart + NK - 1) / NK : 0;
  auto issue = [&](int i, u32x4_t w[2]) __attribute__((always_inline)) {
    const int g = g0 + 4 * (kpart + i * NK) + kb;
    const int poff = (g * O + prow) * 32;  // past the end -> zeros
    w[0] = load_b128_stream(rp, poff, 0);
    w[1] = load_b128_stream(rp, poff + 16, 0);
  };
  u32x4_t ring[PD][2];
#pragma unroll
  for (int i = 0; i < PD; ++i)
    if (i < mine) issue(i, ring[i]);
  // 4. per-row coefficients of the output rows this thread finishes (raw bits)
  const int orow_f = row0 + t;
  const bool finisher = t < 16 * NT && orow_f < O;
  const auto rc = buffer_resource(a.coef, size_t(O) * 4);
  const auto rs = buffer_resource(a.srow, size_t(O) * 2);
  const unsigned a1_raw = __builtin_amdgcn_raw_buffer_load_b16(rc, finisher ? orow_f * 2 : kOutOfRange, 0, 0);
  const unsigned a2_raw = __builtin_amdgcn_raw_buffer_load_b16(rc, finisher ? (O + orow_f) * 2 : kOutOfRange, 0, 0);
  const unsigned sr_raw = __builtin_amdgcn_raw_buffer_load_b16(rs, finisher ? orow_f * 2 : kOutOfRange, 0, 0);

  // ---- staging: per batch (one wave) max|u| -> F, digits and activations into LDS, U
  if (t == 0) zero16 = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
  for (int q = 0; q < kTbMaxUnits; ++q) {
    if (q < staged) {
      const int b = wave + q * NW;
      xs[b * 64 + lane] = sx[q];
      float u[8];
      load_products<XDT>(sx[q], st[q], u);
      float mx = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(u[j]));
      mx = row16_max(mx);
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      int F = 0;
      if (mx > 0.f) {
        int e;
        frexpf(mx, &e);
        F = min(14 - e, 126);  // max|u| 2^F in [2^13, 2^14) unless max|u| < 2^-112
      }
      const float scale = ldexpf(1.f, F);
      unsigned w[8];
      int vsum = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        w[j] = __float_as_uint(fmaf(u[j], scale, kTbMagic));  // low 16 bits: v + 128
        vsum += int(int16_t(uint16_t(w[j]))) - 128;
      }
      // byte 0 of w is lo + 128 (mod 256), byte 1 is hi; gather them four at a time
      const unsigned p01 = __builtin_amdgcn_perm(w[1], w[0], 0x05010400u);
      const unsigned p23 = __builtin_amdgcn_perm(w[3], w[2], 0x05010400u);
      const unsigned p45 = __builtin_amdgcn_perm(w[5], w[4], 0x05010400u);
      const unsigned p67 = __builtin_amdgcn_perm(w[7], w[6], 0x05010400u);
      const unsigned lo0 = __builtin_amdgcn_perm(p23, p01, 0x05040100u) ^ 0x80808080u;
      const unsigned lo1 = __builtin_amdgcn_perm(p67, p45, 0x05040100u) ^ 0x80808080u;
      const unsigned hi0 = __builtin_amdgcn_perm(p23, p01, 0x07060302u);
      const unsigned hi1 = __builtin_amdgcn_perm(p67, p45, 0x07060302u);
      uint2* dst = reinterpret_cast<uint2*>(slots + ((b * 8 + (r >> 1)) * 4 + kb) * 2) + (r & 1);
      dst[0] = uint2{hi0, hi1};
      dst[2] = uint2{lo0, lo1};  // the lo operand is the next 16 bytes
      // |partial sums| < 2^24: exact in fp32
      float vs = row16_sum(float(vsum));
      vs += __shfl_xor(vs, 16, 64);
      vs += __shfl_xor(vs, 32, 64);
      if (lane == 0) {
        bscale[b] = ldexpf(1.f, -F);
        bsum[b] = ldexpf(vs, -F);
      }
    }
  }
  __syncthreads();

  // salient dot products: range column cc is element cc & 7 of staging unit cc >> 3
  if (salient && srl < 16 * NT) {
    const uint16_t* xs16 = reinterpret_cast<const uint16_t*>(xs);
    float sv = 0.f;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int cc = int(sidx_raw[q]) - g0 * 128;
      if (sj0 + 16 * q < a.S && cc >= 0 && cc < nbatch * 512)
        sv = fmaf(bf16_bits_to_f32(uint16_t(sval_raw[q])), to_f32<XDT>(xs16[cc]), sv);
    }
    sv = row16_sum(sv);
    if (sj0 == 0) sal_sum[srl] = sv;
  }

  // ---- main loop: eight bit positions per batch, one B read serving both bases
  const float colw = ldexpf((c & 1) ? 1.f : 256.f, -(c >> 1)) * ((c >> 1) == 7 ? -1.f : 1.f);
  float acc[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  const u32x4_t* zp = &zero16;
  for (int base = 0; base < mine; base += PD) {
#pragma unroll
    for (int i = 0; i < PD; ++i) {
      if (base + i < mine) {
        const int b = kpart + (base + i) * NK;
        const u32x4_t* own = slots + ((b * 8 + (c >> 1)) * 4 + kb) * 2 + (c & 1);
        const u32x4_t w0 = ring[i][0], w1 = ring[i][1];
        if (base + i + PD < mine) issue(base + i + PD, ring[i]);
        tb_i32x4_t d0 = {0, 0, 0, 0}, d1 = {0, 0, 0, 0};
#pragma unroll
        for (int p = 0; p < 8; ++p) {
          const u32x4_t bop = *((c >> 1) == p ? own : zp);
          const unsigned m = 0x01010101u << p;
          const u32x4_t a0{w0.x & m, w0.y & m, w0.z & m, w0.w & m};
          const u32x4_t a1v{w1.x & m, w1.y & m, w1.z & m, w1.w & m};
          d0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(tb_i32x4_t, a0),
                                                    __builtin_bit_cast(tb_i32x4_t, bop), d0, 0, 0, 0);
          d1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(tb_i32x4_t, a1v),
                                                    __builtin_bit_cast(tb_i32x4_t, bop), d1, 0, 0, 0);
        }
        const float wsc = colw * bscale[b];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[0][j] = fmaf(float(d0[j]), wsc, acc[0][j]);
          acc[1][j] = fmaf(float(d1[j]), wsc, acc[1][j]);
        }
      }
    }
  }

  // ---- S_b for rows 4 kb + j: sum over the 16 lanes (columns) of the quad
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float s = row16_sum(acc[b][j]);
      if (c == 0) red[kpart][16 * tile + 4 * kb + j][b] = s;
    }
  __syncthreads();
  if (finisher) {
    const float a1 = f16_bits_to_f32(uint16_t(a1_raw));
    const float a2 = f16_bits_to_f32(uint16_t(a2_raw));
    const float sr = f16_bits_to_f32(uint16_t(sr_raw));
    float s0 = 0.f, s1 = 0.f, uu = 0.f;
#pragma unroll
    for (int q = 0; q < NK; ++q) {
      s0 += red[q][t][0];
      s1 += red[q][t][1];
    }
    for (int b = 0; b < nbatch; ++b) uu += bsum[b];
    float y = sr * (a1 * (2.f * s0 - uu) + a2 * (2.f * s1 - uu));
    if (salient) y += sal_sum[t];
    if (a.partial)
      a.partial[size_t(split) * O + orow_f] = y;
    else
      a.out[orow_f] = from_f32<XDT>(y);
  }
}

template <int NT, int NK, int PD>
bool rank_one_for_dtype(int xdt, const RankOneArgs& a, dim3 grid, hipStream_t s) {
  const size_t lds = rank_one_lds_bytes(a.gps);
  if (xdt == kBF16)
    hipLaunchKernelGGL((rank_one_kernel<NT, NK, PD, kBF16>), grid, dim3(NT * NK * 64), lds, s, a);
  else if (xdt == kF16)
    hipLaunchKernelGGL((rank_one_kernel<NT, NK, PD, kF16>), grid, dim3(NT * NK * 64), lds, s, a);
  else
    return false;
  return true;
}

bool dispatch_rank_one(int xdt, int tiles, int kparts, int pd, const RankOneArgs& a, dim3 grid,
                       hipStream_t s) {
#define FX_RANK_ONE_CASE(NT, NK, PD) \
  if (tiles == NT && kparts == NK && pd == PD) return rank_one_for_dtype<NT, NK, PD>(xdt, a, grid, s);
  FX_RANK_ONE_CASE(1, 4, 1)
  FX_RANK_ONE_CASE(1, 4, 2)
  FX_RANK_ONE_CASE(1, 8, 1)
  FX_RANK_ONE_CASE(1, 8, 2)
  FX_RANK_ONE_CASE(1, 8, 3)
  FX_RANK_ONE_CASE(2, 4, 2)
  FX_RANK_ONE_CASE(2, 8, 2)
  FX_RANK_ONE_CASE(3, 4, 1)
  FX_RANK_ONE_CASE(3, 4, 2)
  FX_RANK_ONE_CASE(4, 4, 2)
#undef FX_RANK_ONE_CASE
  return false;
}

}  // namespace fx
