// W3 g128 planar GEMV for gfx950 on the matrix cores: codes are dequantized in
// registers into bf16 MFMA operands and multiplied against exact bf16
// activations with fp32 accumulation.  One launch per GEMV (plus a finish
// launch when K is split over workgroups).
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
//   products are normal fp32.  fp16 activations use the fp16 MFMA with fp16
//   subnormal codes (q * 2^-24) the same way.
// * Columns: one MFMA chain covers 4 groups at once; k-block b of the
//   instruction carries group 4i+b and column c = b + 4m only sees k-block b,
//   so D[row][b + 4m] is the group's dot product for activation row m.  Eight
//   activation rows run two such chains on the same dequantized A operands
//   (rows 4h .. 4h+3 in chain h), so the weights are read once for all eight.
// y[m,o] = sum_g s[g,o] * (D * 2^(133-E) - z[g,o] * sum_{k in g} x[m,k]).
//
// Each wave builds the B operands of its own batch from x: the 16 lanes of
// k-block b each load 8 consecutive activations of group 4i+b, reduce max|x|
// and sum(x) over their DPP row, scale, and scatter the values into the wave's
// LDS stage in operand order (no workgroup barrier; x is L2-resident).  A wave
// applies one batch's operands to RT 16-row tiles.  Wave w of a workgroup
// takes batches w, w + NW, ... of its K split and keeps PD of them in flight.
// K splits across waves are reduced through LDS; across workgroups through
// fp32 partials summed by w3_finish_kernel (stream-ordered, no device-scope
// fences).
//
// Issue order per batch: activations, then the plane rows (non-temporal: read
// once), then scales and zero-points.  A wave's loads complete in issue order,
// so staging waits only for the L2-resident activations and overlaps the
// weight stream; scheduling barriers keep the compiler from reordering them.
// All kernel arguments are read in one scalar round before any branch.
#pragma once
#include "common.h"
#include "w3_mfma_launch.h"

namespace fx {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMfmaMaxRows = 8;  // activation rows per launch (columns b + 4m of NH = ceil(MB / 4) halves)

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

// Bits of a value that is exactly representable in the activation type (a
// power-of-two multiple of one): bf16 keeps the high half of the fp32 bits.
template <int XDT>
__device__ __forceinline__ uint16_t exact_bits(float v) {
  if constexpr (XDT == kBF16) return uint16_t(__float_as_uint(v) >> 16);
  else return f32_to_f16_bits(v);
}

// Build the four 8-element A operands of one plane word (32 columns, steps s = 0..3).
// T_s keeps the code of column 4n + s in bits 4n..4n+2 of nibble n (bit 4n+3 is
// don't-care, masked off below): bitfield inserts take bit 4n from P0, 4n+1
// from P1 and the remaining bits from the un-inverted plane 2.
__device__ __forceinline__ unsigned bitfield_insert(unsigned mask, unsigned a, unsigned b) {
  return (a & mask) | (b & ~mask);  // v_bfi_b32
}

// T_s from three-input bit operations (v_bitop3_b32, gfx950): u = M1 ? b : ~c
// (table 0xB1, operand order b, c, m: the inversion of stored plane 2 folded in),
// then T = M0 ? a : u (table 0xE4).  The complement of the shifted plane differs
// from the shifted complement only in shifted-in bits, which land in bits the
// masks take from the other planes or in the don't-care bit.  Two instructions
// per T_s where the compiler's own rewrite of the inserts took three to four.
__device__ __forceinline__ unsigned select3(unsigned a, unsigned b, unsigned c, unsigned m0, unsigned m1) {
  return __builtin_amdgcn_bitop3_b32(a, __builtin_amdgcn_bitop3_b32(b, c, m1, 0xB1), m0, 0xE4);
}

__device__ __forceinline__ void dequant_word(unsigned p0, unsigned p1, unsigned p2, u32x4_t a[4]) {
  const unsigned M0 = 0x11111111u, M1 = 0x22222222u;
  unsigned tw[4];
  tw[0] = select3(p0, p1 << 1, p2 << 2, M0, M1);
  tw[1] = select3(p0 >> 1, p1, p2 << 1, M0, M1);
  tw[2] = select3(p0 >> 2, p1 >> 1, p2, M0, M1);
  tw[3] = select3(p0 >> 3, p1 >> 2, p2 >> 1, M0, M1);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const unsigned t = tw[s], th = t >> 8;
    a[s].x = t & 0x00070007u;
    a[s].y = th & 0x00070007u;
    a[s].z = t & 0x00700070u;
    a[s].w = th & 0x00700070u;
  }
}

// Field layout (the bind-time repack of the planes, fx_w3_planes_to_fields): the
// three 32-bit words of a 32-column word hold 10 codes each in 3-bit fields at
// bits 0, 3, 6, 9, 12 of each half, and the last two codes' bits in bits 15 / 31
// of the three words.  Register i of the 16 (step i / 4, component i % 4) takes
// field i % 5 of word i / 5 (i < 15) or the spare bits (i = 15): masking leaves
// the code in mantissa bits 0-2, 3-5 or 6-8 of each fp16 half, i.e. the exact
// fp16 subnormals q * 2^(p - 24) for p = 0, 3, 6; fields 3 and 4 are shifted
// down by 9 first.  One AND per two codes, a shift per word and four operations
// for the spare pair: 24 per 32 codes (against 47 for the planes).
__device__ __forceinline__ void dequant_fields(unsigned w0, unsigned w1, unsigned w2, u32x4_t a[4]) {
  const unsigned M0 = 0x00070007u, M3 = 0x00380038u, M6 = 0x01c001c0u;
  const unsigned h0 = w0 >> 9, h1 = w1 >> 9, h2 = w2 >> 9;
  // the spare pair: bit 0 / 16 from w0, 1 / 17 from w1, 2 / 18 from w2 (two
  // selects, table 0xE4: m ? a : b, over a masked w2 term)
  const unsigned spare = __builtin_amdgcn_bitop3_b32(
      w0 >> 15, __builtin_amdgcn_bitop3_b32(w1 >> 14, (w2 >> 13) & 0x00040004u, 0x00020002u, 0xE4), 0x00010001u,
      0xE4);
  a[0] = u32x4_t{w0 & M0, w0 & M3, w0 & M6, h0 & M0};
  a[1] = u32x4_t{h0 & M3, w1 & M0, w1 & M3, w1 & M6};
  a[2] = u32x4_t{h1 & M0, h1 & M3, w2 & M0, w2 & M3};
  a[3] = u32x4_t{w2 & M6, h2 & M0, h2 & M3, spare};
}

// fp6 layout (fx_w3_planes_to_fp6): a lane's three words for one group expand
// into the six fp6 e2m3 registers of v_mfma_scale_f32_16x16x128_f8f6f4's A
// operand (field e at bits [6 e, 6 e + 6): sign and exponent bits zero, the code
// in the mantissa, the exact value q / 8).  Two masks, two shifted masks and one
// register that takes bits 29 and 30 from the low end of the third word.
typedef int i32x8_t __attribute__((ext_vector_type(8)));
constexpr unsigned kFp6M0 = 0xC71C71C7u, kFp6M1 = 0x71C71C71u, kFp6M2 = 0x1C71C71Cu;
__device__ __forceinline__ i32x8_t expand_fp6(unsigned s0, unsigned s1, unsigned s2) {
  const unsigned mid = __builtin_amdgcn_bitop3_b32(s2 << 28, s2 >> 3, 0x60000000u, 0xE4);  // m ? a : b
  return i32x8_t{int(s0 & kFp6M0), int(s2 & kFp6M1), int((s0 >> 1) & kFp6M2), int(s1 & kFp6M0),
                 int(mid & kFp6M1), int((s1 >> 1) & kFp6M2), 0, 0};
}

// fp6-layout B operands of one lane's 8 bf16 activations: two fp8 e4m3 digits,
// hi = fp8(x / S) and lo = fp8((x - hi S) / S) with S = 2^(e - 8) for the group's
// max|x| in [2^(e-1), 2^e) (so |x| / S < 256, inside e4m3's range); hi + lo is x
// exactly down to 2^-10 of the group's maximum (a bf16 value's 8 significant
// bits split 4 + 4).  Returns the group's sum of x (exact values) and the
// epilogue's exponent e - 5 (the A fields carry q / 8).
__device__ __forceinline__ void stage_fp6_8(const float v[8], uint2& hi, uint2& lo, float& sum, int& exp_off) {
  float mx = 0.f, sm = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    mx = fmaxf(mx, fabsf(v[i]));
    sm += v[i];
  }
  mx = row16_max(mx);
  sm = row16_sum(sm);
  int e = 0;
  if (mx > 0.f) frexpf(mx, &e);
  e = max(e, -118);  // S stays a normal float; groups below 2^-118 flush toward zero
  const float S = ldexpf(1.f, e - 8);
  typedef short i16x2_t __attribute__((ext_vector_type(2)));
  unsigned h[2], l[2];
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    const float* x = v + 4 * w;
    i16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(i16x2_t{0, 0}, x[0], x[1], S, false);
    a = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(a, x[2], x[3], S, true);
    const unsigned hw = __builtin_bit_cast(unsigned, a);
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    const f32x2_t b01 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hw, S, false);
    const f32x2_t b23 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hw, S, true);
    i16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(i16x2_t{0, 0}, x[0] - b01.x, x[1] - b01.y, S, false);
    c = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(c, x[2] - b23.x, x[3] - b23.y, S, true);
    h[w] = hw;
    l[w] = __builtin_bit_cast(unsigned, c);
  }
  hi = uint2{h[0], h[1]};
  lo = uint2{l[0], l[1]};
  sum = sm;
  exp_off = e - 5;
}

// Mantissa position p of register i's codes in the field layout (the B operand
// carries the matching 2^-p).
constexpr int kFieldShift[16] = {0, 3, 6, 0, 3, 0, 3, 6, 0, 3, 0, 3, 6, 0, 3, 0};
// The same, a nibble per register (register i at bits 4 i): a lane reads its four
// with shifts (a runtime index into the array would be a memory load).
constexpr unsigned long long field_shift_nibbles() {
  unsigned long long v = 0;
  for (int i = 0; i < 16; ++i) v |= static_cast<unsigned long long>(kFieldShift[i]) << (4 * i);
  return v;
}

// Field-layout B operands of one lane's 8 activations (k-block kb, lanes r =
// 0..15 of the DPP row hold the group's 128 columns): fp16 values x * 2^(E - p)
// (exact: they keep the activation's 8 or 11 significant bits within fp16's
// range) with p the mantissa position of the register each pair meets, the
// group's sum of x and exponent offset.  Shared by both field-layout kernels so
// their bits agree.
// The mantissa positions p of lane r's four element pairs (registers 4 (r % 4) +
// q), a nibble each; formed once per staged batch and shared by its rows (the
// asm keeps it from being hoisted and held across the batch loop, where it cost
// the 4-wave kernel a spill).
__device__ __forceinline__ unsigned field_positions(int r) {
  unsigned rr = unsigned(r & 3);
  asm volatile("" : "+v"(rr));
  return unsigned(field_shift_nibbles() >> (16 * rr)) & 0xffffu;
}

__device__ __forceinline__ void stage_fields8(const float v[8], unsigned fsh, u32x4_t& o, float& sum, int& exp_off) {
  float mx = 0.f, sm = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    mx = fmaxf(mx, fabsf(v[i]));
    sm += v[i];
  }
  mx = row16_max(mx);
  sm = row16_sum(sm);
  const int E = choose_exponent<kF16>(mx);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = E - int((fsh >> (4 * q)) & 0xfu);
    o[q] = f32x2_to_f16x2_bits(ldexpf(v[2 * q], e), ldexpf(v[2 * q + 1], e));
  }
  sum = sm;
  exp_off = subnormal_exponent<kF16>() - E;
}

// Qwen3RMSNorm of 8 activations: round(w * round(h * inv)) in the activation type.
template <int XDT>
__device__ __forceinline__ void normalize8(float v[8], const u32x4_t& wn, float norm_inv) {
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    float a = v[i] * norm_inv, b = v[i + 1] * norm_inv;
    round_pair<XDT>(a, b);
    a *= to_f32<XDT>(uint16_t(wn[i >> 1]));
    b *= to_f32<XDT>(uint16_t(wn[i >> 1] >> 16));
    round_pair<XDT>(a, b);
    v[i] = a;
    v[i + 1] = b;
  }
}

// One (row, group) term of the epilogue: acc + s (D 2^fe - z sum(x)), as two
// fused multiply-adds (the rounding every MFMA kernel of this file shares).
__device__ __forceinline__ float accumulate_group(float acc, float se, float zf, float d, int fe, float sx) {
  return fmaf(se, fmaf(-zf, sx, ldexpf(d, fe)), acc);
}

// Everything one wave loads for one batch, kept as raw bits: this lane's plane
// rows (one per row tile), its 8 activations per row (or, with a permutation,
// its 8 column indices), and the epilogue's scales and zero-points.  Nothing
// loaded is used before consume(), so the prefetched batches stay in flight.
template <int MB, int RT>
struct BatchLoads {
  u32x4_t w[RT][3];
  u32x4_t xv[MB];    // activation bits of rows 0..MB-1 (PERM: xv[0] = 8 int16 columns)
  unsigned s[RT][2]; // scales of rows erow..erow+3 of each tile, two per word
  unsigned z[RT];    // zero-points of rows erow..erow+3, one per byte
  unsigned se[RT][4], ze[RT][4];  // the same as single elements when O % 4 != 0
  u32x4_t wn;        // NORMIN: the RMSNorm weights of this lane's 8 columns
  unsigned za[RT];   // CORR: the zero-point of this lane's A row (row r of each tile, group 4i + k-block)
};

// decoded_bf16 arithmetic (the reference's +-3 correction, csrc/w3_lut.cu:105-122):
// each weight is bf16(s (q - z)), which differs from s (q - z) only where
// |q - z| = 3, by sign(q - z) (bf16(3 s) - 3 s).  So y = sum_g s D_g - s z sum(x) +
// e_g C_g with e_g = bf16(3 s) - 3 s and C_g = sum_k ([q - z = 3] - [q - z = -3]) x_k.
// C comes from the same dequantizer and B operands: the planes are transformed
// bitwise into g(q) = q - c(q) (z = 4: q = 7 -> 6, q = 1 -> 2; z = 3: q = 6 -> 5,
// q = 0 -> 1; every other code unchanged), so C = D - sum_k g(q_k) x_k from a second
// MFMA chain.  In plane bits (b0 = P0, b1 = P1, b2 = ~P2, e = P1 ^ P2 = ~(b1 ^ b2)):
//   z = 4: g0 = b0 & ~e,  g1 = b1 | (b0 & ~b2)      z = 3: g0 = b0 | e,  g1 = b1 & (~b2 | b0)
// and g2 = b2; zmask (all ones where z = 4) selects per lane.  Zero-points must be
// 3 or 4 (the route's contract).
__device__ __forceinline__ void corrected_planes(unsigned p0, unsigned p1, unsigned p2, unsigned zmask,
                                                 unsigned& g0, unsigned& g1) {
  const unsigned e = p1 ^ p2;
  g0 = bitfield_insert(zmask, p0 & ~e, p0 | e);
  g1 = bitfield_insert(zmask, p1 | (p0 & p2), p1 & (p2 | p0));
}

// The K reduction of a workgroup always runs in the order eight waves give it:
// "virtual wave" k accumulates batches k, k + 8, k + 16, ... in turn, and the
// eight sums are added in k order.  A 4-wave workgroup keeps two accumulator
// sets per wave (k = w and k = w + 4), so the result depends only on the payload
// and x, never on the tiling (a fused q|k|v or gate|up GEMV gives the same bits
// as the separate projections whatever waves each plan picks).
constexpr int kSumLanes = 8;

// Workgroup LDS: per wave, B operands [k-block][step][row] (16 B each); zero
// operands [step][row] read by the lanes whose column belongs to another k-block
// (one array for the workgroup: every wave writes all of it, with zeros only,
// before its own first read, so no barrier orders the waves); sum of x and
// subnormal exponent - E per (k-block group, row); the per-wave partial outputs.
// The four k-block stages of a wave are kStageStride<MB> 16-byte slots apart, one
// more than they hold: without the extra slot every k-block started on the same
// LDS bank, and the lanes staging or reading the four k-blocks at once collided.
template <int MB>
constexpr int kStageStride = 16 * MB + 1;

template <int NW, int MB, int RT>
struct MfmaShared {
  u32x4_t bstage[NW][4 * kStageStride<MB>];
  u32x4_t bzero[16 * MB];
  float gsum[NW][4 * MB];
  int gexp[NW][4 * MB];
  float red[kSumLanes][16 * RT * MB];
};

// VEC: O is a multiple of 4, so the four scales / zero-points of a lane are one
// aligned load each.  A separate instantiation (rather than a runtime branch)
// keeps the load count per batch fixed, so the wait before staging covers only
// the activations.
template <int NW, int PD, int MB, int RT, bool PERM, int XDT, int SDT, bool NORMIN, bool VEC, bool FIELDS,
          bool CORR, bool FP6 = false>
__device__ __forceinline__ void w3_mfma_body(
    MfmaShared<NW, MB, RT>& sh, const uint16_t* __restrict__ x, const int16_t* __restrict__ perm,
    const uint8_t* __restrict__ planes, const uint16_t* __restrict__ scales,
    const uint8_t* __restrict__ zeros, float* __restrict__ partial,
    uint16_t* out, int O, int G, int gps, int row_blocks, int swiglu, const ResidualArgs& ra, int x_lds,
    u32x4_t* x_stage, int split) {
  auto& bstage = sh.bstage;
  auto& bzero = sh.bzero;
  auto& gsum = sh.gsum;
  auto& gexp = sh.gexp;
  auto& red = sh.red;
  const int t = threadIdx.x, lane = t & 63, wave = wave_index();
  const int K = G * 128;
  const int row0 = xcd_local_index8(blockIdx.x, row_blocks) * (16 * RT);
  const int g0 = split * gps;
  const int g1 = min(G, g0 + gps);
  const int nbatch = (g1 - g0 + 3) >> 2;
  // absent zero-points read as 0 (empty buffer) and become 4 through this OR
  const unsigned zero_default = zeros ? 0u : 0x04040404u;

  const unsigned go = unsigned(G) * unsigned(O);
  const auto rp = buffer_resource_2g(planes, go * 48u);
  const auto rs = buffer_resource_2g(scales, go * 2u);
  const auto rz = buffer_resource_2g(zeros ? (const void*)zeros : (const void*)scales, zeros ? go : 0u);
  const auto rx = buffer_resource_2g(x, unsigned(MB) * unsigned(K) * 2u);
  const auto rperm = buffer_resource(PERM ? (const void*)perm : (const void*)x, PERM ? size_t(K) * 2 : 0);
  // NORMIN: the row's RMSNorm weights, and 1 / rms from the tile partials (each
  // wave reduces them itself, in a fixed order: lane l adds partials l, l + 64,
  // ..., then the wave total), loaded ahead of every other load
  const auto rwn = buffer_resource(NORMIN ? (const void*)ra.pro_weight : (const void*)x, NORMIN ? size_t(K) * 2 : 0);
  float norm_inv = 1.f;
  float pp[kMaxNormPartialsPerLane];
  if constexpr (NORMIN) {
    const auto rpp = buffer_resource(ra.pro_partial, size_t(ra.pro_n) * 4);
#pragma unroll
    for (int k = 0; k < kMaxNormPartialsPerLane; ++k) {
      const int idx = (lane & 63) + 64 * k;
      pp[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rpp, idx < ra.pro_n ? idx * 4 : kOutOfRange, 0, 0));
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // the output index of this thread's epilogue row (residual: lanes 0..15 of wave
  // 0, row row0 + lane; SwiGLU: thread t, pair row0 / 2 + t), loaded ahead of the
  // weight stream so the epilogue does not wait a round trip for it
  int ep_to = -1;
  if (ra.ep_index) {
    const int n_idx = ra.ep_residual ? O : O / 2;
    const int at = ra.ep_residual ? (wave == 0 && lane < 16 ? row0 + lane : n_idx)
                                   : (2 * t < 16 * RT ? row0 / 2 + t : n_idx);
    const auto rix = buffer_resource(ra.ep_index, size_t(n_idx) * 2);
    ep_to = int(int16_t(__builtin_amdgcn_raw_buffer_load_b16(rix, at < n_idx ? at * 2 : kOutOfRange, 0, 0)));
  }

  const int r = lane & 15;    // A role: row within tile; x role: 8-column chunk
  const int kb = lane >> 4;   // A role: k-block = group slot; D role: row block
  const int c = lane & 15;    // B / D role: column
  const int cslot = c & 3, cm = c >> 2;
  // activation rows 4h .. 4h+3 sit in the D columns of half h (MB = 8: two MFMA
  // chains share every dequantized A operand)
  constexpr int NH = (MB + 3) / 4;
  u32x4_t* my_stage = bstage[wave];
  uint16_t* stage16 = reinterpret_cast<uint16_t*>(my_stage);
  for (int i = lane; i < 16 * MB; i += 64) bzero[i] = u32x4_t{0u, 0u, 0u, 0u};
  // operand of step st for half h: bsrc[h][st * MB]; rmc[h] the lane's activation row (clamped)
  const u32x4_t* bsrc[NH];
  int rmc[NH];
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const int row = cm + 4 * h;
    rmc[h] = row < MB ? row : 0;
    bsrc[h] = ((cslot == kb && row < MB) ? my_stage + kb * kStageStride<MB> : bzero) + rmc[h];
  }
  // FP6: the B operand of group slot g's instruction is this lane's 32 bytes of
  // [slot][digit][k-block] in the stage when its column is g (hi digit) or 4 + g
  // (lo digit), else zeros; D column g then holds the hi dot and 4 + g the lo dot
  const u32x4_t* fp6_src[4];
  if constexpr (FP6) {
#pragma unroll
    for (int g = 0; g < 4; ++g)
      fp6_src[g] = (cslot == g && c < 8) ? my_stage + ((g * 2 + (c >> 2)) * 4 + kb) * 2 : bzero;
  }
  const int plane_stride = O * 16;
  int prow[RT];  // the lane's A row of each tile, clamped into [0, O)
#pragma unroll
  for (int tt = 0; tt < RT; ++tt) prow[tt] = min(row0 + 16 * tt + r, O - 1);
  // x role: lane (kb, r) owns columns 8r .. 8r+7 of its group; they land in
  // steps 4(r>>2) + s, operand slots je (weight 1) and je + 4 (weight 16).
  const int xstep = 4 * (r >> 2);
  const int je = ((r >> 1) & 1) + 2 * (r & 1);

  // live = false: every load of the batch is out of range (returns zeros, no
  // memory access), so a wave issues the same loads whatever its batch count
  auto issue = [&](int batch, BatchLoads<MB, RT>& L, bool live) __attribute__((always_inline)) {
    const int gb = g0 + 4 * batch;
    const int col = (gb + kb) * 128 + 8 * r;
    const bool real = live && gb + kb < G;
    if constexpr (PERM) {
      L.xv[0] = load_b128(rperm, real ? col * 2 : kOutOfRange, 0);
    } else {
#pragma unroll
      for (int m = 0; m < MB; ++m) L.xv[m] = load_b128(rx, real ? (m * K + col) * 2 : kOutOfRange, 0);
    }
    if constexpr (NORMIN) L.wn = load_b128(rwn, real ? col * 2 : kOutOfRange, 0);
    if constexpr (CORR) {  // the A row's zero-point (needed by the dequant, ahead of the planes)
#pragma unroll
      for (int tt = 0; tt < RT; ++tt)
        L.za[tt] = __builtin_amdgcn_raw_buffer_load_b8(rz, real ? gb * O + lane_times_rows(kb, O) + row0 + 16 * tt + r : kOutOfRange,
                                                       0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    // groups past G: past the end -> zeros; rows past O read row O - 1 (never
    // stored), since the plane stride rides in the scalar offset, which the
    // range check does not cover
    if constexpr (FP6) {
      // [G / 4, O, k-block, slot, 3 words]: the lane's 48 bytes of the batch are contiguous
#pragma unroll
      for (int tt = 0; tt < RT; ++tt) {
        const int poff = live ? ((gb >> 2) * O + prow[tt]) * 192 + kb * 48 : kOutOfRange;
        L.w[tt][0] = load_b128_stream(rp, poff, 0);
        L.w[tt][1] = load_b128_stream(rp, poff, 16);
        L.w[tt][2] = load_b128_stream(rp, poff, 32);
      }
    } else {
      const int gbase = gb * 3 * O + lane_times_rows(kb, 3 * O);  // gb is wave-uniform
#pragma unroll
      for (int tt = 0; tt < RT; ++tt) {
        const int poff = live ? (gbase + prow[tt]) * 16 : kOutOfRange;
        L.w[tt][0] = load_b128_stream(rp, poff, 0);
        L.w[tt][1] = load_b128_stream(rp, poff, plane_stride);
        L.w[tt][2] = load_b128_stream(rp, poff, 2 * plane_stride);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    const int eoff = gb * O + lane_times_rows(cslot, O) + row0 + 4 * kb;
#pragma unroll
    for (int tt = 0; tt < RT; ++tt) {
      const int e = eoff + 16 * tt;
      if constexpr (VEC) {
        const uint2 s4 = __builtin_bit_cast(
            uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, live ? e * 2 : kOutOfRange, 0, 0));
        L.s[tt][0] = s4.x;
        L.s[tt][1] = s4.y;
        L.z[tt] = __builtin_amdgcn_raw_buffer_load_b32(rz, live ? e : kOutOfRange, 0, 0);
      } else {  // O not a multiple of 4 (tests, tiny layers): element loads, packed in consume()
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          L.se[tt][j] = __builtin_amdgcn_raw_buffer_load_b16(rs, live ? (e + j) * 2 : kOutOfRange, 0, 0);
          L.ze[tt][j] = __builtin_amdgcn_raw_buffer_load_b8(rz, live ? e + j : kOutOfRange, 0, 0);
        }
      }
    }
  };

  // B operands of one batch for activation row m from this lane's 8 values.
  auto stage_row = [&](int m, const float v[8]) __attribute__((always_inline)) {
    if constexpr (FP6) {
      // the lane's 8 columns of slot kb sit in B k-block r / 4, bytes 8 (r % 4) ..
      uint2 hi, lo;
      float sm;
      int ge;
      stage_fp6_8(v, hi, lo, sm, ge);
      uint2* st8 = reinterpret_cast<uint2*>(my_stage);
      st8[((kb * 2 + 0) * 4 + (r >> 2)) * 4 + (r & 3)] = hi;
      st8[((kb * 2 + 1) * 4 + (r >> 2)) * 4 + (r & 3)] = lo;
      if (r == 0) {
        gsum[wave][kb * MB + m] = sm;
        gexp[wave][kb * MB + m] = ge;
      }
    } else if constexpr (FIELDS) {
      // the lane's 8 columns are elements 0..7 of step r, one 16-byte write
      u32x4_t o;
      float sm;
      int ge;
      stage_fields8(v, field_positions(r), o, sm, ge);
      my_stage[kb * kStageStride<MB> + r * MB + m] = o;
      if (r == 0) {
        gsum[wave][kb * MB + m] = sm;
        gexp[wave][kb * MB + m] = ge;
      }
    } else {
      float mx = 0.f, sm = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        mx = fmaxf(mx, fabsf(v[i]));
        sm += v[i];
      }
      mx = row16_max(mx);
      sm = row16_sum(sm);
      const int E = choose_exponent<XDT>(mx);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        uint16_t* dst = stage16 + (kb * kStageStride<MB> + (xstep + s) * MB + m) * 8;
        dst[je] = exact_bits<XDT>(ldexpf(v[s], E));
        dst[je + 4] = exact_bits<XDT>(ldexpf(v[4 + s], E - 4));
      }
      if (r == 0) {
        gsum[wave][kb * MB + m] = sm;
        gexp[wave][kb * MB + m] = subnormal_exponent<XDT>() - E;
      }
    }
  };

  static_assert(kSumLanes % NW == 0, "waves per workgroup must divide the reduction lanes");
  constexpr int VS = kSumLanes / NW;  // accumulator sets per wave
  float acc_sets[VS][RT][NH][4];
#pragma unroll
  for (int v = 0; v < VS; ++v)
#pragma unroll
    for (int tt = 0; tt < RT; ++tt)
#pragma unroll
      for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc_sets[v][tt][h][j] = 0.f;
  int cur_batch = 0;
  auto consume = [&](const BatchLoads<MB, RT>& L, float (&acc)[RT][NH][4]) __attribute__((always_inline)) {
    const int gb = g0 + 4 * cur_batch;
    if constexpr (NORMIN) {
      // 1 / rms from the tile partials, at the wave's first batch: in the loop
      // it follows the ring issue on every path, so the wait for the partials
      // (issued before the ring) leaves the batch's loads in flight.  Computed
      // ahead of the loop, it was placed between the activation and the plane
      // loads, and the wait put a full round trip ahead of the weight stream
      // (+1.3 us per call).
      if (cur_batch == wave) {
        float total = 0.f;
#pragma unroll
        for (int k = 0; k < kMaxNormPartialsPerLane; ++k) total += pp[k];
        norm_inv = rsqrtf(wave_total(total) / float(K) + ra.pro_eps);
      }
    }
    if constexpr (PERM) {
      const bool real = gb + kb < G;
      const unsigned pw[4] = {L.xv[0].x, L.xv[0].y, L.xv[0].z, L.xv[0].w};
      const uint16_t* xs16 = reinterpret_cast<const uint16_t*>(x_stage);
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int src = int(int16_t(pw[i >> 1] >> (16 * (i & 1))));
          uint16_t bits;
          if (x_lds)  // from the workgroup's LDS copy of x (entries outside [0, K) read zero)
            bits = real && unsigned(src) < unsigned(K) ? xs16[m * K + src] : uint16_t(0);
          else
            bits = uint16_t(__builtin_amdgcn_raw_buffer_load_b16(rx, real ? (m * K + src) * 2 : kOutOfRange, 0, 0));
          v[i] = to_f32<XDT>(bits);
        }
        stage_row(m, v);
      }
    } else {
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        const unsigned xw[4] = {L.xv[m].x, L.xv[m].y, L.xv[m].z, L.xv[m].w};
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = to_f32<XDT>(uint16_t(xw[i >> 1] >> (16 * (i & 1))));
        if constexpr (NORMIN) normalize8<XDT>(v, L.wn, norm_inv);
        stage_row(m, v);
      }
    }
    __builtin_amdgcn_wave_barrier();

    f32x4_t d[RT][NH], dg[CORR ? RT : 1][CORR ? NH : 1];
#pragma unroll
    for (int tt = 0; tt < RT; ++tt)
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        d[tt][h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        if constexpr (CORR) dg[tt][h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
    unsigned zmask[RT];
    if constexpr (CORR) {
#pragma unroll
      for (int tt = 0; tt < RT; ++tt)
        zmask[tt] = ((L.za[tt] | zero_default) & 0xffu) == 4u ? 0xffffffffu : 0u;  // absent zero-points: 4
    }
    if constexpr (FP6) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const u32x4_t b0 = fp6_src[g][0], b1 = fp6_src[g][1];
        const i32x8_t bv = {int(b0.x), int(b0.y), int(b0.z), int(b0.w), int(b1.x), int(b1.y), int(b1.z), int(b1.w)};
#pragma unroll
        for (int tt = 0; tt < RT; ++tt) {
          const u32x4_t* w = L.w[tt];  // slot g: words 3 g .. 3 g + 2 of the lane's twelve
          const i32x8_t av = expand_fp6(w[(3 * g) / 4][(3 * g) % 4], w[(3 * g + 1) / 4][(3 * g + 1) % 4],
                                        w[(3 * g + 2) / 4][(3 * g + 2) % 4]);
          // A fp6 e2m3 (cbsz 2), B fp8 e4m3 (blgp 0), unit block scales (E8M0 127)
          d[tt][0] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, d[tt][0], 2, 0, 0, 127, 0, 127);
        }
      }
      // column g += column 4 + g: the lo digit's dot into the hi digit's lane
#pragma unroll
      for (int tt = 0; tt < RT; ++tt)
#pragma unroll
        for (int j = 0; j < 4; ++j) d[tt][0][j] += dpp_move<kDppRowShl4>(d[tt][0][j]);
    } else
#pragma unroll
    for (int word = 0; word < 4; ++word) {
      u32x4_t a[RT][4], ag[CORR ? RT : 1][4];
#pragma unroll
      for (int tt = 0; tt < RT; ++tt) {
        const u32x4_t* w = L.w[tt];
        if constexpr (FIELDS) dequant_fields(w[0][word], w[1][word], w[2][word], a[tt]);
        else dequant_word(w[0][word], w[1][word], w[2][word], a[tt]);
        if constexpr (CORR) {
          unsigned g0, g1;
          corrected_planes(w[0][word], w[1][word], w[2][word], zmask[tt], g0, g1);
          dequant_word(g0, g1, w[2][word], ag[tt]);
        }
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          const u32x4_t b = bsrc[h][(4 * word + s) * MB];
#pragma unroll
          for (int tt = 0; tt < RT; ++tt) {
            if constexpr (XDT == kBF16 && !FIELDS)
              d[tt][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  __builtin_bit_cast(bf16x8_t, a[tt][s]), __builtin_bit_cast(bf16x8_t, b), d[tt][h], 0, 0, 0);
            else
              d[tt][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                  __builtin_bit_cast(f16x8_t, a[tt][s]), __builtin_bit_cast(f16x8_t, b), d[tt][h], 0, 0, 0);
            if constexpr (CORR) {
              if constexpr (XDT == kBF16)
                dg[tt][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8_t, ag[tt][s]), __builtin_bit_cast(bf16x8_t, b), dg[tt][h], 0, 0, 0);
              else
                dg[tt][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(f16x8_t, ag[tt][s]), __builtin_bit_cast(f16x8_t, b), dg[tt][h], 0, 0, 0);
            }
          }
        }
      }
    }
    float sxv[NH];
    int fev[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      sxv[h] = gsum[wave][cslot * MB + rmc[h]];
      fev[h] = gexp[wave][cslot * MB + rmc[h]];
    }
#pragma unroll
    for (int tt = 0; tt < RT; ++tt) {
      unsigned sw[2] = {L.s[tt][0], L.s[tt][1]}, zw = L.z[tt];
      if constexpr (!VEC) {
        sw[0] = L.se[tt][0] | (L.se[tt][1] << 16);
        sw[1] = L.se[tt][2] | (L.se[tt][3] << 16);
        zw = L.ze[tt][0] | (L.ze[tt][1] << 8) | (L.ze[tt][2] << 16) | (L.ze[tt][3] << 24);
      }
      zw |= zero_default;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const unsigned sb = (j & 1) ? (sw[j >> 1] >> 16) : (sw[j >> 1] & 0xffffu);
        const float se = to_f32<SDT>(uint16_t(sb));
        const float zf = float((zw >> (8 * j)) & 0xffu);
#pragma unroll
        for (int h = 0; h < NH; ++h) acc[tt][h][j] = accumulate_group(acc[tt][h][j], se, zf, d[tt][h][j], fev[h], sxv[h]);
        if constexpr (CORR) {
          // bf16(3 s) - 3 s: 3 s is exact in fp32 (s has 8 significant bits)
          const float eps = round_to<kBF16>(3.f * se) - 3.f * se;
#pragma unroll
          for (int h = 0; h < NH; ++h) acc[tt][h][j] += eps * ldexpf(d[tt][h][j] - dg[tt][h][j], fev[h]);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  };

  // my batches: wave, wave + NW, ...; the i-th is batch wave + i*NW
  // (the i-th batch of this wave feeds accumulator set i % VS, virtual wave
  // wave + (i % VS) * NW)
  const int mine = wave < nbatch ? (nbatch - wave + NW - 1) / NW : 0;
  // PERM with x_lds: the workgroup copies x [MB, K] into LDS once (16-byte
  // chunks, up to kXChunks per thread), so the per-value gather reads LDS, not
  // global memory.  The chunks are loaded ahead of the weight ring: loads complete
  // in issue order, so waiting for them leaves the ring's weights in flight.
  constexpr int kXChunks = 4;
  u32x4_t xc[PERM ? kXChunks : 1];
  const int n16 = MB * K / 8;
  if constexpr (PERM) {
    if (x_lds) {
#pragma unroll
      for (int j = 0; j < kXChunks; ++j) {
        const int c = t + j * NW * 64;
        xc[j] = load_b128(rx, c < n16 ? c * 16 : kOutOfRange, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  BatchLoads<MB, RT> ring[PD];
#pragma unroll
  for (int i = 0; i < PD; ++i)
    issue(wave + i * NW, ring[i], i < mine);
  if constexpr (PERM) {
    __builtin_amdgcn_sched_barrier(0);
    if (x_lds) {
#pragma unroll
      for (int j = 0; j < kXChunks; ++j) {
        const int c = t + j * NW * 64;
        if (c < n16) x_stage[c] = xc[j];
      }
      __syncthreads();
    }
  }
  // batches always accumulate into set 0; with two sets they are swapped after
  // every batch (register moves, not a second unrolled copy of the loop body),
  // so after an odd count set 0 holds the wave's second virtual wave
  for (int base = 0; base < mine; base += PD) {
#pragma unroll
    for (int i = 0; i < PD; ++i) {
      if (base + i < mine) {
        cur_batch = wave + (base + i) * NW;
        consume(ring[i], acc_sets[0]);
        if (base + i + PD < mine) issue(wave + (base + i + PD) * NW, ring[i], true);
        if constexpr (VS == 2) {
#pragma unroll
          for (int tt = 0; tt < RT; ++tt)
#pragma unroll
            for (int h = 0; h < NH; ++h)
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const float keep = acc_sets[0][tt][h][j];
                acc_sets[0][tt][h][j] = acc_sets[1][tt][h][j];
                acc_sets[1][tt][h][j] = keep;
              }
        }
      }
    }
  }
  const bool odd = VS == 2 && (mine & 1);

  // sum the four group slots of each activation row (lanes c = 4m .. 4m+3)
#pragma unroll
  for (int v = 0; v < VS; ++v) {
#pragma unroll
    for (int tt = 0; tt < RT; ++tt)
#pragma unroll
      for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float a = acc_sets[v][tt][h][j];
          a += dpp_move<kDppXor1>(a);
          a += dpp_move<kDppXor2>(a);
          acc_sets[v][tt][h][j] = a;
        }
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      if (cslot == 0 && cm + 4 * h < MB) {
#pragma unroll
        for (int tt = 0; tt < RT; ++tt)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            red[wave + (odd ? 1 - v : v) * NW][(16 * tt + 4 * kb + j) * MB + cm + 4 * h] = acc_sets[v][tt][h][j];
      }
    }
  }
  __syncthreads();
  if (ra.ep_residual) {
    // MB = 1, RT = 1: out = round(residual + round(y)) for the tile's 16 rows
    // (threads 0..15, wave 0), and the tile's sum of out^2 (DPP row sum)
    if (wave == 0) {
      float h2 = 0.f;
      const int orow = row0 + lane;
      if (lane < 16 && orow < O) {
        float total = 0.f;
#pragma unroll
        for (int k = 0; k < kSumLanes; ++k) total += red[k][lane];
        const float h = round_to<XDT>(to_f32<XDT>(ra.ep_residual[orow]) + round_to<XDT>(total));
        out[orow] = from_f32<XDT>(h);
        if (ra.ep_index && unsigned(ep_to) < unsigned(O)) ra.ep_sorted[ep_to] = from_f32<XDT>(h);
        h2 = h * h;
      }
      h2 = row16_sum(h2);
      if (lane == 0) ra.ep_partial[row0 / 16] = h2;
    }
    return;
  }
  if (swiglu) {
    // rows come in (gate, up) pairs (MB = 1, one K split): each pair is rounded
    // to the activation dtype as a separate GEMV would store it, then
    // act = round(round(silu(g)) * u) as Qwen3MLP computes it; out holds O / 2
    for (int i = 2 * t; i < 16 * RT; i += 2 * NW * 64) {
      float tg = 0.f, tu = 0.f;
#pragma unroll
      for (int k = 0; k < kSumLanes; ++k) {
        tg += red[k][i];
        tu += red[k][i + 1];
      }
      const int orow = row0 + i;
      if (orow < O) {
        const float g = round_to<XDT>(tg), u = round_to<XDT>(tu);
        const float sg = round_to<XDT>(g / (1.f + __expf(-g)));
        if (!ra.ep_index) out[orow / 2] = from_f32<XDT>(sg * u);
        else if (unsigned(ep_to) < unsigned(O / 2)) out[ep_to] = from_f32<XDT>(sg * u);
      }
    }
    return;
  }
  for (int i = t; i < 16 * RT * MB; i += NW * 64) {
    float total = 0.f;
#pragma unroll
    for (int k = 0; k < kSumLanes; ++k) total += red[k][i];
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


// grid (row_blocks = ceil(O / (16 RT)), splits) workgroups of NW*64 threads.
// Workgroup: rows [16 RT b, +16 RT), groups [gps*split, +gps) with gps a
// multiple of 4.  Rows past O and groups past G need no masking: padded groups
// have zero activations (so D = 0 and sum(x) = 0), and rows past O are never
// stored.  x is [MB, 128 G] row-major; with PERM, sorted column k reads x
// column perm[k] -- from the workgroup's LDS copy of x when x_lds is set (the
// launch then carries MB * K * 2 bytes of dynamic LDS and K * MB / 8 must not
// exceed 4 chunks per thread), else one 2-byte global load per value.  swiglu != 0 (MB = 1, one split, O even): the payload's rows
// interleave gate and up rows, and out receives SiLU(gate) * up, O / 2 values.
// One-row, one-tile, single-prefetch instantiations (the decode shapes) are held
// to 80 VGPRs, six waves per SIMD: a 24576-row gate|up grid of 4-wave workgroups
// then fits in one residency round.
// VSEL picks the scale / zero-point load form: 0 at run time from O % 4, 1 the
// vector form only (O % 4 == 0), 2 the element form only.  A kernel holding both
// is allocated registers for the costlier element form, which may spill and
// then needs a scratch segment on every launch; the normalising instantiations
// are split.
// FIELDS: the payload is the field layout (one activation row, one batch in
// flight per wave).  NORMIN takes no permutation: its caller hands it h and the
// norm weights in the payload's sorted column order (a producer epilogue's
// ep_index output, weights reordered once at bind time).
// CORR: decoded_bf16 arithmetic (bf16 scales, zero-points 3 or 4; planar layout).
template <int NW, int PD, int MB, int RT, bool PERM, int XDT, int SDT, bool NORMIN = false, int VSEL = 0,
          bool FIELDS = false, bool CORR = false, bool FP6 = false>
__global__ __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu(MB == 1 && RT == 1 && PD == 1 && !CORR && !FP6 ? 6 : 1)))
void w3_mfma_kernel(
    const uint16_t* __restrict__ x, const int16_t* __restrict__ perm,
    const uint8_t* __restrict__ planes, const uint16_t* __restrict__ scales,
    const uint8_t* __restrict__ zeros, float* __restrict__ partial,
    uint16_t* out, int O, int G, int gps, int row_blocks, int swiglu, ResidualArgs ra, int x_lds,
    StridedArgs sb) {
  // one scalar-load round for every argument (otherwise the pointer loads sink
  // below the first branch and add a second round trip before the first load)
  asm volatile("" ::"s"(x), "s"(perm), "s"(planes), "s"(scales), "s"(zeros), "s"(partial), "s"(out),
               "s"(O), "s"(G), "s"(gps), "s"(row_blocks), "s"(swiglu), "s"(ra.ep_residual), "s"(ra.ep_partial),
               "s"(ra.ep_index), "s"(ra.ep_sorted), "s"(x_lds), "s"(sb.x), "s"(sb.planes), "s"(sb.scales),
               "s"(sb.zeros), "s"(sb.out));
  // a strided batch: grid.y walks the payloads (one K split each); row blocks
  // per payload are a multiple of 8 at the batched shapes, so the XCD mapping of
  // blockIdx.x holds within every payload
  int split = blockIdx.y;
  if (sb.planes) {
    const long long p = blockIdx.y;
    x += p * sb.x;
    planes += p * sb.planes;
    scales += p * sb.scales;
    if (zeros) zeros += p * sb.zeros;
    out += p * sb.out;
    split = 0;
  }
  if constexpr (NORMIN)
    asm volatile("" ::"s"(ra.pro_partial), "s"(ra.pro_n), "s"(ra.pro_weight), "s"(ra.pro_eps));
  static_assert(!FIELDS || (MB == 1 && PD == 1), "field layout: one activation row, one batch in flight");
  static_assert(!(PERM && NORMIN), "the normalising prologue reads its activations in sorted order");
  static_assert(!CORR || (SDT == kBF16 && !FIELDS && !NORMIN), "decoded_bf16: bf16 scales, planar layout");
  static_assert(!FP6 || (FIELDS && !PERM && !CORR && XDT == kBF16 && VSEL == 1),
                "fp6 layout: one bf16 activation row, sorted columns, vector scale loads");
  __shared__ MfmaShared<NW, MB, RT> sh;
  extern __shared__ u32x4_t x_stage[];  // PERM with x_lds: x [MB, K], MB * K * 2 bytes of dynamic LDS
  if (VSEL == 1 || (VSEL == 0 && (O & 3) == 0))
    w3_mfma_body<NW, PD, MB, RT, PERM, XDT, SDT, NORMIN, VSEL != 2, FIELDS, CORR, FP6>(sh, x, perm, planes, scales, zeros,
                                                                           partial, out, O, G, gps, row_blocks,
                                                                           swiglu, ra, x_lds, x_stage, split);
  else
    w3_mfma_body<NW, PD, MB, RT, PERM, XDT, SDT, NORMIN, VSEL == 1, FIELDS, CORR, FP6>(sh, x, perm, planes, scales, zeros,
                                                                           partial, out, O, G, gps, row_blocks,
                                                                           swiglu, ra, x_lds, x_stage, split);
}

}  // namespace fx
