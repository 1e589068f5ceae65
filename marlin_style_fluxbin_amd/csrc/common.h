// Shared device helpers for the gfx950 kernels: dtype codes, exact bf16/fp16
// conversions (round-to-nearest-even), wave64 reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fx {

// dtype codes shared with include/fluxbin_amd.h
enum : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(uint32_t(b) << 16);
}

// Round to nearest even in one instruction (v_cvt_pk_bf16_f32 on gfx950); NaN
// stays NaN (quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return float(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, _Float16(f));
}
// Two floats to fp16 (lo = a, hi = b), rounded as f32_to_f16_bits rounds each:
// one packed convert on gfx950 instead of two converts and an OR.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ unsigned f32x2_to_f16x2_bits(float a, float b) {
  return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2_t{a, b}, f16x2_t));
}

template <int DT>
__device__ __forceinline__ float to_f32(uint16_t bits) {
  if constexpr (DT == kBF16) return bf16_bits_to_f32(bits);
  else return f16_bits_to_f32(bits);
}

template <int DT>
__device__ __forceinline__ uint16_t from_f32(float v) {
  if constexpr (DT == kBF16) return f32_to_bf16_bits(v);
  else return f32_to_f16_bits(v);
}

// Round a float to the storage dtype and back (the rounding point of a cast).
template <int DT>
__device__ __forceinline__ float round_to(float v) {
  return to_f32<DT>(from_f32<DT>(v));
}

// round_to on two values at once: one packed convert (v_cvt_pk_bf16_f32 /
// v_cvt_pk_f16_f32 on gfx950) and the two widenings, the same bits as two
// round_to calls.
// round_pair_bits also returns the two stored values (a in the low half).
template <int DT>
__device__ __forceinline__ unsigned round_pair_bits(float& a, float& b) {
  typedef float f2_t __attribute__((ext_vector_type(2)));
  if constexpr (DT == kBF16) {
    typedef __bf16 b2_t __attribute__((ext_vector_type(2)));
    const unsigned p = __builtin_bit_cast(unsigned, __builtin_convertvector(f2_t{a, b}, b2_t));
    a = __uint_as_float(p << 16);
    b = __uint_as_float(p & 0xffff0000u);
    return p;
  } else {
    typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
    const h2_t h = __builtin_convertvector(f2_t{a, b}, h2_t);
    const f2_t w = __builtin_convertvector(h, f2_t);
    a = w.x;
    b = w.y;
    return __builtin_bit_cast(unsigned, h);
  }
}
template <int DT>
__device__ __forceinline__ void round_pair(float& a, float& b) {
  (void)round_pair_bits<DT>(a, b);
}

// Butterfly sum over the 64 lanes of a wavefront (xor shuffles lower to DPP /
// ds_swizzle on gfx950).  Every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, 64));
  return v;
}


// DPP lane moves within the 16-lane rows of a wavefront.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7 - i within each half row
constexpr int kDppMirror = 0x140;     // lane i <-> 15 - i within each row
constexpr int kDppRowShl4 = 0x104;    // lane i reads lane i + 4 of its row (0 past the row end)

// Sum / max over each 16-lane row; every lane of the row gets the same bits
// (each step adds a lane's value to its partner's, and both partners form the
// same commutative sum).
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_move<kDppXor1>(v);
  v += dpp_move<kDppXor2>(v);
  v += dpp_move<kDppHalfMirror>(v);
  v += dpp_move<kDppMirror>(v);
  return v;
}

// row16_max takes magnitudes only (non-negative, not NaN: every caller forms
// them with fmaxf from 0, which drops NaN).  Their bit patterns order as the
// values do, so an unsigned max of the bits is the float max -- one DPP-combined
// integer instruction per step, where a float max first canonicalises its DPP
// operand (three more instructions per step).
template <int CTRL>
__device__ __forceinline__ unsigned dpp_move_u(unsigned v) {
  return unsigned(__builtin_amdgcn_update_dpp(0, int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_max(float v) {
  unsigned u = __float_as_uint(v);
  u = max(u, dpp_move_u<kDppXor1>(u));
  u = max(u, dpp_move_u<kDppXor2>(u));
  u = max(u, dpp_move_u<kDppHalfMirror>(u));
  u = max(u, dpp_move_u<kDppMirror>(u));
  return __uint_as_float(u);
}

// Max over the 64 lanes of values that are never NaN (attention scores: finite
// or -inf) through order-preserving unsigned keys (a non-negative float with its
// sign bit set, a negative one with every bit flipped): an integer max per step,
// where fmaxf first canonicalises the shuffled operand.  Equal to wave_max on
// such values (up to the sign of a zero maximum).
__device__ __forceinline__ unsigned float_order_key(float f) {
  const unsigned b = __float_as_uint(f);
  return b ^ (unsigned(int(b) >> 31) | 0x80000000u);
}
__device__ __forceinline__ float float_from_order_key(unsigned k) {
  return __uint_as_float(k ^ (int(k) < 0 ? 0x80000000u : 0xffffffffu));
}
__device__ __forceinline__ float wave_max_not_nan(float v) {
  unsigned k = float_order_key(v);
  // within each 16-lane row by DPP (one combined instruction per step), then
  // across the four rows
  k = max(k, dpp_move_u<kDppXor1>(k));
  k = max(k, dpp_move_u<kDppXor2>(k));
  k = max(k, dpp_move_u<kDppHalfMirror>(k));
  k = max(k, dpp_move_u<kDppMirror>(k));
  k = max(k, unsigned(__shfl_xor(int(k), 16, 64)));
  k = max(k, unsigned(__shfl_xor(int(k), 32, 64)));
  return float_from_order_key(k);
}

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
// lane_index * rows for a lane index below 4 and rows <= 3 * 2^20 (every entry
// point checks O <= 2^20 before a launch): both factors and the product fit 24
// bits, so the full-rate 24-bit multiply gives the 32-bit product
// (v_mul_lo_u32 runs at quarter rate).
__device__ __forceinline__ int lane_times_rows(int lane_index, int rows) {
  return int(__umul24(unsigned(lane_index), unsigned(rows)));
}


// Index of the calling wave in its workgroup, as a wave-uniform (scalar) value:
// the compiler cannot tell that threadIdx.x / 64 is the same across a wave, and
// treats everything derived from it (batch counts, loop guards, addresses) as
// divergent -- vector compares, exec-masked branches, and loads sunk behind
// guards that convergent cross-lane operations cannot follow.
__device__ __forceinline__ int wave_index() { return __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6); }

// Sum over the 64 lanes of a wave (DPP within rows of 16, then lanes 16 and 32
// apart); every lane gets the same bits.
__device__ __forceinline__ float wave_total(float v) {
  v = row16_sum(v);
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

// RMSNorm reductions run over 512-element batches: lane l of the wave serving
// batch b holds elements [8 (64 b + l), +8), sums their squares with fused
// multiply-adds in element order, and the batch total is wave_total of that.
// The batch totals are added in batch order.
constexpr int kNormBatch = 512;
template <int DT>
__device__ __forceinline__ float sum_sq8(const u32x4_t& v) {
  float ss = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float lo = to_f32<DT>(uint16_t(v[w])), hi = to_f32<DT>(uint16_t(v[w] >> 16));
    ss = fmaf(lo, lo, ss);
    ss = fmaf(hi, hi, ss);
  }
  return ss;
}

// Buffer resource over [base, base + bytes): loads at offsets past the end
// return zero instead of touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_resource(const void* base, size_t bytes) {
  // (a 64-bit unsigned compare has no scalar form on gfx9: as a vector compare
  // it put the descriptor in VGPRs, and every load through it in a waterfall loop)
  const int records = (bytes >> 31) != 0 ? 0x7fffffff : int(bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), short(0), records, 0x00020000);
}

// The same over a size below 2 GiB (the GEMV payload arrays and activations:
// every entry point checks their sizes before a launch), formed in 32-bit
// arithmetic, so no clamp and no compare reach the vector unit.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_resource_2g(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), short(0), int(bytes), 0x00020000);
}

__device__ __forceinline__ u32x4_t load_b128(__amdgpu_buffer_rsrc_t r, int offset, int soffset) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, offset, soffset, 0));
}

constexpr int kOutOfRange = int(0x80000000u);  // > every record count: loads return 0

// Streaming load of weights that are read exactly once per launch: aux bit 1 is
// the non-temporal policy, so the lines do not displace the activations and
// per-row metadata that other workgroups still read from L2 (measured 0.3-0.7 us
// per GEMV at the Qwen3-8B shapes on MI355X).
__device__ __forceinline__ u32x4_t load_b128_stream(__amdgpu_buffer_rsrc_t r, int offset, int soffset) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, offset, soffset, 2));
}

// Workgroup x index -> row block, so that the workgroups one XCD runs (hardware
// dispatch deals consecutive workgroup ids round-robin over MI355X's 8 XCDs)
// take consecutive row blocks and share the per-row metadata cache lines in
// that XCD's L2.  A bijection for any grid size; the XCD count is a compile-time
// constant (shifts and masks, no integer division ahead of the first load), and
// a partition mode that exposes fewer XCDs only loses the locality.
constexpr int kXcdCount = 8;
__device__ __forceinline__ int xcd_local_index8(unsigned linear, unsigned total) {
  const unsigned xcd = linear % kXcdCount, local = linear / kXcdCount;
  const unsigned q = total / kXcdCount, rem = total % kXcdCount;
  return int(xcd < rem ? xcd * (q + 1) + local : rem * (q + 1) + (xcd - rem) * q + local);
}

}  // namespace fx
