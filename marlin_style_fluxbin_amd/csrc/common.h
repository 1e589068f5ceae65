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

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t(0x7fc0u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return float(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, _Float16(f));
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

}  // namespace fx
