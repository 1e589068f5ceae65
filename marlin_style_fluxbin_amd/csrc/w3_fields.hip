// The W3 field layout: its bind-time repack from the reference's planar payload,
// and the MFMA GEMV instantiations that read it (one activation row; identity or
// permuted column order, the normalising prologue identity only).  Layout: same array shape as the planes, [G, 3, O, 16] bytes =
// per (group, row) three member rows of four little-endian 32-bit words.  The
// codes of sorted columns 32 w + t (t < 32) sit in word w of the members:
// i = t / 2, h = t % 2; for i < 15 the code occupies bits [16 h + 3 f, +3) of
// member i / 5 (f = i % 5); for i = 15 its bit k occupies bit 15 + 16 h of
// member k.  Three bits per code, as the planes.
#include "w3_mfma_inst.h"

namespace fx {

// One thread per (group, row).  Plane 2 is stored inverted in the planes.
__global__ __launch_bounds__(256) void w3_planes_to_fields_kernel(const uint8_t* __restrict__ planes,
                                                                  uint8_t* __restrict__ fields, int O, int G) {
  const long idx = long(blockIdx.x) * 256 + threadIdx.x;  // g * O + o
  if (idx >= long(G) * O) return;
  const long g = idx / O, o = idx % O;
  const u32x4_t* src = reinterpret_cast<const u32x4_t*>(planes);
  const u32x4_t p0 = src[(g * 3 + 0) * O + o], p1 = src[(g * 3 + 1) * O + o], p2 = src[(g * 3 + 2) * O + o];
  u32x4_t f[3];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const unsigned b0 = p0[w], b1 = p1[w], b2 = ~p2[w];
    unsigned m[3] = {0u, 0u, 0u};
#pragma unroll
    for (int t = 0; t < 32; ++t) {
      const unsigned q = ((b0 >> t) & 1u) | (((b1 >> t) & 1u) << 1) | (((b2 >> t) & 1u) << 2);
      const int i = t >> 1, h = t & 1;
      if (i < 15) {
        m[i / 5] |= q << (16 * h + 3 * (i % 5));
      } else {
#pragma unroll
        for (int k = 0; k < 3; ++k) m[k] |= ((q >> k) & 1u) << (15 + 16 * h);
      }
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) f[k][w] = m[k];
  }
  u32x4_t* dst = reinterpret_cast<u32x4_t*>(fields);
#pragma unroll
  for (int k = 0; k < 3; ++k) dst[(g * 3 + k) * O + o] = f[k];
}

void launch_planes_to_fields(const uint8_t* planes, uint8_t* fields, int O, int G, hipStream_t s) {
  const long n = long(G) * O;
  hipLaunchKernelGGL(w3_planes_to_fields_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, planes, fields,
                     O, G);
}

// fp6 layout (the gfx950 scaled f8f6f4 matrix instruction's fp6 e2m3 A operand):
// bytes of the planes' size ordered [G / 4, O, k-block kb (4), group slot (4), 3
// words].  Field e of A lane block kb multiplies group column
// 32 (2 (kb % 2) + e / 16) + 16 (kb / 2) + e % 16 (the instruction's pairing with
// fp8 B elements); mantissa bit j of field e is bit 6 e + j of six registers R0..R5,
// expanded from the three words s0..s2 as R0 = s0 & M0, R2 = (s0 >> 1) & M2,
// R3 = s1 & M0, R5 = (s1 >> 1) & M2, R1 = s2 & M1, R4 = (s2 >> 3 | bits 29, 30
// from s2 bits 1, 2) & M1 (expand_fp6).  fp6_stored_bit inverts that map.
__device__ __forceinline__ int fp6_stored_bit(int reg, int bit) {
  if (reg == 0 || reg == 3) return (reg / 3) * 32 + bit;
  if (reg == 2 || reg == 5) return (reg == 2 ? 0 : 32) + bit + 1;
  if (reg == 1) return 64 + bit;
  return 64 + ((bit == 29 || bit == 30) ? bit - 28 : bit + 3);
}

// One thread per (batch of 4 groups, row, k-block): its 48 output bytes.
__global__ __launch_bounds__(256) void w3_planes_to_fp6_kernel(const uint8_t* __restrict__ planes,
                                                               uint8_t* __restrict__ out, int O, int G) {
  const long idx = long(blockIdx.x) * 256 + threadIdx.x;  // (bt * O + o) * 4 + kb
  if (idx >= long(G / 4) * O * 4) return;
  const int kb = int(idx & 3);
  const long bo = idx >> 2;
  const long bt = bo / O, o = bo % O;
  const u32x4_t* src = reinterpret_cast<const u32x4_t*>(planes);
  unsigned words[12];
#pragma unroll
  for (int i = 0; i < 12; ++i) words[i] = 0u;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const long g = 4 * bt + b;
    const u32x4_t p0 = src[(g * 3 + 0) * O + o], p1 = src[(g * 3 + 1) * O + o], p2 = src[(g * 3 + 2) * O + o];
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const int col = 32 * (2 * (kb & 1) + e / 16) + 16 * (kb >> 1) + e % 16;  // kb is per-thread
      const int w = col >> 5, t = col & 31;
      const unsigned b0 = (p0[w] >> t) & 1u, b1 = (p1[w] >> t) & 1u, b2 = (~p2[w] >> t) & 1u;
      const unsigned bits[3] = {b0, b1, b2};
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const int pos = 6 * e + j;
        const int sb = fp6_stored_bit(pos >> 5, pos & 31);
        words[3 * b + (sb >> 5)] |= bits[j] << (sb & 31);
      }
    }
  }
  u32x4_t* dst = reinterpret_cast<u32x4_t*>(out + idx * 48);
  dst[0] = u32x4_t{words[0], words[1], words[2], words[3]};
  dst[1] = u32x4_t{words[4], words[5], words[6], words[7]};
  dst[2] = u32x4_t{words[8], words[9], words[10], words[11]};
}

void launch_planes_to_fp6(const uint8_t* planes, uint8_t* out, int O, int G, hipStream_t s) {
  const long n = long(G / 4) * O * 4;
  hipLaunchKernelGGL(w3_planes_to_fp6_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, planes, out, O, G);
}

// fp6-layout GEMVs: one bf16 activation row, sorted columns, O % 16 == 0 (vector
// scale loads), K % 512 == 0; the normalising prologue with two row tiles per
// wave, as the field layout's.
template <int NW, int SDT, bool NORMIN>
void launch_fp6(const MfmaArgs& a, dim3 grid, hipStream_t s) {
  constexpr int RT = NORMIN ? 2 : 1;
  hipLaunchKernelGGL((w3_mfma_kernel<NW, 1, 1, RT, false, kBF16, SDT, NORMIN, 1, true, false, true>), grid,
                     dim3(NW * 64), 0, s, a.x, a.perm, a.planes, a.scales, a.zeros, a.partial, a.out, a.O, a.G, a.gps,
                     a.row_blocks, a.swiglu, a.res, 0, a.batch);
}

bool dispatch_mfma_fp6(int nw, bool normin, int sdt, const MfmaArgs& a, dim3 grid, hipStream_t s) {
#define FX_FP6_CASE(W, S)                                      \
  if (nw == W && sdt == S) {                                   \
    if (normin) launch_fp6<W, S, true>(a, grid, s);            \
    else launch_fp6<W, S, false>(a, grid, s);                  \
    return true;                                               \
  }
  FX_FP6_CASE(4, kBF16) FX_FP6_CASE(4, kF16) FX_FP6_CASE(8, kBF16) FX_FP6_CASE(8, kF16)
#undef FX_FP6_CASE
  return false;
}

// Plain and normalising kernels each come as the vector (O % 4 == 0) and the
// element-wise scale-load form, so the decode shapes' kernel carries registers
// for its own path only.
// The normalising prologue with vector scale loads runs two 16-row tiles per
// wave (fields_row_tiles): each normalised, staged batch of activations then
// feeds 32 rows, which halves the per-row cost of the RMSNorm arithmetic
// (24576 x 4096 gate|up with SwiGLU 11.6 -> 10.7 us, 6144 x 4096 5.5 -> 5.1 us).
// PERM (plain and residual forms only): sorted column k reads x[perm[k]], one
// 2-byte gather per value in the staging, as the planar kernel's permuted form.
template <int NW, int XDT, int SDT, bool NORMIN, bool PERM>
void launch_fields(const MfmaArgs& a, dim3 grid, hipStream_t s) {
  if (a.O % 4 == 0) {
    constexpr int RT = NORMIN ? 2 : 1;  // fields_row_tiles
    hipLaunchKernelGGL((w3_mfma_kernel<NW, 1, 1, RT, PERM, XDT, SDT, NORMIN, 1, true>), grid, dim3(NW * 64),
                       PERM ? x_lds_bytes(a, 1) : 0, s, a.x, a.perm, a.planes, a.scales, a.zeros, a.partial, a.out,
                       a.O, a.G, a.gps, a.row_blocks, a.swiglu, a.res, PERM ? a.x_lds : 0, a.batch);
  } else {
    hipLaunchKernelGGL((w3_mfma_kernel<NW, 1, 1, 1, PERM, XDT, SDT, NORMIN, 2, true>), grid, dim3(NW * 64),
                       PERM ? x_lds_bytes(a, 1) : 0, s, a.x, a.perm, a.planes, a.scales, a.zeros, a.partial, a.out,
                       a.O, a.G, a.gps, a.row_blocks, a.swiglu, a.res, PERM ? a.x_lds : 0, a.batch);
  }
}

bool dispatch_mfma_fields(int nw, bool normin, int xdt, int sdt, const MfmaArgs& a, dim3 grid, hipStream_t s) {
  if (normin && a.perm) return false;
#define FX_FIELDS_CASE(W, X, S)                                                     \
  if (nw == W && xdt == X && sdt == S) {                                            \
    if (normin) launch_fields<W, X, S, true, false>(a, grid, s);                    \
    else if (a.perm) launch_fields<W, X, S, false, true>(a, grid, s);               \
    else launch_fields<W, X, S, false, false>(a, grid, s);                          \
    return true;                                                                    \
  }
  FX_FIELDS_CASE(4, kBF16, kBF16) FX_FIELDS_CASE(4, kBF16, kF16) FX_FIELDS_CASE(4, kF16, kBF16)
  FX_FIELDS_CASE(4, kF16, kF16) FX_FIELDS_CASE(8, kBF16, kBF16) FX_FIELDS_CASE(8, kBF16, kF16)
  FX_FIELDS_CASE(8, kF16, kBF16) FX_FIELDS_CASE(8, kF16, kF16)
#undef FX_FIELDS_CASE
  return false;
}

}  // namespace fx
