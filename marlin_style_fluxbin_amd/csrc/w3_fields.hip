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
