// MFMA W3 GEMV instantiations whose staging normalises the activation row
// (RMSNorm from the previous GEMV's tile partial sums).
#include "w3_mfma_inst.h"

namespace fx {

// Separate kernels for the vector (O % 4 == 0, the decode shapes) and element
// scale / zero-point loads, so the vector one is allocated registers for its
// own path only.
template <int NW, int XDT, int SDT>
void launch_mfma_normin(const MfmaArgs& a, dim3 grid, hipStream_t s) {
  if (a.O % 4 == 0)
    hipLaunchKernelGGL((w3_mfma_kernel<NW, 1, 1, 1, false, XDT, SDT, true, 1>), grid, dim3(NW * 64), 0, s, a.x,
                       a.perm, a.planes, a.scales, a.zeros, a.partial, a.out, a.O, a.G, a.gps, a.row_blocks,
                       a.swiglu, a.res, 0, a.batch);
  else
    hipLaunchKernelGGL((w3_mfma_kernel<NW, 1, 1, 1, false, XDT, SDT, true, 2>), grid, dim3(NW * 64), 0, s, a.x,
                       a.perm, a.planes, a.scales, a.zeros, a.partial, a.out, a.O, a.G, a.gps, a.row_blocks,
                       a.swiglu, a.res, 0, a.batch);
}

bool dispatch_mfma_normin(int nw, int xdt, int sdt, const MfmaArgs& a, dim3 grid, hipStream_t s) {
#define FX_NORMIN_CASE(W, X, S) \
  if (nw == W && xdt == X && sdt == S) { launch_mfma_normin<W, X, S>(a, grid, s); return true; }
  FX_NORMIN_CASE(4, kBF16, kBF16) FX_NORMIN_CASE(4, kBF16, kF16) FX_NORMIN_CASE(4, kF16, kBF16)
  FX_NORMIN_CASE(4, kF16, kF16) FX_NORMIN_CASE(8, kBF16, kBF16) FX_NORMIN_CASE(8, kBF16, kF16)
  FX_NORMIN_CASE(8, kF16, kBF16) FX_NORMIN_CASE(8, kF16, kF16)
#undef FX_NORMIN_CASE
  return false;
}

}  // namespace fx
