// MFMA W3 GEMV instantiations with decoded_bf16 arithmetic: the reference's +-3
// correction (csrc/w3_lut.cu:105-122) as a second MFMA chain on transformed planes
// (w3_mfma.hip, corrected_planes).  One activation row, one 16-row tile and one
// batch in flight per wave, bf16 scales, planar payload; identity or permuted order.
#include "w3_mfma_inst.h"

namespace fx {

template <int NW, bool PERM, int XDT>
void launch_mfma_corr(const MfmaArgs& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((w3_mfma_kernel<NW, 1, 1, 1, PERM, XDT, kBF16, false, 0, false, true>), grid, dim3(NW * 64),
                     PERM ? x_lds_bytes(a, 1) : 0, s, a.x, a.perm, a.planes, a.scales, a.zeros, a.partial, a.out, a.O,
                     a.G, a.gps, a.row_blocks, a.swiglu, a.res, PERM ? a.x_lds : 0, a.batch);
}

bool dispatch_mfma_corr(int nw, int xdt, const MfmaArgs& a, dim3 grid, hipStream_t s) {
  const bool p = a.perm != nullptr;
#define FX_CORR_CASE(W, X)                                  \
  if (nw == W && xdt == X) {                                \
    if (p) launch_mfma_corr<W, true, X>(a, grid, s);        \
    else launch_mfma_corr<W, false, X>(a, grid, s);         \
    return true;                                            \
  }
  FX_CORR_CASE(4, kBF16) FX_CORR_CASE(4, kF16) FX_CORR_CASE(8, kBF16) FX_CORR_CASE(8, kF16)
#undef FX_CORR_CASE
  return false;
}

}  // namespace fx
