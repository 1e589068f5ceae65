// Template launch/dispatch bodies for the MFMA W3 GEMV instantiation units.
#pragma once
#include "w3_mfma.hip"
#include "w3_mfma_launch.h"

namespace fx {

template <int NW, int PD, int MB, int RT, bool PERM, int XDT, int SDT>
void launch_mfma(const MfmaArgs& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((w3_mfma_kernel<NW, PD, MB, RT, PERM, XDT, SDT>), grid, dim3(NW * 64),
                     PERM ? x_lds_bytes(a, MB) : 0, s, a.x, a.perm, a.planes, a.scales, a.zeros, a.partial,
                     a.out, a.O, a.G, a.gps, a.row_blocks, a.swiglu, a.res, PERM ? a.x_lds : 0, a.batch);
}

template <int NW, int PD, int MB, int RT, bool PERM, int XDT>
bool mfma_sdt(int sdt, const MfmaArgs& a, dim3 g, hipStream_t s) {
  if (sdt == kBF16) { launch_mfma<NW, PD, MB, RT, PERM, XDT, kBF16>(a, g, s); return true; }
  if (sdt == kF16) { launch_mfma<NW, PD, MB, RT, PERM, XDT, kF16>(a, g, s); return true; }
  return false;
}

template <int NW, int PD, int RT, bool PERM, int XDT>
bool mfma_mb(int mb, int sdt, const MfmaArgs& a, dim3 g, hipStream_t s) {
  switch (mb) {
    case 1: return mfma_sdt<NW, PD, 1, RT, PERM, XDT>(sdt, a, g, s);
    case 2: return mfma_sdt<NW, PD, 2, RT, PERM, XDT>(sdt, a, g, s);
    case 4: return mfma_sdt<NW, PD, 4, RT, PERM, XDT>(sdt, a, g, s);
    case 8: return mfma_sdt<NW, PD, 8, RT, PERM, XDT>(sdt, a, g, s);
    default: return false;
  }
}

template <int RT, bool PERM, int XDT>
bool mfma_dispatch(int nw, int pd, int mb, int sdt, const MfmaArgs& a, dim3 g, hipStream_t s) {
#define FX_MFMA_CASE(W, P) \
  if (nw == W && pd == P) return mfma_mb<W, P, RT, PERM, XDT>(mb, sdt, a, g, s);
  FX_MFMA_CASE(4, 1) FX_MFMA_CASE(4, 2)
  FX_MFMA_CASE(8, 1) FX_MFMA_CASE(8, 2)
#undef FX_MFMA_CASE
  return false;
}

}  // namespace fx
