// Template launch/dispatch bodies for the MFMA W3 GEMV instantiation units.
#pragma once
#include <mutex>

#include "w3_mfma.hip"
#include "w3_mfma_launch.h"

namespace fx {

template <int NW, int TR, int MB, int XDT, int SDT>
void launch_mfma(const MfmaArgs& a, dim3 grid, size_t lds, hipStream_t s) {
  static std::once_flag once;
  std::call_once(once, [] {
    // allow the full gfx950 LDS (160 KiB) for the dynamic allocation
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&w3_mfma_kernel<NW, TR, MB, XDT, SDT>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  });
  hipLaunchKernelGGL((w3_mfma_kernel<NW, TR, MB, XDT, SDT>), grid, dim3(NW * 64), lds, s, a.planes,
                     a.scales, a.zeros, a.xs, a.sx, a.fe, a.partial, a.out, a.O, a.G, a.gps);
}

template <int NW, int TR, int MB, int XDT>
bool mfma_sdt(int sdt, const MfmaArgs& a, dim3 g, size_t lds, hipStream_t s) {
  if (sdt == kBF16) { launch_mfma<NW, TR, MB, XDT, kBF16>(a, g, lds, s); return true; }
  if (sdt == kF16) { launch_mfma<NW, TR, MB, XDT, kF16>(a, g, lds, s); return true; }
  return false;
}

template <int NW, int TR, int XDT>
bool mfma_mb(int mb, int sdt, const MfmaArgs& a, dim3 g, size_t lds, hipStream_t s) {
  switch (mb) {
    case 1: return mfma_sdt<NW, TR, 1, XDT>(sdt, a, g, lds, s);
    case 2: return mfma_sdt<NW, TR, 2, XDT>(sdt, a, g, lds, s);
    case 4: return mfma_sdt<NW, TR, 4, XDT>(sdt, a, g, lds, s);
    default: return false;
  }
}

template <int XDT>
bool mfma_dispatch(int nw, int tr, int mb, int sdt, const MfmaArgs& a, dim3 g, size_t lds,
                   hipStream_t s) {
  if (nw == 2 && tr == 1) return mfma_mb<2, 1, XDT>(mb, sdt, a, g, lds, s);
  if (nw == 4 && tr == 1) return mfma_mb<4, 1, XDT>(mb, sdt, a, g, lds, s);
  if (nw == 4 && tr == 2) return mfma_mb<4, 2, XDT>(mb, sdt, a, g, lds, s);
  if (nw == 8 && tr == 1) return mfma_mb<8, 1, XDT>(mb, sdt, a, g, lds, s);
  if (nw == 8 && tr == 2) return mfma_mb<8, 2, XDT>(mb, sdt, a, g, lds, s);
  return false;
}

}  // namespace fx
