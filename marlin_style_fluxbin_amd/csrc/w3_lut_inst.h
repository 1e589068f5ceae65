// Template launch/dispatch bodies for the per-M instantiation units.
#pragma once
#include "w3_lut_launch.h"
#include "w3_lut.hip"

namespace fx {

template <int M, int RPT, int XDT, int SDT, bool DEC>
void launch_lut(const LutArgs& a, dim3 grid, hipStream_t stream) {
  hipLaunchKernelGGL((w3_lut_kernel<M, RPT, XDT, SDT, DEC>), grid, dim3(kLutThreads), 0,
                     stream, a.x, a.planes, a.scales, a.zeros, a.perm, a.partial, a.out, a.O,
                     a.G, a.gps, a.mode);
}

template <int M, int RPT, int XDT>
bool dispatch_sdt(int sdt, bool dec, const LutArgs& a, dim3 grid, hipStream_t s) {
  if (sdt == kBF16) {
    if (dec) launch_lut<M, RPT, XDT, kBF16, true>(a, grid, s);
    else launch_lut<M, RPT, XDT, kBF16, false>(a, grid, s);
    return true;
  }
  if (sdt == kF16 && !dec) {
    launch_lut<M, RPT, XDT, kF16, false>(a, grid, s);
    return true;
  }
  return false;
}

template <int M, int RPT>
bool dispatch_xdt(int xdt, int sdt, bool dec, const LutArgs& a, dim3 grid, hipStream_t s) {
  if (xdt == kBF16) return dispatch_sdt<M, RPT, kBF16>(sdt, dec, a, grid, s);
  if (xdt == kF16) return dispatch_sdt<M, RPT, kF16>(sdt, dec, a, grid, s);
  return false;
}

template <int M>
bool dispatch_rpt(int rpt, int xdt, int sdt, bool dec, const LutArgs& a, dim3 grid,
                  hipStream_t s) {
  switch (rpt) {
    case 1: return dispatch_xdt<M, 1>(xdt, sdt, dec, a, grid, s);
    case 2: return dispatch_xdt<M, 2>(xdt, sdt, dec, a, grid, s);
    case 4: return dispatch_xdt<M, 4>(xdt, sdt, dec, a, grid, s);
    default: return false;
  }
}

}  // namespace fx
