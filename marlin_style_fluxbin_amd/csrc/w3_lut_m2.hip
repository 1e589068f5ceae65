// Instantiations of the W3 LUT GEMV for blocks of 2 activation row(s).
#include "w3_lut_inst.h"

namespace fx {
bool dispatch_lut_m2(int rpt, int xdt, int sdt, bool dec, const LutArgs& a, dim3 grid,
                     hipStream_t s) {
  return dispatch_rpt<2>(rpt, xdt, sdt, dec, a, grid, s);
}
}  // namespace fx
