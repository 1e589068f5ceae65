// Instantiations of the W3 LUT GEMV for blocks of 8 activation row(s).
#include "w3_lut_inst.h"

namespace fx {
bool dispatch_lut_m8(int rpt, int xdt, int sdt, bool dec, const LutArgs& a, dim3 grid,
                     hipStream_t s) {
  return dispatch_rpt<8>(rpt, xdt, sdt, dec, a, grid, s);
}
}  // namespace fx
