// Instantiations of the MFMA W3 GEMV: f16 activations, 2 row tile(s) per wave, identity column order.
#include "w3_mfma_inst.h"

namespace fx {
bool dispatch_mfma_f16_t2(int nw, int pd, int mb, int sdt, const MfmaArgs& a, dim3 grid,
                          hipStream_t s) {
  return mfma_dispatch<2, false, kF16>(nw, pd, mb, sdt, a, grid, s);
}
}  // namespace fx
