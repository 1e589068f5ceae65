// Instantiations of the MFMA W3 GEMV: bf16 activations, 1 row tile(s) per wave, identity column order.
#include "w3_mfma_inst.h"

namespace fx {
bool dispatch_mfma_bf16_t1(int nw, int pd, int mb, int sdt, const MfmaArgs& a, dim3 grid,
                          hipStream_t s) {
  return mfma_dispatch<1, false, kBF16>(nw, pd, mb, sdt, a, grid, s);
}
}  // namespace fx
