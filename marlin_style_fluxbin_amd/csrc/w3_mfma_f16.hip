// Instantiations of the MFMA W3 GEMV for fp16 activations.
#include "w3_mfma_inst.h"

namespace fx {
bool dispatch_mfma_f16(int nw, int tr, int mb, int sdt, const MfmaArgs& a, dim3 grid,
                       hipStream_t s) {
  return mfma_dispatch<kF16>(nw, tr, mb, sdt, a, grid, s);
}
}  // namespace fx
