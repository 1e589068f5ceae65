// Instantiations of the shared-staging field-layout kernel for fp16 activations.
#include "w3_fields_wide.h"

namespace fx {
bool dispatch_fields_wide_f16(const WidePlan& p, int sdt, int mode, const MfmaArgs& a, dim3 grid, hipStream_t s) {
  return dispatch_fields_wide_xdt<kF16>(p, sdt, mode, a, grid, s);
}
}  // namespace fx
