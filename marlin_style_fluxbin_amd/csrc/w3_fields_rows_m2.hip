// Instantiations of the shared-staging field-layout kernel for 2 activation rows.
#include "w3_fields_wide.h"

namespace fx {
bool dispatch_fields_rows_m2(const WidePlan& p, int xdt, int sdt, const MfmaArgs& a, int M, dim3 grid, hipStream_t s) {
  if (xdt == kBF16) return dispatch_fields_rows_mb<2, kBF16>(p, sdt, a, M, grid, s);
  if (xdt == kF16) return dispatch_fields_rows_mb<2, kF16>(p, sdt, a, M, grid, s);
  return false;
}
}  // namespace fx
