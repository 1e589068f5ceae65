// Instantiations of the MFMA W3 GEMV for bf16 activations, and the x packer.
#include "w3_mfma_inst.h"

namespace fx {
bool dispatch_mfma_bf16(int nw, int tr, int mb, int sdt, const MfmaArgs& a, dim3 grid,
                        hipStream_t s) {
  return mfma_dispatch<kBF16>(nw, tr, mb, sdt, a, grid, s);
}

bool launch_xprep(int xdt, const uint16_t* x, const int16_t* perm, uint16_t* xs, float* sx,
                  int* fe, int K, int mb, hipStream_t s) {
  if (xdt == kBF16)
    hipLaunchKernelGGL(w3_xprep_kernel<kBF16>, dim3((K / 128 + 3) / 4, mb), dim3(256), 0, s, x, perm, xs, sx, fe, K, mb);
  else if (xdt == kF16)
    hipLaunchKernelGGL(w3_xprep_kernel<kF16>, dim3((K / 128 + 3) / 4, mb), dim3(256), 0, s, x, perm, xs, sx, fe, K, mb);
  else
    return false;
  return true;
}
}  // namespace fx
