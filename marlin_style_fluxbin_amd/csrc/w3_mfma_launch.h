// Launch plumbing for the MFMA W3 GEMV (w3_mfma.hip), shared by its
// instantiation units (w3_mfma_bf16.hip, w3_mfma_f16.hip) and the C ABI.
#pragma once
#include "common.h"

namespace fx {

struct MfmaArgs {
  const uint8_t* planes;
  const uint16_t* scales;
  const uint8_t* zeros;
  const uint16_t* xs;
  const float* sx;
  const int* fe;
  float* partial;  // null: write out directly (single K split)
  uint16_t* out;
  int O, G, gps;
};

bool dispatch_mfma_bf16(int nw, int tr, int mb, int sdt, const MfmaArgs& a, dim3 grid,
                        hipStream_t s);
bool dispatch_mfma_f16(int nw, int tr, int mb, int sdt, const MfmaArgs& a, dim3 grid,
                       hipStream_t s);
// x [mb, K] -> packed B operands, per-group sums, exponents (one launch)
bool launch_xprep(int xdt, const uint16_t* x, const int16_t* perm, uint16_t* xs, float* sx,
                  int* fe, int K, int mb, hipStream_t s);

}  // namespace fx
