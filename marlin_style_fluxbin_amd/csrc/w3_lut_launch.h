// Launch plumbing shared by the per-M instantiation units (w3_lut_m*.hip) and
// the C ABI (capi.hip).
#pragma once
#include "common.h"

namespace fx {

struct LutArgs {
  const uint16_t* x;
  const uint8_t* planes;
  const uint16_t* scales;
  const uint8_t* zeros;
  const int16_t* perm;
  float* partial;
  uint16_t* out;
  int O, G, gps, mode;
};

// One instantiation unit per activation-row block (w3_lut_m{1,2,4,8}.hip).
bool dispatch_lut_m1(int rpt, int xdt, int sdt, bool dec, const LutArgs& a, dim3 grid, hipStream_t s);
bool dispatch_lut_m2(int rpt, int xdt, int sdt, bool dec, const LutArgs& a, dim3 grid, hipStream_t s);
bool dispatch_lut_m4(int rpt, int xdt, int sdt, bool dec, const LutArgs& a, dim3 grid, hipStream_t s);
bool dispatch_lut_m8(int rpt, int xdt, int sdt, bool dec, const LutArgs& a, dim3 grid, hipStream_t s);

inline bool dispatch_lut(int m_block, int rpt, int xdt, int sdt, bool dec, const LutArgs& a,
                         dim3 grid, hipStream_t s) {
  switch (m_block) {
    case 1: return dispatch_lut_m1(rpt, xdt, sdt, dec, a, grid, s);
    case 2: return dispatch_lut_m2(rpt, xdt, sdt, dec, a, grid, s);
    case 4: return dispatch_lut_m4(rpt, xdt, sdt, dec, a, grid, s);
    case 8: return dispatch_lut_m8(rpt, xdt, sdt, dec, a, grid, s);
    default: return false;
  }
}

}  // namespace fx
