// Thin C-ABI driver around the reference's own LUT headers, compiled where they
// lie under /root/reference/src/fluxbin_style/csrc (see oracle/Makefile).  The
// output library goes to oracle/_ref/ and is only used by tests to check the C
// restatement in oracle/kernel_order.c bit-for-bit.  No reference source is
// copied here: the headers are included from the reference tree at build time.
#include "lut8_unsigned.cuh"
#include "lut8.cuh"

extern "C" void ref_build_unsigned_table(const float* values, float* table) {
  for (unsigned lane = 0; lane < 32; ++lane)
    fluxbin_w3_lut::build_lane_unsigned(table, values, lane);
}

extern "C" void ref_build_signed_table(const float* values, float* table) {
  for (unsigned lane = 0; lane < 32; ++lane)
    fluxbin_lut::build_lane(table, values, lane);
}

extern "C" unsigned ref_pattern(unsigned word) { return fluxbin_lut::pattern(word); }
