// Launch plumbing for the two-base binary-basis GEMV (two_base.hip), shared with
// the C ABI.
#pragma once
#include "common.h"
#include "w3_mfma_launch.h"  // ResidualArgs: the decoder residual stream around a GEMV

namespace fx {

// Rank-one two-base payload with salient columns, batch 1:
//   y[o] = s_r[o] (a1[o] (B1[o,:] . u) + a2[o] (B2[o,:] . u)) + sum_j sal[o,j] x[idx[j]],
//   u[k] = t_c[k] x[k],  B in {-1, +1} stored as bits (1 = +1).
struct RankOneArgs {
  const uint16_t* x;       // [K] activations (fp16 / bf16)
  const uint8_t* planes;   // [G, O, 2, 16] sign bits, bit j of byte c = column 128 g + 8 c + j
  const uint16_t* coef;    // fp16 [2, O]: a1, a2
  const uint16_t* srow;    // fp16 [O]
  const uint16_t* tcol;    // fp16 [K]
  const uint16_t* sal;     // bf16 [O, S] (null when S == 0)
  const int32_t* sal_idx;  // [S] column indices
  float* partial;          // null: write out directly (single K split)
  uint16_t* out;           // [O]
  int O, G, S, gps;
  int row_blocks;  // ceil(O / (16 * tiles)); the grid is (row_blocks, K splits)
};

constexpr int kRankOneMaxBatches = 24;  // four-group batches one workgroup stages (48 KB LDS)
constexpr int kRankOneMaxUnits = 4;     // staging units (8 columns) per thread

// Dynamic LDS of one workgroup: 2 KB per staged four-group batch.
inline size_t rank_one_lds_bytes(int gps) { return size_t(gps / 4) * 2048; }

// tiles 16-row tiles per workgroup, kparts waves per tile splitting the K range,
// pd batches of sign loads in flight per wave; instantiated (tiles, kparts, pd):
// (1,4,1..2) (1,8,1..3) (2,4,2) (2,8,2) (3,4,1..2) (4,4,2).  False otherwise.
bool dispatch_rank_one(int xdt, int tiles, int kparts, int pd, const RankOneArgs& a, dim3 grid,
                       hipStream_t s);

}  // namespace fx

namespace fx {

// Hybrid g128/s8 payload in the reference's planar deployment layout, batch 1:
//   y[o] = sum_g sum_b rows[g,o,b] (B_b[o, g, :] . (x_g * cols[g, :, b]))
//        + sum_g sum_b srows[g,o,b] (R_b[o, g, :] . (x[128 g + idx[g, :]] * scols[g, :, b]))
// with B, R in {-1, +1} stored as bits (1 = +1).
constexpr int kHybridMaxSegments = 4;  // layouts one launch may concatenate along O (q|k|v, gate|up)

struct HybridArgs {
  const uint16_t* x;       // [K] activations (fp16 / bf16)
  const uint8_t* codes;    // [G, O, 2, 16]: bit j of byte c of base b = column 8 c + j
  const float* rows;       // [G, O, 2]
  const float* cols;       // [G, 128, 2]        of segment 0
  const int16_t* idx;      // [G, 8] refinement columns inside each group, segment 0
  const uint8_t* scodes;   // [G, O, 2, 1]: bit j = refinement column j
  const float* srows;      // [G, O, 2]
  const float* scols;      // [G, 8, 2]          of segment 0
  float* partial;          // null: write out directly (single K split)
  uint16_t* out;           // [O]
  int O, G, gps;
  int row_blocks;  // ceil(O / (16 * tiles)); the grid is (row_blocks, K splits)
  // Rows [seg_start[s], seg_start[s + 1]) use segment s's column-side arrays
  // (segment 0: cols / idx / scols above); every start is a multiple of the
  // workgroup's 16 * tiles rows, so a workgroup lies in one segment.
  int nseg;
  int seg_start[kHybridMaxSegments];
  const float* seg_cols[kHybridMaxSegments];
  const int16_t* seg_idx[kHybridMaxSegments];
  const float* seg_scols[kHybridMaxSegments];
  // Decoder residual stream (one K split): res.ep_residual set: out =
  // round(residual + round(y)) and per-16-row sums of out^2 into res.ep_partial;
  // the normalising instantiations read x = round(w * round(h * rsqrt(sum(
  // res.pro_partial) / K + eps))), the RMSNorm of h, as the W3 kernel does.
  ResidualArgs res;
};

constexpr int kHybridMaxBatches = 36;  // four-group batches one workgroup stages (117 KB LDS)

// Dynamic LDS of one workgroup: main digit operands (2 KB), refinement operands
// (256 B) and activations (1 KB) per staged batch.
inline size_t hybrid_lds_bytes(int gps) { return size_t(gps / 4) * (2048 + 256 + 1024); }

// Activation prologues of the hybrid GEMV: plain x; normalising (a.x holds h,
// a.res the partials, weight and eps of its RMSNorm); SwiGLU (a.x holds gate |
// up, 2K values, and the GEMV reads round(round(silu(gate)) * up), as the SwiGLU
// kernel computes it).
enum : int { kHyProPlain = 0, kHyProNorm = 1, kHyProSwiglu = 2 };

// Instantiated (tiles, kparts): (1,4) (1,8) (2,4) (3,4) (4,2) (5,2) (6,2), each
// with every prologue.  False otherwise.
bool dispatch_hybrid(int xdt, int tiles, int kparts, int prologue, const HybridArgs& a, dim3 grid, hipStream_t s);

}  // namespace fx
