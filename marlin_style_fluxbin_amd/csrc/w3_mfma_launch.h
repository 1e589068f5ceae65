// Launch plumbing for the MFMA W3 GEMV (w3_mfma.hip), shared by its
// instantiation units (w3_mfma_{bf16,f16}_t{1,2}[_perm].hip) and the C ABI.
#pragma once
#include "common.h"

namespace fx {

// Decoder-layer residual stream around a one-row GEMV (one K split, one tile per
// wave):
// * epilogue (ep_residual set): out = round(residual + round(y)) -- the layer's
//   residual add -- and ep_partial[tile] = sum over the tile's 16 rows of out^2;
// * prologue (NORMIN instantiations): x holds h (such an epilogue's out); the
//   GEMV reads x = round(weight * round(h * rsqrt(sum(pro_partial) / K + eps))),
//   the RMSNorm of h, from the pro_n tile partials.
// * output order for a column-permuted consumer (ep_index set): the residual
//   epilogue also writes row o of out to ep_sorted[ep_index[o]], and the SwiGLU
//   epilogue writes value r to out[ep_index[r]] instead of out[r].  With
//   ep_index = the inverse of the next GEMV's permutation, that GEMV reads its
//   activations in its own sorted column order, contiguous, with no gather.
//   Entries outside the output's range are not written.
struct ResidualArgs {
  const uint16_t* ep_residual;  // null: plain epilogue
  float* ep_partial;
  const float* pro_partial;
  int pro_n;
  const uint16_t* pro_weight;
  float pro_eps;
  const int16_t* ep_index;  // null: outputs in row order only
  uint16_t* ep_sorted;      // residual epilogue: the reordered copy of out
};
constexpr int kMaxNormPartialsPerLane = 4;  // prologue: K <= 4 * 64 * 16

// Strided batch of one-row GEMVs in one launch (grid.y = payloads, one K split):
// payload p reads x + p * x, planes + p * planes, ... (element strides) and writes
// out + p * out.  All zero: a single GEMV (grid.y counts K splits).
struct StridedArgs {
  long long x, planes, scales, zeros, out;
};

struct MfmaArgs {
  const uint16_t* x;     // [mb, K] activations of this launch
  const int16_t* perm;   // null: identity
  const uint8_t* planes;
  const uint16_t* scales;
  const uint8_t* zeros;
  float* partial;  // null: write out directly (single K split)
  uint16_t* out;
  int O, G, gps;
  int row_blocks;  // ceil(O / (16 * tiles)); the grid is (row_blocks, K splits)
  int swiglu;      // 1: rows interleave (gate, up); out gets SiLU(gate) * up (mb 1, one split)
  ResidualArgs res;
  int x_lds;       // permuted kernels: 1 = gather from an LDS copy of x (x_lds_fits)
  StridedArgs batch;
};

// The permuted kernels gather x[perm] from an LDS copy of x when the activation
// rows fit: at most 48 KB of LDS and four 16-byte chunks per thread.  A global
// 2-byte load per value measured 1.3-1.6x the identity-order time at the Qwen3-8B
// shapes (gate/up 6.9 -> 9.1 us, down 7.4 -> 11.7 us).
inline bool x_lds_fits(int mb, int K, int nw) {
  return size_t(mb) * K * 2 <= 48 * 1024 && mb * (K / 8) <= 4 * nw * 64;
}
inline size_t x_lds_bytes(const MfmaArgs& a, int mb) { return a.x_lds ? size_t(mb) * a.G * 128 * 2 : 0; }

// nw waves per workgroup in {4, 8}; pd batches in flight per wave in {1, 2};
// mb activation rows in {1, 2, 4, 8}; tiles 16-row tiles per wave in {1, 2};
// sdt the scale dtype; the permutation instantiations are used when a.perm is
// set.  False if no instantiation matches.
#define FX_MFMA_DECL(NAME) \
  bool NAME(int nw, int pd, int mb, int sdt, const MfmaArgs& a, dim3 grid, hipStream_t s);
FX_MFMA_DECL(dispatch_mfma_bf16_t1)
FX_MFMA_DECL(dispatch_mfma_bf16_t2)
FX_MFMA_DECL(dispatch_mfma_f16_t1)
FX_MFMA_DECL(dispatch_mfma_f16_t2)
FX_MFMA_DECL(dispatch_mfma_bf16_t1_perm)
FX_MFMA_DECL(dispatch_mfma_bf16_t2_perm)
FX_MFMA_DECL(dispatch_mfma_f16_t1_perm)
FX_MFMA_DECL(dispatch_mfma_f16_t2_perm)
#undef FX_MFMA_DECL

// decoded_bf16 arithmetic (the +-3 correction as a second MFMA chain): one
// activation row, one tile and one batch in flight per wave, bf16 scales, planar
// payload, identity or permuted order; nw in {4, 8}.
bool dispatch_mfma_corr(int nw, int xdt, const MfmaArgs& a, dim3 grid, hipStream_t s);

// The normalising-prologue instantiations: one activation row, one 16-row tile
// and one batch in flight per wave, no permutation; nw in {4, 8}.
bool dispatch_mfma_normin(int nw, int xdt, int sdt, const MfmaArgs& a, dim3 grid, hipStream_t s);

// The field-layout instantiations (a.planes holds fields, w3_fields.hip): one
// activation row and one batch in flight per wave, one K split; plain (identity
// or permuted column order, a.perm) or normalising prologue (identity order
// only: false when a.perm is set); nw in {4, 8}.  Row tiles per wave:
// fields_row_tiles (a.row_blocks must count tiles of that many 16-row tiles).
bool dispatch_mfma_fields(int nw, bool normin, int xdt, int sdt, const MfmaArgs& a, dim3 grid, hipStream_t s);
inline int fields_row_tiles(bool normin, int O) { return normin && O % 4 == 0 ? 2 : 1; }

// The field-layout kernel with workgroup-shared staging (w3_fields_wide.h):
// workgroups of tiles 16-row tiles x parts K parts (one wave each), prefetch
// batches in flight per wave, stage staged batches per wave (the plan needs
// ceil(G / 4) <= stage * tiles * parts).  One activation row, one K split,
// O % 16 == 0 and G % 4 == 0 (the batch offsets ride in the loads' scalar
// offset, which the range check does not cover, so every live load must be in
// bounds); the grid is (ceil(O / (16 tiles)), payloads).  mode 0 plain,
// 1 normalising prologue, 2 permuted columns (a.perm; x in LDS, x_lds_fits).
struct WidePlan {
  int tiles, parts, prefetch, stage;
};
// The instantiated plans (tiles, parts, batches in flight, staged batches per wave).
#define FX_WIDE_PLANS(X) X(1, 8, 1, 1) X(1, 8, 3, 3) X(2, 4, 2, 1) X(3, 4, 2, 1) X(4, 2, 4, 1)
inline bool wide_plan_instantiated(const WidePlan& p) {
#define FX_WIDE_IS(T, P, PD, S) \
  if (p.tiles == T && p.parts == P && p.prefetch == PD && p.stage == S) return true;
  FX_WIDE_PLANS(FX_WIDE_IS)
#undef FX_WIDE_IS
  return false;
}
// Dynamic LDS of a plan: the staged batches (4 k-blocks of 17 16-byte slots
// each), one zero operand per MFMA step, the groups' sums and exponent offsets,
// the 8 virtual waves' sums of the 16 T rows and, permuted, a copy of x.
constexpr int kWideStage = 4 * 17;
constexpr int kWideVirtualWaves = 8;
inline size_t wide_lds_bytes(int T, int G, bool perm) {
  const size_t nb = size_t(G + 3) / 4;
  return nb * kWideStage * 16 + 16 * 16 + nb * 4 * 8 + size_t(kWideVirtualWaves) * 16 * T * 4 +
         (perm ? size_t(G) * 128 * 2 : 0);
}
// The M-row form (w3_fields_rows_kernel): MB = 2, 4 or 8 activation rows of
// which the first M are live, plain epilogue, identity order; the same plans and
// two more of one tile (12 and 16 parts, the M-row form only).  Static LDS for at
// most rows_batch_limit(MB) batches (K <= 512 * limit), except under a solo plan
// (one tile), where each wave restages one slot of its own and only the plan's
// staging bounds K.
#define FX_ROWS_PLANS(X) FX_WIDE_PLANS(X) X(1, 12, 2, 2) X(1, 16, 2, 2)
inline bool rows_plan_instantiated(const WidePlan& p) {
#define FX_ROWS_IS(T, P, PD, S) \
  if (p.tiles == T && p.parts == P && p.prefetch == PD && p.stage == S) return true;
  FX_ROWS_PLANS(FX_ROWS_IS)
#undef FX_ROWS_IS
  return false;
}
inline int rows_batch_limit(int mb) { return mb == 8 ? 8 : 24; }
inline bool rows_plan_solo(const WidePlan& p) { return p.tiles == 1; }
bool dispatch_fields_rows_m2(const WidePlan& p, int xdt, int sdt, const MfmaArgs& a, int M, dim3 grid, hipStream_t s);
bool dispatch_fields_rows_m4(const WidePlan& p, int xdt, int sdt, const MfmaArgs& a, int M, dim3 grid, hipStream_t s);
bool dispatch_fields_rows_m8(const WidePlan& p, int xdt, int sdt, const MfmaArgs& a, int M, dim3 grid, hipStream_t s);
inline bool dispatch_fields_rows(const WidePlan& p, int mb, int xdt, int sdt, const MfmaArgs& a, int M, dim3 grid,
                                 hipStream_t s) {
  if (mb == 2) return dispatch_fields_rows_m2(p, xdt, sdt, a, M, grid, s);
  if (mb == 4) return dispatch_fields_rows_m4(p, xdt, sdt, a, M, grid, s);
  if (mb == 8) return dispatch_fields_rows_m8(p, xdt, sdt, a, M, grid, s);
  return false;
}
bool dispatch_fields_wide_bf16(const WidePlan& p, int sdt, int mode, const MfmaArgs& a, dim3 grid, hipStream_t s);
bool dispatch_fields_wide_f16(const WidePlan& p, int sdt, int mode, const MfmaArgs& a, dim3 grid, hipStream_t s);
inline bool dispatch_fields_wide(const WidePlan& p, int xdt, int sdt, int mode, const MfmaArgs& a, dim3 grid,
                                 hipStream_t s) {
  if (xdt == kBF16) return dispatch_fields_wide_bf16(p, sdt, mode, a, grid, s);
  if (xdt == kF16) return dispatch_fields_wide_f16(p, sdt, mode, a, grid, s);
  return false;
}

// The bind-time repack planes [G, 3, O, 16] -> fields [G, 3, O, 16].
void launch_planes_to_fields(const uint8_t* planes, uint8_t* fields, int O, int G, hipStream_t s);
// fp6 layout (G % 4 == 0): the bind-time repack and the one-row GEMV launches
// (bf16 activations, vector scale loads; normin: two row tiles per wave).
void launch_planes_to_fp6(const uint8_t* planes, uint8_t* out, int O, int G, hipStream_t s);
bool dispatch_mfma_fp6(int nw, bool normin, int sdt, const MfmaArgs& a, dim3 grid, hipStream_t s);

inline bool dispatch_mfma(int xdt, int tiles, int nw, int pd, int mb, int sdt, const MfmaArgs& a,
                          dim3 grid, hipStream_t s) {
  const bool p = a.perm != nullptr;
  if (xdt == kBF16 && tiles == 1)
    return p ? dispatch_mfma_bf16_t1_perm(nw, pd, mb, sdt, a, grid, s)
             : dispatch_mfma_bf16_t1(nw, pd, mb, sdt, a, grid, s);
  if (xdt == kBF16 && tiles == 2)
    return p ? dispatch_mfma_bf16_t2_perm(nw, pd, mb, sdt, a, grid, s)
             : dispatch_mfma_bf16_t2(nw, pd, mb, sdt, a, grid, s);
  if (xdt == kF16 && tiles == 1)
    return p ? dispatch_mfma_f16_t1_perm(nw, pd, mb, sdt, a, grid, s)
             : dispatch_mfma_f16_t1(nw, pd, mb, sdt, a, grid, s);
  if (xdt == kF16 && tiles == 2)
    return p ? dispatch_mfma_f16_t2_perm(nw, pd, mb, sdt, a, grid, s)
             : dispatch_mfma_f16_t2(nw, pd, mb, sdt, a, grid, s);
  return false;
}

}  // namespace fx
