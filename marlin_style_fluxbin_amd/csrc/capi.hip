// extern "C" boundary of libfluxbin_amd.so (declarations: include/fluxbin_amd.h).
// Validates arguments, picks kernel instantiations and tilings, launches on the
// caller's stream.  Nothing here allocates or synchronises.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "../../include/fluxbin_amd.h"
#include "common.h"
#include "w3_lut_launch.h"
#include "w3_lut.hip"
#include "w3_mfma_launch.h"
#include "norms_launch.h"
#include "decode_launch.h"
#include "lm_head_launch.h"
#include "two_base_launch.h"

using fx::LutArgs;
using fx::MfmaArgs;

namespace {

thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(FX_EHIP, "%s: %s", what, hipGetErrorString(e));
  return FX_OK;
}

int device_cu_count() {
  static std::mutex lock;
  static int cached[64] = {0};
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return 256;
  std::lock_guard<std::mutex> guard(lock);
  if (cached[device] == 0) {
    int count = 0;
    if (hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        count <= 0)
      count = 256;
    cached[device] = count;
  }
  return cached[device];
}

bool is_half_dtype(int dt) { return dt == FX_F16 || dt == FX_BF16; }

int validate_payload(const void* x, int x_dtype, const uint8_t* planes, const void* scales,
                     int scale_dtype, int M, int O, int K, int arithmetic) {
  if (!x || !planes || !scales) return fail(FX_EINVAL, "x, planes and scales must be non-null");
  if (!is_half_dtype(x_dtype)) return fail(FX_EINVAL, "x dtype must be fp16 or bf16");
  if (!is_half_dtype(scale_dtype)) return fail(FX_EINVAL, "scale dtype must be fp16 or bf16");
  if (M < 1 || M > 64) return fail(FX_EINVAL, "M must be in [1,64], got %d", M);
  if (O < 1 || O > (1 << 20)) return fail(FX_EINVAL, "O out of range: %d", O);
  if (K < 128 || K % 128 != 0 || K > 32768 * 4)
    return fail(FX_EINVAL, "K must be a positive multiple of 128, got %d", K);
  if (reinterpret_cast<uintptr_t>(planes) % 16 != 0)
    return fail(FX_EINVAL, "planes must be 16-byte aligned");
  // kernels address the payload with 32-bit byte offsets
  if (size_t(K / 128) * 3 * size_t(O) * 16 > 0x7fffffffu || size_t(M) * K * 2 > 0x7fffffffu)
    return fail(FX_EINVAL, "payload of %d x %d exceeds 2 GiB", O, K);
  if (arithmetic != FX_ARITH_STRUCTURAL && arithmetic != FX_ARITH_DECODED_BF16)
    return fail(FX_EINVAL, "unknown arithmetic %d", arithmetic);
  if (arithmetic == FX_ARITH_DECODED_BF16 && scale_dtype != FX_BF16)
    return fail(FX_EINVAL, "decoded_bf16 arithmetic requires bf16 scales");
  return FX_OK;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// ------------------------------------------------------------------ LUT kernel
int rows_per_thread_from_tile(int row_tile) {
  switch (row_tile) {
    case 256: return 1;
    case 512: return 2;
    case 1024: return 4;
    default: return -1;
  }
}

// Largest supported LUT activation-row block not above m.
int lut_block_for(int m) { return m >= 8 ? 8 : m >= 4 ? 4 : m >= 2 ? 2 : 1; }

struct LutTile {
  int rpt, gps, splits, row_tiles;
};

LutTile make_lut_tile(int O, int G, int rpt, int gps) {
  LutTile t;
  t.rpt = rpt;
  t.gps = gps < 1 ? 1 : (gps > G ? G : gps);
  t.splits = (G + t.gps - 1) / t.gps;
  t.row_tiles = (O + fx::kLutThreads * rpt - 1) / (fx::kLutThreads * rpt);
  return t;
}

// LUT tiling for the decoded route: one row per thread, enough K splits for
// about two workgroups per CU.
LutTile default_lut_tile(int O, int G) {
  const int row_tiles = (O + fx::kLutThreads - 1) / fx::kLutThreads;
  int splits = (2 * device_cu_count() + row_tiles - 1) / row_tiles;
  splits = splits < 1 ? 1 : (splits > G ? G : splits);
  return make_lut_tile(O, G, 1, (G + splits - 1) / splits);
}

// Direct (one split) or partial mode over M rows in LUT blocks of 8/4/2/1.
// In partial mode block b writes partial[s][m][o] of its own [splits, mb, O] slice.
int run_lut(const void* x, int x_dtype, const uint8_t* planes, const void* scales, int scale_dtype,
            const uint8_t* zeros, const int16_t* perm, float* partial, void* out, int M, int O,
            int K, int arithmetic, const LutTile& tile, bool partial_mode, hipStream_t stream) {
  const int G = K / 128;
  const bool dec = arithmetic == FX_ARITH_DECODED_BF16;
  int done = 0;
  while (done < M) {
    const int mb = lut_block_for(M - done);
    LutArgs a;
    a.x = static_cast<const uint16_t*>(x) + size_t(done) * K;
    a.planes = planes;
    a.scales = static_cast<const uint16_t*>(scales);
    a.zeros = zeros;
    a.perm = perm;
    a.partial = partial ? partial + size_t(tile.splits) * size_t(done) * O : nullptr;
    a.out = out ? static_cast<uint16_t*>(out) + size_t(done) * O : nullptr;
    a.O = O;
    a.G = G;
    a.gps = tile.gps;
    a.mode = partial_mode ? fx::kModePartial : fx::kModeDirect;
    const dim3 grid(tile.row_tiles, tile.splits);
    if (!fx::dispatch_lut(mb, tile.rpt, x_dtype, scale_dtype, dec, a, grid, stream))
      return fail(FX_EINVAL, "no LUT kernel for M-block %d rpt %d dtypes %d/%d", mb, tile.rpt,
                  x_dtype, scale_dtype);
    int rc = check_launch("w3_lut_kernel");
    if (rc) return rc;
    done += mb;
  }
  return FX_OK;
}

int launch_finish(const float* partial, void* out, int out_dtype, int splits, int MO,
                  hipStream_t s) {
  const dim3 grid((MO + 255) / 256);
  if (out_dtype == FX_BF16)
    hipLaunchKernelGGL(fx::w3_finish_kernel<fx::kBF16>, grid, dim3(256), 0, s, partial,
                       static_cast<uint16_t*>(out), MO, splits);
  else
    hipLaunchKernelGGL(fx::w3_finish_kernel<fx::kF16>, grid, dim3(256), 0, s, partial,
                       static_cast<uint16_t*>(out), MO, splits);
  return check_launch("w3_finish_kernel");
}

// Decoded route for the fast entry point: LUT partials + finish (or direct).
size_t lut_route_workspace(int M, int O, int K) {
  const LutTile t = default_lut_tile(O, K / 128);
  if (t.splits == 1) return 0;
  return size_t(t.splits) * size_t(lut_block_for(M)) * size_t(O) * sizeof(float);
}

int run_lut_route(const void* x, int x_dtype, const uint8_t* planes, const void* scales,
                  int scale_dtype, const uint8_t* zeros, const int16_t* perm, void* workspace,
                  size_t workspace_bytes, void* out, int M, int O, int K, int arithmetic,
                  hipStream_t s) {
  const LutTile tile = default_lut_tile(O, K / 128);
  if (tile.splits == 1)
    return run_lut(x, x_dtype, planes, scales, scale_dtype, zeros, perm, nullptr, out, M, O, K,
                   arithmetic, tile, false, s);
  const size_t need = lut_route_workspace(M, O, K);
  if (!workspace || workspace_bytes < need)
    return fail(FX_EINVAL, "workspace needs %zu bytes, got %zu", need, workspace_bytes);
  float* partial = static_cast<float*>(workspace);
  int done = 0;
  while (done < M) {  // finish per LUT block: each block's partials are [splits, mb, O]
    const int mb = lut_block_for(M - done);
    const void* xb = static_cast<const uint16_t*>(x) + size_t(done) * K;
    void* ob = static_cast<uint16_t*>(out) + size_t(done) * O;
    int rc = run_lut(xb, x_dtype, planes, scales, scale_dtype, zeros, perm, partial, nullptr, mb,
                     O, K, arithmetic, tile, true, s);
    if (rc) return rc;
    rc = launch_finish(partial, ob, x_dtype, tile.splits, mb * O, s);
    if (rc) return rc;
    done += mb;
  }
  return FX_OK;
}

// ------------------------------------------------------------------ MFMA kernel
struct MfmaPlan {
  int nw, pd, tiles;  // waves per workgroup, batches in flight per wave, 16-row tiles per wave
  int gps, splits, row_blocks;
};

int mfma_chunk_for(int m) { return m >= 8 ? 8 : m >= 4 ? 4 : m >= 2 ? 2 : 1; }

MfmaPlan make_mfma_plan(int O, int G, int nw, int pd, int gps, int tiles) {
  MfmaPlan p;
  p.nw = nw;
  p.pd = pd;
  p.tiles = tiles;
  const int gmax = (G + 3) / 4 * 4;
  p.gps = gps < 4 ? 4 : (gps + 3) / 4 * 4;
  if (p.gps > gmax) p.gps = gmax;
  p.splits = (G + p.gps - 1) / p.gps;
  p.row_blocks = (O + 16 * tiles - 1) / (16 * tiles);
  return p;
}

// Default (from graph-timed sweeps over the Qwen3-8B shapes on MI355X): one
// 16-row tile and one batch in flight per wave (more tiles or a deeper ring
// cost occupancy and measured slower), eight waves splitting K inside the
// workgroup, and a K split over workgroups only for very narrow outputs (a
// split costs a finish launch, which is more than idle CUs cost at these sizes).
// Four waves instead when eight would not all be resident at once (~6 waves of
// this kernel per SIMD): a second residency round costs more than the longer
// per-wave K loop (fused gate|up, 24576 x 4096: 10.3 us with 4 waves, 11.7 us
// with 8).
// mb: activation rows per launch.  Eight rows: two 16-row tiles per wave share
// each staged batch of the eight rows where the grid still covers the CUs (the
// wide gate/up shape, 4 waves; with 16+ batches per row block, two K splits and
// 8 waves), measured at Qwen3-8B shapes (graph-timed, rotating payloads): gate/up
// 13.95 -> 13.09 us, down 15.11 -> 12.50 us; q/o keeps the one-row plan (7.0 us).
MfmaPlan default_mfma_plan(int O, int G, int mb = 1, int waves_per_simd = 6) {
  if (mb == 8) {
    const int batches = (G + 3) / 4;
    const int cus = device_cu_count();
    const int blocks2 = (O + 31) / 32;  // row blocks of two 16-row tiles
    if (batches >= 16 && blocks2 < cus) return make_mfma_plan(O, G, 8, 1, (batches + 1) / 2 * 4, 2);
    if (batches <= 8 && blocks2 >= cus) return make_mfma_plan(O, G, 4, 1, batches * 4, 2);
  }
  const int tiles = 1;
  const int row_blocks = (O + 15) / 16;
  const int batches = (G + 3) / 4;
  int splits = 1;
  if (row_blocks < 32) splits = (64 + row_blocks - 1) / row_blocks;
  if (splits > batches) splits = batches;
  const int per_split = (batches + splits - 1) / splits;  // batches per workgroup
  const long resident_waves = 4L * waves_per_simd * device_cu_count();
  const int nw = per_split >= 8 && long(row_blocks) * splits * 8 <= resident_waves ? 8 : 4;
  return make_mfma_plan(O, G, nw, 1, per_split * 4, tiles);
}

// The MFMA path needs workspace only for fp32 partials when K is split over
// workgroups: [splits, mb, O] for the largest activation chunk mb.
size_t mfma_workspace(int M, int O, const MfmaPlan& p) {
  const int mb = mfma_chunk_for(M);
  return p.splits > 1 ? size_t(p.splits) * mb * O * sizeof(float) : 0;
}

int run_mfma(const void* x, int x_dtype, const uint8_t* planes, const void* scales,
             int scale_dtype, const uint8_t* zeros, const int16_t* perm, void* workspace,
             size_t workspace_bytes, void* out, int M, int O, int K, const MfmaPlan& p,
             hipStream_t s, int swiglu = 0, const int16_t* out_index = nullptr, bool corrected = false) {
  const int G = K / 128;
  const size_t need = mfma_workspace(M, O, p);
  if (need > 0) {
    if (!workspace || workspace_bytes < need)
      return fail(FX_EINVAL, "workspace needs %zu bytes, got %zu", need, workspace_bytes);
    if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
      return fail(FX_EINVAL, "workspace must be 256-byte aligned");
  }
  float* partial = p.splits > 1 ? static_cast<float*>(workspace) : nullptr;
  int done = 0;
  while (done < M) {
    const int mb = mfma_chunk_for(M - done);
    uint16_t* ob = static_cast<uint16_t*>(out) + size_t(done) * O;
    MfmaArgs a;
    a.x = static_cast<const uint16_t*>(x) + size_t(done) * K;
    a.perm = perm;
    a.planes = planes;
    a.scales = static_cast<const uint16_t*>(scales);
    a.zeros = zeros;
    a.partial = partial;
    a.out = ob;
    a.O = O;
    a.G = G;
    a.gps = p.gps;
    a.row_blocks = p.row_blocks;
    a.swiglu = swiglu;
    a.res = fx::ResidualArgs{};
    a.res.ep_index = out_index;
    a.x_lds = perm && fx::x_lds_fits(mb, K, p.nw);
    a.batch = fx::StridedArgs{};
    const dim3 grid(p.row_blocks, p.splits);
    if (corrected) {
      if (mb != 1 || p.tiles != 1 || p.pd != 1 || scale_dtype != FX_BF16 ||
          !fx::dispatch_mfma_corr(p.nw, x_dtype, a, grid, s))
        return fail(FX_EINVAL, "no decoded_bf16 MFMA kernel for waves %d tiles %d rows %d", p.nw, p.tiles, mb);
    } else if (!fx::dispatch_mfma(x_dtype, p.tiles, p.nw, p.pd, mb, scale_dtype, a, grid, s)) {
      return fail(FX_EINVAL, "no MFMA kernel for waves %d prefetch %d tiles %d rows %d", p.nw,
                  p.pd, p.tiles, mb);
    }
    int rc = check_launch("w3_mfma_kernel");
    if (rc) return rc;
    if (partial) {
      rc = launch_finish(partial, ob, x_dtype, p.splits, mb * O, s);
      if (rc) return rc;
    }
    done += mb;
  }
  return FX_OK;
}

// ------------------------------------------------------------------ two-base GEMV
struct TwoBasePlan {
  int nt, nk, pd;  // row tiles per workgroup, waves per tile along K, batches in flight
  int gps, splits, row_blocks;
};

bool two_base_instantiated(int nt, int nk, int pd) {
  switch (nt * 100 + nk * 10 + pd) {
    case 141: case 142: case 181: case 182: case 183: case 242: case 282: case 341: case 342:
    case 442:
      return true;
  }
  return false;
}

// K split so that one workgroup stages at most kRankOneMaxBatches batches and
// each thread at most kRankOneMaxUnits 8-column units.
TwoBasePlan make_two_base_plan(int O, int G, int nt, int nk, int pd, int gps) {
  TwoBasePlan p;
  p.nt = nt;
  p.nk = nk;
  p.pd = pd;
  const int gmax = (G + 3) / 4 * 4;
  p.gps = gps < 4 ? 4 : (gps + 3) / 4 * 4;
  if (p.gps > gmax) p.gps = gmax;
  const int cap = 4 * std::min(fx::kRankOneMaxBatches, fx::kRankOneMaxUnits * nt * nk);
  if (p.gps > cap) p.gps = cap;
  p.splits = (G + p.gps - 1) / p.gps;
  p.row_blocks = (O + 16 * nt - 1) / (16 * nt);
  return p;
}

// Default (graph-timed on MI355X): enough row tiles per workgroup to land near
// one workgroup per CU (the dispatcher starts ~one workgroup per 2.7 ns, and each
// workgroup stages its K range once), waves along K so every wave owns one to
// three batches, and a K split over workgroups only for narrow outputs or K
// beyond one workgroup's staging capacity.
TwoBasePlan default_two_base_plan(int O, int G) {
  const int cus = device_cu_count();
  const int tiles_total = (O + 15) / 16;
  int nt = tiles_total / cus;
  nt = nt < 1 ? 1 : (nt > 3 ? 3 : nt);
  const int row_blocks = (tiles_total + nt - 1) / nt;
  const int batches = (G + 3) / 4;
  int splits = 1;
  if (row_blocks < 32) splits = (64 + row_blocks - 1) / row_blocks;
  if (splits > batches) splits = batches;
  int per_split = (batches + splits - 1) / splits;
  const int nk = (nt == 1 && per_split >= 8) ? 8 : 4;
  const int cap = std::min(fx::kRankOneMaxBatches, fx::kRankOneMaxUnits * nt * nk);
  if (per_split > cap) {
    splits = (batches + cap - 1) / cap;
    per_split = (batches + splits - 1) / splits;
  }
  // one batch of sign loads in flight per wave measured fastest at the gate
  // shape (a second one issued up front queues behind the first in HBM)
  return make_two_base_plan(O, G, nt, nk, 1, per_split * 4);
}

size_t two_base_workspace(int O, const TwoBasePlan& p) {
  return p.splits > 1 ? size_t(p.splits) * O * sizeof(float) : 0;
}

int run_rank_one(const void* x, int x_dtype, const uint8_t* planes, const void* coef,
                 const void* srow, const void* tcol, const void* salient,
                 const int32_t* salient_idx, int n_salient, void* workspace,
                 size_t workspace_bytes, void* out, int O, int K, const TwoBasePlan& p,
                 hipStream_t s) {
  if (!x || !planes || !coef || !srow || !tcol || !out)
    return fail(FX_EINVAL, "x, planes, coef, srow, tcol and out must be non-null");
  if (!is_half_dtype(x_dtype)) return fail(FX_EINVAL, "x dtype must be fp16 or bf16");
  if (O < 1 || O > (1 << 20)) return fail(FX_EINVAL, "O out of range: %d", O);
  if (K < 128 || K % 128 != 0 || K > 32768 * 4)
    return fail(FX_EINVAL, "K must be a positive multiple of 128, got %d", K);
  if (n_salient < 0 || n_salient > 32)
    return fail(FX_EINVAL, "n_salient must be in [0, 32], got %d", n_salient);
  if (n_salient > 0 && (!salient || !salient_idx))
    return fail(FX_EINVAL, "salient values and indices must be non-null when n_salient > 0");
  if (reinterpret_cast<uintptr_t>(planes) % 16 || reinterpret_cast<uintptr_t>(x) % 16 ||
      reinterpret_cast<uintptr_t>(tcol) % 16)
    return fail(FX_EINVAL, "planes, x and tcol must be 16-byte aligned");
  if (size_t(K / 128) * size_t(O) * 32 > 0x7fffffffu)
    return fail(FX_EINVAL, "payload of %d x %d exceeds 2 GiB", O, K);
  if (!two_base_instantiated(p.nt, p.nk, p.pd))
    return fail(FX_EINVAL, "no two-base kernel for tiles %d kparts %d prefetch %d", p.nt, p.nk, p.pd);
  const size_t need = two_base_workspace(O, p);
  if (need > 0) {
    if (!workspace || workspace_bytes < need)
      return fail(FX_EINVAL, "workspace needs %zu bytes, got %zu", need, workspace_bytes);
    if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
      return fail(FX_EINVAL, "workspace must be 256-byte aligned");
  }
  fx::RankOneArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.planes = planes;
  a.coef = static_cast<const uint16_t*>(coef);
  a.srow = static_cast<const uint16_t*>(srow);
  a.tcol = static_cast<const uint16_t*>(tcol);
  a.sal = static_cast<const uint16_t*>(salient);
  a.sal_idx = salient_idx;
  a.partial = p.splits > 1 ? static_cast<float*>(workspace) : nullptr;
  a.out = static_cast<uint16_t*>(out);
  a.O = O;
  a.G = K / 128;
  a.S = n_salient;
  a.gps = p.gps;
  a.row_blocks = p.row_blocks;
  if (!fx::dispatch_rank_one(x_dtype, p.nt, p.nk, p.pd, a, dim3(p.row_blocks, p.splits), s))
    return fail(FX_EINVAL, "no two-base kernel for tiles %d kparts %d prefetch %d", p.nt, p.nk, p.pd);
  int rc = check_launch("rank_one_kernel");
  if (rc || p.splits == 1) return rc;
  return launch_finish(a.partial, out, x_dtype, p.splits, O, s);
}

// Hybrid layout.  The kernel holds 134 VGPRs per lane, so a CU runs 12 of its
// waves; a plan keeps every workgroup resident in one round where the rows
// allow it: nt = ceil(tiles / CUs) 16-row tiles per workgroup (at most
// max_tiles), and K parts nk = 4 for nt = 2..3, 2 for nt = 4..6 (8 or 12 waves
// per workgroup), nt = 1: 8 (4 when the split has fewer than 8 batches).  The
// results do not depend on the plan (the kernel sums eight virtual K parts in a
// fixed order).  Measured at the Qwen3-8B decode launches (rotating payloads,
// HIP graph): q|k|v 6144 x 4096 11.5 -> 8.4 us ((1, 8) -> (2, 4)), gate|up
// 24576 x 4096 17.8 -> 13.7 us ((3, 4) -> (6, 2)); o and down stay (1, 8).
// At most `max_splits` K splits (the caller's workspace); staging holds 3.3 KB
// of LDS per batch.
constexpr int kHybridMaxTiles = 6;

TwoBasePlan default_hybrid_plan(int O, int G, int max_splits, int max_tiles = kHybridMaxTiles) {
  const int cus = device_cu_count();
  const int tiles_total = (O + 15) / 16;
  int nt = (tiles_total + cus - 1) / cus;
  nt = nt < 1 ? 1 : (nt > max_tiles ? max_tiles : nt);
  const int row_blocks = (tiles_total + nt - 1) / nt;
  const int batches = (G + 3) / 4;
  int splits = 1;
  if (row_blocks < 32) splits = (64 + row_blocks - 1) / row_blocks;
  if (splits > batches) splits = batches;
  int per_split = (batches + splits - 1) / splits;
  const int nk = nt == 1 ? (per_split >= 8 ? 8 : 4) : (nt <= 3 ? 4 : 2);
  const int cap = std::min(fx::kHybridMaxBatches, 4 * nt * nk);
  if (per_split > cap) {
    splits = (batches + cap - 1) / cap;
    per_split = (batches + splits - 1) / splits;
  }
  if (splits > max_splits && max_splits >= 1) {  // fewer, longer splits (never beyond the cap)
    const int fewer = std::max(max_splits, (batches + cap - 1) / cap);
    splits = fewer;
    per_split = (batches + splits - 1) / splits;
  }
  TwoBasePlan p;
  p.nt = nt;
  p.nk = nk;
  p.pd = 1;
  p.gps = per_split * 4;
  p.splits = (G + p.gps - 1) / p.gps;
  p.row_blocks = (O + 16 * nt - 1) / (16 * nt);
  return p;
}

// One launch over n_seg layouts concatenated along O (n_seg = 1: one layout).
int run_hybrid(const void* x, int x_dtype, int n_seg, const int* seg_rows, const uint8_t* codes, const float* rows,
               const float* const* cols, const int16_t* const* idx, const uint8_t* scodes, const float* srows,
               const float* const* scols, void* workspace, size_t workspace_bytes, void* out, int K,
               const fx::ResidualArgs& res, bool swiglu_in, hipStream_t s) {
  if (n_seg < 1 || n_seg > fx::kHybridMaxSegments)
    return fail(FX_EINVAL, "n_segments must be in [1, %d], got %d", fx::kHybridMaxSegments, n_seg);
  if (!seg_rows || !cols || !idx || !scols) return fail(FX_EINVAL, "segment arrays must be non-null");
  long total = 0;
  for (int i = 0; i < n_seg; ++i) {
    if (seg_rows[i] < 1) return fail(FX_EINVAL, "segment %d has %d rows", i, seg_rows[i]);
    if (n_seg > 1 && seg_rows[i] % 16)
      return fail(FX_EINVAL, "segment %d has %d rows: concatenated segments must be multiples of 16", i,
                  seg_rows[i]);
    if (!cols[i] || !idx[i] || !scols[i]) return fail(FX_EINVAL, "segment %d: columns, indices and sparse columns "
                                                      "must be non-null", i);
    if (reinterpret_cast<uintptr_t>(cols[i]) % 16) return fail(FX_EINVAL, "segment %d: columns must be 16-byte "
                                                                "aligned", i);
    total += seg_rows[i];
  }
  if (total > 65536) return fail(FX_EINVAL, "O must be in [1, 65536], got %ld", total);
  const int O = int(total);
  if (!x || !codes || !rows || !scodes || !srows || !out)
    return fail(FX_EINVAL, "x, every layout field and out must be non-null");
  if (!is_half_dtype(x_dtype)) return fail(FX_EINVAL, "x dtype must be fp16 or bf16");
  if (K < 128 || K % 128 != 0 || K > 131072)
    return fail(FX_EINVAL, "K must be a multiple of 128 in [128, 131072], got %d", K);
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(codes) % 16 ||
      reinterpret_cast<uintptr_t>(rows) % 16 || reinterpret_cast<uintptr_t>(srows) % 16)
    return fail(FX_EINVAL, "x, codes, rows, columns and sparse rows must be 16-byte aligned");
  const int G = K / 128;
  if (size_t(G) * size_t(O) * 32 > 0x7fffffffu) return fail(FX_EINVAL, "payload exceeds 2 GiB");
  // the residual epilogue writes the output itself: one K split
  const int max_splits = res.ep_residual ? 1
                                         : int(std::min<size_t>(workspace ? workspace_bytes / (size_t(O) * 4) : 0, 1 << 20));
  // a workgroup's rows must lie in one segment: every segment start on its
  // 16 * tiles grid (fewer tiles per workgroup until they are)
  TwoBasePlan p = default_hybrid_plan(O, G, max_splits < 1 ? 1 : max_splits);
  for (;;) {
    bool aligned = true;
    for (int i = 1, start = seg_rows[0]; i < n_seg; start += seg_rows[i], ++i) aligned = aligned && start % (16 * p.nt) == 0;
    if (aligned || p.nt == 1) break;
    p = default_hybrid_plan(O, G, max_splits < 1 ? 1 : max_splits, p.nt - 1);
  }
  if (res.ep_residual && p.splits > 1)
    return fail(FX_EINVAL, "K = %d needs %d K splits; the residual epilogue takes one", K, p.splits);
  const size_t need = two_base_workspace(O, p);
  if (need > 0) {
    if (!workspace || workspace_bytes < need)
      return fail(FX_EINVAL, "workspace needs %zu bytes, got %zu", need, workspace_bytes);
    if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
      return fail(FX_EINVAL, "workspace must be 16-byte aligned");
  }
  fx::HybridArgs a{};
  a.res = res;
  a.x = static_cast<const uint16_t*>(x);
  a.codes = codes;
  a.rows = rows;
  a.cols = cols[0];
  a.idx = idx[0];
  a.scodes = scodes;
  a.srows = srows;
  a.scols = scols[0];
  a.partial = p.splits > 1 ? static_cast<float*>(workspace) : nullptr;
  a.out = static_cast<uint16_t*>(out);
  a.O = O;
  a.G = G;
  a.gps = p.gps;
  a.row_blocks = p.row_blocks;
  a.nseg = n_seg;
  for (int i = 0, start = 0; i < fx::kHybridMaxSegments; ++i) {
    const bool used = i < n_seg;
    a.seg_start[i] = used ? start : O;
    a.seg_cols[i] = used ? cols[i] : cols[0];
    a.seg_idx[i] = used ? idx[i] : idx[0];
    a.seg_scols[i] = used ? scols[i] : scols[0];
    if (used) start += seg_rows[i];
  }
  const int prologue = res.pro_partial ? fx::kHyProNorm : swiglu_in ? fx::kHyProSwiglu : fx::kHyProPlain;
  if (!fx::dispatch_hybrid(x_dtype, p.nt, p.nk, prologue, a, dim3(p.row_blocks, p.splits), s))
    return fail(FX_EINVAL, "no hybrid kernel for tiles %d kparts %d", p.nt, p.nk);
  int rc = check_launch("hybrid_kernel");
  if (rc || p.splits == 1) return rc;
  return launch_finish(a.partial, out, x_dtype, p.splits, O, s);
}

// Explicit tiling of the public config entry: waves = tiles * kparts.
bool two_base_config(int O, int G, int waves, int prefetch, int groups_per_split, int tiles,
                     TwoBasePlan* plan) {
  if (tiles < 1 || waves < tiles || waves % tiles || groups_per_split < 1) return false;
  const int nk = waves / tiles;
  if (!two_base_instantiated(tiles, nk, prefetch)) return false;
  *plan = make_two_base_plan(O, G, tiles, nk, prefetch, groups_per_split);
  return true;
}

}  // namespace

extern "C" {

int fx_abi_version(void) { return 19; }

const char* fx_last_error(void) { return g_error; }

int fx_w3_inline_main(const void* x, int x_dtype, const uint8_t* planes, const void* scales,
                      int scale_dtype, const uint8_t* zeros, const int16_t* perm,
                      float* partial, int M, int O, int K, int groups_per_split, int row_tile,
                      int arithmetic, void* stream) {
  int rc = validate_payload(x, x_dtype, planes, scales, scale_dtype, M, O, K, arithmetic);
  if (rc) return rc;
  if (!partial) return fail(FX_EINVAL, "partial workspace must be non-null");
  const int rpt = rows_per_thread_from_tile(row_tile);
  if (rpt < 0) return fail(FX_EINVAL, "row_tile must be 256, 512 or 1024");
  const int G = K / 128;
  if (groups_per_split < 1 || groups_per_split > G)
    return fail(FX_EINVAL, "groups_per_split must be in [1, K/128]");
  if (lut_block_for(M) != M) return fail(FX_EINVAL, "inline_main supports M in {1,2,4,8}");
  return run_lut(x, x_dtype, planes, scales, scale_dtype, zeros, perm, partial, nullptr, M, O, K,
                 arithmetic, make_lut_tile(O, G, rpt, groups_per_split), true,
                 static_cast<hipStream_t>(stream));
}

int fx_w3_finish(const float* partial, void* out, int out_dtype, int splits, int M, int O,
                 void* stream) {
  if (!partial || !out) return fail(FX_EINVAL, "partial and out must be non-null");
  if (!is_half_dtype(out_dtype)) return fail(FX_EINVAL, "out dtype must be fp16 or bf16");
  if (splits < 1 || M < 1 || O < 1) return fail(FX_EINVAL, "splits, M and O must be positive");
  return launch_finish(partial, out, out_dtype, splits, M * O, static_cast<hipStream_t>(stream));
}

int fx_w3_m1_out(const void* x, int x_dtype, const uint8_t* planes, const void* scales,
                 int scale_dtype, const uint8_t* zeros, const int16_t* perm, float* workspace,
                 void* out, int M, int O, int K, int groups_per_split, int row_tile,
                 int arithmetic, void* stream) {
  int rc = validate_payload(x, x_dtype, planes, scales, scale_dtype, M, O, K, arithmetic);
  if (rc) return rc;
  if (!out) return fail(FX_EINVAL, "out must be non-null");
  const int rpt = rows_per_thread_from_tile(row_tile);
  if (rpt < 0) return fail(FX_EINVAL, "row_tile must be 256, 512 or 1024");
  const int G = K / 128;
  if (groups_per_split < 1 || groups_per_split > G)
    return fail(FX_EINVAL, "groups_per_split must be in [1, K/128]");
  if (lut_block_for(M) != M) return fail(FX_EINVAL, "m1_out supports M in {1,2,4,8}");
  const LutTile tile = make_lut_tile(O, G, rpt, groups_per_split);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (tile.splits == 1)
    return run_lut(x, x_dtype, planes, scales, scale_dtype, zeros, perm, nullptr, out, M, O, K,
                   arithmetic, tile, false, s);
  if (!workspace) return fail(FX_EINVAL, "workspace must be non-null when K is split");
  rc = run_lut(x, x_dtype, planes, scales, scale_dtype, zeros, perm, workspace, nullptr, M, O, K,
               arithmetic, tile, true, s);
  if (rc) return rc;
  return launch_finish(workspace, out, x_dtype, tile.splits, M * O, s);
}

// The decoded_bf16 kernel holds ~90 VGPRs: five of its waves fit per SIMD.
constexpr int kCorrWavesPerSimd = 5;

size_t fx_w3_gemv_workspace_bytes(int M, int O, int K) {
  if (M < 1 || O < 1 || K < 128 || K % 128) return 0;
  const int G = K / 128;
  const size_t mfma = mfma_workspace(M, O, default_mfma_plan(O, G, mfma_chunk_for(M)));
  const size_t corr = M == 1 ? mfma_workspace(1, O, default_mfma_plan(O, G, 1, kCorrWavesPerSimd)) : 0;
  const size_t lut = lut_route_workspace(M, O, K);
  return std::max({mfma, corr, lut});
}

int fx_w3_gemv(const void* x, int x_dtype, const uint8_t* planes, const void* scales,
               int scale_dtype, const uint8_t* zeros, const int16_t* perm, void* workspace,
               size_t workspace_bytes, void* out, int M, int O, int K, int arithmetic,
               void* stream) {
  int rc = validate_payload(x, x_dtype, planes, scales, scale_dtype, M, O, K, arithmetic);
  if (rc) return rc;
  if (!out) return fail(FX_EINVAL, "out must be non-null");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // decoded_bf16: one activation row on the matrix cores (the +-3 correction as a
  // second MFMA chain); more rows on the table kernel
  if (arithmetic == FX_ARITH_DECODED_BF16 && M == 1)
    return run_mfma(x, x_dtype, planes, scales, scale_dtype, zeros, perm, workspace, workspace_bytes, out, 1, O,
                    K, default_mfma_plan(O, K / 128, 1, kCorrWavesPerSimd), s, 0, nullptr, true);
  if (arithmetic == FX_ARITH_DECODED_BF16)
    return run_lut_route(x, x_dtype, planes, scales, scale_dtype, zeros, perm, workspace,
                         workspace_bytes, out, M, O, K, arithmetic, s);
  return run_mfma(x, x_dtype, planes, scales, scale_dtype, zeros, perm, workspace,
                  workspace_bytes, out, M, O, K, default_mfma_plan(O, K / 128, mfma_chunk_for(M)), s);
}

// ------------------------------------------------------------------ allocation-free GEMV
// Scratch of fx_w3_gemv_noalloc: the fp32 K-split partials that fx_w3_gemv keeps in
// its caller's workspace.  One copy per GPU, held until the process ends.  Host
// code never uses the array's name as an address (in host code it is a host-side
// stand-in): each device's address comes from hipGetSymbolAddress, resolved once
// per device with that device current, and only that address reaches kernels.
constexpr size_t kNoallocScratchBytes = size_t(4) << 20;
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_for_current_device(void** out) {
  int device = -1;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return fail(FX_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (device < 0 || device >= kMaxDevices) return fail(FX_EINVAL, "device %d out of range", device);
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(FX_EHIP, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return FX_OK;
}
}  // namespace

int fx_w3_gemv_noalloc(const void* x, int x_dtype, const uint8_t* planes, const void* scales, int scale_dtype,
                       const uint8_t* zeros, const int16_t* perm, void* out, int M, int O, int K, int arithmetic,
                       void* stream) {
  int rc = validate_payload(x, x_dtype, planes, scales, scale_dtype, M, O, K, arithmetic);
  if (rc) return rc;
  if (!out) return fail(FX_EINVAL, "out must be non-null");
  const size_t need = fx_w3_gemv_workspace_bytes(M, O, K);
  if (need > kNoallocScratchBytes)
    return fail(FX_EINVAL, "M=%d O=%d K=%d needs %zu bytes of K-split scratch; the allocation-free entry "
                "holds %zu (use fx_w3_gemv with a caller workspace)", M, O, K, need, kNoallocScratchBytes);
  void* ws = nullptr;
  if ((rc = scratch_for_current_device(&ws))) return rc;
  return fx_w3_gemv(x, x_dtype, planes, scales, scale_dtype, zeros, perm, ws, kNoallocScratchBytes, out, M, O,
                    K, arithmetic, stream);
}

// One-row plan with one K split and one tile and batch in flight per wave (the
// residual epilogue and the normalising prologue need all of K in one workgroup).
MfmaPlan single_split_plan(int O, int G) {
  MfmaPlan p = default_mfma_plan(O, G);
  if (p.splits > 1 || p.pd != 1 || p.tiles != 1) p = make_mfma_plan(O, G, 8, 1, G, 1);
  return p;
}

// Payload format check of the one-row entry points.
int check_format(int payload_format) {
  if (payload_format != FX_W3_PLANAR && payload_format != FX_W3_FIELDS && payload_format != FX_W3_FP6)
    return fail(FX_EINVAL, "payload_format must be FX_W3_PLANAR, FX_W3_FIELDS or FX_W3_FP6, got %d", payload_format);
  return FX_OK;
}

// An output index (int16, one entry per output value) must be 2-byte aligned;
// its entries are bounds-checked by the kernels.
int check_out_index(const int16_t* out_index) {
  if (out_index && reinterpret_cast<uintptr_t>(out_index) % 2 != 0)
    return fail(FX_EINVAL, "out_index must be 2-byte aligned");
  return FX_OK;
}

// ------------------------------------------------------------------ field-layout plans
namespace {
// The calling thread's field-layout plan (fx_w3_fields_plan): tiles > 0 a
// shared-staging plan, otherwise the one-tile kernel.
thread_local fx::WidePlan g_fields_plan{0, 0, 0, 0};
constexpr size_t kWideMaxLds = 64 * 1024;
}  // namespace

// Why a shared-staging plan cannot run a shape (null: it can).
const char* wide_plan_misfit(const fx::WidePlan& p, int O, int G, bool perm) {
  if (!fx::wide_plan_instantiated(p)) return "the plan has only the M-row form (fx_w3_gemv_fields_rows)";
  if (O % 16 || G % 4) return "it needs O % 16 == 0 and K % 512 == 0";
  if (G / 4 > p.stage * p.tiles * p.parts) return "K has more batches than its waves stage";
  if (fx::wide_lds_bytes(p.tiles, G, perm) > kWideMaxLds) return "its LDS would exceed 64 KB";
  if (perm && !fx::x_lds_fits(1, G * 128, p.tiles * p.parts)) return "the permuted copy of x does not fit";
  return nullptr;
}

// One-row field-layout launch (one K split; batch payloads on grid.y when
// a.batch is set); epilogue and prologue from a.
int run_fields(const MfmaArgs& base, int x_dtype, int scale_dtype, bool normin, hipStream_t s, int batch = 1) {
  const bool perm = base.perm != nullptr;
  if (normin && perm) return fail(FX_EINVAL, "the normalising prologue takes no permutation");
  // the one-tile kernel unless the thread asked for a shared-staging plan: no such
  // plan measured faster at the Qwen3-8B shapes (per launch or in a strided batch)
  const fx::WidePlan w = g_fields_plan;
  if (w.tiles > 0) {
    if (const char* why = wide_plan_misfit(w, base.O, base.G, perm))
      return fail(FX_EINVAL, "field-layout plan (%d, %d, %d, %d) cannot run O = %d, K = %d: %s", w.tiles, w.parts,
                  w.prefetch, w.stage, base.O, base.G * 128, why);
  }
  if (w.tiles > 0) {
    MfmaArgs a = base;
    a.row_blocks = (base.O / 16 + w.tiles - 1) / w.tiles;
    a.gps = base.G;
    a.x_lds = 0;
    if (batch > 1 && a.row_blocks % 8)
      return fail(FX_EINVAL, "a batch needs XCD-aligned row blocks (a multiple of 8), got %d", a.row_blocks);
    const int mode = normin ? 1 : perm ? 2 : 0;
    if (!fx::dispatch_fields_wide(w, x_dtype, scale_dtype, mode, a, dim3(a.row_blocks, batch), s))
      return fail(FX_EINVAL, "no shared-staging field-layout kernel for this plan and dtype");
    return check_launch("w3_fields_wide_kernel");
  }
  MfmaPlan p = single_split_plan(base.O, base.G);
  const int tiles = fx::fields_row_tiles(normin, base.O);
  if (tiles != p.tiles) p = make_mfma_plan(base.O, base.G, p.nw, 1, base.G, tiles);
  if (batch > 1 && p.row_blocks % 8)
    return fail(FX_EINVAL, "a batch needs O / 16 to be a multiple of 8 (XCD-aligned row blocks), got O = %d", base.O);
  MfmaArgs a = base;
  a.gps = p.gps;
  a.row_blocks = p.row_blocks;
  a.x_lds = a.perm && fx::x_lds_fits(1, base.G * 128, p.nw);
  if (!fx::dispatch_mfma_fields(p.nw, normin, x_dtype, scale_dtype, a, dim3(p.row_blocks, batch), s))
    return fail(FX_EINVAL, "no field-layout MFMA kernel for waves %d", p.nw);
  return check_launch("w3_mfma_kernel (field layout)");
}

// One-row fp6-layout launch (one K split, batch payloads on grid.y when a.batch
// is set): bf16 activations in sorted column order, O % 16 == 0, K % 512 == 0.
int run_fp6(const MfmaArgs& base, int x_dtype, int scale_dtype, bool normin, hipStream_t s, int batch = 1) {
  if (x_dtype != FX_BF16) return fail(FX_EINVAL, "the fp6 layout takes bf16 activations");
  if (base.perm) return fail(FX_EINVAL, "the fp6 layout takes activations in sorted column order (no permutation)");
  if (base.O % 16 || base.G % 4) return fail(FX_EINVAL, "the fp6 layout needs O %% 16 == 0 and K %% 512 == 0");
  MfmaPlan p = single_split_plan(base.O, base.G);
  const int tiles = fx::fields_row_tiles(normin, base.O);
  if (tiles != p.tiles) p = make_mfma_plan(base.O, base.G, p.nw, 1, base.G, tiles);
  if (batch > 1 && p.row_blocks % 8)
    return fail(FX_EINVAL, "a batch needs O / 16 to be a multiple of 8 (XCD-aligned row blocks), got O = %d", base.O);
  MfmaArgs a = base;
  a.gps = p.gps;
  a.row_blocks = p.row_blocks;
  a.x_lds = 0;
  if (!fx::dispatch_mfma_fp6(p.nw, normin, scale_dtype, a, dim3(p.row_blocks, batch), s))
    return fail(FX_EINVAL, "no fp6-layout MFMA kernel for waves %d", p.nw);
  return check_launch("w3_mfma_kernel (fp6 layout)");
}

// Field-layout GEMV of M <= 8 activation rows.  One row: run_fields.  More: the
// M-row kernel (rows padded to MB = 2, 4 or 8); under a plan of several tiles, in
// chunks of four rows where eight rows' staged operands would not fit its LDS
// (K > 4096).  Default plan (measured at the Qwen3-8B shapes): for four or eight
// rows, three tiles x four K parts sharing each staged batch where the row tiles
// fill every CU three times over; else one tile x eight parts up to K = 4096 (a
// batch each), one tile x sixteen parts past it (K <= 16384).
fx::WidePlan default_rows_plan(int O, int G, int mb) {
  const int tiles = O / 16, nb = G / 4;
  if (mb >= 4 && tiles >= 3 * device_cu_count() && nb <= 8) return {3, 4, 2, 1};
  if (nb <= 8) return {1, 8, 1, 1};
  return {1, 16, 2, 2};
}

const char* rows_plan_misfit(const fx::WidePlan& p, int O, int G, int mb) {
  if (O % 16 || G % 4) return "it needs O % 16 == 0 and K % 512 == 0";
  if (G / 4 > p.stage * p.tiles * p.parts) return "K has more batches than its waves stage";
  if (!fx::rows_plan_solo(p) && G / 4 > fx::rows_batch_limit(mb))
    return "K has more batches than its LDS holds for these rows";
  if (16 * p.tiles * mb > 64 * p.tiles * p.parts) return "too few waves for one thread per output value";
  return nullptr;
}

int fx_w3_gemv_fields_rows(const void* x, int x_dtype, const uint8_t* fields, const void* scales, int scale_dtype,
                           const uint8_t* zeros, void* out, int M, int O, int K, void* stream) {
  int rc = validate_payload(x, x_dtype, fields, scales, scale_dtype, M, O, K, FX_ARITH_STRUCTURAL);
  if (rc) return rc;
  if (!out) return fail(FX_EINVAL, "out must be non-null");
  if (M < 1 || M > 8) return fail(FX_EINVAL, "M must be in [1, 8], got %d", M);
  MfmaArgs a{};
  a.planes = fields;
  a.scales = static_cast<const uint16_t*>(scales);
  a.zeros = zeros;
  a.O = O;
  a.G = K / 128;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (M == 1) {
    a.x = static_cast<const uint16_t*>(x);
    a.out = static_cast<uint16_t*>(out);
    return run_fields(a, x_dtype, scale_dtype, false, s);
  }
  for (int done = 0; done < M;) {
    int mb = M - done <= 2 ? 2 : M - done <= 4 ? 4 : 8;
    const fx::WidePlan w = g_fields_plan.tiles > 0 ? g_fields_plan : default_rows_plan(O, a.G, mb);
    // eight rows' operands of every batch exceed the LDS: chunks of four
    if (mb == 8 && !fx::rows_plan_solo(w) && a.G / 4 > fx::rows_batch_limit(8)) mb = 4;
    const int rows = std::min(mb, M - done);
    if (const char* why = rows_plan_misfit(w, O, a.G, mb))
      return fail(FX_EINVAL, "field-layout plan (%d, %d, %d, %d) cannot run %d rows of O = %d, K = %d: %s", w.tiles,
                  w.parts, w.prefetch, w.stage, mb, O, K, why);
    a.x = static_cast<const uint16_t*>(x) + size_t(done) * K;
    a.out = static_cast<uint16_t*>(out) + size_t(done) * O;
    a.row_blocks = (O / 16 + w.tiles - 1) / w.tiles;
    if (!fx::dispatch_fields_rows(w, mb, x_dtype, scale_dtype, a, rows, dim3(a.row_blocks), s))
      return fail(FX_EINVAL, "no M-row field-layout kernel for this plan and dtype");
    if ((rc = check_launch("w3_fields_rows_kernel"))) return rc;
    done += rows;
  }
  return FX_OK;
}

int fx_w3_fields_plan(int tiles, int parts, int prefetch, int stage) {
  if (tiles > 0 && !fx::wide_plan_instantiated(fx::WidePlan{tiles, parts, prefetch, stage}) &&
      !fx::rows_plan_instantiated(fx::WidePlan{tiles, parts, prefetch, stage}))
    return fail(FX_EINVAL, "no shared-staging kernel for plan (%d, %d, %d, %d)", tiles, parts, prefetch, stage);
  g_fields_plan = tiles > 0 ? fx::WidePlan{tiles, parts, prefetch, stage} : fx::WidePlan{tiles < 0 ? -1 : 0, 0, 0, 0};
  return FX_OK;
}


int fx_w3_gemv_swiglu(const void* x, int x_dtype, const uint8_t* planes, const void* scales,
                      int scale_dtype, const uint8_t* zeros, const int16_t* perm, const int16_t* out_index,
                      void* out, int O, int K, int payload_format, void* stream) {
  int rc = validate_payload(x, x_dtype, planes, scales, scale_dtype, 1, O, K, FX_ARITH_STRUCTURAL);
  if (rc) return rc;
  if ((rc = check_format(payload_format))) return rc;
  if ((rc = check_out_index(out_index))) return rc;
  if (!out) return fail(FX_EINVAL, "out must be non-null");
  if (O % 2) return fail(FX_EINVAL, "the interleaved gate|up payload needs an even row count, got %d", O);
  const int G = K / 128;
  if (payload_format == FX_W3_FIELDS) {
    MfmaArgs a{};
    a.x = static_cast<const uint16_t*>(x);
    a.perm = perm;
    a.planes = planes;
    a.scales = static_cast<const uint16_t*>(scales);
    a.zeros = zeros;
    a.out = static_cast<uint16_t*>(out);
    a.O = O;
    a.G = G;
    a.swiglu = 1;
    a.res.ep_index = out_index;
    return run_fields(a, x_dtype, scale_dtype, false, static_cast<hipStream_t>(stream));
  }
  if (payload_format == FX_W3_FP6) {
    MfmaArgs a{};
    a.x = static_cast<const uint16_t*>(x);
    a.perm = perm;
    a.planes = planes;
    a.scales = static_cast<const uint16_t*>(scales);
    a.zeros = zeros;
    a.out = static_cast<uint16_t*>(out);
    a.O = O;
    a.G = G;
    a.swiglu = 1;
    a.res.ep_index = out_index;
    return run_fp6(a, x_dtype, scale_dtype, false, static_cast<hipStream_t>(stream));
  }
  MfmaPlan p = default_mfma_plan(O, G);
  if (p.splits > 1) p = make_mfma_plan(O, G, 8, 1, G, 1);  // the fused epilogue needs one K split
  return run_mfma(x, x_dtype, planes, scales, scale_dtype, zeros, perm, nullptr, 0, out, 1, O, K, p,
                  static_cast<hipStream_t>(stream), 1, out_index);
}

int fx_w3_gemv_residual(const void* x, int x_dtype, const uint8_t* planes, const void* scales,
                        int scale_dtype, const uint8_t* zeros, const int16_t* perm, const void* residual,
                        void* out, float* tile_sumsq, const int16_t* out_index, void* sorted_out, int O, int K,
                        int payload_format, void* stream) {
  int rc = validate_payload(x, x_dtype, planes, scales, scale_dtype, 1, O, K, FX_ARITH_STRUCTURAL);
  if (rc) return rc;
  if ((rc = check_format(payload_format))) return rc;
  if (!residual || !out || !tile_sumsq) return fail(FX_EINVAL, "residual, out and tile_sumsq must be non-null");
  if ((rc = check_out_index(out_index))) return rc;
  if (!out_index != !sorted_out) return fail(FX_EINVAL, "out_index and sorted_out are given together or not at all");
  if (sorted_out && (sorted_out == out || sorted_out == residual))
    return fail(FX_EINVAL, "sorted_out must not alias out or residual");
  const int G = K / 128;
  const MfmaPlan p = single_split_plan(O, G);
  MfmaArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.perm = perm;
  a.planes = planes;
  a.scales = static_cast<const uint16_t*>(scales);
  a.zeros = zeros;
  a.out = static_cast<uint16_t*>(out);
  a.O = O;
  a.G = G;
  a.gps = p.gps;
  a.row_blocks = p.row_blocks;
  a.res.ep_residual = static_cast<const uint16_t*>(residual);
  a.res.ep_partial = tile_sumsq;
  a.res.ep_index = out_index;
  a.res.ep_sorted = static_cast<uint16_t*>(sorted_out);
  if (payload_format == FX_W3_FIELDS) return run_fields(a, x_dtype, scale_dtype, false, static_cast<hipStream_t>(stream));
  if (payload_format == FX_W3_FP6) return run_fp6(a, x_dtype, scale_dtype, false, static_cast<hipStream_t>(stream));
  a.x_lds = perm && fx::x_lds_fits(1, K, p.nw);
  if (!fx::dispatch_mfma(x_dtype, 1, p.nw, 1, 1, scale_dtype, a, dim3(p.row_blocks, 1), static_cast<hipStream_t>(stream)))
    return fail(FX_EINVAL, "no MFMA kernel for waves %d", p.nw);
  return check_launch("w3_mfma_kernel (residual epilogue)");
}

int fx_w3_gemv_rmsnormed(const void* h, int x_dtype, const uint8_t* planes, const void* scales, int scale_dtype,
                         const uint8_t* zeros, const float* tile_sumsq, int n_tiles, const void* norm_weight,
                         float eps, const int16_t* out_index, void* out, int O, int K, int swiglu,
                         int payload_format, void* stream) {
  int rc = validate_payload(h, x_dtype, planes, scales, scale_dtype, 1, O, K, FX_ARITH_STRUCTURAL);
  if (rc) return rc;
  if ((rc = check_format(payload_format))) return rc;
  if ((rc = check_out_index(out_index))) return rc;
  if (out_index && !swiglu) return fail(FX_EINVAL, "out_index applies to the SwiGLU output (swiglu = 1)");
  if (!tile_sumsq || !norm_weight || !out) return fail(FX_EINVAL, "tile_sumsq, norm weight and out must be non-null");
  if (n_tiles != (K + 15) / 16) return fail(FX_EINVAL, "n_tiles must be ceil(K / 16) = %d, got %d", (K + 15) / 16, n_tiles);
  if (n_tiles > 64 * fx::kMaxNormPartialsPerLane) return fail(FX_EINVAL, "K = %d too large for the normalising prologue", K);
  if (reinterpret_cast<uintptr_t>(norm_weight) % 16 != 0) return fail(FX_EINVAL, "norm weight must be 16-byte aligned");
  if (swiglu && O % 2) return fail(FX_EINVAL, "the interleaved gate|up payload needs an even row count, got %d", O);
  const int G = K / 128;
  const MfmaPlan p = single_split_plan(O, G);
  MfmaArgs a{};
  a.x = static_cast<const uint16_t*>(h);
  a.planes = planes;
  a.scales = static_cast<const uint16_t*>(scales);
  a.zeros = zeros;
  a.out = static_cast<uint16_t*>(out);
  a.O = O;
  a.G = G;
  a.gps = p.gps;
  a.row_blocks = p.row_blocks;
  a.swiglu = swiglu ? 1 : 0;
  a.res.pro_partial = tile_sumsq;
  a.res.pro_n = n_tiles;
  a.res.pro_weight = static_cast<const uint16_t*>(norm_weight);
  a.res.pro_eps = eps;
  a.res.ep_index = out_index;
  if (payload_format == FX_W3_FIELDS) return run_fields(a, x_dtype, scale_dtype, true, static_cast<hipStream_t>(stream));
  if (payload_format == FX_W3_FP6) return run_fp6(a, x_dtype, scale_dtype, true, static_cast<hipStream_t>(stream));
  if (!fx::dispatch_mfma_normin(p.nw, x_dtype, scale_dtype, a, dim3(p.row_blocks, 1), static_cast<hipStream_t>(stream)))
    return fail(FX_EINVAL, "no normalising MFMA kernel for waves %d", p.nw);
  return check_launch("w3_mfma_kernel (normalising prologue)");
}

int fx_w3_gemv_strided_batched(const void* x, int x_dtype, long long x_stride, const uint8_t* planes,
                               long long planes_stride, const void* scales, int scale_dtype, long long scales_stride,
                               const uint8_t* zeros, long long zeros_stride, void* out, long long out_stride,
                               int batch, int O, int K, int payload_format, void* stream) {
  int rc = validate_payload(x, x_dtype, planes, scales, scale_dtype, 1, O, K, FX_ARITH_STRUCTURAL);
  if (rc) return rc;
  if ((rc = check_format(payload_format))) return rc;
  if (!out) return fail(FX_EINVAL, "out must be non-null");
  if (batch < 1 || batch > 65535) return fail(FX_EINVAL, "batch must be in [1, 65535], got %d", batch);
  const int G = K / 128;
  const long long planes_bytes = 3LL * G * O * 16;
  if (batch > 1 && (planes_stride < planes_bytes || scales_stride < 1LL * G * O || (zeros && zeros_stride < 1LL * G * O) ||
                    x_stride < K || out_stride < O))
    return fail(FX_EINVAL, "strides must cover one payload, activation row and output row each");
  if (planes_stride % 16 || x_stride % 8)
    return fail(FX_EINVAL, "planes stride must be a multiple of 16 bytes and x stride of 8 elements");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (payload_format == FX_W3_FIELDS || payload_format == FX_W3_FP6) {
    MfmaArgs a{};
    a.x = static_cast<const uint16_t*>(x);
    a.planes = planes;
    a.scales = static_cast<const uint16_t*>(scales);
    a.zeros = zeros;
    a.out = static_cast<uint16_t*>(out);
    a.O = O;
    a.G = G;
    if (batch > 1) a.batch = fx::StridedArgs{x_stride, planes_stride, scales_stride, zeros_stride, out_stride};
    return payload_format == FX_W3_FP6 ? run_fp6(a, x_dtype, scale_dtype, false, s, batch)
                                       : run_fields(a, x_dtype, scale_dtype, false, s, batch);
  }
  MfmaPlan p = single_split_plan(O, G);
  if (batch > 1 && p.row_blocks % 8)
    return fail(FX_EINVAL, "a batch needs O / 16 to be a multiple of 8 (XCD-aligned row blocks), got O = %d", O);
  MfmaArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.planes = planes;
  a.scales = static_cast<const uint16_t*>(scales);
  a.zeros = zeros;
  a.out = static_cast<uint16_t*>(out);
  a.O = O;
  a.G = G;
  a.gps = p.gps;
  a.row_blocks = p.row_blocks;
  if (batch > 1) a.batch = fx::StridedArgs{x_stride, planes_stride, scales_stride, zeros_stride, out_stride};
  const dim3 grid(p.row_blocks, batch);
  if (!fx::dispatch_mfma(x_dtype, 1, p.nw, 1, 1, scale_dtype, a, grid, s))
    return fail(FX_EINVAL, "no MFMA kernel for waves %d", p.nw);
  return check_launch("w3_mfma_kernel (strided batch)");
}

int fx_w3_planes_to_fields(const uint8_t* planes, uint8_t* fields, int O, int K, void* stream) {
  if (!planes || !fields) return fail(FX_EINVAL, "planes and fields must be non-null");
  if (O < 1 || K < 128 || K % 128) return fail(FX_EINVAL, "O must be positive and K a multiple of 128");
  if (reinterpret_cast<uintptr_t>(planes) % 16 != 0 || reinterpret_cast<uintptr_t>(fields) % 16 != 0)
    return fail(FX_EINVAL, "planes and fields must be 16-byte aligned");
  if (planes == fields) return fail(FX_EINVAL, "the repack cannot run in place");
  fx::launch_planes_to_fields(planes, fields, O, K / 128, static_cast<hipStream_t>(stream));
  return check_launch("w3_planes_to_fields_kernel");
}

int fx_w3_planes_to_fp6(const uint8_t* planes, uint8_t* fp6, int O, int K, void* stream) {
  if (!planes || !fp6) return fail(FX_EINVAL, "planes and fp6 must be non-null");
  if (O < 1 || K < 512 || K % 512) return fail(FX_EINVAL, "O must be positive and K a multiple of 512");
  if (reinterpret_cast<uintptr_t>(planes) % 16 != 0 || reinterpret_cast<uintptr_t>(fp6) % 16 != 0)
    return fail(FX_EINVAL, "planes and fp6 must be 16-byte aligned");
  if (planes == fp6) return fail(FX_EINVAL, "the repack cannot run in place");
  fx::launch_planes_to_fp6(planes, fp6, O, K / 128, static_cast<hipStream_t>(stream));
  return check_launch("w3_planes_to_fp6_kernel");
}

int fx_w3_gemv_fp6(const void* x, int x_dtype, const uint8_t* fp6, const void* scales, int scale_dtype,
                   const uint8_t* zeros, void* out, int O, int K, void* stream) {
  int rc = validate_payload(x, x_dtype, fp6, scales, scale_dtype, 1, O, K, FX_ARITH_STRUCTURAL);
  if (rc) return rc;
  if (!out) return fail(FX_EINVAL, "out must be non-null");
  MfmaArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.planes = fp6;
  a.scales = static_cast<const uint16_t*>(scales);
  a.zeros = zeros;
  a.out = static_cast<uint16_t*>(out);
  a.O = O;
  a.G = K / 128;
  return run_fp6(a, x_dtype, scale_dtype, false, static_cast<hipStream_t>(stream));
}

int fx_w3_gemv_fields(const void* x, int x_dtype, const uint8_t* fields, const void* scales, int scale_dtype,
                      const uint8_t* zeros, void* out, int O, int K, void* stream) {
  int rc = validate_payload(x, x_dtype, fields, scales, scale_dtype, 1, O, K, FX_ARITH_STRUCTURAL);
  if (rc) return rc;
  if (!out) return fail(FX_EINVAL, "out must be non-null");
  MfmaArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.planes = fields;
  a.scales = static_cast<const uint16_t*>(scales);
  a.zeros = zeros;
  a.out = static_cast<uint16_t*>(out);
  a.O = O;
  a.G = K / 128;
  return run_fields(a, x_dtype, scale_dtype, false, static_cast<hipStream_t>(stream));
}

size_t fx_w3_gemv_config_workspace_bytes(int M, int O, int K, int waves, int prefetch,
                                         int groups_per_split, int tiles) {
  if (M < 1 || O < 1 || K < 128 || K % 128 || tiles < 1) return 0;
  const int G = K / 128;
  return mfma_workspace(M, O, make_mfma_plan(O, G, waves, prefetch, groups_per_split, tiles));
}

int fx_w3_gemv_config(const void* x, int x_dtype, const uint8_t* planes, const void* scales,
                      int scale_dtype, const uint8_t* zeros, const int16_t* perm, void* workspace,
                      size_t workspace_bytes, void* out, int M, int O, int K, int waves,
                      int prefetch, int groups_per_split, int tiles, void* stream) {
  int rc = validate_payload(x, x_dtype, planes, scales, scale_dtype, M, O, K, FX_ARITH_STRUCTURAL);
  if (rc) return rc;
  if (!out) return fail(FX_EINVAL, "out must be non-null");
  const bool supported = (waves == 4 || waves == 8) &&
                         (prefetch == 1 || prefetch == 2) &&
                         (tiles == 1 || tiles == 2);
  if (!supported)
    return fail(FX_EINVAL, "unsupported waves/prefetch/tiles %d/%d/%d", waves, prefetch, tiles);
  const int G = K / 128;
  if (groups_per_split < 1) return fail(FX_EINVAL, "groups_per_split must be positive");
  return run_mfma(x, x_dtype, planes, scales, scale_dtype, zeros, perm, workspace,
                  workspace_bytes, out, M, O, K,
                  make_mfma_plan(O, G, waves, prefetch, groups_per_split, tiles),
                  static_cast<hipStream_t>(stream));
}

namespace {

// Kernel pointers of the restore instantiations, indexed [scale bf16][weight bf16].
using RestoreFn = void (*)(const uint8_t*, const uint16_t*, const uint8_t*, uint16_t*, int, int, int);
using RestorePermutedFn = void (*)(const uint8_t*, const uint16_t*, const uint8_t*, const int16_t*,
                                   uint16_t*, int, int, int, int, int);
constexpr RestoreFn kRestore[2][2] = {
    {fx::w3_restore_kernel<fx::kF16, fx::kF16>, fx::w3_restore_kernel<fx::kF16, fx::kBF16>},
    {fx::w3_restore_kernel<fx::kBF16, fx::kF16>, fx::w3_restore_kernel<fx::kBF16, fx::kBF16>}};
constexpr RestorePermutedFn kRestorePermuted[2][2] = {
    {fx::w3_restore_permuted_kernel<fx::kF16, fx::kF16>,
     fx::w3_restore_permuted_kernel<fx::kF16, fx::kBF16>},
    {fx::w3_restore_permuted_kernel<fx::kBF16, fx::kF16>,
     fx::w3_restore_permuted_kernel<fx::kBF16, fx::kBF16>}};

}  // namespace

int fx_w3_restore(const uint8_t* planes, const void* scales, int scale_dtype,
                  const uint8_t* zeros, const int16_t* perm, void* weight, int weight_dtype,
                  int O, int K, void* stream) {
  if (!planes || !scales || !weight) return fail(FX_EINVAL, "planes, scales, weight non-null");
  if (!is_half_dtype(scale_dtype) || !is_half_dtype(weight_dtype))
    return fail(FX_EINVAL, "scale and weight dtypes must be fp16 or bf16");
  if (O < 1 || K < 128 || K % 128) return fail(FX_EINVAL, "bad O/K");
  if (perm && K > 32768) return fail(FX_EINVAL, "int16 permutation entries address K <= 32768");
  if (reinterpret_cast<uintptr_t>(planes) % 16 != 0)
    return fail(FX_EINVAL, "planes must be 16-byte aligned");
  const int G = K / 128;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* sc = static_cast<const uint16_t*>(scales);
  uint16_t* w = static_cast<uint16_t*>(weight);
  const int sb = scale_dtype == FX_BF16, wb = weight_dtype == FX_BF16;
  const int weight16 = reinterpret_cast<uintptr_t>(weight) % 16 == 0;
  if (!perm) {
    // one workgroup per (16-row block, kRestoreGroups groups)
    const size_t blocks =
        size_t((O + 15) / 16) * size_t((G + fx::kRestoreGroups - 1) / fx::kRestoreGroups);
    if (blocks > size_t(INT32_MAX)) return fail(FX_EINVAL, "O * K too large");
    hipLaunchKernelGGL(kRestore[sb][wb], dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s,
                       planes, sc, zeros, w, O, G, weight16);
    return check_launch("w3_restore_kernel");
  }
  // whole rows staged in LDS: at most 32 KB for K <= 16384, one row (<= 64 KB) above
  const int rows = std::max(1, fx::kRestoreStageBytes / (2 * K));
  const int perm16 = reinterpret_cast<uintptr_t>(perm) % 16 == 0;
  hipLaunchKernelGGL(kRestorePermuted[sb][wb], dim3((O + rows - 1) / rows),
                     dim3(fx::kRestoreStageThreads), size_t(rows) * K * 2, s, planes, sc, zeros,
                     perm, w, O, G, rows, weight16, perm16);
  return check_launch("w3_restore_permuted_kernel");
}

int fx_rmsnorm(const void* x, const void* residual, const void* weight, void* out,
               void* residual_out, int rows, int hidden, float eps, int dtype, void* stream) {
  if (!x || !weight || !out) return fail(FX_EINVAL, "x, weight and out must be non-null");
  if (residual && !residual_out) return fail(FX_EINVAL, "a residual needs residual_out");
  if (!is_half_dtype(dtype)) return fail(FX_EINVAL, "dtype must be fp16 or bf16");
  if (rows < 1 || hidden < 8 || hidden % 8 != 0 || hidden > (1 << 20))
    return fail(FX_EINVAL, "rows must be positive and hidden a multiple of 8, got %d x %d", rows, hidden);
  const void* ptrs[5] = {x, residual, weight, out, residual_out};
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return fail(FX_EINVAL, "tensors must be 16-byte aligned");
  if (!(eps >= 0.f)) return fail(FX_EINVAL, "eps must be non-negative");
  fx::launch_rmsnorm(dtype, static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(residual),
                     static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out),
                     static_cast<uint16_t*>(residual_out), rows, hidden, eps,
                     static_cast<hipStream_t>(stream));
  return check_launch("rmsnorm_kernel");
}

int fx_head_norm_rope(int ntensors, const void* const* inputs, void* const* outputs,
                      const void* const* weights, const int* heads, const int* rope,
                      const long long* strides, int batch, int seq, int head_dim,
                      const void* cos, const void* sin, const long long* cos_strides,
                      const int* position, float eps, int rope_mode, int dtype, void* stream) {
  if (ntensors < 1 || ntensors > fx::kMaxHeadTensors)
    return fail(FX_EINVAL, "ntensors must be in [1,%d]", fx::kMaxHeadTensors);
  if (!inputs || !outputs || !heads || !rope || !strides)
    return fail(FX_EINVAL, "tensor arrays must be non-null");
  if (!is_half_dtype(dtype)) return fail(FX_EINVAL, "dtype must be fp16 or bf16");
  if (batch < 1 || seq < 1 || head_dim < 2 || head_dim % 2 || head_dim > 4096)
    return fail(FX_EINVAL, "bad batch/seq/head_dim %d/%d/%d", batch, seq, head_dim);
  if (rope_mode < fx::kRopeNone || rope_mode > fx::kRopeFused)
    return fail(FX_EINVAL, "unknown rope_mode %d", rope_mode);
  if (!(eps >= 0.f)) return fail(FX_EINVAL, "eps must be non-negative");
  fx::HeadNormRopeArgs a = {};
  a.ntensors = ntensors;
  a.seq = seq;
  a.head_dim = head_dim;
  a.eps = eps;
  a.rope_mode = rope_mode;
  a.position = position;
  bool any_rope = false;
  long long total_rows = 0;
  for (int i = 0; i < ntensors; ++i) {
    if (!inputs[i] || !outputs[i]) return fail(FX_EINVAL, "tensor %d: null input or output", i);
    if (heads[i] < 1) return fail(FX_EINVAL, "tensor %d: heads must be positive", i);
    fx::HeadTensor& t = a.t[i];
    t.in = inputs[i];
    t.out = outputs[i];
    t.weight = weights ? weights[i] : nullptr;
    for (int j = 0; j < 3; ++j) {
      t.in_stride[j] = strides[6 * i + j];
      t.out_stride[j] = strides[6 * i + 3 + j];
    }
    t.heads = heads[i];
    t.rope = rope[i] ? 1 : 0;
    any_rope = any_rope || (t.rope && rope_mode != fx::kRopeNone);
    const long long r = (long long)batch * heads[i] * seq;
    if (r > (1 << 24)) return fail(FX_EINVAL, "tensor %d: too many rows", i);
    a.rows[i] = int(r);
    total_rows += r;
  }
  if (total_rows > (1 << 26)) return fail(FX_EINVAL, "too many rows");
  if (any_rope) {
    if (!cos || !sin || !cos_strides) return fail(FX_EINVAL, "RoPE needs cos, sin and their strides");
    a.cos = cos;
    a.sin = sin;
    a.cs_stride[0] = cos_strides[0];
    a.cs_stride[1] = cos_strides[1];
  }
  fx::launch_head_norm_rope(dtype, a, static_cast<hipStream_t>(stream));
  return check_launch("head_norm_rope_kernel");
}

// Query-head groups per attention split workgroup (decode.hip: group g scores
// heads g * 4 / groups, ... of the KV head).
constexpr int kAttnDefaultGroups = 1;

// Attention workspace: the fp32 partials, [Hq, splits, D] outputs then
// [Hq, splits, 2] (max, sum).
size_t fx_decode_attention_workspace_bytes(int n_q_heads, int max_len, int head_dim) {
  if (n_q_heads < 1 || max_len < 1 || (head_dim != 64 && head_dim != 128 && head_dim != 256)) return 0;
  // the most splits any position can use: one key per thread
  const int keys = fx::attn_keys_per_block(head_dim, 1);
  const size_t splits = (size_t(max_len) + keys - 1) / keys;
  return size_t(n_q_heads) * splits * (size_t(head_dim) + 2) * sizeof(float);
}

namespace {
// The calling thread's attention plan (fx_decode_attention_plan): 0 = the default.
thread_local int g_attn_kpt = 0, g_attn_groups = 0;

int decode_attention(const void* q, const void* k_cache, const void* v_cache, void* workspace,
                     size_t workspace_bytes, void* out, int n_q_heads, int n_kv_heads, int max_len,
                     int head_dim, int position, float scale, int dtype, void* stream,
                     const fx::AttnPre& pre, const int16_t* out_index) {
  if (!q || !k_cache || !v_cache || !out) return fail(FX_EINVAL, "q, caches and out must be non-null");
  if (int rc = check_out_index(out_index)) return rc;
  if (!is_half_dtype(dtype)) return fail(FX_EINVAL, "dtype must be fp16 or bf16");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(FX_EINVAL, "head_dim must be 64, 128 or 256, got %d", head_dim);
  if (n_kv_heads < 1 || n_q_heads < n_kv_heads || n_q_heads % n_kv_heads)
    return fail(FX_EINVAL, "query heads %d must be a positive multiple of KV heads %d", n_q_heads, n_kv_heads);
  if (max_len < 1 || max_len > (1 << 22) || position < 0 || position >= max_len)
    return fail(FX_EINVAL, "position %d outside the cache [0, %d)", position, max_len);
  const void* vec[5] = {q, k_cache, v_cache, out, nullptr};
  for (int i = 0; i < 3; ++i)
    if (reinterpret_cast<uintptr_t>(vec[i]) % 16 != 0) return fail(FX_EINVAL, "q and caches must be 16-byte aligned");
  const size_t need = fx_decode_attention_workspace_bytes(n_q_heads, max_len, head_dim);
  if (!workspace || workspace_bytes < need)
    return fail(FX_EINVAL, "attention workspace needs %zu bytes, got %zu", need, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) return fail(FX_EINVAL, "workspace must be 16-byte aligned");
  fx::AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k_cache);
  a.v = static_cast<const uint16_t*>(v_cache);
  a.partial = static_cast<float*>(workspace);
  a.out = static_cast<uint16_t*>(out);
  a.out_index = out_index;
  a.Hq = n_q_heads;
  a.Hk = n_kv_heads;
  a.Lmax = max_len;
  a.pos = position;
  // keys per thread: one split (direct output) when some kpt covers the
  // context in one workgroup; else the kpt with the fewest keys per CU
  // (ceil(workgroups / CUs) * kpt, the split launch's bytes on its busiest CU),
  // ties to the larger kpt (fewer partials for the combine launch)
  const int n = position + 1, cus = device_cu_count();
  const auto splits_for = [&](int kpt) {
    const int keys = fx::attn_keys_per_block(head_dim, kpt);
    return (n + keys - 1) / keys;
  };
  a.kpt = 0;
  for (int kpt : {1, 2, 4})
    if (splits_for(kpt) == 1) {
      a.kpt = kpt;
      break;
    }
  if (a.kpt == 0) {
    long best = 0;
    for (int kpt : {4, 2, 1}) {
      const long load = (long(n_kv_heads) * splits_for(kpt) + cus - 1) / cus * kpt;
      if (a.kpt == 0 || load < best) {
        a.kpt = kpt;
        best = load;
      }
    }
  }
  if (g_attn_kpt) a.kpt = g_attn_kpt;
  a.splits = splits_for(a.kpt);
  // query-head groups: a group per kAttnHeadsPerPass / groups heads, no more
  // groups than a KV head has query heads
  const int per_kv = n_q_heads / n_kv_heads;
  a.groups = g_attn_groups ? g_attn_groups : kAttnDefaultGroups;
  while (a.groups > 1 && a.groups > per_kv) a.groups /= 2;
  if (a.splits > 65535) return fail(FX_EINVAL, "position %d needs %d key splits (at most 65535)", position, a.splits);
  a.scale = scale;
  a.pre = pre;
  fx::launch_decode_attention(dtype, head_dim, a, static_cast<hipStream_t>(stream));
  return check_launch("attn_split_kernel");
}

}  // namespace

int fx_decode_attention_plan(int keys_per_thread, int head_groups) {
  if (keys_per_thread != 0 && keys_per_thread != 1 && keys_per_thread != 2 && keys_per_thread != 4)
    return fail(FX_EINVAL, "keys_per_thread must be 0 (default), 1, 2 or 4, got %d", keys_per_thread);
  if (head_groups != 0 && head_groups != 1 && head_groups != 2 && head_groups != 4)
    return fail(FX_EINVAL, "head_groups must be 0 (default), 1, 2 or 4, got %d", head_groups);
  g_attn_kpt = keys_per_thread;
  g_attn_groups = head_groups;
  return FX_OK;
}

int fx_decode_attention(const void* q, const void* k_cache, const void* v_cache, void* workspace,
                        size_t workspace_bytes, const int16_t* out_index, void* out, int n_q_heads,
                        int n_kv_heads, int max_len, int head_dim, int position, float scale, int dtype,
                        void* stream) {
  return decode_attention(q, k_cache, v_cache, workspace, workspace_bytes, out, n_q_heads, n_kv_heads, max_len,
                          head_dim, position, scale, dtype, stream, fx::AttnPre{}, out_index);
}

int fx_decode_attention_rope(const void* q, const void* k, const void* v, const void* q_norm_weight,
                             const void* k_norm_weight, const void* cos, const void* sin, float eps,
                             int rope_mode, void* k_cache, void* v_cache, void* workspace,
                             size_t workspace_bytes, const int16_t* out_index, void* out, int n_q_heads,
                             int n_kv_heads, int max_len, int head_dim, int position, float scale, int dtype,
                             void* stream) {
  if (!k || !v || !q_norm_weight || !k_norm_weight || !cos || !sin)
    return fail(FX_EINVAL, "raw k, v, norm weights, cos and sin must be non-null");
  if (rope_mode != FX_ROPE_STOCK && rope_mode != FX_ROPE_FUSED)
    return fail(FX_EINVAL, "rope_mode must be FX_ROPE_STOCK or FX_ROPE_FUSED");
  const void* vec[6] = {k, v, q_norm_weight, k_norm_weight, cos, sin};
  for (const void* p : vec)
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
      return fail(FX_EINVAL, "raw k, v, norm weights, cos and sin must be 16-byte aligned");
  fx::AttnPre pre{static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                  static_cast<const uint16_t*>(q_norm_weight), static_cast<const uint16_t*>(k_norm_weight),
                  static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin), eps, rope_mode};
  return decode_attention(q, k_cache, v_cache, workspace, workspace_bytes, out, n_q_heads, n_kv_heads, max_len,
                          head_dim, position, scale, dtype, stream, pre, out_index);
}

// LM head: one workgroup per CU (4 waves, one 8 KB row in flight per wave at
// hidden 4096: 32 KB per CU), fewer when the vocabulary has fewer rows.  Measured
// at 151936 x 4096 (HIP events, 20 calls): 177.0 us against 189.8 us for two
// workgroups per CU with two rows per wave (128 KB per CU in flight); a plain
// streaming read of the same 1.24 GB peaks at 24-32 KB per CU in flight too
// (7.3 TB/s) and falls to 5-6 TB/s at 64-128 KB.
constexpr int kLmBlocksPerCu = 1;

size_t fx_lm_head_argmax_workspace_bytes(void) {
  return fx::kLmCounterBytes + size_t(fx::kLmMaxBlocks) * (sizeof(float) + sizeof(int));
}

namespace {
// The workspace's partial arrays and the grid of a vocab-row LM head (the same
// for the streaming launch and a later merge of its partials).
int lm_head_workspace(void* workspace, size_t workspace_bytes, int vocab, fx::LmHeadArgs* a) {
  if (!workspace) return fail(FX_EINVAL, "workspace must be non-null");
  if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) return fail(FX_EINVAL, "workspace must be 16-byte aligned");
  const size_t need = fx_lm_head_argmax_workspace_bytes();
  if (workspace_bytes < need)
    return fail(FX_EINVAL, "LM-head workspace needs %zu bytes, got %zu", need, workspace_bytes);
  if (vocab < 1) return fail(FX_EINVAL, "vocab must be positive, got %d", vocab);
  a->arrival = static_cast<unsigned*>(workspace);
  a->part_val = reinterpret_cast<float*>(static_cast<char*>(workspace) + fx::kLmCounterBytes);
  a->part_idx = reinterpret_cast<int*>(a->part_val + fx::kLmMaxBlocks);
  a->V = vocab;
  const long groups = (long(vocab) + fx::kLmRowsInFlight - 1) / fx::kLmRowsInFlight;  // one wave's rows at a time
  a->blocks = int(std::min<long>({long(fx::kLmMaxBlocks), long(kLmBlocksPerCu) * device_cu_count(),
                                  (groups + fx::kLmWaves - 1) / fx::kLmWaves}));
  return FX_OK;
}

int lm_head_args(const void* hidden, const void* norm_weight, float eps, const void* weight, void* logits,
                 void* workspace, size_t workspace_bytes, int vocab, int hidden_size, int dtype, fx::LmHeadArgs* a) {
  if (!hidden || !weight || !logits) return fail(FX_EINVAL, "hidden, weight, logits and workspace must be non-null");
  if (!is_half_dtype(dtype)) return fail(FX_EINVAL, "dtype must be fp16 or bf16");
  if (hidden_size < 512 || hidden_size > 512 * fx::kLmMaxChunks || hidden_size % 512)
    return fail(FX_EINVAL, "hidden size must be a multiple of 512 in [512, %d], got %d", 512 * fx::kLmMaxChunks,
                hidden_size);
  const void* vec[3] = {hidden, norm_weight, weight};
  for (const void* p : vec)
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
      return fail(FX_EINVAL, "hidden, norm weight and weight must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(logits) % 2 != 0) return fail(FX_EINVAL, "logits must be 2-byte aligned");
  int rc = lm_head_workspace(workspace, workspace_bytes, vocab, a);
  if (rc) return rc;
  a->x = static_cast<const uint16_t*>(hidden);
  a->norm_w = static_cast<const uint16_t*>(norm_weight);
  a->eps = eps;
  a->w = static_cast<const uint16_t*>(weight);
  a->logits = static_cast<uint16_t*>(logits);
  a->K = hidden_size;
  return FX_OK;
}
}  // namespace

int fx_lm_head_argmax(const void* hidden, const void* norm_weight, float eps, const void* weight, void* logits,
                      long long* prediction, void* workspace, size_t workspace_bytes, int vocab,
                      int hidden_size, int dtype, void* stream) {
  if (!prediction) return fail(FX_EINVAL, "hidden, weight, logits, prediction and workspace must be non-null");
  if (reinterpret_cast<uintptr_t>(prediction) % 8 != 0) return fail(FX_EINVAL, "prediction must be 8-byte aligned");
  fx::LmHeadArgs a{};
  int rc = lm_head_args(hidden, norm_weight, eps, weight, logits, workspace, workspace_bytes, vocab, hidden_size,
                        dtype, &a);
  if (rc) return rc;
  a.prediction = prediction;
  fx::launch_lm_head_argmax(dtype, a, static_cast<hipStream_t>(stream));
  return check_launch("lm_head_argmax_kernel");
}

int fx_lm_head_logits(const void* hidden, const void* norm_weight, float eps, const void* weight, void* logits,
                      void* workspace, size_t workspace_bytes, int vocab, int hidden_size, int dtype, void* stream) {
  fx::LmHeadArgs a{};
  int rc = lm_head_args(hidden, norm_weight, eps, weight, logits, workspace, workspace_bytes, vocab, hidden_size,
                        dtype, &a);
  if (rc) return rc;
  fx::launch_lm_head_partials(dtype, a, static_cast<hipStream_t>(stream));
  return check_launch("lm_head_argmax_kernel");
}

int fx_lm_head_merge(void* workspace, size_t workspace_bytes, int vocab, long long* prediction, void* stream) {
  if (!prediction) return fail(FX_EINVAL, "prediction must be non-null");
  if (reinterpret_cast<uintptr_t>(prediction) % 8 != 0) return fail(FX_EINVAL, "prediction must be 8-byte aligned");
  fx::LmHeadArgs a{};
  int rc = lm_head_workspace(workspace, workspace_bytes, vocab, &a);
  if (rc) return rc;
  a.prediction = prediction;
  fx::launch_lm_head_merge(a, static_cast<hipStream_t>(stream));
  return check_launch("lm_head_merge_kernel");
}

int fx_decode_embed(const long long* token, const void* table, int vocab, int hidden, void* out, float* tile_sumsq,
                    const int16_t* out_index, void* sorted_out, void* lm_workspace, size_t lm_workspace_bytes,
                    int lm_vocab, long long* prediction, int dtype, void* stream) {
  if (!token || !table || !out || !tile_sumsq) return fail(FX_EINVAL, "token, table, out and tile_sumsq must be non-null");
  if (!out_index != !sorted_out) return fail(FX_EINVAL, "out_index and sorted_out are given together or not at all");
  if (out_index && reinterpret_cast<uintptr_t>(out_index) % 16 != 0)
    return fail(FX_EINVAL, "out_index must be 16-byte aligned");
  if (sorted_out && (sorted_out == out || reinterpret_cast<uintptr_t>(sorted_out) % 2 != 0))
    return fail(FX_EINVAL, "sorted_out must be 2-byte aligned and must not alias out");
  if (!is_half_dtype(dtype)) return fail(FX_EINVAL, "dtype must be fp16 or bf16");
  if (vocab < 1) return fail(FX_EINVAL, "vocab must be positive, got %d", vocab);
  if (hidden < 16 || hidden % 16 || hidden > (1 << 20))
    return fail(FX_EINVAL, "hidden must be a positive multiple of 16, got %d", hidden);
  if (reinterpret_cast<uintptr_t>(table) % 16 || reinterpret_cast<uintptr_t>(out) % 16 ||
      reinterpret_cast<uintptr_t>(token) % 8 || reinterpret_cast<uintptr_t>(tile_sumsq) % 4)
    return fail(FX_EINVAL, "table and out must be 16-byte aligned, token 8-byte and tile_sumsq 4-byte aligned");
  fx::LmHeadArgs merge{};
  if (prediction) {
    if (reinterpret_cast<uintptr_t>(prediction) % 8 != 0)
      return fail(FX_EINVAL, "prediction must be 8-byte aligned");
    int rc = lm_head_workspace(lm_workspace, lm_workspace_bytes, lm_vocab, &merge);
    if (rc) return rc;
    merge.prediction = prediction;
  }
  if (!fx::launch_decode_embed(dtype, token, static_cast<const uint16_t*>(table), vocab, hidden,
                               static_cast<uint16_t*>(out), tile_sumsq, out_index, static_cast<uint16_t*>(sorted_out),
                               merge, static_cast<hipStream_t>(stream)))
    return fail(FX_EINVAL, "no embedding kernel for dtype %d", dtype);
  return check_launch("decode_embed_kernel");
}

int fx_silu_mul(const void* gate, const void* up, void* out, int n, int dtype, void* stream) {
  if (!gate || !up || !out) return fail(FX_EINVAL, "gate, up and out must be non-null");
  if (!is_half_dtype(dtype)) return fail(FX_EINVAL, "dtype must be fp16 or bf16");
  if (n < 1) return fail(FX_EINVAL, "n must be positive");
  fx::launch_silu_mul(dtype, static_cast<const uint16_t*>(gate), static_cast<const uint16_t*>(up),
                      static_cast<uint16_t*>(out), n, static_cast<hipStream_t>(stream));
  return check_launch("silu_mul_kernel");
}

size_t fx_two_base_gemv_workspace_bytes(int O, int K) {
  if (O < 1 || K < 128 || K % 128) return 0;
  return two_base_workspace(O, default_two_base_plan(O, K / 128));
}

int fx_two_base_gemv(const void* x, int x_dtype, const uint8_t* planes, const void* coef,
                     const void* srow, const void* tcol, const void* salient,
                     const int32_t* salient_idx, int n_salient, void* workspace,
                     size_t workspace_bytes, void* out, int O, int K, void* stream) {
  if (O < 1 || K < 128 || K % 128)
    return fail(FX_EINVAL, "O must be positive and K a positive multiple of 128, got %d/%d", O, K);
  return run_rank_one(x, x_dtype, planes, coef, srow, tcol, salient, salient_idx, n_salient,
                      workspace, workspace_bytes, out, O, K, default_two_base_plan(O, K / 128),
                      static_cast<hipStream_t>(stream));
}

size_t fx_two_base_gemv_config_workspace_bytes(int O, int K, int waves, int prefetch,
                                               int groups_per_split, int tiles) {
  TwoBasePlan p;
  if (O < 1 || K < 128 || K % 128 || !two_base_config(O, K / 128, waves, prefetch, groups_per_split, tiles, &p))
    return 0;
  return two_base_workspace(O, p);
}

int fx_two_base_gemv_config(const void* x, int x_dtype, const uint8_t* planes, const void* coef,
                            const void* srow, const void* tcol, const void* salient,
                            const int32_t* salient_idx, int n_salient, void* workspace,
                            size_t workspace_bytes, void* out, int O, int K, int waves,
                            int prefetch, int groups_per_split, int tiles, void* stream) {
  if (O < 1 || K < 128 || K % 128)
    return fail(FX_EINVAL, "O must be positive and K a positive multiple of 128, got %d/%d", O, K);
  TwoBasePlan p;
  if (!two_base_config(O, K / 128, waves, prefetch, groups_per_split, tiles, &p))
    return fail(FX_EINVAL, "unsupported waves/prefetch/tiles %d/%d/%d", waves, prefetch, tiles);
  return run_rank_one(x, x_dtype, planes, coef, srow, tcol, salient, salient_idx, n_salient,
                      workspace, workspace_bytes, out, O, K, p, static_cast<hipStream_t>(stream));
}

size_t fx_hybrid_gemv_workspace_bytes(int O, int K) {
  if (O < 1 || K < 128 || K % 128) return 0;
  return two_base_workspace(O, default_hybrid_plan(O, K / 128, 1 << 20));
}

int fx_hybrid_gemv(const void* x, int x_dtype, const uint8_t* codes, const float* rows,
                   const float* columns, const int16_t* indices, const uint8_t* sparse_codes,
                   const float* sparse_rows, const float* sparse_columns, void* workspace,
                   size_t workspace_bytes, void* out, int O, int K, void* stream) {
  if (O < 1 || O > 65536) return fail(FX_EINVAL, "O must be in [1, 65536], got %d", O);
  if (!columns || !indices || !sparse_columns)
    return fail(FX_EINVAL, "x, every layout field and out must be non-null");
  return run_hybrid(x, x_dtype, 1, &O, codes, rows, &columns, &indices, sparse_codes, sparse_rows, &sparse_columns,
                    workspace, workspace_bytes, out, K, fx::ResidualArgs{}, false, static_cast<hipStream_t>(stream));
}

int fx_hybrid_gemv_segments(const void* x, int x_dtype, int n_segments, const int* segment_rows,
                            const uint8_t* codes, const float* rows, const float* const* columns,
                            const int16_t* const* indices, const uint8_t* sparse_codes, const float* sparse_rows,
                            const float* const* sparse_columns, void* workspace, size_t workspace_bytes, void* out,
                            int K, void* stream) {
  return run_hybrid(x, x_dtype, n_segments, segment_rows, codes, rows, columns, indices, sparse_codes, sparse_rows,
                    sparse_columns, workspace, workspace_bytes, out, K, fx::ResidualArgs{}, false,
                    static_cast<hipStream_t>(stream));
}

int fx_hybrid_gemv_residual(const void* x, int x_dtype, const uint8_t* codes, const float* rows,
                            const float* columns, const int16_t* indices, const uint8_t* sparse_codes,
                            const float* sparse_rows, const float* sparse_columns, const void* residual, void* out,
                            float* tile_sumsq, int O, int K, int swiglu, void* stream) {
  if (O < 1 || O > 65536) return fail(FX_EINVAL, "O must be in [1, 65536], got %d", O);
  if (!columns || !indices || !sparse_columns)
    return fail(FX_EINVAL, "x, every layout field and out must be non-null");
  if (!residual || !out || !tile_sumsq) return fail(FX_EINVAL, "residual, out and tile_sumsq must be non-null");
  fx::ResidualArgs res{};
  res.ep_residual = static_cast<const uint16_t*>(residual);
  res.ep_partial = tile_sumsq;
  return run_hybrid(x, x_dtype, 1, &O, codes, rows, &columns, &indices, sparse_codes, sparse_rows, &sparse_columns,
                    nullptr, 0, out, K, res, swiglu != 0, static_cast<hipStream_t>(stream));
}

int fx_hybrid_gemv_segments_rmsnormed(const void* h, int x_dtype, int n_segments, const int* segment_rows,
                                      const uint8_t* codes, const float* rows, const float* const* columns,
                                      const int16_t* const* indices, const uint8_t* sparse_codes,
                                      const float* sparse_rows, const float* const* sparse_columns,
                                      const float* tile_sumsq, int n_tiles, const void* norm_weight, float eps,
                                      void* workspace, size_t workspace_bytes, void* out, int K, void* stream) {
  if (!tile_sumsq || !norm_weight) return fail(FX_EINVAL, "tile_sumsq and norm weight must be non-null");
  if (n_tiles != (K + 15) / 16) return fail(FX_EINVAL, "n_tiles must be ceil(K / 16) = %d, got %d", (K + 15) / 16, n_tiles);
  if (n_tiles > 64 * fx::kMaxNormPartialsPerLane) return fail(FX_EINVAL, "K = %d too large for the normalising prologue", K);
  if (reinterpret_cast<uintptr_t>(norm_weight) % 16 != 0) return fail(FX_EINVAL, "norm weight must be 16-byte aligned");
  fx::ResidualArgs res{};
  res.pro_partial = tile_sumsq;
  res.pro_n = n_tiles;
  res.pro_weight = static_cast<const uint16_t*>(norm_weight);
  res.pro_eps = eps;
  return run_hybrid(h, x_dtype, n_segments, segment_rows, codes, rows, columns, indices, sparse_codes, sparse_rows,
                    sparse_columns, workspace, workspace_bytes, out, K, res, false, static_cast<hipStream_t>(stream));
}

}  // extern "C"
