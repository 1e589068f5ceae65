// extern "C" boundary of libfluxbin_amd.so (declarations: include/fluxbin_amd.h).
// Validates arguments, picks kernel instantiations and tilings, launches on the
// caller's stream.  Nothing here allocates or synchronises.
#include <cstdio>
#include <cstdarg>
#include <cstring>
#include <mutex>

#include "../../include/fluxbin_amd.h"
#include "common.h"
#include "w3_lut_launch.h"
#include "w3_lut.hip"

using fx::LutArgs;

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
  if (arithmetic != FX_ARITH_STRUCTURAL && arithmetic != FX_ARITH_DECODED_BF16)
    return fail(FX_EINVAL, "unknown arithmetic %d", arithmetic);
  if (arithmetic == FX_ARITH_DECODED_BF16 && scale_dtype != FX_BF16)
    return fail(FX_EINVAL, "decoded_bf16 arithmetic requires bf16 scales");
  return FX_OK;
}

int rows_per_thread_from_tile(int row_tile) {
  switch (row_tile) {
    case 256: return 1;
    case 512: return 2;
    case 1024: return 4;
    default: return -1;
  }
}

// Largest supported activation-row block not above m.
int m_block_for(int m) { return m >= 8 ? 8 : m >= 4 ? 4 : m >= 2 ? 2 : 1; }

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct Tile {
  int rpt, gps, splits, row_tiles;
};

Tile make_tile(int O, int G, int rpt, int gps) {
  Tile t;
  t.rpt = rpt;
  t.gps = gps < 1 ? 1 : (gps > G ? G : gps);
  t.splits = (G + t.gps - 1) / t.gps;
  t.row_tiles = (O + fx::kLutThreads * rpt - 1) / (fx::kLutThreads * rpt);
  return t;
}

// Default tiling: one row per thread, enough K splits to give every CU about
// two workgroups.
Tile default_tile(int M, int O, int K) {
  const int G = K / 128;
  const int rpt = 1;
  const int row_tiles = (O + fx::kLutThreads * rpt - 1) / (fx::kLutThreads * rpt);
  const int target = 2 * device_cu_count();
  int splits = (target + row_tiles - 1) / row_tiles;
  if (splits < 1) splits = 1;
  if (splits > G) splits = G;
  const int gps = (G + splits - 1) / splits;
  (void)M;
  return make_tile(O, G, rpt, gps);
}

size_t fused_workspace_bytes(int M, int O, const Tile& t) {
  if (t.splits == 1) return 0;
  const int mb = m_block_for(M);
  return align_up(size_t(t.row_tiles) * sizeof(unsigned), 256) +
         size_t(t.splits) * size_t(mb) * size_t(O) * sizeof(float);
}

// Launch the GEMV over all M rows in blocks of 8/4/2/1 activation rows.
int run_lut(const void* x, int x_dtype, const uint8_t* planes, const void* scales, int scale_dtype,
            const uint8_t* zeros, const int16_t* perm, float* partial, unsigned* counters,
            void* out, int M, int O, int K, int arithmetic, const Tile& tile, int mode,
            hipStream_t stream) {
  const int G = K / 128;
  const bool dec = arithmetic == FX_ARITH_DECODED_BF16;
  int done = 0;
  while (done < M) {
    const int mb = m_block_for(M - done);
    LutArgs a;
    a.x = static_cast<const uint16_t*>(x) + size_t(done) * K;
    a.planes = planes;
    a.scales = static_cast<const uint16_t*>(scales);
    a.zeros = zeros;
    a.perm = perm;
    a.partial = partial;
    a.counters = counters;
    a.out = static_cast<uint16_t*>(out) + size_t(done) * O;
    a.O = O;
    a.G = G;
    a.gps = tile.gps;
    a.splits = tile.splits;
    a.mode = tile.splits == 1 && mode != fx::kModePartial ? fx::kModeDirect : mode;
    // In partial mode each M block writes its own slice of the [splits, M, O]
    // buffer; the kernel indexes partial[(s*mb + m)*O + o], so blocks after the
    // first use a separate region.
    if (mode == fx::kModePartial && partial)
      a.partial = partial + size_t(tile.splits) * size_t(done) * O;
    const dim3 grid(tile.row_tiles, tile.splits);
    if (!fx::dispatch_lut(mb, tile.rpt, x_dtype, scale_dtype, dec, a, grid, stream))
      return fail(FX_EINVAL, "no kernel for M-block %d rpt %d dtypes %d/%d", mb, tile.rpt,
                  x_dtype, scale_dtype);
    int rc = check_launch("w3_lut_kernel");
    if (rc) return rc;
    done += mb;
  }
  return FX_OK;
}

}  // namespace

extern "C" {

int fx_abi_version(void) { return 1; }

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
  Tile tile = make_tile(O, G, rpt, groups_per_split);
  // Partial mode writes [splits, M, O]; M blocks are laid out per block (see run_lut),
  // which equals [splits, M, O] only when M is a single block.
  if (m_block_for(M) != M) return fail(FX_EINVAL, "inline_main supports M in {1,2,4,8}");
  return run_lut(x, x_dtype, planes, scales, scale_dtype, zeros, perm, partial, nullptr, nullptr,
                 M, O, K, arithmetic, tile, fx::kModePartial, static_cast<hipStream_t>(stream));
}

int fx_w3_finish(const float* partial, void* out, int out_dtype, int splits, int M, int O,
                 void* stream) {
  if (!partial || !out) return fail(FX_EINVAL, "partial and out must be non-null");
  if (!is_half_dtype(out_dtype)) return fail(FX_EINVAL, "out dtype must be fp16 or bf16");
  if (splits < 1 || M < 1 || O < 1) return fail(FX_EINVAL, "splits, M and O must be positive");
  const int MO = M * O;
  const dim3 grid((MO + 255) / 256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (out_dtype == FX_BF16)
    hipLaunchKernelGGL(fx::w3_finish_kernel<fx::kBF16>, grid, dim3(256), 0, s, partial,
                       static_cast<uint16_t*>(out), MO, splits);
  else
    hipLaunchKernelGGL(fx::w3_finish_kernel<fx::kF16>, grid, dim3(256), 0, s, partial,
                       static_cast<uint16_t*>(out), MO, splits);
  return check_launch("w3_finish_kernel");
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
  if (m_block_for(M) != M) return fail(FX_EINVAL, "m1_out supports M in {1,2,4,8}");
  Tile tile = make_tile(O, G, rpt, groups_per_split);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (tile.splits == 1)
    return run_lut(x, x_dtype, planes, scales, scale_dtype, zeros, perm, nullptr, nullptr, out,
                   M, O, K, arithmetic, tile, fx::kModeDirect, s);
  if (!workspace) return fail(FX_EINVAL, "workspace must be non-null when K is split");
  rc = run_lut(x, x_dtype, planes, scales, scale_dtype, zeros, perm, workspace, nullptr, nullptr,
               M, O, K, arithmetic, tile, fx::kModePartial, s);
  if (rc) return rc;
  return fx_w3_finish(workspace, out, x_dtype, tile.splits, M, O, stream);
}

size_t fx_w3_gemv_workspace_bytes(int M, int O, int K) {
  if (M < 1 || O < 1 || K < 128 || K % 128) return 0;
  return fused_workspace_bytes(M, O, default_tile(M, O, K));
}

size_t fx_w3_gemv_tile_workspace_bytes(int M, int O, int K, int rows_per_thread,
                                       int groups_per_split) {
  if (M < 1 || O < 1 || K < 128 || K % 128) return 0;
  return fused_workspace_bytes(M, O, make_tile(O, K / 128, rows_per_thread, groups_per_split));
}

static int gemv_with_tile(const void* x, int x_dtype, const uint8_t* planes, const void* scales,
                          int scale_dtype, const uint8_t* zeros, const int16_t* perm,
                          void* workspace, size_t workspace_bytes, void* out, int M, int O, int K,
                          int arithmetic, const Tile& tile, hipStream_t s) {
  if (!out) return fail(FX_EINVAL, "out must be non-null");
  if (tile.splits == 1)
    return run_lut(x, x_dtype, planes, scales, scale_dtype, zeros, perm, nullptr, nullptr, out, M,
                   O, K, arithmetic, tile, fx::kModeDirect, s);
  const size_t need = fused_workspace_bytes(M, O, tile);
  if (!workspace || workspace_bytes < need)
    return fail(FX_EINVAL, "workspace needs %zu bytes, got %zu", need, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
    return fail(FX_EINVAL, "workspace must be 256-byte aligned");
  unsigned* counters = static_cast<unsigned*>(workspace);
  float* partial = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                            align_up(size_t(tile.row_tiles) * sizeof(unsigned), 256));
  return run_lut(x, x_dtype, planes, scales, scale_dtype, zeros, perm, partial, counters, out, M,
                 O, K, arithmetic, tile, fx::kModeFused, s);
}

int fx_w3_gemv(const void* x, int x_dtype, const uint8_t* planes, const void* scales,
               int scale_dtype, const uint8_t* zeros, const int16_t* perm, void* workspace,
               size_t workspace_bytes, void* out, int M, int O, int K, int arithmetic,
               void* stream) {
  int rc = validate_payload(x, x_dtype, planes, scales, scale_dtype, M, O, K, arithmetic);
  if (rc) return rc;
  return gemv_with_tile(x, x_dtype, planes, scales, scale_dtype, zeros, perm, workspace,
                        workspace_bytes, out, M, O, K, arithmetic, default_tile(M, O, K),
                        static_cast<hipStream_t>(stream));
}

int fx_w3_gemv_tile(const void* x, int x_dtype, const uint8_t* planes, const void* scales,
                    int scale_dtype, const uint8_t* zeros, const int16_t* perm, void* workspace,
                    size_t workspace_bytes, void* out, int M, int O, int K, int arithmetic,
                    int rows_per_thread, int groups_per_split, void* stream) {
  int rc = validate_payload(x, x_dtype, planes, scales, scale_dtype, M, O, K, arithmetic);
  if (rc) return rc;
  if (rows_per_thread != 1 && rows_per_thread != 2 && rows_per_thread != 4)
    return fail(FX_EINVAL, "rows_per_thread must be 1, 2 or 4");
  const int G = K / 128;
  if (groups_per_split < 1 || groups_per_split > G)
    return fail(FX_EINVAL, "groups_per_split must be in [1, K/128]");
  return gemv_with_tile(x, x_dtype, planes, scales, scale_dtype, zeros, perm, workspace,
                        workspace_bytes, out, M, O, K, arithmetic,
                        make_tile(O, G, rows_per_thread, groups_per_split),
                        static_cast<hipStream_t>(stream));
}

int fx_w3_restore(const uint8_t* planes, const void* scales, int scale_dtype,
                  const uint8_t* zeros, const int16_t* perm, void* weight, int weight_dtype,
                  int O, int K, void* stream) {
  if (!planes || !scales || !weight) return fail(FX_EINVAL, "planes, scales, weight non-null");
  if (!is_half_dtype(scale_dtype) || !is_half_dtype(weight_dtype))
    return fail(FX_EINVAL, "scale and weight dtypes must be fp16 or bf16");
  if (O < 1 || K < 128 || K % 128) return fail(FX_EINVAL, "bad O/K");
  if (reinterpret_cast<uintptr_t>(planes) % 16 != 0)
    return fail(FX_EINVAL, "planes must be 16-byte aligned");
  const int G = K / 128;
  const dim3 grid((O * G + 255) / 256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* sc = static_cast<const uint16_t*>(scales);
  uint16_t* w = static_cast<uint16_t*>(weight);
  if (scale_dtype == FX_BF16 && weight_dtype == FX_BF16)
    hipLaunchKernelGGL((fx::w3_restore_kernel<fx::kBF16, fx::kBF16>), grid, dim3(256), 0, s,
                       planes, sc, zeros, perm, w, O, G);
  else if (scale_dtype == FX_BF16 && weight_dtype == FX_F16)
    hipLaunchKernelGGL((fx::w3_restore_kernel<fx::kBF16, fx::kF16>), grid, dim3(256), 0, s,
                       planes, sc, zeros, perm, w, O, G);
  else if (scale_dtype == FX_F16 && weight_dtype == FX_BF16)
    hipLaunchKernelGGL((fx::w3_restore_kernel<fx::kF16, fx::kBF16>), grid, dim3(256), 0, s,
                       planes, sc, zeros, perm, w, O, G);
  else
    hipLaunchKernelGGL((fx::w3_restore_kernel<fx::kF16, fx::kF16>), grid, dim3(256), 0, s, planes,
                       sc, zeros, perm, w, O, G);
  return check_launch("w3_restore_kernel");
}

}  // extern "C"
