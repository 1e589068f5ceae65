// Qwen3 RMSNorm (optionally fused with the residual add) and per-head
// RMSNorm + rotary embedding for gfx950, single pass over each row, fp32
// reductions across the wavefront (DPP / xor shuffles) and LDS.
//
// Rounding points are those of the stock HF modules the reference patches
// (fused_modules.py:30-85, transformers modeling_qwen3.py Qwen3RMSNorm /
// apply_rotary_pos_emb):
//   s      = round(x + residual)                      (fused residual add)
//   normed = round(fp32(s) * rsqrt(mean(fp32(s)^2) + eps))
//   y      = round(weight * normed)
//   rope   = round(round(y * cos) + round(rotate_half(y) * sin))   stock
//          = round(round(y * cos) + rotate_half(y) * sin)          fused (addcmul)
// where round() is the cast to the tensor dtype (bf16 or fp16).
#include "common.h"
#include "norms_launch.h"

namespace fx {

typedef unsigned u32x4n_t __attribute__((ext_vector_type(4)));

template <int DT>
__device__ __forceinline__ float rnd(float v) { return round_to<DT>(v); }

// rows x hidden, hidden % 8 == 0.  TPR threads per row (64 or 256), 256 threads
// per block.  s = round(x + residual) (written to residual_out) or x; the sum of
// s^2 in the shared 512-element batch order (wave w of a row takes batches
// w, w + TPR/64, ...; lanes past the row read zeros); y = round(w * round(s * inv)).
// When a lane's chunks fit in registers (hidden <= kNormRegChunks * 512 * TPR/64)
// every load -- x, residual and weight -- is issued before the first use and y
// is formed from registers: one global round trip.  Longer rows re-read s (their
// own chunks, so in-place calls are safe).
constexpr int kMaxNormBatches = (1 << 20) / kNormBatch;
constexpr int kNormRegChunks = 4;
template <int DT, int TPR>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ residual,
                                                      const uint16_t* __restrict__ weight,
                                                      uint16_t* out, uint16_t* residual_out,
                                                      int rows, int hidden, float eps) {
  asm volatile("" ::"s"(x), "s"(residual), "s"(weight), "s"(out), "s"(residual_out), "s"(rows), "s"(hidden),
               "s"(eps));
  constexpr int kRowsPerBlock = 256 / TPR, kWavesPerRow = TPR / 64;
  __shared__ float bsum[kWavesPerRow > 1 ? kMaxNormBatches : 1];
  const int t = threadIdx.x;
  // the row from the scalar wave index: t / TPR looks lane-dependent to the
  // compiler, which then built the row's descriptors in VGPRs (waterfall loops)
  const int local = wave_index() / (TPR / 64), tl = t % TPR;
  const int row = blockIdx.x * kRowsPerBlock + local;
  const bool live = row < rows;
  const int chunks = hidden / 8;
  const int nb = (hidden + kNormBatch - 1) / kNormBatch;
  const int wr = tl / 64, lane = tl & 63;
  const size_t base = size_t(live ? row : 0) * hidden;

  if (nb <= kNormRegChunks * kWavesPerRow) {
    const auto rx = buffer_resource(x + base, size_t(hidden) * 2);
    const auto rr = buffer_resource(residual ? residual + base : x, residual ? size_t(hidden) * 2 : 0);
    const auto rw = buffer_resource(weight, size_t(hidden) * 2);
    u32x4_t sv[kNormRegChunks], wv[kNormRegChunks], rv[kNormRegChunks];
    bool ok[kNormRegChunks];
#pragma unroll
    for (int q = 0; q < kNormRegChunks; ++q) {
      const int c = 64 * (wr + q * kWavesPerRow) + lane;
      ok[q] = live && c < chunks;
      const int off = ok[q] ? c * 16 : kOutOfRange;
      sv[q] = load_b128(rx, off, 0);
      rv[q] = load_b128(rr, off, 0);
      wv[q] = load_b128(rw, off, 0);
    }
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < kNormRegChunks; ++q) {
      const int b = wr + q * kWavesPerRow;
      if (b >= nb) break;  // wave-uniform
      if (residual) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float lo = rnd<DT>(to_f32<DT>(uint16_t(sv[q][w])) + to_f32<DT>(uint16_t(rv[q][w])));
          const float hi = rnd<DT>(to_f32<DT>(uint16_t(sv[q][w] >> 16)) + to_f32<DT>(uint16_t(rv[q][w] >> 16)));
          sv[q][w] = unsigned(from_f32<DT>(lo)) | (unsigned(from_f32<DT>(hi)) << 16);
        }
        if (ok[q]) *reinterpret_cast<u32x4_t*>(residual_out + base + 8 * (64 * b + lane)) = sv[q];
      }
      const float bs = wave_total(sum_sq8<DT>(sv[q]));
      if constexpr (kWavesPerRow == 1) ss += bs;  // batch order
      else if (lane == 0) bsum[b] = bs;
    }
    if constexpr (kWavesPerRow > 1) {
      __syncthreads();
      for (int b = 0; b < nb; ++b) ss += bsum[b];
    }
    const float inv = rsqrtf(ss / float(hidden) + eps);
#pragma unroll
    for (int q = 0; q < kNormRegChunks; ++q) {
      if (!ok[q]) continue;
      u32x4_t yv;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float n0 = rnd<DT>(to_f32<DT>(uint16_t(sv[q][w])) * inv);
        const float n1 = rnd<DT>(to_f32<DT>(uint16_t(sv[q][w] >> 16)) * inv);
        const float y0 = to_f32<DT>(uint16_t(wv[q][w])) * n0;
        const float y1 = to_f32<DT>(uint16_t(wv[q][w] >> 16)) * n1;
        yv[w] = unsigned(from_f32<DT>(y0)) | (unsigned(from_f32<DT>(y1)) << 16);
      }
      *reinterpret_cast<u32x4_t*>(out + base + 8 * (64 * (wr + q * kWavesPerRow) + lane)) = yv;
    }
    return;
  }

  // with a residual, pass 2 reads the rounded sum back from residual_out
  const uint16_t* src = residual ? residual_out : x;
  float ss = 0.f;
  for (int b = wr; b < nb; b += kWavesPerRow) {
    const int c = 64 * b + lane;
    u32x4n_t xv = {0u, 0u, 0u, 0u};
    if (live && c < chunks) {
      xv = *reinterpret_cast<const u32x4n_t*>(x + base + 8 * c);
      if (residual) {
        const u32x4n_t rv = *reinterpret_cast<const u32x4n_t*>(residual + base + 8 * c);
        u32x4n_t sv;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float lo = rnd<DT>(to_f32<DT>(uint16_t(xv[w])) + to_f32<DT>(uint16_t(rv[w])));
          const float hi = rnd<DT>(to_f32<DT>(uint16_t(xv[w] >> 16)) + to_f32<DT>(uint16_t(rv[w] >> 16)));
          sv[w] = unsigned(from_f32<DT>(lo)) | (unsigned(from_f32<DT>(hi)) << 16);
        }
        *reinterpret_cast<u32x4n_t*>(residual_out + base + 8 * c) = sv;
        xv = sv;
      }
    }
    const float bs = wave_total(sum_sq8<DT>(__builtin_bit_cast(u32x4_t, xv)));
    if constexpr (kWavesPerRow == 1) ss += bs;  // batch order
    else if (lane == 0) bsum[b] = bs;
  }
  if constexpr (kWavesPerRow > 1) {
    __syncthreads();
    for (int b = 0; b < nb; ++b) ss += bsum[b];
  }
  if (!live) return;
  const float inv = rsqrtf(ss / float(hidden) + eps);
  for (int c = tl; c < chunks; c += TPR) {
    const u32x4n_t sv = *reinterpret_cast<const u32x4n_t*>(src + base + 8 * c);
    const u32x4n_t wv = *reinterpret_cast<const u32x4n_t*>(weight + 8 * c);
    u32x4n_t yv;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float n0 = rnd<DT>(to_f32<DT>(uint16_t(sv[w])) * inv);
      const float n1 = rnd<DT>(to_f32<DT>(uint16_t(sv[w] >> 16)) * inv);
      const float y0 = to_f32<DT>(uint16_t(wv[w])) * n0;
      const float y1 = to_f32<DT>(uint16_t(wv[w] >> 16)) * n1;
      yv[w] = unsigned(from_f32<DT>(y0)) | (unsigned(from_f32<DT>(y1)) << 16);
    }
    *reinterpret_cast<u32x4n_t*>(out + base + 8 * c) = yv;
  }
}

// One wave per (tensor, batch, head, position) row of head_dim values.  Lane l
// owns the rotate-half pairs (i, i + D/2) for i = l, l + 64, ... < D/2, so the
// rotation needs no lane exchange.
template <int DT>
__global__ __launch_bounds__(256) void head_norm_rope_kernel(HeadNormRopeArgs a) {
  const int lane = threadIdx.x & 63;
  // a row belongs to one wave: select its tensor with scalar (wave-uniform)
  // values so the descriptors are read with scalar loads
  int row = __builtin_amdgcn_readfirstlane(int(blockIdx.x) * 4 + int(threadIdx.x >> 6));
  int ti = 0;
  while (ti < a.ntensors && row >= a.rows[ti]) {
    row -= a.rows[ti];
    ++ti;
  }
  if (ti >= a.ntensors) return;
  ti = __builtin_amdgcn_readfirstlane(ti);
  row = __builtin_amdgcn_readfirstlane(row);
  const HeadTensor& T = a.t[ti];
  const int S = a.seq, H = T.heads;
  const int b = row / (H * S), h = (row / S) % H, s = row % S;
  const uint16_t* in = static_cast<const uint16_t*>(T.in) + b * T.in_stride[0] + h * T.in_stride[1] +
                       s * T.in_stride[2];
  uint16_t* out = static_cast<uint16_t*>(T.out) + b * T.out_stride[0] + h * T.out_stride[1] +
                  s * T.out_stride[2];
  const int half = a.head_dim / 2;
  const uint16_t* w = static_cast<const uint16_t*>(T.weight);

  float inv = 1.f;
  if (w) {
    float ss = 0.f;
    for (int i = lane; i < half; i += 64) {
      const float lo = to_f32<DT>(in[i]), hi = to_f32<DT>(in[i + half]);
      ss += lo * lo + hi * hi;
    }
    ss = wave_total(ss);
    inv = rsqrtf(ss / float(a.head_dim) + a.eps);
  }
  const bool rope = T.rope && a.rope_mode != kRopeNone;
  const uint16_t* cs = nullptr;
  const uint16_t* sn = nullptr;
  if (rope) {
    long long pos_off = b * a.cs_stride[0] + s * a.cs_stride[1];
    if (a.position) pos_off += (long long)(a.position[0]) * a.head_dim;
    cs = static_cast<const uint16_t*>(a.cos) + pos_off;
    sn = static_cast<const uint16_t*>(a.sin) + pos_off;
  }
  for (int i = lane; i < half; i += 64) {
    float lo = to_f32<DT>(in[i]), hi = to_f32<DT>(in[i + half]);
    if (w) {
      lo = rnd<DT>(to_f32<DT>(w[i]) * rnd<DT>(lo * inv));
      hi = rnd<DT>(to_f32<DT>(w[i + half]) * rnd<DT>(hi * inv));
    }
    if (rope) {
      const float c0 = to_f32<DT>(cs[i]), c1 = to_f32<DT>(cs[i + half]);
      const float s0 = to_f32<DT>(sn[i]), s1 = to_f32<DT>(sn[i + half]);
      // rotate_half(y) = (-y[half:], y[:half])
      float r0 = -hi * s0, r1 = lo * s1;
      if (a.rope_mode == kRopeStock) {
        r0 = rnd<DT>(r0);
        r1 = rnd<DT>(r1);
      }
      const float o0 = rnd<DT>(lo * c0) + r0;
      const float o1 = rnd<DT>(hi * c1) + r1;
      lo = o0;
      hi = o1;
    }
    out[i] = from_f32<DT>(lo);
    out[i + half] = from_f32<DT>(hi);
  }
}

bool launch_rmsnorm(int dt, const uint16_t* x, const uint16_t* residual, const uint16_t* weight,
                    uint16_t* out, uint16_t* residual_out, int rows, int hidden, float eps,
                    hipStream_t s) {
  const bool wide = hidden > 1024;
  const int rpb = wide ? 1 : 4;
  const dim3 grid((rows + rpb - 1) / rpb);
  if (dt == kBF16) {
    if (wide) hipLaunchKernelGGL((rmsnorm_kernel<kBF16, 256>), grid, dim3(256), 0, s, x, residual, weight, out, residual_out, rows, hidden, eps);
    else hipLaunchKernelGGL((rmsnorm_kernel<kBF16, 64>), grid, dim3(256), 0, s, x, residual, weight, out, residual_out, rows, hidden, eps);
  } else if (dt == kF16) {
    if (wide) hipLaunchKernelGGL((rmsnorm_kernel<kF16, 256>), grid, dim3(256), 0, s, x, residual, weight, out, residual_out, rows, hidden, eps);
    else hipLaunchKernelGGL((rmsnorm_kernel<kF16, 64>), grid, dim3(256), 0, s, x, residual, weight, out, residual_out, rows, hidden, eps);
  } else {
    return false;
  }
  return true;
}

bool launch_head_norm_rope(int dt, const HeadNormRopeArgs& a, hipStream_t s) {
  int total = 0;
  for (int i = 0; i < a.ntensors; ++i) total += a.rows[i];
  const dim3 grid((total + 3) / 4);
  if (dt == kBF16) hipLaunchKernelGGL(head_norm_rope_kernel<kBF16>, grid, dim3(256), 0, s, a);
  else if (dt == kF16) hipLaunchKernelGGL(head_norm_rope_kernel<kF16>, grid, dim3(256), 0, s, a);
  else return false;
  return true;
}

}  // namespace fx
