// Batch-1 decode kernels for gfx950: grouped-query attention over a static KV
// cache (split over key chunks, then combined), and the SwiGLU activation.
//
// Attention semantics (stock HF Qwen3 attention through SDPA with a boolean
// mask): for query head h of KV head g = h / (Hq / Hk),
//   s_j = (q_h . k_{g,j}) * scale            j = 0 .. pos (later slots masked)
//   o_h = sum_j softmax(s)_j v_{g,j}
// with fp32 scores, probabilities and accumulation (SDPA's math form), rounded
// once to the activation dtype.  KV cache layout [Hk, Lmax, D].
#include "common.h"
#include "decode_launch.h"

namespace fx {

typedef unsigned u32x4d_t __attribute__((ext_vector_type(4)));

constexpr int kAttnChunk = 64;  // keys per workgroup (one per lane)

// grid (Hk, ceil(Lmax / 64)), 256 threads: wave w serves query heads
// g*G + w, g*G + w + 4, ... (G = Hq / Hk).  Lane l scores key chunk*64 + l, then
// the wave accumulates P.V with lane l owning output dims l, l + 64, ...
// partial[(h * splits + chunk) * (D + 2)] = {running max m, sum l, o[0..D)}.
template <int DT, int D>
__global__ __launch_bounds__(256) void attn_split_kernel(const uint16_t* __restrict__ q,
                                                         const uint16_t* __restrict__ kc,
                                                         const uint16_t* __restrict__ vc,
                                                         float* __restrict__ partial, int Hq, int Hk,
                                                         int Lmax, int pos, float scale) {
  __shared__ float qs[4][D];
  __shared__ float ps[4][kAttnChunk];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = blockIdx.x, chunk = blockIdx.y, splits = gridDim.y;
  const int G = Hq / Hk;
  const int j = chunk * kAttnChunk + lane;
  const bool live = j <= pos;
  const int first = chunk * kAttnChunk;
  for (int hl = wave; hl < G; hl += 4) {
    const int h = g * G + hl;
    float* out = partial + (size_t(h) * splits + chunk) * (D + 2);
    if (first > pos) {  // chunk entirely in the future: empty partial
      if (lane == 0) {
        out[0] = -INFINITY;
        out[1] = 0.f;
      }
      for (int d = lane; d < D; d += 64) out[2 + d] = 0.f;
      continue;
    }
    for (int d = lane; d < D; d += 64) qs[wave][d] = to_f32<DT>(q[size_t(h) * D + d]);
    __builtin_amdgcn_wave_barrier();
    float s = -INFINITY;
    if (live) {
      const uint16_t* krow = kc + (size_t(g) * Lmax + j) * D;
      float acc = 0.f;
#pragma unroll 4
      for (int d = 0; d < D; d += 8) {
        const u32x4d_t kv = *reinterpret_cast<const u32x4d_t*>(krow + d);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          acc += qs[wave][d + 2 * w] * to_f32<DT>(uint16_t(kv[w]));
          acc += qs[wave][d + 2 * w + 1] * to_f32<DT>(uint16_t(kv[w] >> 16));
        }
      }
      s = acc * scale;
    }
    const float m = wave_max(s);  // finite: key `first` <= pos is live
    const float p = live ? __expf(s - m) : 0.f;
    const float l = wave_sum(p);
    ps[wave][lane] = p;
    __builtin_amdgcn_wave_barrier();
    const int keys = min(kAttnChunk, pos - first + 1);
    float o[D / 64];
#pragma unroll
    for (int i = 0; i < D / 64; ++i) o[i] = 0.f;
    const uint16_t* vbase = vc + (size_t(g) * Lmax + first) * D;
    for (int jj = 0; jj < keys; ++jj) {
      const float pj = ps[wave][jj];
#pragma unroll
      for (int i = 0; i < D / 64; ++i) o[i] += pj * to_f32<DT>(vbase[size_t(jj) * D + lane + 64 * i]);
    }
    if (lane == 0) {
      out[0] = m;
      out[1] = l;
    }
#pragma unroll
    for (int i = 0; i < D / 64; ++i) out[2 + lane + 64 * i] = o[i];
    __builtin_amdgcn_wave_barrier();  // qs / ps reused by this wave's next head
  }
}

// grid Hq, 64 threads: o_h = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c.
template <int DT, int D>
__global__ __launch_bounds__(64) void attn_combine_kernel(const float* __restrict__ partial,
                                                          uint16_t* __restrict__ out, int splits) {
  const int h = blockIdx.x, lane = threadIdx.x;
  const float* base = partial + size_t(h) * splits * (D + 2);
  float M = -INFINITY;
  for (int c = 0; c < splits; ++c) M = fmaxf(M, base[size_t(c) * (D + 2)]);
  float L = 0.f;
  float o[D / 64];
#pragma unroll
  for (int i = 0; i < D / 64; ++i) o[i] = 0.f;
  for (int c = 0; c < splits; ++c) {
    const float* pc = base + size_t(c) * (D + 2);
    const float mc = pc[0];
    if (mc == -INFINITY) continue;
    const float w = __expf(mc - M);
    L += w * pc[1];
#pragma unroll
    for (int i = 0; i < D / 64; ++i) o[i] += w * pc[2 + lane + 64 * i];
  }
  const float inv = 1.f / L;
#pragma unroll
  for (int i = 0; i < D / 64; ++i) out[size_t(h) * D + lane + 64 * i] = from_f32<DT>(o[i] * inv);
}

// SwiGLU of Qwen3MLP: act = round(round(silu(gate)) * up), silu(g) = g / (1 + e^-g).
template <int DT>
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gate,
                                                       const uint16_t* __restrict__ up,
                                                       uint16_t* __restrict__ out, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float g = to_f32<DT>(gate[i]);
  const float s = round_to<DT>(g / (1.f + __expf(-g)));
  out[i] = from_f32<DT>(s * to_f32<DT>(up[i]));
}

template <int DT>
bool attn_for_dim(int D, const AttnArgs& a, hipStream_t s) {
  const dim3 grid(a.Hk, a.splits);
  if (D == 128) {
    hipLaunchKernelGGL((attn_split_kernel<DT, 128>), grid, dim3(256), 0, s, a.q, a.k, a.v, a.partial, a.Hq, a.Hk, a.Lmax, a.pos, a.scale);
    hipLaunchKernelGGL((attn_combine_kernel<DT, 128>), dim3(a.Hq), dim3(64), 0, s, a.partial, a.out, a.splits);
  } else if (D == 64) {
    hipLaunchKernelGGL((attn_split_kernel<DT, 64>), grid, dim3(256), 0, s, a.q, a.k, a.v, a.partial, a.Hq, a.Hk, a.Lmax, a.pos, a.scale);
    hipLaunchKernelGGL((attn_combine_kernel<DT, 64>), dim3(a.Hq), dim3(64), 0, s, a.partial, a.out, a.splits);
  } else if (D == 256) {
    hipLaunchKernelGGL((attn_split_kernel<DT, 256>), grid, dim3(256), 0, s, a.q, a.k, a.v, a.partial, a.Hq, a.Hk, a.Lmax, a.pos, a.scale);
    hipLaunchKernelGGL((attn_combine_kernel<DT, 256>), dim3(a.Hq), dim3(64), 0, s, a.partial, a.out, a.splits);
  } else {
    return false;
  }
  return true;
}

bool launch_decode_attention(int dt, int D, const AttnArgs& a, hipStream_t s) {
  if (dt == kBF16) return attn_for_dim<kBF16>(D, a, s);
  if (dt == kF16) return attn_for_dim<kF16>(D, a, s);
  return false;
}

bool launch_silu_mul(int dt, const uint16_t* gate, const uint16_t* up, uint16_t* out, int n,
                     hipStream_t s) {
  const dim3 grid((n + 255) / 256);
  if (dt == kBF16) hipLaunchKernelGGL(silu_mul_kernel<kBF16>, grid, dim3(256), 0, s, gate, up, out, n);
  else if (dt == kF16) hipLaunchKernelGGL(silu_mul_kernel<kF16>, grid, dim3(256), 0, s, gate, up, out, n);
  else return false;
  return true;
}

}  // namespace fx
