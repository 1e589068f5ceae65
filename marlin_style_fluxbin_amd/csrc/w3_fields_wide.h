// Field-layout GEMVs with workgroup-shared activation staging: the one-row form
// (w3_fields_wide_kernel, plans for sweeps and tests) and the M-row form
// (w3_fields_rows_kernel, the default of fx_w3_gemv_fields_rows, further down).
//
// A workgroup owns T 16-row tiles and splits K into P parts: wave (tile, part)
// multiplies its tile by the batches (4 groups, 512 columns) of its part.  The
// workgroup builds the B operands of every batch once (wave w stages batches w,
// w + T P, ...) into LDS, so the T tiles share one staging instead of each wave
// staging the batch it multiplies; each wave keeps PD batches of weights in
// flight and issues them before any wait.
//
// Same arithmetic, same bits as the one-tile field-layout kernel (w3_mfma.hip)
// for every plan: the same B operands (stage_fields8), the same 16-MFMA chain
// per batch and epilogue term (accumulate_group), and the same K order -- the
// eight "virtual waves" k = 0..7 of a row each sum batches k, k + 8, ... in
// turn, their group slots meet through the same two DPP adds, and the eight
// sums are added in k order.  Part p serves virtual waves p, p + P, ... and
// walks each one's batches before the next, so a wave holds one accumulator set.
//
// Measured on MI355X at the Qwen3-8B shapes, it is not the default: no plan beat
// the one-tile kernel per launch (gate/up 12288 x 4096: 6.25 us one-tile, 6.81
// at (1,8,1,1), 7.36 at (3,4,2,1)), and in a strided batch of 50 payloads it won
// 2-7% only at the narrow shapes.  The counters show why: VALU per weight fell
// (304 -> 213 per wave-batch at (3,4,2,1)) but every wave waits at the barrier
// after the staging for the slowest wave of its workgroup, and a wave's serial
// chain got longer (wave cycles 2510 -> 3467), which is what bounds a launch
// whose loads all issue at once.  The plans stay for sweeps and the
// plan-independence tests (fx_w3_fields_plan).
//
// Issue order: norm partials and output indices, the activations (and norm
// weights or column indices) of the wave's staged batches, then the weight ring
// (planes, non-temporal, then scales and zero-points).  Loads complete in issue
// order, so the staging waits only for the L2-resident activations.
#pragma once
#include "w3_mfma.hip"
#include "w3_mfma_launch.h"

namespace fx {

static_assert(kWideStage == 4 * kStageStride<1> && kWideVirtualWaves == kSumLanes, "LDS layout of wide_lds_bytes");

template <int T, int P, int PD, int S, int XDT, int SDT, bool NORMIN, bool PERM>
__global__ __launch_bounds__(T * P * 64) void w3_fields_wide_kernel(
    const uint16_t* __restrict__ x, const int16_t* __restrict__ perm, const uint8_t* __restrict__ fields,
    const uint16_t* __restrict__ scales, const uint8_t* __restrict__ zeros, uint16_t* out, int O, int G,
    int row_blocks, int swiglu, ResidualArgs ra, StridedArgs sb) {
  constexpr int NW = T * P;
  static_assert(kSumLanes % P == 0, "parts must divide the eight virtual waves");
  static_assert(16 * T <= 64 * NW, "one thread per output row");
  static_assert(!(PERM && NORMIN), "the normalising prologue reads its activations in sorted order");
  asm volatile("" ::"s"(x), "s"(perm), "s"(fields), "s"(scales), "s"(zeros), "s"(out), "s"(O), "s"(G),
               "s"(row_blocks), "s"(swiglu), "s"(ra.ep_residual), "s"(ra.ep_partial), "s"(ra.ep_index),
               "s"(ra.ep_sorted), "s"(sb.x), "s"(sb.planes), "s"(sb.scales), "s"(sb.zeros), "s"(sb.out));
  if constexpr (NORMIN)
    asm volatile("" ::"s"(ra.pro_partial), "s"(ra.pro_n), "s"(ra.pro_weight), "s"(ra.pro_eps));
  if (sb.planes) {  // strided batch: grid.y walks the payloads
    const long long p = blockIdx.y;
    x += p * sb.x;
    fields += p * sb.planes;
    scales += p * sb.scales;
    if (zeros) zeros += p * sb.zeros;
    out += p * sb.out;
  }
  const int nbatch = (G + 3) >> 2;
  extern __shared__ u32x4_t lds[];
  u32x4_t* bst = lds;                                            // [nbatch][4 k-blocks][kStageStride]
  u32x4_t* bzero = bst + nbatch * kWideStage;                    // [16 steps]
  float* gsum = reinterpret_cast<float*>(bzero + 16);            // [nbatch][4]
  int* gexp = reinterpret_cast<int*>(gsum + 4 * nbatch);         // [nbatch][4]
  float* red = reinterpret_cast<float*>(gexp + 4 * nbatch);      // [8 virtual waves][16 T rows]
  u32x4_t* xs = reinterpret_cast<u32x4_t*>(red + kSumLanes * 16 * T);  // PERM: x [K]

  const int t = threadIdx.x, lane = t & 63, wave = wave_index();
  const int part = wave % P, tile = wave / P;
  const int K = G * 128;
  const int row_base = xcd_local_index8(blockIdx.x, row_blocks) * (16 * T);
  const int row0 = row_base + 16 * tile;
  const unsigned zero_default = zeros ? 0u : 0x04040404u;

  const unsigned go = unsigned(G) * unsigned(O);
  const auto rp = buffer_resource_2g(fields, go * 48u);
  const auto rs = buffer_resource_2g(scales, go * 2u);
  const auto rz = buffer_resource_2g(zeros ? (const void*)zeros : (const void*)scales, zeros ? go : 0u);
  const auto rx = buffer_resource_2g(x, unsigned(K) * 2u);
  const auto rperm = buffer_resource(PERM ? (const void*)perm : (const void*)x, PERM ? size_t(K) * 2 : 0);
  const auto rwn = buffer_resource(NORMIN ? (const void*)ra.pro_weight : (const void*)x, NORMIN ? size_t(K) * 2 : 0);

  float pp[kMaxNormPartialsPerLane];
  if constexpr (NORMIN) {
    const auto rpp = buffer_resource(ra.pro_partial, size_t(ra.pro_n) * 4);
#pragma unroll
    for (int k = 0; k < kMaxNormPartialsPerLane; ++k) {
      const int idx = lane + 64 * k;
      pp[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rpp, idx < ra.pro_n ? idx * 4 : kOutOfRange, 0, 0));
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // the output index of this thread's epilogue row (residual: row row_base + t;
  // SwiGLU: pair row_base / 2 + t)
  int ep_to = -1;
  if (ra.ep_index) {
    const int n_idx = ra.ep_residual ? O : O / 2;
    const int at = ra.ep_residual ? (t < 16 * T ? row_base + t : n_idx) : (2 * t < 16 * T ? row_base / 2 + t : n_idx);
    const auto rix = buffer_resource(ra.ep_index, size_t(n_idx) * 2);
    ep_to = int(int16_t(__builtin_amdgcn_raw_buffer_load_b16(rix, at < n_idx ? at * 2 : kOutOfRange, 0, 0)));
  }

  const int r = lane & 15;   // A role: row within tile; x role: 8-column chunk
  const int kb = lane >> 4;  // A role: k-block = group slot; D role: row block
  const int c = lane & 15;   // B / D role: column (c < 4: group slot c of the one activation row)
  const int cslot = c & 3;

  // staging loads: batch wave + NW i of the workgroup, this lane's 8 columns
  u32x4_t sx[S], sw[NORMIN ? S : 1];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    const int b = wave + NW * i;
    const int g = 4 * b + kb;
    const bool real = b < nbatch && g < G;
    const int col = g * 128 + 8 * r;
    if constexpr (PERM) sx[i] = load_b128(rperm, real ? col * 2 : kOutOfRange, 0);
    else sx[i] = load_b128(rx, real ? col * 2 : kOutOfRange, 0);
    if constexpr (NORMIN) sw[i] = load_b128(rwn, real ? col * 2 : kOutOfRange, 0);
  }
  constexpr int kXChunks = 4;
  u32x4_t xc[PERM ? kXChunks : 1];
  const int n16 = K / 8;
  if constexpr (PERM) {
#pragma unroll
    for (int j = 0; j < kXChunks; ++j) {
      const int cc = t + j * NW * 64;
      xc[j] = load_b128(rx, cc < n16 ? cc * 16 : kOutOfRange, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // this wave's batch sequence: virtual waves k = part, part + P, ... (< 8), each
  // one's batches k, k + 8, ... (< nbatch); b >= nbatch ends it
  struct Seq {
    int k, b;
  };
  auto advance = [&](Seq s) __attribute__((always_inline)) {
    s.b += kSumLanes;
    if (s.b >= nbatch) {
      s.k += P;
      s.b = s.k;
    }
    return s;
  };
  auto live = [&](Seq s) __attribute__((always_inline)) { return s.k < kSumLanes && s.b < nbatch; };

  // Load offsets: the lane's part is fixed (group slot, row), the batch's part
  // is wave-uniform and rides in the scalar offset, so a batch costs no vector
  // address arithmetic.  live = false: the lane offset is out of range (zeros,
  // no memory access), so every wave issues the same loads whatever its batch
  // count.
  // The scalar offset is not range-checked: every live load is in bounds by the
  // plan's contract (O % 16 == 0, G % 4 == 0), and tiles past O issue none.
  const int plane_stride = O * 16;
  const int p_lane = (lane_times_rows(kb, 3 * O) + row0 + r) * 16;
  const int e_lane = lane_times_rows(cslot, O) + row0 + 4 * kb;
  const bool tile_on = row0 < O;
  auto issue = [&](int batch, BatchLoads<1, 1>& L, bool live_batch) __attribute__((always_inline)) {
    const bool on = live_batch && tile_on;
    const int pv = on ? p_lane : kOutOfRange;
    const int ps = batch * 4 * 3 * plane_stride;
    L.w[0][0] = load_b128_stream(rp, pv, ps);
    L.w[0][1] = load_b128_stream(rp, pv, ps + plane_stride);
    L.w[0][2] = load_b128_stream(rp, pv, ps + 2 * plane_stride);
    __builtin_amdgcn_sched_barrier(0);
    const int ev = on ? e_lane : kOutOfRange;
    const uint2 s4 = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, on ? 2 * e_lane : kOutOfRange,
                                                                                     batch * 4 * O * 2, 0));
    L.s[0][0] = s4.x;
    L.s[0][1] = s4.y;
    L.z[0] = __builtin_amdgcn_raw_buffer_load_b32(rz, ev, batch * 4 * O, 0);
  };

  BatchLoads<1, 1> ring[PD];
  Seq is{part, part};
#pragma unroll
  for (int i = 0; i < PD; ++i) {
    const bool on = live(is);
    issue(is.b, ring[i], on);
    if (on) is = advance(is);
  }
  __builtin_amdgcn_sched_barrier(0);

  if (wave == 0 && lane < 16) bzero[lane] = u32x4_t{0u, 0u, 0u, 0u};
  if constexpr (PERM) {
#pragma unroll
    for (int j = 0; j < kXChunks; ++j) {
      const int cc = t + j * NW * 64;
      if (cc < n16) xs[cc] = xc[j];
    }
    __syncthreads();
  }
  float norm_inv = 1.f;
  if constexpr (NORMIN) {
    float total = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxNormPartialsPerLane; ++k) total += pp[k];
    norm_inv = rsqrtf(wave_total(total) / float(K) + ra.pro_eps);
  }
#pragma unroll
  for (int i = 0; i < S; ++i) {
    const int b = wave + NW * i;
    if (b < nbatch) {
      float v[8];
      if constexpr (PERM) {
        const bool real = 4 * b + kb < G;
        const unsigned pw[4] = {sx[i].x, sx[i].y, sx[i].z, sx[i].w};
        const uint16_t* xs16 = reinterpret_cast<const uint16_t*>(xs);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int src = int(int16_t(pw[j >> 1] >> (16 * (j & 1))));
          v[j] = to_f32<XDT>(real && unsigned(src) < unsigned(K) ? xs16[src] : uint16_t(0));
        }
      } else {
        const unsigned xw[4] = {sx[i].x, sx[i].y, sx[i].z, sx[i].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = to_f32<XDT>(uint16_t(xw[j >> 1] >> (16 * (j & 1))));
        if constexpr (NORMIN) normalize8<XDT>(v, sw[i], norm_inv);
      }
      u32x4_t o;
      float sm;
      int ge;
      stage_fields8(v, field_positions(r), o, sm, ge);
      bst[b * kWideStage + kb * kStageStride<1> + r] = o;
      if (r == 0) {
        gsum[4 * b + kb] = sm;
        gexp[4 * b + kb] = ge;
      }
    }
  }
  __syncthreads();

  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  auto consume = [&](int b, const BatchLoads<1, 1>& L) __attribute__((always_inline)) {
    const u32x4_t* bsrc = c == kb ? bst + b * kWideStage + kb * kStageStride<1> : bzero;
    f32x4_t d = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int word = 0; word < 4; ++word) {
      u32x4_t a[4];
      dequant_fields(L.w[0][0][word], L.w[0][1][word], L.w[0][2][word], a);
#pragma unroll
      for (int s = 0; s < 4; ++s)
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a[s]),
                                                   __builtin_bit_cast(f16x8_t, bsrc[4 * word + s]), d, 0, 0, 0);
    }
    const float sxv = gsum[4 * b + cslot];
    const int fev = gexp[4 * b + cslot];
    const unsigned zw = L.z[0] | zero_default;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const unsigned sbits = (j & 1) ? (L.s[0][j >> 1] >> 16) : (L.s[0][j >> 1] & 0xffffu);
      acc[j] = accumulate_group(acc[j], to_f32<SDT>(uint16_t(sbits)), float((zw >> (8 * j)) & 0xffu), d[j], fev, sxv);
    }
  };
  // a virtual wave's sum: its four group slots meet (lanes c^1, c^2), and lanes
  // c = 0 hold rows 4 kb .. 4 kb + 3 of the tile
  auto finish = [&](int k) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float a = acc[j];
      a += dpp_move<kDppXor1>(a);
      a += dpp_move<kDppXor2>(a);
      acc[j] = a;
    }
    if (c == 0)
      *reinterpret_cast<f32x4_t*>(red + k * 16 * T + 16 * tile + 4 * kb) = f32x4_t{acc[0], acc[1], acc[2], acc[3]};
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = 0.f;
  };

  Seq cs{part, part};
  bool more = live(cs);
  while (more) {
#pragma unroll
    for (int i = 0; i < PD; ++i) {
      if (more) {
        consume(cs.b, ring[i]);
        const bool on = live(is);
        issue(is.b, ring[i], on);
        if (on) is = advance(is);
        const Seq nx = advance(cs);
        if (nx.k != cs.k) finish(cs.k);
        cs = nx;
        more = live(cs);
      }
    }
  }
  __syncthreads();

  // row i's sum over the virtual waves that hold batches, in k order (all eight
  // reads issued at once; a virtual wave without batches is skipped -- it held
  // +0, which adds nothing to a sum that starts at +0)
  const int nk = nbatch < kSumLanes ? nbatch : kSumLanes;
  auto k_order_sum = [&](int i) __attribute__((always_inline)) {
    float v[kSumLanes];
#pragma unroll
    for (int k = 0; k < kSumLanes; ++k) v[k] = red[k * 16 * T + i];
    float total = 0.f;
#pragma unroll
    for (int k = 0; k < kSumLanes; ++k)
      if (k < nk) total += v[k];
    return total;
  };
  if (ra.ep_residual) {
    // out = round(residual + round(y)); each 16-row tile's sum of out^2 (DPP row sum)
    if (t < 16 * T) {
      const int orow = row_base + t;
      float h2 = 0.f;
      if (orow < O) {
        const float total = k_order_sum(t);
        const float h = round_to<XDT>(to_f32<XDT>(ra.ep_residual[orow]) + round_to<XDT>(total));
        out[orow] = from_f32<XDT>(h);
        if (ra.ep_index && unsigned(ep_to) < unsigned(O)) ra.ep_sorted[ep_to] = from_f32<XDT>(h);
        h2 = h * h;
      }
      h2 = row16_sum(h2);
      const int tile_id = orow / 16;
      if (r == 0 && tile_id < (O + 15) / 16) ra.ep_partial[tile_id] = h2;
    }
    return;
  }
  if (swiglu) {
    // (gate, up) row pairs: act = round(round(silu(g)) * u), O / 2 outputs
    if (2 * t < 16 * T) {
      const int i = 2 * t;
      const float tg = k_order_sum(i), tu = k_order_sum(i + 1);
      const int orow = row_base + i;
      if (orow < O) {
        const float g = round_to<XDT>(tg), u = round_to<XDT>(tu);
        const float sg = round_to<XDT>(g / (1.f + __expf(-g)));
        if (!ra.ep_index) out[orow / 2] = from_f32<XDT>(sg * u);
        else if (unsigned(ep_to) < unsigned(O / 2)) out[ep_to] = from_f32<XDT>(sg * u);
      }
    }
    return;
  }
  if (t < 16 * T) {
    const int orow = row_base + t;
    if (orow < O) out[orow] = from_f32<XDT>(k_order_sum(t));
  }
}

// The same plan structure for MB activation rows (MB in {2, 4, 8}; plain
// epilogue, identity column order): a workgroup stages each batch of all its
// rows once for its T tiles, which is where sharing pays most -- eight rows cost
// a wave about as many staging instructions as its dequant and multiplies --
// and each wave runs ceil(MB / 4) MFMA chains on one dequantized A operand (rows
// 4h .. 4h+3 in chain h), as the one-tile kernel does for several rows.  Rows
// m >= M load zeros and are not stored.
//
// Order of the sums: each batch's products reduce to one fp32 partial per output
// (its four group slots meet through lanes c^1, c^2) and the partials add in
// batch order, so any assignment of batches to waves -- every plan -- gives the
// same bits.  Part p of a tile takes batches p, p + P, ...; with one tile (a
// "solo" plan) wave w takes batches w, w + P, ..., exactly the ones it stages,
// so it skips the workgroup barrier and restages one LDS slot of its own per
// batch: any K the plan's waves stage runs with eight rows.  Other plans stage
// every batch into LDS before the barrier (the host checks ceil(G / 4) against
// both limits, the plan's staging and rows_max_batches).
template <int MB>
constexpr int rows_max_batches() { return MB == 8 ? 8 : 24; }  // rows_batch_limit

template <int T, int P, int S, int MB>
struct RowsShared {
  static constexpr int NB = T == 1 ? P : T * P * S < rows_max_batches<MB>() ? T * P * S : rows_max_batches<MB>();
  static constexpr int NR = T == 1 ? P * S : NB;  // batches a launch can hold (the host's limits)
  u32x4_t bst[NB][4 * kStageStride<MB>];
  u32x4_t bzero[16 * MB];
  float gsum[NB][4 * MB];
  int gexp[NB][4 * MB];
  float red[NR][16 * T * MB];
};

template <int T, int P, int PD, int S, int MB, int XDT, int SDT>
__global__ __launch_bounds__(T * P * 64) void w3_fields_rows_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ fields, const uint16_t* __restrict__ scales,
    const uint8_t* __restrict__ zeros, uint16_t* __restrict__ out, int M, int O, int G, int row_blocks) {
  constexpr int NW = T * P, NH = (MB + 3) / 4;
  constexpr bool SOLO = T == 1;
  constexpr int JMAX = SOLO ? S : T * S;  // batches per wave (the host checks ceil(G / 4) <= NW S)
  static_assert(16 * T * MB <= 64 * NW, "one thread per output value");
  asm volatile("" ::"s"(x), "s"(fields), "s"(scales), "s"(zeros), "s"(out), "s"(M), "s"(O), "s"(G), "s"(row_blocks));
  __shared__ RowsShared<T, P, S, MB> sh;
  const int nbatch = (G + 3) >> 2;
  const int t = threadIdx.x, lane = t & 63, wave = wave_index();
  const int part = wave % P, tile = wave / P;
  const int K = G * 128;
  const int row_base = xcd_local_index8(blockIdx.x, row_blocks) * (16 * T);
  const int row0 = row_base + 16 * tile;
  const unsigned zero_default = zeros ? 0u : 0x04040404u;

  const unsigned go = unsigned(G) * unsigned(O);
  const auto rp = buffer_resource_2g(fields, go * 48u);
  const auto rs = buffer_resource_2g(scales, go * 2u);
  const auto rz = buffer_resource_2g(zeros ? (const void*)zeros : (const void*)scales, zeros ? go : 0u);
  const auto rx = buffer_resource_2g(x, unsigned(M) * unsigned(K) * 2u);  // rows past M read zeros

  const int r = lane & 15, kb = lane >> 4, c = lane & 15, cslot = c & 3, cm = c >> 2;

  // staging loads of batch wave + NW i, all rows
  u32x4_t sx[S][MB];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    const int b = wave + NW * i;
    const int g = 4 * b + kb;
    const bool real = b < nbatch && g < G;
#pragma unroll
    for (int m = 0; m < MB; ++m) sx[i][m] = load_b128(rx, real && m < M ? (m * K + g * 128 + 8 * r) * 2 : kOutOfRange, 0);
  }
  __builtin_amdgcn_sched_barrier(0);

  // this wave's batches: c0 + CS j
  constexpr int CS = SOLO ? NW : P;
  const int c0 = SOLO ? wave : part;

  // the scalar offset is not range-checked: live loads are in bounds by the
  // plan's contract (O % 16 == 0, G % 4 == 0), tiles past O issue none
  const int plane_stride = O * 16;
  const int p_lane = (lane_times_rows(kb, 3 * O) + row0 + r) * 16;
  const int e_lane = lane_times_rows(cslot, O) + row0 + 4 * kb;
  const bool tile_on = row0 < O;
  auto issue = [&](int batch, BatchLoads<1, 1>& L) __attribute__((always_inline)) {
    const bool on = batch < nbatch && tile_on;
    const int pv = on ? p_lane : kOutOfRange;
    const int ps = on ? batch * 4 * 3 * plane_stride : 0;
    L.w[0][0] = load_b128_stream(rp, pv, ps);
    L.w[0][1] = load_b128_stream(rp, pv, ps + plane_stride);
    L.w[0][2] = load_b128_stream(rp, pv, ps + 2 * plane_stride);
    __builtin_amdgcn_sched_barrier(0);
    const uint2 s4 = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, on ? 2 * e_lane : kOutOfRange,
                                                                                     on ? batch * 4 * O * 2 : 0, 0));
    L.s[0][0] = s4.x;
    L.s[0][1] = s4.y;
    L.z[0] = __builtin_amdgcn_raw_buffer_load_b32(rz, on ? e_lane : kOutOfRange, on ? batch * 4 * O : 0, 0);
  };

  BatchLoads<1, 1> ring[PD];
#pragma unroll
  for (int i = 0; i < PD; ++i) issue(c0 + CS * i, ring[i]);
  __builtin_amdgcn_sched_barrier(0);

  // the staged operands of the wave's i-th staged batch, all rows, into LDS slot `slot`
  auto stage = [&](int i, int slot) __attribute__((always_inline)) {
    const unsigned fsh = field_positions(r);
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const unsigned xw[4] = {sx[i][m].x, sx[i][m].y, sx[i][m].z, sx[i][m].w};
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = to_f32<XDT>(uint16_t(xw[j >> 1] >> (16 * (j & 1))));
      u32x4_t o;
      float sm;
      int ge;
      stage_fields8(v, fsh, o, sm, ge);
      sh.bst[slot][kb * kStageStride<MB> + r * MB + m] = o;
      if (r == 0) {
        sh.gsum[slot][kb * MB + m] = sm;
        sh.gexp[slot][kb * MB + m] = ge;
      }
    }
  };
  // a wave's own LDS writes and reads stay in program order (LDS executes a
  // wave's instructions in order; this keeps the compiler from moving them)
  auto wave_order = []() __attribute__((always_inline)) {
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
  };

  if constexpr (SOLO) {
    for (int i = lane; i < 16 * MB; i += 64) sh.bzero[i] = u32x4_t{0u, 0u, 0u, 0u};  // every wave: the same zeros
    wave_order();
  } else {
    for (int i = lane; i < 16 * MB; i += 64)
      if (wave == 0) sh.bzero[i] = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int b = wave + NW * i;
      if (b < nbatch && b < RowsShared<T, P, S, MB>::NB) stage(i, b);
    }
    __syncthreads();
  }

  // chain h: activation rows 4h .. 4h+3 sit in the D columns (column c = slot + 4 row)
  int rmc[NH];
  bool data[NH];
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const int row = cm + 4 * h;
    rmc[h] = row < MB ? row : 0;
    data[h] = cslot == kb && row < MB;
  }
  // one batch: its products, reduced over the four group slots, into red[b]
  auto consume = [&](int b, int slot, const BatchLoads<1, 1>& L) __attribute__((always_inline)) {
    const u32x4_t* bsrc[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) bsrc[h] = (data[h] ? &sh.bst[slot][kb * kStageStride<MB>] : sh.bzero) + rmc[h];
    f32x4_t d[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) d[h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int word = 0; word < 4; ++word) {
      u32x4_t a[4];
      dequant_fields(L.w[0][0][word], L.w[0][1][word], L.w[0][2][word], a);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int h = 0; h < NH; ++h)
          d[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a[s]),
                                                      __builtin_bit_cast(f16x8_t, bsrc[h][(4 * word + s) * MB]), d[h],
                                                      0, 0, 0);
    }
    const unsigned zw = L.z[0] | zero_default;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const float sxv = sh.gsum[slot][cslot * MB + rmc[h]];
      const int fev = sh.gexp[slot][cslot * MB + rmc[h]];
      float acc[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const unsigned sbits = (j & 1) ? (L.s[0][j >> 1] >> 16) : (L.s[0][j >> 1] & 0xffffu);
        const float se = to_f32<SDT>(uint16_t(sbits)), zf = float((zw >> (8 * j)) & 0xffu);
        float a = accumulate_group(0.f, se, zf, d[h][j], fev, sxv);
        a += dpp_move<kDppXor1>(a);
        a += dpp_move<kDppXor2>(a);
        acc[j] = a;
      }
      // lanes with slot 0 hold rows 4 kb + j of the tile, activation row cm + 4h
      if (cslot == 0 && cm + 4 * h < MB) {
#pragma unroll
        for (int j = 0; j < 4; ++j) sh.red[b][(16 * tile + 4 * kb + j) * MB + cm + 4 * h] = acc[j];
      }
    }
  };

#pragma unroll
  for (int j = 0; j < JMAX; ++j) {
    const int b = c0 + CS * j;
    if (b < nbatch) {
      if constexpr (SOLO) {
        stage(j, wave);
        wave_order();
      }
      consume(b, SOLO ? wave : b, ring[j % PD]);
      if constexpr (SOLO) wave_order();
      issue(c0 + CS * (j + PD), ring[j % PD]);
    }
  }
  __syncthreads();

  if (t < 16 * T * MB) {
    float total = 0.f;
    for (int b = 0; b < nbatch; ++b) total += sh.red[b][t];
    const int m = t % MB, orow = row_base + t / MB;
    if (orow < O && m < M) out[size_t(m) * O + orow] = from_f32<XDT>(total);
  }
}

template <int T, int P, int PD, int S, int MB, int XDT>
bool fields_rows_sdt(int sdt, const MfmaArgs& a, int M, dim3 grid, hipStream_t s) {
#define FX_ROWS_LAUNCH(SDT)                                                                                     \
  hipLaunchKernelGGL((w3_fields_rows_kernel<T, P, PD, S, MB, XDT, SDT>), grid, dim3(T * P * 64), 0, s, a.x, a.planes, \
                     a.scales, a.zeros, a.out, M, a.O, a.G, a.row_blocks)
  if (sdt == kF16) { FX_ROWS_LAUNCH(kF16); return true; }
  if (sdt == kBF16) { FX_ROWS_LAUNCH(kBF16); return true; }
#undef FX_ROWS_LAUNCH
  return false;
}

template <int MB, int XDT>
bool dispatch_fields_rows_mb(const WidePlan& p, int sdt, const MfmaArgs& a, int M, dim3 grid, hipStream_t s) {
#define FX_ROWS_CASE(T, P, PD, S) \
  if (p.tiles == T && p.parts == P && p.prefetch == PD && p.stage == S) return fields_rows_sdt<T, P, PD, S, MB, XDT>(sdt, a, M, grid, s);
  FX_ROWS_PLANS(FX_ROWS_CASE)
#undef FX_ROWS_CASE
  return false;
}

// mode: 0 plain (identity order), 1 normalising prologue, 2 permuted columns.
template <int T, int P, int PD, int S, int XDT, int SDT>
void launch_fields_wide(int mode, const MfmaArgs& a, dim3 grid, hipStream_t s) {
  const size_t lds = wide_lds_bytes(T, a.G, mode == 2);
#define FX_WIDE_LAUNCH(NORMIN, PERM)                                                                          \
  hipLaunchKernelGGL((w3_fields_wide_kernel<T, P, PD, S, XDT, SDT, NORMIN, PERM>), grid, dim3(T * P * 64), lds, s, \
                     a.x, a.perm, a.planes, a.scales, a.zeros, a.out, a.O, a.G, a.row_blocks, a.swiglu, a.res, a.batch)
  if (mode == 1) FX_WIDE_LAUNCH(true, false);
  else if (mode == 2) FX_WIDE_LAUNCH(false, true);
  else FX_WIDE_LAUNCH(false, false);
#undef FX_WIDE_LAUNCH
}

template <int T, int P, int PD, int S, int XDT>
bool fields_wide_sdt(int sdt, int mode, const MfmaArgs& a, dim3 grid, hipStream_t s) {
  if (sdt == kF16) { launch_fields_wide<T, P, PD, S, XDT, kF16>(mode, a, grid, s); return true; }
  if (sdt == kBF16) { launch_fields_wide<T, P, PD, S, XDT, kBF16>(mode, a, grid, s); return true; }
  return false;
}

template <int XDT>
bool dispatch_fields_wide_xdt(const WidePlan& p, int sdt, int mode, const MfmaArgs& a, dim3 grid, hipStream_t s) {
#define FX_WIDE_CASE(T, P, PD, S) \
  if (p.tiles == T && p.parts == P && p.prefetch == PD && p.stage == S) return fields_wide_sdt<T, P, PD, S, XDT>(sdt, mode, a, grid, s);
  FX_WIDE_PLANS(FX_WIDE_CASE)
#undef FX_WIDE_CASE
  return false;
}

}  // namespace fx
