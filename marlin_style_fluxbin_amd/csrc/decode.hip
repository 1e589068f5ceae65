// Batch-1 decode kernels for gfx950: grouped-query attention over a static KV
// cache (split over key chunks, then combined by a second kernel), and the
// SwiGLU activation.
//
// Attention semantics (stock HF Qwen3 attention through SDPA with a boolean
// mask): for query head h of KV head g = h / (Hq / Hk),
//   s_j = (q_h . k_{g,j}) * scale            j = 0 .. pos (later slots masked)
//   o_h = sum_j softmax(s)_j v_{g,j}
// with fp32 scores, probabilities and accumulation (SDPA's math form), rounded
// once to the activation dtype.  KV cache layout [Hk, Lmax, D].
#include "common.h"
#include "decode_launch.h"
#include "lm_head_launch.h"
#include "norms_launch.h"

namespace fx {

// Query heads scored per pass over a KV head's chunk (the chunk's K and V stay
// in registers across passes).
constexpr int kAttnHeadsPerPass = 4;
constexpr int kDppRowRor8 = 0x128;  // lane i <- lane (i + 8) mod 16 within each row

// Sum over the DB lanes (8, 16 or 32) that hold one key row; every lane of the
// group receives the same bits.
template <int DB>
__device__ __forceinline__ float key_row_sum(float v) {
  v += dpp_move<kDppXor1>(v);
  v += dpp_move<kDppXor2>(v);
  v += dpp_move<kDppHalfMirror>(v);
  if constexpr (DB >= 16) v += dpp_move<kDppMirror>(v);
  if constexpr (DB == 32) v += __shfl_xor(v, 16, 64);
  return v;
}

// grid (Hk, splits), 256 threads; splits = ceil((pos + 1) / (KS * KPT)); G = Hq / Hk
// query heads per KV head (from the host: a device-side divide runs on the VALU,
// and the q / partial descriptors derived from it landed in VGPRs, every load
// through them in a waterfall loop).
// Thread t holds dims [8 db, 8 db + 8) (db = t % DB, DB = D / 8) of keys
// first + ks + KS i, i < KPT (ks = t / DB, KS = 256 / DB key rows per pass):
// a key row is DB consecutive lanes reading 16 B each (coalesced), and every
// K and V load of the chunk is issued before the first use.  Keys past pos
// load zeros (out-of-range buffer offsets), so junk in future cache slots is
// never read.  Per pass of up to 4 query heads: s = (q . k) * scale reduced over
// the DB lanes of the row, chunk max over the workgroup, p = e^(s - m),
// l = sum p, o = sum p v per thread, reduced over the key rows through LDS.
// po[(h * splits + chunk) * D + d] = o[d] and pml[(h * splits + chunk) * 2] =
// {m, l} (plain stores: the combine kernel reads them after this launch ends);
// with one split the output o / l is written instead.
// PRE: q is the raw projection; each query head is normalised (q_norm) and
// rotated before scoring, and the key and value of position pos are formed here
// from the raw projections (k_norm, RoPE; v as is) -- by the workgroup whose
// chunk holds pos, which also writes them into the caches.  Rounding points of
// head_norm_rope_kernel: y = round(w * round(x * inv)), stock RoPE
// round(round(y * cos) + round(rotate_half(y) * sin)) (fused: the second term
// unrounded); the head's sum of squares is taken over the DB lanes of a row.
template <int DT, int D>
__device__ __forceinline__ u32x4_t head_norm_rope8(const u32x4_t& x, const u32x4_t& w, const u32x4_t& cs,
                                                  const u32x4_t& sn, bool lower, float eps, int rope_mode) {
  constexpr int DB = D / 8;
  const float inv = rsqrtf(key_row_sum<DB>(sum_sq8<DT>(x)) / float(D) + eps);
  // element pairs: each rounding point is one packed convert (round_pair)
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    float a = to_f32<DT>(uint16_t(x[e >> 1])) * inv, b = to_f32<DT>(uint16_t(x[e >> 1] >> 16)) * inv;
    round_pair<DT>(a, b);
    a *= to_f32<DT>(uint16_t(w[e >> 1]));
    b *= to_f32<DT>(uint16_t(w[e >> 1] >> 16));
    round_pair<DT>(a, b);
    y[e] = a;
    y[e + 1] = b;
  }
  u32x4_t o;
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    float rot[2], yc[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      // rotate_half(y) = (-y[D/2:], y[:D/2]): the partner dim sits DB/2 lanes away
      // (DB = 16: a DPP rotate by 8 within the row)
      float partner;
      if constexpr (DB == 16) partner = dpp_move<kDppRowRor8>(y[e + h]);
      else partner = __shfl_xor(y[e + h], DB / 2, 64);
      const float c = to_f32<DT>(uint16_t(cs[e >> 1] >> (16 * h)));
      const float sv = to_f32<DT>(uint16_t(sn[e >> 1] >> (16 * h)));
      rot[h] = (lower ? -partner : partner) * sv;
      yc[h] = y[e + h] * c;
    }
    if (rope_mode == kRopeStock) round_pair<DT>(rot[0], rot[1]);
    round_pair<DT>(yc[0], yc[1]);
    float r0 = yc[0] + rot[0], r1 = yc[1] + rot[1];
    o[e >> 1] = round_pair_bits<DT>(r0, r1);
  }
  return o;
}

template <int DT, int D, int KPT, bool PRE, int NG>
__global__ __launch_bounds__(256 * NG) void attn_split_kernel(const uint16_t* __restrict__ q,
                                                         const uint16_t* kc, const uint16_t* vc,
                                                         float* __restrict__ po, float* __restrict__ pml,
                                                         uint16_t* __restrict__ out,
                                                         const int16_t* __restrict__ out_index, int G,
                                                         int Lmax, int pos, int splits,
                                                         float scale, AttnPre pre) {
  asm volatile("" ::"s"(q), "s"(kc), "s"(vc), "s"(po), "s"(pml), "s"(out), "s"(out_index), "s"(G),
               "s"(Lmax), "s"(pos), "s"(splits), "s"(scale));
  if constexpr (PRE)
    asm volatile("" ::"s"(pre.k_raw), "s"(pre.v_raw), "s"(pre.q_weight), "s"(pre.k_weight), "s"(pre.cos),
                 "s"(pre.sin), "s"(pre.eps), "s"(pre.rope_mode));
  // NG head groups of 256 threads: group grp scores query heads grp * HB + ...
  // of each pass against the same chunk (its K and V rows come from L1 after
  // the first group's loads), so a wave's serial chain covers HB heads, not 4
  static_assert(kAttnHeadsPerPass % NG == 0, "head groups must divide the heads of a pass");
  constexpr int DB = D / 8, KS = 256 / DB, HB = kAttnHeadsPerPass / NG;
  __shared__ float red_o[NG][KS][HB][D];
  __shared__ float red_l[NG][KS][HB];
  __shared__ float red_m[NG][4][HB];
  __shared__ u32x4_t qsh[PRE ? 4 * NG : 1][HB][DB];  // PRE: normalised queries of each wave
  const int grp = int(threadIdx.x) >> 8, t = int(threadIdx.x) & 255, lane = t & 63, wave = wave_index();
  const int gw = wave & 3;  // wave within the head group
  const int db = t % DB, ks = t / DB;
  const int g = blockIdx.x, chunk = blockIdx.y;
  const int first = chunk * (KS * KPT);
  const auto rq = buffer_resource(q + size_t(g) * G * D, size_t(G) * D * 2);
  const auto rk = buffer_resource(kc + size_t(g) * Lmax * D, size_t(Lmax) * D * 2);
  const auto rv = buffer_resource(vc + size_t(g) * Lmax * D, size_t(Lmax) * D * 2);

  // ---- loads: first pass's queries (PRE: with the norm weights, RoPE rows and,
  // in the chunk holding pos, the raw key and value of pos), then the chunk's
  // keys and values -- loads complete in issue order, so the query (and pos
  // key) normalisation overlaps the K/V stream
  u32x4_t qr[HB], kr[KPT], vr[KPT];
  bool live[KPT];
  const bool lower = db < DB / 2;
  const bool has_pos = first <= pos && pos < first + KS * KPT;  // workgroup-uniform
  u32x4_t qw, cs, sn, kraw, vraw, kw;
  // PRE: the rows of a wave split the pass's query heads (row r of the wave
  // normalises heads r, r + rows, ...; each row loads its own heads' raw slices)
  // and share the results through the wave's LDS slot
  constexpr int kRows = 64 / DB;
  constexpr int kOwn = HB > kRows ? HB / kRows : 1;  // heads one row normalises per pass
  const int qrow = lane / DB;
  u32x4_t qown[kOwn];
  auto load_own = [&](int h0) __attribute__((always_inline)) {
#pragma unroll
    for (int o = 0; o < kOwn; ++o) {
      const int hh = o * kRows + qrow, h = h0 + hh;
      qown[o] = load_b128(rq, hh < HB && h < G ? (h * D + 8 * db) * 2 : kOutOfRange, 0);
    }
  };
  if constexpr (PRE) {
    load_own(grp * HB);
  } else {
#pragma unroll
    for (int hh = 0; hh < HB; ++hh) {
      const int h = grp * HB + hh;
      qr[hh] = load_b128(rq, h < G ? (h * D + 8 * db) * 2 : kOutOfRange, 0);
    }
  }
  if constexpr (PRE) {
    const auto rd = [&](const uint16_t* p, bool on) {
      return load_b128(buffer_resource(p, D * 2), on ? 16 * db : kOutOfRange, 0);
    };
    qw = rd(pre.q_weight, true);
    cs = rd(pre.cos, true);
    sn = rd(pre.sin, true);
    kraw = rd(pre.k_raw + size_t(g) * D, has_pos);
    vraw = rd(pre.v_raw + size_t(g) * D, has_pos);
    kw = rd(pre.k_weight, has_pos);
  }
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int j = first + ks + KS * i;
    live[i] = j <= pos;
    kr[i] = load_b128(rk, live[i] ? (j * D + 8 * db) * 2 : kOutOfRange, 0);
  }
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int j = first + ks + KS * i;
    vr[i] = load_b128(rv, live[i] ? (j * D + 8 * db) * 2 : kOutOfRange, 0);
  }
  auto normalise_queries = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int o = 0; o < kOwn; ++o) {
      const int hh = o * kRows + qrow;
      const u32x4_t v = head_norm_rope8<DT, D>(qown[o], qw, cs, sn, lower, pre.eps, pre.rope_mode);
      if (hh < HB) qsh[wave][hh][db] = v;
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int hh = 0; hh < HB; ++hh) qr[hh] = qsh[wave][hh][db];
    __builtin_amdgcn_wave_barrier();
  };
  if constexpr (PRE) {
    // first pass's queries and the pos key: normalised and rotated while the
    // chunk's K/V rows stream in
    normalise_queries();
    if (has_pos) {
      const u32x4_t kpos = head_norm_rope8<DT, D>(kraw, kw, cs, sn, lower, pre.eps, pre.rope_mode);
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        if (first + ks + KS * i == pos) {
          kr[i] = kpos;
          vr[i] = vraw;
          if (grp == 0) {  // one group writes the caches
            const size_t at = (size_t(g) * Lmax + pos) * D + 8 * db;
            *reinterpret_cast<u32x4_t*>(const_cast<uint16_t*>(kc) + at) = kpos;
            *reinterpret_cast<u32x4_t*>(const_cast<uint16_t*>(vc) + at) = vraw;
          }
        }
      }
    }
  }

  // every group runs the same number of passes (the barriers inside are workgroup-wide)
  for (int pass = 0; pass * NG * HB < G; ++pass) {
    const int h0 = (pass * NG + grp) * HB;
    if (!PRE && pass > 0) {
#pragma unroll
      for (int hh = 0; hh < HB; ++hh)
        qr[hh] = load_b128(rq, h0 + hh < G ? ((h0 + hh) * D + 8 * db) * 2 : kOutOfRange, 0);
    }
    float kf[KPT][8];
#pragma unroll
    for (int i = 0; i < KPT; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) kf[i][e] = to_f32<DT>(uint16_t(kr[i][e >> 1] >> (16 * (e & 1))));
    if constexpr (PRE) {
      if (pass > 0) {
        load_own(h0);
        normalise_queries();
      }
    }
    float s[HB][KPT];
    float mt[HB];
#pragma unroll
    for (int hh = 0; hh < HB; ++hh) {
      float qf[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[e] = to_f32<DT>(uint16_t(qr[hh][e >> 1] >> (16 * (e & 1))));
      mt[hh] = -INFINITY;
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += qf[e] * kf[i][e];
        acc = key_row_sum<DB>(acc) * scale;
        s[hh][i] = live[i] ? acc : -INFINITY;
        mt[hh] = fmaxf(mt[hh], s[hh][i]);
      }
      mt[hh] = wave_max_not_nan(mt[hh]);  // scores are finite or -inf (keys past pos)
    }
    if (lane == 0) {
#pragma unroll
      for (int hh = 0; hh < HB; ++hh) red_m[grp][gw][hh] = mt[hh];
    }
    __syncthreads();
    float o[HB][8], lt[HB];
#pragma unroll
    for (int hh = 0; hh < HB; ++hh) {
      // the chunk's first key is live, so m is finite
      const float m = fmaxf(fmaxf(red_m[grp][0][hh], red_m[grp][1][hh]), fmaxf(red_m[grp][2][hh], red_m[grp][3][hh]));
      mt[hh] = m;
      lt[hh] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[hh][e] = 0.f;
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        const float p = live[i] ? __expf(s[hh][i] - m) : 0.f;
        lt[hh] += p;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[hh][e] += p * to_f32<DT>(uint16_t(vr[i][e >> 1] >> (16 * (e & 1))));
      }
    }
#pragma unroll
    for (int hh = 0; hh < HB; ++hh) {
      float4* dst = reinterpret_cast<float4*>(&red_o[grp][ks][hh][8 * db]);
      dst[0] = make_float4(o[hh][0], o[hh][1], o[hh][2], o[hh][3]);
      dst[1] = make_float4(o[hh][4], o[hh][5], o[hh][6], o[hh][7]);
      if (db == 0) red_l[grp][ks][hh] = lt[hh];
    }
    __syncthreads();
    for (int idx = t; idx < HB * D; idx += 256) {
      const int hh = idx / D, d = idx % D, h = h0 + hh;
      float total = 0.f;
#pragma unroll
      for (int r = 0; r < KS; ++r) total += red_o[grp][r][hh][d];
      if (h < G) {
        if (splits == 1) {
          // the whole context is this chunk: o = sum p v / sum p
          float l = 0.f;
#pragma unroll
          for (int r = 0; r < KS; ++r) l += red_l[grp][r][hh];
          const int n_out = int(gridDim.x) * G * D;
          int at = (g * G + h) * D + d;
          if (out_index) at = out_index[at];
          if (unsigned(at) < unsigned(n_out)) out[at] = from_f32<DT>(total * (1.f / l));
        } else {
          const size_t slot = size_t(g * G + h) * splits + chunk;
          po[slot * D + d] = total;
          if (d == 0) {
            float l = 0.f;
#pragma unroll
            for (int r = 0; r < KS; ++r) l += red_l[grp][r][hh];
            pml[slot * 2] = mt[hh];
            pml[slot * 2 + 1] = l;
          }
        }
      }
    }
    __syncthreads();  // LDS reused by the next pass
  }
}

// grid Hq, 256 threads: o_h = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c over the
// head's splits, taken in blocks of 64 (a running max rescales earlier blocks).
// Every wave forms the block's maximum and weighted sum itself (lane c holds
// split c's max and sum: no LDS round for them).  Thread t sums output dim
// t % D over the splits t / D, t / D + PARTS, ... of the block (PARTS = 256 / D
// threads per dim, whose partial sums meet in LDS once at the end), taking each
// split's weight from its own load of that split's max.  The block's maxima and
// sums and this thread's first kPre split values are issued in one load round
// (kPre * PARTS splits: 32 at D = 128, every block of a decode length's splits).
template <int DT, int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ po,
                                                          const float* __restrict__ pml,
                                                          uint16_t* __restrict__ out,
                                                          const int16_t* __restrict__ out_index, int splits) {
  asm volatile("" ::"s"(po), "s"(pml), "s"(out), "s"(out_index), "s"(splits));
  static_assert(D <= 256, "one output dim per thread");
  constexpr int PARTS = 256 / D;  // threads per output dim
  constexpr int kPre = 16;
  __shared__ float ored[PARTS][D];
  const int h = blockIdx.x, t = threadIdx.x, lane = t & 63;
  // where this thread's output dim goes, loaded ahead of the partials
  const int n_out = int(gridDim.x) * D;
  const int at = out_index ? (t < D ? int(out_index[h * D + t]) : -1) : h * D + t;
  const float* vo = po + size_t(h) * splits * D;
  const float* ml = pml + size_t(h) * splits * 2;
  float M = -INFINITY, L = 0.f, o = 0.f;
  const int part = t / D, d0 = t % D;
  for (int c0 = 0; c0 < splits; c0 += 64) {
    const int n = min(64, splits - c0);
    const float mc = lane < n ? ml[size_t(c0 + lane) * 2] : -INFINITY;
    const float lc = lane < n ? ml[size_t(c0 + lane) * 2 + 1] : 0.f;
    float v0[kPre], m0[kPre];
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
      const int cc = part + u * PARTS;
      v0[u] = cc < n ? vo[size_t(c0 + cc) * D + d0] : 0.f;
      m0[u] = cc < n ? ml[size_t(c0 + cc) * 2] : -INFINITY;
    }
    const float Mn = fmaxf(M, wave_max_not_nan(mc));  // split maxima: finite, -inf past n
    const float rescale = M == -INFINITY ? 0.f : __expf(M - Mn);
    L = L * rescale + wave_sum(lane < n ? __expf(mc - Mn) * lc : 0.f);
    o *= rescale;
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
      const int cc = part + u * PARTS;
      o += (cc < n ? __expf(m0[u] - Mn) : 0.f) * v0[u];
    }
    for (int cc = part + kPre * PARTS; cc < n; cc += PARTS)
      o += __expf(ml[size_t(c0 + cc) * 2] - Mn) * vo[size_t(c0 + cc) * D + d0];
    M = Mn;
  }
  ored[part][d0] = o;
  __syncthreads();
  const float inv = 1.f / L;
  if (t < D) {  // D <= 256: thread t holds output dim t
    float total = 0.f;
#pragma unroll
    for (int p2 = 0; p2 < PARTS; ++p2) total += ored[p2][t];
    if (unsigned(at) < unsigned(n_out)) out[at] = from_f32<DT>(total * inv);
  }
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

// Start of a decode step on the residual-stream chain (one workgroup of 256
// threads): the embedding row of *token into `out`, and per 16-element tile of
// it the sum of squares (elements in order, fp32) into `tile_sumsq` -- the
// partials the first layer's normalising q|k|v GEMV reads, as every later layer
// reads its predecessor's residual epilogue; then, when `merge` is set, the
// argmax merge of the previous step's LM-head partials into its prediction.
// One launch in place of the embedding gather, the first RMSNorm and the
// previous step's merge.  A token outside [0, vocab) gives a NaN row (and NaN
// tile sums), so the step's logits are NaN rather than another token's.
template <int DT>
__global__ __launch_bounds__(256) void decode_embed_kernel(const long long* __restrict__ token,
                                                           const uint16_t* __restrict__ table, int vocab,
                                                           int hidden, uint16_t* __restrict__ out,
                                                           float* __restrict__ tile_sumsq,
                                                           const int16_t* __restrict__ out_index,
                                                           uint16_t* __restrict__ sorted_out, LmHeadArgs merge) {
  asm volatile("" ::"s"(token), "s"(table), "s"(vocab), "s"(hidden), "s"(out), "s"(tile_sumsq), "s"(out_index),
               "s"(sorted_out));
  const long long tok = *token;
  const bool valid = tok >= 0 && tok < vocab;
  const auto rt = buffer_resource(table + (valid ? size_t(tok) * hidden : 0), size_t(hidden) * 2);
  const auto ri = buffer_resource(out_index ? (const void*)out_index : (const void*)table,
                                  out_index ? size_t(hidden) * 2 : 0);
  const int tiles = hidden / 16;
  for (int tile = threadIdx.x; tile < tiles; tile += 256) {
    const u32x4_t a = load_b128(rt, tile * 32, 0), b = load_b128(rt, tile * 32 + 16, 0);
    u32x4_t ia{}, ib{};
    if (out_index) {
      ia = load_b128(ri, tile * 32, 0);
      ib = load_b128(ri, tile * 32 + 16, 0);
    }
    u32x4_t* dst = reinterpret_cast<u32x4_t*>(out + size_t(tile) * 16);
    float ss = 0.f;
    if (valid) {
      dst[0] = a;
      dst[1] = b;
      if (out_index) {  // the same row in the next GEMV's sorted column order
        const u32x4_t v[2] = {a, b}, ix[2] = {ia, ib};
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int to = int(int16_t(ix[h][e >> 1] >> (16 * (e & 1))));
            if (unsigned(to) < unsigned(hidden)) sorted_out[to] = uint16_t(v[h][e >> 1] >> (16 * (e & 1)));
          }
      }
      const u32x4_t v[2] = {a, b};
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = to_f32<DT>(uint16_t(v[h][e >> 1] >> (16 * (e & 1))));
          ss = fmaf(x, x, ss);
        }
    } else {
      const unsigned nan2 = DT == kBF16 ? 0x7fc07fc0u : 0x7e007e00u;
      dst[0] = dst[1] = u32x4_t{nan2, nan2, nan2, nan2};
      if (out_index) {
        const u32x4_t ix[2] = {ia, ib};
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int to = int(int16_t(ix[h][e >> 1] >> (16 * (e & 1))));
            if (unsigned(to) < unsigned(hidden)) sorted_out[to] = uint16_t(nan2);
          }
      }
      ss = __builtin_nanf("");
    }
    tile_sumsq[tile] = ss;
  }
  if (merge.prediction) merge_argmax_partials(merge.part_val, merge.part_idx, merge.blocks, merge.prediction);
}

bool launch_decode_embed(int dt, const long long* token, const uint16_t* table, int vocab, int hidden,
                         uint16_t* out, float* tile_sumsq, const int16_t* out_index, uint16_t* sorted_out,
                         const LmHeadArgs& merge, hipStream_t s) {
  if (dt == kBF16)
    hipLaunchKernelGGL(decode_embed_kernel<kBF16>, dim3(1), dim3(256), 0, s, token, table, vocab, hidden, out,
                       tile_sumsq, out_index, sorted_out, merge);
  else if (dt == kF16)
    hipLaunchKernelGGL(decode_embed_kernel<kF16>, dim3(1), dim3(256), 0, s, token, table, vocab, hidden, out,
                       tile_sumsq, out_index, sorted_out, merge);
  else
    return false;
  return true;
}

template <int DT, int D, int KPT, int NG>
void attn_split_launch(const AttnArgs& a, float* po, float* pml, hipStream_t s) {
  if (a.pre.k_raw)
    hipLaunchKernelGGL((attn_split_kernel<DT, D, KPT, true, NG>), dim3(a.Hk, a.splits), dim3(256 * NG), 0, s, a.q,
                       a.k, a.v, po, pml, a.out, a.out_index, a.Hq / a.Hk, a.Lmax, a.pos, a.splits, a.scale, a.pre);
  else
    hipLaunchKernelGGL((attn_split_kernel<DT, D, KPT, false, NG>), dim3(a.Hk, a.splits), dim3(256 * NG), 0, s, a.q,
                       a.k, a.v, po, pml, a.out, a.out_index, a.Hq / a.Hk, a.Lmax, a.pos, a.splits, a.scale, a.pre);
}

template <int DT, int D, int KPT>
void attn_launch(const AttnArgs& a, hipStream_t s) {
  float* po = a.partial;
  float* pml = a.partial + size_t(a.Hq) * a.splits * D;
  if (a.groups == 4) attn_split_launch<DT, D, KPT, 4>(a, po, pml, s);
  else if (a.groups == 2) attn_split_launch<DT, D, KPT, 2>(a, po, pml, s);
  else attn_split_launch<DT, D, KPT, 1>(a, po, pml, s);
  if (a.splits > 1)
    hipLaunchKernelGGL((attn_combine_kernel<DT, D>), dim3(a.Hq), dim3(256), 0, s, po, pml, a.out, a.out_index,
                       a.splits);
}

template <int DT, int D>
bool attn_for_kpt(int kpt, const AttnArgs& a, hipStream_t s) {
  switch (kpt) {
    case 1: attn_launch<DT, D, 1>(a, s); return true;
    case 2: attn_launch<DT, D, 2>(a, s); return true;
    case 4: attn_launch<DT, D, 4>(a, s); return true;
  }
  return false;
}

template <int DT>
bool attn_for_dim(int D, const AttnArgs& a, hipStream_t s) {
  switch (D) {
    case 64: return attn_for_kpt<DT, 64>(a.kpt, a, s);
    case 128: return attn_for_kpt<DT, 128>(a.kpt, a, s);
    case 256: return attn_for_kpt<DT, 256>(a.kpt, a, s);
  }
  return false;
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
