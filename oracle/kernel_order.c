/*
 * Plain C restatement of the reference kernel's fp32 evaluation order.
 * TEST INFRASTRUCTURE ONLY: loaded by tests through oracle/kernel_order.py.
 *
 * Follows maxiu188-afk/Marlin_Style_Fluxbin:
 *   csrc/lut8_unsigned.cuh:13-27   unsigned subset-sum LUT, exact add order
 *   csrc/lut8.cuh:18-28            signed (+-v) subset-sum LUT, exact add order
 *   csrc/w3_lut.cu:57-123          per-group LUT lookups, (a0 + 2 a1) - 4 a2,
 *                                  x scale, optional +-3 bf16-rounding correction
 *   csrc/w3_lut.cu:141-150         sequential fp32 split reduction
 * Build with -ffp-contract=off (the reference compiles with --fmad=false), so
 * every + and * rounds separately.  The LUT builders are checked bit-for-bit
 * against the reference's own header compiled into oracle/_ref/.
 */
#include <stdint.h>
#include <string.h>

void oracle_lut_unsigned(const float *values, float *table) {
  for (unsigned lane = 0; lane < 32; ++lane) {
    float sum = 0.f;
    for (int bit = 0; bit < 8; ++bit) sum += ((lane >> bit) & 1u) ? values[bit] : 0.f;
    table[lane] = sum;
  }
  for (unsigned bit = 5; bit < 8; ++bit)
    for (unsigned base = 1u << bit; base < (1u << (bit + 1)); base += 32)
      for (unsigned lane = 0; lane < 32; ++lane)
        table[base + lane] = table[base + lane - (1u << bit)] + values[bit];
}

void oracle_lut_signed(const float *values, float *table) {
  for (unsigned lane = 0; lane < 32; ++lane) {
    float sum = 0.f;
    for (int bit = 0; bit < 8; ++bit) sum += ((lane >> bit) & 1u) ? values[bit] : -values[bit];
    table[lane] = sum;
  }
  for (unsigned bit = 5; bit < 8; ++bit) {
    float twice = values[bit] + values[bit];
    for (unsigned base = 1u << bit; base < (1u << (bit + 1)); base += 32)
      for (unsigned lane = 0; lane < 32; ++lane)
        table[base + lane] = table[base + lane - (1u << bit)] + twice;
  }
}

static float round_bf16(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  memcpy(&v, &u, 4);
  return v;
}

/*
 * x: K fp32 values (the bf16/fp16 activation widened); planes [G,3,O,16];
 * scales [G,O] fp32 holding bf16 values; perm [K] int16 or NULL;
 * out: O fp32 values after the split reduction (before the final dtype cast).
 */
void oracle_w3_kernel_order(const float *x, const uint8_t *planes, const float *scales,
                            const int16_t *perm, int O, int G, int gps, int decoded,
                            float *out) {
  float lut[16 * 256];
  int splits = (G + gps - 1) / gps;
  for (int o = 0; o < O; ++o) out[o] = 0.f;
  for (int s = 0; s < splits; ++s) {
    int g_end = (s + 1) * gps < G ? (s + 1) * gps : G;
    /* per-split partial results, one per row */
    for (int o = 0; o < O; ++o) {
      float result = 0.f;
      for (int g = s * gps; g < g_end; ++g) {
        for (int c = 0; c < 16; ++c) {
          float v[8];
          for (int j = 0; j < 8; ++j) {
            int k = g * 128 + c * 8 + j;
            v[j] = x[perm ? perm[k] : k];
          }
          oracle_lut_unsigned(v, lut + c * 256);
        }
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, corr = 0.f;
        const uint8_t *p0 = planes + ((size_t)(g * 3 + 0) * O + o) * 16;
        const uint8_t *p1 = planes + ((size_t)(g * 3 + 1) * O + o) * 16;
        const uint8_t *p2 = planes + ((size_t)(g * 3 + 2) * O + o) * 16;
        for (int c = 0; c < 16; ++c) {
          unsigned b0 = p0[c], b1 = p1[c], b2 = p2[c];
          a0 += lut[c * 256 + b0];
          a1 += lut[c * 256 + b1];
          a2 += lut[c * 256 + b2];
          if (decoded) {
            unsigned plus = b0 & b1 & (~b2 & 0xffu);
            unsigned minus = b0 & (~b1 & 0xffu) & b2;
            corr += lut[c * 256 + plus] - lut[c * 256 + minus];
          }
        }
        float scale = scales[(size_t)g * O + o];
        float two_a1 = 2.f * a1;
        float four_a2 = 4.f * a2;
        float integer_dot = (a0 + two_a1) - four_a2;
        float value = integer_dot * scale;
        if (decoded) {
          float three = 3.f * scale;
          float delta = round_bf16(three) - three;
          value += corr * delta;
        }
        result += value;
      }
      /* finish_m1: sequential over splits */
      out[o] += result;
    }
  }
}
