/*
 * Plain-C restatement of the bfp8 quantiser/dequantiser and the fp32 SwiGLU formula.
 * ORACLE / TEST INFRASTRUCTURE ONLY: used by tests/ to cross-check oracle/bfp8.py and
 * oracle/mlp.py; never linked into the product library.
 *
 * Quantiser: shared exponent = largest frexp exponent of the group's non-zero values, scale
 * 2^(E-7), mantissa = round-half-even(v / scale) clamped to [-127, 127] -- the block-float rule of
 * the reference's bf8_exact (scripts/ci/ordered_cache_hw_plan.py:243-260), grouped along K.
 * SwiGLU: (silu(x Wg^T) * (x Wu^T)) Wd^T + residual, fp32 accumulation in K order
 * (scripts/ci/mlp-sweep.py:121-126; docker/qwen-c2-graft/graft/layer.py:357).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bf16_to_f32(uint16_t b) {
  uint32_t w = (uint32_t)b << 16;
  float f;
  memcpy(&f, &w, 4);
  return f;
}

uint16_t oracle_f32_to_bf16_rne(float f) {
  uint32_t w;
  memcpy(&w, &f, 4);
  if ((w & 0x7f800000u) == 0x7f800000u && (w & 0x007fffffu)) return (uint16_t)((w >> 16) | 0x40);
  uint32_t bias = 0x7fffu + ((w >> 16) & 1u);
  return (uint16_t)((w + bias) >> 16);
}

/* Block-float quantiser with `mbits` magnitude bits (7: bfp8, 3: bf4).  Returns the number of
 * groups holding a non-finite value (their output is left zero). */
int oracle_quantize_bfp(const uint16_t* w, int rows, int cols, int8_t* q, uint8_t* e8, int mbits) {
  const int qmax = (1 << mbits) - 1;
  int bad = 0;
  int groups = cols / 16;
  for (int r = 0; r < rows; ++r) {
    for (int g = 0; g < groups; ++g) {
      const uint16_t* src = w + (size_t)r * cols + (size_t)g * 16;
      int8_t* dq = q + (size_t)r * cols + (size_t)g * 16;
      double v[16];
      int shared = -100000, any = 0, finite = 1;
      for (int i = 0; i < 16; ++i) {
        v[i] = (double)bf16_to_f32(src[i]);
        if (!isfinite(v[i])) finite = 0;
        if (v[i] != 0.0) {
          int ex;
          frexp(v[i], &ex);
          if (ex > shared) shared = ex;
          any = 1;
        }
      }
      if (!finite) {
        ++bad;
        memset(dq, 0, 16);
        e8[(size_t)r * groups + g] = 0;
        continue;
      }
      if (!any) {
        memset(dq, 0, 16);
        e8[(size_t)r * groups + g] = 0;
        continue;
      }
      int e = shared + 127 - mbits;
      if (e < 1) e = 1;
      if (e > 254) e = 254;
      double scale = ldexp(1.0, e - 127);
      for (int i = 0; i < 16; ++i) {
        double t = nearbyint(v[i] / scale); /* default rounding mode: half to even */
        if (t > qmax) t = qmax;
        if (t < -qmax) t = -qmax;
        dq[i] = (int8_t)t;
      }
      e8[(size_t)r * groups + g] = (uint8_t)e;
    }
  }
  return bad;
}

int oracle_quantize_bfp8(const uint16_t* w, int rows, int cols, int8_t* q, uint8_t* e8) {
  return oracle_quantize_bfp(w, rows, cols, q, e8, 7);
}

void oracle_dequantize_bfp8(const int8_t* q, const uint8_t* e8, int rows, int cols, float* out) {
  int groups = cols / 16;
  for (int r = 0; r < rows; ++r)
    for (int g = 0; g < groups; ++g) {
      uint8_t e = e8[(size_t)r * groups + g];
      double scale = e ? ldexp(1.0, (int)e - 127) : 0.0;
      for (int i = 0; i < 16; ++i) {
        size_t k = (size_t)r * cols + (size_t)g * 16 + i;
        out[k] = (float)((double)q[k] * scale);
      }
    }
}

/* out[M,H] = residual + ((silu(x Wg^T) * (x Wu^T)) Wd^T); all fp32, sequential K accumulation.
 * x [M,H], wg/wu [I,H], wd [H,I]; residual may be NULL; hidden [M,I] is scratch. */
void oracle_swiglu_f32(const float* x, const float* wg, const float* wu, const float* wd,
                       const float* residual, float* hidden, float* out, int M, int H, int I) {
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < I; ++n) {
      float g = 0.f, u = 0.f;
      for (int k = 0; k < H; ++k) {
        g += x[(size_t)m * H + k] * wg[(size_t)n * H + k];
        u += x[(size_t)m * H + k] * wu[(size_t)n * H + k];
      }
      float s = g / (1.0f + expf(-g));
      hidden[(size_t)m * I + n] = s * u;
    }
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < H; ++n) {
      float y = 0.f;
      for (int k = 0; k < I; ++k) y += hidden[(size_t)m * I + k] * wd[(size_t)n * I + k];
      out[(size_t)m * H + n] = residual ? residual[(size_t)m * H + n] + y : y;
    }
}
