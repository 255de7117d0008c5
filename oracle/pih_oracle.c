/* pih_oracle.c — CPU restatement of the reference's hot-path arithmetic.
 * TEST INFRASTRUCTURE ONLY (see pih_oracle.h for the rules and the pinning
 * of each function).  Built with -O2 -ffp-contract=off -fopenmp. */
#include "pih_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- threads */
static int g_threads = 1;

void po_set_threads(int threads) { g_threads = threads < 1 ? 1 : threads; }
int po_get_threads(void) { return g_threads; }

#define PO_PARALLEL_FOR _Pragma("omp parallel for schedule(static) num_threads(g_threads)")
#define PO_PARALLEL_FOR_REDUCE_OR(v) _Pragma("omp parallel for schedule(static) num_threads(g_threads) reduction(|:err)")

/* ----------------------------------------------------------------- codecs */
static inline uint32_t f2u(float v) { uint32_t u; memcpy(&u, &v, 4); return u; }
static inline float u2f(uint32_t u) { float v; memcpy(&v, &u, 4); return v; }

uint16_t po_bf16_from_f32(float value) {
  /* include/pih/core/bfloat16.h:13-23: NaN keeps its sign and becomes quiet,
   * everything else rounds to nearest even on the upper 16 bits. */
  const uint32_t raw = f2u(value);
  if ((raw & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((raw >> 16) | 0x0040u);
  return (uint16_t)((raw + 0x7fffu + ((raw >> 16) & 1u)) >> 16);
}

float po_bf16_to_f32(uint16_t bits) { return u2f((uint32_t)bits << 16); }

uint16_t po_f16_from_f32(float value) {
  /* src/core/float16.cpp:8-49 (RNE, overflow to infinity, quiet NaN). */
  const uint32_t raw = f2u(value);
  const uint16_t sign = (uint16_t)((raw >> 16) & 0x8000u);
  const uint32_t exponent = (raw >> 23) & 0xffu;
  const uint32_t mantissa = raw & 0x7fffffu;
  if (exponent == 0xffu) return (uint16_t)(sign | (mantissa == 0 ? 0x7c00u : 0x7e00u));
  const int unbiased = (int)exponent - 127;
  if (unbiased > 15) return (uint16_t)(sign | 0x7c00u);
  if (unbiased >= -14) {
    uint32_t he = (uint32_t)(unbiased + 15);
    uint32_t hm = mantissa >> 13;
    const uint32_t rem = mantissa & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) {
      if (++hm == 0x400u) {
        hm = 0;
        if (++he >= 31u) return (uint16_t)(sign | 0x7c00u);
      }
    }
    return (uint16_t)(sign | (he << 10) | hm);
  }
  if (unbiased < -25) return sign;
  const uint32_t significand = 0x800000u | mantissa;
  const uint32_t shift = (uint32_t)(-14 - unbiased + 13);
  uint32_t hm = significand >> shift;
  const uint32_t rem = significand & ((1u << shift) - 1u);
  const uint32_t halfway = 1u << (shift - 1u);
  if (rem > halfway || (rem == halfway && (hm & 1u))) ++hm;
  return (uint16_t)(sign | hm);
}

float po_f16_to_f32(uint16_t bits) {
  /* src/core/float16.cpp:51-68 */
  const int negative = (bits & 0x8000u) != 0;
  const uint32_t e = (bits >> 10) & 0x1fu;
  const uint32_t m = bits & 0x3ffu;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 0x1f) v = m == 0 ? INFINITY : NAN;
  else v = ldexpf(1.0f + (float)m / 1024.0f, (int)e - 15);
  return negative ? -v : v;
}

int po_e4m3_decode(uint8_t bits, float* value) {
  /* deepseek_fp8_activation_codec.cpp:11-25: e4m3fn, bias 7, no infinity,
   * S.1111.111 is the only NaN code and is rejected. */
  const uint32_t e = (bits >> 3) & 0x0fu, m = bits & 0x07u;
  if (e == 0x0fu && m == 0x07u) { *value = 0.0f; return 1; }
  const float mag = e == 0 ? ldexpf((float)m, -9) : ldexpf(1.0f + (float)m / 8.0f, (int)e - 7);
  *value = (bits & 0x80u) ? -mag : mag;
  return 0;
}

/* 256-entry decode table (the decode is exact, so the table changes no bit of
 * any result; NaN codes decode to 0 and are caught by the validity table). */
static float g_e4m3[256];
static uint8_t g_e4m3_nan[256];
static float g_e2m1[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                           -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
static int g_tables_ready = 0;
static void po_tables(void) {
  if (g_tables_ready) return;
  for (int b = 0; b < 256; ++b) g_e4m3_nan[b] = (uint8_t)po_e4m3_decode((uint8_t)b, &g_e4m3[b]);
  g_tables_ready = 1;
}

int po_e4m3_encode(float value, uint8_t* bits) {
  /* deepseek_fp8_activation_codec.cpp:27-51 picks the nearest finite code by
   * exhaustive search, preferring the even code on a tie.  Codes are monotone
   * in magnitude, so that is round-half-to-even on the code grid, computed
   * here directly from the float's bits. */
  if (!isfinite(value) || fabsf(value) > 448.0f) { *bits = 0; return 1; }
  const uint8_t sign = signbit(value) ? 0x80u : 0x00u;
  const float mag = fabsf(value);
  if (mag == 0.0f) { *bits = sign; return 0; }
  const uint32_t raw = f2u(mag);
  const int exp = (int)((raw >> 23) & 0xffu) - 127;
  uint32_t code;
  if (exp < -6) {
    /* subnormal grid: multiples of 2^-9 (code 8 is the smallest normal). */
    code = (uint32_t)nearbyintf(mag * 512.0f);
  } else {
    const uint32_t mant = raw & 0x7fffffu;
    uint32_t q = mant >> 20;
    const uint32_t rem = mant & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) ++q;
    int e = exp;
    if (q == 8u) { q = 0; ++e; }
    code = ((uint32_t)(e + 7) << 3) | q;
  }
  *bits = (uint8_t)(sign | code);
  return 0;
}

int po_mxfp4_decode_scalar(uint8_t e2m1_bits, uint8_t ue8m0_bits, double* value) {
  /* deepseek_mxfp4_codec.cpp:9-19 */
  static const double kMag[8] = {0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0};
  if (e2m1_bits > 0x0f || ue8m0_bits == 0xff) { *value = 0.0; return 1; }
  const double mag = kMag[e2m1_bits & 7u];
  *value = ldexp((e2m1_bits & 8u) ? -mag : mag, (int)ue8m0_bits - 127);
  return 0;
}

int po_mxfp4_decode_row(const uint8_t* packed, const uint8_t* scale_bits,
                        uint32_t logical_k, float* out) {
  /* deepseek_mxfp4_codec.cpp:21-46 */
  if (logical_k == 0) return 1;
  for (uint32_t k = 0; k < logical_k; ++k) {
    const uint8_t byte = packed[k / 2u];
    const uint8_t nib = (k & 1u) == 0 ? (byte & 0x0fu) : (byte >> 4);
    double d;
    if (po_mxfp4_decode_scalar(nib, scale_bits[k / 32u], &d)) return 2;
    if (!isfinite(d) || fabs(d) > 3.4028234663852886e38) return 3;
    out[k] = (float)d;
  }
  return 0;
}

/* ------------------------------------------------------- activation quant */
int po_fp8_quant_ue8m0(const float* input, uint32_t tokens, uint32_t logical_k,
                       uint8_t* codes, uint8_t* scale_bits) {
  /* deepseek_fp8_activation_codec.cpp:53-107 */
  if (tokens == 0 || logical_k == 0 || logical_k % 128u) return 1;
  const uint32_t groups = logical_k / 128u;
  int status = 0;
  PO_PARALLEL_FOR
  for (int64_t tg = 0; tg < (int64_t)tokens * groups; ++tg) {
    const size_t begin = (size_t)tg * 128u;
    float amax = 0.0f;
    int bad = 0;
    for (uint32_t i = 0; i < 128u; ++i) {
      const float v = input[begin + i];
      if (!isfinite(v)) bad = 1;
      amax = fmaxf(amax, fabsf(v));
    }
    if (bad) { status = 2; continue; }
    amax = fmaxf(amax, 1.0e-4f);
    const int e = (int)ceil(log2((double)amax / (double)448.0f));
    if (e < -127 || e > 127) { status = 3; continue; }
    const float scale = ldexpf(1.0f, e);
    scale_bits[tg] = (uint8_t)(e + 127);
    for (uint32_t i = 0; i < 128u; ++i) {
      float nv = input[begin + i] / scale;
      nv = nv < -448.0f ? -448.0f : (nv > 448.0f ? 448.0f : nv);
      po_e4m3_encode(nv, &codes[begin + i]);
    }
  }
  return status;
}

int po_fp8_quant_f32(const float* input, uint32_t tokens, uint32_t logical_k,
                     uint8_t* codes, float* scales) {
  if (tokens == 0 || logical_k == 0 || logical_k % 128u) return 1;
  const uint32_t groups = logical_k / 128u;
  int status = 0;
  PO_PARALLEL_FOR
  for (int64_t tg = 0; tg < (int64_t)tokens * groups; ++tg) {
    const size_t begin = (size_t)tg * 128u;
    float amax = 0.0f;
    int bad = 0;
    for (uint32_t i = 0; i < 128u; ++i) {
      const float v = input[begin + i];
      if (!isfinite(v)) bad = 1;
      amax = fmaxf(amax, fabsf(v));
    }
    if (bad) { status = 2; continue; }
    const float s = fmaxf(amax, 1.0e-4f) / 448.0f;
    scales[tg] = s;
    for (uint32_t i = 0; i < 128u; ++i) {
      float nv = input[begin + i] / s;
      nv = nv < -448.0f ? -448.0f : (nv > 448.0f ? 448.0f : nv);
      po_e4m3_encode(nv, &codes[begin + i]);
    }
  }
  return status;
}

/* ------------------------------------------------------------------ GEMMs */
int po_fp8_gemm_ue8m0(const uint8_t* a, const uint8_t* a_scale_bits,
                      const uint8_t* w, const uint8_t* w_scale_bits,
                      uint32_t m, uint32_t n, uint32_t k, float* out) {
  /* src/model/deepseek_fp8_gemm_oracle.cpp:10-80 */
  if (m == 0 || n == 0 || n % 128u || k == 0 || k % 128u) return 1;
  po_tables();
  const uint32_t kb = k / 128u;
  int status = 0;
  PO_PARALLEL_FOR
  for (int64_t idx = 0; idx < (int64_t)m * n; ++idx) {
    const uint32_t row = (uint32_t)(idx / n), col = (uint32_t)(idx % n);
    const uint8_t* ar = a + (size_t)row * k;
    const uint8_t* wr = w + (size_t)col * k;
    float acc = 0.0f;
    int bad = 0;
    for (uint32_t b = 0; b < kb && !bad; ++b) {
      const uint8_t sa = a_scale_bits[(size_t)row * kb + b];
      const uint8_t sw = w_scale_bits[(size_t)(col / 128u) * kb + b];
      if (sa == 0xffu || sw == 0xffu) { bad = 2; break; }
      float local = 0.0f;
      for (uint32_t i = 0; i < 128u; ++i) {
        const uint8_t x = ar[b * 128u + i], y = wr[b * 128u + i];
        if (g_e4m3_nan[x] | g_e4m3_nan[y]) { bad = 3; break; }
        local += g_e4m3[x] * g_e4m3[y];
      }
      acc += local * ldexpf(1.0f, (int)sa - 127) * ldexpf(1.0f, (int)sw - 127);
      if (!isfinite(acc)) bad = 4;
    }
    if (bad) { status = bad; continue; }
    out[idx] = acc;
  }
  return status;
}

int po_fp8_gemm_f32(const uint8_t* a, const float* a_scale, const uint8_t* w,
                    const float* w_scale, uint32_t m, uint32_t n, uint32_t k,
                    float* out) {
  if (m == 0 || n == 0 || n % 128u || k == 0 || k % 128u) return 1;
  po_tables();
  const uint32_t kb = k / 128u;
  int status = 0;
  PO_PARALLEL_FOR
  for (int64_t idx = 0; idx < (int64_t)m * n; ++idx) {
    const uint32_t row = (uint32_t)(idx / n), col = (uint32_t)(idx % n);
    const uint8_t* ar = a + (size_t)row * k;
    const uint8_t* wr = w + (size_t)col * k;
    float acc = 0.0f;
    int bad = 0;
    for (uint32_t b = 0; b < kb && !bad; ++b) {
      float local = 0.0f;
      for (uint32_t i = 0; i < 128u; ++i) {
        const uint8_t x = ar[b * 128u + i], y = wr[b * 128u + i];
        if (g_e4m3_nan[x] | g_e4m3_nan[y]) { bad = 3; break; }
        local += g_e4m3[x] * g_e4m3[y];
      }
      acc += local * a_scale[(size_t)row * kb + b] * w_scale[(size_t)(col / 128u) * kb + b];
      if (!isfinite(acc)) bad = 4;
    }
    if (bad) { status = bad; continue; }
    out[idx] = acc;
  }
  return status;
}

int po_fp4_gemm(const uint8_t* a, const uint8_t* a_scale_bits,
                const uint8_t* packed, const uint8_t* w_scale_bits, uint32_t m,
                uint32_t n, uint32_t k, float* out) {
  /* src/model/deepseek_fp4_gemm_oracle.cpp:11-91 */
  if (m == 0 || n == 0 || k == 0 || k % 128u) return 1;
  po_tables();
  const uint32_t k32 = k / 32u, k128 = k / 128u;
  int status = 0;
  PO_PARALLEL_FOR
  for (int64_t idx = 0; idx < (int64_t)m * n; ++idx) {
    const uint32_t row = (uint32_t)(idx / n), col = (uint32_t)(idx % n);
    float acc = 0.0f;
    int bad = 0;
    for (uint32_t b = 0; b < k32 && !bad; ++b) {
      const uint8_t sa = a_scale_bits[(size_t)row * k128 + b / 4u];
      const uint8_t sw = w_scale_bits[(size_t)col * k32 + b];
      if (sa == 0xffu || sw == 0xffu) { bad = 2; break; }
      const float as = ldexpf(1.0f, (int)sa - 127);
      const float ws = ldexpf(1.0f, (int)sw - 127);
      float local = 0.0f;
      for (uint32_t i = 0; i < 32u; ++i) {
        const uint32_t kk = b * 32u + i;
        const uint8_t x = a[(size_t)row * k + kk];
        if (g_e4m3_nan[x]) { bad = 3; break; }
        const uint8_t p = packed[(size_t)col * (k / 2u) + kk / 2u];
        const uint8_t nib = (kk & 1u) == 0 ? (p & 0x0fu) : (p >> 4);
        local += g_e4m3[x] * g_e2m1[nib];
      }
      acc += local * as * ws;
      if (!isfinite(acc)) bad = 4;
    }
    if (bad) { status = bad; continue; }
    out[idx] = acc;
  }
  return status;
}

int po_mxfp4_bf16_gemm(const uint16_t* x, const uint8_t* packed,
                       const uint8_t* w_scale_bits, uint32_t m, uint32_t n,
                       uint32_t k, float* out) {
  if (m == 0 || n == 0 || k == 0 || k % 32u) return 1;
  const uint32_t k32 = k / 32u;
  int status = 0;
  PO_PARALLEL_FOR
  for (int64_t idx = 0; idx < (int64_t)m * n; ++idx) {
    const uint32_t row = (uint32_t)(idx / n), col = (uint32_t)(idx % n);
    float acc = 0.0f;
    int bad = 0;
    for (uint32_t kk = 0; kk < k; ++kk) {
      const uint8_t sw = w_scale_bits[(size_t)col * k32 + kk / 32u];
      if (sw == 0xffu) { bad = 2; break; }
      const uint8_t p = packed[(size_t)col * (k / 2u) + kk / 2u];
      const uint8_t nib = (kk & 1u) == 0 ? (p & 0x0fu) : (p >> 4);
      const float wv = ldexpf(g_e2m1[nib], (int)sw - 127);
      acc += po_bf16_to_f32(x[(size_t)row * k + kk]) * wv;
    }
    if (bad || !isfinite(acc)) { status = bad ? bad : 4; continue; }
    out[idx] = acc;
  }
  return status;
}

int po_w4a16_sym(const uint16_t* x, const uint8_t* packed,
                 const uint16_t* scales_f16, uint32_t m, uint32_t n, uint32_t k,
                 uint16_t* out) {
  /* kernels/cuda/qwen_bf16_primitives.cu:98-149 (per-output loop body). */
  if (m == 0 || n == 0 || k == 0 || k % 128u) return 11;
  int status = 0;
  PO_PARALLEL_FOR
  for (int64_t idx = 0; idx < (int64_t)m * n; ++idx) {
    const uint32_t row = (uint32_t)(idx / n), col = (uint32_t)(idx % n);
    float acc = 0.0f;
    int bad = 0;
    for (uint32_t i = 0; i < k; ++i) {
      const uint8_t p = packed[(size_t)col * (k / 2u) + i / 2u];
      const uint8_t nib = (i & 1u) == 0 ? (p & 0x0fu) : (p >> 4);
      if (nib == 0x08u) { bad = 12; break; }
      const int32_t q = nib < 8u ? (int32_t)nib : (int32_t)nib - 16;
      const float s = po_f16_to_f32(scales_f16[(size_t)col * (k / 128u) + i / 128u]);
      if (!(s > 0.0f) || !isfinite(s)) { bad = 13; break; }
      acc += po_bf16_to_f32(x[(size_t)row * k + i]) * ((float)q * s);
    }
    if (!bad && !isfinite(acc)) bad = 14;
    if (bad) { status = bad; continue; }
    out[idx] = po_bf16_from_f32(acc);
  }
  return status;
}

static inline float asym_weight(const uint32_t* qweight, const uint16_t* scales,
                                const uint32_t* zeros, uint32_t k, uint32_t col,
                                uint32_t i) {
  const uint32_t groups = k / 128u, zwords = (groups + 7u) / 8u;
  const uint32_t q = (qweight[(size_t)col * (k / 8u) + i / 8u] >> (4u * (i % 8u))) & 0xfu;
  const uint32_t g = i / 128u;
  const uint32_t z = (zeros[(size_t)col * zwords + g / 8u] >> (4u * (g % 8u))) & 0xfu;
  const float s = po_bf16_to_f32(scales[(size_t)col * groups + g]);
  return (float)((int32_t)q - (int32_t)z) * s;
}

int po_w4a16_asym(const uint16_t* x, const uint32_t* qweight,
                  const uint16_t* scales_bf16, const uint32_t* zeros,
                  uint32_t m, uint32_t n, uint32_t k, uint16_t* out) {
  if (m == 0 || n == 0 || k == 0 || k % 128u) return 11;
  int status = 0;
  PO_PARALLEL_FOR
  for (int64_t idx = 0; idx < (int64_t)m * n; ++idx) {
    const uint32_t row = (uint32_t)(idx / n), col = (uint32_t)(idx % n);
    float acc = 0.0f;
    for (uint32_t i = 0; i < k; ++i)
      acc += po_bf16_to_f32(x[(size_t)row * k + i]) *
             asym_weight(qweight, scales_bf16, zeros, k, col, i);
    if (!isfinite(acc)) { status = 14; continue; }
    out[idx] = po_bf16_from_f32(acc);
  }
  return status;
}

int po_w4a16_asym_dequant(const uint32_t* qweight, const uint16_t* scales_bf16,
                          const uint32_t* zeros, uint32_t n, uint32_t k,
                          float* w) {
  if (n == 0 || k == 0 || k % 128u) return 11;
  PO_PARALLEL_FOR
  for (int64_t col = 0; col < (int64_t)n; ++col)
    for (uint32_t i = 0; i < k; ++i)
      w[(size_t)col * k + i] = asym_weight(qweight, scales_bf16, zeros, k, (uint32_t)col, i);
  return 0;
}

void po_bf16_gemm(const uint16_t* a, const uint16_t* w, uint32_t m, uint32_t n,
                  uint32_t k, float* out) {
  PO_PARALLEL_FOR
  for (int64_t idx = 0; idx < (int64_t)m * n; ++idx) {
    const uint32_t row = (uint32_t)(idx / n), col = (uint32_t)(idx % n);
    const uint16_t* ar = a + (size_t)row * k;
    const uint16_t* wr = w + (size_t)col * k;
    float acc = 0.0f;
    for (uint32_t i = 0; i < k; ++i) acc += po_bf16_to_f32(ar[i]) * po_bf16_to_f32(wr[i]);
    out[idx] = acc;
  }
}

/* DeepSeek LM head (plugins/kernels/deepseek-v4-sm89/native/
 * deepseek_endpoint.cu:94-115): logits[r, v] = sum_h x[r, h] * W[v, h] in
 * the reference block's order -- 256 strided fp32 partial sums (thread t
 * takes h = t, t + 256, ...), then the shared-memory tree halving 128, 64,
 * ..., 1 (reduce_sum, :13-24).  Bit 64 when an x or W element read is
 * non-finite, bit 128 when the sum is; the logit is written either way. */
uint32_t po_lm_head(const uint16_t* x, const uint16_t* w, uint32_t rows, uint32_t vocab,
                    uint32_t hidden, float* logits) {
  uint32_t err = 0;
  PO_PARALLEL_FOR_REDUCE_OR(err)
  for (int64_t idx = 0; idx < (int64_t)rows * vocab; ++idx) {
    const uint32_t row = (uint32_t)(idx / vocab), word = (uint32_t)(idx % vocab);
    float part[256];
    for (uint32_t t = 0; t < 256; ++t) {
      float acc = 0.0f;
      for (uint32_t h = t; h < hidden; h += 256) {
        const float xv = po_bf16_to_f32(x[(size_t)row * hidden + h]);
        const float wv = po_bf16_to_f32(w[(size_t)word * hidden + h]);
        if (!isfinite(xv) || !isfinite(wv)) err |= 64u;
        acc += xv * wv;
      }
      part[t] = acc;
    }
    for (uint32_t width = 128; width != 0; width >>= 1)
      for (uint32_t t = 0; t < width; ++t) part[t] += part[t + width];
    if (!isfinite(part[0])) err |= 128u;
    logits[(size_t)row * vocab + word] = part[0];
  }
  return err;
}

/* ------------------------------------------ DeepSeek V4.1 32-block formats */
/* Expert FP4 32x32 block -> FP8 e4m3 + shared UE8M0
 * (plugins/model-deepseek-v41/weight_expert_convert.cpp:33-63): shared =
 * max(row scale) - 6 (NaN scale 255: code 1; max < 6: code 2); value =
 * e2m1 magnitude * 2^(row - max + 6) rounded to the nearest e4m3 code, ties
 * to the even code; both zero codes give +0, other negatives keep the sign
 * (also when they round to zero).  Below 2^-30 every magnitude rounds to 0;
 * above it the float product is exact, so po_e4m3_encode applies. */
int po_v41_fp4_block_to_fp8(const uint8_t* packed, const uint8_t* scales, uint8_t* weight, uint8_t* scale) {
  static const float mags[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  unsigned maximum = 0;
  for (int r = 0; r < 32; ++r) {
    if (scales[r] == 255) return 1;
    if (scales[r] > maximum) maximum = scales[r];
  }
  if (maximum < 6) return 2;
  *scale = (uint8_t)(maximum - 6);
  for (int r = 0; r < 32; ++r) {
    const int shift = (int)scales[r] - (int)maximum + 6;
    for (int c = 0; c < 32; ++c) {
      const unsigned nib = (packed[r * 16 + c / 2] >> ((c & 1) * 4)) & 15u;
      const unsigned mag = nib & 7u;
      uint8_t code = 0;
      if (mag && shift >= -30) po_e4m3_encode(ldexpf(mags[mag], shift), &code);
      if ((nib & 8u) && mag) code |= 0x80u;
      weight[r * 32 + c] = code;
    }
  }
  return 0;
}

/* The tensor form (ConvertExpertFp4Tensor, :64-100): packed [rows, cols/2],
 * scales [rows, cols/32] -> e4m3 [rows, cols], UE8M0 [rows/32, cols/32];
 * returns the first failing block's code. */
int po_v41_fp4_to_fp8(const uint8_t* packed, const uint8_t* scales, uint32_t rows, uint32_t cols, uint8_t* weight,
                      uint8_t* out_scales) {
  uint8_t blk_packed[512], blk_scales[32], blk_out[1024];
  for (uint32_t r0 = 0; r0 < rows; r0 += 32)
    for (uint32_t g = 0; g < cols / 32; ++g) {
      for (uint32_t r = 0; r < 32; ++r) {
        memcpy(blk_packed + r * 16, packed + (size_t)(r0 + r) * (cols / 2) + g * 16, 16);
        blk_scales[r] = scales[(size_t)(r0 + r) * (cols / 32) + g];
      }
      const int st = po_v41_fp4_block_to_fp8(blk_packed, blk_scales, blk_out, &out_scales[(size_t)(r0 / 32) * (cols / 32) + g]);
      if (st) return st;
      for (uint32_t r = 0; r < 32; ++r) memcpy(weight + (size_t)(r0 + r) * cols + g * 32, blk_out + r * 32, 32);
    }
  return 0;
}

/* wo_a block dequantisation (weight_dequantize.cpp:24-50): e4m3 x scale in
 * fp32, bf16 round to nearest even.  Codes: 1 scale not finite and > 0,
 * 2 NaN source code, 3 non-finite fp32 product, 4 bf16 overflow. */
int po_v41_dequant_block(const uint8_t* src, float scale, uint32_t block, uint16_t* out) {
  if ((block != 32 && block != 128) || !isfinite(scale) || scale <= 0.0f) return 1;
  po_tables();
  for (uint32_t i = 0; i < block * block; ++i) {
    if (g_e4m3_nan[src[i]]) return 2;
    const float v = g_e4m3[src[i]] * scale;
    if (!isfinite(v)) return 3;
    const uint16_t h = po_bf16_from_f32(v);
    if (!isfinite(po_bf16_to_f32(h))) return 4;
    out[i] = h;
  }
  return 0;
}

/* The V4.1 linear's activation quant (plugins/model-deepseek-v41/
 * linear_fp8.cu:18-34), per (row, 32 k): amax of the finite values, floor
 * 1e-4, times the fp32 constant 1/448; the exponent of that product, plus
 * one unless it is a power of two, is the scale 2^e (byte e + 127); codes
 * are clamp(x / 2^e, +-448) rounded to nearest even, non-finite inputs
 * encode 0 and raise bit 1. */
uint32_t po_v41_quant32(const uint16_t* x, uint32_t rows, uint32_t k, uint8_t* codes, uint8_t* scales) {
  uint32_t err = 0;
  for (size_t g = 0; g < (size_t)rows * (k / 32); ++g) {
    float maximum = 0.0f;
    for (int l = 0; l < 32; ++l) {
      const float v = po_bf16_to_f32(x[g * 32 + l]);
      if (!isfinite(v)) err |= 1u;
      else maximum = fmaxf(maximum, fabsf(v));
    }
    const float scaled = fmaxf(maximum, 1e-4f) * (1.0f / 448.0f);
    const uint32_t bits = f2u(scaled);
    const int e = (int)((bits >> 23) & 255u) - 127 + ((bits & 0x7fffffu) != 0u);
    scales[g] = (uint8_t)(e + 127);
    const float scale = ldexpf(1.0f, e);
    for (int l = 0; l < 32; ++l) {
      const float v = po_bf16_to_f32(x[g * 32 + l]);
      const float q = isfinite(v) ? fminf(fmaxf(v / scale, -448.0f), 448.0f) : 0.0f;
      po_e4m3_encode(q, &codes[g * 32 + l]);
    }
  }
  return err;
}

/* The V4.1 projection (linear_fp8.cu:39-76): per 32-deep group a sequential
 * fp32 dot of the decoded operands, term = (dot * 2^(sa-127)) * 2^(sb-127),
 * accumulated in group order; bf16 out.  sb is the 32x32 block's scale
 * (fp4 = 0) or the weight row's per-32 scale (fp4 = 1, e2m1 weights, even
 * k in the low nibble).  Bits: 1 a NaN operand or a 255 scale, 2 a
 * non-finite term, accumulator or bf16 output. */
uint32_t po_v41_linear(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, uint32_t rows,
                       uint32_t n, uint32_t k, int fp4, uint16_t* out) {
  po_tables();
  uint32_t err = 0;
  const uint32_t groups = k / 32;
  PO_PARALLEL_FOR_REDUCE_OR(err)
  for (int64_t idx = 0; idx < (int64_t)rows * n; ++idx) {
    const uint32_t t = (uint32_t)(idx / n), col = (uint32_t)(idx % n);
    float acc = 0.0f;
    for (uint32_t g = 0; g < groups; ++g) {
      float dot = 0.0f;
      for (uint32_t i = 0; i < 32; ++i) {
        const uint8_t ac = a[(size_t)t * k + g * 32 + i];
        float av = g_e4m3_nan[ac] ? NAN : g_e4m3[ac], bv;
        if (fp4) {
          const uint8_t byte = w[(size_t)col * (k / 2) + g * 16 + i / 2];
          bv = g_e2m1[(byte >> ((i & 1) * 4)) & 15u];
        } else {
          const uint8_t wc = w[(size_t)col * k + g * 32 + i];
          bv = g_e4m3_nan[wc] ? NAN : g_e4m3[wc];
        }
        if (!isfinite(av) || !isfinite(bv)) err |= 1u;
        dot += av * bv;
      }
      const uint8_t sab = sa[(size_t)t * groups + g];
      const uint8_t sbb = sw[(size_t)(fp4 ? col : col / 32) * groups + g];
      if (sab == 255 || sbb == 255) err |= 1u;
      const float term = (dot * ldexpf(1.0f, (int)sab - 127)) * ldexpf(1.0f, (int)sbb - 127);
      acc += term;
      if (!isfinite(term) || !isfinite(acc)) err |= 2u;
    }
    const uint16_t h = po_bf16_from_f32(acc);
    if (!isfinite(po_bf16_to_f32(h))) err |= 2u;
    out[idx] = h;
  }
  return err;
}

/* ------------------------------------------------------------ elementwise */
void po_silu_mul(const uint16_t* gate, const uint16_t* up, size_t count,
                 uint16_t* out) {
  /* plugins/model-qwen3/qwen3_cpu_oracle.cpp:114-126 */
  for (size_t i = 0; i < count; ++i) {
    const float g = po_bf16_to_f32(gate[i]);
    out[i] = po_bf16_from_f32((g / (1.0f + expf(-g))) * po_bf16_to_f32(up[i]));
  }
}

int po_swiglu(const float* gate, const float* up, size_t count, float limit,
              float* out) {
  /* src/model/deepseek_expert_swiglu_oracle.cpp:11-42 */
  for (size_t i = 0; i < count; ++i) {
    float g = gate[i], u = up[i];
    if (!isfinite(g) || !isfinite(u)) return 1;
    if (limit > 0.0f) {
      g = fminf(g, limit);
      u = u < -limit ? -limit : (u > limit ? limit : u);
    }
    const float v = (g / (1.0f + expf(-g))) * u;
    if (!isfinite(v)) return 2;
    out[i] = v;
  }
  return 0;
}

/* ------------------------------------------------------------ router top-k */
typedef struct {
  uint32_t expert;
  float base, selection;
} po_ranked;

/* (selection descending, expert ascending): the order of the reference's
 * partial_sort comparator (deepseek_learned_router.cpp:57-64). */
static int ranked_before(const po_ranked* a, const po_ranked* b) {
  if (a->selection != b->selection) return a->selection > b->selection;
  return a->expert < b->expert;
}

static float stable_softplus(float v) {
  /* deepseek_learned_router.cpp:10-13 */
  return v > 0.0f ? v + log1pf(expf(-v)) : log1pf(expf(v));
}

int po_router_topk(const float* scores, const float* bias, uint32_t tokens,
                   uint32_t experts, uint32_t topk, uint32_t mode, float scale,
                   uint32_t* ids, float* weights) {
  if (tokens == 0 || experts == 0 || topk == 0 || topk > experts || topk > 32 ||
      (mode != 1 && mode != 2))
    return 1;
  if (mode == 2 && bias)
    for (uint32_t e = 0; e < experts; ++e)
      if (!isfinite(bias[e])) return 3;
  for (size_t i = 0; i < (size_t)tokens * experts; ++i)
    if (!isfinite(scores[i])) return 2;
  int bad = 0;
  PO_PARALLEL_FOR
  for (uint32_t t = 0; t < tokens; ++t) {
    const float* s = scores + (size_t)t * experts;
    po_ranked best[32];
    uint32_t count = 0;
    float mx = -INFINITY;
    for (uint32_t e = 0; e < experts; ++e) mx = s[e] > mx ? s[e] : mx;
    for (uint32_t e = 0; e < experts; ++e) {
      po_ranked r;
      r.expert = e;
      if (mode == 2) {
        /* deepseek_learned_router.cpp:44-52: base = sqrt(softplus(raw)),
         * selection = base + bias */
        r.base = sqrtf(stable_softplus(s[e]));
        r.selection = r.base + (bias ? bias[e] : 0.0f);
      } else {
        /* softmax is strictly increasing in the score, so the top-k of the
         * probabilities is the top-k of the scores */
        r.base = s[e];
        r.selection = s[e];
      }
      /* insertion into the sorted best-k list */
      uint32_t at = count;
      while (at > 0 && ranked_before(&r, &best[at - 1])) --at;
      if (at >= topk) continue;
      const uint32_t last = count < topk ? count++ : topk - 1;
      for (uint32_t j = last; j > at; --j) best[j] = best[j - 1];
      best[at] = r;
    }
    uint32_t* oid = ids + (size_t)t * topk;
    float* ow = weights + (size_t)t * topk;
    if (mode == 2) {
      /* deepseek_learned_router.cpp:65-81: weights base / sum(base) * 1.5 */
      float den = 0.0f;
      for (uint32_t j = 0; j < topk; ++j) den += best[j].base;
      if (!isfinite(den) || den <= 0.0f) {
#pragma omp atomic write
        bad = 4;
        continue;
      }
      for (uint32_t j = 0; j < topk; ++j) {
        oid[j] = best[j].expert;
        ow[j] = best[j].base / den * scale;
      }
    } else {
      /* BASELINE: p = softmax over all experts (exp of score - max, summed
       * in expert order), then the selected p renormalised to sum 1 */
      float sum = 0.0f;
      for (uint32_t e = 0; e < experts; ++e) sum += expf(s[e] - mx);
      float psel = 0.0f, p[32];
      for (uint32_t j = 0; j < topk; ++j) {
        p[j] = expf(best[j].base - mx) / sum;
        psel += p[j];
      }
      for (uint32_t j = 0; j < topk; ++j) {
        oid[j] = best[j].expert;
        ow[j] = p[j] / psel * scale;
      }
    }
  }
  return bad;
}

/* -------------------------------------------------------- MoE route plan */
typedef struct {
  uint32_t expert, token, ordinal;
  float weight;
} po_route;

static int route_cmp(const void* l, const void* r) {
  const po_route* a = (const po_route*)l;
  const po_route* b = (const po_route*)r;
  if (a->expert != b->expert) return a->expert < b->expert ? -1 : 1;
  if (a->token != b->token) return a->token < b->token ? -1 : 1;
  return a->ordinal < b->ordinal ? -1 : (a->ordinal > b->ordinal);
}

int po_route_plan(const uint32_t* topk_ids, const float* topk_weights,
                  uint32_t tokens, uint32_t topk, uint32_t experts,
                  uint32_t* expert_offsets, uint32_t* row_token,
                  float* row_weight, uint32_t* token_rows) {
  /* deepseek_expert_subwave_plan.cpp:32-101 */
  if (tokens == 0 || topk == 0 || experts == 0) return 1;
  const size_t routes = (size_t)tokens * topk;
  po_route* r = (po_route*)malloc(routes * sizeof(po_route));
  if (!r) return 1;
  for (uint32_t t = 0; t < tokens; ++t) {
    for (uint32_t j = 0; j < topk; ++j) {
      const size_t i = (size_t)t * topk + j;
      const float w = topk_weights[i];
      if (topk_ids[i] >= experts) { free(r); return 2; }
      if (!isfinite(w) || w < 0.0f) { free(r); return 4; }
      for (uint32_t p = 0; p < j; ++p)
        if (topk_ids[(size_t)t * topk + p] == topk_ids[i]) { free(r); return 3; }
      r[i].expert = topk_ids[i];
      r[i].token = t;
      r[i].ordinal = j;
      r[i].weight = w;
    }
  }
  qsort(r, routes, sizeof(po_route), route_cmp);
  size_t cursor = 0;
  for (uint32_t e = 0; e < experts; ++e) {
    expert_offsets[e] = (uint32_t)cursor;
    while (cursor < routes && r[cursor].expert == e) ++cursor;
  }
  expert_offsets[experts] = (uint32_t)cursor;
  for (size_t i = 0; i < routes; ++i) {
    row_token[i] = r[i].token;
    row_weight[i] = r[i].weight;
    token_rows[(size_t)r[i].token * topk + r[i].ordinal] = (uint32_t)i;
  }
  free(r);
  return 0;
}

int po_ordered_accumulate(const uint16_t* expert_out_bf16,
                          const uint32_t* row_token, uint32_t rows,
                          uint32_t tokens, uint32_t hidden, float* acc) {
  /* src/model/deepseek_expert_accumulator_oracle.cpp:20-67: the rows are
   * already in (expert, token) order, so each token's sum runs over its
   * experts in increasing id, exactly as add_expert() is called. */
  for (uint32_t r = 0; r < rows; ++r) {
    const uint32_t t = row_token[r];
    if (t >= tokens) return 1;
    for (uint32_t c = 0; c < hidden; ++c) {
      const float v = po_bf16_to_f32(expert_out_bf16[(size_t)r * hidden + c]);
      if (!isfinite(v)) return 2;
      acc[(size_t)t * hidden + c] += v;
      if (!isfinite(acc[(size_t)t * hidden + c])) return 3;
    }
  }
  return 0;
}

int po_finalize(const float* acc, const uint16_t* shared_bf16, size_t count,
                uint16_t* out) {
  /* deepseek_expert_accumulator_oracle.cpp:69-85 then the bf16 store of
   * expert_finalize (plugins/kernels/deepseek-v4-sm89/native/
   * deepseek_expert_accumulate.cu:41-56). */
  for (size_t i = 0; i < count; ++i) {
    const float v = acc[i] + (shared_bf16 ? po_bf16_to_f32(shared_bf16[i]) : 0.0f);
    if (!isfinite(v)) return 1;
    out[i] = po_bf16_from_f32(v);
  }
  return 0;
}

/* ----------------------------------------------------- routed expert chain */
static int round_bf16_vec(float* v, size_t count) {
  for (size_t i = 0; i < count; ++i) {
    const float r = po_bf16_to_f32(po_bf16_from_f32(v[i]));
    if (!isfinite(r)) return 1;
    v[i] = r;
  }
  return 0;
}

static int project_fp4(const float* in, uint32_t tokens, uint32_t in_size,
                       uint32_t out_size, const uint8_t* packed,
                       const uint8_t* scales, float* out) {
  /* deepseek_routed_expert_oracle.cpp:34-46 */
  uint8_t* q = (uint8_t*)malloc((size_t)tokens * in_size);
  uint8_t* s = (uint8_t*)malloc((size_t)tokens * (in_size / 128u));
  int st = (q && s) ? po_fp8_quant_ue8m0(in, tokens, in_size, q, s) : 1;
  if (!st) st = po_fp4_gemm(q, s, packed, scales, tokens, out_size, in_size, out);
  if (!st) st = round_bf16_vec(out, (size_t)tokens * out_size);
  free(q);
  free(s);
  return st;
}

int po_routed_expert_fp4(const uint16_t* input_bf16, const float* route_weights,
                         uint32_t tokens, uint32_t hidden,
                         uint32_t intermediate, const uint8_t* w1_packed,
                         const uint8_t* w1_scales, const uint8_t* w2_packed,
                         const uint8_t* w2_scales, const uint8_t* w3_packed,
                         const uint8_t* w3_scales, uint16_t* out_bf16) {
  /* src/model/deepseek_routed_expert_oracle.cpp:50-95 */
  if (tokens == 0 || hidden == 0 || intermediate == 0 || hidden % 128u ||
      intermediate % 128u)
    return 1;
  for (uint32_t t = 0; t < tokens; ++t)
    if (!isfinite(route_weights[t]) || route_weights[t] < 0.0f) return 1;
  const size_t nx = (size_t)tokens * hidden, ni = (size_t)tokens * intermediate;
  float* x = (float*)malloc(nx * sizeof(float));
  float* gate = (float*)malloc(ni * sizeof(float));
  float* up = (float*)malloc(ni * sizeof(float));
  float* mid = (float*)malloc(ni * sizeof(float));
  float* y = (float*)malloc(nx * sizeof(float));
  int st = (x && gate && up && mid && y) ? 0 : 1;
  if (!st) for (size_t i = 0; i < nx; ++i) x[i] = po_bf16_to_f32(input_bf16[i]);
  if (!st) st = project_fp4(x, tokens, hidden, intermediate, w1_packed, w1_scales, gate);
  if (!st) st = project_fp4(x, tokens, hidden, intermediate, w3_packed, w3_scales, up);
  if (!st) st = po_swiglu(gate, up, ni, 10.0f, mid);
  if (!st) {
    for (uint32_t t = 0; t < tokens; ++t)
      for (uint32_t c = 0; c < intermediate; ++c) mid[(size_t)t * intermediate + c] *= route_weights[t];
    st = round_bf16_vec(mid, ni);
  }
  if (!st) st = project_fp4(mid, tokens, intermediate, hidden, w2_packed, w2_scales, y);
  if (!st) for (size_t i = 0; i < nx; ++i) out_bf16[i] = po_bf16_from_f32(y[i]);
  free(x); free(gate); free(up); free(mid); free(y);
  return st;
}

int po_expert_fp8(const uint16_t* input_bf16, const float* route_weights,
                  uint32_t tokens, uint32_t hidden, uint32_t intermediate,
                  const uint8_t* w13, const float* w13_scale, const uint8_t* w2,
                  const float* w2_scale, float limit, uint16_t* out_bf16) {
  if (tokens == 0 || hidden == 0 || intermediate == 0 || hidden % 128u ||
      intermediate % 128u)
    return 1;
  const size_t nx = (size_t)tokens * hidden, ni = (size_t)tokens * intermediate;
  const uint32_t n13 = 2u * intermediate;
  float* x = (float*)malloc(nx * sizeof(float));
  uint8_t* xq = (uint8_t*)malloc(nx);
  float* xs = (float*)malloc((nx / 128u) * sizeof(float));
  float* gu = (float*)malloc((size_t)tokens * n13 * sizeof(float));
  float* gate = (float*)malloc(ni * sizeof(float));
  float* up = (float*)malloc(ni * sizeof(float));
  float* mid = (float*)malloc(ni * sizeof(float));
  uint8_t* mq = (uint8_t*)malloc(ni);
  float* ms = (float*)malloc((ni / 128u) * sizeof(float));
  float* y = (float*)malloc(nx * sizeof(float));
  int st = (x && xq && xs && gu && gate && up && mid && mq && ms && y) ? 0 : 1;
  if (!st) for (size_t i = 0; i < nx; ++i) x[i] = po_bf16_to_f32(input_bf16[i]);
  if (!st) st = po_fp8_quant_f32(x, tokens, hidden, xq, xs);
  if (!st) st = po_fp8_gemm_f32(xq, xs, w13, w13_scale, tokens, n13, hidden, gu);
  if (!st) {
    for (uint32_t t = 0; t < tokens; ++t)
      for (uint32_t c = 0; c < intermediate; ++c) {
        gate[(size_t)t * intermediate + c] = gu[(size_t)t * n13 + c];
        up[(size_t)t * intermediate + c] = gu[(size_t)t * n13 + intermediate + c];
      }
    st = round_bf16_vec(gate, ni);
  }
  if (!st) st = round_bf16_vec(up, ni);
  if (!st) st = po_swiglu(gate, up, ni, limit, mid);
  if (!st) {
    for (uint32_t t = 0; t < tokens; ++t)
      for (uint32_t c = 0; c < intermediate; ++c) mid[(size_t)t * intermediate + c] *= route_weights[t];
    st = round_bf16_vec(mid, ni);
  }
  if (!st) st = po_fp8_quant_f32(mid, tokens, intermediate, mq, ms);
  if (!st) st = po_fp8_gemm_f32(mq, ms, w2, w2_scale, tokens, hidden, intermediate, y);
  if (!st) for (size_t i = 0; i < nx; ++i) out_bf16[i] = po_bf16_from_f32(y[i]);
  free(x); free(xq); free(xs); free(gu); free(gate); free(up); free(mid);
  free(mq); free(ms); free(y);
  return st;
}
