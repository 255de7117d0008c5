// Device-side helpers shared by every gfx950 kernel of the packs: bf16 and
// e4m3fn codecs written from the format definitions, wave reductions, and
// the CDNA4 MFMA operand types.
//
// Formats (the reference defines them in include/pih/core/bfloat16.h:13-27
// and plugins/model-deepseek-v4-flash/deepseek_fp8_activation_codec.cpp:11-51):
//   bf16   upper half of an IEEE binary32, round-to-nearest-even, NaN kept
//          quiet with its sign.
//   e4m3fn 1.4.3, bias 7, no infinities, S.1111.111 is the only NaN, largest
//          finite magnitude 448, subnormals are multiples of 2^-9.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pih_amd {

// 16 bytes by a non-temporal load (data read once)
__device__ __forceinline__ uint4 load16_nt(const uint4* p) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// LDS byte address of a __shared__ object (wave-uniform)
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p);
}

// Global -> LDS DMA of 16 (dma16) or 4 (dma4) bytes per lane: lane l's data
// lands at LDS byte lds + 16 l (resp. 4 l); lds is wave-uniform and goes to
// M0.  Issued as inline asm so that the compiler, which cannot tell which
// LDS bytes a DMA writes, adds no conservative vmcnt waits before LDS reads;
// the kernel orders the waits itself (an explicit s_waitcnt vmcnt, or a
// compiler wait for a load issued after the DMA: loads complete in issue
// order, and the compiler's count, which omits the DMA, only waits longer).
// M0 is written here only; nothing else in these kernels uses it.
// The address is a wave-uniform base (SGPRs) plus a per-lane 32-bit offset,
// or (dma4v) a per-lane 64-bit address.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(off), "s"(base)
               : "memory");
}
__device__ __forceinline__ void dma16nt(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt" ::"s"(lds), "v"(off), "s"(base)
               : "memory");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds), "v"(off), "s"(base)
               : "memory");
}
__device__ __forceinline__ void dma4v(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(lds), "v"(src) : "memory");
}

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v8s __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// Error bits OR-ed into the caller's u32 flag.
constexpr uint32_t kErrCode = 1u;     // invalid code / non-finite input
constexpr uint32_t kErrScale = 2u;    // scale byte 0xFF or exponent out of range
constexpr uint32_t kErrNonFinite = 4u;  // non-finite result (not written)

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

// fp32 -> bf16 bits by v_cvt_pk_bf16_f32: round to nearest even, a NaN
// keeps its sign and upper payload with the quiet bit set, i.e.
// (raw + 0x7fff + ((raw >> 16) & 1)) >> 16 and (raw >> 16) | 0x40 for a
// NaN (the same bits for all 2^32 inputs, checked on gfx950 with IEEE fp32
// denormals, the kernels' mode).
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{lo, hi}, v2bf));
}
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float v) { return f32x2_to_bf16x2(v, 0.0f) & 0xffffu; }

__device__ __forceinline__ float bf16_round(float v) {
  return bf16_bits_to_f32(f32_to_bf16_bits(v));
}

// SiLU x / (1 + e^-x) with the quotient as v_rcp_f32, a product and one FMA
// correction, sign restored: bit-equal to the IEEE quotient for every
// finite x whose denominator stays below 2^126 (all 2^32 inputs checked on
// gfx950).  `big` is set for the others (x < -87.3: the reciprocal
// underflows); there the caller uses silu_ieee.
__device__ __forceinline__ float silu_rcp(float x, bool& big) {
  const float d = 1.0f + expf(-x);
  big |= !(d < 0x1p126f);
  const float r = __builtin_amdgcn_rcpf(d);
  const float q = x * r;
  return __builtin_copysignf(__builtin_fmaf(__builtin_fmaf(-q, d, x), r, q), x);
}
__device__ __forceinline__ float silu_ieee(float x) { return x / (1.0f + expf(-x)); }

// Nearest finite e4m3fn code with ties to the even code; |v| <= 448 and
// finite is the caller's contract (every quantizer clamps first).
// Exponent e of the UE8M0 scale 2^e of a 128-value group with absolute
// maximum amax (amax >= 1e-4): the smallest e with amax <= 448 * 2^e.
__device__ __forceinline__ int ue8m0_exponent(float amax) {
  // start from the exponent of amax/448 and correct by exact comparisons
  int e = (int)((__float_as_uint(amax) >> 23) & 0xffu) - 127 - 8;
  // 448*2^e is exact for every e reached here (amax in [1e-4, FLT_MAX])
  while (amax > ldexpf(448.0f, e)) ++e;
  while (amax <= ldexpf(448.0f, e - 1)) --e;
  return e;
}

// e4m3 codes of v[0..3] / scale (clamped to the e4m3 range), rounded to
// nearest even by the hardware pack (v_cvt_pk_fp8_f32: operand a to the low
// byte of the selected half-word, b to the high byte); byte i is v[i].
__device__ __forceinline__ uint32_t e4m3_quant4(const float* v, float scale) {
  float q[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) q[i] = fminf(fmaxf(v[i] / scale, -448.0f), 448.0f);
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], w, true);
  return (uint32_t)w;
}

// e4m3_quant4 for an fp32 scale with inv = 1 / scale (one IEEE division per
// group instead of one per value): q0 = v * inv, the remainder v - q0 * scale
// exactly by an FMA, q = q0 + remainder * inv (Markstein's correction step,
// IBM J. Res. Dev. 34(1), 1990), sign of v kept for v = -0.  q can differ
// from v / scale in the last fp32 bit, but for every bf16 v with |v| <= amax
// and scale = max(amax, 1e-4) / 448, amax any positive bf16, the e4m3 code
// is the same (an exhaustive check over all 1.07e9 pairs is in the tests).
__device__ __forceinline__ uint32_t e4m3_quant4_recip(const float* v, float scale, float inv) {
  float q[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float q0 = v[i] * inv;
    const float rem = __builtin_fmaf(-q0, scale, v[i]);
    q[i] = fminf(fmaxf(__builtin_copysignf(__builtin_fmaf(rem, inv, q0), v[i]), -448.0f), 448.0f);
  }
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], w, true);
  return (uint32_t)w;
}

// e4m3_quant4 with the scale given as its exact reciprocal (a power of two):
// codes of v[0..3] * inv.
__device__ __forceinline__ uint32_t e4m3_quant4_mul(const float* v, float inv) {
  float q[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) q[i] = fminf(fmaxf(v[i] * inv, -448.0f), 448.0f);
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], w, true);
  return (uint32_t)w;
}

__device__ __forceinline__ uint32_t e4m3_encode(float v) {
  const uint32_t raw = __float_as_uint(v);
  const uint32_t sign = (raw >> 24) & 0x80u;
  const uint32_t mag_bits = raw & 0x7fffffffu;
  if (mag_bits == 0) return sign;
  const int exp = (int)(mag_bits >> 23) - 127;
  uint32_t code;
  if (exp < -6) {
    // Subnormal grid 2^-9; the scaling by 512 is exact, rintf rounds half to
    // even.  A result of 8 is the smallest normal code, which is correct.
    code = (uint32_t)__builtin_rintf(__uint_as_float(mag_bits) * 512.0f);
  } else {
    const uint32_t mant = mag_bits & 0x7fffffu;
    uint32_t q = mant >> 20;
    const uint32_t rem = mant & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) ++q;
    int e = exp;
    if (q == 8u) {
      q = 0;
      ++e;
    }
    code = ((uint32_t)(e + 7) << 3) | q;
  }
  return sign | code;
}

__device__ __forceinline__ float e4m3_decode(uint32_t bits) {
  const uint32_t e = (bits >> 3) & 0x0fu, m = bits & 7u;
  const float mag = e == 0 ? (float)m * 0x1p-9f
                           : __uint_as_float(((e + 120u) << 23) | (m << 20));
  return (bits & 0x80u) ? -mag : mag;
}

// Non-zero when any byte of w is an e4m3fn NaN code (x111 1111).
__device__ __forceinline__ uint32_t e4m3_nan_bytes(uint32_t w) {
  return ((w & 0x7f7f7f7fu) + 0x01010101u) & 0x80808080u;
}

// The word with its NaN codes (bit 7 of their byte set in `nan`, as
// e4m3_nan_bytes returns) replaced by +0: the value the reference's decode
// gives a NaN code while it raises the error bit
// (plugins/kernels/deepseek-v4-sm89/native/deepseek_fp8_gemm.cu:11-17).
__device__ __forceinline__ uint32_t e4m3_nan_to_zero(uint32_t w, uint32_t nan) { return w & ~((nan >> 7) * 0xffu); }

// e2m1 magnitudes {0, .5, 1, 1.5, 2, 3, 4, 6}, bit 3 is the sign.
__device__ __forceinline__ float e2m1_decode(uint32_t nib) {
  const uint32_t m = nib & 7u;
  // exact: value = m/2 for m < 4, else (m-2) for m in {4,5} -> 2,3 and 4,6.
  const float mag = m < 4u ? (float)m * 0.5f : (m == 4u ? 2.0f : m == 5u ? 3.0f : m == 6u ? 4.0f : 6.0f);
  return (nib & 8u) ? -mag : mag;
}

// 2^e as a float for e in [-126, 127].
__device__ __forceinline__ float exp2i(int e) {
  return __uint_as_float((uint32_t)(e + 127) << 23);
}

// 2^(b-127) for a UE8M0 byte b in [0, 254] (b = 0 is 2^-127, a subnormal).
__device__ __forceinline__ float ue8m0_value(uint32_t b) {
  return b == 0 ? 0x1p-127f : __uint_as_float(b << 23);
}

template <int kWidth>
__device__ __forceinline__ float reduce_max_xor(float v) {
#pragma unroll
  for (int off = kWidth / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWidth));
  return v;
}

template <int kWidth>
__device__ __forceinline__ float reduce_sum_xor(float v) {
#pragma unroll
  for (int off = kWidth / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWidth);
  return v;
}

// gfx950 has 8 XCDs; workgroups are dealt to them round-robin.  Renumber the
// grid so that each XCD walks one contiguous range of the logical tile order
// (neighbouring tiles share operand tiles in that XCD's L2).
__device__ __forceinline__ uint32_t xcd_chunked_tile(uint32_t bid, uint32_t grid) {
  constexpr uint32_t kXcd = 8;
  if (grid % kXcd) return bid;
  return (bid % kXcd) * (grid / kXcd) + bid / kXcd;
}

}  // namespace pih_amd
