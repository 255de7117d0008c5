// DeepSeek V4.1 32-block weight and activation formats for gfx950:
//
//   V41Quant32     bf16 [rows, K] -> e4m3 + one UE8M0 scale per (row, 32 k):
//                  the V4.1 linear's Quantize kernel
//                  (plugins/model-deepseek-v41/linear_fp8.cu:18-34): amax
//                  over the finite values of the group, floored at 1e-4,
//                  times the fp32 constant 1/448; the scale exponent is that
//                  product's exponent, rounded up unless it is a power of
//                  two; codes are the clamped x / 2^e rounded to nearest
//                  even.  Error bit 1 for a non-finite input (it encodes 0).
//   V41Fp4ToFp8    the expert FP4 -> FP8 32x32 conversion
//                  (weight_expert_convert.cpp:33-100): packed e2m1 [rows,
//                  cols/2] + UE8M0 [rows, cols/32] -> e4m3 [rows, cols] +
//                  one UE8M0 per 32x32 block [rows/32, cols/32].  Shared
//                  scale = max(row scale) - 6; each value e2m1 * 2^(row -
//                  shared) rounded to e4m3 with ties to even; both e2m1 zero
//                  codes give +0, other negatives keep the sign.  Error bit 1
//                  for a NaN (255) row scale, 2 for a shared scale below 0;
//                  such a block is not written.
//   V41BlockDequant  e4m3 [rows, cols] x one scale per square block of 32 or
//                  128 (UE8M0, 0 meaning 2^-127, or fp32) -> bf16, fp32
//                  product rounded to nearest even (weight_dequantize.cpp:
//                  17-50).  Error bits: 1 NaN code, 2 invalid scale, 4 a
//                  non-finite product or bf16; those elements are not
//                  written.
// The reference rejects a whole tensor on the first error; these kernels
// flag it and the caller discards the output (no partial result is valid).
#include "device_common.hpp"
#include "kernels.hpp"

namespace pih_amd {
namespace {

// one thread per element; the 32 lanes of a half-wave form one group
__global__ __launch_bounds__(256) void v41_quant32_kernel(const uint16_t* in, uint8_t* codes, uint8_t* scales,
                                                          uint32_t* err, uint64_t groups) {
  const uint32_t lane32 = threadIdx.x & 31u;
  uint32_t bad = 0;
  for (uint64_t g = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 5; g < groups;
       g += ((uint64_t)gridDim.x * blockDim.x) >> 5) {
    const uint64_t i = g * 32 + lane32;
    const float v = bf16_bits_to_f32(in[i]);
    const bool fin = __builtin_isfinite(v);
    if (!fin) bad = 1;
    const float amax = reduce_max_xor<32>(fin ? fabsf(v) : 0.0f);
    const float scaled = fmaxf(amax, 1.0e-4f) * (1.0f / 448.0f);
    const uint32_t bits = __float_as_uint(scaled);
    const int e = (int)((bits >> 23) & 255u) - 127 + ((bits & 0x7fffffu) != 0u);
    if (lane32 == 0) scales[g] = (uint8_t)(e + 127);
    // x / 2^e as a product with the exact power of two 2^-e (e in [-22, 121])
    const float q = fin ? fminf(fmaxf(v * exp2i(-e), -448.0f), 448.0f) : 0.0f;
    codes[i] = (uint8_t)e4m3_encode(q);
  }
  if (bad) atomicOr(err, 1u);
}

// one wave per 32x32 block: lane l converts row l/2, columns 16(l&1) .. +16
__global__ __launch_bounds__(64) void v41_fp4_to_fp8_kernel(const uint8_t* packed, const uint8_t* scales,
                                                            uint8_t* weight, uint8_t* out_scales, uint32_t* err,
                                                            uint32_t rows, uint32_t cols) {
  const uint32_t gb = cols / 32, blk = blockIdx.x;
  const uint32_t r0 = (blk / gb) * 32, g = blk % gb, lane = threadIdx.x;
  const uint32_t row = r0 + (lane >> 1), c0 = g * 32 + (lane & 1) * 16;
  const uint32_t s = scales[(uint64_t)row * (cols / 32) + g];
  const uint32_t smax = (uint32_t)reduce_max_xor<64>((float)s);
  const bool nan_scale = __any(s == 255u);
  if (nan_scale || smax < 6u) {
    if (lane == 0) atomicOr(err, nan_scale ? 1u : 2u);
    return;
  }
  const int shift = (int)s - (int)smax + 6;  // <= 6
  const uint2 w = *reinterpret_cast<const uint2*>(packed + (uint64_t)row * (cols / 2) + c0 / 2);
  uint32_t out[4] = {0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const uint32_t nib = ((j < 8 ? w.x : w.y) >> (4 * (j & 7))) & 15u;
    const uint32_t mag = nib & 7u;
    uint32_t code = 0;
    // below 2^-30 every e2m1 magnitude rounds to +-0 in e4m3 (half the
    // smallest subnormal is 2^-10)
    if (mag && shift >= -30) code = e4m3_encode(e2m1_decode(mag) * exp2i(shift));
    if ((nib & 8u) && mag) code |= 0x80u;
    out[j >> 2] |= code << (8 * (j & 3));
  }
  *reinterpret_cast<uint4*>(weight + (uint64_t)row * cols + c0) = uint4{out[0], out[1], out[2], out[3]};
  if (lane == 0) out_scales[(uint64_t)(r0 / 32) * gb + g] = (uint8_t)(smax - 6u);
}

// eight elements per thread (one 8-byte load; eight columns share a block)
template <bool F32_SCALE>
__global__ __launch_bounds__(256) void v41_dequant_kernel(const uint8_t* src, const void* scales, uint16_t* out,
                                                          uint32_t* err, uint32_t rows, uint32_t cols,
                                                          uint32_t block) {
  const uint64_t total = (uint64_t)rows * cols / 8;
  const uint32_t sc_cols = cols / block;
  uint32_t bad = 0;
  for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t e0 = t * 8;
    const uint32_t row = (uint32_t)(e0 / cols), col = (uint32_t)(e0 % cols);
    const uint64_t si = (uint64_t)(row / block) * sc_cols + col / block;
    float scale;
    bool scale_ok;
    if constexpr (F32_SCALE) {
      scale = static_cast<const float*>(scales)[si];
      scale_ok = __builtin_isfinite(scale) && scale > 0.0f;
    } else {
      const uint32_t b = static_cast<const uint8_t*>(scales)[si];
      scale = ue8m0_value(b);
      scale_ok = b != 255u;
    }
    if (!scale_ok) {
      bad |= 2u;
      continue;
    }
    const uint2 w = *reinterpret_cast<const uint2*>(src + e0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t code = ((j < 4 ? w.x : w.y) >> (8 * (j & 3))) & 0xffu;
      if ((code & 0x7fu) == 0x7fu) {
        bad |= 1u;
        continue;
      }
      const float v = e4m3_decode(code) * scale;
      const uint32_t h = f32_to_bf16_bits(v);
      if (!__builtin_isfinite(v) || (h & 0x7f80u) == 0x7f80u) {
        bad |= 4u;
        continue;
      }
      out[e0 + j] = (uint16_t)h;
    }
  }
  if (bad) atomicOr(err, bad);
}

uint32_t grid_for(uint64_t work, uint32_t per_block) {
  const uint64_t g = (work + per_block - 1) / per_block;
  return (uint32_t)(g < 1 ? 1 : g > 16384 ? 16384 : g);
}

}  // namespace

St LaunchV41Quant32(const V41Quant32Args& a) {
  if (!a.input || !a.codes || !a.scales || !a.error_flag || !a.stream) return Invalid("v41_quant_null_argument");
  if (a.rows == 0 || a.k == 0 || a.k % 32) return Invalid("v41_quant_shape_invalid");
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  const uint64_t groups = (uint64_t)a.rows * (a.k / 32);
  hipLaunchKernelGGL(v41_quant32_kernel, dim3(grid_for(groups, 8)), dim3(256), 0, a.stream, a.input, a.codes,
                     a.scales, a.error_flag, groups);
  return AfterLaunch("v41_quant_launch_failed");
}

St LaunchV41Fp4ToFp8(const V41Fp4ToFp8Args& a) {
  if (!a.packed || !a.scales || !a.weight || !a.weight_scales || !a.error_flag || !a.stream)
    return Invalid("v41_fp4_to_fp8_null_argument");
  if (a.rows == 0 || a.cols == 0 || a.rows % 32 || a.cols % 32) return Invalid("v41_fp4_to_fp8_shape_invalid");
  const uint64_t blocks = (uint64_t)(a.rows / 32) * (a.cols / 32);
  if (blocks > 0x7fffffffull) return Invalid("v41_fp4_to_fp8_shape_invalid");
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  hipLaunchKernelGGL(v41_fp4_to_fp8_kernel, dim3((uint32_t)blocks), dim3(64), 0, a.stream, a.packed, a.scales,
                     a.weight, a.weight_scales, a.error_flag, a.rows, a.cols);
  return AfterLaunch("v41_fp4_to_fp8_launch_failed");
}

St LaunchV41BlockDequant(const V41BlockDequantArgs& a) {
  if (!a.source || !a.scales || !a.output || !a.error_flag || !a.stream) return Invalid("v41_dequant_null_argument");
  if ((a.block != 32 && a.block != 128) || a.rows == 0 || a.cols == 0 || a.rows % a.block || a.cols % a.block)
    return Invalid("v41_dequant_shape_invalid");
  if (a.scale_f32 > 1) return Invalid("v41_dequant_scale_storage_invalid");
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  const uint32_t grid = grid_for((uint64_t)a.rows * a.cols / 8, 256);
  if (a.scale_f32)
    hipLaunchKernelGGL(v41_dequant_kernel<true>, dim3(grid), dim3(256), 0, a.stream, a.source, a.scales, a.output,
                       a.error_flag, a.rows, a.cols, a.block);
  else
    hipLaunchKernelGGL(v41_dequant_kernel<false>, dim3(grid), dim3(256), 0, a.stream, a.source, a.scales, a.output,
                       a.error_flag, a.rows, a.cols, a.block);
  return AfterLaunch("v41_dequant_launch_failed");
}

}  // namespace pih_amd
