// Elementwise kernels of the linear path for gfx950:
//   SwiGLU   out = bf16(silu(min(g,L)) * clamp(u,-L,L) * w[row]) — the
//            reference's expert/shared SwiGLU (plugins/kernels/deepseek-v4-
//            sm89/native/deepseek_expert_swiglu.cu:11-74) with L = 10; L <= 0
//            gives the plain SiLU-mul used by the BASELINE MoE chain.
//   SiLU-mul out = bf16((g / (1 + exp(-g))) * u), the Qwen MLP activation
//            (plugins/model-qwen3/qwen3_cpu_oracle.cpp:114-126).
//   MXFP4 decode  e2m1 nibble (low nibble = even k) * 2^(scale-127) -> bf16,
//            one UE8M0 scale per 32 values (reference
//            kernels/cuda/deepseek_mxfp4_decode.cu:13-73 and
//            plugins/model-deepseek-v4-flash/deepseek_mxfp4_codec.cpp:9-46).
//            Every e2m1 value times a power of two in [2^-127, 2^127] is a
//            bf16 number, so the decode is exact.
// All arithmetic is fp32 with no contraction (the build passes
// -ffp-contract=off), in the reference's operation order.
#include <algorithm>

#include "device_common.hpp"
#include "kernels.hpp"

namespace pih_amd {
namespace {

__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t* gate, const uint16_t* up,
                                                     const float* weights, uint16_t* out,
                                                     uint32_t* err, uint32_t rows, uint32_t cols,
                                                     float limit) {
  const uint64_t total = (uint64_t)rows * cols;
  uint32_t bad = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t row = (uint32_t)(i / cols);
    float g = bf16_bits_to_f32(gate[i]);
    float u = bf16_bits_to_f32(up[i]);
    const float w = weights ? weights[row] : 1.0f;
    if (!__builtin_isfinite(g) || !__builtin_isfinite(u) || !__builtin_isfinite(w) || w < 0.0f) {
      bad |= 1u;
      continue;
    }
    if (limit > 0.0f) {
      g = fminf(g, limit);
      u = fminf(fmaxf(u, -limit), limit);
    }
    float v = (g / (1.0f + expf(-g))) * u;
    if (weights) v = v * w;
    if (!__builtin_isfinite(v)) {
      bad |= 2u;
      continue;
    }
    out[i] = (uint16_t)f32_to_bf16_bits(v);
  }
  if (bad) atomicOr(err, bad);
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* gate, const uint16_t* up,
                                                       uint16_t* out, uint64_t count) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const float g = bf16_bits_to_f32(gate[i]);
    const float u = bf16_bits_to_f32(up[i]);
    out[i] = (uint16_t)f32_to_bf16_bits((g / (1.0f + expf(-g))) * u);
  }
}

__global__ __launch_bounds__(256) void mxfp4_decode_kernel(const uint8_t* packed,
                                                           const uint8_t* scales, uint16_t* out,
                                                           uint32_t* err, uint32_t rows,
                                                           uint32_t k) {
  const uint64_t pairs = (uint64_t)rows * (k / 2u);
  uint32_t bad = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < pairs;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t row = (uint32_t)(i / (k / 2u)), kp = (uint32_t)(i % (k / 2u));
    const uint32_t kk = 2u * kp;
    const uint8_t s = scales[(uint64_t)row * (k / 32u) + kk / 32u];
    if (s == 0xffu) {
      bad |= 2u;
      continue;
    }
    const uint8_t b = packed[i];
    const float sc = ue8m0_value(s);
    const float lo = e2m1_decode(b & 0xfu) * sc;
    const float hi = e2m1_decode(b >> 4) * sc;
    const uint32_t o = f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
    reinterpret_cast<uint32_t*>(out)[i] = o;
  }
  if (bad) atomicOr(err, bad);
}

uint32_t grid_for(uint64_t items) {
  uint64_t b = (items + 255) / 256;
  if (b == 0) b = 1;
  return (uint32_t)(b > 16384 ? 16384 : b);
}


// Scan of bf16 operands for a non-finite element, run only when `trigger`
// is already set in *err (so a clean call costs one flag read per block).
// Used for the DeepSeek LM head's bit 64 (deepseek_endpoint.cu:94-115 sets
// it when any x or W element it reads is non-finite): every logit reads its
// whole x row and W row, and a non-finite operand makes the dot non-finite,
// so the GEMM's non-finite-logit bit is set whenever bit 64 is due.
__global__ __launch_bounds__(256) void nonfinite_scan_kernel(const uint4* x, uint64_t nx, const uint4* w,
                                                             uint64_t nw, uint32_t* err, uint32_t trigger,
                                                             uint32_t bit) {
  if (!(__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & trigger)) return;
  const uint64_t total = nx + nw, stride = (uint64_t)gridDim.x * blockDim.x;
  uint32_t bad = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const uint4 v = i < nx ? x[i] : w[i - nx];
    const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      bad |= ((q[j] & 0x7f80u) == 0x7f80u) | ((q[j] & 0x7f800000u) == 0x7f800000u);
  }
  if (bad) atomicOr(err, bit);
}

// e4m3 NaN codes (0x7F / 0xFF bytes) anywhere in two byte buffers: the big
// tile FP8 path's test (16 bytes per load, the tails byte by byte).
__global__ __launch_bounds__(256) void nan_code_scan_kernel(const uint8_t* a, uint64_t na, const uint8_t* w,
                                                            uint64_t nw, uint32_t* err, uint32_t bit) {
  const uint64_t va = na / 16, vw = nw / 16, total = va + vw, stride = (uint64_t)gridDim.x * blockDim.x;
  const uint64_t t0 = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t bad = 0;
  for (uint64_t i = t0; i < total; i += stride) {
    const uint4 v = i < va ? reinterpret_cast<const uint4*>(a)[i] : reinterpret_cast<const uint4*>(w)[i - va];
    bad |= e4m3_nan_bytes(v.x) | e4m3_nan_bytes(v.y) | e4m3_nan_bytes(v.z) | e4m3_nan_bytes(v.w);
  }
  if (t0 < 16) {
    for (uint64_t i = va * 16 + t0; i < na; i += 16) bad |= e4m3_nan_bytes(a[i]);
    for (uint64_t i = vw * 16 + t0; i < nw; i += 16) bad |= e4m3_nan_bytes(w[i]);
  }
  if (bad) atomicOr(err, bit);
}

}  // namespace

St LaunchNanCodeScan(const NanCodeScanArgs& a) {
  if (!a.a || !a.w || !a.error_flag || !a.stream || !a.bit) return Invalid("nan_code_scan_null_argument");
  if ((reinterpret_cast<uintptr_t>(a.a) | reinterpret_cast<uintptr_t>(a.w)) % 16)
    return Invalid("nan_code_scan_alignment_invalid");
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  const uint64_t vec = (a.a_bytes + a.w_bytes) / 16;
  const uint32_t grid = (uint32_t)std::min<uint64_t>((vec + 255) / 256, 4096);
  hipLaunchKernelGGL(nan_code_scan_kernel, dim3(grid ? grid : 1), dim3(256), 0, a.stream,
                     static_cast<const uint8_t*>(a.a), a.a_bytes, static_cast<const uint8_t*>(a.w), a.w_bytes,
                     a.error_flag, a.bit);
  return AfterLaunch("nan_code_scan_launch_failed");
}

St LaunchSwiGlu(const SwiGluArgs& a) {
  if (!a.gate || !a.up || !a.out || !a.error_flag || !a.stream) return Invalid("swiglu_null_argument");
  if (a.rows == 0 || a.cols == 0) return Invalid("swiglu_shape_invalid");
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  hipLaunchKernelGGL(swiglu_kernel, dim3(grid_for((uint64_t)a.rows * a.cols)), dim3(256), 0,
                     a.stream, a.gate, a.up, a.weights, a.out, a.error_flag, a.rows, a.cols,
                     a.limit);
  return AfterLaunch("swiglu_launch_failed");
}

St LaunchSiluMul(const SiluMulArgs& a) {
  if (!a.gate || !a.up || !a.out || !a.stream) return Invalid("silu_mul_null_argument");
  if (a.count == 0) return Invalid("silu_mul_shape_invalid");
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(grid_for(a.count)), dim3(256), 0, a.stream, a.gate, a.up,
                     a.out, a.count);
  return AfterLaunch("silu_mul_launch_failed");
}

St LaunchMxfp4Decode(const Mxfp4DecodeArgs& a) {
  if (!a.packed || !a.scales || !a.out || !a.error_flag || !a.stream)
    return Invalid("mxfp4_decode_null_argument");
  if (a.rows == 0 || a.k == 0 || a.k % 32u) return Invalid("mxfp4_decode_shape_invalid");
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  hipLaunchKernelGGL(mxfp4_decode_kernel, dim3(grid_for((uint64_t)a.rows * a.k / 2u)), dim3(256), 0,
                     a.stream, a.packed, a.scales, a.out, a.error_flag, a.rows, a.k);
  return AfterLaunch("mxfp4_decode_launch_failed");
}

St LaunchNonfiniteScan(const NonfiniteScanArgs& a) {
  if (!a.x || !a.w || !a.error_flag || !a.stream) return Invalid("nonfinite_scan_null_argument");
  if (a.x_elems % 8 || a.w_elems % 8 || (reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.w)) % 16)
    return Invalid("nonfinite_scan_shape_invalid");
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  const uint64_t vec = (a.x_elems + a.w_elems) / 8;
  const uint32_t grid = (uint32_t)std::min<uint64_t>((vec + 255) / 256, 2048);
  hipLaunchKernelGGL(nonfinite_scan_kernel, dim3(grid ? grid : 1), dim3(256), 0, a.stream,
                     reinterpret_cast<const uint4*>(a.x), a.x_elems / 8, reinterpret_cast<const uint4*>(a.w),
                     a.w_elems / 8, a.error_flag, a.trigger_bit, a.set_bit);
  return AfterLaunch("nonfinite_scan_launch_failed");
}

}  // namespace pih_amd
