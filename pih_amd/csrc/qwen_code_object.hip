// The gfx950 Qwen code object (qwen3-gfx950/gfx950/qwen_bf16_primitives.hsaco):
// kernels the Qwen model plugin loads by name and launches itself with a
// packed kernel-argument buffer, replacing the sm_89/sm_90 cubin of
// kernels/cuda/qwen_bf16_primitives.cu for this hot path.  Symbol names,
// parameter order, kernarg offsets, launch geometry, error codes and error
// publication follow that file:
//
//   pih_qwen_w4a16_gemm_compat_v1(input@0, packed_weight@8, scales@16,
//       output@24, error_flag@32, m@40, n@48, k@56)          64-byte kernarg
//     (qwen_bf16_primitives.cu:98-149, plan qwen3_int4_gemm_plan.cpp:73-85)
//     y[m, n] = bf16(sum_k x[m, k] * q[n, k] * s[n, k/128]); q is the signed
//     nibble (low nibble = even k) of packed [N][K/2]; nibble 0x8 is
//     reserved; s is an fp16 scale per (n, 128 k).  The launch is
//     ceil(m*n/256) blocks of 256 threads; anything else, a null pointer,
//     m = 0 or m > 4096 publishes error 11.  Errors are first-wins CAS of
//     11 (launch), 12 (reserved nibble), 13 (scale not finite and > 0),
//     14 (non-finite output); an element with an error is not written.
//     The reference accepts only the five Qwen3-0.6B (n, k) pairs; this
//     kernel also accepts any n % 256 == 0 and k % 128 == 0 (Qwen3-8B).
//
//   pih_qwen_silu_mul_bf16_v1(gate@0, up@8, output@16, elements@24)
//     (qwen_bf16_primitives.cu:274-283): out = bf16(silu(g) * u), any grid.
//
// W4A16 decomposition: every output of a block lies in one x row (n is a
// multiple of 256), so block b computes 256 consecutive W rows for row
// m = 256 b / n.  Wave w streams rows 64w .. 64w+63 of those; for each
// 1024-deep K chunk lane l owns k [16l, 16l+16) (8 packed bytes: a wave
// reads one 512-byte row segment per load) and keeps one fp32 partial per
// row; a transpose-reduction over the 64 lanes then leaves row r's total in
// lane r.  The per-(row, 128 k) scale multiplies the lane's integer-weight
// dot product (the sum order differs from the reference's strict k order;
// results agree to fp32 rounding).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr uint32_t kErrLaunch = 11, kErrReservedNibble = 12, kErrScale = 13, kErrNonFinite = 14;

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16(float v) {
  const uint32_t raw = __float_as_uint(v);
  if ((raw & 0x7fffffffu) > 0x7f800000u) return (raw >> 16) | 0x0040u;
  return (raw + 0x7fffu + ((raw >> 16) & 1u)) >> 16;
}

// IEEE binary16 -> fp32 (all classes)
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
  if (e == 0x1fu) return __uint_as_float(sign | 0x7f800000u | (mant << 13));
  if (e == 0) return mant ? __uint_as_float(sign) + (sign ? -1.0f : 1.0f) * (float)mant * 0x1p-24f
                          : __uint_as_float(sign);
  return __uint_as_float(sign | ((e + 112u) << 23) | (mant << 13));
}

__device__ __forceinline__ void publish(uint32_t* flag, uint32_t code) {
  if (flag) atomicCAS(flag, 0u, code);
}

// non-zero when a nibble of w equals 8
__device__ __forceinline__ uint32_t reserved_nibbles(uint32_t w) {
  const uint32_t t = w ^ 0x88888888u;
  return (t - 0x11111111u) & ~t & 0x88888888u;
}

// sum over the 8 signed nibbles of w (low nibble first) times x[0..7]
__device__ __forceinline__ float dot8(uint32_t w, const float* x) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int32_t q = (int32_t)((w >> (4 * j)) & 0xfu);
    s = __builtin_fmaf(x[j], (float)(q < 8 ? q : q - 16), s);
  }
  return s;
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void pih_qwen_w4a16_gemm_compat_v1(
    const uint16_t* input, const uint8_t* packed_weight, const uint16_t* scales, uint16_t* output,
    uint32_t* error_flag, uint64_t m, uint64_t n, uint64_t k) {
  const uint64_t elements = m * n;
  const uint64_t expected_blocks = (elements + 255u) / 256u;
  if (error_flag == nullptr || input == nullptr || packed_weight == nullptr || scales == nullptr ||
      output == nullptr || m == 0 || m > 4096 || n == 0 || (n & 255u) != 0 || k == 0 || (k & 127u) != 0 ||
      blockDim.x != 256 || gridDim.x != expected_blocks) {
    if (threadIdx.x == 0) publish(error_flag, kErrLaunch);
    return;
  }
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint64_t first = (uint64_t)blockIdx.x * 256u;
  const uint64_t row = first / n;
  const uint64_t n0 = first - row * n + wave * 64u;  // this wave's first W row
  const uint64_t kb = k / 2u, kgroups = k / 128u;
  const uint16_t* x = input + row * k;

  float part[64];
#pragma unroll
  for (int r = 0; r < 64; ++r) part[r] = 0.0f;
  uint64_t bad_nib = 0, bad_scale = 0;  // per-row flags of this lane's k slices

  for (uint64_t c = 0; c < k; c += 1024u) {
    const uint64_t k0 = c + lane * 16u;  // this lane's 16 k of the chunk
    if (k0 >= k) continue;               // a last chunk shorter than 1024
    float xv[16];
    const uint4 x01 = *reinterpret_cast<const uint4*>(x + k0);
    const uint4 x23 = *reinterpret_cast<const uint4*>(x + k0 + 8);
    const uint32_t xw[8] = {x01.x, x01.y, x01.z, x01.w, x23.x, x23.y, x23.z, x23.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      xv[2 * j] = bf16_to_f32(xw[j] & 0xffffu);
      xv[2 * j + 1] = bf16_to_f32(xw[j] >> 16);
    }
    const uint64_t g = k0 / 128u;
#pragma unroll
    for (int r = 0; r < 64; ++r) {
      const uint64_t wr = n0 + r;
      const uint2 w = *reinterpret_cast<const uint2*>(packed_weight + wr * kb + k0 / 2u);
      const float s = f16_to_f32(scales[wr * kgroups + g]);
      if (reserved_nibbles(w.x) | reserved_nibbles(w.y)) bad_nib |= 1ull << r;
      if (!(s > 0.0f) || !__builtin_isfinite(s)) bad_scale |= 1ull << r;
      part[r] = __builtin_fmaf(s, dot8(w.x, xv) + dot8(w.y, xv + 8), part[r]);
    }
  }

  // transpose-reduce: after the stage with distance d, lane l keeps the
  // rows whose bit log2(d) equals lane bit log2(d); lane r ends with row r
#pragma unroll
  for (int d = 32, half = 32; d >= 1; d >>= 1, half >>= 1) {
    const bool hi = (lane & (uint32_t)d) != 0;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      const float send = hi ? part[i] : part[i + half];
      const float keep = hi ? part[i + half] : part[i];
      part[i] = keep + __shfl_xor(send, d, 64);
    }
  }
  // row flags: OR over the lanes (every lane covers a slice of every row)
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    bad_nib |= ((uint64_t)__shfl_xor((uint32_t)(bad_nib >> 32), d, 64) << 32) | __shfl_xor((uint32_t)bad_nib, d, 64);
    bad_scale |=
        ((uint64_t)__shfl_xor((uint32_t)(bad_scale >> 32), d, 64) << 32) | __shfl_xor((uint32_t)bad_scale, d, 64);
  }
  // an element with a failure is not written (the reference returns at its
  // first failing k; a reserved nibble is reported before a bad scale)
  if ((bad_nib >> lane) & 1u) {
    publish(error_flag, kErrReservedNibble);
    return;
  }
  if ((bad_scale >> lane) & 1u) {
    publish(error_flag, kErrScale);
    return;
  }
  const float y = part[0];
  if (!__builtin_isfinite(y)) {
    publish(error_flag, kErrNonFinite);
    return;
  }
  output[row * n + n0 + lane] = (uint16_t)f32_to_bf16(y);
}

extern "C" __global__ __launch_bounds__(256) void pih_qwen_silu_mul_bf16_v1(const uint16_t* gate, const uint16_t* up,
                                                                          uint16_t* output, uint64_t elements) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < elements; i += stride) {
    const float g = bf16_to_f32(gate[i]);
    const float silu = g / (1.0f + expf(-g));
    output[i] = (uint16_t)f32_to_bf16(silu * bf16_to_f32(up[i]));
  }
}
