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
// W4A16 on the matrix cores, inside the model's launch geometry (ceil(m*n /
// 256) blocks of 256 threads; which 256 outputs a block computes is the
// kernel's choice as long as every output is computed once):
//   * m a multiple of 16: block b computes a 16 x 16 output tile (x rows
//     16 (b / (n/16)) .., W rows 16 (b % (n/16)) ..), its 4 waves splitting
//     K, so each W row is read by m/16 blocks instead of m;
//   * otherwise (decode): block b computes 256 W rows of x row 256 b / n,
//     64 per wave, every wave walking all of K.
// Per 128-deep group: a lane loads 16 bytes of its W row (32 nibbles, k
// [32lg, 32lg+32) of the group) and the 32 matching x values; MFMA j of the
// four 16x16x32 bf16 MFMAs takes k [32lg + 8j, +8) from every lane (the
// order of k inside one MFMA does not matter as long as both operands use
// it).  Nibbles become the bf16 values 128 + u (u = q + 8, two masks and
// four v_perm per word, x permuted to the same order), so the MFMA sums
// x (128 + u) and the group's result is s (sum - 136 sum_k x) with the
// fp16 scale s of (W row, group).  The sum order differs from the
// reference's strict k order; results agree to fp32 rounding.
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

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// 8 nibbles of a word (k offsets 0..7, low first), each the signed q with
// 8 subtracted away: u = q + 8 as the bf16 value 128 + u, in the order
// k = 0, 2, 4, 6, 1, 3, 5, 7 (two masks and four v_perm under the 0x43
// exponent byte of 128)
__device__ __forceinline__ v4i nibbles_to_bf16(uint32_t w) {
  const uint32_t t = w ^ 0x88888888u;  // two's complement nibble -> q + 8
  const uint32_t lo = t & 0x0F0F0F0Fu, hi = (t >> 4) & 0x0F0F0F0Fu;
  constexpr uint32_t kExp = 0x43434343u;
  return v4i{(int)__builtin_amdgcn_perm(kExp, lo, 0x04010400u), (int)__builtin_amdgcn_perm(kExp, lo, 0x04030402u),
             (int)__builtin_amdgcn_perm(kExp, hi, 0x04010400u), (int)__builtin_amdgcn_perm(kExp, hi, 0x04030402u)};
}

// eight bf16 x values (k = 0..7) into the order nibbles_to_bf16 produces
__device__ __forceinline__ v4i x_in_nibble_order(v4i v) {
  const uint32_t w0 = (uint32_t)v[0], w1 = (uint32_t)v[1], w2 = (uint32_t)v[2], w3 = (uint32_t)v[3];
  return v4i{(int)__builtin_amdgcn_perm(w1, w0, 0x05040100u), (int)__builtin_amdgcn_perm(w3, w2, 0x05040100u),
             (int)__builtin_amdgcn_perm(w1, w0, 0x07060302u), (int)__builtin_amdgcn_perm(w3, w2, 0x07060302u)};
}

__device__ __forceinline__ float sum8(v4i v) {
  float s = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q) s += bf16_to_f32((uint32_t)v[q] & 0xffffu) + bf16_to_f32((uint32_t)v[q] >> 16);
  return s;
}

// One 128-deep group of one 16-row W block against 16 x rows (A operand
// rows): w = the lane's 16 packed bytes (W row lr, k [32lg, 32lg+32) of the
// group), x = its 32 x values in four 8-value pieces (x row lr of the A
// operand), xs_t = the group's sum of x over the 128 k for A row 4lg + t.
// Adds s * (sum x (128+u) - 136 sum x) to acc[t] and flags the W row's
// reserved nibbles and bad scale.
__device__ __forceinline__ void group_mma(v4i w, const v4i (&x)[4], v4f xs, float s, v4f& acc, uint32_t& bad_nib,
                                          uint32_t& bad_scale) {
  v4f pq = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (reserved_nibbles((uint32_t)w[j])) bad_nib = 1;
    pq = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, x_in_nibble_order(x[j])),
                                                 __builtin_bit_cast(v8bf, nibbles_to_bf16((uint32_t)w[j])), pq, 0, 0,
                                                 0);
  }
  if (!(s > 0.0f) || !__builtin_isfinite(s)) bad_scale = 1;
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = __builtin_fmaf(s, __builtin_fmaf(-136.0f, xs[t], pq[t]), acc[t]);
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
  const uint32_t lr = lane & 15, lg = lane >> 4;
  const uint64_t kb = k / 2u, groups = k / 128u;

  if (m % 16u == 0) {
    // ---- 16 x 16 output tiles, the 4 waves splitting the K groups
    __shared__ float s_acc[4][4][64];
    __shared__ uint32_t s_bad[4][16];
    const uint64_t ctiles = n / 16u;
    const uint64_t xr0 = (blockIdx.x / ctiles) * 16u, wr0 = (blockIdx.x % ctiles) * 16u;
    const uint16_t* xrow = input + (xr0 + lr) * k + lg * 32u;
    const uint8_t* wrow = packed_weight + (wr0 + lr) * kb + lg * 16u;
    const uint16_t* srow = scales + (wr0 + lr) * groups;
    const uint64_t g0 = wave * groups / 4u, g1 = (wave + 1) * groups / 4u;
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
    uint32_t bad_nib = 0, bad_scale = 0;
    for (uint64_t g = g0; g < g1; ++g) {
      const v4i w = *reinterpret_cast<const v4i*>(wrow + g * 64u);
      v4i x[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = *reinterpret_cast<const v4i*>(xrow + g * 128u + j * 8u);
      const float s = f16_to_f32(srow[g]);
      // the group's x sum of A row lr, then of the rows 4lg + t this lane
      // holds results for
      float part = sum8(x[0]) + sum8(x[1]) + sum8(x[2]) + sum8(x[3]);
      part += __shfl_xor(part, 16, 64);
      part += __shfl_xor(part, 32, 64);
      v4f xs;
#pragma unroll
      for (int t = 0; t < 4; ++t) xs[t] = __shfl(part, (int)(4u * lg + t), 64);
      group_mma(w, x, xs, s, acc, bad_nib, bad_scale);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) s_acc[wave][t][lane] = acc[t];
    // per W row (column lr): OR over the lanes and waves that saw it
    const uint32_t flags = (bad_nib ? 1u : 0u) | (bad_scale ? 2u : 0u);
    if (lg == 0) s_bad[wave][lr] = 0;
    __syncthreads();
    if (flags) atomicOr(&s_bad[wave][lr], flags);
    __syncthreads();
    if (wave == 0) {
      const uint32_t rf = s_bad[0][lr] | s_bad[1][lr] | s_bad[2][lr] | s_bad[3][lr];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float y = s_acc[0][t][lane] + s_acc[1][t][lane] + s_acc[2][t][lane] + s_acc[3][t][lane];
        uint32_t code = 0;
        if (rf & 1u) code = kErrReservedNibble;
        else if (rf & 2u) code = kErrScale;
        else if (!__builtin_isfinite(y)) code = kErrNonFinite;
        if (code) {
          publish(error_flag, code);
          continue;
        }
        output[(xr0 + 4u * lg + t) * n + wr0 + lr] = (uint16_t)f32_to_bf16(y);
      }
    }
    return;
  }

  // ---- decode: 256 W rows of one x row, 64 per wave, all of K per wave
  const uint64_t first = (uint64_t)blockIdx.x * 256u;
  const uint64_t row = first / n;
  const uint64_t n0 = first - row * n + wave * 64u;  // this wave's first W row
  const uint16_t* xrow = input + row * k + lg * 32u;
  v4f acc[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) acc[b] = v4f{0.f, 0.f, 0.f, 0.f};
  uint32_t bad_nib[4] = {0, 0, 0, 0}, bad_scale[4] = {0, 0, 0, 0};
  // next group's operands load while this one computes
  v4i wn[4], xn[4];
  uint32_t sn[4];
  auto load = [&](uint64_t g) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint64_t wr = n0 + 16u * b + lr;
      wn[b] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(packed_weight + wr * kb + g * 64u + lg * 16u));
      sn[b] = scales[wr * groups + g];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) xn[j] = *reinterpret_cast<const v4i*>(xrow + g * 128u + j * 8u);
  };
  load(0);
  for (uint64_t g = 0; g < groups; ++g) {
    v4i w[4], x[4];
    uint32_t sc[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) w[b] = wn[b], sc[b] = sn[b];
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = xn[j];
    if (g + 1 < groups) load(g + 1);
    // every A row is this x row: the group's x sum is one value
    float part = sum8(x[0]) + sum8(x[1]) + sum8(x[2]) + sum8(x[3]);
    part += __shfl_xor(part, 16, 64);
    part += __shfl_xor(part, 32, 64);
    const v4f xs = v4f{part, part, part, part};
#pragma unroll
    for (int b = 0; b < 4; ++b) group_mma(w[b], x, xs, f16_to_f32(sc[b]), acc[b], bad_nib[b], bad_scale[b]);
  }
  // lane (lr, lg) holds W row n0 + 16b + lr in all four rows t (one x row);
  // the row's flags are the OR over the four lanes lg of that row
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    uint32_t f = (bad_nib[b] ? 1u : 0u) | (bad_scale[b] ? 2u : 0u);
    f |= __shfl_xor(f, 16, 64);
    f |= __shfl_xor(f, 32, 64);
    if (lg != 0) continue;
    const float y = acc[b][0];
    uint32_t code = 0;
    if (f & 1u) code = kErrReservedNibble;
    else if (f & 2u) code = kErrScale;
    else if (!__builtin_isfinite(y)) code = kErrNonFinite;
    if (code) {
      publish(error_flag, code);
      continue;
    }
    output[row * n + n0 + 16u * b + lr] = (uint16_t)f32_to_bf16(y);
  }
}

// pih_qwen_w4a16_gemm_gfx950_v1: the same operation, packet and error codes
// in the launch geometry the gfx950 plan chooses (pih_qwen_int4_gemm_plan_
// create_v1, replacing qwen3_int4_gemm_plan.cpp:44-63 at the model's call
// site): grid (n / 16, ceil(m / 16)), 64 * waves threads (1..16 waves).
// Block (bx, by) computes x rows 16 by .. 16 by + 15 (rows past m read row
// m - 1 and are not stored) against W rows 16 bx .. 16 bx + 15; wave w
// takes the 128-deep groups [w G / waves, (w + 1) G / waves) with its next
// group's loads in flight, and the waves' partial tiles meet in LDS in wave
// order.  n % 16, k % 128, m <= 4096 and the geometry are checked; a
// mismatch publishes 11.
extern "C" __global__ __launch_bounds__(1024) void pih_qwen_w4a16_gemm_gfx950_v1(
    const uint16_t* input, const uint8_t* packed_weight, const uint16_t* scales, uint16_t* output,
    uint32_t* error_flag, uint64_t m, uint64_t n, uint64_t k) {
  const uint32_t waves = blockDim.x / 64u;
  if (error_flag == nullptr || input == nullptr || packed_weight == nullptr || scales == nullptr ||
      output == nullptr || m == 0 || m > 4096 || n == 0 || (n & 15u) != 0 || k == 0 || (k & 127u) != 0 ||
      blockDim.x % 64u != 0 || waves == 0 || waves > 16 || blockDim.y != 1 || blockDim.z != 1 ||
      gridDim.x != n / 16u || gridDim.y != (m + 15u) / 16u || gridDim.z != 1) {
    if (threadIdx.x == 0 && blockIdx.x == 0 && blockIdx.y == 0) publish(error_flag, kErrLaunch);
    return;
  }
  __shared__ float s_acc[16][4][64];
  __shared__ uint32_t s_bad[16][16];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t lr = lane & 15, lg = lane >> 4;
  const uint64_t kb = k / 2u, groups = k / 128u;
  const uint64_t xr0 = (uint64_t)blockIdx.y * 16u, wr0 = (uint64_t)blockIdx.x * 16u;
  const uint64_t xrow_i = xr0 + lr < m ? xr0 + lr : m - 1;
  const uint16_t* xrow = input + xrow_i * k + lg * 32u;
  const uint8_t* wrow = packed_weight + (wr0 + lr) * kb + lg * 16u;
  const uint16_t* srow = scales + (wr0 + lr) * groups;
  const uint64_t g0 = wave * groups / waves, g1 = (wave + 1) * groups / waves;
  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
  uint32_t bad_nib = 0, bad_scale = 0;
  // two groups of loads in flight (a decode wave has one or two groups)
  const v4i z4 = v4i{0, 0, 0, 0};
  v4i wn[2] = {z4, z4}, xn[2][4] = {{z4, z4, z4, z4}, {z4, z4, z4, z4}};
  uint32_t sn[2] = {0, 0};
  auto load = [&](int b, uint64_t g) {
    wn[b] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wrow + g * 64u));
#pragma unroll
    for (int j = 0; j < 4; ++j) xn[b][j] = *reinterpret_cast<const v4i*>(xrow + g * 128u + j * 8u);
    sn[b] = srow[g];
  };
  if (g0 < g1) load(0, g0);
  if (g0 + 1 < g1) load(1, g0 + 1);
  for (uint64_t g = g0; g < g1; ++g) {
    const int b = (int)((g - g0) & 1u);
    const v4i w = b ? wn[1] : wn[0];
    v4i x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = b ? xn[1][j] : xn[0][j];
    const float s = f16_to_f32(b ? sn[1] : sn[0]);
    if (g + 2 < g1) {
      if (b) load(1, g + 2);
      else load(0, g + 2);
    }
    // the group's x sum of A row lr, then of the rows 4lg + t this lane
    // holds results for
    float part = sum8(x[0]) + sum8(x[1]) + sum8(x[2]) + sum8(x[3]);
    part += __shfl_xor(part, 16, 64);
    part += __shfl_xor(part, 32, 64);
    v4f xs;
#pragma unroll
    for (int t = 0; t < 4; ++t) xs[t] = __shfl(part, (int)(4u * lg + t), 64);
    group_mma(w, x, xs, s, acc, bad_nib, bad_scale);
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) s_acc[wave][t][lane] = acc[t];
  const uint32_t flags = (bad_nib ? 1u : 0u) | (bad_scale ? 2u : 0u);
  if (lg == 0) s_bad[wave][lr] = 0;
  __syncthreads();
  if (flags) atomicOr(&s_bad[wave][lr], flags);
  __syncthreads();
  if (wave == 0) {
    uint32_t rf = 0;
    for (uint32_t w = 0; w < waves; ++w) rf |= s_bad[w][lr];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint64_t row = xr0 + 4u * lg + t;
      float y = s_acc[0][t][lane];
      for (uint32_t w = 1; w < waves; ++w) y += s_acc[w][t][lane];
      if (row >= m) continue;
      uint32_t code = 0;
      if (rf & 1u) code = kErrReservedNibble;
      else if (rf & 2u) code = kErrScale;
      else if (!__builtin_isfinite(y)) code = kErrNonFinite;
      if (code) {
        publish(error_flag, code);
        continue;
      }
      output[row * n + wr0 + lr] = (uint16_t)f32_to_bf16(y);
    }
  }
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
