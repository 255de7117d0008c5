// Device body of the FP8 activation quantizer (bf16 rows -> e4m3fn codes +
// one scale per (row, 128 columns)), shared by the quant entry's kernel and
// the layer's fused route-mask + quant launch.
//
// UE8M0 form follows the reference codec
// (plugins/model-deepseek-v4-flash/deepseek_fp8_activation_codec.cpp:53-107)
// and kernel (plugins/kernels/deepseek-v4-sm89/native/
// deepseek_fp8_activation_quant.cu:12-60): amax floored at 1e-4, scale
// exponent e = ceil(log2(amax/448)) found exactly as the least integer with
// amax <= 448*2^e, scale byte e+127, codes = e4m3(clamp(x/2^e, +-448)) with
// round-to-nearest-even.  A non-finite input sets bit 1 and counts as zero
// magnitude (reference kernel behaviour); an exponent outside UE8M0 sets
// bit 2 and uses scale 1.
// fp32 form: s = max(amax,1e-4)/448, codes = e4m3(clamp(x/s, +-448)); x/s
// through e4m3_quant4_recip (same codes as the division for every input).
//
// One 16-lane segment owns one 128-column group (8 bf16 per lane, one
// 16-byte load), so the amax reduction is four xor-shuffles; a segment
// issues the loads of kQuantGroupsInFlight groups before it converts the
// first, so a wave keeps 4 KB of input in flight (one group per segment
// kept 1 KB and streamed at 3.1 TB/s on the cfg4 activations).
#pragma once
#include "device_common.hpp"
#include "kernels.hpp"

namespace pih_amd {

constexpr uint32_t kQuantGroupsInFlight = 4;

// Quantizes groups seg0, seg0 + seg_step, ... (< row_count * k / 128) for
// the 16-lane segment this thread belongs to (sub = lane & 15); returns the
// error bits it saw.
template <int FMT, bool GATHER>
__device__ __forceinline__ uint32_t quant_groups(const uint16_t* __restrict__ in, const uint32_t* __restrict__ rows,
                                                 uint8_t* __restrict__ codes, void* __restrict__ scales,
                                                 uint32_t row_count, uint32_t k, uint32_t input_rows, uint64_t seg0,
                                                 uint64_t seg_step) {
  constexpr uint32_t G = kQuantGroupsInFlight;
  const uint32_t gpr = k / 128u;
  const uint64_t groups = (uint64_t)row_count * gpr;
  const uint32_t sub = threadIdx.x & 15u;
  uint32_t bad = 0;
  for (uint64_t base = seg0; base < groups; base += seg_step * G) {
    uint4 x[G];
    uint32_t row[G], kg[G];
    bool live[G], ok[G];
    // loads first, unconditional (a load under a branch is waited for on
    // the spot): a group past the end reads the last group again and is
    // skipped below; a rejected gather index reads row 0 and counts as zeros
    uint32_t src[G];
#pragma unroll
    for (uint32_t i = 0; i < G; ++i) {
      const uint64_t gi = base + i * seg_step;
      live[i] = gi < groups;
      const uint64_t gc = live[i] ? gi : groups - 1;
      row[i] = (uint32_t)(gc / gpr);
      kg[i] = (uint32_t)(gc % gpr);
      src[i] = GATHER ? rows[row[i]] : row[i];
    }
#pragma unroll
    for (uint32_t i = 0; i < G; ++i) {
      ok[i] = src[i] < input_rows;
      if (live[i] && !ok[i]) bad |= kErrCode;
      x[i] = *reinterpret_cast<const uint4*>(in + (uint64_t)(ok[i] ? src[i] : 0u) * k + kg[i] * 128u + sub * 8u);
    }
#pragma unroll
    for (uint32_t i = 0; i < G; ++i) {
      if (!live[i]) continue;  // uniform across the segment
      const uint64_t gi = base + i * seg_step;
      const uint32_t w[4] = {ok[i] ? x[i].x : 0u, ok[i] ? x[i].y : 0u, ok[i] ? x[i].z : 0u, ok[i] ? x[i].w : 0u};
      float v[8];
      float amax = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = bf16_bits_to_f32(w[j] & 0xffffu);
        v[2 * j + 1] = bf16_bits_to_f32(w[j] >> 16);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (__builtin_isfinite(v[j])) {
          amax = fmaxf(amax, fabsf(v[j]));
        } else {
          bad |= kErrCode;
          v[j] = 0.0f;
        }
      }
      amax = reduce_max_xor<16>(amax);
      amax = fmaxf(amax, 1.0e-4f);
      float scale = 1.0f;
      int ue8m0_e = 0;
      if constexpr (FMT == kScaleUe8m0) {
        int e = ue8m0_exponent(amax);
        if (e < -127 || e > 127) {
          bad |= kErrScale;
          e = 0;
        }
        ue8m0_e = e;
        if (sub == 0) static_cast<uint8_t*>(scales)[gi] = (uint8_t)(e + 127);
      } else {
        scale = amax / 448.0f;
        if (sub == 0) static_cast<float*>(scales)[gi] = scale;
      }
      uint32_t packed[2];
      if constexpr (FMT == kScaleUe8m0) {
        // x / 2^e as the product with the exact power of two 2^-e: the same
        // correctly rounded value as the division, without its VALU cost
        const float inv = ldexpf(1.0f, -ue8m0_e);
        packed[0] = e4m3_quant4_mul(v, inv);
        packed[1] = e4m3_quant4_mul(v + 4, inv);
      } else {
        const float inv = 1.0f / scale;
        packed[0] = e4m3_quant4_recip(v, scale, inv);
        packed[1] = e4m3_quant4_recip(v + 4, scale, inv);
      }
      *reinterpret_cast<uint2*>(codes + (uint64_t)row[i] * k + kg[i] * 128u + sub * 8u) =
          make_uint2(packed[0], packed[1]);
    }
  }
  return bad;
}

// Blocks of 256 threads for `groups` groups: one segment per group and
// kQuantGroupsInFlight groups per segment, at most 16384 blocks.
inline uint32_t QuantBlocks(uint64_t groups) {
  uint64_t blocks = (groups * 16 + 256 * kQuantGroupsInFlight - 1) / (256 * kQuantGroupsInFlight);
  return (uint32_t)(blocks > 16384 ? 16384 : blocks < 1 ? 1 : blocks);
}

}  // namespace pih_amd
