// FP8 activation quantizer for gfx950: bf16 rows -> e4m3fn codes plus one
// scale per (row, 128 columns).
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
// fp32 form: s = max(amax,1e-4)/448, codes = e4m3(clamp(x/s, +-448)).
//
// One 16-lane segment owns one 128-column group (8 bf16 per lane, one
// 16-byte load), so a wave quantizes four groups per step and the amax
// reduction is four xor-shuffles.
#include "device_common.hpp"
#include "kernels.hpp"

namespace pih_amd {
namespace {

template <int FMT>
__global__ __launch_bounds__(256) void fp8_quant_kernel(const uint16_t* __restrict__ in,
                                                        const uint32_t* __restrict__ rows,
                                                        uint8_t* __restrict__ codes,
                                                        void* __restrict__ scales, uint32_t* err,
                                                        uint32_t row_count, uint32_t k,
                                                        uint32_t input_rows) {
  const uint32_t gpr = k / 128u;
  const uint64_t groups = (uint64_t)row_count * gpr;
  const uint32_t sub = threadIdx.x & 15u;
  const uint64_t seg0 = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4;
  const uint64_t seg_step = ((uint64_t)gridDim.x * blockDim.x) >> 4;
  uint32_t bad = 0;
  for (uint64_t gi = seg0; gi < groups; gi += seg_step) {
    const uint32_t row = (uint32_t)(gi / gpr), kg = (uint32_t)(gi % gpr);
    uint32_t src = rows ? rows[row] : row;
    bool ok = src < input_rows;
    if (!ok) bad |= kErrCode;
    uint4 x = make_uint4(0, 0, 0, 0);
    if (ok) x = *reinterpret_cast<const uint4*>(in + (uint64_t)src * k + kg * 128u + sub * 8u);
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
    float v[8];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16_bits_to_f32(w[i] & 0xffffu);
      v[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (__builtin_isfinite(v[i])) {
        amax = fmaxf(amax, fabsf(v[i]));
      } else {
        bad |= kErrCode;
        v[i] = 0.0f;
      }
    }
    amax = reduce_max_xor<16>(amax);
    amax = fmaxf(amax, 1.0e-4f);
    float scale;
    if constexpr (FMT == kScaleUe8m0) {
      int e = ue8m0_exponent(amax);
      if (e < -127 || e > 127) {
        bad |= kErrScale;
        e = 0;
      }
      scale = ldexpf(1.0f, e);
      if (sub == 0) static_cast<uint8_t*>(scales)[gi] = (uint8_t)(e + 127);
    } else {
      scale = amax / 448.0f;
      if (sub == 0) static_cast<float*>(scales)[gi] = scale;
    }
    const uint32_t packed[2] = {e4m3_quant4(v, scale), e4m3_quant4(v + 4, scale)};
    *reinterpret_cast<uint2*>(codes + (uint64_t)row * k + kg * 128u + sub * 8u) =
        make_uint2(packed[0], packed[1]);
  }
  if (bad) atomicOr(err, bad);
}

}  // namespace

St LaunchFp8Quant(const Fp8QuantArgs& a) {
  if (!a.input || !a.codes || !a.scales || !a.error_flag || !a.stream)
    return Invalid("fp8_quant_null_argument");
  if (a.row_count == 0 || a.k == 0 || a.k % 128u) return Invalid("fp8_quant_shape_invalid");
  if (a.fmt != kScaleF32 && a.fmt != kScaleUe8m0) return Invalid("fp8_quant_scale_format_invalid");
  const uint32_t input_rows = a.rows ? a.input_rows : a.row_count;
  if (input_rows == 0) return Invalid("fp8_quant_input_rows_invalid");
  const uint64_t groups = (uint64_t)a.row_count * (a.k / 128u);
  uint64_t blocks = (groups * 16 + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  if (a.fmt == kScaleUe8m0) {
    hipLaunchKernelGGL(fp8_quant_kernel<kScaleUe8m0>, dim3((uint32_t)blocks), dim3(256), 0, a.stream,
                       a.input, a.rows, a.codes, a.scales, a.error_flag, a.row_count, a.k,
                       input_rows);
  } else {
    hipLaunchKernelGGL(fp8_quant_kernel<kScaleF32>, dim3((uint32_t)blocks), dim3(256), 0, a.stream,
                       a.input, a.rows, a.codes, a.scales, a.error_flag, a.row_count, a.k,
                       input_rows);
  }
  return AfterLaunch("fp8_quant_launch_failed");
}

}  // namespace pih_amd
