// FP8 activation quantizer entry for gfx950: bf16 rows (optionally gathered
// through a row index) -> e4m3fn codes plus one scale per (row, 128
// columns); the arithmetic is quant_groups (fp8_quant_device.hpp).
#include "fp8_quant_device.hpp"

namespace pih_amd {
namespace {

template <int FMT, bool GATHER>
__global__ __launch_bounds__(256) void fp8_quant_kernel(const uint16_t* __restrict__ in,
                                                        const uint32_t* __restrict__ rows,
                                                        uint8_t* __restrict__ codes,
                                                        void* __restrict__ scales, uint32_t* err,
                                                        uint32_t row_count, uint32_t k,
                                                        uint32_t input_rows) {
  const uint64_t seg0 = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4;
  const uint64_t seg_step = ((uint64_t)gridDim.x * blockDim.x) >> 4;
  const uint32_t bad = quant_groups<FMT, GATHER>(in, rows, codes, scales, row_count, k, input_rows, seg0, seg_step);
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
  const uint32_t blocks = QuantBlocks((uint64_t)a.row_count * (a.k / 128u));
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(256), 0, a.stream, a.input, a.rows, a.codes, a.scales,
                       a.error_flag, a.row_count, a.k, input_rows);
  };
  if (a.fmt == kScaleUe8m0) {
    if (a.rows) launch(fp8_quant_kernel<kScaleUe8m0, true>);
    else launch(fp8_quant_kernel<kScaleUe8m0, false>);
  } else {
    if (a.rows) launch(fp8_quant_kernel<kScaleF32, true>);
    else launch(fp8_quant_kernel<kScaleF32, false>);
  }
  return AfterLaunch("fp8_quant_launch_failed");
}

}  // namespace pih_amd
