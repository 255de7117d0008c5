// Small-M block-scaled GEMM for gfx950: FP8 (e4m3) or MXFP4 (e2m1) weights
// against e4m3 activations with m <= 64 rows, the decode-time form of the
// dense FP8 GEMM (reference plugins/kernels/deepseek-v4-sm89/native/
// deepseek_fp8_gemm.cu:11-107, oracle src/model/deepseek_fp8_gemm_oracle.cpp:
// 10-80), the per-expert FP4 GEMM (deepseek_fp4_gemm.cu:11-104, oracle
// src/model/deepseek_fp4_gemm_oracle.cpp:11-91) and the grouped FP8 GEMM
// (deepseek_attention_dense_primitives.cu:205-250).
//
// With a few activation rows the work is a weight stream, and the 128x128
// tiles of gemm_mfma.hip give such a call N/128 blocks (8 for N = 1024): a
// handful of CUs each walking all of K.  Here a block owns 16 weight rows
// and one chunk of up to 64 activation rows (grid z), and its waves split K
// into runs of at most SPW 128-deep steps, so N/16 blocks x chunks x up to
// 16 waves cover the GPU (a chunk past the first streams its weight rows
// again, mostly from L2 and MALL, as the blocks of one weight block run
// side by side):
//   * every load of a wave's batch of SPW steps (its W run, the activation
//     rows, the scales; one batch unless K is long for the wave count) is
//     issued before the batch's first wait: the W fragments in the MFMA operand
//     layout (FP8: lane (lr, lg) holds row lr, bytes [16lg, +16) and
//     [64 + 16lg, +16) of the step; FP4: bytes [16lg, +16) of the row's 64),
//     non-temporal;
//   * the MFMA is issued transposed (W block as the first operand), so a
//     lane's four results are four consecutive output columns of one
//     activation row; UE8M0 scales ride in the instruction's E8M0 operands
//     (FP4: one per lane, the 32-k block the lane holds) and the steps chain
//     on the accumulator; fp32 scales (FP8 only) add each step's product
//     with one FMA per output, as the tiled kernel does;
//   * the waves' partial sums meet in LDS in fixed wave order, so a result
//     does not depend on timing.
// Error bits (the caller's numbering): e4m3 NaN codes in W or A and
// activation rows out of range -> err_code, UE8M0 0xFF -> err_scale, a
// non-finite result -> err_nonfinite (the element is stored only when
// write_nonfinite is set, as the reference's grouped kernel does).
#include <algorithm>

#include "device_common.hpp"
#include "kernels.hpp"

namespace pih_amd {
namespace {

enum SmallWeight : int { kSmallFp8 = 0, kSmallFp4 = 1 };

__device__ __forceinline__ v8i cat8(v4i x, v4i y) { return v8i{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]}; }

struct SmallParams {
  const uint8_t* a;
  const void* a_scale;
  const uint8_t* w;
  const void* w_scale;
  void* out;
  uint32_t* err;
  uint32_t m, n, k, a_rows_total;
  uint32_t a_row_stride, a_prob_row;
  uint64_t out_row_stride;
  uint32_t out_prob_col;
  uint32_t check_codes, write_nonfinite, out_f32;
  uint32_t err_code, err_scale, err_nonfinite;
};

// BATCHED: a wave's run may be longer than SPW steps and is walked in
// batches of SPW; otherwise the host guarantees one batch.
template <int WF, int SCALE, int WAVES, int MT, int SPW, bool BATCHED>
__global__ __launch_bounds__(WAVES * 64) void small_m_gemm_kernel(SmallParams p) {
  extern __shared__ __align__(16) float red[];  // [WAVES][MT][4][64]
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t lr = lane & 15, lg = lane >> 4;
  const uint32_t prob = blockIdx.y, n0 = blockIdx.x * 16, rbase = blockIdx.z * kSmallMChunkRows;
  const uint32_t K = p.k, KB = K / 128;
  const uint32_t s0 = wave * KB / WAVES, s1 = (wave + 1) * KB / WAVES;  // runs differ by at most one step
  const uint32_t cnt = s1 - s0;
  uint32_t bad = 0;

  const uint32_t wrow = n0 + lr;
  const uint64_t wrow_g = (uint64_t)prob * p.n + wrow;
  const uint8_t* wp = p.w + wrow_g * (WF == kSmallFp8 ? K : K / 2) + lg * 16;
  uint64_t arow[MT];
#pragma unroll
  for (int c = 0; c < MT; ++c) {
    // rows past m read row m - 1: their sums are never stored
    const uint32_t i = min(rbase + 16u * c + lr, p.m - 1);
    uint64_t r = (uint64_t)i * p.a_row_stride + (uint64_t)prob * p.a_prob_row;
    if (r >= p.a_rows_total) {
      bad |= kErrCode;
      r = 0;
    }
    arow[c] = r;
  }

  const uint8_t* wsb = static_cast<const uint8_t*>(p.w_scale);
  const uint8_t* asb = static_cast<const uint8_t*>(p.a_scale);
  v4f acc[MT];
#pragma unroll
  for (int c = 0; c < MT; ++c) acc[c] = v4f{0.f, 0.f, 0.f, 0.f};
  // the run in batches of SPW steps
  const uint32_t nb = BATCHED ? cnt : min(cnt, (uint32_t)SPW);
  for (uint32_t b0 = 0; b0 < nb; b0 += SPW) {
    const uint32_t bn = min((uint32_t)SPW, cnt - b0);
    // ---- every load of the batch, before any wait (steps past the run
    // repeat its last step and are not computed)
    v4i wl[SPW][2];
    v4i al[SPW][MT][2];
    uint32_t sw[SPW], sa[SPW][MT];
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const uint32_t st = s0 + b0 + min((uint32_t)j, bn - 1);
      if constexpr (WF == kSmallFp8) {
        wl[j][0] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wp + (uint64_t)st * 128));
        wl[j][1] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wp + (uint64_t)st * 128 + 64));
      } else {
        wl[j][0] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wp + (uint64_t)st * 64));
      }
#pragma unroll
      for (int c = 0; c < MT; ++c) {
        const uint8_t* ap = p.a + arow[c] * K + (uint64_t)st * 128 + lg * 16;
        al[j][c][0] = *reinterpret_cast<const v4i*>(ap);
        al[j][c][1] = *reinterpret_cast<const v4i*>(ap + 64);
      }
      if constexpr (WF == kSmallFp8) {
        // one scale per (128 W rows, 128 k): the same for the block's 16 rows
        const uint64_t si = ((uint64_t)prob * (p.n / 128) + n0 / 128) * KB + st;
        sw[j] = SCALE == kScaleF32 ? reinterpret_cast<const uint32_t*>(wsb)[si] : wsb[si];
      } else {
        // one scale per (W row, 32 k): the block the lane's 32 values are in
        sw[j] = wsb[wrow_g * (K / 32) + st * 4 + lg];
      }
#pragma unroll
      for (int c = 0; c < MT; ++c) {
        const uint64_t si = arow[c] * KB + st;
        sa[j][c] = SCALE == kScaleF32 ? reinterpret_cast<const uint32_t*>(asb)[si] : asb[si];
      }
    }

#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      if ((uint32_t)j >= bn) break;  // wave-uniform
      if (p.check_codes) {
        // NaN codes count as 0 (and raise the code bit), as the reference
        // decodes them
        uint32_t nan = 0;
        auto clean = [&nan](v4i& v) __attribute__((always_inline)) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t nq = e4m3_nan_bytes((uint32_t)v[q]);
            v[q] = (int)e4m3_nan_to_zero((uint32_t)v[q], nq);
            nan |= nq;
          }
        };
        if constexpr (WF == kSmallFp8) {
          clean(wl[j][0]);
          clean(wl[j][1]);
        }
#pragma unroll
        for (int c = 0; c < MT; ++c) {
          clean(al[j][c][0]);
          clean(al[j][c][1]);
        }
        if (nan) bad |= kErrCode;
      }
      if constexpr (SCALE == kScaleUe8m0) {
        // a 0xFF scale raises the scale bit and its block adds nothing (the
        // reference skips the block): the operand bytes it scales become 0
        uint32_t ff = 0;
        if (sw[j] == 0xffu) {
          ff = 1;
          sw[j] = 127;
          wl[j][0] = v4i{0, 0, 0, 0};
          wl[j][1] = v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int c = 0; c < MT; ++c)
          if (sa[j][c] == 0xffu) {
            ff = 1;
            sa[j][c] = 127;
            al[j][c][0] = v4i{0, 0, 0, 0};
            al[j][c][1] = v4i{0, 0, 0, 0};
          }
        if (ff) bad |= kErrScale;
      }
      const v8i wop = WF == kSmallFp8 ? cat8(wl[j][0], wl[j][1]) : cat8(wl[j][0], v4i{0, 0, 0, 0});
      constexpr int kFmtW = WF == kSmallFp8 ? 0 : 4;
#pragma unroll
      for (int c = 0; c < MT; ++c) {
        const v8i aop = cat8(al[j][c][0], al[j][c][1]);
        if constexpr (SCALE == kScaleUe8m0) {
          acc[c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wop, aop, acc[c], kFmtW, 0, 0, (int)sw[j], 0,
                                                                    (int)sa[j][c]);
        } else {
          const v4f t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wop, aop, v4f{0.f, 0.f, 0.f, 0.f}, kFmtW, 0,
                                                                         0, 127, 0, 127);
          const float cf = __uint_as_float(sa[j][c]) * __uint_as_float(sw[j]);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[c][i] = __builtin_fmaf(t[i], cf, acc[c][i]);
        }
      }
    }
  }

  // ---- the waves' sums in wave order; lane (lr, lg) of column block c holds
  // out[16c + lr][n0 + 4lg + i]
#pragma unroll
  for (int c = 0; c < MT; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[((wave * MT + c) * 4 + i) * 64 + lane] = acc[c][i];
  __syncthreads();
  if (tid < 64u * MT) {
    const uint32_t c = tid / 64, l = tid % 64;
    const uint32_t row = rbase + 16 * c + (l & 15), col = n0 + 4 * (l >> 4);
    if (row < p.m) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) s += red[((w * MT + c) * 4 + i) * 64 + l];
        v[i] = s;
      }
      const bool fin = __builtin_isfinite(v[0]) && __builtin_isfinite(v[1]) && __builtin_isfinite(v[2]) &&
                       __builtin_isfinite(v[3]);
      if (!fin) bad |= kErrNonFinite;
      const uint64_t o = (uint64_t)row * p.out_row_stride + (uint64_t)prob * p.out_prob_col + col;
      if (p.out_f32) {
        float* dst = static_cast<float*>(p.out) + o;
        if (fin || p.write_nonfinite) *reinterpret_cast<v4f*>(dst) = v4f{v[0], v[1], v[2], v[3]};
        else
          for (int i = 0; i < 4; ++i)
            if (__builtin_isfinite(v[i])) dst[i] = v[i];
      } else {
        uint16_t* dst = static_cast<uint16_t*>(p.out) + o;
        if (fin || p.write_nonfinite)
          *reinterpret_cast<uint2*>(dst) = uint2{f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16),
                                                 f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16)};
        else
          for (int i = 0; i < 4; ++i)
            if (__builtin_isfinite(v[i])) dst[i] = (uint16_t)f32_to_bf16_bits(v[i]);
      }
    }
  }
  if (bad) {
    const uint32_t bits = ((bad & kErrCode) ? p.err_code : 0u) | ((bad & kErrScale) ? p.err_scale : 0u) |
                          ((bad & kErrNonFinite) ? p.err_nonfinite : 0u);
    if (bits) atomicOr(p.err, bits);
  }
}

template <int WF, int SCALE, int WAVES, int MT, int SPW, bool B>
void launch_cfg(const SmallParams& sp, uint32_t problems, hipStream_t s) {
  const size_t lds = (size_t)WAVES * MT * 4 * 64 * sizeof(float);
  const uint32_t chunks = (sp.m + kSmallMChunkRows - 1) / kSmallMChunkRows;
  hipLaunchKernelGGL((small_m_gemm_kernel<WF, SCALE, WAVES, MT, SPW, B>), dim3(sp.n / 16, problems, chunks),
                     dim3(WAVES * 64), lds, s, sp);
}

// MT 16-row activation blocks per chunk (m 33..48 runs as 4); SPW the
// batch: 2 or 4 steps with one activation block, 2 with more
template <int WF, int SCALE, int WAVES, bool B>
void launch_mt(const SmallParams& sp, uint32_t problems, uint32_t run, hipStream_t s) {
  const uint32_t mt = (std::min(sp.m, kSmallMChunkRows) + 15) / 16;
  if (mt == 1) {
    if (run <= 2) launch_cfg<WF, SCALE, WAVES, 1, 2, B>(sp, problems, s);
    else launch_cfg<WF, SCALE, WAVES, 1, 4, B>(sp, problems, s);
  } else if (mt == 2) {
    launch_cfg<WF, SCALE, WAVES, 2, 2, B>(sp, problems, s);
  } else {
    launch_cfg<WF, SCALE, WAVES, 4, 2, B>(sp, problems, s);
  }
}

// Waves per block: the fewest of 4, 8, 16 whose runs are at most 4 (one
// activation block) or 2 steps (one batch), doubled while the grid has
// fewer than 2048 waves and every run keeps at least two steps; 0 when no
// single-batch split fits (the caller then runs 8 waves in batches: the
// batch loop's registers do not fit 16 waves per block).
int pick_waves(uint32_t blocks, uint32_t kb, uint32_t m) {
  const uint32_t spw = m <= 16 ? 4 : 2;
  int waves = 0;
  for (int w : {4, 8, 16})
    if ((kb + w - 1) / w <= spw) {
      waves = w;
      break;
    }
  if (!waves) return 0;
  while (waves < 16 && blocks * (uint32_t)waves < 2048 && kb >= 4u * (uint32_t)waves) waves *= 2;
  return waves;
}

template <int WF, int SCALE>
void launch_waves(const SmallParams& sp, uint32_t problems, int waves, hipStream_t s) {
  const uint32_t kb = sp.k / 128;
  if (!waves) {
    launch_mt<WF, SCALE, 8, true>(sp, problems, (kb + 7) / 8, s);
    return;
  }
  const uint32_t run = (kb + waves - 1) / waves;
  if (waves == 4) launch_mt<WF, SCALE, 4, false>(sp, problems, run, s);
  else if (waves == 8) launch_mt<WF, SCALE, 8, false>(sp, problems, run, s);
  else launch_mt<WF, SCALE, 16, false>(sp, problems, run, s);
}

St launch_small(SmallParams sp, int wf, ScaleFmt fmt, uint32_t problems, hipStream_t s, bool& taken) {
  taken = false;
  if (sp.m == 0 || sp.n % 16 || sp.k % 128 || !SmallMTakes(sp.m, sp.n, problems)) return Ok();
  const uint32_t chunks = (sp.m + kSmallMChunkRows - 1) / kSmallMChunkRows;
  const int waves = pick_waves(sp.n / 16 * problems * chunks, sp.k / 128, std::min(sp.m, kSmallMChunkRows));
  taken = true;
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  if (wf == kSmallFp4) launch_waves<kSmallFp4, kScaleUe8m0>(sp, problems, waves, s);
  else if (fmt == kScaleF32) launch_waves<kSmallFp8, kScaleF32>(sp, problems, waves, s);
  else launch_waves<kSmallFp8, kScaleUe8m0>(sp, problems, waves, s);
  return AfterLaunch("small_m_gemm_launch_failed");
}

}  // namespace

St LaunchFp8SmallM(const BlockGemmArgs& a, bool& taken) {
  SmallParams sp{};
  sp.a = a.a;
  sp.a_scale = a.a_scale;
  sp.w = a.w;
  sp.w_scale = a.w_scale;
  sp.out = a.out;
  sp.err = a.error_flag;
  sp.m = a.m;
  sp.n = a.n;
  sp.k = a.k;
  sp.a_rows_total = a.a_rows_total;
  sp.a_row_stride = a.a_row_stride;
  sp.a_prob_row = a.a_prob_row;
  sp.out_row_stride = a.out_row_stride ? a.out_row_stride : a.n;
  sp.out_prob_col = a.out_prob_col;
  sp.check_codes = a.check_codes ? 1u : 0u;
  sp.write_nonfinite = a.write_nonfinite ? 1u : 0u;
  sp.out_f32 = a.out_kind == kOutF32 ? 1u : 0u;
  sp.err_code = a.err_code_bit;
  sp.err_scale = a.err_scale_bit;
  sp.err_nonfinite = a.err_nonfinite_bit;
  return launch_small(sp, kSmallFp8, a.scale_fmt, a.problems, a.stream, taken);
}

St LaunchFp4SmallM(const Fp4GemmArgs& a, bool& taken) {
  SmallParams sp{};
  sp.a = static_cast<const uint8_t*>(a.a);
  sp.a_scale = a.a_scale;
  sp.w = a.w;
  sp.w_scale = a.w_scale;
  sp.out = a.out;
  sp.err = a.error_flag;
  sp.m = a.m;
  sp.n = a.n;
  sp.k = a.k;
  sp.a_rows_total = a.a_rows_total;
  sp.a_row_stride = 1;
  sp.out_row_stride = a.n;
  sp.check_codes = 1;
  sp.out_f32 = a.out_kind == kOutF32 ? 1u : 0u;
  sp.err_code = 1u;
  sp.err_scale = 2u;
  sp.err_nonfinite = 4u;
  return launch_small(sp, kSmallFp4, kScaleUe8m0, a.problems, a.stream, taken);
}

}  // namespace pih_amd
