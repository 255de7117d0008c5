// Block-scaled FP8 GEMM for gfx950 on v_mfma_scale_f32_16x16x128_f8f6f4.
//
// Semantics (reference src/model/deepseek_fp8_gemm_oracle.cpp:10-80 and the
// kernel plugins/kernels/deepseek-v4-sm89/native/deepseek_fp8_gemm.cu:26-78):
//   out[m,n] = sum_kb (sum_{i<128} A[m,128kb+i] * W[n,128kb+i])
//                     * sa[m,kb] * sw[n/128,kb]
// with e4m3fn operands and either UE8M0 scale bytes (2^(b-127)) or fp32
// scales.  One 16x16x128 MFMA covers exactly one 128-deep scale block, so
//   UE8M0: the scales ride in the MFMA's own E8M0 scale operands and the
//          hardware accumulates acc += 2^(sa-127) 2^(sw-127) A.W exactly as
//          the oracle's power-of-two block products;
//   fp32 : each block's product is taken with unit scales and added to the
//          fp32 accumulator with one FMA by sa*sw (DeepSeek-V3 style).
//
// Tiling: 256 threads = 4 waves, block tile 128 (rows) x 128 (W rows), each
// wave 64x64 = 4x4 MFMA tiles.  A and W tiles are staged through LDS (rows
// padded to 144 B so the 16 rows a ds_read_b128 touches fall on distinct
// banks), double-buffered with one barrier per 128-deep step and a
// register prefetch of the next step's global loads.
//
// Problems: strided (dense GEMM, the reference's grouped projection whose
// A rows are t*G+g) or MoE segments whose row ranges come from
// device-resident expert offsets; a MoE tile finds its expert with a
// block-wide scan over the per-expert tile counts, so no host round trip is
// needed between the routing scan and the GEMM.
#include "device_common.hpp"
#include "kernels.hpp"

namespace pih_amd {
namespace {

constexpr int BM = 128, BN = 128, BKB = 128, LDS_ROW = 144, THREADS = 256;

struct GemmParams {
  const uint8_t* a;
  const void* a_scale;
  const uint32_t* a_gather;
  const uint8_t* w;
  const void* w_scale;
  void* out;
  const float* row_weight;
  const uint32_t* offsets;
  uint32_t* err;
  uint32_t m, n, k, problems, a_rows_total;
  uint32_t a_row_stride, a_prob_row;
  uint64_t out_row_stride;
  uint32_t out_prob_col;
  uint32_t n_tiles, m_tiles_per, tiles_total;
  float limit;
  uint32_t err_code, err_scale, err_nonfinite;
};

// Expert lookup for MoE tile g: returns false when g is past the last tile.
// Tile counts per expert are ceil(rows_e / BM); the block scans them.
__device__ bool moe_find_tile(const uint32_t* offsets, uint32_t experts, uint32_t m_bound,
                              uint32_t g, uint32_t* err, uint32_t err_code, uint32_t& expert,
                              uint32_t& row0, uint32_t& rows) {
  __shared__ uint32_t s_scan[THREADS];
  __shared__ uint32_t s_res[3];
  const uint32_t tid = threadIdx.x;
  const uint32_t per = (experts + THREADS - 1) / THREADS;
  uint32_t cnt = 0;
  for (uint32_t j = 0; j < per; ++j) {
    const uint32_t e = tid * per + j;
    if (e < experts) {
      const uint32_t lo = offsets[e], hi = offsets[e + 1];
      cnt += hi > lo ? (hi - lo + BM - 1) / BM : 0;
    }
  }
  if (tid == 0) s_res[0] = 0xffffffffu;
  s_scan[tid] = cnt;
  __syncthreads();
  for (uint32_t off = 1; off < THREADS; off <<= 1) {
    const uint32_t v = tid >= off ? s_scan[tid - off] : 0u;
    __syncthreads();
    s_scan[tid] += v;
    __syncthreads();
  }
  const uint32_t incl = s_scan[tid], excl = incl - cnt;
  if (g >= excl && g < incl) {
    uint32_t acc = excl;
    for (uint32_t j = 0; j < per; ++j) {
      const uint32_t e = tid * per + j;
      if (e >= experts) break;
      const uint32_t lo = offsets[e], hi = offsets[e + 1];
      const uint32_t t = hi > lo ? (hi - lo + BM - 1) / BM : 0;
      if (g < acc + t) {
        s_res[0] = e;
        s_res[1] = g - acc;
        break;
      }
      acc += t;
    }
  }
  __syncthreads();
  if (s_res[0] == 0xffffffffu) return false;
  expert = s_res[0];
  const uint32_t lo = offsets[expert], hi = offsets[expert + 1];
  row0 = lo + s_res[1] * BM;
  rows = min((uint32_t)BM, hi - row0);
  if (hi > m_bound || lo > hi) {
    if (tid == 0) atomicOr(err, err_code);
    return false;
  }
  return true;
}

template <int SCALE, int OUT, bool MOE, bool CHECK>
__global__ __launch_bounds__(THREADS, 2) void fp8_block_gemm_kernel(GemmParams p) {
  __shared__ __align__(16) uint8_t sA[2][BM * LDS_ROW];
  __shared__ __align__(16) uint8_t sB[2][BN * LDS_ROW];
  __shared__ __align__(16) uint32_t sAs[2][BM];

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t wm = wave >> 1, wn = wave & 1, lr = lane & 15, lg = lane >> 4;

  const uint32_t tile = xcd_chunked_tile(blockIdx.x, gridDim.x);
  if (tile >= p.tiles_total) return;
  const uint32_t mtot = MOE ? p.tiles_total / p.n_tiles : p.problems * p.m_tiles_per;
  const uint32_t nt = tile / mtot, g = tile % mtot;

  uint32_t prob, row0, rows;
  if constexpr (MOE) {
    if (!moe_find_tile(p.offsets, p.problems, p.m, g, p.err, p.err_code, prob, row0, rows)) return;
  } else {
    prob = g / p.m_tiles_per;
    row0 = (g % p.m_tiles_per) * BM;
    rows = min((uint32_t)BM, p.m - row0);
  }

  const uint32_t K = p.k, KB = K / BKB;
  const uint32_t col16 = tid & 7;
  uint32_t bad = 0;

  // A rows this thread stages (r = tid/8 + 32 i) and the row whose scale it
  // stages (r = tid, tid < BM).
  // Rows past the tile's end (and rejected gather indices) read A row 0:
  // every load stays unconditional and in bounds, and the rows they feed
  // are never stored (an output row depends on its own A row only).
  auto a_source = [&](uint32_t r) -> uint64_t {
    if (r >= rows) return 0;
    uint64_t src;
    if constexpr (MOE) {
      const uint32_t logical = row0 + r;
      src = p.a_gather ? p.a_gather[logical] : logical;
    } else {
      src = (uint64_t)(row0 + r) * p.a_row_stride + (uint64_t)prob * p.a_prob_row;
    }
    if (src >= p.a_rows_total) {
      bad |= kErrCode;
      return 0;
    }
    return src;
  };
  const uint8_t* a_ptr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) a_ptr[i] = p.a + a_source((tid >> 3) + 32 * i) * K + col16 * 16;
  const uint64_t s_src = a_source(tid < BM ? tid : 0);

  const uint8_t* w_base = p.w + (uint64_t)prob * p.n * K;
  const uint8_t* w_ptr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t r = (tid >> 3) + 32 * i;
    uint32_t wrow;
    if constexpr (OUT == kOutSwiGlu) {
      const uint32_t half = r >> 6, j = (r & 63) >> 4, rr = r & 15;
      const uint32_t base = nt * 64 + half * 32 + (j & 1) * 16 + rr;
      wrow = j < 2 ? base : p.n / 2 + base;
    } else {
      wrow = nt * BN + r;
    }
    w_ptr[i] = w_base + (uint64_t)wrow * K + col16 * 16;
  }
  // weight scale rows (128-row blocks) used by this tile
  const uint32_t ws_stride = KB;
  const uint64_t ws_prob = (uint64_t)prob * (p.n / 128) * KB;
  uint32_t wblk0, wblk1;
  if constexpr (OUT == kOutSwiGlu) {
    wblk0 = (nt * 64) / 128;
    wblk1 = (p.n / 2 + nt * 64) / 128;
  } else {
    wblk0 = wblk1 = nt;
  }

  v4i ra[4], rb[4];
  uint32_t rsa = 0;
  auto gload = [&](uint32_t kb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ra[i] = *reinterpret_cast<const v4i*>(a_ptr[i] + (uint64_t)kb * BKB);
      rb[i] = *reinterpret_cast<const v4i*>(w_ptr[i] + (uint64_t)kb * BKB);
    }
    if (SCALE == kScaleF32) {
      rsa = __float_as_uint(static_cast<const float*>(p.a_scale)[s_src * KB + kb]);
    } else {
      rsa = static_cast<const uint8_t*>(p.a_scale)[s_src * KB + kb];
      if (rsa == 0xffu && tid < rows) bad |= kErrScale;
    }
    if constexpr (CHECK) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t ta = e4m3_nan_bytes(ra[i][0]) | e4m3_nan_bytes(ra[i][1]) |
                            e4m3_nan_bytes(ra[i][2]) | e4m3_nan_bytes(ra[i][3]);
        const uint32_t tb = e4m3_nan_bytes(rb[i][0]) | e4m3_nan_bytes(rb[i][1]) |
                            e4m3_nan_bytes(rb[i][2]) | e4m3_nan_bytes(rb[i][3]);
        if ((ta && (tid >> 3) + 32 * i < rows) || tb) bad |= kErrCode;
      }
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t r = (tid >> 3) + 32 * i;
      *reinterpret_cast<v4i*>(&sA[buf][r * LDS_ROW + col16 * 16]) = ra[i];
      *reinterpret_cast<v4i*>(&sB[buf][r * LDS_ROW + col16 * 16]) = rb[i];
    }
    if (tid < BM) sAs[buf][tid] = rsa;
  };

  v4f acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = v4f{0.f, 0.f, 0.f, 0.f};

  // rows of this wave's 16-row sub-tiles that exist
  uint32_t ms_live = 0;
#pragma unroll
  for (int ms = 0; ms < 4; ++ms)
    if (wm * 64 + ms * 16 < rows) ms_live = ms + 1;

  gload(0);
  lstore(0);
  __syncthreads();

  for (uint32_t kb = 0; kb < KB; ++kb) {
    const int buf = kb & 1;
    if (kb + 1 < KB) gload(kb + 1);

    // weight scales of this step (uniform across the block)
    uint32_t ws0b, ws1b;
    float ws0f, ws1f;
    if constexpr (SCALE == kScaleF32) {
      const float* ws = static_cast<const float*>(p.w_scale) + ws_prob;
      ws0f = ws[(uint64_t)wblk0 * ws_stride + kb];
      ws1f = ws[(uint64_t)wblk1 * ws_stride + kb];
    } else {
      const uint8_t* ws = static_cast<const uint8_t*>(p.w_scale) + ws_prob;
      ws0b = ws[(uint64_t)wblk0 * ws_stride + kb];
      ws1b = ws[(uint64_t)wblk1 * ws_stride + kb];
      if (ws0b == 0xffu || ws1b == 0xffu) bad |= kErrScale;
    }

    if (ms_live) {
      v8i bv[4];
#pragma unroll
      for (int ns = 0; ns < 4; ++ns) {
        const uint8_t* pb = &sB[buf][(wn * 64 + ns * 16 + lr) * LDS_ROW + lg * 32];
        const uint4 x0 = *reinterpret_cast<const uint4*>(pb);
        const uint4 x1 = *reinterpret_cast<const uint4*>(pb + 16);
        bv[ns] = v8i{(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w,
                     (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
      }
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) {
        if (ms >= (int)ms_live) break;
        const uint8_t* pa = &sA[buf][(wm * 64 + ms * 16 + lr) * LDS_ROW + lg * 32];
        const uint4 x0 = *reinterpret_cast<const uint4*>(pa);
        const uint4 x1 = *reinterpret_cast<const uint4*>(pa + 16);
        const v8i av = v8i{(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w,
                           (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
        if constexpr (SCALE == kScaleF32) {
          const uint4 s4 = *reinterpret_cast<const uint4*>(&sAs[buf][wm * 64 + ms * 16 + 4 * lg]);
          const float sa[4] = {__uint_as_float(s4.x), __uint_as_float(s4.y),
                               __uint_as_float(s4.z), __uint_as_float(s4.w)};
#pragma unroll
          for (int ns = 0; ns < 4; ++ns) {
            const v4f t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                av, bv[ns], v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 127, 0, 127);
            const float wsv = (OUT == kOutSwiGlu && ns >= 2) ? ws1f : ws0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[ms][ns][i] = __builtin_fmaf(t[i], sa[i] * wsv, acc[ms][ns][i]);
          }
        } else {
          const int sab = (int)sAs[buf][wm * 64 + ms * 16 + lr];
#pragma unroll
          for (int ns = 0; ns < 4; ++ns) {
            const int wsb = (int)((OUT == kOutSwiGlu && ns >= 2) ? ws1b : ws0b);
            acc[ms][ns] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                av, bv[ns], acc[ms][ns], 0, 0, 0, sab, 0, wsb);
          }
        }
      }
    }
    if (kb + 1 < KB) lstore(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue
#pragma unroll
  for (int ms = 0; ms < 4; ++ms) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t r = wm * 64 + ms * 16 + 4 * lg + i;
      if (r >= rows) continue;
      uint64_t orow;
      if constexpr (MOE) {
        orow = (uint64_t)(row0 + r) * p.out_row_stride;
      } else {
        orow = (uint64_t)(row0 + r) * p.out_row_stride + (uint64_t)prob * p.out_prob_col;
      }
      if constexpr (OUT == kOutSwiGlu) {
        const float rw = p.row_weight ? p.row_weight[row0 + r] : 1.0f;
#pragma unroll
        for (int ns = 0; ns < 2; ++ns) {
          float gt = bf16_round(acc[ms][ns][i]);
          float up = bf16_round(acc[ms][ns + 2][i]);
          if (!__builtin_isfinite(gt) || !__builtin_isfinite(up)) {
            bad |= kErrNonFinite;
            continue;
          }
          if (p.limit > 0.0f) {
            gt = fminf(gt, p.limit);
            up = fminf(fmaxf(up, -p.limit), p.limit);
          }
          float v = (gt / (1.0f + expf(-gt))) * up;
          v = v * rw;
          if (!__builtin_isfinite(v)) {
            bad |= kErrNonFinite;
            continue;
          }
          const uint32_t col = nt * 64 + wn * 32 + ns * 16 + lr;
          static_cast<uint16_t*>(p.out)[orow + col] = (uint16_t)f32_to_bf16_bits(v);
        }
      } else {
#pragma unroll
        for (int ns = 0; ns < 4; ++ns) {
          const float v = acc[ms][ns][i];
          if (!__builtin_isfinite(v)) {
            bad |= kErrNonFinite;
            continue;
          }
          const uint32_t col = nt * BN + wn * 64 + ns * 16 + lr;
          if constexpr (OUT == kOutF32) {
            static_cast<float*>(p.out)[orow + col] = v;
          } else {
            static_cast<uint16_t*>(p.out)[orow + col] = (uint16_t)f32_to_bf16_bits(v);
          }
        }
      }
    }
  }
  if (bad) {
    const uint32_t bits = ((bad & kErrCode) ? p.err_code : 0u) |
                          ((bad & kErrScale) ? p.err_scale : 0u) |
                          ((bad & kErrNonFinite) ? p.err_nonfinite : 0u);
    atomicOr(p.err, bits);
  }
}

template <int SCALE, int OUT, bool MOE, bool CHECK>
void launch_one(const GemmParams& gp, uint32_t grid, hipStream_t s) {
  hipLaunchKernelGGL((fp8_block_gemm_kernel<SCALE, OUT, MOE, CHECK>), dim3(grid), dim3(THREADS), 0,
                     s, gp);
}

template <int SCALE, int OUT>
void dispatch_moe_check(const GemmParams& gp, uint32_t grid, hipStream_t s, bool moe, bool check) {
  if (moe) {
    if (check) launch_one<SCALE, OUT, true, true>(gp, grid, s);
    else launch_one<SCALE, OUT, true, false>(gp, grid, s);
  } else {
    if (check) launch_one<SCALE, OUT, false, true>(gp, grid, s);
    else launch_one<SCALE, OUT, false, false>(gp, grid, s);
  }
}

}  // namespace

St LaunchFp8BlockGemm(const BlockGemmArgs& a) {
  if (!a.a || !a.a_scale || !a.w || !a.w_scale || !a.out || !a.error_flag || !a.stream)
    return Invalid("fp8_gemm_null_argument");
  if (a.k == 0 || a.k % 128 || a.n == 0 || a.n % 128 || a.problems == 0 || a.m == 0)
    return Invalid("fp8_gemm_shape_invalid");
  if (a.out_kind == kOutSwiGlu && (a.n % 256)) return Invalid("fp8_gemm_swiglu_shape_invalid");
  if (a.scale_fmt != kScaleF32 && a.scale_fmt != kScaleUe8m0) return Invalid("fp8_gemm_scale_format_invalid");
  if (a.out_kind != kOutBf16 && a.out_kind != kOutF32 && a.out_kind != kOutSwiGlu)
    return Invalid("fp8_gemm_output_type_invalid");
  if (a.moe && !a.offsets) return Invalid("fp8_gemm_offsets_missing");
  if (a.a_rows_total == 0) return Invalid("fp8_gemm_a_rows_invalid");

  GemmParams gp{};
  gp.a = a.a;
  gp.a_scale = a.a_scale;
  gp.a_gather = a.a_gather;
  gp.w = a.w;
  gp.w_scale = a.w_scale;
  gp.out = a.out;
  gp.row_weight = a.row_weight;
  gp.offsets = a.offsets;
  gp.err = a.error_flag;
  gp.m = a.m;
  gp.n = a.n;
  gp.k = a.k;
  gp.problems = a.problems;
  gp.a_rows_total = a.a_rows_total;
  gp.a_row_stride = a.a_row_stride;
  gp.a_prob_row = a.a_prob_row;
  gp.out_row_stride = a.out_row_stride ? a.out_row_stride
                                        : (a.out_kind == kOutSwiGlu ? a.n / 2 : a.n);
  gp.out_prob_col = a.out_prob_col;
  gp.limit = a.swiglu_limit;
  gp.err_code = a.err_code_bit;
  gp.err_scale = a.err_scale_bit;
  gp.err_nonfinite = a.err_nonfinite_bit;
  gp.n_tiles = a.n / BN;
  uint64_t mt;
  if (a.moe) {
    // sum_e ceil(rows_e/BM) <= rows/BM + (number of non-empty experts)
    mt = (uint64_t)a.m / BM + (a.problems < a.m ? a.problems : a.m);
    gp.m_tiles_per = 0;
  } else {
    gp.m_tiles_per = (a.m + BM - 1) / BM;
    mt = (uint64_t)gp.m_tiles_per * a.problems;
  }
  const uint64_t total = mt * gp.n_tiles;
  if (total == 0 || total > 0x7fffffffull - 8) return Invalid("fp8_gemm_grid_too_large");
  gp.tiles_total = (uint32_t)total;
  const uint32_t grid = (uint32_t)((total + 7) / 8 * 8);

  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  const bool check = a.check_codes;
  if (a.scale_fmt == kScaleF32) {
    if (a.out_kind == kOutBf16) dispatch_moe_check<kScaleF32, kOutBf16>(gp, grid, a.stream, a.moe, check);
    else if (a.out_kind == kOutF32) dispatch_moe_check<kScaleF32, kOutF32>(gp, grid, a.stream, a.moe, check);
    else dispatch_moe_check<kScaleF32, kOutSwiGlu>(gp, grid, a.stream, a.moe, check);
  } else {
    if (a.out_kind == kOutBf16) dispatch_moe_check<kScaleUe8m0, kOutBf16>(gp, grid, a.stream, a.moe, check);
    else if (a.out_kind == kOutF32) dispatch_moe_check<kScaleUe8m0, kOutF32>(gp, grid, a.stream, a.moe, check);
    else dispatch_moe_check<kScaleUe8m0, kOutSwiGlu>(gp, grid, a.stream, a.moe, check);
  }
  return AfterLaunch("fp8_gemm_launch_failed");
}

}  // namespace pih_amd
