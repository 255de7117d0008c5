// MFMA GEMM family for gfx950: block-scaled FP8, MXFP4-weight and BF16
// GEMMs over dense, strided-batched and MoE-segmented problems.
//
//   out = A . W^T   (A [rows, K] activations, W [N, K] weights, row-major)
//
// Operand kinds (one template instance each):
//   kFp8     A e4m3, W e4m3, one scale per (A row, 128 k) and per
//            (128 W rows, 128 k), fp32 or UE8M0
//            (reference src/model/deepseek_fp8_gemm_oracle.cpp:10-80,
//            plugins/kernels/deepseek-v4-sm89/native/deepseek_fp8_gemm.cu).
//            One v_mfma_scale_f32_16x16x128_f8f6f4 covers exactly one
//            128-deep scale block: UE8M0 scales ride in the instruction's
//            E8M0 scale operands (hardware applies 2^(sa-127) 2^(sw-127) to
//            the exact block product); fp32 scales are applied by one FMA per
//            output and block (DeepSeek-V3 style).
//   kFp4     A e4m3 + UE8M0 per (row, 128 k); W e2m1 packed two per byte
//            (low nibble = even k) + UE8M0 per (W row, 32 k)
//            (reference src/model/deepseek_fp4_gemm_oracle.cpp:11-91).  The
//            same MX instruction with the B operand in FP4 format and the
//            lane's own 32-element block scale: the MX-FP4 MFMA of CDNA4.
//   kBf16    A, W bf16; two v_mfma_f32_16x16x32_bf16 per 64-deep step
//            (the GemmPlan C = A.W^T of src/backend/cuda/gemm_plan.cpp).
//   kBf16Fp4 A bf16; W MXFP4 dequantised exactly into bf16 in registers
//            (every e2m1 value times 2^(s-127) is a bf16 number; one
//            v_cvt_scalef32_pk_bf16_fp4 per byte), then bf16 MFMAs.
//   kMx8     A e4m3 + UE8M0 per (row, 32 k); W e4m3 + UE8M0 per (32 rows,
//            32 k): the DeepSeek V4.1 FP8 linear
//            (plugins/model-deepseek-v41/linear_fp8.cu:39-76), on the MX
//            instruction with both operands in the FP8 lane map (lane group g
//            holds k [16g, 16g+16) and [64+16g, 64+16g+16)) and each lane
//            group's scale byte covering k block g of the step (measured on
//            gfx950: lane group g's scale applies to k [32g, 32g+32)).
//   kMx4     as kMx8 with W e2m1 + UE8M0 per (row, 32 k) (the V4.1 mixed
//            FP8/FP4 linear).
//
// Tiling: 256 threads = 4 waves, block tile 128 A rows x 128 W rows, each
// wave 64x64 = 4x4 MFMA 16x16 tiles.  Per K step A and W tiles go through
// LDS, double-buffered with one barrier per step, next step prefetched into
// registers.  128-byte and 64-byte tile rows are dense with XOR-swizzled
// 16-byte slots (chunk c of row r in slot c ^ ((r >> 1) & 7), resp.
// c ^ ((r >> 2) & 3)), so that the 16 lanes of one ds_write_b128 or
// ds_read_b128 cycle touch 64 distinct 4-byte banks; 32-byte rows are padded
// to 48 B.  Every global load is unconditional and in bounds (rows
// past a tile's end read row 0 and are never stored).
//
// Problems: strided (dense GEMM; the reference's grouped projection whose A
// rows are t*G+g) or MoE segments from device-resident expert offsets; a
// MoE tile finds its expert by a block-wide scan of per-expert tile counts.
// The grid is renumbered so that each XCD walks one contiguous range of
// tiles (tiles of the same expert and W slice share that XCD's L2).
//
// Epilogues: bf16 or fp32 store, or the fused gate/up SwiGLU: the W tile
// holds 64 gate rows and the 64 matching up rows, so every lane owns a
// gate/up pair and writes mid = bf16(silu(g') * u' * route_weight) with
// g, u the bf16-rounded GEMM results (clamped when limit > 0).
#include <mutex>

#include "device_common.hpp"
#include "kernels.hpp"

namespace pih_amd {
namespace {

enum Kind : int { kFp8 = 0, kFp4 = 1, kBf16 = 2, kBf16Fp4 = 3, kMx8 = 4, kMx4 = 5 };

constexpr int BM = 128, BN = 128, THREADS = 256, A_STEP_BYTES = 128;
constexpr int LDS_A = A_STEP_BYTES;

// Byte offset of 16-byte chunk c of tile row r in a tile of ROW-byte rows.
template <int ROW>
__device__ __forceinline__ uint32_t lds_at(uint32_t r, uint32_t c) {
  if constexpr (ROW == 128) return r * 128 + ((c ^ ((r >> 1) & 7u)) << 4);
  else if constexpr (ROW == 64) return r * 64 + ((c ^ ((r >> 2) & 3u)) << 4);
  else return r * (ROW + 16) + (c << 4);
}
template <int ROW>
constexpr int lds_row_bytes() { return ROW == 128 || ROW == 64 ? ROW : ROW + 16; }

template <int KIND>
struct Traits;
template <>
struct Traits<kFp8> {
  static constexpr int K_STEP = 128, B_STEP_BYTES = 128, A_ELEM = 1;
};
template <>
struct Traits<kFp4> {
  static constexpr int K_STEP = 128, B_STEP_BYTES = 64, A_ELEM = 1;
};
template <>
struct Traits<kBf16> {
  static constexpr int K_STEP = 64, B_STEP_BYTES = 128, A_ELEM = 2;
};
template <>
struct Traits<kBf16Fp4> {
  static constexpr int K_STEP = 64, B_STEP_BYTES = 32, A_ELEM = 2;
};
template <>
struct Traits<kMx8> {
  static constexpr int K_STEP = 128, B_STEP_BYTES = 128, A_ELEM = 1;
};
template <>
struct Traits<kMx4> {
  static constexpr int K_STEP = 128, B_STEP_BYTES = 64, A_ELEM = 1;
};

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
  uint32_t light_rows;  // MoE: experts with at most this many rows are skipped
  float limit;
  uint32_t err_code, err_scale, err_nonfinite;
  uint32_t write_nonfinite;  // store a non-finite result as well as flagging it
  // when set, the kernel runs only if (*run_if & run_bit) != 0 (the checking
  // half of the big-tile dense FP8 path: it works only when the code scan
  // found a NaN code, and the big-tile kernel then steps aside)
  const uint32_t* run_if;
  uint32_t run_bit;
};

// Expert lookup for MoE tile g: returns false when g is past the last tile.
__device__ bool moe_find_tile(const uint32_t* offsets, uint32_t experts, uint32_t m_bound, uint32_t light_rows,
                              uint32_t g, uint32_t* err, uint32_t err_code, uint32_t& expert, uint32_t& row0,
                              uint32_t& rows) {
  __shared__ uint32_t s_scan[THREADS];
  __shared__ uint32_t s_res[2];
  const uint32_t tid = threadIdx.x;
  const uint32_t per = (experts + THREADS - 1) / THREADS;
  uint32_t cnt = 0;
  for (uint32_t j = 0; j < per; ++j) {
    const uint32_t e = tid * per + j;
    if (e < experts) {
      const uint32_t lo = offsets[e], hi = offsets[e + 1];
      cnt += hi > lo + light_rows ? (hi - lo + BM - 1) / BM : 0;
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
      const uint32_t t = hi > lo + light_rows ? (hi - lo + BM - 1) / BM : 0;
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
  if (hi > m_bound || lo > hi) {
    if (tid == 0) atomicOr(err, err_code);
    return false;
  }
  row0 = lo + s_res[1] * BM;
  rows = min((uint32_t)BM, hi - row0);
  return true;
}

__device__ __forceinline__ v8i cat8(v4i x, v4i y) {
  return v8i{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
}

__device__ __forceinline__ uint32_t ff_bytes(uint32_t w) {
  // non-zero when any byte of w is 0xFF
  const uint32_t n = ~w;
  return (n - 0x01010101u) & ~n & 0x80808080u;
}

// An operand fragment whose E8M0 block scale is 0xFF (the reference skips
// that block) becomes zeros with scale 127, so its products add exactly 0;
// the test is wave-wide, and the select runs only in a wave that has one.
template <typename S>
__device__ __forceinline__ void zero_ff_row(S& scale, v8i& frag) {
  const bool ff = (uint32_t)scale == 0xffu;
  if (__builtin_amdgcn_ballot_w64(ff)) {
    if (ff) {
      scale = 127;
      frag = v8i{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }
}

// 8 e2m1 nibbles of `w` (low nibble first) times the power of two `scale`
// as 8 bf16 values.  v_cvt_scalef32_pk_bf16_fp4 converts one byte (two
// nibbles, low first) per instruction; the product is exact for every UE8M0
// scale 0..254 (checked against decode-multiply-truncate over all 256 bytes
// and all 255 scales on gfx950, overflow to inf included).
__device__ __forceinline__ v8s dequant8_fp4(uint32_t w, float scale) {
  typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
  const v2bf b0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0);
  const v2bf b1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1);
  const v2bf b2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2);
  const v2bf b3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3);
  const v4i o{__builtin_bit_cast(int, b0), __builtin_bit_cast(int, b1), __builtin_bit_cast(int, b2),
              __builtin_bit_cast(int, b3)};
  return __builtin_bit_cast(v8s, o);
}

template <int KIND, int SCALE, int OUT, bool MOE, bool CHECK>
__global__ __launch_bounds__(THREADS, 2) void mfma_gemm_kernel(GemmParams p) {
  using T = Traits<KIND>;
  constexpr int B_STEP = T::B_STEP_BYTES;
  constexpr int LDS_B = lds_row_bytes<B_STEP>();
  constexpr int B_CPR = B_STEP / 16;             // 16-byte chunks per W row per step
  constexpr int B_LOADS = BN * B_CPR / THREADS;  // per thread
  constexpr bool MX = KIND == kMx8 || KIND == kMx4;  // per-32 scales on both operands
  constexpr bool FP8A = KIND == kFp8 || KIND == kFp4 || MX;
  constexpr bool BSCALE_ROW = KIND == kFp4 || KIND == kBf16Fp4 || MX;  // per-row MX scales
  constexpr bool ASCALE = KIND == kFp8 || KIND == kFp4 || MX;
  constexpr bool E8M0_A = (KIND == kFp8 && SCALE == kScaleUe8m0) || KIND == kFp4;
  // FP8 lane map for A (and kMx8's W): chunks lg and lg + 4 of the step
  constexpr bool LANE_MAP_MX = KIND == kFp4 || MX;

  __shared__ __align__(16) uint8_t sA[2][BM * LDS_A];
  __shared__ __align__(16) uint8_t sB[2][BN * LDS_B];
  __shared__ __align__(16) uint32_t sAs[2][BM];
  __shared__ __align__(16) uint32_t sBs[2][BSCALE_ROW ? BN : 1];

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t wm = wave >> 1, wn = wave & 1, lr = lane & 15, lg = lane >> 4;

  // the scan (or an earlier call) set the bit before this launch began
  if (p.run_if && !(__hip_atomic_load(p.run_if, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & p.run_bit)) return;
  const uint32_t tile = xcd_chunked_tile(blockIdx.x, gridDim.x);
  if (tile >= p.tiles_total) return;
  const uint32_t mtot = MOE ? p.tiles_total / p.n_tiles : p.problems * p.m_tiles_per;
  const uint32_t nt = tile / mtot, g = tile % mtot;

  uint32_t prob, row0, rows;
  if constexpr (MOE) {
    if (!moe_find_tile(p.offsets, p.problems, p.m, p.light_rows, g, p.err, p.err_code, prob, row0, rows)) return;
  } else {
    prob = g / p.m_tiles_per;
    row0 = (g % p.m_tiles_per) * BM;
    rows = min((uint32_t)BM, p.m - row0);
  }

  const uint32_t K = p.k, KB = K / T::K_STEP;
  const uint64_t a_row_bytes = (uint64_t)K * T::A_ELEM;
  const uint64_t b_row_bytes = (uint64_t)K * B_STEP / T::K_STEP;
  uint32_t bad = 0;

  // Rows past the tile's end (and rejected gather indices) read A row 0:
  // loads stay unconditional and in bounds, and the output rows they feed
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
  const uint32_t a_col = tid & 7;
  const uint8_t* a_ptr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) a_ptr[i] = p.a + a_source((tid >> 3) + 32 * i) * a_row_bytes + a_col * 16;
  const uint64_t s_src = a_source(tid < BM ? tid : 0);

  // W rows this thread stages; for the SwiGLU epilogue the tile's 128 rows
  // are 64 gate rows and the 64 matching up rows, arranged so that each
  // wave's MFMA columns pair gate (ns = 0,1) with up (ns = 2,3).
  auto w_row = [&](uint32_t r) -> uint32_t {
    if constexpr (OUT == kOutSwiGlu) {
      const uint32_t half = r >> 6, j = (r & 63) >> 4, rr = r & 15;
      const uint32_t base = nt * 64 + half * 32 + (j & 1) * 16 + rr;
      return j < 2 ? base : p.n / 2 + base;
    } else {
      return nt * BN + r;
    }
  };
  const uint8_t* w_base = p.w + (uint64_t)prob * p.n * b_row_bytes;
  const uint8_t* w_ptr[B_LOADS];
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    const uint32_t c = tid + THREADS * i;
    w_ptr[i] = w_base + (uint64_t)w_row(c / B_CPR) * b_row_bytes + (c % B_CPR) * 16;
  }
  // per-row MX scale words (kFp4: 4 bytes per 128-deep step; kBf16Fp4: 2)
  const uint8_t* ws_row = nullptr;
  if constexpr (KIND == kMx8)  // one scale row per 32 W rows
    ws_row = static_cast<const uint8_t*>(p.w_scale) +
             ((uint64_t)prob * (p.n / 32) + w_row(tid < BN ? tid : 0) / 32) * (K / 32);
  else if constexpr (BSCALE_ROW)
    ws_row = static_cast<const uint8_t*>(p.w_scale) +
             ((uint64_t)prob * p.n + w_row(tid < BN ? tid : 0)) * (K / 32);
  // FP8 block scales (128-row blocks) used by this tile
  const uint64_t ws_prob = (uint64_t)prob * (p.n / 128) * (K / 128);
  uint32_t wblk0 = nt, wblk1 = nt;
  if constexpr (OUT == kOutSwiGlu) {
    wblk0 = (nt * 64) / 128;
    wblk1 = (p.n / 2 + nt * 64) / 128;
  }

  v4i ra[4], rb[B_LOADS];
  uint32_t rsa = 0, rsb = 0;
  auto gload = [&](uint32_t kb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) ra[i] = *reinterpret_cast<const v4i*>(a_ptr[i] + (uint64_t)kb * A_STEP_BYTES);
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) rb[i] = *reinterpret_cast<const v4i*>(w_ptr[i] + (uint64_t)kb * B_STEP);
    if constexpr (MX) {
      // four per-32 scale bytes per row and step; a 255 (NaN) scale raises
      // the error bit and propagates through the MFMA as the reference's
      // 2^128 term does
      rsa = *reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(p.a_scale) + s_src * (K / 32) +
                                               (uint64_t)kb * 4);
      if (ff_bytes(rsa) && tid < rows) bad |= kErrScale;
      rsb = *reinterpret_cast<const uint32_t*>(ws_row + (uint64_t)kb * 4);
      if (ff_bytes(rsb) && tid < BN) bad |= kErrScale;
    } else if constexpr (ASCALE) {
      if constexpr (E8M0_A) {
        // a 0xFF scale raises the scale bit and stays 0xFF in LDS: the
        // compute zeroes that row's fragment, so its block adds nothing, as
        // the reference skips it
        rsa = static_cast<const uint8_t*>(p.a_scale)[s_src * (K / 128) + kb];
        if (rsa == 0xffu && tid < rows) bad |= kErrScale;
      } else {
        rsa = __float_as_uint(static_cast<const float*>(p.a_scale)[s_src * (K / 128) + kb]);
      }
    }
    if constexpr (KIND == kFp4) {
      rsb = *reinterpret_cast<const uint32_t*>(ws_row + (uint64_t)kb * 4);
      // 0xFF bytes stay: the compute zeroes the fragment they scale
      if (ff_bytes(rsb) && tid < BN) bad |= kErrScale;
    } else if constexpr (KIND == kBf16Fp4) {
      rsb = *reinterpret_cast<const uint16_t*>(ws_row + (uint64_t)kb * 2);
      if (ff_bytes(rsb) && tid < BN) bad |= kErrScale;
    }
    if constexpr (CHECK && MX) {
      // NaN codes raise the error bit and stay NaN (the V4.1 decode gives
      // NaN, so the output is non-finite as well)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t t = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) t |= e4m3_nan_bytes((uint32_t)ra[i][q]);
        if (t && (tid >> 3) + 32 * i < rows) bad |= kErrCode;
      }
      if constexpr (KIND == kMx8) {
        uint32_t t = 0;
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) t |= e4m3_nan_bytes((uint32_t)rb[i][q]);
        if (t) bad |= kErrCode;
      }
    } else if constexpr (CHECK && FP8A) {
      // NaN codes count as 0 in the sum (and raise the code bit), as the
      // reference decodes them
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t t = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t nq = e4m3_nan_bytes((uint32_t)ra[i][q]);
          ra[i][q] = (int)e4m3_nan_to_zero((uint32_t)ra[i][q], nq);
          t |= nq;
        }
        if (t && (tid >> 3) + 32 * i < rows) bad |= kErrCode;
      }
      if constexpr (KIND == kFp8) {
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) {
          uint32_t t = 0;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t nq = e4m3_nan_bytes((uint32_t)rb[i][q]);
            rb[i][q] = (int)e4m3_nan_to_zero((uint32_t)rb[i][q], nq);
            t |= nq;
          }
          if (t) bad |= kErrCode;
        }
      }
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<v4i*>(&sA[buf][lds_at<A_STEP_BYTES>((tid >> 3) + 32 * i, a_col)]) = ra[i];
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const uint32_t c = tid + THREADS * i;
      *reinterpret_cast<v4i*>(&sB[buf][lds_at<B_STEP>(c / B_CPR, c % B_CPR)]) = rb[i];
    }
    if constexpr (ASCALE)
      if (tid < BM) sAs[buf][tid] = rsa;
    if constexpr (BSCALE_ROW)
      if (tid < BN) sBs[buf][tid] = rsb;
  };

  v4f acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = v4f{0.f, 0.f, 0.f, 0.f};

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

    uint32_t ws0b = 127, ws1b = 127;
    float ws0f = 1.0f, ws1f = 1.0f;
    if constexpr (KIND == kFp8) {
      if constexpr (SCALE == kScaleF32) {
        const float* ws = static_cast<const float*>(p.w_scale) + ws_prob;
        ws0f = ws[(uint64_t)wblk0 * (K / 128) + kb];
        ws1f = ws[(uint64_t)wblk1 * (K / 128) + kb];
      } else {
        const uint8_t* ws = static_cast<const uint8_t*>(p.w_scale) + ws_prob;
        ws0b = ws[(uint64_t)wblk0 * (K / 128) + kb];
        ws1b = ws[(uint64_t)wblk1 * (K / 128) + kb];
        if (ws0b == 0xffu || ws1b == 0xffu) bad |= kErrScale;
      }
    }
    // a 0xFF W block scale: that block's MFMAs run with both E8M0 scales 0
    // (2^-254 times a sum below 2^25 is below the fp32 range, so exactly
    // zero is added), as the reference skips the block
    const bool wff0 = ws0b == 0xffu, wff1 = ws1b == 0xffu;
    ws0b = wff0 ? 0u : ws0b;
    ws1b = wff1 ? 0u : ws1b;

    if (ms_live) {
      // W operands for this wave's four 16-column blocks
      v8i bv[4];
      uint32_t bsc[4];
#pragma unroll
      for (int ns = 0; ns < 4; ++ns) {
        const uint32_t brow = wn * 64 + ns * 16 + lr;
        const uint8_t* pb = &sB[buf][brow * LDS_B];
        if constexpr (KIND == kFp8 || KIND == kBf16) {  // chunks 2lg, 2lg + 1
          const uint32_t o = lds_at<128>(brow, 2 * lg);
          bv[ns] = cat8(*reinterpret_cast<const v4i*>(&sB[buf][o]), *reinterpret_cast<const v4i*>(&sB[buf][o ^ 16]));
        } else if constexpr (KIND == kMx8) {  // FP8 lane map: chunks lg, lg + 4
          const uint32_t o = lds_at<128>(brow, lg);
          bv[ns] = cat8(*reinterpret_cast<const v4i*>(&sB[buf][o]), *reinterpret_cast<const v4i*>(&sB[buf][o ^ 64]));
          bsc[ns] = (sBs[buf][brow] >> (8 * lg)) & 0xffu;
        } else if constexpr (KIND == kFp4 || KIND == kMx4) {
          bv[ns] = cat8(*reinterpret_cast<const v4i*>(&sB[buf][lds_at<64>(brow, lg)]), v4i{0, 0, 0, 0});
          bsc[ns] = (sBs[buf][brow] >> (8 * lg)) & 0xffu;
          if constexpr (KIND == kFp4) zero_ff_row(bsc[ns], bv[ns]);
        } else {  // kBf16Fp4: 16 nibbles = k 16*lg .. 16*lg+15 of the step
          const uint2 w2 = *reinterpret_cast<const uint2*>(pb + lg * 8);
          const float sc = ue8m0_value((sBs[buf][brow] >> (8 * (lg >> 1))) & 0xffu);
          const v8s lo = dequant8_fp4(w2.x, sc), hi = dequant8_fp4(w2.y, sc);
          bv[ns] = cat8(__builtin_bit_cast(v4i, lo), __builtin_bit_cast(v4i, hi));
        }
      }
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) {
        if (ms >= (int)ms_live) break;
        const uint32_t arow = wm * 64 + ms * 16 + lr;
        // FP8 A against FP4 B: the instruction pairs an FP8 lane group g's
        // two 16-byte halves with k [16g, 16g+16) and [64+16g, 64+16g+16),
        // while an FP4 lane group g holds k [32g, 32g+32) contiguously
        // (measured on gfx950); same-format operands just use the same map.
        // chunks lg and lg + 4 (kFp4) or 2lg and 2lg + 1 of the 128-byte row
        const uint32_t ao = lds_at<A_STEP_BYTES>(arow, LANE_MAP_MX ? lg : 2 * lg);
        const v4i a0 = *reinterpret_cast<const v4i*>(&sA[buf][ao]);
        const v4i a1 = *reinterpret_cast<const v4i*>(&sA[buf][ao ^ (LANE_MAP_MX ? 64u : 16u)]);
        if constexpr (KIND == kFp8 && SCALE == kScaleF32) {
          const v4i s4 = *reinterpret_cast<const v4i*>(&sAs[buf][wm * 64 + ms * 16 + 4 * lg]);
          const v8i av = cat8(a0, a1);
#pragma unroll
          for (int ns = 0; ns < 4; ++ns) {
            const v4f t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv[ns], v4f{0.f, 0.f, 0.f, 0.f},
                                                                           0, 0, 0, 127, 0, 127);
            const float wsv = (OUT == kOutSwiGlu && ns >= 2) ? ws1f : ws0f;
#pragma unroll
            for (int i = 0; i < 4; ++i)
              acc[ms][ns][i] = __builtin_fmaf(t[i], __uint_as_float((uint32_t)s4[i]) * wsv, acc[ms][ns][i]);
          }
        } else if constexpr (KIND == kFp8) {
          int sab = (int)sAs[buf][arow];
          v8i av = cat8(a0, a1);
          zero_ff_row(sab, av);
#pragma unroll
          for (int ns = 0; ns < 4; ++ns) {
            const bool wff = (OUT == kOutSwiGlu && ns >= 2) ? wff1 : wff0;
            const int wsb = (int)((OUT == kOutSwiGlu && ns >= 2) ? ws1b : ws0b);
            acc[ms][ns] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv[ns], acc[ms][ns], 0, 0, 0,
                                                                           wff ? 0 : sab, 0, wsb);
          }
        } else if constexpr (KIND == kFp4) {
          int sab = (int)sAs[buf][arow];
          v8i av = cat8(a0, a1);
          zero_ff_row(sab, av);
#pragma unroll
          for (int ns = 0; ns < 4; ++ns)
            acc[ms][ns] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv[ns], acc[ms][ns], 0, 4, 0, sab,
                                                                           0, (int)bsc[ns]);
        } else if constexpr (MX) {
          // lane group lg supplies the scales of k block lg of the step
          const int sab = (int)((sAs[buf][arow] >> (8 * lg)) & 0xffu);
          const v8i av = cat8(a0, a1);
#pragma unroll
          for (int ns = 0; ns < 4; ++ns)
            acc[ms][ns] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                av, bv[ns], acc[ms][ns], 0, KIND == kMx4 ? 4 : 0, 0, sab, 0, (int)bsc[ns]);
        } else {  // bf16 A: 16 k per lane = two 16x16x32 MFMAs
#pragma unroll
          for (int ns = 0; ns < 4; ++ns) {
            const v4i b0 = v4i{bv[ns][0], bv[ns][1], bv[ns][2], bv[ns][3]};
            const v4i b1 = v4i{bv[ns][4], bv[ns][5], bv[ns][6], bv[ns][7]};
            acc[ms][ns] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(v8bf, a0), __builtin_bit_cast(v8bf, b0), acc[ms][ns], 0, 0, 0);
            acc[ms][ns] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(v8bf, a1), __builtin_bit_cast(v8bf, b1), acc[ms][ns], 0, 0, 0);
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
          if (!__builtin_isfinite(v) && p.err_nonfinite) {
            bad |= kErrNonFinite;
            if (!p.write_nonfinite) continue;
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
    const uint32_t bits = ((bad & kErrCode) ? p.err_code : 0u) | ((bad & kErrScale) ? p.err_scale : 0u) |
                          ((bad & kErrNonFinite) ? p.err_nonfinite : 0u);
    if (bits) atomicOr(p.err, bits);
  }
}

template <int KIND, int SCALE, int OUT, bool MOE, bool CHECK>
void launch_one(const GemmParams& gp, uint32_t grid, hipStream_t s) {
  hipLaunchKernelGGL((mfma_gemm_kernel<KIND, SCALE, OUT, MOE, CHECK>), dim3(grid), dim3(THREADS), 0, s, gp);
}

template <int KIND, int SCALE, int OUT>
void dispatch_mc(const GemmParams& gp, uint32_t grid, hipStream_t s, bool moe, bool check) {
  if (moe) {
    if (check) launch_one<KIND, SCALE, OUT, true, true>(gp, grid, s);
    else launch_one<KIND, SCALE, OUT, true, false>(gp, grid, s);
  } else {
    if (check) launch_one<KIND, SCALE, OUT, false, true>(gp, grid, s);
    else launch_one<KIND, SCALE, OUT, false, false>(gp, grid, s);
  }
}

template <int KIND, int SCALE>
void dispatch_out(const GemmParams& gp, uint32_t grid, hipStream_t s, OutKind out, bool moe, bool check) {
  if (out == kOutBf16) dispatch_mc<KIND, SCALE, kOutBf16>(gp, grid, s, moe, check);
  else if (out == kOutF32) dispatch_mc<KIND, SCALE, kOutF32>(gp, grid, s, moe, check);
  else dispatch_mc<KIND, SCALE, kOutSwiGlu>(gp, grid, s, moe, check);
}

// Shared host setup: tile counts, grid, common fields.
St prepare(GemmParams& gp, uint32_t& grid, uint32_t m, uint32_t n, uint32_t k, uint32_t problems, bool moe,
           OutKind out, uint64_t out_row_stride, uint32_t light_rows = 0) {
  gp.m = m;
  gp.n = n;
  gp.k = k;
  gp.problems = problems;
  gp.n_tiles = n / BN;
  gp.out_row_stride = out_row_stride ? out_row_stride : (out == kOutSwiGlu ? n / 2 : n);
  uint64_t mt;
  gp.light_rows = moe ? light_rows : 0;
  if (moe) {
    // sum_e ceil(rows_e/BM) <= rows/BM + (number of tiled experts), and a
    // tiled expert has more than light_rows rows
    const uint64_t tiled = m / ((uint64_t)light_rows + 1);
    mt = (uint64_t)m / BM + (problems < tiled ? problems : tiled);
    gp.m_tiles_per = 0;
  } else {
    gp.m_tiles_per = (m + BM - 1) / BM;
    mt = (uint64_t)gp.m_tiles_per * problems;
  }
  const uint64_t total = mt * gp.n_tiles;
  if (total > 0x7fffffffull - 8 || (total == 0 && gp.light_rows == 0)) return Invalid("gemm_grid_too_large");
  gp.tiles_total = (uint32_t)total;
  grid = (uint32_t)((total + 7) / 8 * 8);  // 0: every expert is light, nothing to tile
  return RequireCleanLastError();
}

// The tiled and the weight-streaming experts of one MXFP4 MoE launch are
// independent (disjoint output rows; the error word is only OR-ed), so the
// tiled kernel (MFMA work) runs on a per-device auxiliary stream forked from
// the caller's and the streaming kernel (HBM work) on the caller's, joined
// before the entry returns.  The auxiliary stream has the default priority.
// A device's record + wait pairs are serialized, so concurrent callers cannot
// interleave them; a capturing stream keeps both launches on itself.
struct ForkStreams {
  std::mutex mu;
  hipStream_t aux = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  bool broken = false;
};
ForkStreams g_fork[64];

// The current device's fork streams, locked, with the auxiliary stream
// already waiting for the work enqueued on `s`; null (nothing locked) when
// `s` is capturing or the streams cannot be made.
ForkStreams* ForkBegin(hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return nullptr;
  }
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return nullptr;
  }
  ForkStreams& f = g_fork[dev];
  f.mu.lock();
  if (!f.aux && !f.broken) {
    if (hipStreamCreateWithFlags(&f.aux, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&f.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&f.join, hipEventDisableTiming) != hipSuccess) {
      f.broken = true;
      (void)hipGetLastError();
    }
  }
  if (f.broken || hipEventRecord(f.fork, s) != hipSuccess || hipStreamWaitEvent(f.aux, f.fork, 0) != hipSuccess) {
    (void)hipGetLastError();
    f.mu.unlock();
    return nullptr;
  }
  return &f;
}

// Makes `s` wait for the auxiliary stream's work and unlocks.
St ForkEnd(ForkStreams* f, hipStream_t s) {
  St r = Ok();
  if (hipEventRecord(f->join, f->aux) != hipSuccess || hipStreamWaitEvent(s, f->join, 0) != hipSuccess)
    r = Internal("fp4_gemm_stream_join_failed");
  f->mu.unlock();
  return r;
}

}  // namespace

St LaunchFp8BlockGemm(const BlockGemmArgs& a) {
  if (!a.a || !a.a_scale || !a.w || !a.w_scale || !a.out || !a.error_flag || !a.stream)
    return Invalid("fp8_gemm_null_argument");
  if (a.k == 0 || a.k % 128 || a.n == 0 || a.n % 128 || a.problems == 0 || a.m == 0)
    return Invalid("fp8_gemm_shape_invalid");
  if ((a.out_kind == kOutSwiGlu || a.out_kind == kOutSwiGluFp8) && (a.n % 256))
    return Invalid("fp8_gemm_swiglu_shape_invalid");
  if (a.scale_fmt != kScaleF32 && a.scale_fmt != kScaleUe8m0) return Invalid("fp8_gemm_scale_format_invalid");
  if (a.out_kind != kOutBf16 && a.out_kind != kOutF32 && a.out_kind != kOutSwiGlu && a.out_kind != kOutSwiGluFp8)
    return Invalid("fp8_gemm_output_type_invalid");
  // the quantised SwiGLU output exists in the MoE kernel only
  if (a.out_kind == kOutSwiGluFp8 && (!a.moe || a.check_codes || !a.out_scale))
    return Invalid("fp8_gemm_output_type_invalid");
  if (a.moe && !a.offsets) return Invalid("fp8_gemm_offsets_missing");
  if (a.a_rows_total == 0) return Invalid("fp8_gemm_a_rows_invalid");
  if (a.moe && !a.check_codes) return LaunchFp8MoeGemm(a);
  // One large dense problem: the MoE kernel's big tiles.  Their MFMAs do
  // not decode NaN codes as zeros.  With check_codes a persistent launch
  // handles codes in its tiles: a code's NaN reaches every sum over its A
  // or W row, so a block whose sums came out non-finite looks for codes in
  // its operand rows and, finding one, computes itself again the
  // reference's way.  Otherwise a scan raises the code bit first if A or W
  // holds a code, the big-tile kernel then exits at once, and the checking
  // 128 x 128 kernel enqueued after it (which otherwise exits at once)
  // computes the result; a bit set before the call takes the checking
  // kernel too, with the same result.  (With check_codes only one problem
  // of contiguous rows: the tiles then read exactly the bytes the check
  // covers.)
  const bool contiguous1 = a.problems == 1 && a.a_row_stride == 1 && a.a_prob_row == 0 && a.out_prob_col == 0 &&
                           (a.out_row_stride == 0 || a.out_row_stride == a.n) && a.a_rows_total >= a.m;
  const bool dense_ok = !a.moe && !a.a_gather && (a.out_kind == kOutBf16 || a.out_kind == kOutF32) &&
                        (contiguous1 || !a.check_codes) && (uint64_t)a.a_rows_total * a.k <= 0xffffffffull &&
                        (uint64_t)a.n * a.k <= 0xffffffffull;
  // Above 64 rows the big tiles also take what the 128 x 128 kernel took
  // before (more than 256 rows, or too many 128 x 128 tiles for the small-M
  // kernel) and the small-M kernel's 64-row chunks once together they would
  // stream more than 20 MB of weights (each chunk streams all of W).
  // DeepSeek launch_fp8_gemm, K -> N at M rows, us before -> after:
  // 4096 -> 1024 M 384 63 -> 26; 8192 -> 4096 M 128 56 -> 50, M 256 111 ->
  // 50, M 384 122 -> 51; 4096 -> 2048 M 192 30 -> 27, M 512 63 -> 28;
  // 2048 -> 4096 M 256 26 -> 18; 1024 -> 32768 M 100 22 -> 17.  Below
  // those sizes the small-M kernel stays faster (4096 -> 1024 at M 256: 16
  // against 26 us: a big tile's 32 K steps take ~0.8 us each).
  // At 33..64 rows the big tiles also win where the small-M kernel's one
  // pass over W (~1.15 TB/s at 64 rows) takes longer than a round of big
  // tiles (~0.8 us per 128-deep K step + ~5 us): 1024 -> 32768 at M 64,
  // 25 -> 16 us.
  bool big = BigTileWorthIt(a.m, a.n * a.problems);
  const uint64_t w_bytes = (uint64_t)a.n * a.k * a.problems;
  if (a.m > kSmallMChunkRows) {
    const uint64_t chunks = (a.m + kSmallMChunkRows - 1) / kSmallMChunkRows;
    big = big || a.m > kSmallMRows || !SmallMTakes(a.m, a.n, a.problems) || chunks * w_bytes > (20ull << 20);
  } else if (a.m > 32) {
    big = big || w_bytes / 1150 > (uint64_t)(a.k / 128) * 800 + 5000;  // ns
  }
  const bool dense1 = dense_ok && big;
  if (dense1) {
    BigTileArgs b;
    b.a = a.a;
    b.a_scale = a.a_scale;
    b.w = a.w;
    b.w_scale = a.w_scale;
    b.out = a.out;
    b.error_flag = a.error_flag;
    b.stream = a.stream;
    b.m = a.m;
    b.n = a.n;
    b.k = a.k;
    b.problems = a.problems;
    b.a_rows_total = a.a_rows_total;
    b.a_row_stride = a.a_row_stride;
    b.a_prob_row = a.a_prob_row;
    b.out_row_stride = a.out_row_stride;
    b.out_prob_col = a.out_prob_col;
    b.scale_fmt = a.scale_fmt;
    b.out_kind = a.out_kind;
    b.err_code_bit = a.err_code_bit;
    b.err_scale_bit = a.err_scale_bit;
    b.err_nonfinite_bit = a.err_nonfinite_bit;
    b.write_nonfinite = a.write_nonfinite;
    if (!a.check_codes || !a.err_code_bit) return LaunchBigTileGemm(b);
    b.code_check = true;
    bool done = false;
    St s = LaunchBigTileGemm(b, &done);
    if (!s.ok() || done) return s;
  }
  if (!a.moe && a.m <= kSmallMRows && (a.out_kind == kOutBf16 || a.out_kind == kOutF32)) {
    // a few activation rows: weight streaming over 16-row blocks
    bool taken = false;
    St s = LaunchFp8SmallM(a, taken);
    if (!s.ok() || taken) return s;
  }
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
  gp.a_rows_total = a.a_rows_total;
  gp.a_row_stride = a.a_row_stride;
  gp.a_prob_row = a.a_prob_row;
  gp.out_prob_col = a.out_prob_col;
  gp.limit = a.swiglu_limit;
  gp.err_code = a.err_code_bit;
  gp.err_scale = a.err_scale_bit;
  gp.err_nonfinite = a.err_nonfinite_bit;
  gp.write_nonfinite = a.write_nonfinite ? 1u : 0u;
  if (dense1) {  // the checking half (a.check_codes here)
    gp.run_if = a.error_flag;
    gp.run_bit = a.err_code_bit;
  }
  uint32_t grid;
  St s = prepare(gp, grid, a.m, a.n, a.k, a.problems, a.moe, a.out_kind, a.out_row_stride);
  if (!s.ok()) return s;
  if (a.scale_fmt == kScaleF32) dispatch_out<kFp8, kScaleF32>(gp, grid, a.stream, a.out_kind, a.moe, a.check_codes);
  else dispatch_out<kFp8, kScaleUe8m0>(gp, grid, a.stream, a.out_kind, a.moe, a.check_codes);
  return AfterLaunch("fp8_gemm_launch_failed");
}

St LaunchFp4Gemm(const Fp4GemmArgs& a) {
  if (!a.a || !a.w || !a.w_scale || !a.out || !a.error_flag || !a.stream) return Invalid("fp4_gemm_null_argument");
  if (a.act == kActE4m3 && !a.a_scale) return Invalid("fp4_gemm_null_argument");
  if (a.k == 0 || a.k % 128 || a.n == 0 || a.n % 128 || a.problems == 0 || a.m == 0)
    return Invalid("fp4_gemm_shape_invalid");
  if (a.out_kind == kOutSwiGlu && (a.n % 256)) return Invalid("fp4_gemm_swiglu_shape_invalid");
  if (a.out_kind != kOutBf16 && a.out_kind != kOutF32 && a.out_kind != kOutSwiGlu)
    return Invalid("fp4_gemm_output_type_invalid");
  if (a.act != kActE4m3 && a.act != kActBf16) return Invalid("fp4_gemm_activation_type_invalid");
  if (a.moe && !a.offsets) return Invalid("fp4_gemm_offsets_missing");
  if (a.a_rows_total == 0) return Invalid("fp4_gemm_a_rows_invalid");
  // Dense batches above 64 rows the small-M kernel does not take well (more
  // than 256 rows, or 64-row chunks that together would stream more than
  // 40 MB of weights and scales): the big tiles with the FP4 W operand,
  // after a scan that raises the NaN-code bit if A holds a code; they then
  // exit at once, and the checking 128 x 128 kernel enqueued after them
  // (which otherwise exits at once) computes the result.  DeepSeek
  // launch_fp4_gemm, K -> N, us before -> after: 7168 -> 4096 M 256 86 ->
  // 55, M 512 98 -> 56, M 2048 111 -> 77; 4096 -> 2048 M 512 51 -> 30;
  // 2048 -> 4096 M 512 29 -> 21 (M 128 at 7168 -> 4096, two chunks of
  // 15.6 MB, stays on the small-M kernel: 45 against 55 us).
  bool dense_big = false;
  if (a.m > kSmallMChunkRows && Fp4DenseBigTileTakes(a)) {
    const uint64_t w_bytes = (uint64_t)a.n * (a.k / 2) + (uint64_t)a.n * (a.k / 32);
    const uint64_t chunks = (a.m + kSmallMChunkRows - 1) / kSmallMChunkRows;
    dense_big = a.m > kSmallMRows || !SmallMTakes(a.m, a.n, 1) || chunks * w_bytes > (40ull << 20);
  }
  if (dense_big) {
    NanCodeScanArgs sc;
    sc.a = a.a;
    sc.a_bytes = (uint64_t)a.m * a.k;
    sc.w = a.a;  // e2m1 weights hold no NaN code
    sc.w_bytes = 0;
    sc.error_flag = a.error_flag;
    sc.bit = 1u;
    sc.stream = a.stream;
    St s = LaunchNanCodeScan(sc);
    if (!s.ok()) return s;
    if (!(s = LaunchFp4DenseBigTile(a, a.error_flag, 1u)).ok()) return s;
  } else if (!a.moe && a.problems == 1 && a.act == kActE4m3 && a.m <= kSmallMRows &&
             (a.out_kind == kOutBf16 || a.out_kind == kOutF32)) {
    // a few activation rows (the per-expert decode call): weight streaming
    bool taken = false;
    St s = LaunchFp4SmallM(a, taken);
    if (!s.ok() || taken) return s;
  }
  GemmParams gp{};
  gp.a = static_cast<const uint8_t*>(a.a);
  gp.a_scale = a.a_scale;
  gp.a_gather = a.a_gather;
  gp.w = a.w;
  gp.w_scale = a.w_scale;
  gp.out = a.out;
  gp.row_weight = a.row_weight;
  gp.offsets = a.offsets;
  gp.err = a.error_flag;
  gp.a_rows_total = a.a_rows_total;
  gp.a_row_stride = 1;
  gp.limit = a.swiglu_limit;
  gp.err_code = 1u;
  gp.err_scale = 2u;
  gp.err_nonfinite = 4u;
  if (dense_big) {  // the checking half
    gp.run_if = a.error_flag;
    gp.run_bit = 1u;
  }
  // MoE: the light experts go to the weight-streaming kernel, the tiles
  // here cover the others
  uint32_t grid;
  St s = prepare(gp, grid, a.m, a.n, a.k, a.problems, a.moe, a.out_kind, 0, a.moe ? Fp4MoeLightRows(a) : 0);
  if (!s.ok()) return s;
  // every expert within the streaming kernel's rows (a caller's bound): no
  // tiled launch, whose tile scan alone costs ~4-5 us
  const bool all_light = a.moe && a.max_expert_rows && a.max_expert_rows <= Fp4MoeLightRows(a);
  if (grid && !all_light) {
    // The 128 x 256 FP4 tiles and the streaming kernel run one after the
    // other: a big-tile block needs most of a CU's LDS and cannot start on
    // a CU the streaming blocks hold, so forked they overlapped worse than
    // in sequence (512 tokens 800 -> 768 us, 64 tokens 343 -> 305 us).  The
    // 128 x 128 tiles (bf16 activations) fork beside the streaming kernel.
    const bool big = a.moe && Fp4MoeBigTileTakes(a);
    ForkStreams* f = gp.light_rows && !big ? ForkBegin(a.stream) : nullptr;
    const hipStream_t hs = f ? f->aux : a.stream;
    if (big) {
      Fp4GemmArgs big = a;
      big.stream = hs;
      s = LaunchFp4MoeBigTile(big, gp.light_rows);
    } else {
      if (a.act == kActE4m3) dispatch_out<kFp4, kScaleUe8m0>(gp, grid, hs, a.out_kind, a.moe, !a.moe);
      else dispatch_out<kBf16Fp4, kScaleUe8m0>(gp, grid, hs, a.out_kind, a.moe, false);
      s = AfterLaunch("fp4_gemm_launch_failed");
    }
    if (f) {
      if (s.ok()) s = LaunchFp4MoeStream(a);
      const St joined = ForkEnd(f, a.stream);
      return s.ok() ? joined : s;
    }
  }
  if (!s.ok() || gp.light_rows == 0) return s;
  return LaunchFp4MoeStream(a);
}

St LaunchBf16Gemm(const Bf16GemmArgs& a) {
  if (!a.a || !a.w || !a.out || !a.stream) return Invalid("bf16_gemm_null_argument");
  if (a.m == 0 || a.n == 0 || a.k == 0) return Invalid("bf16_gemm_shape_invalid");
  if (a.out_kind != kOutBf16 && a.out_kind != kOutF32) return Invalid("bf16_gemm_output_type_invalid");
  // Batches of 2..255 rows against very wide weights (the LM heads: a round
  // of 256-column tiles without a K split) take the big tiles, which stream
  // the weights once (twice through L2 above 128 rows) with the batch in one
  // M tile, where the GEMV re-reads the batch's rows from L2 for every 16
  // weight rows and the 128 x 128 kernel is MFMA-bound on its small tiles
  // (DeepSeek LM head, 4096 -> 129280: m = 2 186 -> 165 us, m = 16 194 ->
  // 170 us, m = 64 177 us, m = 128 233 -> 186 us, m = 200 364 -> 285 us;
  // m = 1 stays on the GEMV, 159 us).
  const bool wide = a.m >= 2 && a.m < 256 && a.n % 128 == 0 && a.k % 64 == 0 && a.n / 256 >= 192;
  if (a.m <= 64 && !wide) return LaunchBf16Gemv(a);
  if (a.n % 128 || a.k % 64) return Invalid("bf16_gemm_shape_invalid");
  if ((Bf16BigTiles(a.m, a.n, a.k) || wide) && (uint64_t)a.m * a.k * 2 <= 0xffffffffull &&
      (uint64_t)a.n * a.k * 2 <= 0xffffffffull) {
    BigTileArgs b;
    b.a = a.a;
    b.w = a.w;
    b.out = a.out;
    b.stream = a.stream;
    b.m = a.m;
    b.n = a.n;
    b.k = a.k;
    b.bf16 = true;
    b.out_kind = a.out_kind;
    // the GemmPlan contract has no error flag; the LM head passes one for
    // its non-finite-logit bit (the logit is stored either way)
    if (a.error_flag && a.nonfinite_bit) {
      b.error_flag = a.error_flag;
      b.err_code_bit = b.err_scale_bit = 0u;
      b.err_nonfinite_bit = a.nonfinite_bit;
    }
    b.write_nonfinite = true;
    // fewer tiles than CUs: K split into fp32 partial sums in the caller's
    // workspace (sized by Bf16GemmWorkspaceBytes), then summed in split
    // order; the reduce stores 8 or 16 bytes per lane, so the workspace and
    // the output must start on 16-byte boundaries (torch allocations do)
    const uint32_t splits = DenseKSplits(a.m, a.n, a.k / 64);
    const uint64_t ws_bytes = (uint64_t)splits * a.m * a.n * 4;
    const bool aligned =
        reinterpret_cast<uintptr_t>(a.workspace) % 16 == 0 && reinterpret_cast<uintptr_t>(a.out) % 16 == 0;
    if (splits > 1 && a.workspace && a.workspace_bytes >= ws_bytes && aligned) {
      BigTileArgs p = b;
      p.out = a.workspace;
      p.out_kind = kOutF32;
      p.out_row_stride = a.n;
      p.k_splits = splits;
      p.error_flag = nullptr;
      St s = LaunchBigTileGemm(p);
      if (!s.ok()) return s;
      return LaunchSplitKReduce(static_cast<const float*>(a.workspace), splits, a.m, a.n, a.out, a.out_kind,
                                b.error_flag, b.err_nonfinite_bit, a.stream);
    }
    return LaunchBigTileGemm(b);
  }
  GemmParams gp{};
  gp.a = reinterpret_cast<const uint8_t*>(a.a);
  gp.w = reinterpret_cast<const uint8_t*>(a.w);
  gp.out = a.out;
  gp.a_rows_total = a.m;
  gp.a_row_stride = 1;
  uint32_t grid;
  St s = prepare(gp, grid, a.m, a.n, a.k, 1, false, a.out_kind, 0);
  if (!s.ok()) return s;
  // the GemmPlan contract has no error flag; the LM head passes one for its
  // non-finite-logit bit (the logit is stored either way)
  gp.err = a.error_flag && a.nonfinite_bit ? a.error_flag : nullptr;
  gp.err_nonfinite = gp.err ? a.nonfinite_bit : 0u;
  gp.write_nonfinite = 1u;
  if (a.out_kind == kOutBf16) launch_one<kBf16, kScaleUe8m0, kOutBf16, false, false>(gp, grid, a.stream);
  else launch_one<kBf16, kScaleUe8m0, kOutF32, false, false>(gp, grid, a.stream);
  return AfterLaunch("bf16_gemm_launch_failed");
}

St LaunchMx32Gemm(const Mx32GemmArgs& a) {
  if (!a.a || !a.a_scale || !a.w || !a.w_scale || !a.out || !a.error_flag || !a.stream)
    return Invalid("mx32_gemm_null_argument");
  // 128-deep MX steps and 128-row W tiles
  if (a.m == 0 || a.n == 0 || a.k == 0 || a.k % 128 || a.n % 128) return Invalid("mx32_gemm_shape_invalid");
  GemmParams gp{};
  gp.a = a.a;
  gp.a_scale = a.a_scale;
  gp.w = a.w;
  gp.w_scale = a.w_scale;
  gp.out = a.out;
  gp.err = a.error_flag;
  gp.a_rows_total = a.m;
  gp.a_row_stride = 1;
  // V4.1 error bits: 1 for an invalid operand or scale, 2 for a non-finite
  // result, which is stored as the reference stores it
  gp.err_code = 1u;
  gp.err_scale = 1u;
  gp.err_nonfinite = 2u;
  gp.write_nonfinite = 1u;
  uint32_t grid;
  St s = prepare(gp, grid, a.m, a.n, a.k, 1, false, kOutBf16, 0);
  if (!s.ok()) return s;
  if (a.fp4_weight) launch_one<kMx4, kScaleUe8m0, kOutBf16, false, true>(gp, grid, a.stream);
  else launch_one<kMx8, kScaleUe8m0, kOutBf16, false, true>(gp, grid, a.stream);
  return AfterLaunch("mx32_gemm_launch_failed");
}

uint64_t Bf16GemmWorkspaceBytes(uint32_t m, uint32_t n, uint32_t k) {
  if (m <= 64) return Bf16GemvWorkspaceBytes(m, n, k);
  // the big tiles' K split (fp32 partial sums); without this workspace the
  // call runs unsplit
  if (n % 128 || k % 64 || !Bf16BigTiles(m, n, k)) return 0;
  const uint32_t splits = DenseKSplits(m, n, k / 64);
  return splits > 1 ? (uint64_t)splits * m * n * 4 : 0;
}

}  // namespace pih_amd
