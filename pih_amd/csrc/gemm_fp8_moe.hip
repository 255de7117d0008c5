// MoE-segmented FP8 block-scaled grouped GEMM for gfx950, 128 x 256 tiles.
//
//   out[row, :] = A[gather[row], :] . W[e]^T   for the rows of expert e
//
// A e4m3 [a_rows_total, K] with one scale per (A row, 128 k); W e4m3
// [E][N][K] with one scale per (128 W rows, 128 k); scales fp32 or UE8M0
// (reference src/model/deepseek_fp8_gemm_oracle.cpp:10-80 per element; the
// expert segments are the device offsets of the route plan, the reference's
// host plan deepseek_expert_subwave_plan.cpp:32-101).
//
// Design (measured on MI355X; one 16x16x128 FP8 MFMA per 32 clk per SIMD;
// LDS has 64 four-byte banks and serves 16 lanes of a 16-byte access per
// cycle):
//   * one block of 512 threads (8 waves, two per SIMD) per CU owns a tile of
//     128 A rows x 256 W rows; each 128-deep K step moves 48 KB with full
//     128-byte lines (8 lanes per row) straight into LDS by DMA
//     (global_load_lds_dwordx4: no staging registers, no ds_write), as dense
//     128-byte rows whose 16-byte chunk c sits in slot c ^ ((row >> 1) & 7):
//     the 16 rows of one operand-fragment read hit 64 distinct banks;
//   * three LDS stages (149 KB), loads issued two steps ahead, one barrier
//     per step; the DMAs are inline asm and the waits explicit vmcnt counts
//     (seven loads per wave and step), so the compiler adds no waits of its
//     own before LDS reads; tiles with every row block live issue the
//     step's loads between its MFMA groups (issued together after the
//     barrier they stalled the waves' in-order MFMA issue);
//   * the output is computed transposed, C^T = W . A^T: the MFMA's first
//     operand is a 16-row W block and its second a 16-row A block, so a lane
//     owns four consecutive output columns of one row.  That makes the fp32
//     A-row scale a single value per lane and 16-byte block, and the
//     epilogue stores 8 or 16 contiguous bytes per lane;
//   * wave (wm, wn) computes A rows wm*64 + [0,64) against W rows
//     wn*64 + [0,64): 4 x 4 MFMAs of 16x16x128 per K step;
//   * fp32 scales: each MFMA starts from zero and the lane adds
//     t * (a_scale[row] * w_scale[block]) in fp32 (DeepSeek-V3 promotion,
//     bit-identical to the 128x128-tile kernel), software-pipelined so the
//     FMAs of one A block run while the next block's MFMAs execute; UE8M0
//     scales ride in the MFMA's E8M0 operands and the MFMAs chain on the
//     accumulator.
// Tile order: see moe_tile (streaming and multi-tile experts interleaved;
// an 8 M x 4 N grouping of the multi-tile ones cut the L2-miss bytes by
// 9 % but ran 3 % slower than M-fastest groups of 32).
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "device_common.hpp"
#include "kernels.hpp"

namespace pih_amd {
namespace {

constexpr int BM = 128, BN = 256, LDS_ROW = 128, GROUP_M = 32, STAGES = 3;
// eight waves (2 x 4, one 64 x 64 output block each)
constexpr int NCW = 8, NTH = 64 * NCW;
constexpr uint32_t A_BYTES = BM * LDS_ROW, W_BYTES = BN * LDS_ROW, SA_BYTES = 512, SW_BYTES = 256;
constexpr uint32_t STAGE = A_BYTES + W_BYTES + SA_BYTES + SW_BYTES, DUMMY_BYTES = 256;
// s_waitcnt immediates (gfx9 encoding: vmcnt [3:0] and [15:14], expcnt
// [6:4], lgkmcnt [11:8]; an all-ones field does not wait)
constexpr int kWaitVm7 = 0x0F77;     // vmcnt(7)
// operand kinds: e4m3 with block scales, bf16 (no scales), or e4m3 (kOpFp4)
// or bf16 (kOpBf16Fp4) A against MXFP4 W (e2m1 two per byte, UE8M0 per W
// row and 32 k)
enum : int { kOpFp8 = 0, kOpBf16 = 1, kOpFp4 = 2, kOpBf16Fp4 = 3 };
// added to kOutBf16 / kOutF32 in the kernel's output-kind argument: the
// dense FP8 GEMM with the NaN-code check in its tiles
constexpr int kOutCodeCheck = 16;
// static LDS of a block: the FP8 stages (the staged epilogue needs as
// much), or three bf16 x FP4 stages (256-byte A rows), plus the scratch word
template <int OP>
constexpr uint32_t smem_bytes() {
  return (OP == kOpBf16Fp4 ? 3 * (BM * 256 + BN * 64 + BN * 4) : STAGES * STAGE) + DUMMY_BYTES;
}
constexpr int kWaitVm0 = 0x0F70;     // vmcnt(0)
constexpr uint32_t kCodePitch = 144;  // staged e4m3 code rows (128 bytes + 16)
// s_waitcnt immediate waiting for vmcnt <= n (n < 64; bits [3:0] and [15:14])
constexpr int vmcnt_enc(int n) { return ((n >> 4) << 14) | 0x0F70 | (n & 15); }
static_assert(vmcnt_enc(7) == kWaitVm7 && vmcnt_enc(0) == kWaitVm0, "vmcnt encoding");
// stores one lane of a persistent block issues per tile of plain output
constexpr uint32_t kStoreOps = 16;

// LDS byte address of a __shared__ object
// a pointer the caller knows to be wave-uniform, as SGPRs
__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const uint8_t*>(((uint64_t)hi << 32) | lo);
}

// byte offset of 16-byte chunk c of tile row r (XOR-swizzled slots)
__device__ __forceinline__ uint32_t lds_at(uint32_t r, uint32_t c) { return r * LDS_ROW + ((c ^ ((r >> 1) & 7u)) << 4); }

struct MoeParams {
  const uint8_t* a;
  const void* a_scale;
  const uint32_t* a_gather;
  const uint8_t* w;
  const void* w_scale;
  void* out;
  const float* row_weight;
  const uint32_t* offsets;
  uint32_t* err;
  void* out_scale;  // kOutSwiGluFp8: [rows, n / 256] group scales
  uint32_t m, n, k, experts, a_rows_total;
  // dense: `experts` strided problems of m rows each, ceil(m / 128) M tiles
  // per problem (no offsets, no gather; A row i of problem q is
  // i * a_row_stride + q * a_prob_row, its output row starts at
  // i * out_row_stride + q * out_prob_col); 0 for MoE segments
  uint32_t dense_m_tiles;
  // dense: rows per M tile (BM, or 64 / 32 for GEMMs with too few 128-row
  // tiles to fill the CUs: the dead row blocks skip their MFMAs)
  uint32_t dense_tile_rows;
  uint32_t a_row_stride, a_prob_row;
  uint64_t out_prob_col;
  uint32_t write_nonfinite;  // store a non-finite result (and flag it)
  uint32_t stage_out;        // output rows 16-byte aligned: stores staged in LDS
  const uint32_t* skip_if;   // every block exits at once if (*skip_if & skip_bit)
  uint32_t skip_bit;
  // MoE: experts with at most this many rows are left out (another kernel
  // takes them); 0 takes every expert
  uint32_t light_rows;
  uint64_t out_row_stride;
  // dense: > 1 splits K into this many equal parts, each a problem of its
  // own (problem q: K steps [q KB / k_splits, (q + 1) KB / k_splits), the
  // same A rows and W; its fp32 partial sums at output column offset
  // q * out_prob_col); 0 or 1 otherwise
  uint32_t k_splits;
  uint32_t n_tiles;
  uint32_t vb_end;  // blocks of the one-block-per-tile grid; persistent blocks walk no further
  float limit;
  uint32_t err_code, err_scale, err_nonfinite;
};

typedef unsigned int v2u __attribute__((ext_vector_type(2)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v8i cat8(v4i x, v4i y) {
  return v8i{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
}

// Block -> (expert, first row, rows, N tile); false for blocks past the
// last tile.
//
// Tile order.  An expert with one M tile (<= 128 rows) reads each weight
// tile once and is weight-streaming (HBM) work; an expert with more M
// tiles reuses each weight tile across its M tiles and is MFMA work.  Run
// one after the other the two kinds add up (cfg4: 0.62 ms of streaming,
// 1.40 ms of MFMA work), so the tile sequence interleaves them in
// proportion: position t is a streaming tile when floor((t + 1) L / T)
// steps up (L streaming tiles of T), and each XCD (blocks b % 8) walks one
// contiguous range of the sequence, so its CUs run both kinds at once.
// Streaming experts are ordered by expert index, one M tile x all N tiles
// each; multi-tile experts are expert-major, in groups of up to GROUP_M M
// tiles (kTableGroupM in the persistent walk) walked M-fastest, so
// concurrently running tiles share W in L2.
// The per-expert tile counts are scanned by the whole block (wave-level
// shuffle scans plus the eight wave totals).
__device__ bool moe_tile(const MoeParams& p, uint32_t vb, uint32_t& expert, uint32_t& row0, uint32_t& rows,
                         uint32_t& nt) {
  __shared__ uint32_t s_wave[2][NTH / 64];
  __shared__ uint32_t s_res[3];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t E = p.experts, NTL = p.n_tiles;
  const uint32_t per_t = (E + NTH - 1) / NTH;
  auto m_tiles = [&](uint32_t e) -> uint32_t {
    const uint32_t lo = p.offsets[e], hi = p.offsets[e + 1];
    return hi > lo && hi - lo > p.light_rows ? (hi - lo + BM - 1) / BM : 0u;
  };
  uint32_t cnt_h = 0, cnt_s = 0;  // this thread's multi-tile M tiles / streaming experts
  for (uint32_t j = 0; j < per_t; ++j) {
    const uint32_t e = tid * per_t + j;
    if (e < E) {
      const uint32_t c = m_tiles(e);
      cnt_h += c > 1 ? c : 0u;
      cnt_s += c == 1 ? 1u : 0u;
    }
  }
  uint32_t inc_h = cnt_h, inc_s = cnt_s;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t vh = __shfl_up(inc_h, off, 64), vs = __shfl_up(inc_s, off, 64);
    if ((int)lane >= off) inc_h += vh, inc_s += vs;
  }
  if (lane == 63) s_wave[0][wave] = inc_h, s_wave[1][wave] = inc_s;
  if (tid == 0) s_res[0] = 0xffffffffu;
  __syncthreads();
  uint32_t before_h = 0, before_s = 0, tot_h = 0, tot_s = 0;
#pragma unroll
  for (int w = 0; w < NTH / 64; ++w) {
    const uint32_t vh = s_wave[0][w], vs = s_wave[1][w];
    if (w < (int)wave) before_h += vh, before_s += vs;
    tot_h += vh, tot_s += vs;
  }
  inc_h += before_h, inc_s += before_s;
  const uint32_t exc_h = inc_h - cnt_h, exc_s = inc_s - cnt_s;
  const uint64_t Ls = (uint64_t)tot_s * NTL, T = ((uint64_t)tot_h + tot_s) * NTL;
  const uint32_t per = (uint32_t)((T + 7) / 8);
  const uint32_t xcd = vb & 7, jj = vb >> 3;
  const uint64_t t = (uint64_t)xcd * per + jj;
  if (jj >= per || t >= T) return false;  // same for every thread
  const uint32_t s_lo = (uint32_t)(t * Ls / T), s_hi = (uint32_t)((t + 1) * Ls / T);
  const bool streaming = s_hi > s_lo;
  uint32_t mtile = 0;
  if (streaming) {
    // streaming tile s_lo: expert #(s_lo / NTL) among the one-tile experts
    const uint32_t k = s_lo / NTL;
    nt = s_lo % NTL;
    if (k >= exc_s && k < inc_s) {
      uint32_t acc = exc_s;
      for (uint32_t j = 0; j < per_t; ++j) {
        const uint32_t e = tid * per_t + j;
        if (e >= E) break;
        if (m_tiles(e) == 1) {
          if (k == acc) {
            s_res[0] = e;
            break;
          }
          ++acc;
        }
      }
    }
    __syncthreads();
  } else {
    // multi-tile position h = t - s_hi, expert-major over those experts
    const uint32_t h = (uint32_t)(t - s_hi), slot = h / NTL;
    if (slot >= exc_h && slot < inc_h) {
      uint32_t acc = exc_h;
      for (uint32_t j = 0; j < per_t; ++j) {
        const uint32_t e = tid * per_t + j;
        if (e >= E) break;
        const uint32_t c = m_tiles(e);
        if (c > 1) {
          if (slot < acc + c) {
            s_res[0] = e;
            s_res[1] = acc;
            s_res[2] = c;
            break;
          }
          acc += c;
        }
      }
    }
    __syncthreads();
    if (s_res[0] != 0xffffffffu) {
      const uint32_t mbase = s_res[1], mt = s_res[2];
      const uint32_t local = h - mbase * NTL;
      const uint32_t mg = local / (GROUP_M * NTL);
      const uint32_t gsize = min((uint32_t)GROUP_M, mt - mg * GROUP_M);
      const uint32_t r = local - mg * GROUP_M * NTL;
      mtile = mg * GROUP_M + r % gsize;
      nt = r / gsize;
    }
  }
  const uint32_t e = s_res[0];
  if (e == 0xffffffffu) return false;
  const uint32_t lo = p.offsets[e], hi = p.offsets[e + 1];
  if (hi > p.m || lo > hi) {
    if (tid == 0) atomicOr(p.err, p.err_code);
    return false;
  }
  expert = e;
  row0 = lo + mtile * BM;
  rows = min((uint32_t)BM, hi - row0);
  return true;
}

// M tiles per group in the persistent MoE walk and in dense tile maps (8 ran
// the cfg4 down GEMM 2 % and the grouped 8 x 1024 x 4096 GEMM 7 % faster than 32)
constexpr uint32_t kTableGroupM = 8;

// Dense form: tile t of the problems x M x N tile grid (problem-major),
// each XCD (blocks b % 8) walking one contiguous range, M-fastest in groups
// of GROUP_M so that concurrent tiles share their W tile in L2.
__device__ bool dense_tile(const MoeParams& p, uint32_t vb, uint32_t& prob, uint32_t& row0, uint32_t& rows,
                           uint32_t& nt) {
  const uint32_t MT = p.dense_m_tiles, NTL = p.n_tiles;
  const uint64_t per_prob = (uint64_t)MT * NTL, T = per_prob * p.experts;
  const uint32_t per = (uint32_t)((T + 7) / 8);
  const uint32_t xcd = vb & 7, jj = vb >> 3;
  const uint64_t tt = (uint64_t)xcd * per + jj;
  if (jj >= per || tt >= T) return false;
  prob = (uint32_t)(tt / per_prob);
  const uint64_t t = tt - (uint64_t)prob * per_prob;
  const uint32_t mg = (uint32_t)(t / ((uint64_t)kTableGroupM * NTL));
  const uint32_t gsize = min(kTableGroupM, MT - mg * kTableGroupM);
  const uint32_t r = (uint32_t)(t - (uint64_t)mg * kTableGroupM * NTL);
  row0 = (mg * kTableGroupM + r % gsize) * p.dense_tile_rows;
  nt = r / gsize;
  rows = min(p.dense_tile_rows, p.m - row0);
  return true;
}

// Persistent blocks (one per CU, each walking the tiles vb = blockIdx.x,
// blockIdx.x + gridDim.x, ... of the sequence moe_tile defines) find their
// tiles in a per-block LDS table instead: the experts' row offsets and the
// inclusive counts of multi-tile M tiles and of one-tile experts, built
// once, so a lookup is a binary search in LDS (no global read, no barrier).
constexpr uint32_t kTableExperts = 1024;
struct MoeTable {
  uint32_t* off;    // [E + 1] row offsets
  uint32_t* inc_h;  // [E] M tiles of the multi-tile experts 0..e
  uint32_t* inc_s;  // [E] one-tile experts among 0..e
};

__device__ __forceinline__ void moe_table_build(const MoeParams& p, const MoeTable& t) {
  __shared__ uint32_t s_wave[2][NTH / 64];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, E = p.experts;
  for (uint32_t e = tid; e <= E; e += NTH) t.off[e] = p.offsets[e];
  __syncthreads();
  const uint32_t per_t = (E + NTH - 1) / NTH;
  auto m_tiles = [&](uint32_t e) -> uint32_t {
    const uint32_t lo = t.off[e], hi = t.off[e + 1];
    return hi > lo && hi - lo > p.light_rows ? (hi - lo + BM - 1) / BM : 0u;
  };
  uint32_t cnt_h = 0, cnt_s = 0;
  for (uint32_t j = 0; j < per_t; ++j) {
    const uint32_t e = tid * per_t + j;
    if (e < E) {
      const uint32_t c = m_tiles(e);
      cnt_h += c > 1 ? c : 0u;
      cnt_s += c == 1 ? 1u : 0u;
    }
  }
  uint32_t inc_h = cnt_h, inc_s = cnt_s;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t vh = __shfl_up(inc_h, o, 64), vs = __shfl_up(inc_s, o, 64);
    if ((int)lane >= o) inc_h += vh, inc_s += vs;
  }
  if (lane == 63) s_wave[0][wave] = inc_h, s_wave[1][wave] = inc_s;
  __syncthreads();
  uint32_t acc_h = inc_h - cnt_h, acc_s = inc_s - cnt_s;
#pragma unroll
  for (int w = 0; w < NTH / 64; ++w)
    if (w < (int)wave) acc_h += s_wave[0][w], acc_s += s_wave[1][w];
  for (uint32_t j = 0; j < per_t; ++j) {
    const uint32_t e = tid * per_t + j;
    if (e < E) {
      const uint32_t c = m_tiles(e);
      acc_h += c > 1 ? c : 0u;
      acc_s += c == 1 ? 1u : 0u;
      t.inc_h[e] = acc_h;
      t.inc_s[e] = acc_s;
    }
  }
  __syncthreads();
}

// first e < E with inc[e] > k (inc non-decreasing)
__device__ __forceinline__ uint32_t first_above(const uint32_t* inc, uint32_t E, uint32_t k) {
  uint32_t lo = 0, hi = E;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (inc[mid] > k) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}

// moe_tile's mapping, read from the table; a tile of an invalid segment
// raises the code bit and has no rows
__device__ bool moe_table_tile(const MoeParams& p, const MoeTable& t, uint32_t vb, uint32_t& expert, uint32_t& row0,
                               uint32_t& rows, uint32_t& nt, uint32_t& bad) {
  const uint32_t E = p.experts, NTL = p.n_tiles;
  const uint32_t tot_h = t.inc_h[E - 1], tot_s = t.inc_s[E - 1];
  const uint64_t Ls = (uint64_t)tot_s * NTL, T = ((uint64_t)tot_h + tot_s) * NTL;
  const uint32_t per = (uint32_t)((T + 7) / 8);
  const uint32_t xcd = vb & 7, jj = vb >> 3;
  const uint64_t tt = (uint64_t)xcd * per + jj;
  if (jj >= per || tt >= T || vb >= p.vb_end) return false;
  const uint32_t s_lo = (uint32_t)(tt * Ls / T), s_hi = (uint32_t)((tt + 1) * Ls / T);
  uint32_t e, mtile = 0;
  if (s_hi > s_lo) {
    e = first_above(t.inc_s, E, s_lo / NTL);
    nt = s_lo % NTL;
  } else {
    const uint32_t h = (uint32_t)(tt - s_hi), slot = h / NTL;
    e = first_above(t.inc_h, E, slot);
    if (e < E) {
      const uint32_t c = t.inc_h[e] - (e ? t.inc_h[e - 1] : 0u), mbase = t.inc_h[e] - c;
      const uint32_t local = h - mbase * NTL;
      const uint32_t mg = local / (kTableGroupM * NTL);
      const uint32_t gsize = max(1u, min(kTableGroupM, c - mg * kTableGroupM));
      const uint32_t r = local - mg * kTableGroupM * NTL;
      mtile = mg * kTableGroupM + r % gsize;
      nt = r / gsize;
    }
  }
  // Offsets that are not non-decreasing within [0, m] can make the counts
  // wrap and the table non-monotone: a tile whose rows do not lie inside
  // one valid segment raises the code bit, has no rows and reads expert 0.
  const uint32_t lo = e < E ? t.off[e] : 0u, hi = e < E ? t.off[e + 1] : 0u;
  const uint64_t r0 = lo + (uint64_t)mtile * BM;
  if (e >= E || hi > p.m || lo > hi || r0 >= hi || nt >= NTL) {
    bad |= kErrCode;
    expert = 0;
    row0 = 0;
    rows = 0;
    nt = 0;
    return true;
  }
  expert = e;
  row0 = (uint32_t)r0;
  rows = min((uint32_t)BM, hi - row0);
  return true;
}

// OUT_ARG: the output kind, or kOutBf16 / kOutF32 + kOutCodeCheck for the
// dense FP8 GEMM with the reference's NaN-code check in its persistent tiles
// (CODES): an e4m3 NaN code (0x7F / 0xFF) decodes to NaN in the MFMA, so
// every sum over its A row or W row is NaN; a wave whose 64 x 64 block holds
// a non-finite value looks for codes in the A and W rows that feed it and
// raises the code bit instead of the non-finite bit when it finds one.  The
// launch is followed by the checking 128 x 128 kernel, which runs when the
// bit is set (decoding codes as zeros, as the reference does) and rewrites
// every output.
template <int OP, int SCALE, int OUT_ARG, bool PERSIST>
__global__ __launch_bounds__(NTH, 1) void fp8_moe_gemm_kernel(MoeParams p) {
  constexpr bool CODES = OUT_ARG > kOutCodeCheck;
  constexpr int OUT = CODES ? OUT_ARG - kOutCodeCheck : OUT_ARG;
  static_assert(!CODES || (OP == kOpFp8 && PERSIST && (OUT == kOutBf16 || OUT == kOutF32)), "code check: dense FP8");
  // Stage s at smem + s * STG: A tile, W tile, A-row scales, W scales.
  // (FP4 W: 64-byte tile rows and 4 scale bytes per W row; the array keeps
  // the FP8 size, which the staged epilogue also needs.)
  __shared__ __align__(16) uint8_t smem[smem_bytes<OP>()];
  constexpr bool kF4 = OP == kOpFp4, kBF4 = OP == kOpBf16Fp4, kW4 = kF4 || kBF4;
  // A: 128 bytes of a row per step (256 for bf16 x FP4: 128 k per step);
  // W: 128 bytes (64 for FP4); A-row scales (none for bf16); W scales
  constexpr uint32_t A_ROW = kBF4 ? 256 : LDS_ROW, AB = BM * A_ROW;
  constexpr uint32_t W_ROW = kW4 ? 64 : LDS_ROW, WB = BN * W_ROW, SAB = kBF4 ? 0 : SA_BYTES;
  constexpr uint32_t SWB = kW4 ? BN * 4 : SW_BYTES;
  constexpr uint32_t STG = AB + WB + SAB + SWB;
  static_assert(PERSIST ? STG <= STAGE : 3 * STG + DUMMY_BYTES <= sizeof(smem), "stage layout");
  // LDS stages: 4 for FP4 W outside persistent launches (its stage is
  // 33.5 KB: the loads run three steps ahead), 3 otherwise; the scratch
  // word of the dummy scale loads follows the last stage
  constexpr uint32_t NS = kF4 && !PERSIST ? 4 : 3;
  static_assert(NS * STG + DUMMY_BYTES <= sizeof(smem), "stages fit");
  const uint32_t lds0 = lds_addr(smem);

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t lr = lane & 15, lg = lane >> 4;
  const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t wm = (wv >> 2) & 1u, wn = wv & 3u;
  constexpr bool kSwi = OUT == kOutSwiGlu || OUT == kOutSwiGluFp8;  // gate/up pairs in the tile

  // the masked bit is not changed while this kernel runs: one value for every thread
  if (p.skip_if && (__hip_atomic_load(p.skip_if, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & p.skip_bit)) return;

  // a K step is 128 bytes of an A row: 128 e4m3 or 64 bf16 values (bf16 x
  // FP4: 256 bytes, 128 values), and 64 bytes of an FP4 W row
  constexpr bool kBf = OP == kOpBf16;
  const uint32_t K = p.k, RB = kBf || kBF4 ? 2 * K : K, KBt = kBF4 ? K / 128 : RB / 128, RBW = kW4 ? K / 2 : RB;
  // K steps per tile (a K split's share with dense k_splits: bf16 only, so
  // that the other operand kinds carry no split state in their registers)
  constexpr bool kSplitOk = kBf;
  const bool ksplit = kSplitOk && p.dense_m_tiles && p.k_splits > 1;
  const uint32_t KB = ksplit ? KBt / p.k_splits : KBt;
  uint32_t bad = 0;

  [[maybe_unused]] MoeTable tab{};
  if constexpr (PERSIST) {
    __shared__ uint32_t s_off[kTableExperts + 1], s_inc_h[kTableExperts], s_inc_s[kTableExperts];
    tab = MoeTable{s_off, s_inc_h, s_inc_s};
    if (!p.dense_m_tiles) moe_table_build(p, tab);
  }
  // tile vb of the block sequence: expert (problem), first row, rows, N tile
  auto find_tile = [&](uint32_t vb, uint32_t& e, uint32_t& r0, uint32_t& rs, uint32_t& t) -> bool {
    bool ok;
    if (p.dense_m_tiles) ok = dense_tile(p, vb, e, r0, rs, t);
    else if constexpr (PERSIST) ok = moe_table_tile(p, tab, vb, e, r0, rs, t, bad);
    else ok = moe_tile(p, vb, e, r0, rs, t);
    e = __builtin_amdgcn_readfirstlane(e);
    r0 = __builtin_amdgcn_readfirstlane(r0);
    rs = __builtin_amdgcn_readfirstlane(rs);
    t = __builtin_amdgcn_readfirstlane(t);
    return ok;
  };
  uint32_t vb = blockIdx.x, expert = 0, row0 = 0, rows = 0, nt = 0;
  if (!find_tile(vb, expert, row0, rows, nt)) return;

  // Rows past the tile's end (and rejected gather indices) read A row 0:
  // loads stay unconditional and in bounds, and the output rows they feed
  // are never stored (an output row depends on its own A row only).
  // (Persistent launches have no gather: the next tile's rows are known
  // without a global read.)
  auto a_source = [&](uint32_t r, uint32_t e, uint32_t r0, uint32_t rs) -> uint64_t {
    if (r >= rs) return 0;
    const uint32_t logical = r0 + r;
    uint64_t src;
    if (p.dense_m_tiles) src = (uint64_t)logical * p.a_row_stride + (uint64_t)e * p.a_prob_row;
    else if constexpr (PERSIST) src = logical;
    else src = p.a_gather ? p.a_gather[logical] : logical;
    if (src >= p.a_rows_total) {
      bad |= kErrCode;
      return 0;
    }
    return src;
  };
  // W tile row R: for SwiGLU, wave block R >> 6 holds 32 gate rows (R & 63
  // below 32) and the 32 matching up rows, so each wave owns gate/up pairs
  auto w_row = [&](uint32_t R, uint32_t t) -> uint32_t {
    if constexpr (kSwi) {
      const uint32_t wb = R >> 6, j = (R & 63) >> 4, rr = R & 15;
      const uint32_t base = t * 128 + wb * 32 + (j & 1) * 16 + rr;
      return j >= 2 ? p.n / 2 + base : base;
    } else {
      const uint32_t row = t * BN + R;
      return row < p.n ? row : p.n - 1;
    }
  };
  constexpr uint32_t ESZ = SCALE == kScaleUe8m0 ? 1 : 4;

  // Operand tiles move global -> LDS by DMA
  // (global_load_lds_dwordx4): an instruction lands lane l's 16 bytes at
  // byte 16 l of a wave-uniform 1 KB window, i.e. tile row 8q + (l >> 3),
  // slot l & 7 of window q, so lane l fetches chunk (l & 7) ^ ((row >> 1) & 7)
  // of that row (full 128-byte lines per 8 lanes).  Wave w fills A rows
  // [16w, 16w + 16) and W rows [32w, 32w + 32) of a stage.
  const uint32_t lrow = lane >> 3, lslot = lane & 7;
  // Scales (one dword DMA per wave and step, so every compute wave issues
  // seven loads per step): waves 0 and 1 fetch the A-row scales of rows
  // 64w + (l & 3) * 16 + (l >> 2) into word 64w + l of the stage's scale
  // block (a lane's four A-row scales are then one 16-byte read); wave 2
  // the two W block scales (lane l: block l & 1); waves 3..7 repeat wave
  // 2's load into the scratch word.  UE8M0 bytes come in their aligned
  // dword and are picked out by byte offset.  bf16 operands have no scales
  // (six loads per step).
  struct Ops {
    uint32_t a_off[4], w_off[4];  // byte offsets from the operand bases
    const uint8_t* w_base;        // the expert's (problem's) W
    const uint8_t* s_src;         // this lane's scale source at k step 0
    uint64_t ws_off[2];           // the tile's two W scale blocks (entries)
    uint32_t kb0;                 // the tile's first K step (its K split's)
  };
  // A: a_rows_total rows and W: n rows per expert stay below 2^32 bytes,
  // which the launcher checks
  auto make_ops = [&](uint32_t e, uint32_t r0, uint32_t rs, uint32_t t, Ops& o) __attribute__((always_inline)) {
    o.w_base = ksplit ? p.w : p.w + (uint64_t)e * p.n * RBW;
    if constexpr (kSplitOk) o.kb0 = ksplit ? e * KB : 0u;
    else o.kb0 = 0u;
    // the tile's two 128-row W scale blocks (SwiGLU: gate block, up block)
    uint32_t wblk0, wblk1;
    if constexpr (kSwi) {
      wblk0 = t;
      wblk1 = (p.n / 2 + t * 128) / 128;
    } else {
      wblk0 = min(2 * t, p.n / 128 - 1);
      wblk1 = min(2 * t + 1, p.n / 128 - 1);
    }
    const uint32_t we = ksplit ? 0u : e;
    o.ws_off[0] = ((uint64_t)we * (p.n / 128) + wblk0) * KBt;
    o.ws_off[1] = ((uint64_t)we * (p.n / 128) + wblk1) * KBt;
    if constexpr (kBF4) {
      // 256-byte rows: instruction i lands rows 16 wv + 4 i + (l >> 4), slot
      // l & 15, which holds chunk (l & 15) ^ (row & 15)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t R = 16 * wv + 4 * i + (lane >> 4);
        o.a_off[i] = (uint32_t)(a_source(R, e, r0, rs) * RB) + (((lane & 15u) ^ (R & 15u)) << 4);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t R = 16 * wv + 8 * i + lrow;
        o.a_off[i] = (uint32_t)(a_source(R, e, r0, rs) * RB) + ((lslot ^ ((R >> 1) & 7u)) << 4);
      }
      o.a_off[2] = o.a_off[3] = 0;
    }
    if constexpr (kW4) {
      // 64-byte rows: instruction i lands rows 32 wv + 16 i + (l >> 2), slot
      // l & 3, which holds chunk (l & 3) ^ ((row >> 2) & 3)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t R = 32 * wv + 16 * i + (lane >> 2);
        o.w_off[i] = w_row(R, t) * RBW + (((lane & 3u) ^ ((R >> 2) & 3u)) << 4);
      }
      o.w_off[2] = o.w_off[3] = 0;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t R = 32 * wv + 8 * i + lrow;
        o.w_off[i] = w_row(R, t) * RB + ((lslot ^ ((R >> 1) & 7u)) << 4);
      }
    }
    o.s_src = nullptr;
    if constexpr (kW4) {
      // waves 0, 1: A-row scales as for FP8 (bf16 A: a dummy word); waves
      // 2..5: the 4 scale bytes of W tile row 64 (w - 2) + l per step;
      // waves 6, 7: a dummy word
      // (the dummy words read the first W scale bytes: in bounds)
      if (wv >= 2 && wv < 6) {
        const uint32_t R = 64 * (wv - 2) + lane;
        o.s_src = static_cast<const uint8_t*>(p.w_scale) + ((uint64_t)e * p.n + w_row(R, t)) * (K / 32);
      } else if (kF4 && wv < 2) {
        const uint64_t src = a_source(64 * wv + (lane & 3) * 16 + (lane >> 2), e, r0, rs);
        o.s_src = static_cast<const uint8_t*>(p.a_scale) + src * KBt;
      } else {
        o.s_src = static_cast<const uint8_t*>(p.w_scale);
      }
    } else if constexpr (!kBf) {
      if (wv < 2) {
        const uint64_t src = a_source(64 * wv + (lane & 3) * 16 + (lane >> 2), e, r0, rs);
        o.s_src = static_cast<const uint8_t*>(p.a_scale) + src * KBt * ESZ;
      } else {
        o.s_src = static_cast<const uint8_t*>(p.w_scale) + ((lane & 1) ? o.ws_off[1] : o.ws_off[0]) * ESZ;
      }
    }
  };
  uint32_t s_lds = 0;
  if constexpr (kW4) s_lds = wv < 2 ? AB + WB + 256 * wv : AB + WB + SAB + 256 * (wv - 2);
  else if constexpr (!kBf) s_lds = wv < 2 ? A_BYTES + W_BYTES + 256 * wv : A_BYTES + W_BYTES + SA_BYTES;
  s_lds = __builtin_amdgcn_readfirstlane(s_lds);
  const bool s_scratch = kW4 ? wv >= 6 || (kBF4 && wv < 2) : wv > 2;
  // per-step advance of the scale source: 4 bytes for FP4 W-scale rows
  const uint32_t s_step = kW4 && wv >= 2 && wv < 6 ? 4u : ESZ;
  const uint32_t a_lds = __builtin_amdgcn_readfirstlane(wv * (16 * A_ROW)),
                 w_lds = __builtin_amdgcn_readfirstlane(AB + wv * (32 * W_ROW));
  // A step's loads of one wave, in a fixed order: A rows (kNA), W rows
  // (kNW), then the scale dword (none for bf16).  issue_part issues load
  // `part` alone (parts past the last do nothing), issue all of them.
  constexpr int kNA = kBF4 ? 4 : 2, kNW = kW4 ? 2 : 4, kNLoads = kNA + kNW + (kBf ? 0 : 1);
  auto issue_part = [&](uint32_t stage, uint32_t kbl, const Ops& o, auto NT, int part) __attribute__((always_inline)) {
    const uint32_t base = lds0 + stage * STG, kb = kSplitOk ? kbl + o.kb0 : kbl;
    if (part < kNA) {
      dma16(uniform_ptr(p.a + (uint64_t)kb * A_ROW), o.a_off[part], base + a_lds + part * 1024);
    } else if (part < kNA + kNW) {
      const uint8_t* wb = uniform_ptr(o.w_base + (uint64_t)kb * W_ROW);
      const int i = part - kNA;
      if constexpr (decltype(NT)::value) dma16nt(wb, o.w_off[i], base + w_lds + i * 1024);
      else dma16(wb, o.w_off[i], base + w_lds + i * 1024);
    } else if (part < kNLoads) {
      // scales: a per-lane pointer (UE8M0 bytes come in their aligned dword)
      uintptr_t sp = reinterpret_cast<uintptr_t>(o.s_src) + (uint64_t)kb * s_step;
      if constexpr (ESZ == 1) sp &= ~uintptr_t(3);
      dma4v(reinterpret_cast<const void*>(sp), s_scratch ? lds0 + NS * STG : base + s_lds);
    }
  };
  auto issue = [&](uint32_t stage, uint32_t kb, const Ops& o, auto NT) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < kNLoads; ++q) issue_part(stage, kb, o, NT, q);
  };

  Ops cur;
  make_ops(expert, row0, rows, nt, cur);
  const uint32_t last = KB - 1;
  issue(0, 0, cur, std::false_type{});
  issue(1, min(1u, last), cur, std::false_type{});
  if constexpr (NS == 4) issue(2, min(2u, last), cur, std::false_type{});
  // Persistent blocks: the epilogue's kStoreOps stores of one tile follow
  // the next tile's first two steps' loads, so those two steps wait with
  // vmcnt(loads per step + kStoreOps); the first tile gets as many loads
  // (into the scratch bytes) in place of stores.
  if constexpr (PERSIST) {
#pragma unroll
    for (uint32_t i = 0; i < kStoreOps; ++i) dma4(p.w, lane * 4u, lds0 + NS * STG);
  }
  uint32_t rot = 0;  // stage of the tile's step 0 (persistent blocks)

  for (;;) {
  // ---- one tile: the next one's operands (persistent blocks) are read
  // in this tile's last two steps
  uint32_t e2 = expert, r2 = row0, rs2 = rows, t2 = nt;
  bool has_next = false;
  if constexpr (PERSIST) {
    has_next = __builtin_amdgcn_readfirstlane(find_tile(vb + gridDim.x, e2, r2, rs2, t2) ? 1u : 0u) != 0;
    if (!has_next) e2 = expert, r2 = row0, rs2 = rows, t2 = nt;
  }
  Ops nxt;
  // byte offsets of this lane's UE8M0 A scales (rows wm*64 + r*16 + lr) and
  // of the W block scales within their aligned dwords, at k step 0
  uint32_t a_byte0[4] = {0, 0, 0, 0}, w_byte0[2] = {0, 0};
  if constexpr (ESZ == 1) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      a_byte0[r] = (uint32_t)((reinterpret_cast<uintptr_t>(p.a_scale) +
                               a_source(wm * 64 + r * 16 + lr, expert, row0, rows) * KBt) &
                              3u);
    w_byte0[0] = (uint32_t)((reinterpret_cast<uintptr_t>(p.w_scale) + cur.ws_off[0]) & 3u);
    w_byte0[1] = (uint32_t)((reinterpret_cast<uintptr_t>(p.w_scale) + cur.ws_off[1]) & 3u);
  }
  // live 16-row blocks of this wave's 64-row half
  const uint32_t rb_live =
      __builtin_amdgcn_readfirstlane(rows > wm * 64 ? min(4u, (rows - wm * 64 + 15) / 16) : 0u);

  v4f acc[4][4];  // [W block nb][A block rb]
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = v4f{0.f, 0.f, 0.f, 0.f};

  // compute(stage, kb, FULL, dmas): one K step; dmas(q) issues load q of a
  // later step (q = 0 .. 7; a no-op past the step's loads), called between
  // the MFMA groups so that the loads queue while the matrix pipe works
  auto compute = [&](uint32_t stage, uint32_t kb, auto FULL, auto&& dmas) __attribute__((always_inline)) {
    constexpr bool kFull = decltype(FULL)::value;
    if (!kFull && rb_live == 0) {
#pragma unroll
      for (int q = 0; q < 8; ++q) dmas(q);
      return;
    }
    const uint8_t* sA = smem + stage * STG;
    const uint8_t* sB = sA + AB;
    const uint32_t* sS = reinterpret_cast<const uint32_t*>(sB + WB);
    // operand fragments: lane (lr, lg) holds row lr, bytes [16lg, 16lg+16)
    // and [64+16lg, 64+16lg+16) of the step (the same map for both); the
    // fragment rows start at multiples of 16, so the slot of chunk lg is
    // lg ^ (lr >> 1) and that of chunk lg + 4 is the same slot ^ 4
    const uint32_t rd0 = (lg ^ (lr >> 1)) << 4;
    v8i wf[4];
    [[maybe_unused]] uint32_t wsc[4];
    [[maybe_unused]] v4i wlo[4];
    if constexpr (kW4) {
      // FP4 W (the MFMA's first operand, e2m1): lane (lr, lg) holds the 16
      // bytes = 32 k [32 lg, 32 lg + 32) of the step of row lr, in slot
      // lg ^ ((lr >> 2) & 3) of the 64-byte row, and that block's scale byte
      const uint8_t* sW8 = reinterpret_cast<const uint8_t*>(sS) + SAB;  // [BN rows][4 B]
      const uint32_t rdf = (lg ^ ((lr >> 2) & 3u)) << 4;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const uint32_t row = wn * 64 + nb * 16 + lr;
        wlo[nb] = *reinterpret_cast<const v4i*>(sB + row * 64 + rdf);
        wsc[nb] = sW8[row * 4 + lg];
      }
    } else {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const uint8_t* pb = sB + (wn * 64 + nb * 16 + lr) * LDS_ROW;
        wf[nb] = cat8(*reinterpret_cast<const v4i*>(pb + rd0), *reinterpret_cast<const v4i*>(pb + (rd0 ^ 64)));
      }
    }
    const v4i sa4 = *reinterpret_cast<const v4i*>(sS + wm * 64 + lr * 4);
    // W block scales of this wave's columns: SwiGLU gate (block 0) and up
    // (block 1); otherwise the 128-row block holding columns wn*64 ..
    constexpr bool kSw = kSwi;
    const uint32_t wsel0 = kSw ? 0u : (wn >> 1), wsel1 = kSw ? 1u : (wn >> 1);
    const uint32_t sw0 = sS[128 + wsel0], sw1 = sS[128 + wsel1];
    auto a_frag = [&](int r) -> v8i {
      const uint8_t* pa = sA + (wm * 64 + r * 16 + lr) * LDS_ROW;
      return cat8(*reinterpret_cast<const v4i*>(pa + rd0), *reinterpret_cast<const v4i*>(pa + (rd0 ^ 64)));
    };
    auto live = [&](int r) { return kFull || r < (int)rb_live; };
    if constexpr (kBf) {
      // bf16: the 128-byte step is 64 k; the fragment's first 16 bytes (k
      // 8lg .. 8lg+7) feed one 16x16x32 MFMA and its last 16 (k 32+8lg ..)
      // the second, the same split for both operands
      auto mma = [&](int r, const v8i& af) __attribute__((always_inline)) {
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          const v4i w0{wf[nb][0], wf[nb][1], wf[nb][2], wf[nb][3]}, w1{wf[nb][4], wf[nb][5], wf[nb][6], wf[nb][7]};
          const v4i a0{af[0], af[1], af[2], af[3]}, a1{af[4], af[5], af[6], af[7]};
          acc[nb][r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, w0),
                                                               __builtin_bit_cast(v8bf, a0), acc[nb][r], 0, 0, 0);
          acc[nb][r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, w1),
                                                               __builtin_bit_cast(v8bf, a1), acc[nb][r], 0, 0, 0);
        }
      };
      v8i af = a_frag(0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (live(r)) {
          const v8i afn = a_frag(r < 3 ? r + 1 : 3);
          mma(r, af);
          af = afn;
        }
        __builtin_amdgcn_sched_barrier(0);
        dmas(2 * r);
        dmas(2 * r + 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if constexpr (SCALE == kScaleF32) {
      // fp32 scales: each MFMA starts from zero and its result is added
      // with one FMA per output.  Software-pipelined: the four MFMAs of A
      // block r + 1 are issued before the FMAs of block r, so those read
      // results that finished while the next MFMAs ran (consuming a result
      // right after its MFMA stalls the wave for the MFMA's latency).
      const float fw0 = __uint_as_float(sw0), fw1 = __uint_as_float(sw1);
      // group `slot` of four MFMAs issues loads 2 slot and 2 slot + 1 after
      // its second and fourth MFMA (one load per two MFMAs ran 0-2 % faster
      // than one per group of four)
      auto mfma4 = [&](const v8i& af, v4f (&t)[4], int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          t[nb] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf[nb], af, v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0,
                                                                   127, 0, 127);
          if (nb & 1) {
            __builtin_amdgcn_sched_barrier(0);
            dmas(2 * slot + (nb >> 1));
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      };
      auto fma4 = [&](int r, const v4f (&t)[4]) __attribute__((always_inline)) {
        const float sa = __uint_as_float((uint32_t)sa4[r]);
        const float c0 = sa * fw0, c1 = sa * fw1;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          const float c = (kSwi && nb >= 2) ? c1 : c0;
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[nb][r][i] = __builtin_fmaf(t[nb][i], c, acc[nb][r][i]);
        }
      };
      // A fragments are read one block ahead
      v4f tA[4], tB[4];
      v8i af = a_frag(0), afn = a_frag(1);
      mfma4(af, tA, 0);
      __builtin_amdgcn_sched_barrier(0);
      af = a_frag(2);
      if (live(1)) mfma4(afn, tB, 1);
      __builtin_amdgcn_sched_barrier(0);
      fma4(0, tA);
      afn = a_frag(3);
      __builtin_amdgcn_sched_barrier(0);
      if (live(2)) mfma4(af, tA, 2);
      __builtin_amdgcn_sched_barrier(0);
      if (live(1)) fma4(1, tB);
      __builtin_amdgcn_sched_barrier(0);
      if (live(3)) mfma4(afn, tB, 3);
      __builtin_amdgcn_sched_barrier(0);
      if (live(2)) fma4(2, tA);
      __builtin_amdgcn_sched_barrier(0);
      if (live(3)) fma4(3, tB);
    } else if constexpr (kBF4) {
      // bf16 A against MXFP4 W: 4 x 4 x 4 MFMAs 16x16x32 bf16 per step.
      // MFMA q takes, in lane group lg, k [32 lg + 8 q, +8): dword q of the
      // W lane's 16 bytes (8 e2m1 values of block lg, converted exactly to
      // bf16 times 2^(s-127), one byte per v_cvt_scalef32_pk_bf16_fp4) and
      // chunk 4 lg + q of the A row (slot (4 lg + q) ^ lr of its 256 bytes).
      // A 255 W scale raises the scale bit (the block's products are then
      // not finite, as in the 128 x 128 tile kernel).
      typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
      float wsf[4];
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        bad |= wsc[nb] == 0xffu ? (uint32_t)kErrScale : 0u;
        wsf[nb] = ue8m0_value(wsc[nb]);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v4i wq[4];
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          const uint32_t wd = (uint32_t)wlo[nb][q];
          wq[nb] = v4i{__builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, wsf[nb], 0)),
                       __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, wsf[nb], 1)),
                       __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, wsf[nb], 2)),
                       __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, wsf[nb], 3))};
        }
        const uint32_t slot = ((4 * lg + q) ^ lr) << 4;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (live(r)) {
            const v4i av = *reinterpret_cast<const v4i*>(sA + (wm * 64 + r * 16 + lr) * A_ROW + slot);
#pragma unroll
            for (int nb = 0; nb < 4; ++nb)
              acc[nb][r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, wq[nb]),
                                                                   __builtin_bit_cast(v8bf, av), acc[nb][r], 0, 0, 0);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        dmas(2 * q);
        dmas(2 * q + 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if constexpr (kF4) {
      // e4m3 A against MXFP4 W: both UE8M0 scales ride in the instruction
      // (the W lane's own 32-k block scale, the A row's 128-k scale) and the
      // MFMAs chain on the accumulator.  A 255 scale raises the scale bit and
      // its block adds nothing, as in the 128 x 128 tile kernel: the
      // fragment becomes zeros with scale 127.
      // (branch-free: a wave-uniform branch around these selects made the
      // compiler keep copies of every fragment and spill)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const bool ff = wsc[nb] == 0xffu;
        bad |= ff ? (uint32_t)kErrScale : 0u;
        const int keep = ff ? 0 : -1;
        wlo[nb] &= v4i{keep, keep, keep, keep};
        wsc[nb] = ff ? 127u : wsc[nb];
      }
      auto mma = [&](int r, v8i af) {
        uint32_t sb = ((uint32_t)sa4[r] >> (8 * ((a_byte0[r] + kb) & 3u))) & 0xffu;
        const bool aff = sb == 0xffu;
        if (__builtin_amdgcn_ballot_w64(aff)) {
          if (aff) {
            bad |= kErrScale;
            sb = 127;
            af = v8i{0, 0, 0, 0, 0, 0, 0, 0};
          }
        }
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
          acc[nb][r] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(cat8(wlo[nb], v4i{0, 0, 0, 0}), af,
                                                                       acc[nb][r], 4, 0, 0, (int)wsc[nb], 0, (int)sb);
      };
      v8i af = a_frag(0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (live(r)) {
          const v8i afn = a_frag(r < 3 ? r + 1 : 3);
          mma(r, af);
          af = afn;
        }
        __builtin_amdgcn_sched_barrier(0);
        dmas(2 * r);
        dmas(2 * r + 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      // UE8M0 scales ride in the MFMA's E8M0 operands and the MFMAs chain on
      // the accumulator.  A 255 scale raises the scale bit and its block adds
      // nothing, as the reference skips the block: a W block's MFMAs run with
      // both E8M0 scales 0 (2^-254 times a sum below 2^25 is below the fp32
      // range: exactly zero is added), an A row's fragment bytes become 0.
      // (selects, not an index: a runtime index would put the array in scratch)
      const uint32_t wb0 = wsel0 ? w_byte0[1] : w_byte0[0], wb1 = wsel1 ? w_byte0[1] : w_byte0[0];
      const uint32_t wsh0 = 8 * ((wb0 + kb) & 3u), wsh1 = 8 * ((wb1 + kb) & 3u);
      uint32_t wsb0 = (sw0 >> wsh0) & 0xffu, wsb1 = (sw1 >> wsh1) & 0xffu;
      const bool wff0 = wsb0 == 0xffu, wff1 = wsb1 == 0xffu;  // wave-uniform
      if (wff0 || wff1) bad |= kErrScale;
      wsb0 = wff0 ? 0u : wsb0;
      wsb1 = wff1 ? 0u : wsb1;
      auto mma = [&](int r, v8i af) {
        uint32_t sb = ((uint32_t)sa4[r] >> (8 * ((a_byte0[r] + kb) & 3u))) & 0xffu;
        const bool aff = sb == 0xffu;
        if (__builtin_amdgcn_ballot_w64(aff)) {  // rare: an invalid A-row scale in the wave
          if (aff) {
            bad |= kErrScale;
            sb = 127;
            af = v8i{0, 0, 0, 0, 0, 0, 0, 0};
          }
        }
        const uint32_t sb0 = wff0 ? 0u : sb, sb1 = wff1 ? 0u : sb;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
          acc[nb][r] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              wf[nb], af, acc[nb][r], 0, 0, 0, (int)((kSwi && nb >= 2) ? wsb1 : wsb0), 0,
              (int)((kSwi && nb >= 2) ? sb1 : sb0));
      };
      // A fragments one block ahead (at most four LDS reads in flight)
      v8i af = a_frag(0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (live(r)) {
          const v8i afn = a_frag(r < 3 ? r + 1 : 3);
          mma(r, af);
          af = afn;
        }
        __builtin_amdgcn_sched_barrier(0);
        dmas(2 * r);
        dmas(2 * r + 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // NS LDS stages, loads NS - 1 steps ahead.  The loads issued at step j
  // are the DMAs of step j + NS - 1.  Step j: wait until only the loads of
  // steps j + 1 .. j + NS - 2 are in flight (step j's tiles and scales have
  // landed), barrier (every wave's DMA for step j is visible and step
  // j - 1's compute is done, so its stage may be refilled), compute step j
  // and issue the loads.  Loads past the last step re-read it (into a stage
  // that is never used), or, in a persistent block with a next tile, fetch
  // that tile's first two steps.  Tiles with every 16-row block live issue
  // the loads one or two at a time between the step's MFMA groups: all of
  // them at the top of the step stalled the waves' MFMA issue behind a full
  // load queue (measured on the cfg4 gate/up heavy experts: 6 % faster with
  // fp32 scales, 14 % with UE8M0 scales; the down GEMM 3-5 %).  Tiles with
  // dead blocks (the one-tile experts, weight streaming) issue them all at
  // the top, which keeps their loads as far ahead as possible.
  // The loads are issued by inline asm, so the compiler adds no waits of its
  // own; which tile a load reads is selected, not branched on, so that the
  // step stays one straight line.  (A per-step L2 prefetch of a later step,
  // one 4-byte load per lane and line, measured slower: the tiles already
  // hit L2 about nine times in ten, and the extra load lengthens every wait.)
  // vector loads per wave and step: A 2 (bf16 x FP4: 4), W 4 (FP4: 2),
  // scales 1 (bf16: 0)
  constexpr int kLoads = kBf ? 6 : kF4 ? 5 : 7;
  static_assert(kLoads == kNLoads, "loads per step");
  constexpr int kWaitStep = vmcnt_enc((int)(NS - 2) * kLoads);
  constexpr int kWaitFirstEnc = vmcnt_enc(kLoads + (int)kStoreOps);
  // stages of steps kb + 0, 1, 2 (kb a multiple of 3)
  const uint32_t st0 = rot, st1 = rot == 2 ? 0u : rot + 1, st2 = rot == 0 ? 2u : rot - 1;
  // persistent blocks run steps 0 .. KB - 3 in the unrolled loop and the
  // last two, which load the next tile's first two, after it (KB >= 4)
  const uint32_t KBm = PERSIST ? KB - 2 : KB;
  auto run = [&](auto FULL, auto NT) __attribute__((always_inline)) {
    auto steps = [&]() __attribute__((always_inline)) {
#define PIH_MOE_STEP(J, TAIL, WAIT)                                                                  \
  {                                                                                                  \
    const uint32_t j = kb + (J);                                                                     \
    if ((TAIL) && j >= KBm) return;                                                                  \
    __builtin_amdgcn_s_waitcnt(WAIT);                                                                \
    __builtin_amdgcn_s_barrier();                                                                    \
    const uint32_t ist = PERSIST ? ((J) % 3 == 0 ? st2 : (J) % 3 == 1 ? st0 : st1) : ((J) + NS - 1) % NS; \
    const uint32_t cst = PERSIST ? ((J) % 3 == 0 ? st0 : (J) % 3 == 1 ? st1 : st2) : (J) % NS;       \
    const uint32_t kbl = PERSIST ? j + 2 : min(j + NS - 1, last);                                    \
    const uint32_t jg = kSplitOk ? j + cur.kb0 : j; /* the step's index in the whole K */             \
    if constexpr (decltype(FULL)::value) {                                                           \
      compute(cst, jg, FULL, [&](int q) { issue_part(ist, kbl, cur, NT, q); });                     \
    } else {                                                                                         \
      issue(ist, kbl, cur, NT);                                                                      \
      compute(cst, jg, FULL, [](int) {});                                                            \
    }                                                                                                \
  }
      uint32_t kb = 0;
      if constexpr (PERSIST) {
        // the tile's first two steps wait past the previous tile's stores
        PIH_MOE_STEP(0, true, kWaitFirstEnc)
        PIH_MOE_STEP(1, true, kWaitFirstEnc)
        PIH_MOE_STEP(2, true, kWaitStep)
        PIH_MOE_STEP(3, true, kWaitStep)
        PIH_MOE_STEP(4, true, kWaitStep)
        PIH_MOE_STEP(5, true, kWaitStep)
        kb = 6;
      }
      // unrolled by a multiple of NS, so that every stage index is a constant
      constexpr uint32_t U = NS == 4 ? 8 : 6;
      for (; kb + U < KBm; kb += U) {
        PIH_MOE_STEP(0, false, kWaitStep)
        PIH_MOE_STEP(1, false, kWaitStep)
        PIH_MOE_STEP(2, false, kWaitStep)
        PIH_MOE_STEP(3, false, kWaitStep)
        PIH_MOE_STEP(4, false, kWaitStep)
        PIH_MOE_STEP(5, false, kWaitStep)
        if constexpr (U == 8) {
          PIH_MOE_STEP(6, false, kWaitStep)
          PIH_MOE_STEP(7, false, kWaitStep)
        }
      }
      PIH_MOE_STEP(0, true, kWaitStep)
      PIH_MOE_STEP(1, true, kWaitStep)
      PIH_MOE_STEP(2, true, kWaitStep)
      PIH_MOE_STEP(3, true, kWaitStep)
      PIH_MOE_STEP(4, true, kWaitStep)
      PIH_MOE_STEP(5, true, kWaitStep)
      if constexpr (U == 8) {
        PIH_MOE_STEP(6, true, kWaitStep)
        PIH_MOE_STEP(7, true, kWaitStep)
      }
#undef PIH_MOE_STEP
    };
    steps();
    if constexpr (PERSIST) {
      // the last two steps load the next tile's steps 0 and 1 (or re-read
      // this tile's last step when there is none)
      make_ops(e2, r2, rs2, t2, nxt);
#pragma unroll
      for (uint32_t f = 0; f < 2; ++f) {
        const uint32_t j = KB - 2 + f;
        const uint32_t sj = (rot + j) % 3;
        __builtin_amdgcn_s_waitcnt(kWaitStep);
        __builtin_amdgcn_s_barrier();
        const uint32_t ist = sj == 0 ? 2u : sj - 1, kbl = has_next ? f : last, jg = kSplitOk ? j + cur.kb0 : j;
        // (the UE8M0 FP8 tail issues its loads at the top: interleaved they
        // made the persistent UE8M0 kernels spill)
        if constexpr (decltype(FULL)::value && !(OP == kOpFp8 && SCALE == kScaleUe8m0)) {
          compute(sj, jg, FULL, [&](int q) { issue_part(ist, kbl, nxt, std::false_type{}, q); });
        } else {
          issue(ist, kbl, nxt, std::false_type{});
          compute(sj, jg, FULL, [](int) {});
        }
      }
    }
  };
  // an expert with one M tile reads each weight byte once: its weight
  // loads are non-temporal, so they do not evict the weight tiles that the
  // multi-tile experts' M tiles share in L2 (the tile's first two steps,
  // loaded before this choice, use the default policy); so does a dense
  // GEMM of one M tile (a decode batch against a wide weight), whose A tile
  // every tile reads again
  bool once = p.dense_m_tiles == 1;
  if (!p.dense_m_tiles && rows) {
    uint32_t lo, hi;
    if constexpr (PERSIST) lo = tab.off[expert], hi = tab.off[expert + 1];
    else lo = p.offsets[expert], hi = p.offsets[expert + 1];
    once = hi >= lo && hi - lo <= BM;
  }
  if (__builtin_amdgcn_readfirstlane(once ? 1u : 0u)) run(std::false_type{}, std::true_type{});
  else if (rb_live == 4) run(std::true_type{}, std::false_type{});
  else run(std::false_type{}, std::false_type{});
  // no DMA may still target this block's LDS when its waves end (a
  // persistent block's loads of its next tile stay in flight)
  if (!PERSIST || !has_next) __builtin_amdgcn_s_waitcnt(kWaitVm0);


  // ---- epilogue: lane holds out[row wm*64 + r*16 + lr][4*lg + i] of block nb
  // SwiGLU tiles: bf16(SiLU(g) x u x w) of a gate value g = bf16(ga) clamped
  // to the limit and an up value u = bf16(ua) clamped to +-limit; NaN where
  // g or u is not finite
  auto swiglu_one = [&](float ga, float ua, float w, auto IEEE, bool& big) __attribute__((always_inline)) -> float {
    float gt = bf16_round(ga), up = bf16_round(ua);
    if (!(__builtin_isfinite(gt) && __builtin_isfinite(up))) return __builtin_nanf("");
    if (p.limit > 0.0f) {
      gt = fminf(gt, p.limit);
      up = fminf(fmaxf(up, -p.limit), p.limit);
    }
    const float sl = decltype(IEEE)::value ? silu_ieee(gt) : silu_rcp(gt, big);
    return bf16_round(sl * up * w);
  };
  // the tile's SwiGLU values v[r][h][i] of gate acc[h][r][i] and up
  // acc[h + 2][r][i] with route weight w[r]: SiLU's quotient by reciprocal
  // (silu_rcp), redone with the IEEE division when a lane of the wave needs
  // it (the same bits either way)
  auto swiglu_values = [&](float (&v)[4][2][4], const float (&w)[4]) __attribute__((always_inline)) {
    bool big = false;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) v[r][h][i] = swiglu_one(acc[h][r][i], acc[h + 2][r][i], w[r], std::false_type{}, big);
    if (__builtin_amdgcn_ballot_w64(big)) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < 4; ++i) v[r][h][i] = swiglu_one(acc[h][r][i], acc[h + 2][r][i], w[r], std::true_type{}, big);
    }
  };
  if constexpr (OUT == kOutSwiGluFp8) {
    // SwiGLU x route weight rounded to bf16 (the values the bf16 output
    // holds), then quantised to e4m3 exactly as fp8_quant_kernel would: the
    // tile's 128 output columns of a row (nt*128 ..) are one 128-group, and
    // its absolute maximum meets across the 4 waves of a row half in LDS
    __shared__ float s_amax[BM][4];
    float vq[4][2][4];
    float rwt[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t rr = wm * 64 + r * 16 + lr;
      rwt[r] = rr < rows && p.row_weight ? p.row_weight[row0 + rr] : 1.0f;
    }
    swiglu_values(vq, rwt);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t rr = wm * 64 + r * 16 + lr;
      const bool live = rr < rows;
      float am = 0.0f;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = vq[r][h][i];
          if (!__builtin_isfinite(v)) {
            if (live) bad |= kErrNonFinite;
            v = 0.0f;
          }
          vq[r][h][i] = v;
          am = fmaxf(am, fabsf(v));
        }
      am = fmaxf(am, __shfl_xor(am, 16));
      am = fmaxf(am, __shfl_xor(am, 32));
      if (lg == 0) s_amax[rr][wn] = am;
    }
    __syncthreads();
    const uint32_t groups = p.n / 256;  // 128-groups per output row
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t rr = wm * 64 + r * 16 + lr;
      if (rr >= rows) continue;
      float amax = fmaxf(fmaxf(s_amax[rr][0], s_amax[rr][1]), fmaxf(s_amax[rr][2], s_amax[rr][3]));
      amax = fmaxf(amax, 1.0e-4f);
      float scale, inv;  // inv: the exact 2^-e (UE8M0) or 1 / scale (fp32)
      const uint64_t g = (uint64_t)(row0 + rr) * groups + nt;
      if constexpr (SCALE == kScaleUe8m0) {
        int e = ue8m0_exponent(amax);
        if (e < -127 || e > 127) {
          bad |= kErrScale;
          e = 0;
        }
        scale = ldexpf(1.0f, e);
        inv = ldexpf(1.0f, -e);
        if (wn == 0 && lg == 0) static_cast<uint8_t*>(p.out_scale)[g] = (uint8_t)(e + 127);
      } else {
        scale = amax / 448.0f;
        inv = 1.0f / scale;
        if (wn == 0 && lg == 0) static_cast<float*>(p.out_scale)[g] = scale;
      }
      // codes of row rr, bytes wn*32 + h*16 + 4lg: into the staged tile
      // (rows 144 bytes apart: a store's 16 rows x 4 lanes hit 64 banks) or
      // straight to memory
      uint8_t* dst = p.stage_out ? smem + rr * kCodePitch + wn * 32 + 4 * lg
                                 : static_cast<uint8_t*>(p.out) + (uint64_t)(row0 + rr) * p.out_row_stride + nt * 128 +
                                       wn * 32 + 4 * lg;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        *reinterpret_cast<uint32_t*>(dst + h * 16) =
            SCALE == kScaleUe8m0 ? e4m3_quant4_mul(vq[r][h], inv) : e4m3_quant4_recip(vq[r][h], scale, inv);
    }
    if (p.stage_out) {
      // whole 128-byte code rows, 16 bytes per lane
      __syncthreads();
#pragma unroll
      for (uint32_t c = tid; c < BM * 8; c += NTH) {
        const uint32_t R = c / 8, ch = c % 8;
        if (R < rows)
          *reinterpret_cast<v4i*>(static_cast<uint8_t*>(p.out) + (uint64_t)(row0 + R) * p.out_row_stride + nt * 128 +
                                  ch * 16) = *reinterpret_cast<const v4i*>(smem + R * kCodePitch + ch * 16);
      }
    }
  }
  // Plain outputs: when no live block of the wave holds a non-finite value
  // that must be skipped (the common case), every live block is stored
  // whole, with no per-row or per-column test at all on a full tile;
  // otherwise the per-element path below.
  bool stored = false;
  [[maybe_unused]] bool slow = false;  // wave-uniform
  // CODES: whether an e4m3 NaN code sits in the A rows or W rows of this
  // wave's 64 x 64 block (wave-uniform), and the flags before its stores
  [[maybe_unused]] bool codes = false;
  [[maybe_unused]] const uint32_t bad0 = CODES ? bad : 0u;
  [[maybe_unused]] uint32_t codes_bad = 0;  // CODES: the recomputed block's flag bits
  if constexpr (OUT == kOutBf16 || OUT == kOutF32) {
    bool nonfin = false;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const v4f v = acc[nb][r];
        const bool live = wm * 64 + r * 16 + lr < rows && nt * BN + wn * 64 + nb * 16 + 4 * lg < p.n;
        if (live && !(__builtin_isfinite(v[0]) && __builtin_isfinite(v[1]) && __builtin_isfinite(v[2]) &&
                      __builtin_isfinite(v[3])))
          nonfin = true;
      }
    if constexpr (CODES) {
      // Only a block with a non-finite value can have met a code.  The
      // block's 64 A rows and 64 W rows (K bytes each), four rows of each at
      // a time, lane l reading bytes [16 c, 16 c + 16) for c = l, l + 64, ...
      // (eight loads in flight).  The launcher allows the check on one
      // problem of contiguous rows (tile row R is A row row0 + R < m) with
      // 16-byte aligned operands.  Its values are defined here (behind
      // empty asm statements) so that nothing of this rare path is computed
      // ahead of the K loop and kept live across it.
      if (__builtin_amdgcn_ballot_w64(nonfin)) {
        uint32_t Kc = K, r_base = wm * 64, c_base = nt * BN + wn * 64, c0 = lane * 16;
        asm volatile("" : "+s"(Kc), "+s"(r_base), "+s"(c_base), "+v"(c0));
        uint32_t hit = 0;
        for (uint32_t i0 = 0; i0 < 64; i0 += 4) {
          for (uint32_t c = c0; c < Kc; c += 64 * 16) {
#pragma unroll
            for (uint32_t u = 0; u < 4; ++u) {
              const uint32_t R = r_base + i0 + u, C = c_base + i0 + u;
              if (R < rows) {
                const v4u v = *reinterpret_cast<const v4u*>(p.a + (uint64_t)(row0 + R) * Kc + c);
                hit |= e4m3_nan_bytes(v.x) | e4m3_nan_bytes(v.y) | e4m3_nan_bytes(v.z) | e4m3_nan_bytes(v.w);
              }
              if (C < p.n) {
                const v4u v = *reinterpret_cast<const v4u*>(p.w + (uint64_t)C * Kc + c);
                hit |= e4m3_nan_bytes(v.x) | e4m3_nan_bytes(v.y) | e4m3_nan_bytes(v.z) | e4m3_nan_bytes(v.w);
              }
            }
          }
        }
        codes = __builtin_amdgcn_ballot_w64(hit != 0) != 0;
      }
    }
    if (nonfin) bad |= kErrNonFinite;
    const bool keep_finite = nonfin && p.err_nonfinite && !p.write_nonfinite;
    if constexpr (PERSIST) {
      // Persistent blocks: exactly kStoreOps buffer stores per lane (rows
      // past the tile's end fall outside the buffer's range and columns past
      // n get an offset outside it; the hardware drops both), so the next
      // tile's first waits count them; a wave that must skip non-finite
      // elements stores per element below and then drains its stores.
      slow = __builtin_amdgcn_ballot_w64(keep_finite) != 0;
      if constexpr (CODES) {
        if (codes) {
          // The block again, the reference's way: lane l computes row
          // wm * 64 + l, column by column; each 128-k block is an fp32 sum
          // of decoded products in k order (NaN codes as 0), scaled by the
          // row's and the W block's scales and added in block order; a
          // block with a 0xFF UE8M0 scale adds nothing (bit 2); a
          // non-finite result raises bit 4 and, unless write_nonfinite, is
          // not stored (the reference's fp8_gemm_kernel,
          // deepseek_fp8_gemm.cu:11-70).  Its stores replace the block's;
          // the wait below drains them.
          uint32_t Kc = K, rb = wm * 64, cb = nt * BN + wn * 64;
          asm volatile("" : "+s"(Kc), "+s"(rb), "+s"(cb));
          const uint32_t KBc = Kc / 128, R = rb + lane;
          const bool live_r = R < rows;
          const uint32_t arow = row0 + (live_r ? R : 0u);
          uint32_t rbad = 0;
          for (uint32_t j = 0; j < 64; ++j) {
            const uint32_t C = cb + j;
            if (C >= p.n) break;
            float sum = 0.0f;
            for (uint32_t kb = 0; kb < KBc; ++kb) {
              float sca, scw;
              if constexpr (SCALE == kScaleUe8m0) {
                const uint32_t ba = static_cast<const uint8_t*>(p.a_scale)[(uint64_t)arow * KBc + kb];
                const uint32_t bw = static_cast<const uint8_t*>(p.w_scale)[(uint64_t)(C / 128) * KBc + kb];
                if (ba == 0xffu || bw == 0xffu) {
                  rbad |= kErrScale;
                  continue;
                }
                sca = ue8m0_value(ba);
                scw = ue8m0_value(bw);
              } else {
                sca = reinterpret_cast<const float*>(p.a_scale)[(uint64_t)arow * KBc + kb];
                scw = reinterpret_cast<const float*>(p.w_scale)[(uint64_t)(C / 128) * KBc + kb];
              }
              const uint8_t* ap = p.a + (uint64_t)arow * Kc + kb * 128;
              const uint8_t* wp = p.w + (uint64_t)C * Kc + kb * 128;
              float local = 0.0f;
              for (uint32_t i = 0; i < 128; i += 16) {
                v4u av = *reinterpret_cast<const v4u*>(ap + i), wv = *reinterpret_cast<const v4u*>(wp + i);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                  const uint32_t na = e4m3_nan_bytes(av[q]), nw = e4m3_nan_bytes(wv[q]);
                  if (na | nw) rbad |= kErrCode;
                  const uint32_t xa = e4m3_nan_to_zero(av[q], na), xw = e4m3_nan_to_zero(wv[q], nw);
#pragma unroll
                  for (int t = 0; t < 4; ++t) local = local + e4m3_decode((xa >> (8 * t)) & 0xffu) *
                                                                  e4m3_decode((xw >> (8 * t)) & 0xffu);
                }
              }
              sum = sum + local * sca * scw;
            }
            if (!live_r) continue;
            const uint64_t o = (uint64_t)arow * p.out_row_stride + C;
            const bool fin = __builtin_isfinite(sum);
            if (!fin) rbad |= kErrNonFinite;
            // the first pass's rule: a non-finite result is stored only
            // when the caller asks for it (or keeps no non-finite bit)
            if (fin || !p.err_nonfinite || p.write_nonfinite) {
              if constexpr (OUT == kOutF32) static_cast<float*>(p.out)[o] = sum;
              else static_cast<uint16_t*>(p.out)[o] = (uint16_t)f32_to_bf16_bits(sum);
            }
          }
          // rows past the tile's end computed row row0's values: not theirs
          codes_bad = live_r ? rbad : 0u;
          slow = true;
          stored = true;
        }
      }
      if (!slow) {
        stored = true;
        constexpr uint32_t OSZ = OUT == kOutF32 ? 4 : 2;
        const uint32_t stride_b = p.out_row_stride * OSZ;
        uint8_t* tile_out = static_cast<uint8_t*>(p.out) +
                            ((uint64_t)row0 * p.out_row_stride + (uint64_t)expert * p.out_prob_col + nt * BN) * OSZ;
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(tile_out, 0, rows * stride_b, 0x00020000);
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int nb = 0; nb < 4; ++nb) {
            const uint32_t R = wm * 64 + r * 16 + lr, C = wn * 64 + nb * 16 + 4 * lg;
            const uint32_t off = nt * BN + C < p.n ? R * stride_b + C * OSZ : 0x80000000u;
            const v4f v = acc[nb][r];
            if constexpr (OUT == kOutF32)
              __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v), rsrc, off, 0, 0);
            else
              __builtin_amdgcn_raw_buffer_store_b64(v2u{f32x2_to_bf16x2(v[0], v[1]), f32x2_to_bf16x2(v[2], v[3])}, rsrc,
                                                    off, 0, 0);
          }
      }
    } else if (p.stage_out && !__syncthreads_or(keep_finite)) {
      // one decision for the block: every wave is past its main loop and its
      // DMAs (vmcnt(0) above), so the stages are free for the staged tile
      stored = true;
      // the tile staged in LDS (rows padded by 32 bytes: the 16 rows of a
      // fragment start 8 banks apart), then whole rows stored with 16 bytes
      // per lane: 128-byte lines instead of 16 rows x 32 bytes per store
      constexpr uint32_t OSZ = OUT == kOutF32 ? 4 : 2, PITCH = BN * OSZ + 32, CPR = BN * OSZ / 16;
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          uint8_t* d = smem + (wm * 64 + r * 16 + lr) * PITCH + (wn * 64 + nb * 16 + 4 * lg) * OSZ;
          const v4f v = acc[nb][r];
          if constexpr (OUT == kOutF32) *reinterpret_cast<v4f*>(d) = v;
          else *reinterpret_cast<uint2*>(d) = uint2{f32x2_to_bf16x2(v[0], v[1]), f32x2_to_bf16x2(v[2], v[3])};
        }
      __syncthreads();
#pragma unroll
      for (uint32_t c = tid; c < BM * CPR; c += NTH) {
        const uint32_t R = c / CPR, ch = c % CPR, col = nt * BN + ch * (16 / OSZ);
        if (R < rows && col < p.n)
          *reinterpret_cast<v4i*>(static_cast<uint8_t*>(p.out) +
                                  ((uint64_t)(row0 + R) * p.out_row_stride + (uint64_t)expert * p.out_prob_col + col) *
                                      OSZ) = *reinterpret_cast<const v4i*>(smem + R * PITCH + ch * 16);
      }
    } else if (!__builtin_amdgcn_ballot_w64(keep_finite)) {
      stored = true;
      auto store = [&](int r, int nb) __attribute__((always_inline)) {
        const uint64_t o = (uint64_t)(row0 + wm * 64 + r * 16 + lr) * p.out_row_stride +
                           (uint64_t)expert * p.out_prob_col + nt * BN + wn * 64 + nb * 16 + 4 * lg;
        const v4f v = acc[nb][r];
        if constexpr (OUT == kOutF32) *reinterpret_cast<v4f*>(static_cast<float*>(p.out) + o) = v;
        else
          *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.out) + o) =
              uint2{f32x2_to_bf16x2(v[0], v[1]), f32x2_to_bf16x2(v[2], v[3])};
      };
      if (rows == BM && nt * BN + BN <= p.n) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int nb = 0; nb < 4; ++nb) store(r, nb);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (wm * 64 + r * 16 + lr >= rows) continue;
#pragma unroll
          for (int nb = 0; nb < 4; ++nb)
            if (nt * BN + wn * 64 + nb * 16 + 4 * lg < p.n) store(r, nb);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 4 && OUT != kOutSwiGluFp8 && !stored; ++r) {
    const uint32_t rr = wm * 64 + r * 16 + lr;
    if (rr >= rows) continue;
    const uint64_t orow = (uint64_t)(row0 + rr) * p.out_row_stride + (uint64_t)expert * p.out_prob_col;
    if constexpr (OUT == kOutSwiGlu) {
      const float rwt = p.row_weight ? p.row_weight[row0 + rr] : 1.0f;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t o[4];
        bool ok = true;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float gt = bf16_round(acc[h][r][i]);
          float up = bf16_round(acc[h + 2][r][i]);
          float v = 0.0f;
          if (!__builtin_isfinite(gt) || !__builtin_isfinite(up)) {
            ok = false;
          } else {
            if (p.limit > 0.0f) {
              gt = fminf(gt, p.limit);
              up = fminf(fmaxf(up, -p.limit), p.limit);
            }
            v = (gt / (1.0f + expf(-gt))) * up;
            v = v * rwt;
            if (!__builtin_isfinite(v)) ok = false;
          }
          o[i] = __builtin_isfinite(v) ? f32_to_bf16_bits(v) : 0xffffffffu;
        }
        uint16_t* dst = static_cast<uint16_t*>(p.out) + orow + nt * 128 + wn * 32 + h * 16 + 4 * lg;
        if (ok) {
          *reinterpret_cast<uint2*>(dst) = uint2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
        } else {
          bad |= kErrNonFinite;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (o[i] != 0xffffffffu) dst[i] = (uint16_t)o[i];
        }
      }
    } else {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const uint32_t col = nt * BN + wn * 64 + nb * 16 + 4 * lg;
        if (col >= p.n) continue;
        const v4f v = acc[nb][r];
        const bool fin = __builtin_isfinite(v[0]) && __builtin_isfinite(v[1]) && __builtin_isfinite(v[2]) &&
                         __builtin_isfinite(v[3]);
        if constexpr (OUT == kOutF32) {
          float* dst = static_cast<float*>(p.out) + orow + col;
          if (fin || !p.err_nonfinite || p.write_nonfinite) {
            *reinterpret_cast<v4f*>(dst) = v;
            if (!fin) bad |= kErrNonFinite;
          } else {
            bad |= kErrNonFinite;
            for (int i = 0; i < 4; ++i)
              if (__builtin_isfinite(v[i])) dst[i] = v[i];
          }
        } else {
          uint16_t* dst = static_cast<uint16_t*>(p.out) + orow + col;
          if (fin || !p.err_nonfinite || p.write_nonfinite) {
            *reinterpret_cast<uint2*>(dst) = uint2{f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16),
                                                   f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16)};
            if (!fin) bad |= kErrNonFinite;
          } else {
            bad |= kErrNonFinite;
            for (int i = 0; i < 4; ++i)
              if (__builtin_isfinite(v[i])) dst[i] = (uint16_t)f32_to_bf16_bits(v[i]);
          }
        }
      }
    }
  }
  if constexpr (CODES) {
    // a recomputed block's flags replace those of its first pass
    if (codes) bad = bad0 | codes_bad;
  }
  if constexpr (!PERSIST) {
    break;
  } else {
    if (slow) __builtin_amdgcn_s_waitcnt(kWaitVm0);
    if (!has_next) break;
    vb += gridDim.x;
    expert = e2;
    row0 = r2;
    rows = rs2;
    nt = t2;
    cur = nxt;
    rot = (rot + KB) % 3;
  }
  }  // tiles
  if (bad) {
    const uint32_t bits = ((bad & kErrCode) ? p.err_code : 0u) | ((bad & kErrScale) ? p.err_scale : 0u) |
                          ((bad & kErrNonFinite) ? p.err_nonfinite : 0u);
    if (bits) atomicOr(p.err, bits);
  }
}


template <int OP, int SCALE>
void launch_out(const MoeParams& mp, uint32_t grid, hipStream_t s, OutKind out, bool persist) {
  if constexpr (OP == kOpFp8 || OP == kOpFp4 || OP == kOpBf16Fp4) {
    if (out == kOutSwiGlu) {
      hipLaunchKernelGGL((fp8_moe_gemm_kernel<OP, SCALE, kOutSwiGlu, false>), dim3(grid), dim3(NTH), 0, s, mp);
      return;
    }
  }
  if constexpr (OP == kOpFp8) {
    if (out == kOutSwiGluFp8) {
      hipLaunchKernelGGL((fp8_moe_gemm_kernel<OP, SCALE, kOutSwiGluFp8, false>), dim3(grid), dim3(NTH), 0, s, mp);
      return;
    }
  }
  // (bf16 x FP4 stages leave no LDS for the persistent tile table)
  if constexpr (OP != kOpBf16Fp4) {
    if (persist) {
      if (out == kOutF32)
        hipLaunchKernelGGL((fp8_moe_gemm_kernel<OP, SCALE, kOutF32, true>), dim3(grid), dim3(NTH), 0, s, mp);
      else hipLaunchKernelGGL((fp8_moe_gemm_kernel<OP, SCALE, kOutBf16, true>), dim3(grid), dim3(NTH), 0, s, mp);
      return;
    }
  }
  if (out == kOutF32)
    hipLaunchKernelGGL((fp8_moe_gemm_kernel<OP, SCALE, kOutF32, false>), dim3(grid), dim3(NTH), 0, s, mp);
  else hipLaunchKernelGGL((fp8_moe_gemm_kernel<OP, SCALE, kOutBf16, false>), dim3(grid), dim3(NTH), 0, s, mp);
}

// Blocks of a persistent launch: one per CU, a multiple of 8 (the tile
// sequence is split into 8 XCD ranges by blockIdx % 8); 0 if unknown.
// (Per-device cache in relaxed atomics: concurrent host threads store the
// same value.)
uint32_t PersistentBlocks() {
  static std::atomic<uint32_t> cached[kHostMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kHostMaxDevices) return 0;
  uint32_t v = cached[dev].load(std::memory_order_relaxed);
  if (!v) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 8) return 0;
    v = (uint32_t)cus / 8 * 8;
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// Plain (bf16 / fp32) outputs without an A gather run persistent: a block
// walks its XCD's tiles, the next tile's first loads overlap this tile's
// epilogue and its stores drain under the next tile's first steps.  The
// buffer stores need the tile's output bytes below 2^31; MoE segments need
// the LDS table (at most kTableExperts experts); the last two K steps of a
// tile load the next tile's first two, so a tile has at least four.
bool Persistent(OutKind out, bool gather, bool dense, uint32_t problems, uint64_t row_stride, uint32_t k_steps) {
  const uint64_t osz = out == kOutF32 ? 4 : 2;
  return (out == kOutBf16 || out == kOutF32) && !gather && (dense || problems <= kTableExperts) && k_steps >= 4 &&
         (uint64_t)BM * row_stride * osz < 0x80000000ull && PersistentBlocks() > 0;
}

// Output rows and problem column offsets on 16-byte boundaries: the kernel
// may stage its tile in LDS and store whole rows.
uint32_t StageOut(const void* out, uint64_t row_stride, uint64_t prob_col, OutKind kind) {
  const uint64_t osz = kind == kOutF32 ? 4 : kind == kOutSwiGluFp8 ? 1 : 2;
  return reinterpret_cast<uintptr_t>(out) % 16 == 0 && row_stride * osz % 16 == 0 && prob_col * osz % 16 == 0;
}

}  // namespace

// Called by LaunchFp8BlockGemm for MoE problems without the code scan; the
// shape, format and pointer checks are the caller's.
St LaunchFp8MoeGemm(const BlockGemmArgs& a) {
  MoeParams mp{};
  mp.a = a.a;
  mp.a_scale = a.a_scale;
  mp.a_gather = a.a_gather;
  mp.w = a.w;
  mp.w_scale = a.w_scale;
  mp.out = a.out;
  mp.row_weight = a.row_weight;
  mp.offsets = a.offsets;
  mp.err = a.error_flag;
  mp.m = a.m;
  mp.n = a.n;
  mp.k = a.k;
  mp.experts = a.problems;
  mp.a_rows_total = a.a_rows_total;
  const bool swiglu = a.out_kind == kOutSwiGlu || a.out_kind == kOutSwiGluFp8;
  mp.out_scale = a.out_scale;
  mp.out_row_stride = a.out_row_stride ? a.out_row_stride : (swiglu ? a.n / 2 : a.n);
  mp.n_tiles = swiglu ? a.n / 256 : (a.n + BN - 1) / BN;
  mp.stage_out = StageOut(a.out, mp.out_row_stride, 0, a.out_kind);
  mp.limit = a.swiglu_limit;
  mp.err_code = a.err_code_bit;
  mp.err_scale = a.err_scale_bit;
  mp.err_nonfinite = a.err_nonfinite_bit;
  // sum_e ceil(rows_e / BM) <= m / BM + (number of non-empty experts)
  const uint64_t mt = (uint64_t)a.m / BM + (a.problems < a.m ? a.problems : a.m);
  const uint64_t total = mt * mp.n_tiles;
  if (total == 0 || total > 0x7fffffffull - 8) return Invalid("fp8_gemm_grid_too_large");
  // the tile loads address A and one expert's W by 32-bit byte offsets
  if ((uint64_t)a.a_rows_total * a.k > 0xffffffffull || (uint64_t)a.n * a.k > 0xffffffffull)
    return Invalid("fp8_moe_gemm_operand_too_large");
  const bool persist = Persistent(a.out_kind, a.a_gather != nullptr, false, a.problems, mp.out_row_stride, a.k / 128);
  uint32_t grid = (uint32_t)((total + 7) / 8 * 8);
  mp.vb_end = grid;
  if (persist) grid = std::min(grid, PersistentBlocks());
  St s = RequireCleanLastError();
  if (!s.ok()) return s;
  if (a.scale_fmt == kScaleF32) launch_out<kOpFp8, kScaleF32>(mp, grid, a.stream, a.out_kind, persist);
  else launch_out<kOpFp8, kScaleUe8m0>(mp, grid, a.stream, a.out_kind, persist);
  return AfterLaunch("fp8_moe_gemm_launch_failed");
}

// MXFP4 MoE: the experts with more than light_rows rows on the 128 x 256
// tiles (FP4 W operand; e4m3 or bf16 activations).  Called by
// LaunchFp4Gemm after its checks when Fp4MoeBigTileTakes(a).
bool Fp4MoeBigTileTakes(const Fp4GemmArgs& a) {
  const bool swiglu = a.out_kind == kOutSwiGlu;
  const uint64_t a_row = a.act == kActBf16 ? 2ull * a.k : a.k;
  return a.moe && (a.act == kActE4m3 || a.act == kActBf16) && a.k % 128 == 0 && a.k >= 128 &&
         (swiglu ? a.n % 256 == 0 : a.n % 128 == 0) &&
         (a.out_kind == kOutSwiGlu || a.out_kind == kOutBf16 || a.out_kind == kOutF32) &&
         reinterpret_cast<uintptr_t>(a.w_scale) % 4 == 0 && (uint64_t)a.a_rows_total * a_row <= 0xffffffffull &&
         (uint64_t)a.n * (a.k / 2) <= 0xffffffffull;
}

St LaunchFp4MoeBigTile(const Fp4GemmArgs& a, uint32_t light_rows) {
  MoeParams mp{};
  mp.a = static_cast<const uint8_t*>(a.a);
  mp.a_scale = a.a_scale;
  mp.a_gather = a.a_gather;
  mp.w = a.w;
  mp.w_scale = a.w_scale;
  mp.out = a.out;
  mp.row_weight = a.row_weight;
  mp.offsets = a.offsets;
  mp.err = a.error_flag;
  mp.m = a.m;
  mp.n = a.n;
  mp.k = a.k;
  mp.experts = a.problems;
  mp.a_rows_total = a.a_rows_total;
  mp.light_rows = light_rows;
  const bool swiglu = a.out_kind == kOutSwiGlu;
  mp.out_row_stride = swiglu ? a.n / 2 : a.n;
  mp.n_tiles = swiglu ? a.n / 256 : (a.n + BN - 1) / BN;
  mp.stage_out = StageOut(a.out, mp.out_row_stride, 0, a.out_kind);
  mp.limit = a.swiglu_limit;
  // the MXFP4 error bits: 1 code, 2 scale, 4 non-finite
  mp.err_code = 1u;
  mp.err_scale = 2u;
  mp.err_nonfinite = 4u;
  // sum over the taken experts of ceil(rows / BM) <= m / BM + their count,
  // and at most m / (light_rows + 1) experts have more than light_rows rows
  // (a launch with none then costs a few hundred blocks, not thousands)
  const uint64_t taken = std::min<uint64_t>(a.problems, (uint64_t)a.m / ((uint64_t)light_rows + 1));
  const uint64_t mt = (uint64_t)a.m / BM + taken;
  const uint64_t total = mt * mp.n_tiles;
  if (total == 0) return Ok();  // no expert can have more than light_rows rows
  if (total > 0x7fffffffull - 8) return Invalid("fp4_moe_gemm_grid_too_large");
  const bool bf = a.act == kActBf16;
  const bool persist =
      !bf && Persistent(a.out_kind, a.a_gather != nullptr, false, a.problems, mp.out_row_stride, a.k / 128);
  uint32_t grid = (uint32_t)((total + 7) / 8 * 8);
  mp.vb_end = grid;
  if (persist) grid = std::min(grid, PersistentBlocks());
  St s = RequireCleanLastError();
  if (!s.ok()) return s;
  if (bf) launch_out<kOpBf16Fp4, kScaleUe8m0>(mp, grid, a.stream, a.out_kind, false);
  else launch_out<kOpFp4, kScaleUe8m0>(mp, grid, a.stream, a.out_kind, persist);
  return AfterLaunch("fp4_moe_gemm_launch_failed");
}

// One dense FP4 problem (DeepSeek launch_fp4_gemm at batches the small-M
// kernel does not take well) on the 128 x 256 tiles with the FP4 W operand:
// the dense tile map of LaunchBigTileGemm (M tiles halved to 64 / 32 rows
// while the tiles number fewer than 192), the MXFP4 error bits (1 code, 2
// scale, 4 non-finite, non-finite results not stored), and every block
// exiting at once when skip_if holds the code bit (the caller's NaN-code
// scan of A runs first; W e2m1 has no NaN code).
bool Fp4DenseBigTileTakes(const Fp4GemmArgs& a) {
  return !a.moe && !a.a_gather && a.problems == 1 && a.act == kActE4m3 && a.k % 128 == 0 && a.k >= 512 &&
         a.n % 128 == 0 && (a.out_kind == kOutBf16 || a.out_kind == kOutF32) && a.a_rows_total >= a.m &&
         reinterpret_cast<uintptr_t>(a.w_scale) % 4 == 0 && reinterpret_cast<uintptr_t>(a.a) % 16 == 0 &&
         (uint64_t)a.a_rows_total * a.k <= 0xffffffffull && (uint64_t)a.n * (a.k / 2) <= 0xffffffffull;
}

St LaunchFp4DenseBigTile(const Fp4GemmArgs& a, const uint32_t* skip_if, uint32_t skip_bit) {
  if (!Fp4DenseBigTileTakes(a)) return Invalid("fp4_dense_big_tile_invalid");
  MoeParams mp{};
  mp.a = static_cast<const uint8_t*>(a.a);
  mp.a_scale = a.a_scale;
  mp.w = a.w;
  mp.w_scale = a.w_scale;
  mp.out = a.out;
  mp.err = a.error_flag;
  mp.m = a.m;
  mp.n = a.n;
  mp.k = a.k;
  mp.experts = 1;
  mp.a_rows_total = a.a_rows_total;
  uint32_t tile_rows = BM;
  const uint64_t nt = (a.n + BN - 1) / BN;
  while (tile_rows > 32 && (uint64_t)((a.m + tile_rows - 1) / tile_rows) * nt < 192) tile_rows /= 2;
  mp.dense_tile_rows = tile_rows;
  mp.dense_m_tiles = (a.m + tile_rows - 1) / tile_rows;
  mp.a_row_stride = 1;
  mp.a_prob_row = 0;
  mp.out_row_stride = a.n;
  mp.out_prob_col = 0;
  mp.n_tiles = (uint32_t)nt;
  mp.stage_out = StageOut(a.out, mp.out_row_stride, 0, a.out_kind);
  mp.err_code = 1u;
  mp.err_scale = 2u;
  mp.err_nonfinite = 4u;
  mp.skip_if = skip_if;
  mp.skip_bit = skip_bit;
  const uint64_t total = (uint64_t)mp.dense_m_tiles * mp.n_tiles;
  if (total > 0x7fffffffull - 8) return Invalid("fp4_dense_big_tile_grid_too_large");
  const bool persist = Persistent(a.out_kind, false, true, 1, mp.out_row_stride, a.k / 128);
  uint32_t grid = (uint32_t)((total + 7) / 8 * 8);
  mp.vb_end = grid;
  if (persist) grid = std::min(grid, PersistentBlocks());
  St s = RequireCleanLastError();
  if (!s.ok()) return s;
  launch_out<kOpFp4, kScaleUe8m0>(mp, grid, a.stream, a.out_kind, persist);
  return AfterLaunch("fp4_dense_big_tile_launch_failed");
}

St LaunchBigTileGemm(const BigTileArgs& a, bool* codes_in_tiles) {
  if (codes_in_tiles) *codes_in_tiles = false;
  const bool bf = a.bf16;
  if (!a.a || !a.w || !a.out || !a.stream || (!bf && (!a.a_scale || !a.w_scale || !a.error_flag)))
    return Invalid("big_tile_gemm_null_argument");
  if (a.m == 0 || a.n == 0 || a.k == 0 || a.n % 128 || a.k % (bf ? 64 : 128))
    return Invalid("big_tile_gemm_shape_invalid");
  if (a.out_kind != kOutBf16 && a.out_kind != kOutF32) return Invalid("big_tile_gemm_output_type_invalid");
  if (a.problems == 0) return Invalid("big_tile_gemm_shape_invalid");
  const uint64_t rb = bf ? 2ull * a.k : a.k;
  // K split: one problem, fp32 partial sums, whole K steps of at least 4 per split
  const uint32_t splits = a.k_splits > 1 ? a.k_splits : 1u, ksteps = (uint32_t)(rb / 128);
  if (splits > 1 && (a.problems != 1 || a.a_prob_row != 0 || a.out_kind != kOutF32 || ksteps % splits ||
                     ksteps / splits < 4))
    return Invalid("big_tile_gemm_split_invalid");
  if (a.code_check) {
    if (bf || splits > 1 || a.problems != 1 || a.a_row_stride != 1 || a.a_prob_row != 0 || !a.err_code_bit ||
        (a.a_rows_total && a.a_rows_total < a.m))
      return Invalid("big_tile_gemm_code_check_invalid");
    if ((reinterpret_cast<uintptr_t>(a.a) | reinterpret_cast<uintptr_t>(a.w)) % 16)
      return Invalid("nan_code_scan_alignment_invalid");
  }
  const uint64_t a_rows = a.a_rows_total ? a.a_rows_total : (uint64_t)a.m * a.problems;
  // the tile loads address A and one problem's W by 32-bit byte offsets
  if (a_rows > 0xffffffffull || a_rows * rb > 0xffffffffull || (uint64_t)a.n * rb > 0xffffffffull)
    return Invalid("big_tile_gemm_operand_too_large");
  MoeParams mp{};
  mp.a = static_cast<const uint8_t*>(a.a);
  mp.a_scale = a.a_scale;
  mp.w = static_cast<const uint8_t*>(a.w);
  mp.w_scale = a.w_scale;
  mp.out = a.out;
  mp.err = a.error_flag;
  mp.m = a.m;
  mp.n = a.n;
  mp.k = a.k;
  mp.experts = splits > 1 ? splits : a.problems;
  mp.k_splits = splits;
  mp.a_rows_total = (uint32_t)a_rows;
  // fewer 128-row tiles than about a round on the CUs (and no K split):
  // 64- or 32-row M tiles, up to four times the tiles at the same K depth
  // (same arithmetic per element; the tiles stream their W tile from L2)
  uint32_t tile_rows = BM;
  if (splits == 1) {
    const uint64_t nt = (a.n + BN - 1) / BN;
    while (tile_rows > 32 && (uint64_t)((a.m + tile_rows - 1) / tile_rows) * nt * a.problems < 192) tile_rows /= 2;
  }
  mp.dense_tile_rows = tile_rows;
  mp.dense_m_tiles = (a.m + tile_rows - 1) / tile_rows;
  mp.a_row_stride = a.a_row_stride;
  mp.a_prob_row = a.a_prob_row;
  mp.out_row_stride = a.out_row_stride ? a.out_row_stride : a.n;
  mp.out_prob_col = splits > 1 ? (uint64_t)a.m * mp.out_row_stride : a.out_prob_col;
  mp.n_tiles = (a.n + BN - 1) / BN;
  mp.stage_out = StageOut(a.out, mp.out_row_stride, mp.out_prob_col, a.out_kind);
  mp.err_code = a.error_flag ? a.err_code_bit : 0u;
  mp.err_scale = a.error_flag ? a.err_scale_bit : 0u;
  mp.err_nonfinite = a.error_flag ? a.err_nonfinite_bit : 0u;
  mp.write_nonfinite = a.write_nonfinite ? 1u : 0u;
  mp.skip_if = a.skip_if;
  mp.skip_bit = a.skip_bit;
  const uint64_t total = (uint64_t)mp.dense_m_tiles * mp.n_tiles * mp.experts;
  if (total > 0x7fffffffull - 8) return Invalid("big_tile_gemm_grid_too_large");
  const bool persist = Persistent(a.out_kind, false, true, mp.experts, mp.out_row_stride, ksteps / splits);
  uint32_t grid = (uint32_t)((total + 7) / 8 * 8);
  mp.vb_end = grid;
  if (persist) grid = std::min(grid, PersistentBlocks());
  St s = RequireCleanLastError();
  if (!s.ok()) return s;
  if (a.code_check && persist) {
    // the tiles compute the result with NaN codes as zeros themselves; the
    // code bit may be raised while they run: no skip test
    mp.skip_if = nullptr;
    mp.skip_bit = 0;
    if (codes_in_tiles) *codes_in_tiles = true;
    constexpr int kF32c = kOutF32 + kOutCodeCheck, kBf16c = kOutBf16 + kOutCodeCheck;
    if (a.scale_fmt == kScaleF32) {
      if (a.out_kind == kOutF32)
        hipLaunchKernelGGL((fp8_moe_gemm_kernel<kOpFp8, kScaleF32, kF32c, true>), dim3(grid), dim3(NTH), 0, a.stream, mp);
      else
        hipLaunchKernelGGL((fp8_moe_gemm_kernel<kOpFp8, kScaleF32, kBf16c, true>), dim3(grid), dim3(NTH), 0, a.stream,
                           mp);
    } else {
      if (a.out_kind == kOutF32)
        hipLaunchKernelGGL((fp8_moe_gemm_kernel<kOpFp8, kScaleUe8m0, kF32c, true>), dim3(grid), dim3(NTH), 0, a.stream,
                           mp);
      else
        hipLaunchKernelGGL((fp8_moe_gemm_kernel<kOpFp8, kScaleUe8m0, kBf16c, true>), dim3(grid), dim3(NTH), 0,
                           a.stream, mp);
    }
    return AfterLaunch("big_tile_gemm_launch_failed");
  }
  if (a.code_check) {
    // a scan of exactly the A and W bytes the tiles read raises the bit
    // first, and the tiles exit at once if it is set
    NanCodeScanArgs sc;
    sc.a = a.a;
    sc.a_bytes = (uint64_t)a.m * a.k;
    sc.w = a.w;
    sc.w_bytes = (uint64_t)a.n * a.k;
    sc.error_flag = a.error_flag;
    sc.bit = a.err_code_bit;
    sc.stream = a.stream;
    if (!(s = LaunchNanCodeScan(sc)).ok()) return s;
    mp.skip_if = a.error_flag;
    mp.skip_bit = a.err_code_bit;
  }
  if (bf) launch_out<kOpBf16, kScaleF32>(mp, grid, a.stream, a.out_kind, persist);
  else if (a.scale_fmt == kScaleF32) launch_out<kOpFp8, kScaleF32>(mp, grid, a.stream, a.out_kind, persist);
  else launch_out<kOpFp8, kScaleUe8m0>(mp, grid, a.stream, a.out_kind, persist);
  return AfterLaunch("big_tile_gemm_launch_failed");
}

// ------------------------------------------------ K-split partial-sum reduce
namespace {

// out[i] = (((ws[0][i] + ws[1][i]) + ws[2][i]) + ...) over `splits` slabs of
// `slab` floats, four per thread; bf16 (round to nearest even) or fp32
// stores; a non-finite result is stored and raises `bit` when err is set
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, uint32_t splits, uint64_t slab,
                                                            uint64_t quads, void* out, uint32_t out_f32, uint32_t* err,
                                                            uint32_t bit) {
  bool bad = false;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < quads; i += (uint64_t)gridDim.x * blockDim.x) {
    v4f s = *reinterpret_cast<const v4f*>(ws + 4 * i);
    for (uint32_t q = 1; q < splits; ++q) s += *reinterpret_cast<const v4f*>(ws + q * slab + 4 * i);
    bad |= !(__builtin_isfinite(s[0]) && __builtin_isfinite(s[1]) && __builtin_isfinite(s[2]) && __builtin_isfinite(s[3]));
    if (out_f32) {
      *reinterpret_cast<v4f*>(static_cast<float*>(out) + 4 * i) = s;
    } else {
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + 4 * i) =
          uint2{f32x2_to_bf16x2(s[0], s[1]), f32x2_to_bf16x2(s[2], s[3])};
    }
  }
  if (err && __builtin_amdgcn_ballot_w64(bad) && (threadIdx.x & 63) == 0) atomicOr(err, bit);
}

}  // namespace

uint32_t DenseKSplits(uint32_t m, uint32_t n, uint32_t k_steps) {
  // a split is worth it below one 128 x 256 tile per CU (256 CUs); the
  // smallest split count that reaches a full round, with at least 8 K steps
  // per split, else the largest such count (a GEMM of few tiles: M 128,
  // 12288 -> 4096 has 16)
  const uint64_t tiles = (uint64_t)((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  if (tiles == 0 || tiles >= 192) return 1;
  uint32_t best = 1;
  for (uint32_t s = 2; s <= 8; ++s) {
    if (k_steps % s || k_steps / s < 8) continue;
    if (tiles * s >= 192) return s;
    best = s;
  }
  return best;
}

St LaunchSplitKReduce(const float* ws, uint32_t splits, uint32_t m, uint32_t n, void* out, OutKind out_kind,
                      uint32_t* err, uint32_t bit, hipStream_t stream) {
  if (!ws || !out || !stream || splits < 2 || m == 0 || n == 0 || n % 4) return Invalid("split_k_reduce_invalid");
  const uint64_t count = (uint64_t)m * n, quads = count / 4;
  const uint32_t grid = (uint32_t)std::min<uint64_t>((quads + 255) / 256, 4096);
  St s = RequireCleanLastError();
  if (!s.ok()) return s;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(grid), dim3(256), 0, stream, ws, splits, count, quads, out,
                     out_kind == kOutF32 ? 1u : 0u, err, bit);
  return AfterLaunch("split_k_reduce_launch_failed");
}

}  // namespace pih_amd
