// Light-expert MoE GEMM for gfx950 with MXFP4 weights: the experts that
// received few routed rows (decode batches), e2m1 weights two per byte (low
// nibble = even k) with a UE8M0 scale per (W row, 32 k), activations e4m3
// with a UE8M0 scale per (row, 128 k) or bf16.
//
//   out[row, :] = A[gather[row], :] . W[e]^T   for the rows of expert e
//
// Per element the arithmetic of the tiled kFp4 / kBf16Fp4 kinds of
// gemm_mfma.hip (reference src/model/deepseek_fp4_gemm_oracle.cpp:11-91):
// e4m3 activations use the MX-FP4 MFMA with both UE8M0 scales in the
// instruction's E8M0 operands; bf16 activations multiply the exact bf16
// decode of the weights (v_cvt_scalef32_pk_bf16_fp4 applies the scale).
// Expert segments come from the device route plan (the reference's host
// plan deepseek_expert_subwave_plan.cpp:32-101).
//
// A light expert's work is weight streaming, and the kernel is built for
// that (the 128-row tiles of gemm_mfma.hip spend most of their loads on
// dead activation rows when an expert has a few rows):
//   * a block of 4 waves owns 128 W rows of one light expert (<= 64 rows)
//     and up to 32 (e4m3) or 16 (bf16) of its rows (an expert with more
//     is two to four items); each wave owns 32 W rows (two 16-row MFMA
//     fragments) and loads them into registers,
//     non-temporal, 3-4 steps of 256 k ahead, as whole 128-byte lines (8
//     rows x 128 B per instruction, four per step: the MFMA operand layout,
//     16 rows x 64 B per instruction, streams ~25 % slower from HBM); a
//     wave-private LDS tile turns each step into the operand layout (lane
//     (lr, lg): row lr, bytes [16lg, +16) and [64 + 16lg, +16) of the row's
//     128-byte step, the 32 k of sub-step 0 and of sub-step 1 that the
//     lane's group multiplies);
//   * the expert's activation rows (only the 16-row groups it has: staging
//     loads cost as much as the weight stream when a tile is mostly dead
//     rows) go through a double-buffered LDS tile
//     with XOR-swizzled 16-byte slots (chunk c of row r in slot c ^ (r & 15):
//     16 rows read at one chunk hit 64 distinct banks), loaded kDepth steps
//     ahead together with the weights -- every vector load shares one
//     in-order completion counter, so a younger activation load would make
//     its wait cover every older weight load too;
//   * block scales (unrolled K loops) come 4 steps at a time through LDS:
//     one global->LDS DMA per wave carries its 32 rows x 32 B of weight
//     scales, one of wave 0 the 32 activation rows x 8 B (e4m3).  Loaded
//     per step, 8 bytes of 16 rows per instruction, they touched as many
//     cache lines as the weights themselves (t64 gate/up 178 -> 157 us);
//   * the output is computed transposed (C^T = W . A^T): a lane owns 4
//     consecutive output columns of one row; for the SwiGLU epilogue a
//     wave's fragment 0 holds 16 gate rows and fragment 1 the 16 matching
//     up rows, so each lane owns gate/up pairs.
// The tiled kernels take the heavier experts (their tile scan skips the
// light ones), so every row is produced by exactly one kernel.
#include <type_traits>

#include "device_common.hpp"
#include "kernels.hpp"

namespace pih_amd {
namespace {

constexpr int NTH = 256;    // 4 waves
constexpr int BNW = 128;    // W rows per block
constexpr int KSTEP = 256;  // k per step: 128 weight bytes per row
constexpr uint32_t kWPitch = 144;  // W tile row: one 128-byte step + pad

template <int ACT>
struct Act {
  // rows per pass: a light expert with more rows is done in row chunks
  // (adjacent items, so the later passes over the weights meet them in the
  // caches).  32 (e4m3) and 16 (bf16, 512-byte activation rows) keep the
  // unrolled loops at 3 blocks per CU (<= 168 registers, ~43 KB of LDS;
  // bf16 at K = 7168 stays at 2 for its registers); 64 / 32 held them at 2
  // (64-token layer: e4m3 gate/up 178 -> 148 us with the scale DMA, bf16
  // 223 -> 188 us).
  static constexpr uint32_t MAXR = ACT == kActBf16 ? 16 : 32;
  static constexpr uint32_t ROW = ACT == kActBf16 ? 512 : 256;  // activation bytes per row and step
  static constexpr uint32_t CHUNKS = MAXR * ROW / 16 / NTH;     // 16-byte chunks per thread and step
  static constexpr uint32_t RPI = NTH * 16 / ROW;               // rows per staging instruction
};

struct StreamParams {
  const void* a;
  const uint8_t* a_scale;
  const uint32_t* a_gather;
  const uint8_t* w;
  const uint8_t* w_scale;
  void* out;
  const float* row_weight;
  const uint32_t* offsets;
  uint32_t* err;
  uint32_t m, n, k, experts, a_rows_total;
  uint64_t out_row_stride;
  uint32_t nblk;  // W blocks of BNW rows per expert (SwiGLU: BNW/2 columns each)
  float limit;
};

__device__ __forceinline__ v8i cat8(v4i x, v4i y) {
  return v8i{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
}

// non-zero when any byte of w is 0xFF (a NaN UE8M0 scale)
__device__ __forceinline__ uint32_t ff_bytes(uint32_t w) {
  const uint32_t n = ~w;
  return (n - 0x01010101u) & ~n & 0x80808080u;
}

// Block -> (expert, first row, rows, W block) over the light experts only
// (1 <= rows <= kMoeLightRows).  An expert with more than max_rows rows is
// done in ceil(rows / max_rows) row chunks; items are numbered expert-major,
// then W block, then row chunk, so that the chunks of one W block (which
// stream the same weights) run next to each other, and neighbouring W
// blocks of one expert share its activation rows in L2.  The items are
// split into 8 equal contiguous ranges, one per XCD (blocks b % 8).
// Needs gridDim.x >= 8 * ceil(items / 8).
__device__ bool light_item(const StreamParams& p, uint32_t max_rows, uint32_t& expert, uint32_t& row0,
                           uint32_t& rows, uint32_t& wb) {
  __shared__ uint32_t s_wave[NTH / 64];
  __shared__ uint32_t s_res[2];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t E = p.experts;
  const uint32_t per_t = (E + NTH - 1) / NTH;
  auto chunks = [&](uint32_t lo, uint32_t hi) -> uint32_t {
    return (hi > lo && hi - lo <= kMoeLightRows) ? (hi - lo + max_rows - 1) / max_rows : 0u;
  };
  uint32_t cnt = 0;
  for (uint32_t j = 0; j < per_t; ++j) {
    const uint32_t e = tid * per_t + j;
    if (e < E) cnt += chunks(p.offsets[e], p.offsets[e + 1]);
  }
  uint32_t incl = cnt;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t v = __shfl_up(incl, off, 64);
    if ((int)lane >= off) incl += v;
  }
  if (lane == 63) s_wave[wave] = incl;
  if (tid == 0) s_res[0] = 0xffffffffu;
  __syncthreads();
  uint32_t before = 0, light = 0;
#pragma unroll
  for (int w = 0; w < NTH / 64; ++w) {
    const uint32_t v = s_wave[w];
    if (w < (int)wave) before += v;
    light += v;
  }
  incl += before;
  const uint32_t excl = incl - cnt;  // in row chunks
  const uint32_t total = light * p.nblk;
  const uint32_t per = (total + 7) / 8;
  const uint32_t xcd = blockIdx.x & 7, jj = blockIdx.x >> 3;
  const uint32_t t = xcd * per + jj;
  if (jj >= per || t >= total) return false;  // same for every thread
  // the expert whose items [nblk * c0, nblk * (c0 + c)) contain t, where c0
  // is its first chunk ordinal and c its chunk count
  if (t >= excl * p.nblk && t < incl * p.nblk) {
    uint32_t c0 = excl;
    for (uint32_t j = 0; j < per_t; ++j) {
      const uint32_t e = tid * per_t + j;
      if (e >= E) break;
      const uint32_t c = chunks(p.offsets[e], p.offsets[e + 1]);
      if (t < (c0 + c) * p.nblk) {
        s_res[0] = e;
        s_res[1] = c0;
        break;
      }
      c0 += c;
    }
  }
  __syncthreads();
  const uint32_t e = s_res[0];
  if (e == 0xffffffffu) return false;
  const uint32_t lo = p.offsets[e], hi = p.offsets[e + 1];
  if (hi > p.m || lo > hi) {
    if (tid == 0) atomicOr(p.err, kErrCode);
    return false;
  }
  const uint32_t c = (hi - lo + max_rows - 1) / max_rows;
  const uint32_t local = t - s_res[1] * p.nblk;
  expert = e;
  wb = local / c;
  row0 = lo + (local % c) * max_rows;
  rows = min(max_rows, hi - row0);
  return true;
}

// KBT > 0: the K loop has exactly KBT steps and is unrolled completely (the
// compiler's load waits are then exact; a loop header makes them
// conservative and drains the pipeline once per trip).  KBT == 0: any K.
template <int ACT, int OUT, int KBT>
__global__ __launch_bounds__(NTH, 2) void fp4_moe_stream_kernel(StreamParams p) {
  using C = Act<ACT>;
  constexpr uint32_t MAXR = C::MAXR, ROW = C::ROW, CH = C::CHUNKS, NA = MAXR / 16;
  static_assert(NA == (ACT == kActBf16 ? 1 : 2), "activation fragments per chunk");
  // steps in flight per wave: 3 with an unrolled K loop (the ring then fits
  // the 256 registers of two waves per SIMD), 4 in the generic loop (whose
  // 8-step body needs a depth dividing 8)
  constexpr int kDepth = KBT > 0 ? 3 : 4;
  // whether a chunk of <= 16 rows takes a path computing only its one live
  // activation fragment (the second copy of the step's code fits the
  // registers of the unrolled e4m3 loops and of the short bf16 loop)
  constexpr bool kLiveSplit = KBT > 0 && !(ACT == kActBf16 && KBT > 8);
  constexpr uint32_t CPR = ROW / 16;  // chunks per activation row
  constexpr uint32_t RPI = C::RPI;    // staging instruction i covers rows [i RPI, (i + 1) RPI)
  __shared__ __align__(16) uint8_t sA[2][MAXR * ROW];
  __shared__ __align__(16) uint32_t sSa[2][MAXR];  // e4m3: the row's 2 scale bytes of the step
  __shared__ __align__(16) uint8_t sW[NTH / 64][32 * kWPitch];  // per wave: its 32 W rows of one step
  // weight scales, unrolled K loops: per wave two buffers of [32 rows][32 B]
  // (4 steps each), filled by one global->LDS DMA per 4 steps
  constexpr bool kScaleDma = KBT > 0 && KBT % 4 == 0;
  __shared__ __align__(16) uint8_t sWs[kScaleDma ? NTH / 64 : 1][2][32 * 32];
  // e4m3 activation scales of the same 4 steps, [MAXR rows][8 B], two
  // buffers filled by wave 0 (one 4-byte DMA per lane: row lane / 2)
  constexpr bool kActScaleDma = kScaleDma && ACT == kActE4m3;
  __shared__ __align__(16) uint8_t sSaC[kActScaleDma ? 2 : 1][kActScaleDma ? MAXR * 8 : 4];
  static_assert(!kActScaleDma || MAXR * 2 == 64, "one activation-scale DMA covers the chunk");

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t lr = lane & 15, lg = lane >> 4;

  uint32_t expert, row0, rows, wb;
  if (!light_item(p, MAXR, expert, row0, rows, wb)) return;
  expert = __builtin_amdgcn_readfirstlane(expert);
  row0 = __builtin_amdgcn_readfirstlane(row0);
  rows = __builtin_amdgcn_readfirstlane(rows);
  wb = __builtin_amdgcn_readfirstlane(wb);
  // live 16-row activation fragments of this chunk (wave-uniform)
  const uint32_t na_live = __builtin_amdgcn_readfirstlane((rows + 15) / 16);

  const uint32_t K = p.k, KB = K / KSTEP, last = KB - 1;
  uint32_t bad = 0;

  // Addresses: wave-uniform base (scalar registers, advanced per step) plus
  // a 32-bit per-lane offset (the host checks that the spans fit).
  // Activation tile row r reads the gathered row of logical row row0 + r;
  // rows past the expert read its first row (in bounds, never stored).
  auto a_source = [&](uint32_t r) -> uint32_t {
    const uint32_t logical = row0 + (r < rows ? r : 0u);
    const uint32_t src = p.a_gather ? p.a_gather[logical] : logical;
    if (src >= p.a_rows_total) {
      bad |= kErrCode;
      return 0;
    }
    return src;
  };
  const uint32_t a_row_bytes = K * (ACT == kActBf16 ? 2u : 1u);
  uint32_t a_off[CH], a_st[CH];
#pragma unroll
  for (uint32_t i = 0; i < CH; ++i) {
    const uint32_t q = tid + NTH * i, r = q / CPR, c = q % CPR;
    a_off[i] = a_source(r) * a_row_bytes + c * 16;
    a_st[i] = r * ROW + ((c ^ (r & 15u)) << 4);
  }
  // activation scales (e4m3): thread t < MAXR loads the 2 bytes of row t
  const uint32_t s_off = a_source(tid < MAXR ? tid : 0u) * (K / 128);

  // W rows of this wave: fragment f, fragment row r
  auto w_row = [&](uint32_t f, uint32_t r) -> uint32_t {
    if constexpr (OUT == kOutSwiGlu) {
      const uint32_t c = wb * (BNW / 2) + wave * 16 + r;  // output column
      return f ? p.n / 2 + c : c;
    } else {
      return wb * BNW + wave * 32 + f * 16 + r;
    }
  };
  const uint8_t* w_base = p.w + (uint64_t)expert * p.n * (K / 2);
  const uint8_t* ws_base = p.w_scale + (uint64_t)expert * p.n * (K / 32);
  // line load i: tile row 8i + lane / 8 (fragment i / 2, fragment row
  // 8 (i % 2) + lane / 8), bytes 16 (lane % 8) of the step.  The rows of
  // fragment 1 sit a uniform distance after those of fragment 0, so each
  // load is one per-lane offset plus a wave-uniform one.
  const uint32_t frag_rows = OUT == kOutSwiGlu ? p.n / 2 : 16u;
  const uint32_t w_off = w_row(0, lane >> 3) * (K / 2) + (lane & 7) * 16;
  const uint32_t ws_off = w_row(0, lr) * (K / 32);
  const uint32_t ws_d1 = frag_rows * (K / 32);
  // scale DMA: lane q carries 16 bytes of tile row q / 2 (fragment q / 32)
  const uint32_t sq_row = lane >> 1;
  const uint32_t ws_dma = w_row(sq_row >> 4, sq_row & 15) * (K / 32) + 16 * (lane & 1);
  const uint32_t ws_lds0 = kScaleDma ? lds_addr(&sWs[kScaleDma ? wave : 0][0][0]) : 0u;
  // activation scale DMA: lane q carries the 4 bytes [4 (q & 1), +4) of row
  // q / 2's 8 bytes of the chunk (K / 128 is a multiple of 4 when KBT is)
  const uint32_t sa_dma = kActScaleDma ? a_source(lane >> 1) * (K / 128) + 4 * (lane & 1) : 0u;
  const uint32_t sa_lds0 = kActScaleDma ? lds_addr(&sSaC[0][0]) : 0u;
  uint8_t* wtile = sW[wave];

  v4i rl[kDepth][4];     // weight lines of the step (tile rows 8i .. 8i + 7)
  uint2 rws[kDepth][2];  // weight scales of the step (8 bytes per row)
  v4i ra[kDepth][CH];    // activation chunks
  uint32_t rsa[kDepth];  // activation scales (e4m3)
  auto load = [&](int slot, uint32_t kb) __attribute__((always_inline)) {
    const uint32_t kc = min(kb, last);
    if constexpr (kScaleDma) {
      // chunk kb / 4 into buffer (kb / 4) & 1, ahead of the step's own loads
      // (so the wait for them covers it; the compiler does not count it)
      if (kb % 4 == 0 && kb < KBT) dma16(ws_base + 8 * kb, ws_dma, ws_lds0 + ((kb / 4) & 1) * 1024);
    }
    if constexpr (kActScaleDma) {
      if (kb % 4 == 0 && kb < KBT && wave == 0)
        dma4(p.a_scale + 2 * kb, sa_dma, sa_lds0 + ((kb / 4) & 1) * (MAXR * 8));
    }
    const uint8_t* wb8 = w_base + (uint64_t)kc * 128;
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
      const uint8_t* line = wb8 + (uint64_t)((i & 1) * 8 + (i >> 1) * frag_rows) * (K / 2);  // wave-uniform
      rl[slot][i] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(line + w_off));
    }
    if constexpr (!kScaleDma) {
      const uint8_t* sb8 = ws_base + (uint64_t)kc * 8;
      rws[slot][0] = *reinterpret_cast<const uint2*>(sb8 + ws_off);
      rws[slot][1] = *reinterpret_cast<const uint2*>(sb8 + ws_d1 + ws_off);
    }
    // only the staging instructions that cover live rows (the tile rows past
    // the expert's are never stored; their LDS contents are left stale)
    const uint8_t* ab = static_cast<const uint8_t*>(p.a) + (uint64_t)kc * ROW;
#pragma unroll
    for (uint32_t i = 0; i < CH; ++i) {
      v4i v = v4i{0, 0, 0, 0};  // defined on both paths: the old ring value dies here
      if (i == 0 || i * RPI < rows) v = *reinterpret_cast<const v4i*>(ab + a_off[i]);
      ra[slot][i] = v;
    }
    if constexpr (ACT == kActE4m3 && !kActScaleDma) {
      // the 2 scale bytes of the step, from the aligned 32-bit word that
      // holds them (s_off + 2 kc is even): a full-register load, so the
      // compiler cannot pack it into a half register whose wait would then
      // cover younger loads
      const uint32_t at = s_off + 2 * kc;
      rsa[slot] = *reinterpret_cast<const uint32_t*>(p.a_scale + (at & ~3u)) >> (8 * (at & 3u));
    }
  };
  auto stage = [&](int slot, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t i = 0; i < CH; ++i)
      if (i == 0 || i * RPI < rows) *reinterpret_cast<v4i*>(&sA[buf][a_st[i]]) = ra[slot][i];
    if constexpr (ACT == kActE4m3 && !kActScaleDma) {
      if (tid < MAXR) {
        const uint32_t v = rsa[slot] & 0xffffu;
        sSa[buf][tid] = v;
        if (tid < rows && ((v & 0xffu) == 0xffu || (v >> 8) == 0xffu)) bad |= kErrScale;
      }
    }
  };

  v4f acc[2][NA];  // [W fragment][activation fragment]
#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (uint32_t r = 0; r < NA; ++r) acc[f][r] = v4f{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int slot, int buf, uint32_t kb) __attribute__((always_inline)) {
    if constexpr (kScaleDma) {
      // this step's 8 scale bytes of rows f*16 + lr (the DMA completed before
      // the step's own loads did, which the staging above waited for)
#pragma unroll
      for (int f = 0; f < 2; ++f)
        rws[slot][f] = *reinterpret_cast<const uint2*>(&sWs[wave][(kb / 4) & 1][(f * 16 + lr) * 32 + 8 * (kb % 4)]);
    }
#pragma unroll
    for (int f = 0; f < 2; ++f)
      if (ff_bytes(rws[slot][f].x) | ff_bytes(rws[slot][f].y)) bad |= kErrScale;
    // the step's lines through the wave's tile into the operand layout (a
    // wave's LDS accesses complete in order: no barrier)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<v4i*>(wtile + (8 * i + (lane >> 3)) * kWPitch + (lane & 7) * 16) = rl[slot][i];
    // fragment f, sub-step s: row f*16 + lr, bytes 64 s + 16 lg (read where
    // used, so only the current sub-step's weights occupy registers)
    auto wfrag = [&](int f, int s) -> v4i {
      return *reinterpret_cast<const v4i*>(wtile + (f * 16 + lr) * kWPitch + s * 64 + lg * 16);
    };
    if constexpr (ACT == kActE4m3) {
      auto frag = [&](auto R) __attribute__((always_inline)) {
        constexpr int r = decltype(R)::value;
        const uint32_t row = r * 16 + lr;
        const uint8_t* pa = &sA[buf][row * ROW];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          // FP8 operand: chunks 8s + lg and 8s + 4 + lg of the row
          const uint32_t c0 = 8 * s + lg, c1 = c0 + 4;
          const v8i af = cat8(*reinterpret_cast<const v4i*>(pa + ((c0 ^ lr) << 4)),
                              *reinterpret_cast<const v4i*>(pa + ((c1 ^ lr) << 4)));
          int sa;
          if constexpr (kActScaleDma) {
            // rows past the chunk's hold row 0's scales (a_source)
            sa = sSaC[(kb / 4) & 1][row * 8 + 2 * (kb % 4) + s];
            if (sa == 0xff) bad |= kErrScale;
          } else {
            sa = (int)((sSa[buf][row] >> (8 * s)) & 0xffu);
          }
#pragma unroll
          for (int f = 0; f < 2; ++f) {
            const v4i w4 = wfrag(f, s);
            const int sw = (int)(((s ? rws[slot][f].y : rws[slot][f].x) >> (8 * lg)) & 0xffu);
            acc[f][r] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(cat8(w4, v4i{0, 0, 0, 0}), af, acc[f][r],
                                                                         4, 0, 0, sw, 0, sa);
          }
        }
      };
      // a chunk of <= 16 rows (most decode experts) computes its one live
      // 16-row activation fragment only: the dead fragments' LDS reads and
      // MFMAs cost more than the weight stream (rows past the chunk's in a
      // live fragment hold stale data and are never stored)
      frag(std::integral_constant<int, 0>{});
      if (!kLiveSplit || na_live > 1) {
        frag(std::integral_constant<int, 1>{});
      }
    } else {
      // bf16: MFMA j of sub-step s multiplies k 32lg + 8j .. +7 of the
      // sub-step: weight dword 4s + j (8 nibbles, low first), converted once
      // per fragment, against chunk 16s + 4lg + j of each activation row
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const v4i w4[2] = {wfrag(0, s), wfrag(1, s)};
        float sc[2];
#pragma unroll
        for (int f = 0; f < 2; ++f) sc[f] = ue8m0_value(((s ? rws[slot][f].y : rws[slot][f].x) >> (8 * lg)) & 0xffu);
        // a chunk of <= 16 rows reads and multiplies its one live
        // activation fragment only (a uniform branch around whole copies
        // of the loop, so every fragment index stays a constant)
        auto body = [&](auto NL) __attribute__((always_inline)) {
          constexpr uint32_t nl = decltype(NL)::value;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t c = 16 * s + 4 * lg + j;
            v4i av[nl];
#pragma unroll
            for (uint32_t r = 0; r < nl; ++r)
              av[r] = *reinterpret_cast<const v4i*>(&sA[buf][(r * 16 + lr) * ROW + ((c ^ lr) << 4)]);
#pragma unroll
            for (int f = 0; f < 2; ++f) {
              const uint32_t wd = (uint32_t)w4[f][j];
              const v4i wv{__builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, sc[f], 0)),
                           __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, sc[f], 1)),
                           __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, sc[f], 2)),
                           __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, sc[f], 3))};
#pragma unroll
              for (uint32_t r = 0; r < nl; ++r)
                acc[f][r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, wv),
                                                                    __builtin_bit_cast(v8bf, av[r]), acc[f][r], 0, 0,
                                                                    0);
            }
          }
        };
        if (!kLiveSplit || na_live > 1) body(std::integral_constant<uint32_t, NA>{});
        else body(std::integral_constant<uint32_t, 1>{});
      }
    }
    // Pin this step's results here: the MFMAs read only registers, and the
    // optimiser would otherwise sink them past later barriers, keeping every
    // step's operands live at once.
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
      for (uint32_t r = 0; r < NA; ++r) asm volatile("" : "+v"(acc[f][r]));
  };

  // prologue: steps 0 .. kDepth-1
#pragma unroll
  for (int s = 0; s < kDepth; ++s) load(s, s);

  // Step j: stage step j's activations (loaded kDepth steps ago) into
  // buffer j & 1, barrier (every wave is done with step j - 1's buffer),
  // compute step j, load step j + kDepth into the freed registers.
  if constexpr (KBT > 0) {
#pragma unroll
    for (int j = 0; j < KBT; ++j) {
      stage(j % kDepth, j & 1);
      __syncthreads();
      compute(j % kDepth, j & 1, j);
      // keep the next loads after this step's compute (hoisting them would
      // keep two steps' operands live)
      __builtin_amdgcn_sched_barrier(0);
      if (j + kDepth < KBT) load(j % kDepth, j + kDepth);
    }
  } else {
    // loads past the last step re-read it (in bounds, never used)
#define PIH_STREAM_STEP(J, TAIL)      \
  {                                   \
    const uint32_t j = kb + (J);      \
    if ((TAIL) && j >= KB) goto done; \
    stage((J) % kDepth, (J) & 1);     \
    __syncthreads();                  \
    compute((J) % kDepth, (J) & 1, j); \
    load((J) % kDepth, j + kDepth);   \
  }
    uint32_t kb = 0;
    for (; kb + 8 < KB; kb += 8) {
      PIH_STREAM_STEP(0, false)
      PIH_STREAM_STEP(1, false)
      PIH_STREAM_STEP(2, false)
      PIH_STREAM_STEP(3, false)
      PIH_STREAM_STEP(4, false)
      PIH_STREAM_STEP(5, false)
      PIH_STREAM_STEP(6, false)
      PIH_STREAM_STEP(7, false)
    }
    PIH_STREAM_STEP(0, true)
    PIH_STREAM_STEP(1, true)
    PIH_STREAM_STEP(2, true)
    PIH_STREAM_STEP(3, true)
    PIH_STREAM_STEP(4, true)
    PIH_STREAM_STEP(5, true)
    PIH_STREAM_STEP(6, true)
    PIH_STREAM_STEP(7, true)
#undef PIH_STREAM_STEP
  }
done:

  // ---- epilogue: lane holds out[row r*16 + lr][4*lg + i] of fragment f
#pragma unroll
  for (uint32_t r = 0; r < NA; ++r) {
    const uint32_t rr = r * 16 + lr;
    if (rr >= rows) continue;
    const uint64_t orow = (uint64_t)(row0 + rr) * p.out_row_stride;
    if constexpr (OUT == kOutSwiGlu) {
      const float rwt = p.row_weight ? p.row_weight[row0 + rr] : 1.0f;
      uint32_t o[4];
      bool ok = true;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float gt = bf16_round(acc[0][r][i]);
        float up = bf16_round(acc[1][r][i]);
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
      uint16_t* dst = static_cast<uint16_t*>(p.out) + orow + wb * (BNW / 2) + wave * 16 + 4 * lg;
      if (ok) {
        *reinterpret_cast<uint2*>(dst) = uint2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
      } else {
        bad |= kErrNonFinite;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (o[i] != 0xffffffffu) dst[i] = (uint16_t)o[i];
      }
    } else {
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const uint32_t col = wb * BNW + wave * 32 + f * 16 + 4 * lg;
        const v4f v = acc[f][r];
        const bool fin = __builtin_isfinite(v[0]) && __builtin_isfinite(v[1]) && __builtin_isfinite(v[2]) &&
                         __builtin_isfinite(v[3]);
        if constexpr (OUT == kOutF32) {
          float* dst = static_cast<float*>(p.out) + orow + col;
          if (fin) {
            *reinterpret_cast<v4f*>(dst) = v;
          } else {
            bad |= kErrNonFinite;
            for (int i = 0; i < 4; ++i)
              if (__builtin_isfinite(v[i])) dst[i] = v[i];
          }
        } else {
          uint16_t* dst = static_cast<uint16_t*>(p.out) + orow + col;
          if (fin) {
            *reinterpret_cast<uint2*>(dst) = uint2{f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16),
                                                   f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16)};
          } else {
            bad |= kErrNonFinite;
            for (int i = 0; i < 4; ++i)
              if (__builtin_isfinite(v[i])) dst[i] = (uint16_t)f32_to_bf16_bits(v[i]);
          }
        }
      }
    }
  }
  if (bad) atomicOr(p.err, bad);
}

template <int ACT, int KBT>
void launch_kb(const StreamParams& sp, uint32_t grid, hipStream_t s, OutKind out) {
  if (out == kOutSwiGlu)
    hipLaunchKernelGGL((fp4_moe_stream_kernel<ACT, kOutSwiGlu, KBT>), dim3(grid), dim3(NTH), 0, s, sp);
  else if (out == kOutF32)
    hipLaunchKernelGGL((fp4_moe_stream_kernel<ACT, kOutF32, KBT>), dim3(grid), dim3(NTH), 0, s, sp);
  else
    hipLaunchKernelGGL((fp4_moe_stream_kernel<ACT, kOutBf16, KBT>), dim3(grid), dim3(NTH), 0, s, sp);
}

// fully unrolled K loops for the DeepSeek shapes (K = 7168: 28 steps, the
// V3-shaped gate/up of BASELINE configs[4]; K = 4096: 16 steps, the
// V4-Flash gate/up at hidden 4096, include/pih/model/deepseek_v4_config.h:22;
// K = 2048: 8 steps, both down projections), a loop otherwise
template <int ACT>
void launch_out(const StreamParams& sp, uint32_t grid, hipStream_t s, OutKind out) {
  const uint32_t kb = sp.k / KSTEP;
  if (kb == 28) launch_kb<ACT, 28>(sp, grid, s, out);
  else if (kb == 16) launch_kb<ACT, 16>(sp, grid, s, out);
  else if (kb == 8) launch_kb<ACT, 8>(sp, grid, s, out);
  else launch_kb<ACT, 0>(sp, grid, s, out);
}

}  // namespace

uint32_t Fp4MoeLightRows(const Fp4GemmArgs& a) {
  const uint64_t a_row = (uint64_t)a.k * (a.act == kActBf16 ? 2 : 1);
  const bool fits = a.moe && a.k % KSTEP == 0 && a.n % BNW == 0 &&
                    (uint64_t)a.a_rows_total * a_row < (1ull << 32) && (uint64_t)a.n * (a.k / 2) < (1ull << 32) &&
                    (uint64_t)a.n * (a.k / 32) < (1ull << 32);
  if (!fits) return 0;
  return kMoeLightRows;
}

// Called by LaunchFp4Gemm after its checks, for the light experts of a MoE
// problem (Fp4MoeLightRows(a) > 0).
St LaunchFp4MoeStream(const Fp4GemmArgs& a) {
  StreamParams sp{};
  sp.a = a.a;
  sp.a_scale = a.a_scale;
  sp.a_gather = a.a_gather;
  sp.w = a.w;
  sp.w_scale = a.w_scale;
  sp.out = a.out;
  sp.row_weight = a.row_weight;
  sp.offsets = a.offsets;
  sp.err = a.error_flag;
  sp.m = a.m;
  sp.n = a.n;
  sp.k = a.k;
  sp.experts = a.problems;
  sp.a_rows_total = a.a_rows_total;
  sp.out_row_stride = a.out_kind == kOutSwiGlu ? a.n / 2 : a.n;
  sp.nblk = a.n / BNW;
  sp.limit = a.swiglu_limit;
  // row chunks: at most one per non-empty expert plus rows / (rows per pass)
  const uint64_t per_pass = a.act == kActBf16 ? Act<kActBf16>::MAXR : Act<kActE4m3>::MAXR;
  const uint64_t light = (a.problems < a.m ? a.problems : a.m) + a.m / per_pass;
  const uint64_t total = light * sp.nblk;
  if (total == 0 || total > 0x7fffffffull - 8) return Invalid("fp4_moe_stream_grid_too_large");
  const uint32_t grid = (uint32_t)((total + 7) / 8 * 8);
  if (a.act == kActE4m3) launch_out<kActE4m3>(sp, grid, a.stream, a.out_kind);
  else launch_out<kActBf16>(sp, grid, a.stream, a.out_kind);
  return AfterLaunch("fp4_moe_stream_launch_failed");
}

}  // namespace pih_amd
