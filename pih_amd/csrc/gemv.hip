// Decode GEMV for gfx950: y[m, n] = sum_k x[m, k] * W[n, k] for small m
// (1..64), with W in bf16 or INT4 (W4A16, symmetric reference format or
// asymmetric u32-packed format).  Memory-bound: the kernel streams W once.
//
// Three kernels: gemv_lds_kernel for M <= 4 (x staged in LDS per wave),
// gemv_mid_kernel for 4 < M <= 64 (W and x read as whole 128-byte lines and
// turned into the MFMA layout in LDS), and gemv_kernel, described here, for
// the shapes whose K does not split evenly over the others' waves.
//
// Layout of the work: a block owns 16 W rows (one MFMA column block) and
// its 4, 8 or 16 waves split K into contiguous runs (more waves for small N,
// so every shape keeps ~2048 waves streaming).  Each lane loads 16
// contiguous bytes of a W row per step (lanes 16g..16g+15 take the g-th
// 16-byte piece of 16 different rows), so a wave-wide load covers 16 rows x
// 64 bytes, and a wave issues U steps of loads before consuming them.  The
// x operand comes from global memory (small, L2-resident); rows m >= M of
// the 16-row MFMA tile are zero.
//   bf16 : one v_mfma_f32_16x16x32_bf16 per 16-byte W piece.
//   INT4 : one 16-byte piece is 32 nibbles = a quarter of a 128-deep quant
//          group per lane group, so a wave-wide load covers exactly one
//          group of 16 rows; the nibbles are unpacked to exact small
//          integers (q - z) in bf16, four MFMAs accumulate
//          sum_k x * (q - z) over the group, and the group's scale is
//          applied once: acc += s[n, g] * partial.  The unpack is the same
//          function the dequant entry uses (pinned bit-exact by tests).
// Reduction: the block's waves through LDS in fixed wave order.  There is
// no split across blocks: combining blocks needs a device-scope fence, which
// on gfx950 writes back and invalidates L2 and cost more than the GEMV.
//
// Error reporting for INT4 follows the reference kernel
// (kernels/cuda/qwen_bf16_primitives.cu:98-149): the first failure's code
// is stored with compare-and-swap from 0: 12 reserved nibble (symmetric
// format), 13 scale not finite and positive, 14 non-finite output.
#include "device_common.hpp"
#include "kernels.hpp"

namespace pih_amd {
namespace {

enum WFmt : int { kWBf16 = 0, kWSym = 1, kWAsym = 2 };

constexpr uint32_t kQwenReservedNibble = 12, kQwenBadScale = 13, kQwenNonFinite = 14;

struct GemvParams {
  const uint16_t* x;
  const void* w;
  const uint16_t* scales;
  const uint32_t* zeros;
  void* out;
  uint32_t* err;
  uint32_t m, n, k;
  uint32_t out_f32;
  uint32_t nonfinite_or;  // bf16 weights: OR'd into *err for a non-finite output (0: none)
};

// K elements one wave consumes per 16-byte-per-lane load step.
template <int FMT>
constexpr uint32_t step_k() {
  return FMT == kWBf16 ? 32u : 128u;
}

__device__ __forceinline__ void publish(uint32_t* err, uint32_t code) { atomicCAS(err, 0u, code); }

// Unpack 32 nibbles (one 16-byte piece, nibble j = k offset j) into
// bf16 bit patterns of the exact integers (q - z) (asym) or q (sym).
// Returns false when a symmetric nibble is the reserved code 8.
template <int FMT>
__device__ __forceinline__ bool unpack32(uint4 piece, int zero, v8s out[4]) {
  const uint32_t w[4] = {piece.x, piece.y, piece.z, piece.w};
  bool ok = true;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int nib = (int)((w[i] >> (4 * j)) & 0xfu);
      int q;
      if constexpr (FMT == kWSym) {
        if (nib == 8) ok = false;
        q = nib < 8 ? nib : nib - 16;
      } else {
        q = nib - zero;
      }
      // |q| <= 15: exact in bf16, built from the fp32 bits
      out[i][j] = (short)(__float_as_uint((float)q) >> 16);
    }
  }
  return ok;
}

template <int FMT, int MT, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(GemvParams p) {
  __shared__ float s_red[WAVES][MT][4][64];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t lr = lane & 15, lg = lane >> 4;
  const uint32_t n0 = blockIdx.x * 16;
  const uint32_t nrow = n0 + lr;  // W row this lane loads
  constexpr uint32_t SK = step_k<FMT>();
  const uint32_t k_begin = 0;
  const uint32_t steps = p.k / SK;
  v4f acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  uint32_t bad = 0;

  // Each wave owns a contiguous run of steps; U steps at a time it issues
  // every weight (and x) load first and only then unpacks and multiplies,
  // so U x 16 bytes per lane are in flight per wave.
  // (1024-thread blocks leave 128 VGPRs per lane: INT4 batches shrink there)
  constexpr int U = FMT == kWBf16 ? (MT == 1 ? 8 : MT == 2 ? 4 : 2)
                                  : (WAVES == 16 ? (MT == 1 ? 2 : 1) : (MT == 1 ? 4 : 2));
  constexpr int XL = FMT == kWBf16 ? 1 : 4;  // x loads per step per M tile
  const uint32_t spw = (steps + WAVES - 1) / WAVES;
  const uint32_t s_begin = min(steps, wave * spw), s_end = min(steps, s_begin + spw);
  const uint32_t zwords = (p.k / 128 + 7) / 8;
  auto w_piece = [&](uint32_t k0) -> v4i {
    if constexpr (FMT == kWBf16)
      return *reinterpret_cast<const v4i*>(static_cast<const uint16_t*>(p.w) + (uint64_t)nrow * p.k + k0 + lg * 8);
    else if constexpr (FMT == kWSym)
      return *reinterpret_cast<const v4i*>(static_cast<const uint8_t*>(p.w) + (uint64_t)nrow * (p.k / 2) + k0 / 2 +
                                           lg * 16);
    else
      return *reinterpret_cast<const v4i*>(static_cast<const uint32_t*>(p.w) + (uint64_t)nrow * (p.k / 8) + k0 / 8 +
                                           lg * 4);
  };
  auto x_piece = [&](uint32_t t, uint32_t k0, int i) -> v4i {
    const uint32_t mrow = t * 16 + lr;
    if (mrow >= p.m) return v4i{0, 0, 0, 0};
    const uint32_t off = FMT == kWBf16 ? lg * 8 : lg * 32 + i * 8;
    return *reinterpret_cast<const v4i*>(p.x + (uint64_t)mrow * p.k + k0 + off);
  };
  auto step = [&](uint32_t k0, v4i wp, const v4i* xp, float sc, int zero) {
    if constexpr (FMT == kWBf16) {
#pragma unroll
      for (int t = 0; t < MT; ++t)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, xp[t]),
                                                         __builtin_bit_cast(v8bf, wp), acc[t], 0, 0, 0);
    } else {
      // One 128-deep quant group: lane group lg owns k0 + 32*lg .. +32.
      // Nibble u becomes the bf16 number 128 + u by OR-ing it into the
      // mantissa of 128 (0x4300 | u), two per 32-bit word, three ALU ops a
      // pair; then sum_k x (u - z) = sum_k x (128 + u) - (128 + z) sum_k x,
      // with sum_k x from one more MFMA against ones.  The symmetric format
      // is u = nibble ^ 8 with z = 8 (4-bit two's complement).
      if (!(sc > 0.0f) || !__builtin_isfinite(sc)) bad = bad ? bad : kQwenBadScale;
      uint32_t wd[4] = {(uint32_t)wp[0], (uint32_t)wp[1], (uint32_t)wp[2], (uint32_t)wp[3]};
      if constexpr (FMT == kWSym) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t t = wd[i] ^ 0x88888888u;  // reserved nibble 8 -> 0
          if ((t - 0x11111111u) & ~t & 0x88888888u) bad = kQwenReservedNibble;
          wd[i] = t;
        }
        zero = 8;
      }
      v4i qb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {
          const uint32_t t = (wd[i] >> (8 * pr)) & 0xffu;
          qb[i][pr] = (int)((t & 0xfu) | ((t & 0xf0u) << 12) | 0x43004300u);
        }
      const v8bf ones = __builtin_bit_cast(v8bf, v4i{0x3f803f80, 0x3f803f80, 0x3f803f80, 0x3f803f80});
      const float zc = 128.0f + (float)zero;
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        v4f pq = v4f{0.f, 0.f, 0.f, 0.f}, p1 = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const v8bf xb = __builtin_bit_cast(v8bf, xp[t * 4 + i]);
          pq = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xb, __builtin_bit_cast(v8bf, qb[i]), pq, 0, 0, 0);
          p1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xb, ones, p1, 0, 0, 0);
        }
        // output column of this lane is n0 + lr: its group scale / zero
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] = __builtin_fmaf(__builtin_fmaf(-zc, p1[i], pq[i]), sc, acc[t][i]);
      }
    }
  };
  auto group_scale = [&](uint32_t k0, float& sc, int& zero) {
    const uint32_t grp = k0 / 128u;
    if constexpr (FMT == kWSym) {
      sc = (float)__builtin_bit_cast(_Float16, p.scales[(uint64_t)nrow * (p.k / 128) + grp]);
      zero = 0;
    } else if constexpr (FMT == kWAsym) {
      zero = (int)((p.zeros[(uint64_t)nrow * zwords + grp / 8] >> (4 * (grp % 8))) & 0xfu);
      sc = bf16_bits_to_f32(p.scales[(uint64_t)nrow * (p.k / 128) + grp]);
    } else {
      sc = 1.0f;
      zero = 0;
    }
  };

  uint32_t st = s_begin;
  for (; st + U <= s_end; st += U) {
    v4i wv[U], xv[U][MT * XL];
    float sc[U];
    int zr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t k0 = k_begin + (st + u) * SK;
      wv[u] = w_piece(k0);
      group_scale(k0, sc[u], zr[u]);
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < XL; ++i) xv[u][t * XL + i] = x_piece(t, k0, i);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) step(k_begin + (st + u) * SK, wv[u], xv[u], sc[u], zr[u]);
  }
  for (; st < s_end; ++st) {
    const uint32_t k0 = k_begin + st * SK;
    v4i xv[MT * XL];
    float sc;
    int zr;
    const v4i wp = w_piece(k0);
    group_scale(k0, sc, zr);
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < XL; ++i) xv[t * XL + i] = x_piece(t, k0, i);
    step(k0, wp, xv, sc, zr);
  }
  if (bad) publish(p.err, bad);

  // ---- reduce the block's waves (fixed order)
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_red[wave][t][i][lane] = acc[t][i];
  __syncthreads();
  // thread -> (t, i, lane) output slot; output element m = t*16 + 4*lg + i,
  // n = n0 + lr; the waves' partial sums are added in wave order
  const uint32_t slots = MT * 4 * 64;
  uint32_t nonfinite = 0;
  for (uint32_t slot = tid; slot < slots; slot += WAVES * 64) {
    const uint32_t t = slot / 256, i = (slot / 64) % 4, l = slot % 64;
    const uint32_t mrow = t * 16 + 4 * (l >> 4) + i, col = n0 + (l & 15);
    if (mrow >= p.m) continue;
    float v = 0.0f;
#pragma unroll
    for (int wv = 0; wv < WAVES; ++wv) v += s_red[wv][t][i][l];
    if (!__builtin_isfinite(v)) nonfinite = 1;
    if (p.out_f32) static_cast<float*>(p.out)[(uint64_t)mrow * p.n + col] = v;
    else static_cast<uint16_t*>(p.out)[(uint64_t)mrow * p.n + col] = (uint16_t)f32_to_bf16_bits(v);
  }
  if (nonfinite && FMT != kWBf16) publish(p.err, kQwenNonFinite);
  if (nonfinite && FMT == kWBf16 && p.nonfinite_or) atomicOr(p.err, p.nonfinite_or);
}

// ---------------------------------------------------------------------------
// Small-M decode GEMV (M <= 4): the path BASELINE decode shapes take.
//
// Same 16-row blocks and MFMA operand layout as gemv_kernel; the waves of a
// block split K into equal runs of spw steps (the host picks WAVES dividing
// the step count and U dividing spw).  What makes it stream near HBM speed
// on gfx950 (each point measured on MI355X with a stripped copy of the
// kernel):
//   * W is read with non-temporal loads: it is used exactly once, and the
//     hint measured ~20 % more streaming bandwidth than plain loads;
//   * a wave loads its own slice of x (rows < M, its K run) first, then its
//     first U steps of W, then writes x to a wave-private LDS area: waiting
//     for x leaves W in flight, and no block barrier precedes the math;
//   * the group scales of a batch arrive in vector loads (U bf16 / fp16
//     values of the lane's row) and the zero points in one or two u32,
//     instead of two scalar-per-step loads that cost more than the nibble
//     math;
//   * even U: W arrives as whole 128-byte lines and turns into the MFMA
//     layout through one wave-private LDS tile, reused pair after pair (one
//     tile instead of U / 2 lets 4 rather than 3 blocks of 4 waves share a
//     CU: Qwen3-8B gate+up at m = 1, 13.1 -> 11.6 us);
//   * INT4: the 32 nibbles of a lane's 16-byte piece become bf16 (128 + u)
//     values with two masks and four v_perm per 8 nibbles (x is staged in
//     the matching k order), four MFMAs give sum_k x (128 + u), and the
//     group correction (128 + z) * sum_k x uses row sums of x formed from
//     the same x registers while staging them;
//   * MFMA rows >= M take a copy of row M - 1 instead of zeros (no per-step
//     selects); their sums are discarded.
// Outputs: the waves' partial sums meet in LDS in fixed wave order.
constexpr uint32_t kSmallM = 4;

template <int FMT>
__device__ __forceinline__ v4i nt_piece(const void* w, uint64_t elem_offset) {
  if constexpr (FMT == kWBf16)
    return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(static_cast<const uint16_t*>(w) + elem_offset));
  else if constexpr (FMT == kWSym)
    return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(static_cast<const uint8_t*>(w) + elem_offset));
  else
    return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(static_cast<const uint32_t*>(w) + elem_offset));
}

// 8 nibbles of one word (nibble j = k offset j) -> eight bf16 values
// 128 + u_j in the order k = 0, 2, 4, 6, 1, 3, 5, 7: the low nibbles of the
// four bytes are the even k, the high nibbles the odd k, and one v_perm per
// pair places two of them under the 0x43 exponent byte of 128.  x is staged
// in LDS in the same order (x_in_nibble_order), so the MFMA sees matching
// k on both operands.
__device__ __forceinline__ void nibbles_to_bf16(uint32_t w, v4i& out) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  constexpr uint32_t kExp = 0x43434343u;
  out[0] = (int)__builtin_amdgcn_perm(kExp, lo, 0x04010400u);  // k0, k2
  out[1] = (int)__builtin_amdgcn_perm(kExp, lo, 0x04030402u);  // k4, k6
  out[2] = (int)__builtin_amdgcn_perm(kExp, hi, 0x04010400u);  // k1, k3
  out[3] = (int)__builtin_amdgcn_perm(kExp, hi, 0x04030402u);  // k5, k7
}

// Eight bf16 x values (k = 0..7) into the order nibbles_to_bf16 produces.
__device__ __forceinline__ v4i x_in_nibble_order(v4i v) {
  const uint32_t w0 = (uint32_t)v[0], w1 = (uint32_t)v[1], w2 = (uint32_t)v[2], w3 = (uint32_t)v[3];
  return v4i{(int)__builtin_amdgcn_perm(w1, w0, 0x05040100u), (int)__builtin_amdgcn_perm(w3, w2, 0x05040100u),
             (int)__builtin_amdgcn_perm(w1, w0, 0x07060302u), (int)__builtin_amdgcn_perm(w3, w2, 0x07060302u)};
}

// U consecutive 16-bit scales of one row, starting at a multiple of U.
template <int U>
struct ScaleVec {
  uint32_t w[(U + 1) / 2];
  __device__ __forceinline__ void load(const uint16_t* p) {
    if constexpr (U % 8 == 0) {
#pragma unroll
      for (int i = 0; i < U / 8; ++i) {
        const v4i v = reinterpret_cast<const v4i*>(p)[i];
        w[4 * i] = v[0], w[4 * i + 1] = v[1], w[4 * i + 2] = v[2], w[4 * i + 3] = v[3];
      }
    } else if constexpr (U % 4 == 0) {
#pragma unroll
      for (int i = 0; i < U / 4; ++i) {
        const uint2 v = reinterpret_cast<const uint2*>(p)[i];
        w[2 * i] = v.x, w[2 * i + 1] = v.y;
      }
    } else if constexpr (U % 2 == 0) {
#pragma unroll
      for (int i = 0; i < U / 2; ++i) w[i] = reinterpret_cast<const uint32_t*>(p)[i];
    } else {
      w[0] = *p;
    }
  }
  __device__ __forceinline__ uint32_t bits(int u) const { return (w[u / 2] >> (16 * (u & 1))) & 0xffffu; }
};

// Bytes of LDS the small-M kernel needs: per wave its x slice (rows < M,
// spw steps) and U... per-group row sums, plus the reduction area.
// W pairs of steps pass through a [16 rows][128 + 16 bytes] LDS tile per
// pair (the 16-byte pad keeps the MFMA-layout reads conflict-free).
constexpr uint32_t kWTileRow = 144, kWTile = 16 * kWTileRow;

template <int FMT>
constexpr uint32_t small_m_lds(uint32_t m, uint32_t spw, uint32_t waves, uint32_t u) {
  const uint32_t wtile = u % 2 == 0 ? kWTile : 0;
  return waves * (wtile + m * spw * step_k<FMT>() * 2 + (FMT != kWBf16 ? spw * 16 * 4 : 0)) + waves * 4 * 64 * 4;
}

// Up to kMaxGroup independent problems with the same m and K share one
// launch (the blocks of problem i are block_start[i] .. block_start[i+1]-1);
// a single GEMV is a group of one.
constexpr int kMaxGroup = 8;
struct GemvGroup {
  GemvParams prob[kMaxGroup];
  uint32_t block_start[kMaxGroup + 1];
  uint32_t count;
};

template <int FMT, int WAVES, int U, bool ONE_ROW>
__global__ __launch_bounds__(WAVES * 64) void gemv_lds_kernel(GemvGroup grp, uint32_t spw) {
  extern __shared__ __align__(16) uint8_t smem[];
  // this block's problem: selected field by field with constant indices
  // (indexing the by-value argument with a variable would copy it to scratch)
  uint32_t pi = 0;
#pragma unroll
  for (int i = 1; i < kMaxGroup; ++i)
    if ((uint32_t)i < grp.count && blockIdx.x >= grp.block_start[i]) pi = i;
  GemvParams p = grp.prob[0];
#pragma unroll
  for (int i = 1; i < kMaxGroup; ++i)
    if (pi == (uint32_t)i) p = grp.prob[i];
  const uint32_t block = blockIdx.x - grp.block_start[pi];
  constexpr bool kInt4 = FMT != kWBf16;
  constexpr uint32_t SK = step_k<FMT>();
  // x chunks per lane loaded ahead of the weights: M * spw * 16 <= 512, or
  // (ONE_ROW: m = 1 and the wave's run is one batch) spw * SK / 8 <= 64 * XR
  constexpr int XR = ONE_ROW ? (U + 3) / 4 : 8;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t lr = lane & 15, lg = lane >> 4;
  const uint32_t n0 = block * 16, nrow = n0 + lr;
  const uint32_t K = p.k, M = p.m, G = K / 128;
  const uint32_t s0 = wave * spw, s1 = s0 + spw;  // WAVES * spw == K / SK
  const uint32_t span = spw * SK;                 // this wave's K run
  const uint32_t zwords = (G + 7) / 8;
  // Even U: W is loaded as whole 128-byte lines (8 rows x 128 B per load:
  // two steps of eight rows) and turned into the MFMA layout (16 rows x
  // 64 B per step) through an LDS tile.  Loading the MFMA layout directly
  // touches 16 half lines per instruction and streamed ~17 % slower.
  constexpr bool kT = U % 2 == 0;
  constexpr uint32_t kWBytes = kT ? kWTile : 0;
  // wave-private LDS: W tiles, x[M][span] bf16, then (INT4) row sums [spw][16]
  const uint32_t wave_bytes = kWBytes + M * span * 2 + (kInt4 ? spw * 16 * 4 : 0);
  uint8_t* wt = smem + wave * wave_bytes;
  uint16_t* xs = reinterpret_cast<uint16_t*>(wt + kWBytes);
  float* xsum = reinterpret_cast<float*>(wt + kWBytes + M * span * 2);
  float* red = reinterpret_cast<float*>(smem + WAVES * wave_bytes);  // [WAVES][4][64]

  // ---- this wave's x slice: chunk c = (row m, 16-byte piece j of the run)
  const uint32_t row_chunks = span / 8, chunks = M * row_chunks;
  // chunk -> (row m, piece j); M <= 4, so the row is a count of boundaries
  auto row_of = [&](uint32_t c) -> uint32_t {
    return (uint32_t)(c >= row_chunks) + (uint32_t)(c >= 2 * row_chunks) + (uint32_t)(c >= 3 * row_chunks);
  };
  auto x_chunk = [&](uint32_t c) -> v4i {
    const uint32_t m = row_of(c), j = c - m * row_chunks;
    return *reinterpret_cast<const v4i*>(p.x + (uint64_t)m * K + s0 * SK + j * 8);
  };
  // unconditional loads (lanes past the end repeat the last chunk): a load
  // under a branch makes the compiler wait for it on the spot
  v4i xr[XR];
#pragma unroll
  for (int j = 0; j < XR; ++j) xr[j] = x_chunk(min(lane + 64 * j, chunks - 1));

  // ---- first batch of W, its scales and zero points
  v4i wv[U];
  ScaleVec<U> sv;
  uint32_t zw = 0, zw1 = 0;
  constexpr bool kTwoZeroWords = 8 % U != 0;  // a batch may span two words of 8 zero points
  // scales and zero points go first: loads complete in issue order, so the
  // math of step 0 then waits only for W[0], not for the whole batch
  auto issue = [&](uint32_t sb) {
    if constexpr (kInt4) sv.load(p.scales + (uint64_t)nrow * G + sb);
    if constexpr (FMT == kWAsym) {
      zw = p.zeros[(uint64_t)nrow * zwords + sb / 8];
      if constexpr (kTwoZeroWords) zw1 = p.zeros[(uint64_t)nrow * zwords + min(sb / 8 + 1, zwords - 1)];
    }
    if constexpr (kT) {
      // load 2q + h: rows n0 + 8h + lane / 8, bytes [64 (sb + 2q), +128) of
      // the row, 16 of them per lane
      const uint8_t* wb = static_cast<const uint8_t*>(p.w);
      const uint64_t row_bytes = kInt4 ? K / 2 : (uint64_t)K * 2;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t row = n0 + 8 * (u & 1) + lane / 8;
        wv[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(
            wb + (uint64_t)row * row_bytes + (uint64_t)(sb + (u & ~1)) * 64 + (lane % 8) * 16));
      }
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t k0 = (sb + u) * SK;
        if constexpr (FMT == kWBf16)
          wv[u] = nt_piece<FMT>(p.w, (uint64_t)nrow * K + k0 + lg * 8);
        else if constexpr (FMT == kWSym)
          wv[u] = nt_piece<FMT>(p.w, (uint64_t)nrow * (K / 2) + k0 / 2 + lg * 16);
        else
          wv[u] = nt_piece<FMT>(p.w, (uint64_t)nrow * (K / 8) + k0 / 8 + lg * 4);
      }
    }
  };
  // Even U: the line pair (loads u, u + 1 = rows 0-7 and 8-15 of steps u and
  // u + 1) through the LDS tile into the MFMA layout of steps u and u + 1.
  auto to_mfma_layout = [&](int u) {
    if constexpr (kT) {
      uint8_t* tile = wt;  // one tile per wave: a wave's LDS accesses complete in order
      *reinterpret_cast<v4i*>(tile + (lane / 8) * kWTileRow + (lane % 8) * 16) = wv[u];
      *reinterpret_cast<v4i*>(tile + (8 + lane / 8) * kWTileRow + (lane % 8) * 16) = wv[u + 1];
      wv[u] = *reinterpret_cast<const v4i*>(tile + lr * kWTileRow + lg * 16);
      wv[u + 1] = *reinterpret_cast<const v4i*>(tile + lr * kWTileRow + 64 + lg * 16);
    }
  };
  issue(s0);
  // every load of the wave is in flight before anything waits on one
  __builtin_amdgcn_sched_barrier(0);

  // ---- x to LDS; INT4: row sums of x per 128-group from the same registers
  // (16 lanes hold one group of one row: 16 chunks x 8 values)
  // Branch-free on purpose: a value used only under a branch gets its load
  // sunk into the branch, where the compiler then waits for every earlier
  // load (the W batch included).  Lanes past the end rewrite the last chunk
  // with its own value.
  auto stage = [&](uint32_t c, v4i v) {
    const bool live = c < chunks;
    const uint32_t cc = min(c, chunks - 1);
    reinterpret_cast<v4i*>(xs)[cc] = kInt4 ? x_in_nibble_order(v) : v;
    if constexpr (kInt4) {
      float s = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        s += __uint_as_float((uint32_t)v[q] << 16) + __uint_as_float((uint32_t)v[q] & 0xffff0000u);
      s = live ? s : 0.0f;
      s += __shfl_xor(s, 1);
      s += __shfl_xor(s, 2);
      s += __shfl_xor(s, 4);
      s += __shfl_xor(s, 8);
      if (live && (c & 15) == 0) {
        const uint32_t m = row_of(c);
        xsum[((c - m * row_chunks) / 16) * 16 + m] = s;
      }
    }
  };
#pragma unroll
  for (int j = 0; j < XR; ++j)
    if (64 * j < chunks) stage(lane + 64 * j, xr[j]);  // wave-uniform: skips rounds with no live chunk
  for (uint32_t base = 64 * XR; base < chunks; base += 64) {
    const uint32_t c = base + lane;
    stage(c, x_chunk(min(c, chunks - 1)));
  }
  // the wave reads back only what it wrote: no block barrier needed

  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
  uint32_t bad = 0;
  // MFMA rows >= M read row M - 1 of x: their sums are never stored
  const uint16_t* xrow_ptr = xs + min(lr, M - 1) * span;
  auto compute = [&](uint32_t sb) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (u % 2 == 0) to_mfma_layout(u);
      const uint32_t st = sb + u;            // global step
      const uint32_t kl = (st - s0) * SK;    // k offset inside the wave's run
      if constexpr (FMT == kWBf16) {
        const v4i xv = *reinterpret_cast<const v4i*>(xrow_ptr + kl + lg * 8);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, xv), __builtin_bit_cast(v8bf, wv[u]),
                                                      acc, 0, 0, 0);
      } else {
        v4i xv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) xv[i] = *reinterpret_cast<const v4i*>(xrow_ptr + kl + lg * 32 + i * 8);
        const v4f xsv = *reinterpret_cast<const v4f*>(xsum + (st - s0) * 16 + lg * 4);
        float sc;
        int zero;
        if constexpr (FMT == kWSym) {
          sc = (float)__builtin_bit_cast(_Float16, (uint16_t)sv.bits(u));
          zero = 8;
        } else {
          sc = bf16_bits_to_f32(sv.bits(u));
          const uint32_t zword = kTwoZeroWords && (st / 8 != sb / 8) ? zw1 : zw;
          zero = (int)((zword >> (4 * (st % 8))) & 0xfu);
        }
        if (!(sc > 0.0f) || !__builtin_isfinite(sc)) bad = bad ? bad : kQwenBadScale;
        uint32_t wd[4] = {(uint32_t)wv[u][0], (uint32_t)wv[u][1], (uint32_t)wv[u][2], (uint32_t)wv[u][3]};
        if constexpr (FMT == kWSym) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t t = wd[i] ^ 0x88888888u;  // two's complement nibble -> u = q + 8; reserved 8 -> 0
            if ((t - 0x11111111u) & ~t & 0x88888888u) bad = kQwenReservedNibble;
            wd[i] = t;
          }
        }
        v4i qb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) nibbles_to_bf16(wd[i], qb[i]);
        v4f pq = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i)
          pq = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, xv[i]),
                                                       __builtin_bit_cast(v8bf, qb[i]), pq, 0, 0, 0);
        // rows >= M (copies of row M - 1, stale row sums) are never stored
        const float zc = 128.0f + (float)zero;
        // m = 1: only MFMA row 0 (acc[0] of lanes 0..15) is ever stored
#pragma unroll
        for (int i = 0; i < (ONE_ROW ? 1 : 4); ++i)
          acc[i] = __builtin_fmaf(__builtin_fmaf(-zc, xsv[i], pq[i]), sc, acc[i]);
      }
    }
  };

  compute(s0);
  for (uint32_t sb = s0 + U; sb < s1; sb += U) {
    issue(sb);
    compute(sb);
  }
  if constexpr (kInt4)
    if (bad) publish(p.err, bad);

  // ---- reduce the block's waves in wave order
#pragma unroll
  for (int i = 0; i < 4; ++i) red[(wave * 4 + i) * 64 + lane] = acc[i];
  __syncthreads();
  uint32_t nonfinite = 0;
  if (tid < 256) {
    const uint32_t i = tid / 64, l = tid % 64;
    const uint32_t mrow = 4 * (l >> 4) + i, col = n0 + (l & 15);
    if (mrow < M) {
      float v = 0.0f;
#pragma unroll
      for (int wv2 = 0; wv2 < WAVES; ++wv2) v += red[(wv2 * 4 + i) * 64 + l];
      if (!__builtin_isfinite(v)) nonfinite = 1;
      if (p.out_f32) static_cast<float*>(p.out)[(uint64_t)mrow * p.n + col] = v;
      else static_cast<uint16_t*>(p.out)[(uint64_t)mrow * p.n + col] = (uint16_t)f32_to_bf16_bits(v);
    }
  }
  if constexpr (kInt4)
    if (nonfinite) publish(p.err, kQwenNonFinite);
  if constexpr (!kInt4)
    if (nonfinite && p.nonfinite_or) atomicOr(p.err, p.nonfinite_or);
}

// ---------------------------------------------------------------------------
// Mid-M decode GEMV (4 < M <= 64).
//
// x is too large to stage per block (M x K bf16 is 128 KB at M = 16,
// K = 4096) and every block reads it from L2 again, so x traffic is
// 2M / w_bytes times the W traffic per W row block (4x for INT4 at M = 16,
// 4x for bf16 at M = 64).  What bounds the kernel is therefore how fast a
// CU reads L2-resident data, and that depends on the access pattern of one
// instruction (measured on MI355X, all CUs reading a 512 KB array):
// 16 rows x 64 B per instruction (the MFMA operand layout) ~9 TB/s in
// total, 8 rows x 128 B ~25 TB/s, 1 KB contiguous ~32 TB/s.  So W and x are
// both loaded as whole 128-byte lines, 8 rows per instruction, two MFMA
// steps per line (a W step is 64 bytes of a row in both formats; an x step
// is 64 (bf16) or 256 (INT4) bytes of a row), and each wave turns them into
// the MFMA layout through its own LDS tiles.
//
// A block owns NW 16-row W blocks and its waves split K into equal runs of
// spw steps (WAVES * spw = K / SK, U even and U | spw); a batch of U steps
// issues every W line, the U group scales of each W row in one vector load,
// the zero points in one u32, and every x line before any math, so each
// x fragment feeds NW MFMA column blocks.
//   INT4: nibbles become bf16 (128 + u) by two masks and four v_perm per
//   word (nibbles_to_bf16, x permuted to the same k order in registers), and
//   sum_k x per group comes from one MFMA of x against ones per x fragment,
//   shared by the NW W blocks.
// Rows m >= M of an MFMA tile read row M - 1 of x; their sums are never
// stored.  The waves' partial sums meet in LDS in fixed wave order, one W
// block at a time.
template <int FMT>
constexpr uint32_t mid_x_pitch() {  // bytes per row of an x tile (two steps + pad)
  return FMT == kWBf16 ? 2 * 64 + 16 : 2 * 256 + 16;
}
constexpr uint32_t kMidWPitch = 2 * 64 + 16;

template <int FMT, int MT, int NW, int WAVES, int U>
constexpr uint32_t mid_lds_bytes() {
  return WAVES * (U / 2) * 16 * (NW * kMidWPitch + MT * mid_x_pitch<FMT>()) + WAVES * MT * 4 * 64 * 4;
}

template <int FMT, int MT, int NW, int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void gemv_mid_kernel(GemvGroup grp, uint32_t spw) {
  static_assert(U % 2 == 0, "a batch is whole step pairs");
  extern __shared__ __align__(16) uint8_t smem[];
  uint32_t pi = 0;
#pragma unroll
  for (int i = 1; i < kMaxGroup; ++i)
    if ((uint32_t)i < grp.count && blockIdx.x >= grp.block_start[i]) pi = i;
  GemvParams p = grp.prob[0];
#pragma unroll
  for (int i = 1; i < kMaxGroup; ++i)
    if (pi == (uint32_t)i) p = grp.prob[i];
  const uint32_t block = blockIdx.x - grp.block_start[pi];
  constexpr bool kInt4 = FMT != kWBf16;
  constexpr int P = U / 2;                           // step pairs per batch
  constexpr uint32_t XP = mid_x_pitch<FMT>();        // x tile row pitch
  constexpr int XC = kInt4 ? 4 : 1;                  // 128-byte x lines per row and pair
  constexpr int XL = kInt4 ? 4 : 1;                  // 16-byte x fragments per lane, step and M tile
  constexpr uint32_t kWaveTiles = P * 16 * (NW * kMidWPitch + MT * XP);
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t lr = lane & 15, lg = lane >> 4;
  const uint32_t lrow = lane >> 3, lcol = (lane & 7) * 16;  // line-load position
  const uint32_t n0 = block * 16 * NW;
  const uint32_t K = p.k, M = p.m, G = K / 128;
  const uint32_t s0 = wave * spw, s1 = s0 + spw;
  const uint32_t zwords = (G + 7) / 8;
  const uint64_t w_row_bytes = kInt4 ? K / 2 : (uint64_t)K * 2;
  uint8_t* wtile = smem + wave * kWaveTiles;                 // [P][NW][16][kMidWPitch]
  uint8_t* xtile = wtile + P * NW * 16 * kMidWPitch;         // [P][MT][16][XP]
  float* red = reinterpret_cast<float*>(smem + WAVES * kWaveTiles);  // [WAVES][MT][4][64]

  const uint8_t* wsrc[NW][2];
#pragma unroll
  for (int b = 0; b < NW; ++b)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      wsrc[b][h] = static_cast<const uint8_t*>(p.w) + (uint64_t)(n0 + b * 16 + 8 * h + lrow) * w_row_bytes + lcol;
  const uint8_t* xsrc[MT][2];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      xsrc[t][h] = reinterpret_cast<const uint8_t*>(p.x + (uint64_t)min(t * 16 + 8 * h + lrow, M - 1) * K) + lcol;

  v4i wl[P][NW][2];
  v4i xl[P][MT][2][XC];
  ScaleVec<U> sv[NW];
  uint32_t zw[NW];
  auto issue = [&](uint32_t sb) {
#pragma unroll
    for (int b = 0; b < NW; ++b) {
      const uint32_t row = n0 + b * 16 + lr;
      if constexpr (kInt4) sv[b].load(p.scales + (uint64_t)row * G + sb);
      if constexpr (FMT == kWAsym) zw[b] = p.zeros[(uint64_t)row * zwords + sb / 8];
    }
#pragma unroll
    for (int q = 0; q < P; ++q) {
      const uint64_t st = sb + 2 * q;  // first step of the pair
#pragma unroll
      for (int b = 0; b < NW; ++b)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          wl[q][b][h] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wsrc[b][h] + st * 64));
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int c = 0; c < XC; ++c)
            xl[q][t][h][c] = *reinterpret_cast<const v4i*>(xsrc[t][h] + st * (kInt4 ? 256 : 64) + c * 128);
    }
  };

  v4f acc[NW][MT];
#pragma unroll
  for (int b = 0; b < NW; ++b)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[b][t] = v4f{0.f, 0.f, 0.f, 0.f};
  uint32_t bad = 0;
  const v8bf ones = __builtin_bit_cast(v8bf, v4i{0x3f803f80, 0x3f803f80, 0x3f803f80, 0x3f803f80});

  auto compute = [&](uint32_t sb) {
#pragma unroll
    for (int q = 0; q < P; ++q) {
      // lines -> tiles (row 8h + lrow, bytes c*128 + lcol of the pair)
      uint8_t* wt = wtile + q * NW * 16 * kMidWPitch;
      uint8_t* xt = xtile + q * MT * 16 * XP;
#pragma unroll
      for (int b = 0; b < NW; ++b)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          *reinterpret_cast<v4i*>(wt + (b * 16 + 8 * h + lrow) * kMidWPitch + lcol) = wl[q][b][h];
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int c = 0; c < XC; ++c)
            *reinterpret_cast<v4i*>(xt + (t * 16 + 8 * h + lrow) * XP + c * 128 + lcol) = xl[q][t][h][c];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        // MFMA layout of step s: lane (lr, lg) takes row lr, 16 bytes lg of
        // the step (W and bf16 x) or 64 bytes lg of the step (INT4 x)
        v4i wf[NW], xf[MT][XL];
#pragma unroll
        for (int b = 0; b < NW; ++b)
          wf[b] = *reinterpret_cast<const v4i*>(wt + (b * 16 + lr) * kMidWPitch + s * 64 + lg * 16);
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int i = 0; i < XL; ++i)
            xf[t][i] = *reinterpret_cast<const v4i*>(xt + (t * 16 + lr) * XP +
                                                     (kInt4 ? s * 256 + lg * 64 + i * 16 : s * 64 + lg * 16));
        if constexpr (FMT == kWBf16) {
#pragma unroll
          for (int b = 0; b < NW; ++b)
#pragma unroll
            for (int t = 0; t < MT; ++t)
              acc[b][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, xf[t][0]),
                                                                  __builtin_bit_cast(v8bf, wf[b]), acc[b][t], 0, 0, 0);
        } else {
          const int u = 2 * q + s;  // step inside the batch
          const uint32_t st = sb + u;
          v4f xs[MT];
#pragma unroll
          for (int t = 0; t < MT; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) xf[t][i] = x_in_nibble_order(xf[t][i]);
            xs[t] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; ++i)
              xs[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, xf[t][i]), ones, xs[t], 0, 0,
                                                              0);
          }
#pragma unroll
          for (int b = 0; b < NW; ++b) {
            float sc;
            int zero;
            if constexpr (FMT == kWSym) {
              sc = (float)__builtin_bit_cast(_Float16, (uint16_t)sv[b].bits(u));
              zero = 8;
            } else {
              sc = bf16_bits_to_f32(sv[b].bits(u));
              zero = (int)((zw[b] >> (4 * (st % 8))) & 0xfu);
            }
            if (!(sc > 0.0f) || !__builtin_isfinite(sc)) bad = bad ? bad : kQwenBadScale;
            uint32_t wd[4] = {(uint32_t)wf[b][0], (uint32_t)wf[b][1], (uint32_t)wf[b][2], (uint32_t)wf[b][3]};
            if constexpr (FMT == kWSym) {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const uint32_t v = wd[i] ^ 0x88888888u;  // two's complement nibble -> u = q + 8; reserved 8 -> 0
                if ((v - 0x11111111u) & ~v & 0x88888888u) bad = kQwenReservedNibble;
                wd[i] = v;
              }
            }
            v4i qb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) nibbles_to_bf16(wd[i], qb[i]);
            const float zc = 128.0f + (float)zero;
#pragma unroll
            for (int t = 0; t < MT; ++t) {
              v4f pq = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int i = 0; i < 4; ++i)
                pq = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, xf[t][i]),
                                                             __builtin_bit_cast(v8bf, qb[i]), pq, 0, 0, 0);
#pragma unroll
              for (int i = 0; i < 4; ++i)
                acc[b][t][i] = __builtin_fmaf(__builtin_fmaf(-zc, xs[t][i], pq[i]), sc, acc[b][t][i]);
            }
          }
        }
      }
    }
  };

  for (uint32_t sb = s0; sb < s1; sb += U) {
    issue(sb);
    // every load of the batch is in flight before the first one is used
    __builtin_amdgcn_sched_barrier(0);
    compute(sb);
  }
  if constexpr (kInt4)
    if (bad) publish(p.err, bad);

  // ---- reduce the block's waves in wave order, one W block at a time;
  // lane (lr, lg) of tile t holds rows t*16 + 4*lg + i of column lr
  uint32_t nonfinite = 0;
#pragma unroll
  for (int b = 0; b < NW; ++b) {
    if (b) __syncthreads();  // the previous block's sums have been read
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[((wave * MT + t) * 4 + i) * 64 + lane] = acc[b][t][i];
    __syncthreads();
    for (uint32_t slot = tid; slot < (uint32_t)MT * 256; slot += WAVES * 64) {
      const uint32_t t = slot / 256, i = (slot / 64) % 4, l = slot % 64;
      const uint32_t mrow = t * 16 + 4 * (l >> 4) + i, col = n0 + b * 16 + (l & 15);
      if (mrow >= M) continue;
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) v += red[((w * MT + t) * 4 + i) * 64 + l];
      if (!__builtin_isfinite(v)) nonfinite = 1;
      if (p.out_f32) static_cast<float*>(p.out)[(uint64_t)mrow * p.n + col] = v;
      else static_cast<uint16_t*>(p.out)[(uint64_t)mrow * p.n + col] = (uint16_t)f32_to_bf16_bits(v);
    }
  }
  if constexpr (kInt4)
    if (nonfinite) publish(p.err, kQwenNonFinite);
  if constexpr (!kInt4)
    if (nonfinite && p.nonfinite_or) atomicOr(p.err, p.nonfinite_or);
}

// Exact dequant of an INT4 weight to fp32: w[n, k] = (q - z) * s (asym) or
// q * s (sym), the values the GEMV multiplies (as integers times the
// group scale).
template <int FMT>
__global__ __launch_bounds__(256) void dequant_kernel(const void* wq, const uint16_t* scales,
                                                      const uint32_t* zeros, float* out, uint32_t* err,
                                                      uint32_t n, uint32_t k) {
  const uint64_t pieces = (uint64_t)n * (k / 32u);
  uint32_t bad = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < pieces;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t row = (uint32_t)(i / (k / 32u)), pc = (uint32_t)(i % (k / 32u));
    const uint32_t kk = pc * 32u, grp = kk / 128u;
    uint4 wp;
    int zero = 0;
    float sc;
    if constexpr (FMT == kWSym) {
      wp = *reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(wq) + (uint64_t)row * (k / 2) + kk / 2);
      sc = (float)__builtin_bit_cast(_Float16, scales[(uint64_t)row * (k / 128) + grp]);
    } else {
      wp = *reinterpret_cast<const uint4*>(static_cast<const uint32_t*>(wq) + (uint64_t)row * (k / 8) + kk / 8);
      const uint32_t zwords = (k / 128 + 7) / 8;
      zero = (int)((zeros[(uint64_t)row * zwords + grp / 8] >> (4 * (grp % 8))) & 0xfu);
      sc = bf16_bits_to_f32(scales[(uint64_t)row * (k / 128) + grp]);
    }
    if (!(sc > 0.0f) || !__builtin_isfinite(sc)) bad = bad ? bad : kQwenBadScale;
    v8s q[4];
    if (!unpack32<FMT>(wp, zero, q)) bad = kQwenReservedNibble;
    float* o = out + (uint64_t)row * k + kk;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 8; ++b) o[a * 8 + b] = bf16_bits_to_f32((uint16_t)q[a][b]) * sc;
  }
  if (bad) publish(err, bad);
}

// Waves per block: each block owns 16 W rows and its waves split K, so
// small N gets more waves per block to keep >= ~2048 waves in flight.
template <int FMT>
int waves_for(uint32_t n) {
  const uint32_t rowblks = n / 16;
  return rowblks >= 512 ? 4 : rowblks >= 256 ? 8 : 16;
}

template <int FMT, int MT>
void launch_mt(const GemvParams& p, int waves, hipStream_t s) {
  const dim3 grid(p.n / 16);
  if (waves == 4) hipLaunchKernelGGL((gemv_kernel<FMT, MT, 4>), grid, dim3(256), 0, s, p);
  else if (waves == 8) hipLaunchKernelGGL((gemv_kernel<FMT, MT, 8>), grid, dim3(512), 0, s, p);
  else hipLaunchKernelGGL((gemv_kernel<FMT, MT, 16>), grid, dim3(1024), 0, s, p);
}

template <int FMT, int WAVES, int U, bool ONE_ROW>
St launch_lds(const GemvGroup& g, uint32_t spw, hipStream_t s) {
  const uint32_t lds = small_m_lds<FMT>(g.prob[0].m, spw, WAVES, U);
  static PerDeviceOnce raised;  // LDS above 64 KB must be allowed once per kernel and device
  if (lds > 65536) {
    const St r = raised.run([] {
      return hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_lds_kernel<FMT, WAVES, U, ONE_ROW>),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess
                 ? Ok()
                 : Internal("gemv_lds_attribute_failed");
    });
    if (!r.ok()) return r;
  }
  hipLaunchKernelGGL((gemv_lds_kernel<FMT, WAVES, U, ONE_ROW>), dim3(g.block_start[g.count]), dim3(WAVES * 64), lds, s,
                     g, spw);
  return AfterLaunch("gemv_launch_failed");
}

// Waves per block and steps per batch for the LDS kernel: the waves split
// the K steps evenly (WAVES divides steps).
//   INT4, m = 1: the most of 4, 8, 12 waves whose grid still fits one
//     resident round (<= 4096 waves: 16 per CU on 256 CUs), each wave's run
//     one batch of 1, 2, 4, 6, 8 or 12 steps, so every load of the launch is
//     issued before any wave waits (Qwen3-8B down, K = 12288: 12 waves x 8
//     steps measured 7.7 us against 8.6 us for 8 waves x 12 steps in three
//     batches of 4; 16 waves x 6 steps ran as fast but spills registers).
//   Otherwise: the first of 4, 8, 12, 16 that gives the grid >= 2048 waves
//     (m = 1) or at most 4 steps per wave (m >= 2: each wave stages m rows
//     of x for its run before its first step, so shorter runs measured
//     faster, e.g. 16.7 vs 19.6 us for Qwen3-8B gate+up at m = 4), else the
//     largest that divides; U is the largest of 8, 4, 2, 1 dividing the
//     steps per wave.
// Returns false when no split divides the steps.
template <int FMT>
bool pick_lds_split(uint32_t rowblks, uint32_t k, uint32_t m, int& waves, uint32_t& spw, int& u) {
  const uint32_t steps = k / step_k<FMT>();
  waves = 0;
  if (FMT != kWBf16 && m == 1) {
    for (int w : {4, 8, 12}) {
      const uint32_t run = steps / (uint32_t)w;
      if (steps % (uint32_t)w || (run != 1 && run != 2 && run != 4 && run != 6 && run != 8 && run != 12)) continue;
      if (waves && rowblks * (uint32_t)w > 4096) break;
      waves = w;
    }
    if (waves) {
      spw = steps / waves;
      u = (int)spw;
      return true;
    }
  }
  for (int w : {4, 8, 12, 16}) {
    if (steps % (uint32_t)w) continue;
    waves = w;
    if (m == 1 ? rowblks * (uint32_t)w >= 2048 : steps / (uint32_t)w <= 4) break;
  }
  if (!waves) return false;
  spw = steps / waves;
  u = spw % 8 == 0 ? 8 : spw % 4 == 0 ? 4 : spw % 2 == 0 ? 2 : 1;
  return true;
}

template <int FMT, int WAVES>
St launch_lds_u(const GemvGroup& g, uint32_t spw, int u, hipStream_t s) {
  const bool one = g.prob[0].m == 1 && spw == (uint32_t)u;
  if constexpr (FMT != kWBf16) {
    // batches of 12 and 6 steps come only from the INT4 m = 1 rule (one
    // batch per wave, at most 12 waves: 16 waves of 6 or 12 steps spill)
    if constexpr (WAVES <= 12) {
      if (u == 12) return launch_lds<FMT, WAVES, 12, true>(g, spw, s);
      if (u == 6) return launch_lds<FMT, WAVES, 6, true>(g, spw, s);
    }
  }
  if (u == 8) return one ? launch_lds<FMT, WAVES, 8, true>(g, spw, s) : launch_lds<FMT, WAVES, 8, false>(g, spw, s);
  if (u == 4) return one ? launch_lds<FMT, WAVES, 4, true>(g, spw, s) : launch_lds<FMT, WAVES, 4, false>(g, spw, s);
  if (u == 2) return one ? launch_lds<FMT, WAVES, 2, true>(g, spw, s) : launch_lds<FMT, WAVES, 2, false>(g, spw, s);
  return launch_lds<FMT, WAVES, 1, false>(g, spw, s);
}

// The small-M path for a group (every problem has the same m and k);
// returns false in `taken` when the shape has no even split (the caller
// then uses gemv_kernel per problem).
template <int FMT>
St launch_group_lds(const GemvGroup& g, hipStream_t s, bool& taken) {
  taken = false;
  const GemvParams& p = g.prob[0];
  int waves, u;
  uint32_t spw;
  if (p.m > kSmallM || !pick_lds_split<FMT>(g.block_start[g.count], p.k, p.m, waves, spw, u) ||
      small_m_lds<FMT>(p.m, spw, waves, u) > 160 * 1024)
    return Ok();
  taken = true;
  switch (waves) {
    case 4: return launch_lds_u<FMT, 4>(g, spw, u, s);
    case 8: return launch_lds_u<FMT, 8>(g, spw, u, s);
    case 12: return launch_lds_u<FMT, 12>(g, spw, u, s);
    default: return launch_lds_u<FMT, 16>(g, spw, u, s);
  }
}

template <int FMT, int MT, int NW, int WAVES, int U>
St launch_mid(const GemvGroup& g, uint32_t spw, hipStream_t s) {
  constexpr uint32_t lds = mid_lds_bytes<FMT, MT, NW, WAVES, U>();
  static_assert(lds <= 160 * 1024, "mid GEMV tiles exceed the LDS");
  if constexpr (lds > 65536) {
    static PerDeviceOnce raised;  // LDS above 64 KB must be allowed once per kernel and device
    const St r = raised.run([] {
      return hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_mid_kernel<FMT, MT, NW, WAVES, U>),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess
                 ? Ok()
                 : Internal("gemv_mid_attribute_failed");
    });
    if (!r.ok()) return r;
  }
  hipLaunchKernelGGL((gemv_mid_kernel<FMT, MT, NW, WAVES, U>), dim3(g.block_start[g.count]), dim3(WAVES * 64), lds,
                     s, g, spw);
  return AfterLaunch("gemv_launch_failed");
}

// The mid-M path for a group (same m and k; block_start counts 16-row
// blocks).  Configurations measured fastest on MI355X for the Qwen3-8B
// shapes (per 16-row block count: >= 512 is gate/up):
//   bf16, M <= 16 : one W block per wave, 8 waves (4 at >= 512 blocks), U 4
//   bf16, M 49..64: 4 W blocks per wave and 4 waves at >= 512 blocks (x is
//                   4x the W bytes there), else one W block, 8 waves, U 2
//   bf16, M 17..48: one W block, 8 waves, U 2
//   INT4, M <= 32 : one W block, 8 waves (4 at >= 512 blocks or M > 16), U 2
// Returns with `taken` false when the shape does not split evenly (or INT4
// with M > 32); the caller then uses gemv_kernel.
template <int FMT>
St launch_group_mid(GemvGroup g, hipStream_t s, bool& taken) {
  taken = false;
  const GemvParams& p = g.prob[0];
  const uint32_t mt = (p.m + 15) / 16, rows16 = g.block_start[g.count];
  const uint32_t steps = p.k / step_k<FMT>();
  int nw = 1, waves = 8, u = 2;
  if constexpr (FMT == kWBf16) {
    if (mt == 1) waves = rows16 >= 512 ? 4 : 8, u = 4;
    else if (mt == 4 && rows16 >= 512) nw = 4, waves = 4;
  } else {
    if (mt > 2) return Ok();
    if (mt == 2 || rows16 >= 512) waves = 4;
    // m <= 16 with many row blocks: each x fragment feeds 2 or 4 W blocks,
    // keeping >= 384 blocks (grouped Qwen3-8B [gate, up] at m = 16: the
    // pass 54.3 -> 49.3 us; gate or up alone with 4 W blocks per block
    // left 192 blocks and ran slower than with 2)
    if (mt == 1 && rows16 >= 512) nw = rows16 >= 1024 ? 4 : 2;
  }
  if (steps % (uint32_t)waves || (steps / waves) % (uint32_t)u) return Ok();
  for (uint32_t i = 0; i < g.count; ++i)
    if (g.prob[i].n % (16u * nw)) return Ok();
  for (uint32_t i = 0; i < g.count; ++i) g.block_start[i + 1] = g.block_start[i] + g.prob[i].n / (16u * nw);
  const uint32_t spw = steps / waves;
  taken = true;
  if constexpr (FMT == kWBf16) {
    if (mt == 1) return waves == 4 ? launch_mid<FMT, 1, 1, 4, 4>(g, spw, s) : launch_mid<FMT, 1, 1, 8, 4>(g, spw, s);
    if (mt == 2) return launch_mid<FMT, 2, 1, 8, 2>(g, spw, s);
    if (mt == 3) return launch_mid<FMT, 3, 1, 8, 2>(g, spw, s);
    return nw == 4 ? launch_mid<FMT, 4, 4, 4, 2>(g, spw, s) : launch_mid<FMT, 4, 1, 8, 2>(g, spw, s);
  } else {
    if (mt == 2) return launch_mid<FMT, 2, 1, 4, 2>(g, spw, s);
    if (nw == 4) return launch_mid<FMT, 1, 4, 4, 2>(g, spw, s);
    if (nw == 2) return launch_mid<FMT, 1, 2, 4, 2>(g, spw, s);
    return waves == 4 ? launch_mid<FMT, 1, 1, 4, 2>(g, spw, s) : launch_mid<FMT, 1, 1, 8, 2>(g, spw, s);
  }
}

GemvGroup single(const GemvParams& p) {
  GemvGroup g{};
  g.prob[0] = p;
  g.count = 1;
  g.block_start[1] = p.n / 16;
  return g;
}

template <int FMT>
St launch_gemv(const GemvParams& p, hipStream_t s) {
  bool taken;
  const St st = p.m <= kSmallM ? launch_group_lds<FMT>(single(p), s, taken) : launch_group_mid<FMT>(single(p), s, taken);
  if (taken) return st;
  const int waves = waves_for<FMT>(p.n);
  switch ((p.m + 15) / 16) {
    case 1: launch_mt<FMT, 1>(p, waves, s); break;
    case 2: launch_mt<FMT, 2>(p, waves, s); break;
    case 3: launch_mt<FMT, 3>(p, waves, s); break;
    default: launch_mt<FMT, 4>(p, waves, s); break;
  }
  return AfterLaunch("gemv_launch_failed");
}

}  // namespace

uint64_t W4a16WorkspaceBytes(uint32_t m, uint32_t n, uint32_t k) {
  if (m == 0 || n == 0 || k == 0 || k % 128) return 0;
  (void)m;
  (void)n;
  (void)k;
  return 0;
}

uint64_t Bf16GemvWorkspaceBytes(uint32_t m, uint32_t n, uint32_t k) {
  if (m == 0 || n == 0 || k == 0 || k % 32) return 0;
  (void)m;
  (void)n;
  (void)k;
  return 0;
}

St LaunchBf16Gemv(const Bf16GemmArgs& a) {
  if (!a.a || !a.w || !a.out || !a.stream) return Invalid("bf16_gemv_null_argument");
  if (a.m == 0 || a.m > 64 || a.n == 0 || a.n % 16 || a.k == 0 || a.k % 32)
    return Invalid("bf16_gemv_shape_invalid");
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  GemvParams p{};
  p.x = a.a;
  p.w = a.w;
  p.out = a.out;
  p.m = a.m;
  p.n = a.n;
  p.k = a.k;
  p.out_f32 = a.out_kind == kOutF32;
  if (a.error_flag && a.nonfinite_bit) {
    p.err = a.error_flag;
    p.nonfinite_or = a.nonfinite_bit;
  }
  return launch_gemv<kWBf16>(p, a.stream);
}

St LaunchW4a16(const W4a16Args& a) {
  if (!a.x || !a.qweight || !a.scales || !a.out || !a.error_flag || !a.stream)
    return Invalid("w4a16_null_argument");
  if (!a.symmetric && !a.zeros) return Invalid("w4a16_zeros_missing");
  if (a.m == 0 || a.m > 64 || a.n == 0 || a.n % 16 || a.k == 0 || a.k % 128)
    return Invalid("w4a16_shape_invalid");
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  GemvParams p{};
  p.x = a.x;
  p.w = a.qweight;
  p.scales = a.scales;
  p.zeros = a.zeros;
  p.out = a.out;
  p.err = a.error_flag;
  p.m = a.m;
  p.n = a.n;
  p.k = a.k;
  if (a.symmetric)
    return launch_gemv<kWSym>(p, a.stream);
  return launch_gemv<kWAsym>(p, a.stream);
}

St LaunchW4a16Grouped(const W4a16Args* probs, uint32_t count) {
  if (!probs || count == 0 || count > (uint32_t)kMaxGroup) return Invalid("w4a16_group_size_invalid");
  const W4a16Args& a0 = probs[0];
  if (!a0.error_flag || !a0.stream) return Invalid("w4a16_null_argument");
  if (a0.m == 0 || a0.m > 64 || a0.k == 0 || a0.k % 128) return Invalid("w4a16_shape_invalid");
  GemvGroup g{};
  g.count = count;
  for (uint32_t i = 0; i < count; ++i) {
    const W4a16Args& a = probs[i];
    if (!a.x || !a.qweight || !a.scales || !a.out) return Invalid("w4a16_null_argument");
    if (!a.symmetric && !a.zeros) return Invalid("w4a16_zeros_missing");
    if (a.m != a0.m || a.k != a0.k || a.symmetric != a0.symmetric || a.n == 0 || a.n % 16)
      return Invalid("w4a16_group_shape_invalid");
    GemvParams& p = g.prob[i];
    p.x = a.x;
    p.w = a.qweight;
    p.scales = a.scales;
    p.zeros = a.zeros;
    p.out = a.out;
    p.err = a0.error_flag;
    p.m = a.m;
    p.n = a.n;
    p.k = a.k;
    g.block_start[i + 1] = g.block_start[i] + a.n / 16;
  }
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  bool taken;
  St st;
  if (a0.m <= kSmallM)
    st = a0.symmetric ? launch_group_lds<kWSym>(g, a0.stream, taken) : launch_group_lds<kWAsym>(g, a0.stream, taken);
  else
    st = a0.symmetric ? launch_group_mid<kWSym>(g, a0.stream, taken) : launch_group_mid<kWAsym>(g, a0.stream, taken);
  if (taken) return st;
  for (uint32_t i = 0; i < count; ++i) {  // shapes without the small-M path: one launch each
    const St one = a0.symmetric ? launch_gemv<kWSym>(g.prob[i], a0.stream) : launch_gemv<kWAsym>(g.prob[i], a0.stream);
    if (!one.ok()) return one;
  }
  return Ok();
}

St LaunchW4a16Dequant(const W4a16Args& a, float* out) {
  if (!a.qweight || !a.scales || !out || !a.error_flag || !a.stream) return Invalid("w4a16_dequant_null_argument");
  if (!a.symmetric && !a.zeros) return Invalid("w4a16_zeros_missing");
  if (a.n == 0 || a.k == 0 || a.k % 128) return Invalid("w4a16_dequant_shape_invalid");
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  uint64_t blocks = ((uint64_t)a.n * (a.k / 32) + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  if (a.symmetric)
    hipLaunchKernelGGL(dequant_kernel<kWSym>, dim3((uint32_t)blocks), dim3(256), 0, a.stream, a.qweight, a.scales,
                       a.zeros, out, a.error_flag, a.n, a.k);
  else
    hipLaunchKernelGGL(dequant_kernel<kWAsym>, dim3((uint32_t)blocks), dim3(256), 0, a.stream, a.qweight,
                       a.scales, a.zeros, out, a.error_flag, a.n, a.k);
  return AfterLaunch("w4a16_dequant_launch_failed");
}

}  // namespace pih_amd
