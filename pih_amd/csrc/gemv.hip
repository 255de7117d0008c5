// Decode GEMV for gfx950: y[m, n] = sum_k x[m, k] * W[n, k] for small m
// (1..64), with W in bf16 or INT4 (W4A16, symmetric reference format or
// asymmetric u32-packed format).  Memory-bound: the kernel streams W once.
//
// Layout of the work: a wave owns 16 W rows (one MFMA column block) and a
// contiguous K range; four waves of a block split the block's K range, and
// `ksplit` blocks split K further.  Each lane loads 16 contiguous bytes of a
// W row per step (lanes 16g..16g+15 take the g-th 16-byte piece of 16
// different rows), so a wave-wide load covers 16 rows x 64 bytes.  The x
// operand comes from global memory (it is small and L2-resident); rows
// m >= M of the 16-row MFMA tile are zero.
//   bf16 : one v_mfma_f32_16x16x32_bf16 per 16-byte W piece.
//   INT4 : one 16-byte piece is 32 nibbles = a quarter of a 128-deep quant
//          group per lane group, so a wave-wide load covers exactly one
//          group of 16 rows; the nibbles are unpacked to exact small
//          integers (q - z) in bf16, four MFMAs accumulate
//          sum_k x * (q - z) over the group, and the group's scale is
//          applied once: acc += s[n, g] * partial.  The unpack is the same
//          function the dequant entry uses (pinned bit-exact by tests).
// Reduction: waves of a block through LDS in fixed order; blocks of a
// k-split through an fp32 workspace, the last-arriving block (atomic
// ticket) summing the partials in split order, so results do not depend on
// timing.  Ticket counters live at the start of the workspace, must be zero
// before the first call and are left zero by every completed call.
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

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr uint32_t kQwenReservedNibble = 12, kQwenBadScale = 13, kQwenNonFinite = 14;

struct GemvParams {
  const uint16_t* x;
  const void* w;
  const uint16_t* scales;
  const uint32_t* zeros;
  void* out;
  float* partial;       // [ksplit][m][n] fp32 when ksplit > 1
  uint32_t* tickets;    // [n/16]
  uint32_t* err;
  uint32_t m, n, k;
  uint32_t ksplit;      // blocks along K
  uint32_t k_per_block; // multiple of kStepK
  uint32_t out_f32;
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

template <int FMT, int MT>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvParams p) {
  __shared__ float s_red[kWaves][MT][4][64];
  __shared__ uint32_t s_last;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t lr = lane & 15, lg = lane >> 4;
  const uint32_t rowblk = blockIdx.x, ks = blockIdx.y;
  const uint32_t n0 = rowblk * 16;
  const uint32_t nrow = n0 + lr;  // W row this lane loads
  constexpr uint32_t SK = step_k<FMT>();
  const uint32_t k_begin = ks * p.k_per_block;
  const uint32_t k_end = min(p.k, k_begin + p.k_per_block);
  const uint32_t steps = (k_end - k_begin) / SK;
  // waves interleave over the block's steps
  v4f acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  uint32_t bad = 0;

  for (uint32_t st = wave; st < steps; st += kWaves) {
    const uint32_t k0 = k_begin + st * SK;
    if constexpr (FMT == kWBf16) {
      const uint16_t* wrow = static_cast<const uint16_t*>(p.w) + (uint64_t)nrow * p.k;
      const uint4 wp = *reinterpret_cast<const uint4*>(wrow + k0 + lg * 8);
      const v8bf b = __builtin_bit_cast(v8bf, wp);
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const uint32_t mrow = t * 16 + lr;
        uint4 xp = make_uint4(0, 0, 0, 0);
        if (mrow < p.m) xp = *reinterpret_cast<const uint4*>(p.x + (uint64_t)mrow * p.k + k0 + lg * 8);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, xp), b, acc[t], 0, 0, 0);
      }
    } else {
      // one 128-deep quant group: lane group lg owns k0 + 32*lg .. +32
      const uint32_t grp = k0 / 128u;
      uint4 wp;
      int zero = 0;
      float sc;
      if constexpr (FMT == kWSym) {
        const uint8_t* wrow = static_cast<const uint8_t*>(p.w) + (uint64_t)nrow * (p.k / 2);
        wp = *reinterpret_cast<const uint4*>(wrow + k0 / 2 + lg * 16);
        const uint16_t hb = p.scales[(uint64_t)nrow * (p.k / 128) + grp];
        sc = (float)__builtin_bit_cast(_Float16, hb);
      } else {
        const uint32_t* wrow = static_cast<const uint32_t*>(p.w) + (uint64_t)nrow * (p.k / 8);
        wp = *reinterpret_cast<const uint4*>(wrow + k0 / 8 + lg * 4);
        const uint32_t zwords = (p.k / 128 + 7) / 8;
        zero = (int)((p.zeros[(uint64_t)nrow * zwords + grp / 8] >> (4 * (grp % 8))) & 0xfu);
        sc = bf16_bits_to_f32(p.scales[(uint64_t)nrow * (p.k / 128) + grp]);
      }
      if (!(sc > 0.0f) || !__builtin_isfinite(sc)) bad = bad ? bad : kQwenBadScale;
      v8s q[4];
      if (!unpack32<FMT>(wp, zero, q)) bad = kQwenReservedNibble;
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const uint32_t mrow = t * 16 + lr;
        const uint16_t* xr = p.x + (uint64_t)mrow * p.k + k0 + lg * 32;
        v4f part = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          uint4 xp = make_uint4(0, 0, 0, 0);
          if (mrow < p.m) xp = *reinterpret_cast<const uint4*>(xr + i * 8);
          part = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, xp),
                                                        __builtin_bit_cast(v8bf, q[i]), part, 0, 0, 0);
        }
        // output column of this lane is n0 + lr: its group scale is sc
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] = __builtin_fmaf(part[i], sc, acc[t][i]);
      }
    }
  }
  if (bad) publish(p.err, bad);

  // ---- reduce the block's waves (fixed order)
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_red[wave][t][i][lane] = acc[t][i];
  __syncthreads();
  // thread -> (t, i, lane) output slot; output element m = t*16 + 4*lg + i, n = n0 + lr
  const uint32_t slots = MT * 4 * 64;
  for (uint32_t slot = tid; slot < slots; slot += kThreads) {
    const uint32_t t = slot / 256, i = (slot / 64) % 4, l = slot % 64;
    float v = 0.0f;
#pragma unroll
    for (int wv = 0; wv < kWaves; ++wv) v += s_red[wv][t][i][l];
    s_red[0][t][i][l] = v;
  }
  __syncthreads();

  if (p.ksplit > 1) {
    for (uint32_t slot = tid; slot < slots; slot += kThreads) {
      const uint32_t t = slot / 256, i = (slot / 64) % 4, l = slot % 64;
      const uint32_t mrow = t * 16 + 4 * (l >> 4) + i, col = n0 + (l & 15);
      if (mrow < p.m) p.partial[((uint64_t)ks * p.m + mrow) * p.n + col] = s_red[0][t][i][l];
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
      const uint32_t prev = atomicAdd(&p.tickets[rowblk], 1u);
      s_last = prev == p.ksplit - 1;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
  }
  uint32_t nonfinite = 0;
  for (uint32_t slot = tid; slot < slots; slot += kThreads) {
    const uint32_t t = slot / 256, i = (slot / 64) % 4, l = slot % 64;
    const uint32_t mrow = t * 16 + 4 * (l >> 4) + i, col = n0 + (l & 15);
    if (mrow >= p.m) continue;
    float v;
    if (p.ksplit > 1) {
      v = 0.0f;
      for (uint32_t s = 0; s < p.ksplit; ++s)
        v += __hip_atomic_load(&p.partial[((uint64_t)s * p.m + mrow) * p.n + col], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    } else {
      v = s_red[0][t][i][l];
    }
    if (!__builtin_isfinite(v)) nonfinite = 1;
    if (p.out_f32) static_cast<float*>(p.out)[(uint64_t)mrow * p.n + col] = v;
    else static_cast<uint16_t*>(p.out)[(uint64_t)mrow * p.n + col] = (uint16_t)f32_to_bf16_bits(v);
  }
  if (nonfinite && FMT != kWBf16) publish(p.err, kQwenNonFinite);
  if (p.ksplit > 1 && tid == 0) p.tickets[rowblk] = 0u;
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

struct Plan {
  uint32_t ksplit, k_per_block, mt;
};

template <int FMT>
Plan plan_for(uint32_t m, uint32_t n, uint32_t k) {
  Plan pl;
  pl.mt = (m + 15) / 16;
  const uint32_t sk = step_k<FMT>();
  const uint32_t rowblks = n / 16;
  const uint32_t steps = k / sk;
  // aim for >= 2048 waves in flight while each wave keeps >= 4 steps
  uint32_t ks = (2048 + rowblks * kWaves - 1) / (rowblks * kWaves);
  const uint32_t max_ks = steps / (kWaves * 4) > 0 ? steps / (kWaves * 4) : 1;
  if (ks > max_ks) ks = max_ks;
  if (ks < 1) ks = 1;
  if (ks > 64) ks = 64;
  const uint32_t steps_per_block = (steps + ks - 1) / ks;
  pl.k_per_block = steps_per_block * sk;
  pl.ksplit = (k + pl.k_per_block - 1) / pl.k_per_block;
  return pl;
}

uint64_t workspace_for(uint32_t m, uint32_t n, const Plan& pl) {
  if (pl.ksplit <= 1) return 0;
  const uint64_t tickets = ((uint64_t)(n / 16) * 4 + 255) / 256 * 256;
  return tickets + (uint64_t)pl.ksplit * m * n * 4;
}

template <int FMT>
St launch_gemv(const GemvParams& base, Plan pl, void* ws, uint64_t ws_bytes, hipStream_t s) {
  GemvParams p = base;
  if (!ws) {
    // no workspace: one block column per 16 rows, waves split K in-block
    pl.ksplit = 1;
    pl.k_per_block = p.k;
  }
  p.ksplit = pl.ksplit;
  p.k_per_block = pl.k_per_block;
  if (pl.ksplit > 1) {
    if (!ws || ws_bytes < workspace_for(p.m, p.n, pl)) return Invalid("gemv_workspace_too_small");
    p.tickets = static_cast<uint32_t*>(ws);
    const uint64_t tickets = ((uint64_t)(p.n / 16) * 4 + 255) / 256 * 256;
    p.partial = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + tickets);
  }
  dim3 grid(p.n / 16, pl.ksplit);
  switch (pl.mt) {
    case 1: hipLaunchKernelGGL((gemv_kernel<FMT, 1>), grid, dim3(kThreads), 0, s, p); break;
    case 2: hipLaunchKernelGGL((gemv_kernel<FMT, 2>), grid, dim3(kThreads), 0, s, p); break;
    case 3: hipLaunchKernelGGL((gemv_kernel<FMT, 3>), grid, dim3(kThreads), 0, s, p); break;
    default: hipLaunchKernelGGL((gemv_kernel<FMT, 4>), grid, dim3(kThreads), 0, s, p); break;
  }
  return AfterLaunch("gemv_launch_failed");
}

}  // namespace

uint64_t W4a16WorkspaceBytes(uint32_t m, uint32_t n, uint32_t k) {
  if (m == 0 || n == 0 || k == 0 || k % 128) return 0;
  return workspace_for(m, n, plan_for<kWAsym>(m, n, k));
}

uint64_t Bf16GemvWorkspaceBytes(uint32_t m, uint32_t n, uint32_t k) {
  if (m == 0 || n == 0 || k == 0 || k % 32) return 0;
  return workspace_for(m, n, plan_for<kWBf16>(m, n, k));
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
  return launch_gemv<kWBf16>(p, plan_for<kWBf16>(a.m, a.n, a.k), a.workspace, a.workspace_bytes, a.stream);
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
    return launch_gemv<kWSym>(p, plan_for<kWSym>(a.m, a.n, a.k), a.workspace, a.workspace_bytes, a.stream);
  return launch_gemv<kWAsym>(p, plan_for<kWAsym>(a.m, a.n, a.k), a.workspace, a.workspace_bytes, a.stream);
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
