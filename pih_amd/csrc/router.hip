// MoE router top-k for gfx950: raw router scores [T, E] (the output of the
// router GEMM) -> expert ids and route weights [T, k] in rank order, on the
// device, so nothing travels to the host between the router GEMM and the
// route plan.  Two selections:
//   kRouterSqrtSoftplus  the V4 learned router (plugins/model-deepseek-v4-
//     flash/deepseek_learned_router.cpp:10-81): base = sqrt(softplus(raw))
//     with the stable softplus, ranked by base + bias[e], weights base /
//     sum(base over the top-k, rank order) * scale (1.5 in the reference);
//   kRouterSoftmax  BASELINE's softmax top-k, renormalised: softmax is
//     strictly increasing, so the top-k of the probabilities is the top-k of
//     the scores, and the renormalised weights are exp(s - s_max) over the
//     selected scores divided by their sum (the full softmax denominator
//     cancels).
// Ranking is (selection descending, expert id ascending), the reference's
// partial_sort comparator (deepseek_learned_router.cpp:57-64).
//
// One wavefront per token: lane l holds experts l, l + 64, ... (E <= 1024;
// the kernel is instantiated for the 1, 2, 4, 8 or 16 per lane that E
// needs, so E = 256 keeps 4 candidates and ~35 registers).  Each of the k
// rounds takes every lane's best untaken
// candidate, reduces (selection, id, base) across the wave with xor
// shuffles so every lane knows the winner, and the owning lane marks it
// taken.  Every lane adds the winner's base in rank order, which is the
// reference's summation order for the weight denominator.
//
// Error bits: 1 non-finite score, 2 non-finite bias, 4 top-k weight sum
// non-finite or <= 0.  A non-finite selection value ranks as -inf.
#include "device_common.hpp"
#include "kernels.hpp"

namespace pih_amd {
namespace {

constexpr uint32_t kRouterMaxExperts = 1024;
constexpr uint32_t kRouterMaxTopk = 32;
constexpr uint32_t kRouterWaves = 4;
constexpr uint32_t kNone = 0xffffffffu;

__device__ __forceinline__ float stable_softplus(float v) {
  return v > 0.0f ? v + log1pf(expf(-v)) : log1pf(expf(v));
}

// (a, ia) ranks before (b, ib); kNone ranks after everything.
__device__ __forceinline__ bool ranks_before(float a, uint32_t ia, float b, uint32_t ib) {
  if (ib == kNone) return ia != kNone;
  if (ia == kNone) return false;
  return a > b || (a == b && ia < ib);
}

// PER experts per lane (E <= 64 * PER): the candidates stay in registers
template <int MODE, int PER>
__global__ __launch_bounds__(64 * kRouterWaves) void router_topk_kernel(
    const float* scores, const float* bias, uint32_t* ids, float* weights, uint32_t* err, uint32_t tokens,
    uint32_t experts, uint32_t topk, float scale) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t t = blockIdx.x * kRouterWaves + (threadIdx.x >> 6);
  if (t >= tokens) return;  // whole waves only; no block-level barrier below
  const float* s = scores + (uint64_t)t * experts;
  float sel[PER], base[PER];
  uint32_t taken = 0, bad = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint32_t e = lane + 64u * j;
    sel[j] = -INFINITY;
    base[j] = 0.0f;
    if (e < experts) {
      const float raw = s[e];
      if (!__builtin_isfinite(raw)) bad |= 1u;
      if constexpr (MODE == kRouterSqrtSoftplus) {
        const float b = bias ? bias[e] : 0.0f;
        if (!__builtin_isfinite(b)) bad |= 2u;
        base[j] = sqrtf(stable_softplus(raw));
        sel[j] = base[j] + b;
      } else {
        base[j] = raw;
        sel[j] = raw;
      }
      if (!__builtin_isfinite(sel[j])) sel[j] = -INFINITY;
    } else {
      taken |= 1u << j;
    }
  }
  uint32_t my_id = kNone;
  float my_base = 0.0f, first = 0.0f, den = 0.0f;
  for (uint32_t r = 0; r < topk; ++r) {
    float bv = -INFINITY, bb = 0.0f;
    uint32_t bi = kNone;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const uint32_t e = lane + 64u * j;
      if (!((taken >> j) & 1u) && ranks_before(sel[j], e, bv, bi)) {
        bv = sel[j];
        bi = e;
        bb = base[j];
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const uint32_t oi = __shfl_xor(bi, off, 64);
      const float ob = __shfl_xor(bb, off, 64);
      if (ranks_before(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
        bb = ob;
      }
    }
    if ((bi & 63u) == lane) {
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if ((uint32_t)j == (bi >> 6)) taken |= 1u << j;
    }
    if (r == 0) first = bb;
    if constexpr (MODE == kRouterSqrtSoftplus) {
      den += bb;
    } else {
      bb = expf(bb - first);
      den += bb;
    }
    if (lane == r) {
      my_id = bi;
      my_base = bb;
    }
  }
  if (MODE == kRouterSqrtSoftplus && (!__builtin_isfinite(den) || den <= 0.0f)) bad |= 4u;
  if (lane < topk) {
    ids[(uint64_t)t * topk + lane] = my_id;
    weights[(uint64_t)t * topk + lane] = my_base / den * scale;
  }
  if (bad) atomicOr(err, bad);
}

template <int MODE, int PER>
void launch_per(const RouterTopkArgs& a) {
  hipLaunchKernelGGL((router_topk_kernel<MODE, PER>), dim3((a.tokens + kRouterWaves - 1) / kRouterWaves),
                     dim3(64 * kRouterWaves), 0, a.stream, a.scores, a.bias, a.ids, a.weights, a.error_flag,
                     a.tokens, a.experts, a.topk, a.scale);
}

}  // namespace

St LaunchRouterTopk(const RouterTopkArgs& a) {
  if (!a.scores || !a.ids || !a.weights || !a.error_flag || !a.stream) return Invalid("router_topk_null_argument");
  if (a.tokens == 0 || a.experts == 0 || a.experts > kRouterMaxExperts || a.topk == 0 ||
      a.topk > kRouterMaxTopk || a.topk > a.experts)
    return Invalid("router_topk_shape_invalid");
  if (a.mode != kRouterSoftmax && a.mode != kRouterSqrtSoftplus) return Invalid("router_topk_mode_invalid");
  if (!__builtin_isfinite(a.scale) || a.scale <= 0.0f) return Invalid("router_topk_scale_invalid");
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  const uint32_t per = (a.experts + 63) / 64;
  if (a.mode == kRouterSqrtSoftplus) {
    if (per <= 1) launch_per<kRouterSqrtSoftplus, 1>(a);
    else if (per <= 2) launch_per<kRouterSqrtSoftplus, 2>(a);
    else if (per <= 4) launch_per<kRouterSqrtSoftplus, 4>(a);
    else if (per <= 8) launch_per<kRouterSqrtSoftplus, 8>(a);
    else launch_per<kRouterSqrtSoftplus, 16>(a);
  } else {
    if (per <= 1) launch_per<kRouterSoftmax, 1>(a);
    else if (per <= 2) launch_per<kRouterSoftmax, 2>(a);
    else if (per <= 4) launch_per<kRouterSoftmax, 4>(a);
    else if (per <= 8) launch_per<kRouterSoftmax, 8>(a);
    else launch_per<kRouterSoftmax, 16>(a);
  }
  return AfterLaunch("router_topk_launch_failed");
}

}  // namespace pih_amd
