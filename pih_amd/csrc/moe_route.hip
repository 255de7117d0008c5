// MoE routing glue for gfx950: the device-side route plan (expert histogram,
// exclusive prefix scan into expert offsets, stable permutation), the route
// gather, the ordered expert accumulate, the ordered combine and finalize.
//
// Route plan semantics follow the reference's host plan
// (plugins/model-deepseek-v4-flash/deepseek_expert_subwave_plan.cpp:32-101):
// routes sorted by (expert, token, ordinal), expert_offsets[e] the exclusive
// prefix of per-expert route counts (experts+1 entries).  Here the sort is
// never materialised: a token picks an expert at most once, so a route's
// place inside its expert segment is the number of earlier tokens that chose
// the same expert.  Tokens are processed in chunks of 64 (one wave); each
// chunk builds a 64-bit token mask per expert with LDS atomics (order
// independent, hence deterministic), one block turns the per-chunk
// popcounts into chunk bases and expert offsets, and a final pass computes
// every route's row as offset + chunk base + popcount(mask & lanes_below).
//
// Error bits: 1 expert id out of range, 2 expert repeated within a token,
// 4 route weight non-finite or negative.  An invalid route gets no row
// (token_rows = 0xffffffff) and is left out of the offsets.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "device_common.hpp"
#include "fp8_quant_device.hpp"
#include "kernels.hpp"

// Scratch of the no-allocation route plan (LaunchRoutePlanNoAlloc): the
// per-chunk expert masks and bases, kRoutePlanNoAllocScratchBytes at most.
// Every device the library runs on holds its own copy until the process
// ends.  Host code never passes this name to a kernel (on the host it is a
// stand-in, not a device address); it uses the address hipGetSymbolAddress
// returns for the current device.
static __device__ __align__(256) unsigned char scratch[pih_amd::kRoutePlanNoAllocScratchBytes];

namespace pih_amd {
namespace {

constexpr uint32_t kChunk = 64;
constexpr uint32_t kMaxExperts = 1024;
constexpr uint32_t kMaxTopk = 32;
constexpr uint32_t kNoRow = 0xffffffffu;

// Validates route (t, j) and returns its expert or kNoRow.
__device__ __forceinline__ uint32_t route_expert(const uint32_t* ids, const float* weights,
                                                 uint32_t t, uint32_t j, uint32_t topk,
                                                 uint32_t experts, uint32_t& bad) {
  const uint32_t* row = ids + (uint64_t)t * topk;
  const uint32_t e = row[j];
  if (e >= experts) {
    bad |= 1u;
    return kNoRow;
  }
  for (uint32_t p = 0; p < j; ++p)
    if (row[p] == e) {
      bad |= 2u;
      return kNoRow;
    }
  const float w = weights[(uint64_t)t * topk + j];
  if (!__builtin_isfinite(w) || w < 0.0f) {
    bad |= 4u;
    return kNoRow;
  }
  return e;
}

// Chunk `chunk` of 64 tokens: the 64-bit token mask of every expert, built
// with LDS atomics (order independent) by the block's waves, wave w taking
// the routes j = w, w + waves, ...; s_mask holds `experts` words.
__device__ __forceinline__ void route_mask_chunk(const uint32_t* ids, const float* weights, unsigned long long* masks,
                                                 unsigned long long* s_mask, uint32_t* err, uint32_t chunk,
                                                 uint32_t tokens, uint32_t topk, uint32_t experts) {
  const uint32_t lane = threadIdx.x & (kChunk - 1), wave = threadIdx.x / kChunk, waves = blockDim.x / kChunk;
  for (uint32_t e = threadIdx.x; e < experts; e += blockDim.x) s_mask[e] = 0ull;
  __syncthreads();
  const uint32_t t = chunk * kChunk + lane;
  uint32_t bad = 0;
  if (t < tokens) {
    for (uint32_t j = wave; j < topk; j += waves) {
      const uint32_t e = route_expert(ids, weights, t, j, topk, experts, bad);
      if (e != kNoRow) atomicOr(&s_mask[e], 1ull << lane);
    }
  }
  __syncthreads();
  for (uint32_t e = threadIdx.x; e < experts; e += blockDim.x) masks[(uint64_t)chunk * experts + e] = s_mask[e];
  if (bad) atomicOr(err, bad);
}

__global__ __launch_bounds__(256) void route_mask_kernel(const uint32_t* ids, const float* weights,
                                                         unsigned long long* masks, uint32_t* err, uint32_t tokens,
                                                         uint32_t topk, uint32_t experts) {
  extern __shared__ unsigned long long s_mask[];
  route_mask_chunk(ids, weights, masks, s_mask, err, blockIdx.x, tokens, topk, experts);
}

// The MoE layer's first launch: blocks [0, chunks) build the route masks,
// the blocks after them quantize the token activations (quant_groups over
// the remaining blocks) -- two independent jobs in one launch, the route
// blocks first so the plan's next launch can start as soon as possible.
template <int FMT>
__global__ __launch_bounds__(256) void route_mask_quant_kernel(const uint32_t* ids, const float* weights,
                                                               unsigned long long* masks, uint32_t* err,
                                                               uint32_t tokens, uint32_t topk, uint32_t experts,
                                                               uint32_t chunks, const uint16_t* x, uint8_t* codes,
                                                               void* scales, uint32_t hidden) {
  extern __shared__ unsigned long long s_mask[];
  if (blockIdx.x < chunks) {
    route_mask_chunk(ids, weights, masks, s_mask, err, blockIdx.x, tokens, topk, experts);
    return;
  }
  const uint64_t seg0 = ((uint64_t)(blockIdx.x - chunks) * blockDim.x + threadIdx.x) >> 4;
  const uint64_t seg_step = ((uint64_t)(gridDim.x - chunks) * blockDim.x) >> 4;
  const uint32_t bad = quant_groups<FMT, false>(x, nullptr, codes, scales, tokens, hidden, tokens, seg0, seg_step);
  if (bad) atomicOr(err, bad);
}

// A plan of at most 64 tokens (one chunk) in one launch: block 0 builds the
// chunk's expert masks in LDS, scans their popcounts into the expert offsets
// (256 threads, 4 experts each) and places every route at offset +
// popcount(mask & lanes below) -- the three-launch plan's arithmetic with its
// only chunk base 0, so the same rows -- and, with QFMT >= 0, the blocks after
// it quantize the token activations as route_mask_quant_kernel's do.
template <int QFMT>
__global__ __launch_bounds__(256) void route_plan_one_chunk_kernel(
    const uint32_t* ids, const float* weights, uint32_t* offsets, uint32_t* row_token, float* row_weight,
    uint32_t* token_rows, uint32_t* err, uint32_t tokens, uint32_t topk, uint32_t experts, const uint16_t* x,
    uint8_t* codes, void* scales, uint32_t hidden) {
  extern __shared__ unsigned long long s_mask[];  // [experts] masks, then [experts] u32 offsets
  __shared__ uint32_t s_wave[4];
  if (blockIdx.x != 0) {
    if constexpr (QFMT >= 0) {
      const uint64_t seg0 = ((uint64_t)(blockIdx.x - 1) * blockDim.x + threadIdx.x) >> 4;
      const uint64_t seg_step = ((uint64_t)(gridDim.x - 1) * blockDim.x) >> 4;
      const uint32_t bad = quant_groups<QFMT, false>(x, nullptr, codes, scales, tokens, hidden, tokens, seg0, seg_step);
      if (bad) atomicOr(err, bad);
    }
    return;
  }
  uint32_t* s_off = reinterpret_cast<uint32_t*>(s_mask + experts);
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (uint32_t e = tid; e < experts; e += 256) s_mask[e] = 0ull;
  __syncthreads();
  uint32_t bad = 0;
  if (lane < tokens) {
    for (uint32_t j = wave; j < topk; j += 4) {
      const uint32_t e = route_expert(ids, weights, lane, j, topk, experts, bad);
      if (e != kNoRow) atomicOr(&s_mask[e], 1ull << lane);
    }
  }
  if (bad) atomicOr(err, bad);
  __syncthreads();
  // exclusive scan of the popcounts: thread tid owns experts [4 tid, 4 tid + 4)
  uint32_t pc[4], sum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t e = 4 * tid + i;
    pc[i] = e < experts ? (uint32_t)__popcll(s_mask[e]) : 0u;
    sum += pc[i];
  }
  uint32_t incl = sum;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t v = __shfl_up(incl, o, 64);
    if ((int)lane >= o) incl += v;
  }
  if (lane == 63) s_wave[wave] = incl;
  __syncthreads();
  uint32_t run = incl - sum;
  for (uint32_t w = 0; w < wave; ++w) run += s_wave[w];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t e = 4 * tid + i;
    if (e < experts) {
      s_off[e] = run;
      offsets[e] = run;
    }
    run += pc[i];
  }
  if (tid == 255) offsets[experts] = run;  // the total, every expert counted
  __syncthreads();
  for (uint32_t r = tid; r < tokens * topk; r += 256) {
    const uint32_t t = r / topk, j = r % topk;
    uint32_t ignored = 0;  // reported above
    const uint32_t e = route_expert(ids, weights, t, j, topk, experts, ignored);
    uint32_t row = kNoRow;
    if (e != kNoRow) {
      const unsigned long long below = t ? (~0ull >> (64 - t)) : 0ull;
      row = s_off[e] + (uint32_t)__popcll(s_mask[e] & below);
      row_token[row] = t;
      row_weight[row] = weights[r];
    }
    token_rows[r] = row;
  }
}

// One block, one thread per expert: chunk bases by a walk over the chunks
// (the masks of 16 chunks loaded before they are summed, so the walk waits
// on memory once per 16 chunks), then a block-wide exclusive scan of the
// per-expert totals.
__global__ __launch_bounds__(kMaxExperts) void route_scan_kernel(const unsigned long long* masks,
                                                                 uint32_t* bases,
                                                                 uint32_t* offsets,
                                                                 uint32_t chunks,
                                                                 uint32_t experts) {
  constexpr uint32_t kBatch = 16;
  __shared__ uint32_t s_scan[kMaxExperts];
  const uint32_t e = threadIdx.x;
  uint32_t total = 0;
  if (e < experts) {
    for (uint32_t c0 = 0; c0 < chunks; c0 += kBatch) {
      // unconditional loads (past the end: the last chunk again, not
      // counted); a load under a branch would be waited for on the spot
      unsigned long long mk[kBatch];
#pragma unroll
      for (uint32_t i = 0; i < kBatch; ++i) mk[i] = masks[(uint64_t)min(c0 + i, chunks - 1) * experts + e];
      uint32_t pc[kBatch];
#pragma unroll
      for (uint32_t i = 0; i < kBatch; ++i) pc[i] = c0 + i < chunks ? (uint32_t)__popcll(mk[i]) : 0u;
#pragma unroll
      for (uint32_t i = 0; i < kBatch; ++i) {
        if (c0 + i < chunks) bases[(uint64_t)(c0 + i) * experts + e] = total;
        total += pc[i];
      }
    }
  }
  s_scan[e] = total;
  __syncthreads();
  for (uint32_t off = 1; off < blockDim.x; off <<= 1) {
    const uint32_t v = e >= off ? s_scan[e - off] : 0u;
    __syncthreads();
    s_scan[e] += v;
    __syncthreads();
  }
  if (e < experts) offsets[e] = s_scan[e] - total;
  if (e == experts - 1) offsets[experts] = s_scan[e];
}

// One thread per route (t, j): its row is offset + chunk base + the number
// of earlier tokens of its chunk that chose the same expert.
__global__ __launch_bounds__(256) void route_scatter_kernel(
    const uint32_t* ids, const float* weights, const unsigned long long* masks,
    const uint32_t* bases, const uint32_t* offsets, uint32_t* row_token, float* row_weight,
    uint32_t* token_rows, uint32_t tokens, uint32_t topk, uint32_t experts) {
  const uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= (uint64_t)tokens * topk) return;
  const uint32_t t = (uint32_t)(r / topk), j = (uint32_t)(r % topk);
  const uint32_t chunk = t / kChunk, lane = t % kChunk;
  const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
  uint32_t bad = 0;  // reported by the mask pass
  const uint32_t e = route_expert(ids, weights, t, j, topk, experts, bad);
  uint32_t row = kNoRow;
  if (e != kNoRow) {
    const unsigned long long m = masks[(uint64_t)chunk * experts + e];
    row = offsets[e] + bases[(uint64_t)chunk * experts + e] + (uint32_t)__popcll(m & below);
    row_token[row] = t;
    row_weight[row] = weights[r];
  }
  token_rows[r] = row;
}

// dst[r, :] = src[idx[r], :], 16 bytes per lane.
__global__ __launch_bounds__(256) void gather_kernel(const uint16_t* src, const uint32_t* idx,
                                                     uint16_t* dst, uint32_t* err, uint32_t routes,
                                                     uint32_t tokens, uint32_t hidden) {
  const uint32_t vec = hidden / 8u;
  const uint64_t total = (uint64_t)routes * vec;
  uint32_t bad = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t r = (uint32_t)(i / vec), c = (uint32_t)(i % vec);
    const uint32_t t = idx[r];
    if (t >= tokens) {
      bad |= 1u;
      continue;
    }
    reinterpret_cast<uint4*>(dst)[(uint64_t)r * vec + c] =
        reinterpret_cast<const uint4*>(src)[(uint64_t)t * vec + c];
  }
  if (bad) atomicOr(err, bad);
}

// acc[idx[r], c] += out[r, c]; token indices strictly increasing within one
// call (reference deepseek_expert_accumulate.cu:13-39), so every (r, c) owns
// a distinct accumulator element and the sums are order-exact.
__global__ __launch_bounds__(256) void accumulate_kernel(const uint16_t* out, const uint32_t* idx,
                                                         float* acc, uint32_t* err,
                                                         uint32_t routes, uint32_t tokens,
                                                         uint32_t hidden) {
  const uint64_t total = (uint64_t)routes * hidden;
  uint32_t bad = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t r = (uint32_t)(i / hidden), c = (uint32_t)(i % hidden);
    const uint32_t t = idx[r];
    if (t >= tokens || (r != 0 && t <= idx[r - 1])) {
      bad |= 1u;
      continue;
    }
    const float v = bf16_bits_to_f32(out[i]);
    float* dst = acc + (uint64_t)t * hidden + c;
    const float next = *dst + v;
    if (!__builtin_isfinite(v) || !__builtin_isfinite(next)) {
      bad |= 2u;
      continue;
    }
    *dst = next;
  }
  if (bad) atomicOr(err, bad);
}

// out[t, :] = bf16(sum of t's expert rows in ascending row order (= ascending
// expert id) + shared).  The fp32 adds run in the order the reference's
// accumulator oracle applies them (src/model/
// deepseek_expert_accumulator_oracle.cpp:20-85), so results are bit-exact.
__global__ __launch_bounds__(512) void combine_kernel(const uint16_t* expert_out,
                                                      const uint32_t* token_rows,
                                                      const uint16_t* shared, uint16_t* out,
                                                      uint32_t* err, uint32_t tokens,
                                                      uint32_t topk, uint32_t hidden,
                                                      uint32_t rows) {
  const uint32_t t = blockIdx.x;
  if (t >= tokens) return;
  uint32_t r[kMaxTopk];
  uint32_t n = 0;
  for (uint32_t j = 0; j < topk; ++j) {
    const uint32_t v = token_rows[(uint64_t)t * topk + j];
    if (v < rows) {
      uint32_t p = n++;
      while (p > 0 && r[p - 1] > v) {
        r[p] = r[p - 1];
        --p;
      }
      r[p] = v;
    }
  }
  uint32_t bad = 0;
  const uint32_t vec = hidden / 8u;
  // every row is read once: non-temporal loads
  // rows past n (n <= 8 in the unrolled path) repeat row r[0]; their values
  // are replaced by +0.0f, which leaves the sum unchanged (it starts at +0.0f
  // and so is never -0.0f), so the sum keeps the ascending row order exactly
  constexpr uint32_t kUnroll = 8;
  // block (t, y) covers part y of the row's chunks (few tokens: the rows are
  // split over gridDim.y blocks so that every CU has one)
  const uint32_t per = (vec + gridDim.y - 1) / gridDim.y, c_end = min(vec, (blockIdx.y + 1) * per);
  for (uint32_t c = blockIdx.y * per + threadIdx.x; c < c_end; c += blockDim.x) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    auto add = [&](const uint4& x, bool live) {
      const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] += live ? bf16_bits_to_f32(w[i] & 0xffffu) : 0.0f;
        acc[2 * i + 1] += live ? bf16_bits_to_f32(w[i] >> 16) : 0.0f;
      }
    };
    if (n > 0 && n <= kUnroll) {
      // every load first (unconditional, in bounds), then the adds in order
      uint4 x[kUnroll];
#pragma unroll
      for (uint32_t j = 0; j < kUnroll; ++j)
        x[j] = load16_nt(reinterpret_cast<const uint4*>(expert_out) + (uint64_t)r[j < n ? j : 0] * vec + c);
#pragma unroll
      for (uint32_t j = 0; j < kUnroll; ++j) add(x[j], j < n);
    } else {
      for (uint32_t j = 0; j < n; ++j)
        add(load16_nt(reinterpret_cast<const uint4*>(expert_out) + (uint64_t)r[j] * vec + c), true);
    }
    if (shared) {
      const uint4 x = load16_nt(reinterpret_cast<const uint4*>(shared) + (uint64_t)t * vec + c);
      const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] += bf16_bits_to_f32(w[i] & 0xffffu);
        acc[2 * i + 1] += bf16_bits_to_f32(w[i] >> 16);
      }
    }
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (!__builtin_isfinite(acc[2 * i]) || !__builtin_isfinite(acc[2 * i + 1])) bad |= 4u;
      o[i] = f32_to_bf16_bits(acc[2 * i]) | (f32_to_bf16_bits(acc[2 * i + 1]) << 16);
    }
    reinterpret_cast<uint4*>(out)[(uint64_t)t * vec + c] = make_uint4(o[0], o[1], o[2], o[3]);
  }
  if (bad) atomicOr(err, bad);
}

__global__ __launch_bounds__(256) void finalize_kernel(const float* acc, const uint16_t* shared,
                                                       uint16_t* out, uint32_t* err,
                                                       uint64_t count) {
  uint32_t bad = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const float v = acc[i] + (shared ? bf16_bits_to_f32(shared[i]) : 0.0f);
    if (!__builtin_isfinite(v)) {
      bad |= 4u;
      continue;
    }
    out[i] = (uint16_t)f32_to_bf16_bits(v);
  }
  if (bad) atomicOr(err, bad);
}

uint32_t grid_for(uint64_t items, uint32_t threads = 256, uint32_t cap = 16384) {
  uint64_t b = (items + threads - 1) / threads;
  if (b == 0) b = 1;
  return (uint32_t)(b > cap ? cap : b);
}

}  // namespace

uint64_t RoutePlanWorkspaceBytes(uint32_t tokens, uint32_t topk, uint32_t experts) {
  (void)topk;
  const uint64_t chunks = (tokens + kChunk - 1) / kChunk;
  const uint64_t mask_bytes = chunks * experts * 8ull;
  const uint64_t base_bytes = chunks * experts * 4ull;
  return ((mask_bytes + 255) / 256) * 256 + base_bytes;
}

namespace {

// The plan's three launches; with `quant`, the first launch also quantizes
// the token activations (route_mask_quant_kernel).
St EnqueueRoutePlan(const RoutePlanArgs& a, const Fp8QuantArgs* quant) {
  if (!a.topk_ids || !a.topk_weights || !a.expert_offsets || !a.row_token || !a.row_weight ||
      !a.token_rows || !a.workspace || !a.error_flag || !a.stream)
    return Invalid("route_plan_null_argument");
  if (a.tokens == 0 || a.topk == 0 || a.topk > kMaxTopk || a.experts == 0 ||
      a.experts > kMaxExperts || (uint64_t)a.tokens * a.topk > 0x7fffffffull)
    return Invalid("route_plan_shape_invalid");
  if (a.workspace_bytes < RoutePlanWorkspaceBytes(a.tokens, a.topk, a.experts))
    return Invalid("route_plan_workspace_too_small");
  if (quant) {
    if (!quant->input || !quant->codes || !quant->scales || quant->rows) return Invalid("fp8_quant_null_argument");
    if (quant->row_count != a.tokens || quant->k == 0 || quant->k % 128u) return Invalid("fp8_quant_shape_invalid");
    if (quant->fmt != kScaleF32 && quant->fmt != kScaleUe8m0) return Invalid("fp8_quant_scale_format_invalid");
  }
  const uint32_t chunks = (a.tokens + kChunk - 1) / kChunk;
  const uint64_t mask_bytes = (uint64_t)chunks * a.experts * 8ull;
  auto* masks = static_cast<unsigned long long*>(a.workspace);
  auto* bases = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(a.workspace) +
                                            ((mask_bytes + 255) / 256) * 256);
  const uint32_t lds = a.experts * 8u;
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  if (chunks == 1) {
    // one chunk of tokens (decode batches): the whole plan in one launch
    const uint32_t lds1 = a.experts * 12u;
    if (!quant) {
      hipLaunchKernelGGL(route_plan_one_chunk_kernel<-1>, dim3(1), dim3(256), lds1, a.stream, a.topk_ids,
                         a.topk_weights, a.expert_offsets, a.row_token, a.row_weight, a.token_rows, a.error_flag,
                         a.tokens, a.topk, a.experts, nullptr, nullptr, nullptr, 0u);
    } else {
      const uint32_t grid = 1 + QuantBlocks((uint64_t)quant->row_count * (quant->k / 128u));
      if (quant->fmt == kScaleUe8m0)
        hipLaunchKernelGGL(route_plan_one_chunk_kernel<kScaleUe8m0>, dim3(grid), dim3(256), lds1, a.stream,
                           a.topk_ids, a.topk_weights, a.expert_offsets, a.row_token, a.row_weight, a.token_rows,
                           a.error_flag, a.tokens, a.topk, a.experts, quant->input, quant->codes, quant->scales,
                           quant->k);
      else
        hipLaunchKernelGGL(route_plan_one_chunk_kernel<kScaleF32>, dim3(grid), dim3(256), lds1, a.stream,
                           a.topk_ids, a.topk_weights, a.expert_offsets, a.row_token, a.row_weight, a.token_rows,
                           a.error_flag, a.tokens, a.topk, a.experts, quant->input, quant->codes, quant->scales,
                           quant->k);
    }
    return AfterLaunch("route_plan_launch_failed");
  }
  if (!quant) {
    hipLaunchKernelGGL(route_mask_kernel, dim3(chunks), dim3(256), lds, a.stream, a.topk_ids, a.topk_weights, masks,
                       a.error_flag, a.tokens, a.topk, a.experts);
  } else {
    const uint32_t grid = chunks + QuantBlocks((uint64_t)quant->row_count * (quant->k / 128u));
    if (quant->fmt == kScaleUe8m0)
      hipLaunchKernelGGL(route_mask_quant_kernel<kScaleUe8m0>, dim3(grid), dim3(256), lds, a.stream, a.topk_ids,
                         a.topk_weights, masks, a.error_flag, a.tokens, a.topk, a.experts, chunks, quant->input,
                         quant->codes, quant->scales, quant->k);
    else
      hipLaunchKernelGGL(route_mask_quant_kernel<kScaleF32>, dim3(grid), dim3(256), lds, a.stream, a.topk_ids,
                         a.topk_weights, masks, a.error_flag, a.tokens, a.topk, a.experts, chunks, quant->input,
                         quant->codes, quant->scales, quant->k);
  }
  const uint32_t scan_threads = ((a.experts + 63) / 64) * 64;
  hipLaunchKernelGGL(route_scan_kernel, dim3(1), dim3(scan_threads), 0, a.stream, masks, bases,
                     a.expert_offsets, chunks, a.experts);
  const uint64_t routes = (uint64_t)a.tokens * a.topk;
  hipLaunchKernelGGL(route_scatter_kernel, dim3((uint32_t)((routes + 255) / 256)), dim3(256), 0, a.stream,
                     a.topk_ids, a.topk_weights, masks, bases, a.expert_offsets, a.row_token, a.row_weight,
                     a.token_rows, a.tokens, a.topk, a.experts);
  return AfterLaunch("route_plan_launch_failed");
}

}  // namespace

St LaunchRoutePlan(const RoutePlanArgs& a) { return EnqueueRoutePlan(a, nullptr); }

St LaunchRoutePlanWithQuant(const RoutePlanArgs& a, const Fp8QuantArgs& quant) {
  if (!quant.error_flag || quant.error_flag != a.error_flag || quant.stream != a.stream)
    return Invalid("route_plan_quant_mismatch");
  return EnqueueRoutePlan(a, &quant);
}

namespace {

constexpr int kMaxDevices = 64;

struct ScratchSlot {
  std::mutex lock;
  std::atomic<void*> ptr{nullptr};
};
ScratchSlot g_scratch[kMaxDevices];

// The scratch array's address on the current device, looked up with that
// device current and kept once the lookup has succeeded (a failed lookup is
// retried on the next call).
St NoAllocScratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return Internal("route_plan_noalloc_device_unavailable");
  ScratchSlot& slot = g_scratch[dev];
  void* p = slot.ptr.load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> guard(slot.lock);
    p = slot.ptr.load(std::memory_order_relaxed);
    if (!p) {
      const St clean = RequireCleanLastError();  // an earlier error stays reported, not cleared below
      if (!clean.ok()) return clean;
      void* found = nullptr;
      if (hipGetSymbolAddress(&found, HIP_SYMBOL(scratch)) != hipSuccess || found == nullptr) {
        (void)hipGetLastError();  // this lookup's own error: a later call may retry
        return Internal("route_plan_noalloc_scratch_unavailable");
      }
      slot.ptr.store(found, std::memory_order_release);
      p = found;
    }
  }
  *out = p;
  return Ok();
}

}  // namespace

St LaunchRoutePlanNoAlloc(const RoutePlanArgs& args) {
  if (args.workspace || args.workspace_bytes) return Invalid("route_plan_noalloc_workspace_must_be_zero");
  if (args.tokens == 0 || args.topk == 0 || args.topk > kMaxTopk || args.experts == 0 ||
      args.experts > kMaxExperts || (uint64_t)args.tokens * args.topk > 0x7fffffffull)
    return Invalid("route_plan_shape_invalid");
  if (RoutePlanWorkspaceBytes(args.tokens, args.topk, args.experts) > kRoutePlanNoAllocScratchBytes)
    return Invalid("route_plan_noalloc_plan_exceeds_scratch");
  RoutePlanArgs a = args;
  St s = NoAllocScratch(&a.workspace);
  if (!s.ok()) return s;
  a.workspace_bytes = kRoutePlanNoAllocScratchBytes;
  return LaunchRoutePlan(a);
}

St LaunchRouteGather(const GatherArgs& a) {
  if (!a.source || !a.token_index || !a.dest || !a.error_flag || !a.stream)
    return Invalid("route_gather_null_argument");
  if (a.routes == 0 || a.tokens == 0 || a.hidden == 0 || a.hidden % 8u)
    return Invalid("route_gather_shape_invalid");
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  hipLaunchKernelGGL(gather_kernel, dim3(grid_for((uint64_t)a.routes * a.hidden / 8u)), dim3(256),
                     0, a.stream, a.source, a.token_index, a.dest, a.error_flag, a.routes,
                     a.tokens, a.hidden);
  return AfterLaunch("route_gather_launch_failed");
}

St LaunchOrderedAccumulate(const AccumulateArgs& a) {
  if (!a.expert_out || !a.token_index || !a.acc || !a.error_flag || !a.stream)
    return Invalid("expert_accumulate_null_argument");
  if (a.routes == 0 || a.tokens == 0 || a.hidden == 0 || a.routes > a.tokens)
    return Invalid("expert_accumulate_shape_invalid");
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  hipLaunchKernelGGL(accumulate_kernel, dim3(grid_for((uint64_t)a.routes * a.hidden)), dim3(256), 0,
                     a.stream, a.expert_out, a.token_index, a.acc, a.error_flag, a.routes,
                     a.tokens, a.hidden);
  return AfterLaunch("expert_accumulate_launch_failed");
}

St LaunchMoeCombine(const CombineArgs& a) {
  if (!a.expert_out || !a.token_rows || !a.out || !a.error_flag || !a.stream)
    return Invalid("moe_combine_null_argument");
  if (a.tokens == 0 || a.topk == 0 || a.topk > kMaxTopk || a.hidden == 0 || a.hidden % 8u ||
      a.rows == 0)
    return Invalid("moe_combine_shape_invalid");
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  // one block per token (below 256 tokens: per part of a token's row, up to
  // a block per CU, at least 64 chunks each); its threads cover the part's
  // 16-byte chunks in equal passes (hidden 7168: 896 chunks = 2 passes of
  // 448 threads, where 256 threads left the fourth pass half empty)
  const uint32_t vec = a.hidden / 8u;
  const uint32_t parts = a.tokens < 256u ? std::min((256u + a.tokens - 1) / a.tokens, std::max(1u, vec / 64u)) : 1u;
  const uint32_t pvec = (vec + parts - 1) / parts, passes = (pvec + 511u) / 512u;
  const uint32_t threads = ((pvec + passes - 1) / passes + 63u) / 64u * 64u;
  hipLaunchKernelGGL(combine_kernel, dim3(a.tokens, parts), dim3(threads), 0, a.stream, a.expert_out,
                     a.token_rows, a.shared, a.out, a.error_flag, a.tokens, a.topk, a.hidden,
                     a.rows);
  return AfterLaunch("moe_combine_launch_failed");
}

St LaunchFinalize(const FinalizeArgs& a) {
  if (!a.acc || !a.out || !a.error_flag || !a.stream) return Invalid("expert_finalize_null_argument");
  if (a.count == 0) return Invalid("expert_finalize_shape_invalid");
  St clean = RequireCleanLastError();
  if (!clean.ok()) return clean;
  hipLaunchKernelGGL(finalize_kernel, dim3(grid_for(a.count)), dim3(256), 0, a.stream, a.acc,
                     a.shared, a.out, a.error_flag, a.count);
  return AfterLaunch("expert_finalize_launch_failed");
}

}  // namespace pih_amd
