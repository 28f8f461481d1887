// Router projection, top-2 selection and deterministic expert grouping.
//
// Reference semantics:
//   * logits = x . Wr^T in fp32, p = softmax(logits), (w, i) = topk(p, 2),
//     w /= sum(w)                       (parrot/model.py:520-527)
//   * selection by a strict '>' scan in expert order, so ties go to the lower
//     expert index; route weights renormalised over the two selected
//     exponentials                       (parrot/kernels/moe_bf16.metal:99-129)
//   * capacity C and exact overflow: an assignment whose slot is >= C is
//     computed by the overflow path, never dropped
//                                        (parrot/metal_moe.py:388-406)
// The reference assigns slots with atomics (moe_bf16.metal:130-133), which
// yields an arbitrary order.  Here the slot of assignment a = 2t + k is its
// stable rank among earlier assignments to the same expert, the order of
// torch.where(indices == e) in parrot/model.py:548, computed without atomics:
// block-local ranks in the route kernel, then a per-expert exclusive scan of
// block histograms in the group kernel.
#include "common.h"

namespace parrot {

namespace {

constexpr int kStepsPerChunk = 8;  // 32-wide k steps whose loads are in flight at once

__device__ __forceinline__ bf16x8 load_bf16x8(const uint16_t* p) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  return __builtin_bit_cast(bf16x8, v);
}

// Block-local stable rank of each of the block's assignments and the
// block's per-expert histogram.  `ids` holds expert ids (-1 = padding or an
// id outside [0, experts)).
__device__ __forceinline__ void block_rank(const int* ids, int64_t a0, int64_t n_assign,
                                           int experts, int32_t* positions,
                                           int32_t* block_counts) {
  const int j = threadIdx.x;
  if (j < kRouteAssignPerBlock) {
    const int e = ids[j];
    if (e >= 0 && a0 + j < n_assign) {
      int rank = 0;
      for (int i = 0; i < j; ++i) rank += ids[i] == e;
      positions[a0 + j] = rank;
    }
  } else if (j >= 64 && j - 64 < experts) {
    const int e = j - 64;
    int count = 0;
    for (int i = 0; i < kRouteAssignPerBlock; ++i) count += ids[i] == e;
    block_counts[static_cast<int64_t>(blockIdx.x) * experts + e] = count;
  }
}

// One workgroup routes 16 tokens.  The router projection [16 x dim] .
// [dim x E] runs on v_mfma_f32_16x16x32_bf16 with the 32-wide k steps split
// round-robin over the 4 wavefronts; each wavefront issues the loads of up
// to 8 steps before its MFMAs, and the partial logits are summed in a fixed
// order through LDS.  Fragments: lane l holds row/col (l & 15) and the 8 k
// values at (l >> 4) * 8 of a step; C holds column (l & 15), rows
// 4 (l >> 4) + r.  With GIVEN_LOGITS the fp32 logits are read instead.
template <bool GIVEN_LOGITS>
__global__ __launch_bounds__(256) void route_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wr,
    const float* __restrict__ given, const float* __restrict__ bias,
    int64_t tokens, int dim, int experts, float* __restrict__ out_logits,
    float* __restrict__ probs, float* __restrict__ weights,
    int64_t* __restrict__ indices, int32_t* __restrict__ positions,
    int32_t* __restrict__ block_counts) {
  __shared__ float part_s[4][kRouteTokensPerBlock][kMaxExperts + 1];
  __shared__ int ids_s[kRouteAssignPerBlock];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kRouteTokensPerBlock;

  if constexpr (!GIVEN_LOGITS) {
    const int64_t row = t0 + (lane & 15) < tokens ? t0 + (lane & 15) : tokens - 1;
    const int e0 = min(lane & 15, experts - 1);
    const int e1 = min(16 + (lane & 15), experts - 1);
    const int koff = (lane >> 4) * 8;
    const uint16_t* pa = x + row * dim + koff;
    const uint16_t* pb0 = wr + static_cast<int64_t>(e0) * dim + koff;
    const uint16_t* pb1 = wr + static_cast<int64_t>(e1) * dim + koff;
    const bool two = experts > 16;
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc1 = {0.f, 0.f, 0.f, 0.f};
    const int steps = dim / 32;
    for (int c0 = wave; c0 < steps; c0 += 4 * kStepsPerChunk) {
      bf16x8 a[kStepsPerChunk], b0[kStepsPerChunk], b1[kStepsPerChunk];
#pragma unroll
      for (int i = 0; i < kStepsPerChunk; ++i) {
        const int st = c0 + 4 * i;
        if (st < steps) {
          a[i] = load_bf16x8(pa + st * 32);
          b0[i] = load_bf16x8(pb0 + st * 32);
          if (two) b1[i] = load_bf16x8(pb1 + st * 32);
        }
      }
#pragma unroll
      for (int i = 0; i < kStepsPerChunk; ++i) {
        if (c0 + 4 * i < steps) {
          acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b0[i], acc0, 0, 0, 0);
          if (two) acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b1[i], acc1, 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      part_s[wave][4 * (lane >> 4) + r][lane & 15] = acc0[r];
      part_s[wave][4 * (lane >> 4) + r][16 + (lane & 15)] = acc1[r];
    }
  } else {
    for (int i = threadIdx.x; i < kRouteTokensPerBlock * experts; i += 256) {
      const int tl = i / experts;
      const int e = i - tl * experts;
      const int64_t t = t0 + tl;
      part_s[0][tl][e] = t < tokens ? given[t * experts + e] : 0.0f;
    }
  }
  __syncthreads();

  if (threadIdx.x < kRouteTokensPerBlock) {
    // Runtime loops over the experts keep this code small: it runs once per
    // workgroup, so its instruction fetch is not amortised.
    const int tl = threadIdx.x;
    const int64_t t = t0 + tl;
    auto logit = [&](int e) -> float {
      float v = part_s[0][tl][e];
      if constexpr (!GIVEN_LOGITS) v = ((v + part_s[1][tl][e]) + part_s[2][tl][e]) + part_s[3][tl][e];
      return v + (bias != nullptr ? bias[e] : 0.0f);
    };
    float best = logit(0), runner = logit(1);
    int first = 0, second = 1;
    if (runner > best) {
      const float tmp = best;
      best = runner;
      runner = tmp;
      first = 1;
      second = 0;
    }
#pragma unroll 1
    for (int e = 2; e < experts; ++e) {
      const float v = logit(e);
      if (v > best) {
        runner = best;
        second = first;
        best = v;
        first = e;
      } else if (v > runner) {
        runner = v;
        second = e;
      }
    }
    if (t < tokens) {
      const float e2 = __expf(runner - best);
      const float sel = 1.0f + e2;
      indices[2 * t] = first;
      indices[2 * t + 1] = second;
      weights[2 * t] = 1.0f / sel;
      weights[2 * t + 1] = e2 / sel;
      if (out_logits != nullptr) {
#pragma unroll 1
        for (int e = 0; e < experts; ++e) out_logits[t * experts + e] = logit(e);
      }
      if (probs != nullptr) {
        float denom = 0.0f;
#pragma unroll 1
        for (int e = 0; e < experts; ++e) denom += __expf(logit(e) - best);
        const float inv = 1.0f / denom;
#pragma unroll 1
        for (int e = 0; e < experts; ++e) probs[t * experts + e] = __expf(logit(e) - best) * inv;
      }
    }
    ids_s[2 * tl] = t < tokens ? first : -1;
    ids_s[2 * tl + 1] = t < tokens ? second : -1;
  }
  __syncthreads();
  block_rank(ids_s, static_cast<int64_t>(blockIdx.x) * kRouteAssignPerBlock, 2 * tokens, experts,
             positions, block_counts);
}

// Block-local ranks for top-2 indices supplied by the caller.
__global__ __launch_bounds__(256) void rank_indices_kernel(
    const int64_t* __restrict__ indices, int64_t tokens, int experts,
    int32_t* __restrict__ positions, int32_t* __restrict__ block_counts) {
  __shared__ int ids_s[kRouteAssignPerBlock];
  const int64_t a0 = static_cast<int64_t>(blockIdx.x) * kRouteAssignPerBlock;
  if (threadIdx.x < kRouteAssignPerBlock) {
    const int64_t a = a0 + threadIdx.x;
    const int64_t e = a < 2 * tokens ? indices[a] : -1;
    // Ids outside [0, experts) are excluded from the grouping (slot -1).
    ids_s[threadIdx.x] = (e >= 0 && e < experts) ? static_cast<int>(e) : -1;
    if (a < 2 * tokens && ids_s[threadIdx.x] < 0) positions[a] = -1;
  }
  __syncthreads();
  block_rank(ids_s, a0, 2 * tokens, experts, positions, block_counts);
}

constexpr int kGroupAssign = 256;                                  // assignments per group WG
constexpr int kBlocksPerGroup = kGroupAssign / kRouteAssignPerBlock;  // route blocks per group WG

// Global positions, counts, offsets, the [E, C] slot map and the
// expert-contiguous overflow list.  Workgroup g finalises assignments
// [256 g, 256 g + 256) (route blocks 8 g .. 8 g + 7) and fills the empty map
// slots [256 g, 256 g + 256).  Per-expert bases are exclusive sums of the
// route blocks' histograms, summed by 8 thread groups in a fixed order.
__global__ __launch_bounds__(256) void group_kernel(
    const int64_t* __restrict__ indices, int64_t tokens, int experts, int capacity,
    int n_route_blocks, const int32_t* __restrict__ block_counts,
    int32_t* __restrict__ positions, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ perm,
    int32_t* __restrict__ overflow) {
  __shared__ int before_s[8][kMaxExperts];
  __shared__ int total_s[8][kMaxExperts];
  __shared__ int base_s[kBlocksPerGroup][kMaxExperts];
  __shared__ int cnt_s[kMaxExperts];
  __shared__ int off_s[kMaxExperts + 1];
  __shared__ int ovf_s[kMaxExperts + 1];
  const int gb = blockIdx.x;
  const int tid = threadIdx.x;
  const int first_block = gb * kBlocksPerGroup;
  {
    const int e = tid & 31;
    const int lane_group = tid >> 5;
    int before = 0, total = 0;
    if (e < experts) {
      for (int i = lane_group; i < n_route_blocks; i += 8) {
        const int c = block_counts[static_cast<int64_t>(i) * experts + e];
        before += i < first_block ? c : 0;
        total += c;
      }
    }
    before_s[lane_group][e] = before;
    total_s[lane_group][e] = total;
  }
  __syncthreads();
  if (tid < experts) {
    int before = 0, total = 0;
    for (int g = 0; g < 8; ++g) {
      before += before_s[g][tid];
      total += total_s[g][tid];
    }
    cnt_s[tid] = total;
    for (int j = 0; j < kBlocksPerGroup; ++j) {
      base_s[j][tid] = before;
      const int rb = first_block + j;
      before += rb < n_route_blocks ? block_counts[static_cast<int64_t>(rb) * experts + tid] : 0;
    }
  }
  __syncthreads();
  if (tid == 0) {
    int o = 0, v = 0;
    for (int e = 0; e < experts; ++e) {
      off_s[e] = o;
      ovf_s[e] = v;
      o += cnt_s[e];
      v += max(0, cnt_s[e] - capacity);
    }
    off_s[experts] = o;
    ovf_s[experts] = v;
  }
  __syncthreads();
  const int64_t slot = static_cast<int64_t>(gb) * kGroupAssign + tid;
  if (slot < static_cast<int64_t>(experts) * capacity) {
    const int e = static_cast<int>(slot / capacity);
    const int s = static_cast<int>(slot - static_cast<int64_t>(e) * capacity);
    if (s >= cnt_s[e]) perm[slot] = -1;
  }
  const int64_t a = static_cast<int64_t>(gb) * kGroupAssign + tid;
  const int64_t e64 = a < 2 * tokens ? indices[a] : -1;
  if (e64 >= 0 && e64 < experts) {
    const int e = static_cast<int>(e64);
    const int p = positions[a] + base_s[tid / kRouteAssignPerBlock][e];
    positions[a] = p;
    if (p < capacity) perm[static_cast<int64_t>(e) * capacity + p] = static_cast<int32_t>(a);
    else overflow[ovf_s[e] + p - capacity] = static_cast<int32_t>(a);
  }
  if (gb == 0) {
    if (tid < experts) counts[tid] = cnt_s[tid];
    if (tid <= experts) {
      offsets[tid] = off_s[tid];
      offsets[experts + 1 + tid] = ovf_s[tid];
    }
  }
}

}  // namespace

hipError_t launch_route(const uint16_t* x, const uint16_t* router_w,
                        const float* given_logits, const float* bias,
                        int64_t tokens, int dim, int experts, float* out_logits,
                        float* probs, float* weights, int64_t* indices,
                        int32_t* positions, int32_t* block_counts, hipStream_t s) {
  if (tokens == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((tokens + kRouteTokensPerBlock - 1) / kRouteTokensPerBlock));
  if (given_logits != nullptr) {
    route_kernel<true><<<grid, 256, 0, s>>>(x, router_w, given_logits, bias, tokens, dim, experts,
                                            out_logits, probs, weights, indices, positions,
                                            block_counts);
  } else {
    route_kernel<false><<<grid, 256, 0, s>>>(x, router_w, given_logits, bias, tokens, dim,
                                             experts, out_logits, probs, weights, indices,
                                             positions, block_counts);
  }
  return hipGetLastError();
}

hipError_t launch_rank_indices(const int64_t* indices, int64_t tokens, int experts,
                               int32_t* positions, int32_t* block_counts, hipStream_t s) {
  if (tokens == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(route_blocks(tokens)));
  rank_indices_kernel<<<grid, 256, 0, s>>>(indices, tokens, experts, positions, block_counts);
  return hipGetLastError();
}

int route_blocks(int64_t tokens) {
  return static_cast<int>((tokens + kRouteTokensPerBlock - 1) / kRouteTokensPerBlock);
}

hipError_t launch_group(const int64_t* indices, int64_t tokens, int experts,
                        int capacity, const int32_t* block_counts,
                        int32_t* positions, int32_t* counts, int32_t* offsets,
                        int32_t* perm, int32_t* overflow, hipStream_t s) {
  const int nrb = route_blocks(tokens);
  const int64_t assign_blocks = (2 * tokens + kGroupAssign - 1) / kGroupAssign;
  const int64_t fill_blocks = (static_cast<int64_t>(experts) * capacity + kGroupAssign - 1) / kGroupAssign;
  const int grid = static_cast<int>(max(max(assign_blocks, fill_blocks), int64_t{1}));
  group_kernel<<<grid, 256, 0, s>>>(indices, tokens, experts, capacity, nrb, block_counts,
                                    positions, counts, offsets, perm, overflow);
  return hipGetLastError();
}

}  // namespace parrot
