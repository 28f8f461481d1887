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

constexpr int kTokensPerWave = 16;

__device__ __forceinline__ bf16x8 load_bf16x8(const uint16_t* p) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  return __builtin_bit_cast(bf16x8, v);
}

// Block-local stable rank of each of the block's 128 assignments and the
// block's per-expert histogram.  `ids` holds expert ids (-1 = padding).
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
  } else if (j - kRouteAssignPerBlock < experts) {
    const int e = j - kRouteAssignPerBlock;
    int count = 0;
    for (int i = 0; i < kRouteAssignPerBlock; ++i) count += ids[i] == e;
    block_counts[static_cast<int64_t>(blockIdx.x) * experts + e] = count;
  }
}

// One workgroup = 4 wavefronts x 16 tokens.  With GIVEN_LOGITS the fp32
// logits are read instead of projected (the "identical router logits" entry).
template <bool GIVEN_LOGITS>
__global__ __launch_bounds__(256) void route_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wr,
    const float* __restrict__ given, const float* __restrict__ bias,
    int64_t tokens, int dim, int experts, float* __restrict__ out_logits,
    float* __restrict__ probs, float* __restrict__ weights,
    int64_t* __restrict__ indices, int32_t* __restrict__ positions,
    int32_t* __restrict__ block_counts) {
  __shared__ float logit_s[4][kTokensPerWave][kMaxExperts + 1];
  __shared__ int ids_s[kRouteAssignPerBlock];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kRouteTokensPerBlock + wave * kTokensPerWave;

  if constexpr (!GIVEN_LOGITS) {
    // [16 tokens x dim] . [dim x 32 experts] on v_mfma_f32_16x16x32_bf16.
    // A/B fragments: lane l holds row/col (l & 15) and 8 consecutive k at
    // (l >> 4) * 8 within each 32-wide k step; C: col (l & 15), rows
    // 4 * (l >> 4) + r.
    const int64_t row = t0 + (lane & 15) < tokens ? t0 + (lane & 15) : tokens - 1;
    const int e0 = min(lane & 15, experts - 1);
    const int e1 = min(16 + (lane & 15), experts - 1);
    const uint16_t* pa = x + row * dim + (lane >> 4) * 8;
    const uint16_t* pb0 = wr + static_cast<int64_t>(e0) * dim + (lane >> 4) * 8;
    const uint16_t* pb1 = wr + static_cast<int64_t>(e1) * dim + (lane >> 4) * 8;
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc1 = {0.f, 0.f, 0.f, 0.f};
    if (experts > 16) {
      for (int k = 0; k < dim; k += 32) {
        const bf16x8 a = load_bf16x8(pa + k);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, load_bf16x8(pb0 + k), acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, load_bf16x8(pb1 + k), acc1, 0, 0, 0);
      }
    } else {
      for (int k = 0; k < dim; k += 32) {
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(load_bf16x8(pa + k), load_bf16x8(pb0 + k),
                                                       acc0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      logit_s[wave][4 * (lane >> 4) + r][lane & 15] = acc0[r];
      logit_s[wave][4 * (lane >> 4) + r][16 + (lane & 15)] = acc1[r];
    }
  } else {
    for (int i = lane; i < kTokensPerWave * experts; i += kWave) {
      const int tl = i / experts;
      const int e = i - tl * experts;
      const int64_t t = t0 + tl;
      logit_s[wave][tl][e] = t < tokens ? given[t * experts + e] : 0.0f;
    }
  }
  __syncthreads();

  if (lane < kTokensPerWave) {
    const int64_t t = t0 + lane;
    const float* lg = logit_s[wave][lane];
    float l[kMaxExperts];
#pragma unroll
    for (int e = 0; e < kMaxExperts; ++e) {
      if (e < experts) l[e] = lg[e] + (bias != nullptr ? bias[e] : 0.0f);
    }
    int first = 0, second = 1;
    if (l[1] > l[0]) { first = 1; second = 0; }
#pragma unroll
    for (int e = 2; e < kMaxExperts; ++e) {
      if (e < experts) {
        if (l[e] > l[first]) { second = first; first = e; }
        else if (l[e] > l[second]) { second = e; }
      }
    }
    if (t < tokens) {
      const float mx = l[first];
      const float e2 = __expf(l[second] - mx);
      const float sel = 1.0f + e2;
      indices[2 * t] = first;
      indices[2 * t + 1] = second;
      weights[2 * t] = 1.0f / sel;
      weights[2 * t + 1] = e2 / sel;
      if (out_logits != nullptr) {
        for (int e = 0; e < experts; ++e) out_logits[t * experts + e] = l[e];
      }
      if (probs != nullptr) {
        float denom = 0.0f;
#pragma unroll
        for (int e = 0; e < kMaxExperts; ++e)
          if (e < experts) denom += __expf(l[e] - mx);
        const float inv = 1.0f / denom;
#pragma unroll
        for (int e = 0; e < kMaxExperts; ++e)
          if (e < experts) probs[t * experts + e] = __expf(l[e] - mx) * inv;
      }
    }
    const int j = (wave * kTokensPerWave + lane) * 2;
    ids_s[j] = t < tokens ? first : -1;
    ids_s[j + 1] = t < tokens ? second : -1;
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

// Global positions, counts, offsets, the [E, C] slot map and the
// expert-contiguous overflow list.  Workgroup b finalises route block b and
// fills empty map slots [256 b, 256 b + 256).
__global__ __launch_bounds__(256) void group_kernel(
    const int64_t* __restrict__ indices, int64_t tokens, int experts, int capacity,
    int n_route_blocks, const int32_t* __restrict__ block_counts,
    int32_t* __restrict__ positions, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ perm,
    int32_t* __restrict__ overflow) {
  __shared__ int base_s[kMaxExperts];
  __shared__ int cnt_s[kMaxExperts];
  __shared__ int off_s[kMaxExperts + 1];
  __shared__ int ovf_s[kMaxExperts + 1];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  if (tid < experts) {
    int base = 0, total = 0;
    for (int i = 0; i < n_route_blocks; ++i) {
      const int c = block_counts[static_cast<int64_t>(i) * experts + tid];
      base += i < b ? c : 0;
      total += c;
    }
    base_s[tid] = base;
    cnt_s[tid] = total;
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
  const int64_t slot = static_cast<int64_t>(b) * 256 + tid;
  if (slot < static_cast<int64_t>(experts) * capacity) {
    const int e = static_cast<int>(slot / capacity);
    const int s = static_cast<int>(slot - static_cast<int64_t>(e) * capacity);
    if (s >= cnt_s[e]) perm[slot] = -1;
  }
  if (b < n_route_blocks && tid < kRouteAssignPerBlock) {
    const int64_t a = static_cast<int64_t>(b) * kRouteAssignPerBlock + tid;
    const int64_t e64 = a < 2 * tokens ? indices[a] : -1;
    if (e64 >= 0 && e64 < experts) {
      const int e = static_cast<int>(e64);
      const int p = positions[a] + base_s[e];
      positions[a] = p;
      if (p < capacity) perm[static_cast<int64_t>(e) * capacity + p] = static_cast<int32_t>(a);
      else overflow[ovf_s[e] + p - capacity] = static_cast<int32_t>(a);
    }
  }
  if (b == 0) {
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
  const dim3 grid(static_cast<unsigned>((2 * tokens + kRouteAssignPerBlock - 1) / kRouteAssignPerBlock));
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
  const int64_t fill_blocks = (static_cast<int64_t>(experts) * capacity + 255) / 256;
  const int grid = static_cast<int>(max(static_cast<int64_t>(max(nrb, 1)), fill_blocks));
  group_kernel<<<grid, 256, 0, s>>>(indices, tokens, experts, capacity, nrb, block_counts,
                                    positions, counts, offsets, perm, overflow);
  return hipGetLastError();
}

}  // namespace parrot
