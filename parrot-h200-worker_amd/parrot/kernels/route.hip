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

// ---- block-local ranks and histograms from wavefront ballots ---------------
// Each half-wavefront owns one route block of 32 assignments; lane l holds
// assignment id `id` (-1 = padding or an id outside [0, experts)).  For every
// expert, a ballot of the lanes holding it gives the stable rank (set bits
// below the lane, v_mbcnt) and the block's count (popcount).  Writes
// positions[a] for valid ids and block_counts[block, e] for blocks below
// n_blocks; with positions == NULL (top-2 only) there is nothing to rank.
__device__ __forceinline__ void rank_half_waves(int id, int64_t block, int64_t n_blocks,
                                                int64_t n_assign, int experts,
                                                int32_t* positions, int32_t* block_counts) {
  if (positions == nullptr) return;  // uniform: a top-2-only launch
  const int lane = threadIdx.x & (kWave - 1);
  const uint64_t half = lane < 32 ? 0x00000000ffffffffull : 0xffffffff00000000ull;
  int rank = 0, count = 0;
#pragma unroll 1
  for (int e = 0; e < experts; ++e) {
    const uint64_t m = __ballot(id == e) & half;
    const int below = static_cast<int>(__builtin_amdgcn_mbcnt_hi(
        static_cast<uint32_t>(m >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u)));
    if (id == e) rank = below;
    if ((lane & 31) == e) count = __popcll(m);
  }
  const int64_t a = block * kRouteAssignPerBlock + (lane & 31);
  if (id >= 0 && a < n_assign) positions[a] = rank;
  if ((lane & 31) < experts && block < n_blocks) block_counts[block * experts + (lane & 31)] = count;
}

// The block table row of one route block (kRouteBlockRowBytes bytes, the
// layout common.h states), written by wavefront 0 whose lanes 0-31 hold the
// block's assignment ids (-1 = padding) and lanes 32-63 none: a ballot per
// expert counts its ids (lane 32 + e keeps expert e's count), so lane l
// holds byte l of the row, and lanes 0-15 store it as 16 dwords.
__device__ __forceinline__ void write_block_row(int id, int64_t block, int experts,
                                                uint8_t* block_rows) {
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t byte = lane < 32 ? (id >= 0 ? static_cast<uint32_t>(id) : kNoExpert) : 0u;
#pragma unroll 1
  for (int e = 0; e < experts; ++e) {
    const uint64_t m = __ballot(id == e);
    if (lane == 32 + e) byte = static_cast<uint32_t>(__popcll(m));
  }
  const int b0 = 4 * (lane & 15);
  const uint32_t word = static_cast<uint32_t>(__shfl(static_cast<int>(byte), b0)) |
                        static_cast<uint32_t>(__shfl(static_cast<int>(byte), b0 + 1)) << 8 |
                        static_cast<uint32_t>(__shfl(static_cast<int>(byte), b0 + 2)) << 16 |
                        static_cast<uint32_t>(__shfl(static_cast<int>(byte), b0 + 3)) << 24;
  if (lane < 16)
    reinterpret_cast<uint32_t*>(block_rows + block * kRouteBlockRowBytes)[lane] = word;
}

// One workgroup routes one 16-token route block.  The router projection
// [16 x dim] . [dim x E] runs on v_mfma_f32_16x16x32_bf16 with the 32-wide
// k steps split round-robin over the 4 wavefronts; each wavefront issues the
// loads of up to 8 steps before its MFMAs, and the partial logits are summed
// in a fixed order through LDS.  Fragments: lane l holds row/col (l & 15)
// and the 8 k values at (l >> 4) * 8 of a step; C holds column (l & 15),
// rows 4 (l >> 4) + r.  With GIVEN_LOGITS the fp32 logits are read instead.
// Wavefront 0 then ranks the block (with `positions`) and writes its block
// table row (with `block_rows`).
// This split-K shape keeps short inputs (prefill, decode) latency-bound at
// the minimum.
template <bool GIVEN_LOGITS>
__global__ __launch_bounds__(256) void route_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wr,
    const float* __restrict__ given, const float* __restrict__ bias,
    int64_t tokens, int dim, int experts, float* __restrict__ out_logits,
    float* __restrict__ probs, float* __restrict__ weights,
    int64_t* __restrict__ indices, int32_t* __restrict__ positions,
    int32_t* __restrict__ block_counts, uint8_t* __restrict__ block_rows) {
  // The kernel arguments in one batch of scalar loads before any use.
  asm volatile("" ::"s"(x), "s"(wr), "s"(given), "s"(bias), "s"(tokens), "s"(dim), "s"(experts),
               "s"(out_logits), "s"(probs), "s"(weights), "s"(indices), "s"(positions),
               "s"(block_counts), "s"(block_rows));
  __builtin_amdgcn_sched_barrier(0);
  __shared__ float part_s[4][kRouteTokensPerBlock][kMaxExperts + 1];
  __shared__ int ids_s[kRouteAssignPerBlock];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kRouteTokensPerBlock;
  // This thread's two bias entries for the selection below (experts j and
  // j + 16 of its DPP row).
  const int jb = threadIdx.x & 15;
  float bias0 = 0.0f, bias1 = 0.0f;
  auto load_bias = [&]() {
    bias0 = bias[min(jb, experts - 1)];
    bias1 = bias[min(jb + 16, experts - 1)];
  };

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
    if (bias != nullptr) load_bias();  // in flight across the partial sums' barrier
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      part_s[wave][4 * (lane >> 4) + r][lane & 15] = acc0[r];
      part_s[wave][4 * (lane >> 4) + r][16 + (lane & 15)] = acc1[r];
    }
  } else {
    if (bias != nullptr) load_bias();
    for (int i = threadIdx.x; i < kRouteTokensPerBlock * experts; i += 256) {
      const int tl = i / experts;
      const int e = i - tl * experts;
      const int64_t t = t0 + tl;
      part_s[0][tl][e] = t < tokens ? given[t * experts + e] : 0.0f;
    }
  }
  __syncthreads();

  {
    // Token tl = tid / 16 on DPP row tid / 16; lane j holds experts j, j + 16.
    const int tl = threadIdx.x >> 4;
    const int j = threadIdx.x & 15;
    auto logit = [&](int e, float b) -> float {
      float v = part_s[0][tl][e];
      if constexpr (!GIVEN_LOGITS) v = ((v + part_s[1][tl][e]) + part_s[2][tl][e]) + part_s[3][tl][e];
      return v + b;
    };
    const float l0 = j < experts ? logit(j, bias0) : 0.0f;
    const float l1 = j + 16 < experts ? logit(j + 16, bias1) : 0.0f;
    select_top2(l0, l1, experts, t0 + tl, t0 + tl < tokens, out_logits, probs, weights, indices,
                &ids_s[2 * tl]);
  }
  // Uniform: a top-2-only launch neither ranks nor tabulates the block.
  if (positions == nullptr && block_rows == nullptr) return;
  __syncthreads();
  // Wavefront 0 ranks the block in lanes 0-31; lanes 32-63 carry no
  // assignments and name no block (index gridDim.x is past the last).
  if (threadIdx.x < kWave) {
    const bool mine = threadIdx.x < kRouteAssignPerBlock;
    const int id = mine ? ids_s[threadIdx.x] : -1;
    rank_half_waves(id, mine ? blockIdx.x : gridDim.x, gridDim.x, 2 * tokens, experts, positions,
                    block_counts);
    if (block_rows != nullptr) write_block_row(id, blockIdx.x, experts, block_rows);
  }
}

// Long inputs: one workgroup routes 4 route blocks (64 tokens); wavefront w
// computes the logits of route block 4 blockIdx.x + w over the full K
// (bit-identical to route_kernel's split-K sum), STEPS
// k steps of loads in flight at a time (TWO: a second 16-expert column tile,
// for E > 16).  The router weights (16 or 32 rows, rows past E repeating row
// E - 1) are first staged in LDS with a row stride of dim + 8 elements, so
// the k-step loads that go to memory are the token rows alone.  Same block-local ranks and histograms as
// route_kernel, so the group step is shared.
template <bool TWO, int STEPS>
__global__ __launch_bounds__(256) void route_wide_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wr,
    const float* __restrict__ bias, int64_t tokens, int dim, int experts,
    float* __restrict__ out_logits, float* __restrict__ probs, float* __restrict__ weights,
    int64_t* __restrict__ indices, int32_t* __restrict__ positions,
    int32_t* __restrict__ block_counts, int n_blocks) {
  // The kernel arguments in one batch of scalar loads before any use.
  asm volatile("" ::"s"(x), "s"(wr), "s"(bias), "s"(tokens), "s"(dim), "s"(experts),
               "s"(out_logits), "s"(probs), "s"(weights), "s"(indices), "s"(positions),
               "s"(block_counts), "s"(n_blocks));
  __builtin_amdgcn_sched_barrier(0);
  constexpr int kTokens = 4 * kRouteTokensPerBlock;
  __shared__ float logit_s[kTokens][kMaxExperts + 1];
  __shared__ int ids_s[4 * kRouteAssignPerBlock];
  extern __shared__ __attribute__((aligned(16))) uint16_t wr_s[];  // [16 or 32][dim + 8]
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kTokens;
  {
    const int64_t r = t0 + wave * 16 + (lane & 15);
    const int64_t row = r < tokens ? r : tokens - 1;
    const int koff = (lane >> 4) * 8;
    const uint16_t* pa = x + row * dim + koff;
    {
      const int rs = dim + 8;  // LDS row stride, elements
      const int cpr = dim / 8;  // 16-byte chunks per row
      for (int i = threadIdx.x; i < (TWO ? 32 : 16) * cpr; i += 256) {
        const int r = i / cpr;
        const int c = i - r * cpr;
        *reinterpret_cast<uint4*>(wr_s + r * rs + c * 8) = *reinterpret_cast<const uint4*>(
            wr + static_cast<int64_t>(min(r, experts - 1)) * dim + c * 8);
      }
      __syncthreads();
    }
    const uint16_t* lb0 = wr_s + (lane & 15) * (dim + 8) + koff;
    const uint16_t* lb1 = wr_s + (16 + (lane & 15)) * (dim + 8) + koff;
    // One accumulator chain per k-step residue st % 4, summed as
    // ((c0 + c1) + c2) + c3: the exact arithmetic of route_kernel, whose
    // wavefront w accumulates the steps st = w (mod 4) in ascending order, so
    // a token's logits (and its top-2) do not depend on the batch size.
    static_assert(STEPS % 4 == 0, "a chunk must keep st % 4 == i % 4");
    f32x4 acc0[4], acc1[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      acc0[c] = f32x4{0.f, 0.f, 0.f, 0.f};
      acc1[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const int steps = dim / 32;
    for (int c0 = 0; c0 < steps; c0 += STEPS) {
      bf16x8 a[STEPS], b0[STEPS], b1[STEPS];
#pragma unroll
      for (int i = 0; i < STEPS; ++i) {
        const int st = min(c0 + i, steps - 1);  // unconditional loads, clamped
        a[i] = load_bf16x8(pa + st * 32);
        b0[i] = load_bf16x8(lb0 + st * 32);
        if constexpr (TWO) b1[i] = load_bf16x8(lb1 + st * 32);
      }
#pragma unroll
      for (int i = 0; i < STEPS; ++i) {
        if (c0 + i < steps) {
          acc0[i % 4] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b0[i], acc0[i % 4], 0, 0, 0);
          if constexpr (TWO)
            acc1[i % 4] =
                __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b1[i], acc1[i % 4], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      logit_s[wave * 16 + 4 * (lane >> 4) + r][lane & 15] =
          ((acc0[0][r] + acc0[1][r]) + acc0[2][r]) + acc0[3][r];
      logit_s[wave * 16 + 4 * (lane >> 4) + r][16 + (lane & 15)] =
          ((acc1[0][r] + acc1[1][r]) + acc1[2][r]) + acc1[3][r];
    }
  }
  __syncthreads();
  // Four passes of 16 tokens, one per DPP row.
#pragma unroll 1
  for (int pass = 0; pass < 4; ++pass) {
    const int tl = pass * 16 + (threadIdx.x >> 4);
    const int j = threadIdx.x & 15;
    const float b0 = bias != nullptr && j < experts ? bias[j] : 0.0f;
    const float b1 = bias != nullptr && j + 16 < experts ? bias[j + 16] : 0.0f;
    select_top2(logit_s[tl][j] + b0, logit_s[tl][16 + j] + b1, experts, t0 + tl,
                t0 + tl < tokens, out_logits, probs, weights, indices, &ids_s[2 * tl]);
  }
  __syncthreads();
  // Wavefronts 0 and 1 rank route blocks 4 bx + 2 w (lanes 0-31) and
  // 4 bx + 2 w + 1 (lanes 32-63).
  if (threadIdx.x < 2 * kWave)
    rank_half_waves(ids_s[threadIdx.x], static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 5),
                    n_blocks, 2 * tokens, experts, positions, block_counts);
}

// Block-local ranks for top-2 indices supplied by the caller.
__global__ __launch_bounds__(64) void rank_indices_kernel(
    const int64_t* __restrict__ indices, int64_t tokens, int experts,
    int32_t* __restrict__ positions, int32_t* __restrict__ block_counts, int n_blocks) {
  // The kernel arguments in one batch of scalar loads before any use.
  asm volatile("" ::"s"(indices), "s"(tokens), "s"(experts), "s"(positions), "s"(block_counts),
               "s"(n_blocks));
  __builtin_amdgcn_sched_barrier(0);
  // Lanes 0-31 hold route block 2 bx, lanes 32-63 route block 2 bx + 1.
  const int64_t a = static_cast<int64_t>(blockIdx.x) * 2 * kRouteAssignPerBlock + threadIdx.x;
  const int64_t e = a < 2 * tokens ? indices[a] : -1;
  // Ids outside [0, experts) are excluded from the grouping (slot -1).
  const int id = (e >= 0 && e < experts) ? static_cast<int>(e) : -1;
  if (a < 2 * tokens && id < 0) positions[a] = -1;
  rank_half_waves(id, static_cast<int64_t>(blockIdx.x) * 2 + (threadIdx.x >> 5), n_blocks,
                  2 * tokens, experts, positions, block_counts);
}

// Adds rows lo + g, lo + g + n_groups, ... below `hi` of column e of the
// int32 table [rows, experts] to `all`, and those below `split` also to
// `below`; kColumnLoads independent loads per round trip (g = this thread's
// lane group), clamped to row hi - 1 past the end.
constexpr int kColumnLoads = 16;

__device__ __forceinline__ void sum_column(const int32_t* table, int experts, int e, int g,
                                           int n_groups, int lo, int hi, int split, int& below,
                                           int& all) {
  for (int i0 = lo + g; i0 < hi; i0 += kColumnLoads * n_groups) {
    int v[kColumnLoads];
#pragma unroll
    for (int k = 0; k < kColumnLoads; ++k)
      v[k] = table[static_cast<int64_t>(min(i0 + k * n_groups, hi - 1)) * experts + e];
#pragma unroll
    for (int k = 0; k < kColumnLoads; ++k) {
      const int i = i0 + k * n_groups;
      if (i < hi) {
        all += v[k];
        below += i < split ? v[k] : 0;
      }
    }
  }
}

// Lane groups of a 256-thread workgroup for per-expert column sums: 16
// groups of 16 experts (E <= 16) or 8 groups of 32.
__device__ __forceinline__ int lane_groups(int experts) { return experts <= 16 ? 16 : 8; }

// First level of the histogram scan for long inputs: chunk c's per-expert
// totals over route blocks [256 c, 256 c + 256), summed by lane groups in a
// fixed order.
__global__ __launch_bounds__(256) void chunk_sum_kernel(const int32_t* __restrict__ block_counts,
                                                        int n_blocks, int experts,
                                                        int32_t* __restrict__ chunk_totals) {
  // The kernel arguments in one batch of scalar loads before any use.
  asm volatile("" ::"s"(block_counts), "s"(n_blocks), "s"(experts), "s"(chunk_totals));
  __builtin_amdgcn_sched_barrier(0);
  __shared__ int part_s[16][kMaxExperts];
  const int n_groups = lane_groups(experts);
  const int e_stride = 256 / n_groups;
  const int g = threadIdx.x / e_stride;
  const int e = threadIdx.x - g * e_stride;
  const int first = blockIdx.x * kScanChunk;
  const int last = min(first + kScanChunk, n_blocks);
  int sum = 0, unused = 0;
  if (e < experts) sum_column(block_counts, experts, e, g, n_groups, first, last, last, unused, sum);
  part_s[g][e] = sum;
  __syncthreads();
  if (threadIdx.x < experts) {
    int total = 0;
    for (int k = 0; k < n_groups; ++k) total += part_s[k][threadIdx.x];
    chunk_totals[static_cast<int64_t>(blockIdx.x) * experts + threadIdx.x] = total;
  }
}

constexpr int kGroupAssign = 256;                                  // assignments per group WG
constexpr int kBlocksPerGroup = kGroupAssign / kRouteAssignPerBlock;  // route blocks per group WG

// Global positions, counts, offsets, the [E, C] slot map and the
// expert-contiguous overflow list.  Workgroup g finalises assignments
// [256 g, 256 g + 256) (route blocks 8 g .. 8 g + 7) and fills the empty map
// slots [256 g, 256 g + 256).  Per-expert bases are exclusive sums of the
// route blocks' histograms, summed by lane groups in a fixed order --
// directly over every route block for short inputs, or over chunk totals
// plus at most one chunk of route blocks when `chunk_totals` is given.
__global__ __launch_bounds__(256) void group_kernel(
    const int64_t* __restrict__ indices, int64_t tokens, int experts, int capacity,
    int n_route_blocks, const int32_t* __restrict__ block_counts,
    const int32_t* __restrict__ chunk_totals, int n_chunks,
    int32_t* __restrict__ positions, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ perm,
    int32_t* __restrict__ overflow) {
  // The kernel arguments in one batch of scalar loads before any use.
  asm volatile("" ::"s"(indices), "s"(tokens), "s"(experts), "s"(capacity), "s"(n_route_blocks),
               "s"(block_counts), "s"(chunk_totals), "s"(n_chunks), "s"(positions), "s"(counts),
               "s"(offsets), "s"(perm), "s"(overflow));
  __builtin_amdgcn_sched_barrier(0);
  __shared__ int before_s[16][kMaxExperts];
  __shared__ int total_s[16][kMaxExperts];
  __shared__ int base_s[kBlocksPerGroup][kMaxExperts];
  __shared__ int cnt_s[kMaxExperts];
  __shared__ int off_s[kMaxExperts + 1];
  __shared__ int ovf_s[kMaxExperts + 1];
  const int gb = blockIdx.x;
  const int tid = threadIdx.x;
  const int first_block = gb * kBlocksPerGroup;
  const int n_groups = lane_groups(experts);
  const int e_stride = 256 / n_groups;
  const int lane_group = tid / e_stride;
  {
    const int e = tid - lane_group * e_stride;
    int before = 0, total = 0;
    if (e < experts) {
      if (chunk_totals == nullptr) {
        sum_column(block_counts, experts, e, lane_group, n_groups, 0, n_route_blocks, first_block,
                   before, total);
      } else {
        // Two levels: whole chunks before this workgroup's chunk, then the
        // route blocks of its own chunk before `first_block`.
        const int c0 = first_block / kScanChunk;
        sum_column(chunk_totals, experts, e, lane_group, n_groups, 0, n_chunks, c0, before, total);
        const int hi = min(first_block, n_route_blocks);
        int in_chunk = 0;
        sum_column(block_counts, experts, e, lane_group, n_groups, c0 * kScanChunk, hi, hi, before,
                   in_chunk);
      }
    }
    before_s[lane_group][e] = before;
    total_s[lane_group][e] = total;
  }
  __syncthreads();
  if (tid < experts) {
    int before = 0, total = 0;
    for (int g = 0; g < n_groups; ++g) {
      before += before_s[g][tid];
      total += total_s[g][tid];
    }
    cnt_s[tid] = total;
    if (n_route_blocks > 0) {
      int bc[kBlocksPerGroup];
#pragma unroll
      for (int j = 0; j < kBlocksPerGroup; ++j)
        bc[j] = block_counts[static_cast<int64_t>(min(first_block + j, n_route_blocks - 1)) * experts + tid];
#pragma unroll
      for (int j = 0; j < kBlocksPerGroup; ++j) {
        base_s[j][tid] = before;
        before += first_block + j < n_route_blocks ? bc[j] : 0;
      }
    }
  }
  __syncthreads();
  // Exclusive prefixes of the counts and of the overflow counts: thread e
  // sums entries [0, e) itself (independent LDS reads, no serial chain).
  if (tid <= experts) {
    int o = 0, v = 0;
#pragma unroll
    for (int e = 0; e < kMaxExperts; ++e) {
      const int c = e < tid ? cnt_s[e] : 0;
      o += c;
      v += max(0, c - capacity);
    }
    off_s[tid] = o;
    ovf_s[tid] = v;
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

// Long inputs: persistent wavefronts, each routing 16-token route blocks
// gw, gw + (all wavefronts), ... on its own (no barrier: its LDS is its own).
// A block's rows are read a third of a row (256 k values) at a time, as two
// 512-byte contiguous runs per load instruction (rows 2p and 2p + 1 in
// lanes 0-31 and 32-63), instead of the MFMA fragment pattern (16 rows x 64
// bytes per instruction, which route_kernel and route_wide_kernel use and
// which held them to ~3.5 TB/s at 64K tokens).  The chunks go to LDS (the
// 16-byte chunk c of row r at r * 512 + ((c ^ r) << 4): conflict-free writes
// and fragment reads) and the A fragments are read back from there; the
// router's B fragments for every k step stay in registers (the router is the
// same for every block).  As soon as a third is in LDS, the loads of the
// next third (or of the next block's first) are issued into the same
// registers, so the memory stream runs through the MFMAs, the top-2, the
// ranking and the stores.  (Two thirds in flight need a second register set,
// which only fits with B read from LDS as well: 27.3 against 23.5 us at 64K
// tokens.)  Arithmetic: route_kernel's (four accumulator chains by k-step
// residue, summed ((c0 + c1) + c2) + c3 over the same fragments):
// bit-identical.  dim == 32 kStreamSteps (the model's 768), E <= 16 and
// tokens * dim * 2 < 2^31 (32-bit row offsets).
constexpr int kStreamSteps = 24;
constexpr int kStreamThirds = 3;                 // k chunks of 8 steps
constexpr int kStreamThirdBytes = 512;           // per row
constexpr int kStreamWavesPerGroup = 4;
constexpr int kStreamGroupsPerCu = 2;            // the registers leave two workgroups per CU

struct StreamWaveLds {
  uint8_t rows[kRouteTokensPerBlock * kStreamThirdBytes];
  float logits[kRouteTokensPerBlock][kRouteTokensPerBlock + 1];
  int ids[kRouteAssignPerBlock];
};

__global__ __launch_bounds__(64 * kStreamWavesPerGroup) void route_stream_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wr,
    const float* __restrict__ bias, int64_t tokens, int dim, int experts,
    float* __restrict__ out_logits, float* __restrict__ probs, float* __restrict__ weights,
    int64_t* __restrict__ indices, int32_t* __restrict__ positions,
    int32_t* __restrict__ block_counts, int n_blocks) {
  asm volatile("" ::"s"(x), "s"(wr), "s"(bias), "s"(tokens), "s"(dim), "s"(experts),
               "s"(out_logits), "s"(probs), "s"(weights), "s"(indices), "s"(positions),
               "s"(block_counts), "s"(n_blocks));
  __builtin_amdgcn_sched_barrier(0);
  __shared__ StreamWaveLds lds[kStreamWavesPerGroup];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  StreamWaveLds& L = lds[wave];
  const int stride = __builtin_amdgcn_readfirstlane(gridDim.x * kStreamWavesPerGroup);
  int rb = __builtin_amdgcn_readfirstlane(blockIdx.x * kStreamWavesPerGroup + wave);
  if (rb >= n_blocks) return;  // uniform per wavefront; no barrier follows
  const int half = lane >> 5, cl = lane & 31;
  const int j = lane & 15, h = lane >> 4;
  const int last_row = static_cast<int>(tokens) - 1;
  // Load p of a third reads row 2p + half of its block (rows past the input
  // read the last row), 16-byte chunk 32 third + cl.
  auto chunk = [&](int blk, int p, int third) {
    const int row = min(blk * kRouteTokensPerBlock + half + 2 * p, last_row);
    return *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(x) +
                                           (row * dim * 2 + ((32 * third + cl) << 4)));
  };
#define PARROT_LOAD_THIRD(BLK, T)                                                      \
  a0 = chunk(BLK, 0, T); a1 = chunk(BLK, 1, T); a2 = chunk(BLK, 2, T);                 \
  a3 = chunk(BLK, 3, T); a4 = chunk(BLK, 4, T); a5 = chunk(BLK, 5, T);                 \
  a6 = chunk(BLK, 6, T); a7 = chunk(BLK, 7, T);
  auto put = [&](int p, uint4 v) {
    const int r = 2 * p + half;
    *reinterpret_cast<uint4*>(L.rows + r * kStreamThirdBytes + ((cl ^ r) << 4)) = v;
  };
  uint4 a0, a1, a2, a3, a4, a5, a6, a7;
  PARROT_LOAD_THIRD(rb, 0)
  bf16x8 b[kStreamSteps];
  {
    const uint16_t* pb = wr + static_cast<int64_t>(min(j, experts - 1)) * dim + h * 8;
#pragma unroll
    for (int i = 0; i < kStreamSteps; ++i) b[i] = load_bf16x8(pb + i * 32);
  }
  const float bias0 = bias != nullptr && j < experts ? bias[j] : 0.0f;
  for (;;) {
    const int next = rb + stride;
    f32x4 acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < kStreamThirds; ++t) {
      put(0, a0); put(1, a1); put(2, a2); put(3, a3);
      put(4, a4); put(5, a5); put(6, a6); put(7, a7);
      // The next third, or the next block's first (this block's again past
      // the last: a repeat that is never used).
      if (t + 1 < kStreamThirds) {
        PARROT_LOAD_THIRD(rb, t + 1)
      } else {
        PARROT_LOAD_THIRD(min(next, n_blocks - 1), 0)
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int st = 8 * t + i;
        const int c = 4 * i + h;  // this lane's A fragment: row j, chunk 4 st + lane / 16
        const uint4 av = *reinterpret_cast<const uint4*>(L.rows + j * kStreamThirdBytes +
                                                         ((c ^ j) << 4));
        acc[st % 4] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av),
                                                              b[st], acc[st % 4], 0, 0, 0);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
      L.logits[4 * h + r][j] = ((acc[0][r] + acc[1][r]) + acc[2][r]) + acc[3][r];
    const int64_t t0 = static_cast<int64_t>(rb) * kRouteTokensPerBlock;
#pragma unroll 1
    for (int pass = 0; pass < 4; ++pass) {
      const int tl = pass * 4 + h;
      select_top2(L.logits[tl][j] + bias0, 0.0f, experts, t0 + tl, t0 + tl < tokens, out_logits,
                  probs, weights, indices, &L.ids[2 * tl]);
    }
    rank_half_waves(lane < 32 ? L.ids[lane] : -1, lane < 32 ? rb : n_blocks, n_blocks,
                    2 * tokens, experts, positions, block_counts);
    rb = next;
    if (rb >= n_blocks) break;
  }
#undef PARROT_LOAD_THIRD
}

}  // namespace

// The wide (64-token) route kernel takes over once its workgroups alone
// cover every CU; below that the split-K kernel's shorter chain wins.
constexpr int64_t kWideRouteTokens = 32768;  // the two shapes tie at 32K tokens
constexpr int kWideRouteLdsBytes = 65536;     // the wide kernel's staged router weights
constexpr int64_t kStreamRouteTokens = 32768;  // route_stream_kernel from here (E <= 16, dim 768;
                                              // at 16K tokens the split-K shape is ahead)

// Compute units of the current device (the persistent route grid's size):
// a host-side property query, no stream work, so graph capture may call it.
static hipError_t device_cus(int* cus) {
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
  return hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev);
}

hipError_t launch_route(const uint16_t* x, const uint16_t* router_w,
                        const float* given_logits, const float* bias,
                        int64_t tokens, int dim, int experts, float* out_logits,
                        float* probs, float* weights, int64_t* indices,
                        int32_t* positions, int32_t* block_counts, uint8_t* block_rows,
                        hipStream_t s) {
  if (tokens == 0) return hipSuccess;
  if (block_rows != nullptr && !route_block_rows_supported(tokens)) return hipErrorInvalidValue;
  const int nrb = route_blocks(tokens);
  if (given_logits != nullptr) {
    route_kernel<true><<<nrb, 256, 0, s>>>(x, router_w, given_logits, bias, tokens, dim, experts,
                                           out_logits, probs, weights, indices, positions,
                                           block_counts, block_rows);
  } else if (tokens >= kStreamRouteTokens && block_rows == nullptr &&
             dim == 32 * kStreamSteps && experts <= 16 && tokens * dim * 2 < (int64_t{1} << 31)) {
    // One workgroup per CU slot the kernel's registers leave.
    int cus = 0;
    if (hipError_t e = device_cus(&cus); e != hipSuccess) return e;
    const int groups = (nrb + kStreamWavesPerGroup - 1) / kStreamWavesPerGroup;
    const int grid = min(groups, kStreamGroupsPerCu * cus);
    route_stream_kernel<<<grid, 64 * kStreamWavesPerGroup, 0, s>>>(
        x, router_w, bias, tokens, dim, experts, out_logits, probs, weights, indices, positions,
        block_counts, nrb);
  } else if (tokens >= kWideRouteTokens &&
             (experts > 16 ? 32 : 16) * (dim + 8) * 2 <= kWideRouteLdsBytes) {
    const bool two = experts > 16;
    auto* kernel = two ? route_wide_kernel<true, 8> : route_wide_kernel<false, 12>;
    const size_t lds = static_cast<size_t>(two ? 32 : 16) * (dim + 8) * 2;
    kernel<<<(nrb + 3) / 4, 256, lds, s>>>(x, router_w, bias, tokens, dim, experts, out_logits,
                                           probs, weights, indices, positions, block_counts, nrb);
  } else {
    route_kernel<false><<<nrb, 256, 0, s>>>(x, router_w, given_logits, bias, tokens, dim,
                                            experts, out_logits, probs, weights, indices,
                                            positions, block_counts, block_rows);
  }
  return hipGetLastError();
}

bool route_block_rows_supported(int64_t tokens) { return tokens < kWideRouteTokens; }

hipError_t launch_rank_indices(const int64_t* indices, int64_t tokens, int experts,
                               int32_t* positions, int32_t* block_counts, hipStream_t s) {
  if (tokens == 0) return hipSuccess;
  const int nrb = route_blocks(tokens);
  rank_indices_kernel<<<(nrb + 1) / 2, 64, 0, s>>>(indices, tokens, experts, positions,
                                                   block_counts, nrb);
  return hipGetLastError();
}

int route_blocks(int64_t tokens) {
  return static_cast<int>((tokens + kRouteTokensPerBlock - 1) / kRouteTokensPerBlock);
}

int route_chunks(int64_t tokens) {
  const int nrb = route_blocks(tokens);
  return nrb > kScanChunk ? (nrb + kScanChunk - 1) / kScanChunk : 0;
}

hipError_t launch_group(const int64_t* indices, int64_t tokens, int experts,
                        int capacity, const int32_t* block_counts, int32_t* chunk_totals,
                        int32_t* positions, int32_t* counts, int32_t* offsets,
                        int32_t* perm, int32_t* overflow, hipStream_t s) {
  const int nrb = route_blocks(tokens);
  const int n_chunks = route_chunks(tokens);
  if (n_chunks > 0) {
    chunk_sum_kernel<<<n_chunks, 256, 0, s>>>(block_counts, nrb, experts, chunk_totals);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  }
  const int64_t assign_blocks = (2 * tokens + kGroupAssign - 1) / kGroupAssign;
  const int64_t fill_blocks = (static_cast<int64_t>(experts) * capacity + kGroupAssign - 1) / kGroupAssign;
  const int grid = static_cast<int>(max(max(assign_blocks, fill_blocks), int64_t{1}));
  group_kernel<<<grid, 256, 0, s>>>(indices, tokens, experts, capacity, nrb, block_counts,
                                    n_chunks > 0 ? chunk_totals : nullptr, n_chunks,
                                    positions, counts, offsets, perm, overflow);
  return hipGetLastError();
}

}  // namespace parrot
