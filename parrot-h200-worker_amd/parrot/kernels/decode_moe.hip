// Fused MoE layer for decode steps: T <= 16 tokens in two kernels.
//
// Reference semantics are those of the grouped path (route_kernel, the
// grouped SwiGLU GEMMs, combine_kernel): parrot/model.py:520-551 and
// 571-607 -- logits = x Wr^T (+ bias) in fp32, top-2 with ties to the lower
// expert index, weights renormalised over the two, h = bf16(silu(x Wg^T) *
// (x Wu^T)) per routed assignment and for the shared expert, out =
// bf16(shared + w0 y0 + w1 y1) (+ addend with a second rounding).  Every
// assignment is computed, so capacity and overflow change nothing here.  The
// reference's Apple decode fusion is moe_decode_lanes_bf16 /
// moe_sum_decode_lanes_bf16 (parrot/kernels/moe_bf16.metal:894-1024,
// 1185-1201, driven by parrot/metal_moe.py:182-221).
//
// At decode sizes the layer is a weight stream of ~2 x 2.4 MB per token plus
// the shared expert, and launch latency dominates; the grouped path spends 5
// launches (route, group, gate/up, down, combine).  Here:
//   decode_up_kernel   grid (max(H, Hs) / SW slices, 3T slots): slot 2t + k
//       is token t's k-th routed expert, slot 2T + t token t's shared expert.
//       A routed workgroup recomputes its token's router logits and top-2
//       (every workgroup of a token does the same arithmetic in the same
//       order, so they agree), then one SW-column slice of SwiGLU (SW = 8
//       at one or two tokens, else 16).  Given the MoE input's depth sources
//       instead of the input, every workgroup first mixes and normalises its
//       token's row itself (depth_mix_core.h, the depth-mix kernel's
//       arithmetic), which saves that kernel's launch.
//   decode_down_kernel grid (dim / 16 slices, T): 16 output columns of one
//       token: both weighted routed rows and the shared row, summed in the
//       combine kernel's order, with the addend folded in.
// Weights are the packed fragment-ordered matrices of the grouped path (1 KB
// blocks of 16 rows x 32 k; lane l's 16 bytes are row l % 16, k 8 (l / 16)
// .. +8), so lane l of wavefront w reads 16 contiguous bytes of k step
// s = w, w + 4, ...; partial sums over (k chunk, wavefront) are added in a
// fixed order through LDS.
#include "depth_mix_core.h"

namespace parrot {

namespace {

constexpr int kDecodeMaxTokens = 16;

// decode_up_kernel's LDS row (the slot's token row, dim bf16) is dynamic.
__host__ __device__ __forceinline__ size_t decode_up_lds_bytes(int dim) {
  return static_cast<size_t>((dim + 7) / 8 * 8) * sizeof(uint16_t);
}

// Router k steps per wavefront whose weight fragments are loaded at kernel
// entry (dim 768: all of them); the rest are loaded in the chain itself.
constexpr int kRouteStepSlots = 6;

__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float(uint32_t(v) << 16); }

// Dot product of 8 bf16 pairs in fp32: four v_dot2c_f32_bf16, each adding two
// exact bf16 products to the running sum (4 instructions where unpacking the
// halves and fusing multiply-adds takes 24; decode steps 1-2 % faster on
// MI355X).  Its rounding is neither the exactly rounded sum nor two chained
// FMAs: on 67M random finite inputs it matched the first in 88.7 % and the
// second in 87.3 % of cases, within one fp32 rounding of both.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}
__device__ __forceinline__ float dot8(uint4 a, uint4 b) {
  return dot2(a.w, b.w, dot2(a.z, b.z, dot2(a.y, b.y, dot2(a.x, b.x, 0.0f))));
}

// One 16-byte chunk of an LDS array, read as LDS (ds_read_b128) rather
// than through a generic pointer (flat_load, which also waits on the vector
// memory counter).
typedef uint32_t lds_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 lds_chunk(const uint16_t* base, int chunk) {
  const lds_u32x4 v = ((const __attribute__((address_space(3))) lds_u32x4*)base)[chunk];
  return make_uint4(v.x, v.y, v.z, v.w);
}

// The slot's router logits and top-2, with route_kernel's arithmetic to the
// bit: wavefront c runs the v_mfma_f32_16x16x32_bf16 chain over the 32-wide
// k steps st = c, c + 4, ... (the token row from LDS in A row 0, rows 1-15
// zero; an MFMA output element depends only on its own row and column), one
// 16-expert column tile per ROUTE; the chains are summed ((c0 + c1) + c2) +
// c3, plus the bias, then top-2 with ties to the lower index and weights
// 1 / (1 + e), e / (1 + e), e = exp(l2 - l1).  rb: the fragments of the
// first kRouteStepSlots steps, loaded at kernel entry; pb: the lane's router
// row (column l % 16 of tile h) at its k offset, for the later steps.
template <int ROUTE>
__device__ __forceinline__ void route_slot(const uint16_t* x_lds,
                                           const bf16x8 (&rb)[kRouteStepSlots][ROUTE],
                                           const uint16_t* const (&pb)[ROUTE], const float* bias,
                                           int dim, int experts, float (*chain_s)[kMaxExperts],
                                           int* sel, float* sel_w) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int steps = dim / 32;
  const bool row0 = (lane & 15) == 0;
  auto a_frag = [&](int st) {
    const uint4 av = row0 ? lds_chunk(x_lds, st * 4 + (lane >> 4)) : make_uint4(0u, 0u, 0u, 0u);
    return __builtin_bit_cast(bf16x8, av);
  };
  f32x4 acc[ROUTE];
#pragma unroll
  for (int h = 0; h < ROUTE; ++h) acc[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kRouteStepSlots; ++i) {
    const int st = wave + 4 * i;
    if (st < steps) {
      const bf16x8 a = a_frag(st);
#pragma unroll
      for (int h = 0; h < ROUTE; ++h)
        acc[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, rb[i][h], acc[h], 0, 0, 0);
    }
  }
  for (int st = wave + 4 * kRouteStepSlots; st < steps; st += 4) {
    const bf16x8 a = a_frag(st);
#pragma unroll
    for (int h = 0; h < ROUTE; ++h)
      acc[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          a, __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(pb[h] + st * 32)),
          acc[h], 0, 0, 0);
  }
  // Row 0 of the C fragment: lanes 0-15, register 0.
  if (lane < 16) {
    chain_s[wave][lane] = acc[0][0];
    chain_s[wave][16 + lane] = ROUTE > 1 ? acc[ROUTE - 1][0] : 0.0f;
  }
  __syncthreads();
  if (tid < 16) {
    auto logit = [&](int e) -> float {
      const float v = ((chain_s[0][e] + chain_s[1][e]) + chain_s[2][e]) + chain_s[3][e];
      return v + (bias != nullptr ? bias[e] : 0.0f);
    };
    int first, second;
    float vb, vr;
    row_top2(tid < experts ? logit(tid) : 0.0f, tid + 16 < experts ? logit(tid + 16) : 0.0f,
             experts, first, second, vb, vr);
    if (tid == 0) {
      const float e2 = __expf(vr - vb);
      const float den = 1.0f + e2;
      sel[0] = first;
      sel[1] = second;
      sel_w[0] = 1.0f / den;
      sel_w[1] = e2 / den;
    }
  }
  __syncthreads();
}

template <int ROUTE, int NS, int SW>  // SW: hidden columns per workgroup (8 or 16)
__global__ __launch_bounds__(256) void decode_up_kernel(
    const uint16_t* __restrict__ x, DecodeMix mix, const uint16_t* __restrict__ wr,
    const float* __restrict__ bias, int tokens, int dim, int experts, int hidden_dim,
    int shared_dim, int hstride, const uint16_t* __restrict__ gate_up,
    const uint16_t* __restrict__ shared_gate_up, uint16_t* __restrict__ hidden,
    int64_t* __restrict__ indices, float* __restrict__ weights) {
  __shared__ float chain_s[4][kMaxExperts];
  __shared__ int sel[2];
  __shared__ float sel_w[2];
  // SW = 16: [wave][k chunk][gate 16 | up 16]; SW = 8: [wave][k chunk, step
  // parity][gate 8 | up 8].
  __shared__ float part[4][SW == 16 ? 4 : 8][2 * SW];
  __shared__ DepthMixLds mix_lds;
  // The slot's token row [dim].
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  // The kernel arguments of the load phase in one batch of scalar loads
  // (each field first read on its own would cost a scalar round trip).
  if constexpr (NS > 0) {
    const uint16_t* sp[kMaxDepthSources];
#pragma unroll
    for (int s = 0; s < kMaxDepthSources; ++s) sp[s] = mix.srcs.src[s];
    static_assert(kMaxDepthSources == 9, "the batch below names every source slot");
    asm volatile("" ::"s"(sp[0]), "s"(sp[1]), "s"(sp[2]), "s"(sp[3]), "s"(sp[4]), "s"(sp[5]),
                 "s"(sp[6]), "s"(sp[7]), "s"(sp[8]), "s"(mix.query), "s"(mix.score_w),
                 "s"(mix.out_w), "s"(mix.pend), "s"(mix.pend_lanes), "s"(mix.pend_base));
  }
  asm volatile("" ::"s"(wr), "s"(tokens), "s"(dim), "s"(experts), "s"(hidden_dim),
               "s"(shared_dim));
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int slot = blockIdx.y;
  const int slice = blockIdx.x;
  const bool shared = slot >= 2 * tokens;
  const int H = shared ? shared_dim : hidden_dim;
  if (slice * SW >= H) return;  // uniform
  const int t0 = shared ? slot - 2 * tokens : slot >> 1;  // the slot's token
  // Router weight fragments of this wavefront's chain, loaded right after
  // the input row's loads with no branch between (every slot loads them, the
  // shared slot's go unused; clamped, unconditional loads), so the waits for
  // the input count them exactly and they arrive during the mix.
  const int koff = (lane >> 4) * 8;
  const uint16_t* pb[ROUTE];
  bf16x8 rb[kRouteStepSlots][ROUTE];
  auto load_router = [&]() {
    const int last = dim / 32 - 1;
#pragma unroll
    for (int h = 0; h < ROUTE; ++h)
      pb[h] = wr + static_cast<int64_t>(min(16 * h + (lane & 15), experts - 1)) * dim + koff;
#pragma unroll
    for (int i = 0; i < kRouteStepSlots; ++i)
#pragma unroll
      for (int h = 0; h < ROUTE; ++h)
        rb[i][h] = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const uint4*>(pb[h] + min(wave + 4 * i, last) * 32));
  };
  if constexpr (NS > 0) {
    // The token's input row: depth mix + RMSNorm of its NS sources into
    // LDS, every load issued before the first wait (lanes past the row read
    // chunk 0 and are zeroed).
    const int chunks = dim >> 2;
    const bool has = tid < chunks;
    const int ic = has ? tid : 0;
    const int64_t base = static_cast<int64_t>(t0) * chunks;
    uint2 v[kMaxDepthSources];
#pragma unroll
    for (int s = 0; s < NS; ++s) v[s] = reinterpret_cast<const uint2*>(mix.srcs.src[s])[base + ic];
    const uint2 q = reinterpret_cast<const uint2*>(mix.query)[ic];
    const uint2 g = reinterpret_cast<const uint2*>(mix.score_w)[ic];
    const uint2 g_out = reinterpret_cast<const uint2*>(mix.out_w)[ic];
    // The pending last source's first 8 lanes and its base, loaded
    // unconditionally (from the query row when there is none).
    const bool pending = mix.pend != nullptr;  // uniform
    const int lanes = pending ? mix.pend_lanes : 1;
    const int64_t pstride = pending ? chunks : 0;
    const float4* pc = pending ? reinterpret_cast<const float4*>(mix.pend) +
                                     static_cast<int64_t>(t0) * lanes * chunks + ic
                               : reinterpret_cast<const float4*>(mix.query);
    float4 c[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) c[u] = pc[min(u, lanes - 1) * pstride];
    const uint2 pbv = *(mix.pend_base != nullptr
                            ? reinterpret_cast<const uint2*>(mix.pend_base) + base + ic
                            : reinterpret_cast<const uint2*>(mix.query));
    // Fences: the loads above go out before the router's, and the router's
    // before any use of the input (no load sunk into a branch below).
    asm volatile("" ::: "memory");
    load_router();
    asm volatile("" ::: "memory");
    if (pending) {
      // This chunk's contributions summed over the lanes in order, rounded,
      // then added to the base with a second rounding; the token's first
      // routed workgroup of slice 0 stores the resolved row.  Lanes past
      // the end add -0, the exact identity, so no add sits behind a branch.
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      auto add = [&](const float4& cv, bool on) {
        acc[0] += on ? cv.x : -0.0f;
        acc[1] += on ? cv.y : -0.0f;
        acc[2] += on ? cv.z : -0.0f;
        acc[3] += on ? cv.w : -0.0f;
      };
#pragma unroll
      for (int u = 0; u < 8; ++u) add(c[u], u < lanes);
      for (int l0 = 8; l0 < lanes; l0 += 8) {
#pragma unroll
        for (int u = 0; u < 8; ++u) c[u] = pc[min(l0 + u, lanes - 1) * pstride];
#pragma unroll
        for (int u = 0; u < 8; ++u) add(c[u], l0 + u < lanes);
      }
      uint2 r;
      r.x = pack_bf16x2(acc[0], acc[1]);
      r.y = pack_bf16x2(acc[2], acc[3]);
      if (mix.pend_base != nullptr) {
        r.x = pack_bf16x2(lo_bf16(pbv.x) + lo_bf16(r.x), hi_bf16(pbv.x) + hi_bf16(r.x));
        r.y = pack_bf16x2(lo_bf16(pbv.y) + lo_bf16(r.y), hi_bf16(pbv.y) + hi_bf16(r.y));
      }
      v[NS - 1] = r;
      if (has && !shared && slice == 0 && (slot & 1) == 0)
        reinterpret_cast<uint2*>(mix.pend_out)[base + ic] = r;
    }
#pragma unroll
    for (int s = 0; s < NS; ++s)
      if (!has) v[s] = make_uint2(0u, 0u);
    const int waves = (dim + kDepthDimsPerWave - 1) / kDepthDimsPerWave;
    const uint2 mixed =
        depth_mix_chunk<NS>(v, q, g, has, waves, wave, lane, dim, mix.score_eps, mix_lds);
    const uint2 o = depth_mix_norm_chunk(mixed, g_out, has, waves, wave, lane, dim, mix.out_eps,
                                         mix_lds);
    if (has) reinterpret_cast<uint2*>(xs)[tid] = o;
  } else {
    // The slot's activation row, staged in LDS as bf16 (the barrier before
    // the router, or the shared slot's below, orders it before use).
    load_router();
    for (int i = tid; i < dim / 8; i += 256)
      reinterpret_cast<uint4*>(xs)[i] =
          reinterpret_cast<const uint4*>(x + static_cast<int64_t>(t0) * dim)[i];
  }
  const uint16_t* w;
  if (shared) {
    __syncthreads();
    w = shared_gate_up;
  } else {
    // The router reads the row from LDS once every wavefront has written
    // its part there.
    __syncthreads();
    route_slot<ROUTE>(xs, rb, pb, bias, dim, experts, chain_s, sel, sel_w);
    const int k = slot & 1;
    if (slice == 0 && k == 0 && tid < 2) {
      indices[2 * t0 + tid] = sel[tid];
      weights[2 * t0 + tid] = sel_w[tid];
    }
    w = gate_up + static_cast<int64_t>(sel[k]) * 2 * hidden_dim * dim;
  }
  const int ksteps = dim / 32;
  const int64_t hrow = (shared ? 2 * tokens + t0 : slot) * static_cast<int64_t>(hstride);
  if constexpr (SW == 16) {
    // Packed rows [32 slice, 32 slice + 32): gate group 2 slice, up group
    // 2 slice + 1; block (g, s) at ((g * ksteps) + s) KB.  Wavefront w
    // takes k steps w, w + 4, ..., the weight fragments of up to 8 of them
    // in flight at once.
    const uint4* wg = reinterpret_cast<const uint4*>(w) + (2 * slice) * ksteps * 64 + lane;
    const uint4* wu = wg + ksteps * 64;
    const int c = lane >> 4;
    float ag = 0.0f, au = 0.0f;
    for (int s0 = wave; s0 < ksteps; s0 += 32) {
      uint4 g[8], u[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int st = min(s0 + 4 * i, ksteps - 1);
        g[i] = wg[st * 64];
        u[i] = wu[st * 64];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int st = s0 + 4 * i;
        if (st < ksteps) {
          const uint4 xv = *reinterpret_cast<const uint4*>(xs + st * 32 + c * 8);
          ag += dot8(g[i], xv);
          au += dot8(u[i], xv);
        }
      }
    }
    const int r = lane & 15;
    part[wave][c][r] = ag;
    part[wave][c][16 + r] = au;
    __syncthreads();
    if (tid < 16) {
      float gs = 0.0f, us = 0.0f;
#pragma unroll
      for (int wv = 0; wv < 4; ++wv)
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
          gs += part[wv][cc][tid];
          us += part[wv][cc][16 + tid];
        }
      hidden[hrow + slice * 16 + tid] = f32_to_bf16(swiglu(gs, us));
    }
  } else {
    // Hidden columns [8 slice, 8 slice + 8): rows 8 h .. 8 h + 7 (h = slice
    // % 2) of gate group 2 (slice / 2) and of up group 2 (slice / 2) + 1.
    // Lane l takes row r = l % 8 of them, k chunk kc = (l / 8) % 4 of a
    // 32-wide k step and the step of parity sp = l / 32 in a pair, so one
    // wavefront load covers two k steps of a half block as 4 contiguous
    // 128-byte runs; wavefront w takes step pairs w, w + 4, w + 8 per batch
    // (at dim 768, all 12 pairs in one).
    const int r = lane & 7, kc = (lane >> 3) & 3, sp = lane >> 5;
    const uint4* wg = reinterpret_cast<const uint4*>(w) + (2 * (slice >> 1)) * ksteps * 64 +
                      (slice & 1) * 8 + r + 16 * kc;
    const uint4* wu = wg + ksteps * 64;
    float ag = 0.0f, au = 0.0f;
    for (int p0 = wave; 2 * p0 < ksteps; p0 += 12) {
      uint4 g[3], u[3];
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const int st = min(2 * (p0 + 4 * i) + sp, ksteps - 1);
        g[i] = wg[st * 64];
        u[i] = wu[st * 64];
      }
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const int st = 2 * (p0 + 4 * i) + sp;
        if (st < ksteps) {
          const uint4 xv = *reinterpret_cast<const uint4*>(xs + st * 32 + kc * 8);
          ag += dot8(g[i], xv);
          au += dot8(u[i], xv);
        }
      }
    }
    part[wave][lane >> 3][r] = ag;
    part[wave][lane >> 3][8 + r] = au;
    __syncthreads();
    if (tid < 16) {
      // Lanes 0-7: gate rows, 8-15: up rows, each summed over (wavefront,
      // k chunk, step parity) in a fixed order; lane j < 8 then takes up row
      // j from lane j + 8.
      float v = 0.0f;
#pragma unroll
      for (int wv = 0; wv < 4; ++wv)
#pragma unroll
        for (int j = 0; j < 8; ++j) v += part[wv][j][tid];
      const float us = __shfl_xor(v, 8);
      if (tid < 8) hidden[hrow + slice * 8 + tid] = f32_to_bf16(swiglu(v, us));
    }
  }
}

__global__ __launch_bounds__(256) void decode_down_kernel(
    const uint16_t* __restrict__ hidden, int tokens, int dim, int hidden_dim, int shared_dim,
    int hstride, const int64_t* __restrict__ indices, const float* __restrict__ weights,
    const uint16_t* __restrict__ down, const uint16_t* __restrict__ shared_down,
    const uint16_t* __restrict__ addend, uint16_t* __restrict__ out) {
  __shared__ float part[3][4][4][16];  // [contribution][wave][k chunk][column]
  // The kernel arguments in one batch of scalar loads, then the token's two
  // expert ids (scalar loads too): the routed weights' addresses wait for
  // them, the hidden rows and the shared expert's weights do not.
  asm volatile("" ::"s"(hidden), "s"(indices), "s"(weights), "s"(down), "s"(shared_down),
               "s"(addend), "s"(out), "s"(tokens), "s"(dim), "s"(hidden_dim), "s"(shared_dim),
               "s"(hstride));
  const int t = blockIdx.y;
  const int64_t ex[2] = {indices[2 * t], indices[2 * t + 1]};
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int slice = blockIdx.x;  // output columns [16 slice, 16 slice + 16)
  const int c = lane >> 4;
  // Contribution 0 / 1: routed slot 2t + k (expert indices[2t + k], K = H);
  // contribution 2: the shared expert (K = Hs).  Wavefront w takes k steps
  // w, w + 4, ...; the loads of up to 4 steps of all three are issued
  // before any arithmetic: the hidden rows and the shared weights first,
  // the routed weights last.
  const uint16_t* hrow[3];
  int ks[3];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    const bool sh = q == 2;
    ks[q] = (sh ? shared_dim : hidden_dim) / 32;
    hrow[q] = hidden + (sh ? 2 * tokens + t : 2 * t + q) * static_cast<int64_t>(hstride) + c * 8;
  }
  const uint4* wsh = reinterpret_cast<const uint4*>(shared_down) + slice * ks[2] * 64 + lane;
  float acc[3] = {0.0f, 0.0f, 0.0f};
  auto batch = [&](int s0) {
    uint4 wv[3][4], hv[3][4];
#pragma unroll
    for (int q = 0; q < 3; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        hv[q][i] = *reinterpret_cast<const uint4*>(hrow[q] + min(s0 + 4 * i, ks[q] - 1) * 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) wv[2][i] = wsh[min(s0 + 4 * i, ks[2] - 1) * 64];
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);  // the expert ids' first use (a wait) after these loads
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint4* wb = reinterpret_cast<const uint4*>(
                            down + ex[q] * static_cast<int64_t>(dim) * hidden_dim) +
                        slice * ks[q] * 64 + lane;
#pragma unroll
      for (int i = 0; i < 4; ++i) wv[q][i] = wb[min(s0 + 4 * i, ks[q] - 1) * 64];
    }
    asm volatile("" ::: "memory");
    // The shared expert's products first: its weights were loaded before the
    // routed ones, so they are computed while those arrive (each sum keeps
    // its own order).
#pragma unroll
    for (int qq = 0; qq < 3; ++qq) {
      const int q = (qq + 2) % 3;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (s0 + 4 * i < ks[q]) acc[q] += dot8(wv[q][i], hv[q][i]);
    }
  };
  // The first batch straight-line (its loads are clamped, so it is safe for
  // a wavefront past the k range), so that no address computation is
  // hoisted ahead of its loads; more batches only past 16 k steps.
  batch(wave);
  for (int s0 = wave + 16; s0 < max(ks[0], ks[2]); s0 += 16) batch(s0);
#pragma unroll
  for (int q = 0; q < 3; ++q) part[q][wave][c][lane & 15] = acc[q];
  __syncthreads();
  if (tid < 16) {
    float y[3];
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      float v = 0.0f;
#pragma unroll
      for (int wv = 0; wv < 4; ++wv)
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) v += part[q][wv][cc][tid];
      y[q] = v;
    }
    // combine_kernel's order and rounding points: the shared row and each
    // weighted routed row rounded to bf16 (as the down projection writes
    // them), then added in fp32, shared first.
    const float v = (bf16_round(y[2]) + bf16_round(weights[2 * t] * y[0])) +
                    bf16_round(weights[2 * t + 1] * y[1]);
    const int64_t o = static_cast<int64_t>(t) * dim + slice * 16 + tid;
    uint16_t r = f32_to_bf16(v);
    if (addend != nullptr) r = f32_to_bf16(bf16_to_f32(addend[o]) + bf16_to_f32(r));
    out[o] = r;
  }
}

}  // namespace

int decode_moe_max_tokens() { return kDecodeMaxTokens; }

hipError_t launch_decode_moe(const uint16_t* x, const DecodeMix* mix, int tokens, int dim,
                             int experts, int hidden_dim, int shared_dim,
                             const uint16_t* router_w, const float* bias, const ExpertWeights& w,
                             const uint16_t* addend, uint16_t* out, int64_t* indices,
                             float* weights, uint16_t* hidden, hipStream_t s) {
  if (tokens == 0) return hipSuccess;
  const int hstride = hidden_dim > shared_dim ? hidden_dim : shared_dim;
  const DecodeMix none{};
  // Eight hidden columns per workgroup at one or two tokens (more workgroups
  // streaming less of an expert each), sixteen past that (the input mix is
  // repeated by every workgroup of a token).
  const bool narrow = tokens <= 2;
  const dim3 up_grid(hstride / (narrow ? 8 : 16), 3 * tokens);
  const size_t up_lds = decode_up_lds_bytes(dim);
  const DecodeMix m = mix != nullptr ? *mix : none;
  const bool mixing = m.n_sources > 0;
  auto up = [&](auto kernel) {
    kernel<<<up_grid, 256, up_lds, s>>>(x, m, router_w, bias, tokens, dim, experts, hidden_dim,
                                        shared_dim, hstride, w.gate_up, w.shared_gate_up, hidden,
                                        indices, weights);
  };
  hipError_t e = hipSuccess;
  auto up_sw = [&](auto ns) {
    if (narrow)
      experts <= 16 ? up(decode_up_kernel<1, ns, 8>) : up(decode_up_kernel<2, ns, 8>);
    else
      experts <= 16 ? up(decode_up_kernel<1, ns, 16>) : up(decode_up_kernel<2, ns, 16>);
    return hipSuccess;
  };
  if (mixing)
    e = with_sources(m.n_sources, up_sw);
  else
    e = up_sw(std::integral_constant<int, 0>{});
  if (e == hipSuccess) e = hipGetLastError();
  if (e != hipSuccess) return e;
  decode_down_kernel<<<dim3(dim / 16, tokens), 256, 0, s>>>(
      hidden, tokens, dim, hidden_dim, shared_dim, hstride, indices, weights, w.down,
      w.shared_down, addend, out);
  return hipGetLastError();
}

}  // namespace parrot
