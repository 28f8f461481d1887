// RMSNorm and Block AttnRes depth mixing: HBM-bound row kernels.
//
// One 64-lane wavefront (one workgroup) owns one row, so small token counts
// still spread over every CU; lanes stride over 4-element (8-byte) chunks so
// a wavefront instruction moves 512 contiguous bytes, and every load of a
// row is issued before the first reduction.  Sums are
// fp32 butterfly reductions; every output is rounded to bf16 exactly once,
// at the same point as the reference (parrot/model.py:125-127 for RMSNorm,
// :149-155 for the depth mix, parrot/kernels/moe_bf16.metal:414-433 for the
// mix rounded to bf16 before its consumer RMSNorm).
#include "depth_mix_core.h"

namespace parrot {

namespace {

constexpr int kRowsPerBlock = 1;  // one row per 64-lane workgroup

// y = bf16((x * rsqrt(mean(x^2) + eps)) * w)        (parrot/model.py:125-127)
template <int MAXC>
__global__ __launch_bounds__(64) void rms_norm_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ out, int64_t rows, int dim, float eps) {
  // The kernel arguments in one batch of scalar loads before any use.
  asm volatile("" ::"s"(x), "s"(w), "s"(out), "s"(rows), "s"(dim), "s"(eps));
  __builtin_amdgcn_sched_barrier(0);
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;  // uniform per wavefront
  const int chunks = dim >> 2;
  const uint2* xr = reinterpret_cast<const uint2*>(x + row * dim);
  const uint2* wr = reinterpret_cast<const uint2*>(w);
  uint2* yr = reinterpret_cast<uint2*>(out + row * dim);
  uint2 v[MAXC], g[MAXC];
  // The row's chunks, then the weight's: the weight load is in flight during
  // the reduction instead of a second round trip after it.
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int i = lane + c * kWave;
    v[c] = i < chunks ? xr[i] : make_uint2(0u, 0u);
  }
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int i = lane + c * kWave;
    g[c] = i < chunks ? wr[i] : make_uint2(0u, 0u);
  }
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const float a = lo_bf16(v[c].x), b = hi_bf16(v[c].x);
    const float d = lo_bf16(v[c].y), e = hi_bf16(v[c].y);
    ss += a * a + b * b + d * d + e * e;
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / static_cast<float>(dim) + eps);
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int i = lane + c * kWave;
    if (i < chunks) {
      uint2 o;
      o.x = pack_bf16x2(lo_bf16(v[c].x) * r * lo_bf16(g[c].x),
                        hi_bf16(v[c].x) * r * hi_bf16(g[c].x));
      o.y = pack_bf16x2(lo_bf16(v[c].y) * r * lo_bf16(g[c].y),
                        hi_bf16(v[c].y) * r * hi_bf16(g[c].y));
      yr[i] = o;
    }
  }
}

// Block AttnRes: score_s = <rmsnorm_w(v_s), q>, alpha = softmax_s(score),
// mix = bf16(sum_s alpha_s v_s); optionally y = rmsnorm_out(mix).
// One workgroup per token and one wavefront per 256 dims: a lane owns 4
// consecutive dims of every source, all of whose loads are issued up front;
// the arithmetic is depth_mix_core.h's.  (A single wavefront per token
// serialises ~1500 VALU instructions of unpacking and summing at dim 768 and
// leaves most SIMDs idle.)

// With ROUTE > 0 the kernel also routes the token's normalised row (the MoE
// input) to its top-2 experts, with route_kernel's arithmetic to the bit:
// the logits are the same v_mfma_f32_16x16x32_bf16 chains over the 32-wide
// k steps st = c, c + 4, c + 8, ... for c = 0..3 (the token in A row 0, rows
// 1-15 zero: an MFMA output element depends only on its own row and column),
// summed ((c0 + c1) + c2) + c3, plus the bias; then select_top2.  ROUTE is
// the number of 16-expert tiles (1: E <= 16, 2: E <= 32).  Chain c runs on
// wavefront c % waves; the router weights of a wavefront's first two chains
// (six k steps each: dim 768) are loaded with the sources, the rest in the
// chain itself.
constexpr int kRouteChainSlots = 2;
constexpr int kRouteStepSlots = 6;

// PL > 0 (PL == kPendingHeads): the last source is a pending attention
// output, bf16(base + bf16(sum over heads of pend.contrib)), made here and
// written to pend.out (the depth mix of the MoE module that follows the
// attention).
template <int ROUTE, int NS, int PL = 0>
__global__ __launch_bounds__(64 * kDepthMaxWaves) void depth_mix_kernel(
    DepthSources srcs, const uint16_t* __restrict__ query,
    const uint16_t* __restrict__ score_w, float score_eps,
    const uint16_t* __restrict__ out_w, float out_eps, int64_t tokens, int dim,
    uint16_t* __restrict__ out_mix, uint16_t* __restrict__ out_norm, CombineSource comb,
    RouteOut route, PendingSum pend) {
  __shared__ DepthMixLds mix_lds;
  // The kernel arguments of the load phase in one batch of scalar loads,
  // before anything uses one: a field first read inside a branch, or after
  // an earlier batch was waited for, costs a scalar round trip of its own.
  const uint16_t* sp[kMaxDepthSources];
#pragma unroll
  for (int s = 0; s < kMaxDepthSources; ++s) sp[s] = srcs.src[s];
  static_assert(kMaxDepthSources == 9, "the batch below names every source slot");
  asm volatile("" ::"s"(sp[0]), "s"(sp[1]), "s"(sp[2]), "s"(sp[3]), "s"(sp[4]), "s"(sp[5]),
               "s"(sp[6]), "s"(sp[7]), "s"(sp[8]), "s"(comb.y_shared), "s"(comb.y_routed),
               "s"(comb.addend), "s"(query), "s"(score_w), "s"(out_w), "s"(out_norm),
               "s"(dim), "s"(comb.out), "s"(out_mix), "s"(blockDim.x));
  if constexpr (ROUTE > 0)
    asm volatile("" ::"s"(route.router_w), "s"(route.bias), "s"(route.experts),
                 "s"(route.weights), "s"(route.indices));
  if constexpr (PL > 0) asm volatile("" ::"s"(pend.contrib), "s"(pend.base), "s"(pend.out));
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int waves = blockDim.x >> 6;
  const int64_t tok = blockIdx.x;
  const int chunks = dim >> 2;
  const int i = wave * kWave + lane;  // this lane's 4-dim chunk
  const bool has = i < chunks;
  const int64_t base = tok * chunks;

  // Every load of the workgroup is issued before the first wait.  The NS
  // source slots are loaded (with a combine, the last one too: it holds a
  // valid row and is replaced below), lanes past the row load chunk 0 and
  // zero it afterwards, and only uniform conditions (combine, addend, output
  // norm) guard a load: a load behind a branch on a kernel argument, or
  // inside a per-lane branch, costs a serial round trip each.
  const bool combine = PL == 0 && comb.y_shared != nullptr;  // never with a pending source
  const int ic = has ? i : 0;
  uint2 v[kMaxDepthSources];
#pragma unroll
  for (int s = 0; s < NS; ++s) v[s] = reinterpret_cast<const uint2*>(sp[s])[base + ic];
  uint2 sh = make_uint2(0u, 0u), y0 = sh, y1 = sh;
  uint2 pa = make_uint2(0u, 0u);
  if (combine) {
    sh = reinterpret_cast<const uint2*>(comb.y_shared)[base + ic];
    y0 = reinterpret_cast<const uint2*>(comb.y_routed)[(2 * tok) * chunks + ic];
    y1 = reinterpret_cast<const uint2*>(comb.y_routed)[(2 * tok + 1) * chunks + ic];
    if (comb.addend != nullptr) pa = reinterpret_cast<const uint2*>(comb.addend)[base + ic];
  }
  // The pending attention output's per-head contributions (4 fp32 each).
  float4 pc[PL > 0 ? PL : 1];
  uint2 pbase = make_uint2(0u, 0u);
  if constexpr (PL > 0) {
#pragma unroll
    for (int h = 0; h < PL; ++h)
      pc[h] = reinterpret_cast<const float4*>(pend.contrib)[(tok * PL + h) * chunks + ic];
    // (the query row stands in for a missing base: an unconditional load
    // keeps the waits below exact; a load behind a branch makes the first
    // use of any earlier load wait for every load, vmcnt(0))
    pbase = (pend.base != nullptr ? reinterpret_cast<const uint2*>(pend.base) + base
                                  : reinterpret_cast<const uint2*>(query))[ic];
  }
  const uint2 q = reinterpret_cast<const uint2*>(query)[ic];
  const uint2 g = reinterpret_cast<const uint2*>(score_w)[ic];
  const uint2 g_out = reinterpret_cast<const uint2*>(out_norm != nullptr ? out_w : score_w)[ic];
  // Router weights of this wavefront's first chains (ROUTE > 0).
  const int steps = dim / 32;
  const int koff = (lane >> 4) * 8;
  const uint16_t* pb[2] = {nullptr, nullptr};
  bf16x8 rb[kRouteChainSlots][kRouteStepSlots][ROUTE > 0 ? ROUTE : 1];
  if constexpr (ROUTE > 0) {
#pragma unroll
    for (int h = 0; h < ROUTE; ++h)
      pb[h] = route.router_w +
              static_cast<int64_t>(min(16 * h + (lane & 15), route.experts - 1)) * dim + koff;
    // Every wavefront loads every slot (chains and steps past the last are
    // clamped to it and go unused), with no branch, so that the waits for
    // the loads before these count them exactly.
#pragma unroll
    for (int j = 0; j < kRouteChainSlots; ++j)
#pragma unroll
      for (int i = 0; i < kRouteStepSlots; ++i) {
        const int c = min(wave + j * waves, 3), st = min(c + 4 * i, steps - 1);
#pragma unroll
        for (int h = 0; h < ROUTE; ++h)
          rb[j][i][h] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(pb[h] + st * 32));
      }
  }

  // Lanes past the row hold zeros from here on.
#pragma unroll
  for (int s = 0; s < NS; ++s)
    if (!has) v[s] = make_uint2(0u, 0u);
  if (combine) {
    // The MoE output row: bf16(shared + routed 0 + routed 1), then
    // bf16(addend + that), exactly as the combine kernel; it is the new
    // residual source and the last depth source.
    uint2 o;
    o.x = pack_bf16x2(lo_bf16(sh.x) + lo_bf16(y0.x) + lo_bf16(y1.x),
                      hi_bf16(sh.x) + hi_bf16(y0.x) + hi_bf16(y1.x));
    o.y = pack_bf16x2(lo_bf16(sh.y) + lo_bf16(y0.y) + lo_bf16(y1.y),
                      hi_bf16(sh.y) + hi_bf16(y0.y) + hi_bf16(y1.y));
    if (comb.addend != nullptr) {
      o.x = pack_bf16x2(lo_bf16(pa.x) + lo_bf16(o.x), hi_bf16(pa.x) + hi_bf16(o.x));
      o.y = pack_bf16x2(lo_bf16(pa.y) + lo_bf16(o.y), hi_bf16(pa.y) + hi_bf16(o.y));
    }
    if (has) reinterpret_cast<uint2*>(comb.out)[base + i] = o;
    else o = make_uint2(0u, 0u);
    v[NS - 1] = o;
  }
  if constexpr (PL > 0) {
    // The attention output: the heads' fp32 sum in head order, rounded to
    // bf16, then bf16(base + that) -- the output projection's rounding with
    // its residual addend (parrot_proj_bf16's kStore).
    float4 t = pc[0];
#pragma unroll
    for (int h = 1; h < PL; ++h) {
      t.x += pc[h].x;
      t.y += pc[h].y;
      t.z += pc[h].z;
      t.w += pc[h].w;
    }
    uint2 o;
    o.x = pack_bf16x2(t.x, t.y);
    o.y = pack_bf16x2(t.z, t.w);
    // Without a base, -0 is added: the exact identity for every bf16 value
    // (signed zeros included), so the add sits behind no branch (a branch
    // would take the base's load with it and wait for every load there).
    const uint2 bz = pend.base != nullptr ? pbase : make_uint2(0x80008000u, 0x80008000u);
    o.x = pack_bf16x2(lo_bf16(bz.x) + lo_bf16(o.x), hi_bf16(bz.x) + hi_bf16(o.x));
    o.y = pack_bf16x2(lo_bf16(bz.y) + lo_bf16(o.y), hi_bf16(bz.y) + hi_bf16(o.y));
    if (has) reinterpret_cast<uint2*>(pend.out)[base + i] = o;
    else o = make_uint2(0u, 0u);
    v[NS - 1] = o;
  }
  const uint2 mixed = depth_mix_chunk<NS>(v, q, g, has, waves, wave, lane, dim, score_eps, mix_lds);
  if (out_mix != nullptr && has) reinterpret_cast<uint2*>(out_mix)[base + i] = mixed;
  if (out_norm == nullptr) return;  // uniform over the workgroup
  const uint2 o = depth_mix_norm_chunk(mixed, g_out, has, waves, wave, lane, dim, out_eps,
                                       mix_lds);
  if (has) reinterpret_cast<uint2*>(out_norm)[base + i] = o;
  if constexpr (ROUTE > 0) {
    __shared__ __attribute__((aligned(16))) uint16_t xn[kDepthDimsPerWave * kDepthMaxWaves];
    __shared__ float chain_s[4][kMaxExperts];
    __shared__ int ids_s[8];
    if (has) reinterpret_cast<uint2*>(xn)[i] = o;
    __syncthreads();
    const bool row0 = (lane & 15) == 0;
    auto a_frag = [&](int st) {
      const uint4 av = row0 ? *reinterpret_cast<const uint4*>(&xn[st * 32 + koff])
                            : make_uint4(0u, 0u, 0u, 0u);
      return __builtin_bit_cast(bf16x8, av);
    };
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = wave + j * waves;
      if (c >= 4) break;  // uniform
      f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int i = 0; i < kRouteStepSlots; ++i) {
        const int st = c + 4 * i;
        if (st < steps) {
          const bf16x8 a = a_frag(st);
#pragma unroll
          for (int h = 0; h < ROUTE; ++h) {
            const bf16x8 b = j < kRouteChainSlots
                                 ? rb[j < kRouteChainSlots ? j : 0][i][h]
                                 : __builtin_bit_cast(
                                       bf16x8, *reinterpret_cast<const uint4*>(pb[h] + st * 32));
            acc[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[h], 0, 0, 0);
          }
        }
      }
      for (int st = c + 4 * kRouteStepSlots; st < steps; st += 4) {
        const bf16x8 a = a_frag(st);
#pragma unroll
        for (int h = 0; h < ROUTE; ++h)
          acc[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              a, __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(pb[h] + st * 32)),
              acc[h], 0, 0, 0);
      }
      // Row 0 of the C fragment: lanes 0-15, register 0.
      if (lane < 16) {
        chain_s[c][lane] = acc[0][0];
        chain_s[c][16 + lane] = ROUTE > 1 ? acc[1][0] : 0.0f;
      }
    }
    __syncthreads();
    if (wave == 0) {
      const int experts = route.experts;
      const int j = lane & 15;
      auto logit = [&](int e) -> float {
        const float v = ((chain_s[0][e] + chain_s[1][e]) + chain_s[2][e]) + chain_s[3][e];
        return v + (route.bias != nullptr ? route.bias[e] : 0.0f);
      };
      const float l0 = j < experts ? logit(j) : 0.0f;
      const float l1 = j + 16 < experts ? logit(j + 16) : 0.0f;
      select_top2(l0, l1, experts, tok, lane < 16, nullptr, nullptr, route.weights,
                  route.indices, &ids_s[2 * (lane >> 4)]);
    }
  }
}

// The forward's first launch (parrot/model.py:679, 685-687): the tokens'
// embedding rows gathered by id and written out (the residual stream's first
// source, as nn.Embedding does), and the first module's input, the depth mix
// of that single source and its RMSNorm, with depth_mix_kernel<0, 1>'s
// arithmetic (the same bits for every token; a single source's softmax
// weight is exactly 1, so the mix is the row).  Workgroup 0 also zero-fills
// `zeros` (the forward's router-stat outputs when they are not collected,
// parrot/model.py:719-723).  Ids outside [0, vocab) read the nearest row;
// the host rejects them before an eager launch.
__global__ __launch_bounds__(64 * kDepthMaxWaves) void embed_mix_kernel(
    const int64_t* __restrict__ ids, const uint16_t* __restrict__ table, int64_t vocab,
    const uint16_t* __restrict__ query, const uint16_t* __restrict__ score_w, float score_eps,
    const uint16_t* __restrict__ out_w, float out_eps, int64_t tokens, int dim,
    uint16_t* __restrict__ rows_out, uint16_t* __restrict__ out_norm,
    float* __restrict__ zeros, int n_zeros) {
  __shared__ DepthMixLds mix_lds;
  asm volatile("" ::"s"(ids), "s"(table), "s"(vocab), "s"(query), "s"(score_w), "s"(out_w),
               "s"(dim), "s"(rows_out), "s"(out_norm), "s"(zeros), "s"(n_zeros), "s"(tokens));
  if (blockIdx.x == 0)
    for (int z = threadIdx.x; z < n_zeros; z += blockDim.x) zeros[z] = 0.0f;
  if (static_cast<int64_t>(blockIdx.x) >= tokens) return;  // uniform: the zero-fill-only launch
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int waves = blockDim.x >> 6;
  const int64_t tok = blockIdx.x;
  const int chunks = dim >> 2;
  const int i = wave * kWave + lane;
  const bool has = i < chunks;
  const int ic = has ? i : 0;
  const int64_t id = min(max(ids[tok], int64_t{0}), vocab - 1);
  const uint2 q = reinterpret_cast<const uint2*>(query)[ic];
  const uint2 g = reinterpret_cast<const uint2*>(score_w)[ic];
  const uint2 g_out = reinterpret_cast<const uint2*>(out_w)[ic];
  uint2 v[kMaxDepthSources];
  v[0] = reinterpret_cast<const uint2*>(table)[id * chunks + ic];
  if (!has) v[0] = make_uint2(0u, 0u);
  if (has) reinterpret_cast<uint2*>(rows_out)[tok * chunks + i] = v[0];
  const uint2 mixed = depth_mix_chunk<1>(v, q, g, has, waves, wave, lane, dim, score_eps, mix_lds);
  const uint2 o = depth_mix_norm_chunk(mixed, g_out, has, waves, wave, lane, dim, out_eps,
                                       mix_lds);
  if (has) reinterpret_cast<uint2*>(out_norm)[tok * chunks + i] = o;
}

// The depth mix at large token counts: one wavefront per token, two
// tokens per workgroup, no barrier.  The wavefront does, slice by slice, what
// the wavefronts of depth_mix_kernel do side by side: lane l owns the 4-dim
// chunks l, l + 64, ... (slice w = the chunks of wavefront w there), every
// slice's per-source partials are summed in the same order as
// wave_total_lane63 sums them, and the slice totals are added in slice
// order, so the scores, the mix and its norm are the same bits for every
// token whichever kernel runs it (a token's result does not depend on the
// batch).  What changes is the cost per byte: depth_mix_kernel keeps a
// token's three wavefronts waiting on each other at two barriers and LDS
// round trips, so at large token counts a CU holds ~8 tokens in flight; here
// a token is one wavefront.  The kernel is bound by its VALU work, most of
// it the per-quantity reductions, so the rows' sums are combined through
// LDS (one lane per quantity) instead of by three row broadcasts per
// quantity.  Two tokens per workgroup measured 1-3 % faster than one or
// four at 65536 tokens (MI355X, sources read from HBM), eight 13 % slower.
// NCH: slices (wavefronts of the other kernel), dim <= 256 NCH.
constexpr int kDepthWaveTokensPerGroup = 2;
constexpr int kDepthWaveMinTokens = 4096;  // from here launch_depth_mix takes this kernel

constexpr int kDepthWaveSlices = 4;  // dim <= 1024

template <int NS, int NCH>
__global__ __launch_bounds__(64 * kDepthWaveTokensPerGroup) void depth_mix_wave_kernel(
    DepthSources srcs, const uint16_t* __restrict__ query,
    const uint16_t* __restrict__ score_w, float score_eps,
    const uint16_t* __restrict__ out_w, float out_eps, int64_t tokens, int dim,
    uint16_t* __restrict__ out_mix, uint16_t* __restrict__ out_norm) {
  static_assert(NCH <= kDepthWaveSlices, "dim <= 256 kDepthWaveSlices");
  // Per wavefront: the DPP-row sums of every (slice, row, quantity).  Only
  // the wavefront that writes them reads them (LDS operations of a
  // wavefront complete in order): no barrier.
  __shared__ float red_s[kDepthWaveTokensPerGroup][kDepthWaveSlices][4][2 * kMaxDepthSources];
  __shared__ float red_out_s[kDepthWaveTokensPerGroup][kDepthWaveSlices][4];
  const uint16_t* sp[kMaxDepthSources];
#pragma unroll
  for (int s = 0; s < kMaxDepthSources; ++s) sp[s] = srcs.src[s];
  static_assert(kMaxDepthSources == 9, "the batch below names every source slot");
  asm volatile("" ::"s"(sp[0]), "s"(sp[1]), "s"(sp[2]), "s"(sp[3]), "s"(sp[4]), "s"(sp[5]),
               "s"(sp[6]), "s"(sp[7]), "s"(sp[8]), "s"(query), "s"(score_w), "s"(out_w),
               "s"(out_norm), "s"(dim), "s"(out_mix), "s"(tokens));
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t tok = static_cast<int64_t>(blockIdx.x) * kDepthWaveTokensPerGroup +
                      __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (tok >= tokens) return;  // uniform per wavefront; no barrier follows
  const int chunks = dim >> 2;
  const int64_t base = tok * chunks;
  bool has[NCH];
  int ic[NCH];
#pragma unroll
  for (int w = 0; w < NCH; ++w) {
    has[w] = w * kWave + lane < chunks;
    ic[w] = has[w] ? w * kWave + lane : 0;  // clamped: every load is unconditional
  }
  uint2 v[NCH][kMaxDepthSources];
#pragma unroll
  for (int w = 0; w < NCH; ++w)
#pragma unroll
    for (int s = 0; s < NS; ++s) v[w][s] = reinterpret_cast<const uint2*>(sp[s])[base + ic[w]];
  uint2 q[NCH], g[NCH], g_out[NCH];
#pragma unroll
  for (int w = 0; w < NCH; ++w) {
    q[w] = reinterpret_cast<const uint2*>(query)[ic[w]];
    g[w] = reinterpret_cast<const uint2*>(score_w)[ic[w]];
    g_out[w] = reinterpret_cast<const uint2*>(out_norm != nullptr ? out_w : score_w)[ic[w]];
  }
  // Per slice: the chunk's partials (depth_mix_chunk's products and sums),
  // each summed over its 16-lane DPP row by wave_total_lane63's first four
  // steps (row_sum: every lane of row r then holds the row's sum r_r); lane 0
  // of each row stores its row sums in LDS.  Lane 2s (+1) then adds, per
  // slice, ((r_0 + r_1) + r_2) + r_3 -- lane 63's total of
  // wave_total_lane63, whose three row broadcasts cost three instructions
  // each per quantity -- and the slice totals in slice order.
  float (&red)[kDepthWaveSlices][4][2 * kMaxDepthSources] = red_s[threadIdx.x >> 6];
#pragma unroll
  for (int w = 0; w < NCH; ++w) {
#pragma unroll
    for (int s = 0; s < NS; ++s)
      if (!has[w]) v[w][s] = make_uint2(0u, 0u);
    float wq[4] = {0.f, 0.f, 0.f, 0.f};
    if (has[w]) {
      wq[0] = lo_bf16(q[w].x) * lo_bf16(g[w].x);
      wq[1] = hi_bf16(q[w].x) * hi_bf16(g[w].x);
      wq[2] = lo_bf16(q[w].y) * lo_bf16(g[w].y);
      wq[3] = hi_bf16(q[w].y) * hi_bf16(g[w].y);
    }
    float rs[2 * kMaxDepthSources];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const float e0 = lo_bf16(v[w][s].x), e1 = hi_bf16(v[w][s].x);
      const float e2 = lo_bf16(v[w][s].y), e3 = hi_bf16(v[w][s].y);
      rs[2 * s] = row_sum(e0 * e0 + e1 * e1 + e2 * e2 + e3 * e3);
      rs[2 * s + 1] = row_sum(e0 * wq[0] + e1 * wq[1] + e2 * wq[2] + e3 * wq[3]);
    }
    if ((lane & 15) == 0) {
#pragma unroll
      for (int i = 0; i < 2 * NS; ++i) red[w][lane >> 4][i] = rs[i];
    }
  }
  float tot = 0.0f;
  if (lane < 2 * NS) {
#pragma unroll
    for (int w = 0; w < NCH; ++w)
      tot += ((red[w][0][lane] + red[w][1][lane]) + red[w][2][lane]) + red[w][3][lane];
  }
  float alpha[NS];
  depth_mix_weights<NS>(tot, dim, score_eps, alpha);
  uint2 mixed[NCH];
  float (&red_out)[kDepthWaveSlices][4] = red_out_s[threadIdx.x >> 6];
#pragma unroll
  for (int w = 0; w < NCH; ++w) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      acc[0] += alpha[s] * lo_bf16(v[w][s].x);
      acc[1] += alpha[s] * hi_bf16(v[w][s].x);
      acc[2] += alpha[s] * lo_bf16(v[w][s].y);
      acc[3] += alpha[s] * hi_bf16(v[w][s].y);
    }
    mixed[w].x = pack_bf16x2(acc[0], acc[1]);
    mixed[w].y = pack_bf16x2(acc[2], acc[3]);
    if (out_mix != nullptr && has[w])
      store_stream(reinterpret_cast<uint2*>(out_mix) + base + w * kWave + lane, mixed[w]);
    if (out_norm != nullptr) {
      // The output norm's sum of squares: per slice, row sums to LDS as
      // above, combined below in depth_mix_norm_chunk's order.
      const float r0 = lo_bf16(mixed[w].x), r1 = hi_bf16(mixed[w].x);
      const float r2 = lo_bf16(mixed[w].y), r3 = hi_bf16(mixed[w].y);
      const float sso = row_sum(has[w] ? r0 * r0 + r1 * r1 + r2 * r2 + r3 * r3 : 0.0f);
      if ((lane & 15) == 0) red_out[w][lane >> 4] = sso;
    }
  }
  if (out_norm == nullptr) return;
  float sso_total = 0.0f;
  if (lane == 0) {
#pragma unroll
    for (int w = 0; w < NCH; ++w) {
      const float t = ((red_out[w][0] + red_out[w][1]) + red_out[w][2]) + red_out[w][3];
      sso_total = w == 0 ? t : sso_total + t;
    }
  }
  sso_total = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sso_total), 0));
  const float r = rsqrtf(sso_total / static_cast<float>(dim) + out_eps);
#pragma unroll
  for (int w = 0; w < NCH; ++w) {
    if (!has[w]) continue;
    const float r0 = lo_bf16(mixed[w].x), r1 = hi_bf16(mixed[w].x);
    const float r2 = lo_bf16(mixed[w].y), r3 = hi_bf16(mixed[w].y);
    uint2 o;
    o.x = pack_bf16x2(r0 * r * lo_bf16(g_out[w].x), r1 * r * hi_bf16(g_out[w].x));
    o.y = pack_bf16x2(r2 * r * lo_bf16(g_out[w].y), r3 * r * hi_bf16(g_out[w].y));
    store_stream(reinterpret_cast<uint2*>(out_norm) + base + w * kWave + lane, o);
  }
}

// Chunks of 4 elements per lane, rounded up to an instantiated count.
int chunk_bucket(int dim) {
  const int per_lane = (dim / 4 + kWave - 1) / kWave;
  if (per_lane <= 1) return 1;
  if (per_lane <= 2) return 2;
  if (per_lane <= 3) return 3;
  if (per_lane <= 4) return 4;
  if (per_lane <= 8) return 8;
  return 16;
}

}  // namespace

hipError_t launch_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* out,
                           int64_t rows, int dim, float eps, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  switch (chunk_bucket(dim)) {
    case 1: rms_norm_kernel<1><<<grid, 64, 0, s>>>(x, w, out, rows, dim, eps); break;
    case 2: rms_norm_kernel<2><<<grid, 64, 0, s>>>(x, w, out, rows, dim, eps); break;
    case 3: rms_norm_kernel<3><<<grid, 64, 0, s>>>(x, w, out, rows, dim, eps); break;
    case 4: rms_norm_kernel<4><<<grid, 64, 0, s>>>(x, w, out, rows, dim, eps); break;
    case 8: rms_norm_kernel<8><<<grid, 64, 0, s>>>(x, w, out, rows, dim, eps); break;
    default: rms_norm_kernel<16><<<grid, 64, 0, s>>>(x, w, out, rows, dim, eps); break;
  }
  return hipGetLastError();
}

hipError_t launch_embed_mix(const int64_t* ids, const uint16_t* table, int64_t vocab,
                            const uint16_t* query, const uint16_t* score_w, float score_eps,
                            const uint16_t* out_norm_w, float out_eps, int64_t tokens, int dim,
                            uint16_t* rows_out, uint16_t* out_norm, float* zeros, int n_zeros,
                            hipStream_t s) {
  if (tokens == 0 && n_zeros == 0) return hipSuccess;
  const int waves = (dim + kDepthDimsPerWave - 1) / kDepthDimsPerWave;
  if (waves > kDepthMaxWaves) return hipErrorInvalidValue;
  // With no tokens, one workgroup that only zero-fills.
  const unsigned grid = static_cast<unsigned>(tokens > 0 ? tokens : 1);
  embed_mix_kernel<<<grid, kWave * waves, 0, s>>>(ids, table, vocab, query, score_w, score_eps,
                                                  out_norm_w, out_eps, tokens, dim, rows_out,
                                                  out_norm, zeros, n_zeros);
  return hipGetLastError();
}

hipError_t launch_depth_mix(const DepthSources& srcs, int n_sources,
                            const uint16_t* query, const uint16_t* score_w,
                            float score_eps, const uint16_t* out_norm_w,
                            float out_eps, int64_t tokens, int dim,
                            uint16_t* out_mix, uint16_t* out_norm, const CombineSource* comb,
                            const RouteOut* route, hipStream_t s, const PendingSum* pend) {
  if (tokens == 0) return hipSuccess;
  const int waves = (dim + kDepthDimsPerWave - 1) / kDepthDimsPerWave;
  if (waves > kDepthMaxWaves) return hipErrorInvalidValue;
  const CombineSource none{};
  const RouteOut no_route{};
  const CombineSource c = comb != nullptr ? *comb : none;
  const unsigned grid = static_cast<unsigned>(tokens);
  if (pend != nullptr) {  // with a route, never with a combine (both make the last source)
    if (route == nullptr || comb != nullptr || n_sources < 2) return hipErrorInvalidValue;
    return with_sources(n_sources, [&](auto ns) {
      if constexpr (decltype(ns)::value >= 2) {
        if (route->experts > 16)
          depth_mix_kernel<2, ns, kPendingHeads><<<grid, kWave * waves, 0, s>>>(
              srcs, query, score_w, score_eps, out_norm_w, out_eps, tokens, dim, out_mix,
              out_norm, none, *route, *pend);
        else
          depth_mix_kernel<1, ns, kPendingHeads><<<grid, kWave * waves, 0, s>>>(
              srcs, query, score_w, score_eps, out_norm_w, out_eps, tokens, dim, out_mix,
              out_norm, none, *route, *pend);
        return hipGetLastError();
      }
      return hipErrorInvalidValue;
    });
  }
  const PendingSum no_pend{};
  return with_sources(n_sources, [&](auto ns) {
    if (route == nullptr && comb == nullptr && tokens >= kDepthWaveMinTokens && waves <= 4) {
      const unsigned groups = static_cast<unsigned>(
          (tokens + kDepthWaveTokensPerGroup - 1) / kDepthWaveTokensPerGroup);
      auto wave_kernel = [&](auto nch) {
        depth_mix_wave_kernel<ns, nch><<<groups, kWave * kDepthWaveTokensPerGroup, 0, s>>>(
            srcs, query, score_w, score_eps, out_norm_w, out_eps, tokens, dim, out_mix,
            out_norm);
      };
      switch (waves) {
        case 1: wave_kernel(std::integral_constant<int, 1>{}); break;
        case 2: wave_kernel(std::integral_constant<int, 2>{}); break;
        case 3: wave_kernel(std::integral_constant<int, 3>{}); break;
        default: wave_kernel(std::integral_constant<int, 4>{}); break;
      }
      return hipGetLastError();
    }
    if (route != nullptr && route->experts > 16)
      depth_mix_kernel<2, ns><<<grid, kWave * waves, 0, s>>>(
          srcs, query, score_w, score_eps, out_norm_w, out_eps, tokens, dim, out_mix, out_norm,
          c, *route, no_pend);
    else if (route != nullptr)
      depth_mix_kernel<1, ns><<<grid, kWave * waves, 0, s>>>(
          srcs, query, score_w, score_eps, out_norm_w, out_eps, tokens, dim, out_mix, out_norm,
          c, *route, no_pend);
    else
      depth_mix_kernel<0, ns><<<grid, kWave * waves, 0, s>>>(
          srcs, query, score_w, score_eps, out_norm_w, out_eps, tokens, dim, out_mix, out_norm,
          c, no_route, no_pend);
    return hipGetLastError();
  });
}

}  // namespace parrot
