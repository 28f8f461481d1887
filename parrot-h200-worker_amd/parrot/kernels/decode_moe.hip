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
//   decode_up_kernel   grid (max(H, Hs) / 16 slices, 3T slots): slot 2t + k
//       is token t's k-th routed expert, slot 2T + t token t's shared expert.
//       A routed workgroup recomputes its token's router logits and top-2
//       (every workgroup of a token does the same arithmetic in the same
//       order, so they agree), then one 16-column slice of SwiGLU.  Given the
//       MoE input's depth sources instead of the input, every workgroup first
//       mixes and normalises its token's row itself (depth_mix_core.h, the
//       depth-mix kernel's arithmetic), which saves that kernel's launch.
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

// LDS layout of decode_up_kernel: the token row (dim bf16, 16-byte aligned),
// then the router weights (experts x dim bf16, padded to whole 1 KB groups).
// The router weights are staged only up to kRouterLdsBudget bytes (E = 32 at
// dim 768); past it the router reads them from memory as before.
constexpr size_t kRouterLdsBudget = 48 * 1024;
__host__ __device__ __forceinline__ int router_lds_offset(int dim) { return (dim + 7) / 8 * 8; }
__host__ __device__ __forceinline__ bool router_in_lds(int dim, int experts) {
  return static_cast<size_t>(experts) * dim * sizeof(uint16_t) <= kRouterLdsBudget;
}
__host__ __device__ __forceinline__ size_t decode_up_lds_bytes(int dim, int experts) {
  const size_t chunks = router_in_lds(dim, experts) ? static_cast<size_t>(experts) * dim / 8 : 0;
  return (router_lds_offset(dim) + (chunks + kWave - 1) / kWave * kWave * 8) * sizeof(uint16_t);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float(uint32_t(v) << 16); }

__device__ __forceinline__ float dot8(uint4 a, uint4 b) {
  return lo_bf16(a.x) * lo_bf16(b.x) + hi_bf16(a.x) * hi_bf16(b.x) +
         lo_bf16(a.y) * lo_bf16(b.y) + hi_bf16(a.y) * hi_bf16(b.y) +
         lo_bf16(a.z) * lo_bf16(b.z) + hi_bf16(a.z) * hi_bf16(b.z) +
         lo_bf16(a.w) * lo_bf16(b.w) + hi_bf16(a.w) * hi_bf16(b.w);
}

// Router logits of token t for all experts into lg[0..E), then top-2.
// Thread (e = tid / 8, part = tid % 8) sums the dim / 8 columns of its part;
// the 8 parts of an expert are added in a fixed order by DPP (xor 1, xor 2,
// half-row mirror) inside 8-lane groups.
__device__ __forceinline__ void route_token(const uint16_t* x_row, const uint16_t* wr,
                                            const float* bias, int dim, int experts, float* lg,
                                            int* sel, float* sel_w) {
  const int tid = threadIdx.x;
  const int e = tid >> 3, part = tid & 7;
  float acc = 0.0f;
  if (e < experts) {
    const int n = dim / 64;  // 16-byte chunks per part (dim % 64 == 0)
    const uint4* xa = reinterpret_cast<const uint4*>(x_row) + part * n;
    const uint4* wa = reinterpret_cast<const uint4*>(wr + static_cast<int64_t>(e) * dim) + part * n;
    for (int c0 = 0; c0 < n; c0 += 12) {  // 12 chunks (dim 768) in flight at once
      uint4 xv[12], wv[12];
#pragma unroll
      for (int u = 0; u < 12; ++u) {
        const int c = min(c0 + u, n - 1);
        xv[u] = xa[c];
        wv[u] = wa[c];
      }
#pragma unroll
      for (int u = 0; u < 12; ++u)
        if (c0 + u < n) acc += dot8(xv[u], wv[u]);
    }
  }
  acc += dpp<0xb1>(acc);
  acc += dpp<0x4e>(acc);
  acc += dpp<0x141>(acc);
  if (part == 0 && e < experts) lg[e] = acc + (bias != nullptr ? bias[e] : 0.0f);
  __syncthreads();
  if (tid < 16) {
    int first, second;
    float vb, vr;
    row_top2(tid < experts ? lg[tid] : 0.0f, tid + 16 < experts ? lg[tid + 16] : 0.0f, experts,
             first, second, vb, vr);
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

__global__ __launch_bounds__(256) void decode_up_kernel(
    const uint16_t* __restrict__ x, DecodeMix mix, const uint16_t* __restrict__ wr,
    const float* __restrict__ bias, int tokens, int dim, int experts, int hidden_dim,
    int shared_dim, int hstride, const uint16_t* __restrict__ gate_up,
    const uint16_t* __restrict__ shared_gate_up, uint16_t* __restrict__ hidden,
    int64_t* __restrict__ indices, float* __restrict__ weights) {
  __shared__ float lg[kMaxExperts];
  __shared__ int sel[2];
  __shared__ float sel_w[2];
  __shared__ float part[4][4][32];  // [wave][k chunk][gate 16 | up 16]
  __shared__ DepthMixLds mix_lds;
  // The slot's token row [dim], then (routed slots) the router weights
  // [experts, dim] at element offset xs_elems.
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int slot = blockIdx.y;
  const int slice = blockIdx.x;
  const bool shared = slot >= 2 * tokens;
  const int H = shared ? shared_dim : hidden_dim;
  if (slice * 16 >= H) return;  // uniform
  const int t0 = shared ? slot - 2 * tokens : slot >> 1;  // the slot's token
  const bool staged = router_in_lds(dim, experts);  // uniform
  uint16_t* wr_s = xs + router_lds_offset(dim);
  if (!shared && staged) {
    // Router weights straight into LDS (16 bytes per lane, a wavefront's
    // 64 lanes fill 1 KB), issued before the input mix so they arrive with
    // its sources instead of after it; lanes past the end reread the last
    // chunk into the region's padding.
    const int chunks = experts * dim / 8;
    for (int g = wave; g * kWave < chunks; g += 4) {
      const int c = min(g * kWave + lane, chunks - 1);
      __builtin_amdgcn_global_load_lds(wr + static_cast<int64_t>(c) * 8,
                                       (lds_void_t*)(wr_s + g * kWave * 8), 16, 0, 0);
    }
  }
  if (mix.n_sources > 0) {
    // The token's input row: depth mix + RMSNorm of its sources into LDS,
    // every load issued before the first wait (lanes past the row read
    // chunk 0 and are zeroed, unread slots read source 0 and are zeroed).
    const int chunks = dim >> 2;
    const bool has = tid < chunks;
    const int ic = has ? tid : 0;
    const int64_t base = static_cast<int64_t>(t0) * chunks;
    uint2 v[kMaxDepthSources];
#pragma unroll
    for (int s = 0; s < kMaxDepthSources; ++s)
      v[s] = reinterpret_cast<const uint2*>(mix.srcs.src[s])[base + ic];
    const uint2 q = reinterpret_cast<const uint2*>(mix.query)[ic];
    const uint2 g = reinterpret_cast<const uint2*>(mix.score_w)[ic];
    const uint2 g_out = reinterpret_cast<const uint2*>(mix.out_w)[ic];
    if (mix.pend != nullptr) {
      // The pending last source: this chunk's contributions summed over the
      // lanes in order (the loads of up to 8 lanes in flight at once),
      // rounded, then added to the base with a second rounding; the
      // token's first routed workgroup of slice 0 stores the resolved row.
      const float4* pc = reinterpret_cast<const float4*>(mix.pend) +
                         static_cast<int64_t>(t0) * mix.pend_lanes * chunks + ic;
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      for (int l0 = 0; l0 < mix.pend_lanes; l0 += 8) {
        float4 c[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          c[u] = pc[static_cast<int64_t>(min(l0 + u, mix.pend_lanes - 1)) * chunks];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (l0 + u < mix.pend_lanes) {
            acc[0] += c[u].x;
            acc[1] += c[u].y;
            acc[2] += c[u].z;
            acc[3] += c[u].w;
          }
        }
      }
      uint2 r;
      r.x = pack_bf16x2(acc[0], acc[1]);
      r.y = pack_bf16x2(acc[2], acc[3]);
      if (mix.pend_base != nullptr) {
        const uint2 pb = reinterpret_cast<const uint2*>(mix.pend_base)[base + ic];
        r.x = pack_bf16x2(lo_bf16(pb.x) + lo_bf16(r.x), hi_bf16(pb.x) + hi_bf16(r.x));
        r.y = pack_bf16x2(lo_bf16(pb.y) + lo_bf16(r.y), hi_bf16(pb.y) + hi_bf16(r.y));
      }
#pragma unroll
      for (int s = 0; s < kMaxDepthSources; ++s)
        if (s == mix.n_sources - 1) v[s] = r;
      if (has && !shared && slice == 0 && (slot & 1) == 0)
        reinterpret_cast<uint2*>(mix.pend_out)[base + ic] = r;
    }
#pragma unroll
    for (int s = 0; s < kMaxDepthSources; ++s)
      if (!has || s >= mix.n_sources) v[s] = make_uint2(0u, 0u);
    const int waves = (dim + kDepthDimsPerWave - 1) / kDepthDimsPerWave;
    const uint2 mixed = depth_mix_chunk(v, q, g, has, mix.n_sources, waves, wave, lane, dim,
                                        mix.score_eps, mix_lds);
    const uint2 o = depth_mix_norm_chunk(mixed, g_out, has, waves, wave, lane, dim, mix.out_eps,
                                         mix_lds);
    if (has) reinterpret_cast<uint2*>(xs)[tid] = o;
  } else {
    // The slot's activation row, staged in LDS as bf16; these loads are in
    // flight together with the router's (the barrier in route_token, or the
    // one below, orders them before use).
    for (int i = tid; i < dim / 8; i += 256)
      reinterpret_cast<uint4*>(xs)[i] =
          reinterpret_cast<const uint4*>(x + static_cast<int64_t>(t0) * dim)[i];
  }
  const uint16_t* w;
  if (shared) {
    __syncthreads();
    w = shared_gate_up;
  } else {
    // The router reads the row from LDS once it is mixed there, and its
    // weights from LDS once their direct-to-LDS loads have landed.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    route_token(mix.n_sources > 0 ? xs : x + static_cast<int64_t>(t0) * dim,
                staged ? wr_s : wr, bias, dim, experts, lg, sel, sel_w);
    const int k = slot & 1;
    if (slice == 0 && k == 0 && tid < 2) {
      indices[2 * t0 + tid] = sel[tid];
      weights[2 * t0 + tid] = sel_w[tid];
    }
    w = gate_up + static_cast<int64_t>(sel[k]) * 2 * hidden_dim * dim;
  }
  // Packed rows [32 slice, 32 slice + 32): gate group 2 slice, up group
  // 2 slice + 1; block (g, s) at ((g * ksteps) + s) KB.  Wavefront w takes
  // k steps w, w + 4, ..., the weight fragments of up to 8 of them in
  // flight at once.
  const int ksteps = dim / 32;
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
    const int rr = tid;
    float gs = 0.0f, us = 0.0f;
#pragma unroll
    for (int wv = 0; wv < 4; ++wv)
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        gs += part[wv][cc][rr];
        us += part[wv][cc][16 + rr];
      }
    const int64_t row = shared ? 2 * tokens + t0 : slot;
    hidden[row * hstride + slice * 16 + rr] = f32_to_bf16(swiglu(gs, us));
  }
}

__global__ __launch_bounds__(256) void decode_down_kernel(
    const uint16_t* __restrict__ hidden, int tokens, int dim, int hidden_dim, int shared_dim,
    int hstride, const int64_t* __restrict__ indices, const float* __restrict__ weights,
    const uint16_t* __restrict__ down, const uint16_t* __restrict__ shared_down,
    const uint16_t* __restrict__ addend, uint16_t* __restrict__ out) {
  __shared__ float part[3][4][4][16];  // [contribution][wave][k chunk][column]
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int slice = blockIdx.x;  // output columns [16 slice, 16 slice + 16)
  const int t = blockIdx.y;
  const int c = lane >> 4;
  // Contribution 0 / 1: routed slot 2t + k (expert indices[2t + k], K = H);
  // contribution 2: the shared expert (K = Hs).  Wavefront w takes k steps
  // w, w + 4, ...; the loads of up to 4 steps of all three are issued
  // before any arithmetic.
  const uint4* wb[3];
  const uint16_t* hrow[3];
  int ks[3];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    const bool sh = q == 2;
    ks[q] = (sh ? shared_dim : hidden_dim) / 32;
    const uint16_t* w = sh ? shared_down
                           : down + indices[2 * t + q] * static_cast<int64_t>(dim) * hidden_dim;
    wb[q] = reinterpret_cast<const uint4*>(w) + slice * ks[q] * 64 + lane;
    hrow[q] = hidden + (sh ? 2 * tokens + t : 2 * t + q) * static_cast<int64_t>(hstride) + c * 8;
  }
  float acc[3] = {0.0f, 0.0f, 0.0f};
  const int kmax = max(ks[0], ks[2]);
  for (int s0 = wave; s0 < kmax; s0 += 16) {
    uint4 wv[3][4], hv[3][4];
#pragma unroll
    for (int q = 0; q < 3; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int st = min(s0 + 4 * i, ks[q] - 1);
        wv[q][i] = wb[q][st * 64];
        hv[q][i] = *reinterpret_cast<const uint4*>(hrow[q] + st * 32);
      }
#pragma unroll
    for (int q = 0; q < 3; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (s0 + 4 * i < ks[q]) acc[q] += dot8(wv[q][i], hv[q][i]);
  }
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
    // combine_kernel's order: shared, then the two weighted routed rows.
    const float v = (y[2] + weights[2 * t] * y[0]) + weights[2 * t + 1] * y[1];
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
  decode_up_kernel<<<dim3(hstride / 16, 3 * tokens), 256, decode_up_lds_bytes(dim, experts), s>>>(
      x, mix != nullptr ? *mix : none, router_w, bias, tokens, dim, experts, hidden_dim,
      shared_dim, hstride, w.gate_up, w.shared_gate_up, hidden, indices, weights);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  decode_down_kernel<<<dim3(dim / 16, tokens), 256, 0, s>>>(
      hidden, tokens, dim, hidden_dim, shared_dim, hstride, indices, weights, w.down,
      w.shared_down, addend, out);
  return hipGetLastError();
}

}  // namespace parrot
