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
#include "common.h"

namespace parrot {

namespace {

constexpr int kRowsPerBlock = 1;  // one row per 64-lane workgroup

// y = bf16((x * rsqrt(mean(x^2) + eps)) * w)        (parrot/model.py:125-127)
template <int MAXC>
__global__ __launch_bounds__(64) void rms_norm_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ out, int64_t rows, int dim, float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;  // uniform per wavefront
  const int chunks = dim >> 2;
  const uint2* xr = reinterpret_cast<const uint2*>(x + row * dim);
  const uint2* wr = reinterpret_cast<const uint2*>(w);
  uint2* yr = reinterpret_cast<uint2*>(out + row * dim);
  uint2 v[MAXC];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int i = lane + c * kWave;
    v[c] = i < chunks ? xr[i] : make_uint2(0u, 0u);
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
      const uint2 g = wr[i];
      uint2 o;
      o.x = pack_bf16x2(lo_bf16(v[c].x) * r * lo_bf16(g.x), hi_bf16(v[c].x) * r * hi_bf16(g.x));
      o.y = pack_bf16x2(lo_bf16(v[c].y) * r * lo_bf16(g.y), hi_bf16(v[c].y) * r * hi_bf16(g.y));
      yr[i] = o;
    }
  }
}

// Block AttnRes: score_s = <rmsnorm_w(v_s), q>, alpha = softmax_s(score),
// mix = bf16(sum_s alpha_s v_s); optionally y = rmsnorm_out(mix).
// One wavefront per token.  Every source row is loaded up front (all loads in
// flight together) and kept in registers through the scores and the mix.
template <int MAXC>
__global__ __launch_bounds__(64) void depth_mix_kernel(
    DepthSources srcs, int n_sources, const uint16_t* __restrict__ query,
    const uint16_t* __restrict__ score_w, float score_eps,
    const uint16_t* __restrict__ out_w, float out_eps, int64_t tokens, int dim,
    uint16_t* __restrict__ out_mix, uint16_t* __restrict__ out_norm) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t tok = blockIdx.x;
  if (tok >= tokens) return;
  const int chunks = dim >> 2;
  const int64_t base = tok * (dim >> 2);

  // Combined score weight w_d * q_d for this lane's elements.
  float wq[MAXC][4];
  {
    const uint2* q2 = reinterpret_cast<const uint2*>(query);
    const uint2* w2 = reinterpret_cast<const uint2*>(score_w);
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const int i = lane + c * kWave;
      uint2 q = i < chunks ? q2[i] : make_uint2(0u, 0u);
      uint2 g = i < chunks ? w2[i] : make_uint2(0u, 0u);
      wq[c][0] = lo_bf16(q.x) * lo_bf16(g.x);
      wq[c][1] = hi_bf16(q.x) * hi_bf16(g.x);
      wq[c][2] = lo_bf16(q.y) * lo_bf16(g.y);
      wq[c][3] = hi_bf16(q.y) * hi_bf16(g.y);
    }
  }

  // Every source row stays in registers from its load to the mix (the
  // source loop is unrolled over the maximum count, guarded by n_sources),
  // so a token needs no LDS and no barrier and occupancy is set by VGPRs.
  uint2 v[kMaxDepthSources][MAXC];
#pragma unroll
  for (int s = 0; s < kMaxDepthSources; ++s) {
    if (s < n_sources) {
      const uint2* src = reinterpret_cast<const uint2*>(srcs.src[s]) + base;
#pragma unroll
      for (int c = 0; c < MAXC; ++c) {
        const int i = lane + c * kWave;
        v[s][c] = i < chunks ? src[i] : make_uint2(0u, 0u);
      }
    }
  }
  // Per-lane partial sums of every source, then all 2S wavefront reductions
  // back to back so their latencies overlap.  The reductions leave every
  // lane with the same totals, so the scores are wavefront-uniform.
  float ss[kMaxDepthSources], dq[kMaxDepthSources];
#pragma unroll
  for (int s = 0; s < kMaxDepthSources; ++s) {
    ss[s] = 0.0f;
    dq[s] = 0.0f;
    if (s < n_sources) {
#pragma unroll
      for (int c = 0; c < MAXC; ++c) {
        const float e0 = lo_bf16(v[s][c].x), e1 = hi_bf16(v[s][c].x);
        const float e2 = lo_bf16(v[s][c].y), e3 = hi_bf16(v[s][c].y);
        ss[s] += e0 * e0 + e1 * e1 + e2 * e2 + e3 * e3;
        dq[s] += e0 * wq[c][0] + e1 * wq[c][1] + e2 * wq[c][2] + e3 * wq[c][3];
      }
    }
  }
  float score[kMaxDepthSources];
  float mx = -INFINITY;
#pragma unroll
  for (int s = 0; s < kMaxDepthSources; ++s) {
    score[s] = -INFINITY;
    if (s < n_sources) {
      score[s] = wave_sum(dq[s]) * rsqrtf(wave_sum(ss[s]) / static_cast<float>(dim) + score_eps);
      mx = fmaxf(mx, score[s]);
    }
  }
  float denom = 0.0f;
#pragma unroll
  for (int s = 0; s < kMaxDepthSources; ++s)
    if (s < n_sources) denom += __expf(score[s] - mx);
  const float inv = 1.0f / denom;

  // Keep only the packed bf16 rows live across the reductions: without this
  // the compiler holds the unpacked fp32 copies (twice the registers, half
  // the occupancy) to reuse them in the mix.
#pragma unroll
  for (int s = 0; s < kMaxDepthSources; ++s)
#pragma unroll
    for (int c = 0; c < MAXC; ++c) asm volatile("" : "+v"(v[s][c].x), "+v"(v[s][c].y));

  float acc[MAXC][4];
#pragma unroll
  for (int c = 0; c < MAXC; ++c) acc[c][0] = acc[c][1] = acc[c][2] = acc[c][3] = 0.0f;
#pragma unroll
  for (int s = 0; s < kMaxDepthSources; ++s) {
    if (s < n_sources) {
      const float a = __expf(score[s] - mx) * inv;
#pragma unroll
      for (int c = 0; c < MAXC; ++c) {
        acc[c][0] += a * lo_bf16(v[s][c].x);
        acc[c][1] += a * hi_bf16(v[s][c].x);
        acc[c][2] += a * lo_bf16(v[s][c].y);
        acc[c][3] += a * hi_bf16(v[s][c].y);
      }
    }
  }
  uint2 mixed[MAXC];
  float ss_out = 0.0f;
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    mixed[c].x = pack_bf16x2(acc[c][0], acc[c][1]);
    mixed[c].y = pack_bf16x2(acc[c][2], acc[c][3]);
    const float r0 = lo_bf16(mixed[c].x), r1 = hi_bf16(mixed[c].x);
    const float r2 = lo_bf16(mixed[c].y), r3 = hi_bf16(mixed[c].y);
    ss_out += r0 * r0 + r1 * r1 + r2 * r2 + r3 * r3;
  }
  if (out_mix != nullptr) {
    uint2* dst = reinterpret_cast<uint2*>(out_mix) + base;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const int i = lane + c * kWave;
      if (i < chunks) dst[i] = mixed[c];
    }
  }
  if (out_norm != nullptr) {
    ss_out = wave_sum(ss_out);
    const float r = rsqrtf(ss_out / static_cast<float>(dim) + out_eps);
    const uint2* w2 = reinterpret_cast<const uint2*>(out_w);
    uint2* dst = reinterpret_cast<uint2*>(out_norm) + base;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const int i = lane + c * kWave;
      if (i < chunks) {
        const uint2 g = w2[i];
        uint2 o;
        o.x = pack_bf16x2(lo_bf16(mixed[c].x) * r * lo_bf16(g.x),
                          hi_bf16(mixed[c].x) * r * hi_bf16(g.x));
        o.y = pack_bf16x2(lo_bf16(mixed[c].y) * r * lo_bf16(g.y),
                          hi_bf16(mixed[c].y) * r * hi_bf16(g.y));
        dst[i] = o;
      }
    }
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

hipError_t launch_depth_mix(const DepthSources& srcs, int n_sources,
                            const uint16_t* query, const uint16_t* score_w,
                            float score_eps, const uint16_t* out_norm_w,
                            float out_eps, int64_t tokens, int dim,
                            uint16_t* out_mix, uint16_t* out_norm, hipStream_t s) {
  if (tokens == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((tokens + kRowsPerBlock - 1) / kRowsPerBlock));
#define PARROT_DEPTH(C)                                                          \
  depth_mix_kernel<C><<<grid, 64, 0, s>>>(srcs, n_sources, query, score_w,     \
                                           score_eps, out_norm_w, out_eps,      \
                                           tokens, dim, out_mix, out_norm)
  switch (chunk_bucket(dim)) {
    case 1: PARROT_DEPTH(1); break;
    case 2: PARROT_DEPTH(2); break;
    case 3: PARROT_DEPTH(3); break;
    case 4: PARROT_DEPTH(4); break;
    default: PARROT_DEPTH(8); break;
  }
#undef PARROT_DEPTH
  return hipGetLastError();
}

}  // namespace parrot
