// One token's Block AttnRes mix and output RMSNorm, shared by the depth-mix
// kernel (norm.hip) and the decode MoE that mixes its own input
// (decode_moe.hip), so both produce the same bits.
//
// Reference: Block AttnRes (parrot/model.py:680-710; parrot/metal_moe.py:
// 419-477): score_s = <rmsnorm_w(v_s), q>, alpha = softmax_s(score),
// mix = bf16(sum_s alpha_s v_s), then y = rmsnorm_out(mix) rounded to bf16.
//
// Layout: `waves` wavefronts hold the row, 256 dims each; lane l of
// wavefront w owns the 4 consecutive dims of chunk i = 64 w + l (`has` when
// i < dim / 4).  Wavefronts past `waves` of a larger workgroup take part in
// the barriers with has == false.  Per-source sums (squares and query dot)
// are wavefront sums (in wave_total_lane63's order) combined across the
// wavefronts through LDS in wavefront order, so every wavefront derives the
// same scores; the output norm's sum of squares likewise.
#pragma once
#include <type_traits>

#include "common.h"

namespace parrot {

constexpr int kDepthDimsPerWave = 256;
constexpr int kDepthMaxWaves = 8;  // dim <= 2048

// A wavefront sum with wave_sum's order, in lane 63 only (where the depth
// mix writes its partials from): the 16-lane row sums r0..r3 by the same DPP
// steps, then ((r0 + r1) + r2) + r3 by three row broadcasts masked to rows
// 1, 2 and 3 in turn (the other rows add -0, the exact identity).  No
// readlane: the totals stay in VGPRs.
__device__ __forceinline__ float wave_total_lane63(float v) {
  constexpr int kNegZero = static_cast<int>(0x80000000u);
  v += dpp<0xb1>(v);
  v += dpp<0x4e>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  v += __int_as_float(__builtin_amdgcn_update_dpp(kNegZero, __float_as_int(v), 0x142, 0x2, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(kNegZero, __float_as_int(v), 0x142, 0x4, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(kNegZero, __float_as_int(v), 0x142, 0x8, 0xf, false));
  return v;
}

struct __attribute__((aligned(16))) DepthMixLds {
  // Per (wavefront, DPP row): the row sums of every per-source quantity.
  float rows[kDepthMaxWaves][4][2 * kMaxDepthSources];
  float part_out[kDepthMaxWaves];
};

// The mixing weights alpha_s (wave-uniform) from the per-quantity totals in
// lanes 0 .. 2 NS - 1 (lane 2s: source s's sum of squares, lane 2s + 1: its
// query dot): score_s = dot_s * rsqrt(ss_s / dim + eps), alpha = softmax over
// the sources in order.  Lane 2s evaluates its own score and exponential (one
// division, one rsqrt and one exp per lane instead of one per source in
// every lane); the maximum and the denominator are taken over the scores
// read back in source order, so every value is what the per-source loop
//   mx = max_s score_s; denom = sum_s exp(score_s - mx); alpha_s =
//   exp(score_s - mx) / denom (as exp(...) * (1 / denom))
// gives, bit for bit.
template <int NS>
__device__ __forceinline__ void depth_mix_weights(float tot, int dim, float score_eps,
                                                  float (&alpha)[NS]) {
  const float dot = dpp<0xb1>(tot);  // lane 2s: lane 2s + 1's total
  const float score = dot * rsqrtf(tot / static_cast<float>(dim) + score_eps);
  float mx = -INFINITY;
#pragma unroll
  for (int s = 0; s < NS; ++s)
    mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(score), 2 * s)));
  const float e = __expf(score - mx);
  float denom = 0.0f;
#pragma unroll
  for (int s = 0; s < NS; ++s)
    denom += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), 2 * s));
  const float a = e * (1.0f / denom);
#pragma unroll
  for (int s = 0; s < NS; ++s)
    alpha[s] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 2 * s));
}

// The mix of this lane's chunk as packed bf16 over NS sources (a compile-time
// count: the loops below then hold only the sources read, which at one to
// five sources halves the instructions of a runtime count with guards).
// v: the chunk of each source (zeros for lanes past the row); q, g: the chunk
// of the query and of the score norm's weight.  Contains one barrier.
template <int NS>
__device__ __forceinline__ uint2 depth_mix_chunk(const uint2 (&v)[kMaxDepthSources], uint2 q,
                                                 uint2 g, bool has, int waves, int wave, int lane,
                                                 int dim, float score_eps, DepthMixLds& sh) {
  static_assert(NS >= 1 && NS <= kMaxDepthSources, "one to kMaxDepthSources sources");
  float wq[4] = {0.f, 0.f, 0.f, 0.f};
  if (has) {
    wq[0] = lo_bf16(q.x) * lo_bf16(g.x);
    wq[1] = hi_bf16(q.x) * hi_bf16(g.x);
    wq[2] = lo_bf16(q.y) * lo_bf16(g.y);
    wq[3] = hi_bf16(q.y) * hi_bf16(g.y);
  }

  // Per-source partial sums, each summed over its 16-lane DPP row by
  // wave_total_lane63's first four steps (row_sum: every lane of row r then
  // holds the row's sum r_r); lane 0 of each row stores the row sums.
  float ss[NS], dq[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const float e0 = lo_bf16(v[s].x), e1 = hi_bf16(v[s].x);
    const float e2 = lo_bf16(v[s].y), e3 = hi_bf16(v[s].y);
    ss[s] = e0 * e0 + e1 * e1 + e2 * e2 + e3 * e3;
    dq[s] = e0 * wq[0] + e1 * wq[1] + e2 * wq[2] + e3 * wq[3];
  }
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    ss[s] = row_sum(ss[s]);
    dq[s] = row_sum(dq[s]);
  }
  if ((lane & 15) == 0) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      sh.rows[wave][lane >> 4][2 * s] = ss[s];
      sh.rows[wave][lane >> 4][2 * s + 1] = dq[s];
    }
  }
  __syncthreads();

  // Lane 2s (+1) of every wavefront adds, per wavefront, ((r_0 + r_1) + r_2)
  // + r_3 (the wavefront total of wave_total_lane63, whose three row
  // broadcasts would cost three instructions per quantity), then the
  // wavefront totals in wavefront order; the totals are read back as
  // wave-uniform values.  The loop bounds are compile-time (uniform guards
  // inside), so the LDS reads go out together.
  float tot = 0.0f;
  if (lane < 2 * NS) {
#pragma unroll
    for (int w = 0; w < kDepthMaxWaves; ++w)
      if (w < waves)
        tot += ((sh.rows[w][0][lane] + sh.rows[w][1][lane]) + sh.rows[w][2][lane]) +
               sh.rows[w][3][lane];
  }
  float alpha[NS];
  depth_mix_weights<NS>(tot, dim, score_eps, alpha);

  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    acc[0] += alpha[s] * lo_bf16(v[s].x);
    acc[1] += alpha[s] * hi_bf16(v[s].x);
    acc[2] += alpha[s] * lo_bf16(v[s].y);
    acc[3] += alpha[s] * hi_bf16(v[s].y);
  }
  uint2 mixed;
  mixed.x = pack_bf16x2(acc[0], acc[1]);
  mixed.y = pack_bf16x2(acc[2], acc[3]);
  return mixed;
}

// The output RMSNorm of the mixed row, this lane's chunk as packed bf16
// (g_out: the chunk of the norm's weight).  Contains one barrier.
__device__ __forceinline__ uint2 depth_mix_norm_chunk(uint2 mixed, uint2 g_out, bool has,
                                                      int waves, int wave, int lane, int dim,
                                                      float out_eps, DepthMixLds& sh) {
  const float r0 = lo_bf16(mixed.x), r1 = hi_bf16(mixed.x);
  const float r2 = lo_bf16(mixed.y), r3 = hi_bf16(mixed.y);
  const float sso = wave_total_lane63(has ? r0 * r0 + r1 * r1 + r2 * r2 + r3 * r3 : 0.0f);
  if (lane == 63) sh.part_out[wave] = sso;
  __syncthreads();
  float total = sh.part_out[0];
#pragma unroll
  for (int w = 1; w < kDepthMaxWaves; ++w)
    if (w < waves) total += sh.part_out[w];
  const float r = rsqrtf(total / static_cast<float>(dim) + out_eps);
  uint2 o;
  o.x = pack_bf16x2(r0 * r * lo_bf16(g_out.x), r1 * r * hi_bf16(g_out.x));
  o.y = pack_bf16x2(r2 * r * lo_bf16(g_out.y), r3 * r * hi_bf16(g_out.y));
  return o;
}

// Decode kernels that mix their own input row (one token per workgroup,
// lane chunk i = threadIdx.x): decode_mix_load issues the loads of the
// chunk (the NS sources; lanes past the row read chunk 0) without waiting
// for them, so a kernel can issue its weight loads behind them;
// decode_mix_row zeroes lanes past the row, then mixes and normalises (two
// barriers).
struct DecodeMixLoads {
  uint2 v[kMaxDepthSources];
  uint2 q, g, g_out;
};

template <int NS>
__device__ __forceinline__ void decode_mix_load(const DecodeMix& m, int64_t base, int ic,
                                                DecodeMixLoads& l) {
#pragma unroll
  for (int s = 0; s < NS; ++s) l.v[s] = reinterpret_cast<const uint2*>(m.srcs.src[s])[base + ic];
  l.q = reinterpret_cast<const uint2*>(m.query)[ic];
  l.g = reinterpret_cast<const uint2*>(m.score_w)[ic];
  l.g_out = reinterpret_cast<const uint2*>(m.out_w)[ic];
}

template <int NS>
__device__ __forceinline__ uint2 decode_mix_row(const DecodeMix& m, DecodeMixLoads& l, bool has,
                                                int wave, int lane, int dim, DepthMixLds& sh) {
#pragma unroll
  for (int s = 0; s < NS; ++s)
    if (!has) l.v[s] = make_uint2(0u, 0u);
  const int waves = (dim + kDepthDimsPerWave - 1) / kDepthDimsPerWave;
  const uint2 mixed =
      depth_mix_chunk<NS>(l.v, l.q, l.g, has, waves, wave, lane, dim, m.score_eps, sh);
  return depth_mix_norm_chunk(mixed, l.g_out, has, waves, wave, lane, dim, m.out_eps, sh);
}

// Calls `launch` with std::integral_constant<int, n> for a source count n
// in 1 .. kMaxDepthSources (the kernels' NS); other counts are rejected.
template <typename F>
__host__ hipError_t with_sources(int n, F&& launch) {
  static_assert(kMaxDepthSources == 9, "the cases below name every count");
  switch (n) {
    case 1: return launch(std::integral_constant<int, 1>{});
    case 2: return launch(std::integral_constant<int, 2>{});
    case 3: return launch(std::integral_constant<int, 3>{});
    case 4: return launch(std::integral_constant<int, 4>{});
    case 5: return launch(std::integral_constant<int, 5>{});
    case 6: return launch(std::integral_constant<int, 6>{});
    case 7: return launch(std::integral_constant<int, 7>{});
    case 8: return launch(std::integral_constant<int, 8>{});
    case 9: return launch(std::integral_constant<int, 9>{});
    default: return hipErrorInvalidValue;
  }
}

}  // namespace parrot
