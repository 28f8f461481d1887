// The decode step's q|k|v projection of the local (GQA) layers, with its
// input's depth mix + RMSNorm and the RoPE of q and k, in one launch for up
// to 16 tokens.
//
// Reference semantics: h = attention_norm(depth_mix(sources)) (Block
// AttnRes, parrot/model.py:680-710, computed by depth_mix_core.h, so h has
// the depth-mix kernel's bits); q|k|v = h W^T rounded to bf16 (the bias-free
// nn.Linear maps, parrot/model.py:167-230); q and k rotated by RoPE at the
// device position in fp32 and rounded again (_apply_rope, parrot/model.py:
// 176-205, as rope_even / rope_odd apply it in every fused path here).  The
// projection's fp32 sums run in a different order than a library or MFMA
// GEMM, so its bf16 values may differ from those in the last place.
//
// Grid (N / 16 column blocks, tokens): workgroup (x, t) mixes token t's row
// into LDS (at dim 768 the fourth wavefront idles through the mix, see
// depth_mix_core.h) while its weight chunks are in flight, then each of its
// 16 DPP rows computes one column of q|k|v (decode_gemv.h).  Rotation
// partners (2i, 2i + 1) are adjacent DPP rows, one xor-16 shuffle apart.
#include "decode_gemv.h"
#include "depth_mix_core.h"

namespace parrot {

namespace {

constexpr int kQkvMaxDim = 1024;  // the mix holds a row with 4 wavefronts of 256 dims

__global__ __launch_bounds__(256) void decode_qkv_kernel(DecodeQkvArgs a) {
  __shared__ DepthMixLds mix_lds;
  __shared__ __attribute__((aligned(16))) uint16_t xs[kQkvMaxDim];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int j = tid >> 4, p = tid & 15;
  const int t = blockIdx.y;
  const int col = blockIdx.x * kGemvRows + j;
  const int K = a.dim;
  const int d = a.head_dim;
  const int head = col / d;
  const int w = col - head * d;
  const int H = a.heads, Hk = a.kv_heads;

  uint4 wr[kGemvMaxChunks];
  load_row_chunks(a.w, col, K, p, wr);
  const int pos = min(max(*a.position, 0), a.max_positions - 1);
  const int64_t ti = static_cast<int64_t>(pos) * (d / 2) + w / 2;
  const float rc = a.cos_t[ti], rs = a.sin_t[ti];

  if (a.mix.n_sources > 0) {
    // Token t's input row: depth mix + RMSNorm of its sources into LDS, every
    // load issued before the first wait (lanes past the row read chunk 0 and
    // are zeroed, unread slots read source 0 and are zeroed).
    const DecodeMix& m = a.mix;
    const int chunks = K >> 2;
    const bool has = tid < chunks;
    const int ic = has ? tid : 0;
    const int64_t base = static_cast<int64_t>(t) * chunks;
    uint2 v[kMaxDepthSources];
#pragma unroll
    for (int s = 0; s < kMaxDepthSources; ++s)
      v[s] = reinterpret_cast<const uint2*>(m.srcs.src[s])[base + ic];
    const uint2 q = reinterpret_cast<const uint2*>(m.query)[ic];
    const uint2 g = reinterpret_cast<const uint2*>(m.score_w)[ic];
    const uint2 g_out = reinterpret_cast<const uint2*>(m.out_w)[ic];
#pragma unroll
    for (int s = 0; s < kMaxDepthSources; ++s)
      if (!has || s >= m.n_sources) v[s] = make_uint2(0u, 0u);
    const int waves = (K + kDepthDimsPerWave - 1) / kDepthDimsPerWave;
    const uint2 mixed =
        depth_mix_chunk(v, q, g, has, m.n_sources, waves, wave, lane, K, m.score_eps, mix_lds);
    const uint2 o =
        depth_mix_norm_chunk(mixed, g_out, has, waves, wave, lane, K, m.out_eps, mix_lds);
    if (has) reinterpret_cast<uint2*>(xs)[tid] = o;
  } else {
    for (int i = tid; i < K / 8; i += 256)
      reinterpret_cast<uint4*>(xs)[i] =
          reinterpret_cast<const uint4*>(a.x + static_cast<int64_t>(t) * K)[i];
  }
  __syncthreads();

  const uint4* xt = reinterpret_cast<const uint4*>(xs);
  const int nch = K / 128;
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < kGemvMaxChunks; ++c)
    if (c < nch) acc += dot_bf16x8(wr[c], xt[c * 16 + p]);
  acc = row16_sum(acc);
  // Round as the projection output, then rotate with the partner column.
  const float self = bf16_to_f32(f32_to_bf16(acc));
  const float other = __shfl_xor(self, 16);
  float val = self;
  if (head < H + Hk)
    val = (j & 1) ? rope_odd(other, self, rc, rs) : rope_even(self, other, rc, rs);
  if (p == 0) {
    const uint16_t bits = f32_to_bf16(val);
    if (head < H)
      a.q[(static_cast<int64_t>(t) * H + head) * d + w] = bits;
    else if (head < H + Hk)
      a.k[(static_cast<int64_t>(t) * Hk + head - H) * d + w] = bits;
    else
      a.v[(static_cast<int64_t>(t) * Hk + head - H - Hk) * d + w] = bits;
  }
}

}  // namespace

int decode_qkv_max_dim() { return kQkvMaxDim; }

hipError_t launch_decode_qkv(const DecodeQkvArgs& a, hipStream_t s) {
  if (a.tokens == 0) return hipSuccess;
  const int n = (a.heads + 2 * a.kv_heads) * a.head_dim;
  decode_qkv_kernel<<<dim3(n / kGemvRows, a.tokens), 256, 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace parrot
