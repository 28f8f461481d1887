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

// Loads go out in the order they are needed, each batch behind the one
// before with no wait between: the kernel arguments (one scalar batch), the
// device position (a scalar load), the input row's sources, the weight
// chunks (NCH per lane, unconditional), then the position's cos / sin.  The
// mix waits only for its sources; the weights arrive while it runs.
// GATHER (with NS = 1): the source is the embedding row of the token id,
// gathered here (the id's load goes first, the row's after the weights').
template <int NS, int NCH, bool GATHER = false>  // NS > 0: the input is the depth mix of NS sources
__global__ __launch_bounds__(256) void decode_qkv_kernel(DecodeQkvArgs a) {
  static_assert(!GATHER || NS == 1, "a gathered row is the only source");
  __shared__ DepthMixLds mix_lds;
  __shared__ __attribute__((aligned(16))) uint16_t xs[kQkvMaxDim];
  const DecodeMix& m = a.mix;
  const uint16_t* sp[kMaxDepthSources];
#pragma unroll
  for (int s = 0; s < kMaxDepthSources; ++s) sp[s] = m.srcs.src[s];
  static_assert(kMaxDepthSources == 9, "the batch below names every source slot");
  asm volatile("" ::"s"(sp[0]), "s"(sp[1]), "s"(sp[2]), "s"(sp[3]), "s"(sp[4]), "s"(sp[5]),
               "s"(sp[6]), "s"(sp[7]), "s"(sp[8]), "s"(m.query), "s"(m.score_w), "s"(m.out_w),
               "s"(a.w), "s"(a.position), "s"(a.cos_t), "s"(a.sin_t), "s"(a.dim),
               "s"(a.head_dim), "s"(a.max_positions), "s"(a.x));
  if constexpr (GATHER)
    asm volatile("" ::"s"(a.gather_ids), "s"(a.gather_table), "s"(a.gather_rows),
                 "s"(a.gather_out));
  const int raw_pos = *a.position;
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

  const int chunks = K >> 2;
  const bool has = tid < chunks;
  DecodeMixLoads ml;
  int64_t id_raw = 0;
  if constexpr (GATHER) {
    id_raw = a.gather_ids[t];
    ml.q = reinterpret_cast<const uint2*>(m.query)[has ? tid : 0];
    ml.g = reinterpret_cast<const uint2*>(m.score_w)[has ? tid : 0];
    ml.g_out = reinterpret_cast<const uint2*>(m.out_w)[has ? tid : 0];
  } else if constexpr (NS > 0) {
    decode_mix_load<NS>(m, static_cast<int64_t>(t) * chunks, has ? tid : 0, ml);
  }
  asm volatile("" ::: "memory");
  uint4 wr[NCH];
  load_row_chunks_n<NCH>(a.w, col, K, p, wr);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);  // the id's and position's first uses (waits) after these
  if constexpr (GATHER) {
    const int64_t id = min(max(id_raw, int64_t{0}), static_cast<int64_t>(a.gather_rows - 1));
    ml.v[0] = reinterpret_cast<const uint2*>(a.gather_table)[id * chunks + (has ? tid : 0)];
    asm volatile("" ::: "memory");
  }
  const int pos = min(max(raw_pos, 0), a.max_positions - 1);
  const int64_t ti = static_cast<int64_t>(pos) * (d / 2) + w / 2;
  const float rc = a.cos_t[ti], rs = a.sin_t[ti];
  asm volatile("" ::: "memory");

  if constexpr (NS > 0) {
    // Token t's input row: depth mix + RMSNorm of its sources into LDS.
    if constexpr (GATHER)
      if (blockIdx.x == 0 && has)
        reinterpret_cast<uint2*>(a.gather_out)[static_cast<int64_t>(t) * chunks + tid] = ml.v[0];
    const uint2 o = decode_mix_row<NS>(m, ml, has, wave, lane, K, mix_lds);
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
  for (int c = 0; c < NCH; ++c)
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
  const dim3 grid(n / kGemvRows, a.tokens);
  return with_gemv_chunks<8>(a.dim, [&](auto nch) {
    if (a.gather_ids != nullptr) {
      if (a.mix.n_sources != 1) return hipErrorInvalidValue;
      decode_qkv_kernel<1, nch, true><<<grid, 256, 0, s>>>(a);
      return hipGetLastError();
    }
    if (a.mix.n_sources == 0) {
      decode_qkv_kernel<0, nch><<<grid, 256, 0, s>>>(a);
      return hipGetLastError();
    }
    return with_sources(a.mix.n_sources, [&](auto ns) {
      decode_qkv_kernel<ns, nch><<<grid, 256, 0, s>>>(a);
      return hipGetLastError();
    });
  });
}

}  // namespace parrot
