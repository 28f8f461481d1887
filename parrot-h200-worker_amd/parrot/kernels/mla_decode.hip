// The MLA layers' decode-step projections around the latent attention
// (parrot_decode_attention_latent_f32), for up to 16 tokens.
//
// Reference semantics (parrot/model.py:399-432, the absorbed decode path):
//   latent   = kv_down(x)                                    bf16 [T, r]
//   q_latent = F.linear(x.float(), absorbed_query.float())   fp32 [T, H r]
//   result   = F.linear(context, absorbed_output.float()).to(bf16)
//   out      = addend + result (bf16 add) when an addend is given
// where absorbed_query [H r, dim] and absorbed_output [dim, H r] are the bf16
// absorbed maps (parrot/model.py:366-397).  Every product is exact in fp32
// (bf16 operands, or fp32 context times a bf16 weight) and the sums are fp32,
// so the results differ from a library GEMM only by the order of the fp32
// additions.
//
// Each is a weight stream (1.5 MB for either absorbed map at the default
// widths) that a library GEMM runs as several launches plus dtype copies.
// Here one launch each: a workgroup owns 16 output rows, one per 16-lane DPP
// row; lane p of a row holds the row's 16-byte weight chunks p, p + 16, ...
// (256 contiguous bytes per instruction across the row) in registers, the
// tokens' inputs are staged in LDS once, and each token's 16 partial sums are
// added by four DPP steps in a fixed order.
#include <algorithm>

#include "decode_gemv.h"
#include "depth_mix_core.h"

namespace parrot {

namespace {

// Workgroups [0, nq / 16): q_latent rows of absorbed_query; the rest: latent
// rows of kv_down.  x [T, K] bf16 is staged in LDS (T K 2 bytes); with a
// depth mix (MIX) workgroup (x, t) instead mixes and normalises token t's row
// into LDS (depth_mix_core.h) and serves token t.  The mix's source loads go
// out first (the kernel arguments in one scalar batch before them), then the
// weight chunks (NCH per lane, unconditional), so the mix waits only for its
// sources and the weights arrive while it runs.
template <int NS, int NCH>  // NS > 0: each token's input is the depth mix of NS sources
__global__ __launch_bounds__(256) void mla_decode_in_kernel(
    const uint16_t* __restrict__ x, DecodeMix mix, int tokens, int K,
    const uint16_t* __restrict__ wq, int nq, const uint16_t* __restrict__ wkv, int nl,
    float* __restrict__ q_out, uint16_t* __restrict__ lat_out) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  __shared__ DepthMixLds mix_lds;
  if constexpr (NS > 0) {
    const uint16_t* sp[kMaxDepthSources];
#pragma unroll
    for (int s = 0; s < kMaxDepthSources; ++s) sp[s] = mix.srcs.src[s];
    static_assert(kMaxDepthSources == 9, "the batch below names every source slot");
    asm volatile("" ::"s"(sp[0]), "s"(sp[1]), "s"(sp[2]), "s"(sp[3]), "s"(sp[4]), "s"(sp[5]),
                 "s"(sp[6]), "s"(sp[7]), "s"(sp[8]), "s"(mix.query), "s"(mix.score_w),
                 "s"(mix.out_w), "s"(wq), "s"(wkv), "s"(K), "s"(nq));
  }
  const int tid = threadIdx.x;
  const int j = tid >> 4, p = tid & 15;
  const int blocks_q = nq / kGemvRows;
  const bool is_q = static_cast<int>(blockIdx.x) < blocks_q;  // uniform
  const int row = (is_q ? blockIdx.x : blockIdx.x - blocks_q) * kGemvRows + j;
  const int chunks = K >> 2;
  const bool has = tid < chunks;
  const int t_begin = NS > 0 ? static_cast<int>(blockIdx.y) : 0;
  const int t_end = NS > 0 ? t_begin + 1 : tokens;
  DecodeMixLoads ml;
  if constexpr (NS > 0)
    decode_mix_load<NS>(mix, static_cast<int64_t>(t_begin) * chunks, has ? tid : 0, ml);
  asm volatile("" ::: "memory");
  uint4 wr[NCH];
  load_row_chunks_n<NCH>(is_q ? wq : wkv, row, K, p, wr);
  asm volatile("" ::: "memory");
  if constexpr (NS > 0) {
    const int lane = tid & (kWave - 1), wave = tid >> 6;
    const uint2 o = decode_mix_row<NS>(mix, ml, has, wave, lane, K, mix_lds);
    if (has) reinterpret_cast<uint2*>(xs)[tid] = o;
  } else {
    stage(x, xs, tokens * K * 2);
  }
  __syncthreads();
  const int nch = K / 128;
  for (int t = t_begin; t < t_end; ++t) {
    const uint4* xt = reinterpret_cast<const uint4*>(xs + (t - t_begin) * K);
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      if (c < nch) acc += dot_bf16x8(wr[c], xt[c * 16 + p]);
    acc = row16_sum(acc);
    if (p == 0) {
      if (is_q) q_out[static_cast<int64_t>(t) * nq + row] = acc;
      else lat_out[static_cast<int64_t>(t) * nl + row] = f32_to_bf16(acc);
    }
  }
}

// out [T, n] = bf16(ctx Wo^T) (+ addend, a second bf16 rounding); ctx
// [T, K] is fp32 (the MLA context) or bf16 (XT = uint16_t: the local
// layers' attention output), staged in LDS (T K sizeof(XT) bytes).  The
// kernel arguments come in one scalar batch, then the first (up to) 1024
// 16-byte chunks of ctx (4 per lane, clamped), then the weight chunks (NCH
// per lane, unconditional): the staging waits only for ctx, and the weights
// arrive meanwhile.  Longer ctx (more than 16 KB) is staged 4 chunks per
// lane per round trip after that.
template <typename XT, int NCH>
__global__ __launch_bounds__(256) void decode_out_kernel(
    const XT* __restrict__ ctx, int tokens, int K, const uint16_t* __restrict__ wo, int n,
    const uint16_t* __restrict__ addend, uint16_t* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) uint4 cs[];
  asm volatile("" ::"s"(ctx), "s"(tokens), "s"(K), "s"(wo), "s"(n), "s"(addend), "s"(out));
  __builtin_amdgcn_sched_barrier(0);
  const int tid = threadIdx.x;
  const int j = tid >> 4, p = tid & 15;
  const int row = blockIdx.x * kGemvRows + j;
  const int chunks = tokens * K * static_cast<int>(sizeof(XT)) / 16;
  // Staged through a plain vector type: an array of the uint4 struct copied
  // into LDS is kept in scratch memory across the fences below.
  const u32x4* src = reinterpret_cast<const u32x4*>(ctx);
  u32x4* dst = reinterpret_cast<u32x4*>(cs);
  u32x4 c0[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) c0[u] = src[min(tid + 256 * u, chunks - 1)];
  asm volatile("" ::: "memory");
  uint4 wr[NCH];
  load_row_chunks_n<NCH>(wo, row, K, p, wr);
  asm volatile("" ::: "memory");
  // The LDS holds at least 1024 chunks (decode_out_lds_bytes), so the first
  // batch is stored without a branch (slots past ctx get copies).
#pragma unroll
  for (int u = 0; u < 4; ++u) dst[tid + 256 * u] = c0[u];
  for (int base = tid + 1024; base < chunks; base += 1024) {
    u32x4 c1[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) c1[u] = src[min(base + 256 * u, chunks - 1)];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (base + 256 * u < chunks) dst[base + 256 * u] = c1[u];
  }
  __syncthreads();
  const int nch = K / 128;
  for (int t = 0; t < tokens; ++t) {
    float acc = 0.0f;
    if constexpr (sizeof(XT) == 4) {
      const float4* ct = reinterpret_cast<const float4*>(cs) + t * K / 4;
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        if (c < nch) acc += dot_f32x8(wr[c], ct[2 * (c * 16 + p)], ct[2 * (c * 16 + p) + 1]);
    } else {
      const uint4* ct = cs + t * K / 8;
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        if (c < nch) acc += dot_bf16x8(wr[c], ct[c * 16 + p]);
    }
    acc = row16_sum(acc);
    if (p == 0) {
      const int64_t o = static_cast<int64_t>(t) * n + row;
      uint16_t v = f32_to_bf16(acc);
      if (addend != nullptr) v = f32_to_bf16(bf16_to_f32(addend[o]) + bf16_to_f32(v));
      out[o] = v;
    }
  }
}

}  // namespace

size_t mla_decode_lds_bytes(int tokens, int k, int elem_bytes) {
  return static_cast<size_t>(tokens) * k * elem_bytes;
}

namespace {
// decode_out_kernel's LDS: the staged input, at least 1024 16-byte chunks.
size_t decode_out_lds_bytes(int tokens, int k, int elem_bytes) {
  return std::max<size_t>(mla_decode_lds_bytes(tokens, k, elem_bytes), 1024 * 16);
}
}  // namespace

hipError_t launch_mla_decode_in(const uint16_t* x, const DecodeMix* mix, int tokens, int dim,
                                const uint16_t* wq, int nq, const uint16_t* wkv, int nl,
                                float* q_out, uint16_t* lat_out, hipStream_t s) {
  if (tokens == 0) return hipSuccess;
  const bool mixing = mix != nullptr;
  const DecodeMix m = mixing ? *mix : DecodeMix{};
  const dim3 grid((nq + nl) / kGemvRows, mixing ? tokens : 1);
  const size_t lds = mla_decode_lds_bytes(mixing ? 1 : tokens, dim, 2);
  if (!mixing)
    return with_gemv_chunks(dim, [&](auto nch) {
      mla_decode_in_kernel<0, nch><<<grid, 256, lds, s>>>(x, m, tokens, dim, wq, nq, wkv, nl,
                                                          q_out, lat_out);
      return hipGetLastError();
    });
  return with_gemv_chunks<8>(dim, [&](auto nch) {
    return with_sources(m.n_sources, [&](auto ns) {
      mla_decode_in_kernel<ns, nch><<<grid, 256, lds, s>>>(x, m, tokens, dim, wq, nq, wkv, nl,
                                                           q_out, lat_out);
      return hipGetLastError();
    });
  });
}

hipError_t launch_mla_decode_out(const float* ctx, int tokens, int width, const uint16_t* wo,
                                 int dim, const uint16_t* addend, uint16_t* out, hipStream_t s) {
  if (tokens == 0) return hipSuccess;
  const dim3 grid(dim / kGemvRows);
  return with_gemv_chunks(width, [&](auto nch) {
    decode_out_kernel<float, nch><<<grid, 256, decode_out_lds_bytes(tokens, width, 4), s>>>(
        ctx, tokens, width, wo, dim, addend, out);
    return hipGetLastError();
  });
}

hipError_t launch_decode_linear(const uint16_t* x, int tokens, int k, const uint16_t* w, int n,
                                const uint16_t* addend, uint16_t* out, hipStream_t s) {
  if (tokens == 0) return hipSuccess;
  const dim3 grid(n / kGemvRows);
  return with_gemv_chunks(k, [&](auto nch) {
    decode_out_kernel<uint16_t, nch><<<grid, 256, decode_out_lds_bytes(tokens, k, 2), s>>>(
        x, tokens, k, w, n, addend, out);
    return hipGetLastError();
  });
}

}  // namespace parrot
