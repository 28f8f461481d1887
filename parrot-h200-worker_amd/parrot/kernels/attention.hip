// Causal (optionally sliding-window) attention for prefill and full
// forwards, flash style on v_mfma_f32_16x16x32_bf16.
//
// Reference semantics: scaled_dot_product_attention(q, k, v, is_causal=True)
// of the local GQA layers (parrot/model.py:264-295, key j visible to query i
// iff i - W < j <= i) and of the MLA layers (parrot/model.py:350-360, plain
// causal): softmax(q k^T * scale) v with fp32 scores, softmax and
// accumulation, P rounded to bf16 for its product with V (as flash attention
// does) and one bf16 rounding of the output.  Query head h reads kv head
// h / (H / Hk), so grouped kv heads are never expanded in memory.
//
// Layout: the kernel computes transposed products so that nothing passes
// through LDS inside the key loop.
//   S^T = K Q^T   A = K (lane: key row l % 16, 8 dims), B = Q^T (lane: query
//                 column l % 16, 8 dims): 16-byte row loads of row-major K
//                 and Q.  The accumulator gives lane l the scores of query
//                 l % 16 for keys 4 (l / 16) .. +3 of each 16-key tile.
//   O^T += V^T P^T  B = P^T straight from those registers: lane l's 8 k
//                 values are keys {4g..4g+3, 16+4g..16+4g+3} (g = l / 16) of
//                 the 32-key block, an order of the k dimension that the A
//                 operand V^T (lane: dim row l % 16) follows with two 8-byte
//                 loads from a key-contiguous V^T [.., head_dim, keys >=
//                 roundup(T, 32)].
//   The accumulator gives lane l the output dims 4g .. 4g+3 (+ 16 t) of
//   query l % 16: the softmax statistics of a query live in the lanes that
//   hold its outputs, so rescaling needs no exchange.  The running max of a
//   query (shared by its 4 lanes l % 16 + 16 g, combined by two xor
//   shuffles) is raised lazily, only when a wavefront ballot finds a score
//   more than 2^8 above it, so most blocks exchange nothing.
// A workgroup of 8 wavefronts owns 16 query rows; wavefront w takes key
// blocks w, w + 8, ... (next block's loads in flight during the current
// one), and the partial states (max, sum, O) are merged in wavefront order
// through LDS at the end.
//
// PROJ: the output projection's share of this head instead of the output
// itself (the deferred output sum of the reference's decode,
// parrot/model.py:301-316, applied to whole sequences): the head's rows
// y_h [16, D] (rounded to bf16 exactly as the output would be) times the
// head's D columns of the packed output weight, written as fp32
// contributions [batch, seq, heads, n_out].  Their sum over heads, rounded
// to bf16, is the output projection of y; the next depth mix sums them.
// The weight fragments are loaded once the key loop is done (the block
// registers are free then), while the wavefronts' states are merged.
#include "common.h"

namespace parrot {

namespace {

constexpr int kAttnRows = 16;   // query rows per workgroup
constexpr int kAttnKeys = 32;   // keys per block
constexpr int kAttnWaves = 8;  // wavefronts per workgroup, splitting the key blocks

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;            // FRAG: K in fragment order (kfrag_index)
  const uint16_t* vt;           // FRAG: V in fragment order (vfrag_index)
  int64_t qs[3], ks[3], vs[3];  // element strides: batch, head, row (vt: dim row)
  int seq, heads, kv_heads, window;
  float scale_log2;             // scale * log2(e)
  uint16_t* out;                // [batch, seq, heads, head_dim]
  // PROJ: packed output weight [n_out / 16][heads * head_dim / 32][64][8]
  // (parrot_proj_bf16's layout) and the fp32 contributions
  const uint16_t* w_out;
  int n_out;
  float* contrib;               // [batch, seq, heads, n_out]
};

__device__ __forceinline__ bf16x8 load8(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}

// Combines the 4 lanes l % 16 + 16 g (g = 0..3) that share a query.
__device__ __forceinline__ float query_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  return fmaxf(v, __shfl_xor(v, 32));
}

__device__ __forceinline__ float query_sum(float v) {
  v += __shfl_xor(v, 16);
  return v + __shfl_xor(v, 32);
}

// FRAG: K and V in fragment order [batch, kv heads, ceil(seq / 32), ...]:
// every fragment of a key block is one 1 KB contiguous wavefront load (a
// row-major K or V^T load touches 16 rows per instruction, and at prefill
// sizes the per-CU memory pipeline, not the MFMAs, then sets the time).
template <int D, bool FRAG, int OT = 0>  // OT > 0: PROJ with OT output tiles per wavefront
__global__ __launch_bounds__(64 * kAttnWaves) void causal_attention_kernel(AttnArgs a) {
  constexpr bool PROJ = OT > 0;
  constexpr int KS = D / 32;   // k steps of the score product
  constexpr int NT = D / 16;   // output dim tiles
  __shared__ float m_s[kAttnWaves][kAttnRows];
  __shared__ float l_s[kAttnWaves][kAttnRows];
  __shared__ float f_s[kAttnWaves][kAttnRows];
  __shared__ float o_s[kAttnWaves][D][kAttnRows + 1];

  // The kernel arguments in one batch of scalar loads before any use (a
  // field first read on its own costs a scalar round trip).
  asm volatile("" ::"s"(a.q), "s"(a.k), "s"(a.vt), "s"(a.qs[0]), "s"(a.qs[1]), "s"(a.qs[2]),
               "s"(a.ks[0]), "s"(a.ks[1]), "s"(a.ks[2]), "s"(a.vs[0]), "s"(a.vs[1]),
               "s"(a.vs[2]), "s"(a.seq), "s"(a.heads), "s"(a.kv_heads), "s"(a.window),
               "s"(a.scale_log2), "s"(a.out));
  if constexpr (PROJ) asm volatile("" ::"s"(a.w_out), "s"(a.n_out), "s"(a.contrib));
  __builtin_amdgcn_sched_barrier(0);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4;
  const int c = lane & 15;       // this lane's query (column of S^T and O^T)
  const int q0 = blockIdx.x * kAttnRows;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int T = a.seq;
  const int W = a.window;
  const int kvh = h / (a.heads / a.kv_heads);
  const uint16_t* qb = a.q + b * a.qs[0] + h * a.qs[1];
  const int query = q0 + c;

  // K and V^T of this kv head through buffer resources: the per-lane byte
  // offset is fixed, the block's key offset is uniform (an SGPR), and K rows
  // past the sequence read as zero.
  const int ks2 = static_cast<int>(a.ks[2]), vs2 = static_cast<int>(a.vs[2]);
  const int nblk = (T + kAttnKeys - 1) / kAttnKeys;
  const int64_t bh = static_cast<int64_t>(b) * a.kv_heads + kvh;
  const __amdgpu_buffer_rsrc_t k_rsrc =
      FRAG ? make_rsrc(a.k + bh * nblk * (kAttnKeys * D), static_cast<uint32_t>(nblk) * kAttnKeys * D * 2)
           : make_rsrc(a.k + b * a.ks[0] + kvh * a.ks[1], static_cast<uint32_t>(T) * ks2 * 2);
  const __amdgpu_buffer_rsrc_t v_rsrc =
      FRAG ? make_rsrc(a.vt + bh * nblk * (kAttnKeys * D), static_cast<uint32_t>(nblk) * kAttnKeys * D * 2)
           : make_rsrc(a.vt + b * a.vs[0] + kvh * a.vs[1], static_cast<uint32_t>(D) * vs2 * 2);
  const uint32_t k_off0 = FRAG ? lane * 16 : static_cast<uint32_t>(c * ks2 + 8 * g) * 2;
  const uint32_t k_off1 = FRAG ? k_off0 + KS * 1024 : k_off0 + static_cast<uint32_t>(16 * ks2) * 2;
  const uint32_t v_off = FRAG ? lane * 16 : static_cast<uint32_t>(c * vs2 + 4 * g) * 2;

  // Q^T as the B operand: lane holds query q0 + c, dims 32 s + 8 g .. +8.
  bf16x8 qf[KS];
  {
    const uint16_t* row = qb + static_cast<int64_t>(min(query, T - 1)) * a.qs[2] + 8 * g;
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = load8(row + 32 * s);
  }

  const int q_last = min(q0 + kAttnRows, T) - 1;
  const int k_first = max(0, q0 - W + 1) & ~(kAttnKeys - 1);
  // Running max m is shared by the 4 lanes of a query and only raised when
  // a score exceeds it by more than kLazy (log2 units): until then the
  // probabilities stay below 2^kLazy and nothing is rescaled.  Each lane
  // sums its own probabilities; the 4 partial sums of a query are added once
  // at the end.
  constexpr float kLazy = 8.0f;
  float m = -INFINITY, l = 0.0f;
  f32x4 o[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // One block's operands: K rows k0 + 16 n + c (A operand), V^T rows
  // 16 t + c at keys k0 + 4 g and k0 + 16 + 4 g (4 keys each).
  struct Block {
    bf16x8 k[2][KS];
    uint2 v[NT][2];
  };
  auto load_block = [&](Block& x, int k0) {
    if constexpr (FRAG) {
      // block k0 / 32: K fragments (n, s) at (n KS + s) KB, V fragments t at t KB
      const uint32_t blk = static_cast<uint32_t>(k0 / kAttnKeys) * (kAttnKeys * D * 2);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        x.k[0][s] = __builtin_bit_cast(bf16x8, buffer_load16(k_rsrc, k_off0 + 1024 * s, blk));
        x.k[1][s] = __builtin_bit_cast(bf16x8, buffer_load16(k_rsrc, k_off1 + 1024 * s, blk));
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint4 v = buffer_load16(v_rsrc, v_off + 1024 * t, blk);
        x.v[t][0] = make_uint2(v.x, v.y);
        x.v[t][1] = make_uint2(v.z, v.w);
      }
      return;
    }
    const uint32_t ko = static_cast<uint32_t>(k0) * ks2 * 2;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      x.k[0][s] = __builtin_bit_cast(bf16x8, buffer_load16(k_rsrc, k_off0 + 64 * s, ko));
      x.k[1][s] = __builtin_bit_cast(bf16x8, buffer_load16(k_rsrc, k_off1 + 64 * s, ko));
    }
    // V^T rows hold at least roundup(T, 32) keys, so every block is in
    // range; keys past T are zeroed in `step`.
    const uint32_t vo = static_cast<uint32_t>(k0) * 2;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const uint32_t off = v_off + static_cast<uint32_t>(16 * t * vs2) * 2;
      x.v[t][0] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(v_rsrc, off, vo, 0));
      x.v[t][1] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(v_rsrc, off + 32, vo, 0));
    }
  };

  auto step = [&](const Block& x, int k0) {
    // Scores S^T: lane holds query c, keys k0 + 16 n + 4 g + r, in log2
    // units.  A block every query of the workgroup sees whole (below the
    // diagonal, inside the window, inside the sequence) needs no mask.
    f32x4 sc[2];
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      sc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s)
        sc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x.k[n][s], qf[s], sc[n], 0, 0, 0);
    }
    const bool whole = k0 + kAttnKeys - 1 <= q0 && k0 > q_last - W && k0 + kAttnKeys <= T;
    float p[2][4];
    float mx = -INFINITY;
    if (whole) {
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[n][r] = sc[n][r] * a.scale_log2;
          mx = fmaxf(mx, p[n][r]);
        }
    } else {
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = k0 + 16 * n + 4 * g + r;
          const bool ok = key <= query && key > query - W && key < T;
          p[n][r] = ok ? sc[n][r] * a.scale_log2 : -INFINITY;
          mx = fmaxf(mx, p[n][r]);
        }
    }
    // Raise the shared max only when some lane of the wavefront needs it.
    if (__ballot(mx > m + kLazy) != 0) {
      const float mn = fmaxf(m, query_max(mx));
      const float alpha = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
      l *= alpha;
#pragma unroll
      for (int t = 0; t < NT; ++t) o[t] = o[t] * alpha;
      m = mn;
    }
    // exp2(-inf - m) is 0 for a masked key (m is finite once a key is seen,
    // and a lane whose query has seen none keeps p == -inf, m == -inf: its
    // probabilities are forced to 0 below).
    const bool live = m != -INFINITY;
    bf16x8 pf;
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = live ? __builtin_amdgcn_exp2f(p[n][r] - m) : 0.0f;
        l += e;
        pf[4 * n + r] = static_cast<__bf16>(e);
      }
    // V^T fragments; keys past the sequence read as zero (their P is 0,
    // and the padding bytes there need not be finite).
    const bool in_seq = k0 + kAttnKeys <= T;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      uint2 lo = x.v[t][0], hi = x.v[t][1];
      if (!in_seq) {
        const int ka = k0 + 4 * g, kb2 = k0 + 16 + 4 * g;
        lo.x = (ka + 1 < T ? 0xffffffffu : ka < T ? 0x0000ffffu : 0u) & lo.x;
        lo.y = (ka + 3 < T ? 0xffffffffu : ka + 2 < T ? 0x0000ffffu : 0u) & lo.y;
        hi.x = (kb2 + 1 < T ? 0xffffffffu : kb2 < T ? 0x0000ffffu : 0u) & hi.x;
        hi.y = (kb2 + 3 < T ? 0xffffffffu : kb2 + 2 < T ? 0x0000ffffu : 0u) & hi.y;
      }
      const bf16x8 vfrag = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
      o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vfrag, pf, o[t], 0, 0, 0);
    }
  };

  // Key blocks k0, k0 + 8 x 32, ... of this wavefront, two register sets in
  // ping-pong: the next block's loads are in flight during each step.
  constexpr int kStride = kAttnWaves * kAttnKeys;
  Block x0, x1;
  int k0 = k_first + kAttnKeys * wave;
  if (k0 <= q_last) load_block(x0, k0);
  while (k0 <= q_last) {
    const int k1 = k0 + kStride;
    if (k1 <= q_last) load_block(x1, k1);
    step(x0, k0);
    if (k1 > q_last) break;
    const int k2 = k1 + kStride;
    if (k2 <= q_last) load_block(x0, k2);
    step(x1, k1);
    k0 = k2;
  }
  l = query_sum(l);

  // PROJ: this wavefront's output-weight fragments (tiles wave, wave + 8,
  // ... of the n_out columns; k steps h KS .. h KS + KS - 1 of the packed
  // weight), in flight during the merge.
  bf16x8 wq[PROJ ? OT : 1][KS];
  if constexpr (PROJ) {
    const int ksw = a.heads * D / 32;  // k steps of the packed weight
    const __amdgpu_buffer_rsrc_t w_rsrc =
        make_rsrc(a.w_out, static_cast<uint32_t>(a.n_out) * static_cast<uint32_t>(ksw) * 64u);
#pragma unroll
    for (int j = 0; j < OT; ++j)
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const uint32_t frag = static_cast<uint32_t>((wave + 8 * j) * ksw + h * KS + s);
        wq[j][s] = __builtin_bit_cast(bf16x8, buffer_load16(w_rsrc, frag * 1024u + lane * 16u, 0));
      }
  }

  // Merge the wavefronts' states in wavefront order: one scale factor
  // exp2(m_w - max_w m_w) / sum_w (l_w ...) per (wavefront, query), then
  // each output element is a D-independent weighted sum over wavefronts.
  if (g == 0) {
    m_s[wave][c] = m;
    l_s[wave][c] = l;
  }
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) o_s[wave][16 * t + 4 * g + r][c] = o[t][r];
  __syncthreads();
  if (threadIdx.x < kAttnRows) {
    const int qq = threadIdx.x;
    float mt = m_s[0][qq];
#pragma unroll
    for (int w = 1; w < kAttnWaves; ++w) mt = fmaxf(mt, m_s[w][qq]);
    float f[kAttnWaves];
    float lt = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      f[w] = m_s[w][qq] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_s[w][qq] - mt);
      lt += l_s[w][qq] * f[w];
    }
    const float inv = 1.0f / lt;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) f_s[w][qq] = f[w] * inv;
  }
  __syncthreads();
  if constexpr (!PROJ) {
    for (int i = threadIdx.x; i < kAttnRows * D; i += 64 * kAttnWaves) {
      const int qq = i / D, d = i - qq * D;
      const int row = q0 + qq;
      if (row >= T) continue;
      float ot = 0.0f;
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) ot += o_s[w][d][qq] * f_s[w][qq];
      a.out[((static_cast<int64_t>(b) * T + row) * a.heads + h) * D + d] = f32_to_bf16(ot);
    }
  } else {
    // y_h in LDS (bf16, rows padded to D + 8: the 16 rows of a fragment
    // read land in distinct banks), rows past the sequence zero.
    __shared__ __attribute__((aligned(16))) uint16_t y_s[kAttnRows][D + 8];
    for (int i = threadIdx.x; i < kAttnRows * D; i += 64 * kAttnWaves) {
      const int qq = i / D, d = i - qq * D;
      float ot = 0.0f;
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) ot += o_s[w][d][qq] * f_s[w][qq];
      y_s[qq][d] = q0 + qq < T ? f32_to_bf16(ot) : static_cast<uint16_t>(0);
    }
    __syncthreads();
    // contributions[row, n] = sum_d y_h[row, d] W[n, h D + d]: lane l of the
    // C fragment holds column 16 tile + l % 16, rows 4 (l / 16) + r.
    bf16x8 af[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s)
      af[s] = *reinterpret_cast<const bf16x8*>(&y_s[c][32 * s + 8 * g]);
    float* crow = a.contrib + ((static_cast<int64_t>(b) * T + q0 + 4 * g) * a.heads + h) * a.n_out;
    const int64_t row_stride = static_cast<int64_t>(a.heads) * a.n_out;
#pragma unroll
    for (int j = 0; j < OT; ++j) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[s], wq[j][s], acc, 0, 0, 0);
      const int col = 16 * (wave + 8 * j) + c;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (q0 + 4 * g + r < T) crow[r * row_stride + col] = acc[r];
    }
  }
}

}  // namespace

bool attention_head_dim_supported(int head_dim) {
  return head_dim == 64 || head_dim == 96 || head_dim == 128;
}

hipError_t launch_causal_attention_out(const uint16_t* q, const uint16_t* k_frag,
                                       const uint16_t* v_frag, const int64_t* q_strides, int batch,
                                       int seq, int heads, int kv_heads, int head_dim, int window,
                                       float scale, const uint16_t* w_out, int n_out,
                                       float* contrib, hipStream_t s) {
  if (batch == 0 || seq == 0) return hipSuccess;
  AttnArgs a{};
  a.q = q;
  a.k = k_frag;
  a.vt = v_frag;
  for (int i = 0; i < 3; ++i) a.qs[i] = q_strides[i];
  a.seq = seq;
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.window = window;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.w_out = w_out;
  a.n_out = n_out;
  a.contrib = contrib;
  const dim3 grid((seq + kAttnRows - 1) / kAttnRows, heads, batch);
#define PARROT_ATTN_OUT(D, OT) causal_attention_kernel<D, true, OT><<<grid, 64 * kAttnWaves, 0, s>>>(a)
#define PARROT_ATTN_OUT_D(D)                      \
  switch (n_out) {                                \
    case 512: PARROT_ATTN_OUT(D, 4); break;       \
    case 768: PARROT_ATTN_OUT(D, 6); break;       \
    case 1024: PARROT_ATTN_OUT(D, 8); break;      \
    default: return hipErrorInvalidValue;         \
  }
  switch (head_dim) {
    case 64: PARROT_ATTN_OUT_D(64); break;
    case 96: PARROT_ATTN_OUT_D(96); break;
    case 128: PARROT_ATTN_OUT_D(128); break;
    default: return hipErrorInvalidValue;
  }
#undef PARROT_ATTN_OUT_D
#undef PARROT_ATTN_OUT
  return hipGetLastError();
}

bool attention_out_width_supported(int n_out) {
  return n_out == 512 || n_out == 768 || n_out == 1024;
}

hipError_t launch_causal_attention(const uint16_t* q, const uint16_t* k, const uint16_t* vt,
                                   const int64_t* q_strides, const int64_t* k_strides,
                                   const int64_t* vt_strides, int batch, int seq, int heads,
                                   int kv_heads, int head_dim, int window, float scale,
                                   uint16_t* out, hipStream_t s) {
  if (batch == 0 || seq == 0) return hipSuccess;
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.vt = vt;
  const bool frag = k_strides == nullptr;  // fragment-order K and V
  for (int i = 0; i < 3; ++i) {
    a.qs[i] = q_strides[i];
    a.ks[i] = frag ? 0 : k_strides[i];
    a.vs[i] = frag ? 0 : vt_strides[i];
  }
  a.seq = seq;
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.window = window;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out = out;
  const dim3 grid((seq + kAttnRows - 1) / kAttnRows, heads, batch);
#define PARROT_ATTN(D)                                                                 \
  (frag ? causal_attention_kernel<D, true><<<grid, 64 * kAttnWaves, 0, s>>>(a)         \
        : causal_attention_kernel<D, false><<<grid, 64 * kAttnWaves, 0, s>>>(a))
  switch (head_dim) {
    case 64: PARROT_ATTN(64); break;
    case 96: PARROT_ATTN(96); break;
    case 128: PARROT_ATTN(128); break;
    default: return hipErrorInvalidValue;
  }
#undef PARROT_ATTN
  return hipGetLastError();
}

}  // namespace parrot
