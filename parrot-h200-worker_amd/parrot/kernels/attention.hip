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
#include "common.h"

namespace parrot {

namespace {

constexpr int kAttnRows = 16;   // query rows per workgroup
constexpr int kAttnKeys = 32;   // keys per block
constexpr int kAttnWaves = 8;  // wavefronts per workgroup, splitting the key blocks

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* vt;
  int64_t qs[3], ks[3], vs[3];  // element strides: batch, head, row (vt: dim row)
  int seq, heads, kv_heads, window;
  float scale_log2;             // scale * log2(e)
  uint16_t* out;                // [batch, seq, heads, head_dim]
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

template <int D>
__global__ __launch_bounds__(64 * kAttnWaves) void causal_attention_kernel(AttnArgs a) {
  constexpr int KS = D / 32;   // k steps of the score product
  constexpr int NT = D / 16;   // output dim tiles
  __shared__ float m_s[kAttnWaves][kAttnRows];
  __shared__ float l_s[kAttnWaves][kAttnRows];
  __shared__ float o_s[kAttnWaves][D][kAttnRows + 1];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int c = lane & 15;       // this lane's query (column of S^T and O^T)
  const int q0 = blockIdx.x * kAttnRows;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int T = a.seq;
  const int W = a.window;
  const int kvh = h / (a.heads / a.kv_heads);
  const uint16_t* qb = a.q + b * a.qs[0] + h * a.qs[1];
  const uint16_t* kb = a.k + b * a.ks[0] + kvh * a.ks[1];
  const uint16_t* vb = a.vt + b * a.vs[0] + kvh * a.vs[1];
  const int query = q0 + c;

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
  bf16x8 kf[2][KS];
  uint2 vf[NT][2];
  auto load_block = [&](int k0) {
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const uint16_t* row = kb + static_cast<int64_t>(min(k0 + 16 * n + c, T - 1)) * a.ks[2] + 8 * g;
#pragma unroll
      for (int s = 0; s < KS; ++s) kf[n][s] = load8(row + 32 * s);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      // V^T rows hold at least roundup(T, 32) keys, so every block is in
      // bounds; keys past T are zeroed below.
      const uint16_t* row = vb + static_cast<int64_t>(16 * t + c) * a.vs[2] + k0 + 4 * g;
      vf[t][0] = *reinterpret_cast<const uint2*>(row);
      vf[t][1] = *reinterpret_cast<const uint2*>(row + 16);
    }
  };

  int k0 = k_first + kAttnKeys * wave;
  if (k0 <= q_last) load_block(k0);
  for (; k0 <= q_last; k0 += kAttnWaves * kAttnKeys) {
    bf16x8 kc[2][KS];
    uint2 vc[NT][2];
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int s = 0; s < KS; ++s) kc[n][s] = kf[n][s];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      vc[t][0] = vf[t][0];
      vc[t][1] = vf[t][1];
    }
    const int k_next = k0 + kAttnWaves * kAttnKeys;
    if (k_next <= q_last) load_block(k_next);

    // Scores S^T: lane holds query c, keys k0 + 16 n + 4 g + r, in log2
    // units.  A block every query of the workgroup sees whole (below the
    // diagonal, inside the window, inside the sequence) needs no mask.
    f32x4 sc[2];
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      sc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s)
        sc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kc[n][s], qf[s], sc[n], 0, 0, 0);
    }
    const bool whole = k0 + kAttnKeys - 1 <= q0 && k0 > q_last - W && k0 + kAttnKeys <= T;
    float p[2][4];
    float mx = -INFINITY;
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = k0 + 16 * n + 4 * g + r;
        const bool ok = whole || (key <= query && key > query - W && key < T);
        p[n][r] = ok ? sc[n][r] * a.scale_log2 : -INFINITY;
        mx = fmaxf(mx, p[n][r]);
      }
    // Raise the shared max only when some lane of the wavefront needs it.
    if (__ballot(mx > m + kLazy) != 0) {
      const float mn = fmaxf(m, query_max(mx));
      const float alpha = m == -INFINITY ? 0.0f : exp2f(m - mn);
      l *= alpha;
#pragma unroll
      for (int t = 0; t < NT; ++t) o[t] = o[t] * alpha;
      m = mn;
    }
    bf16x8 pf;
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = p[n][r] == -INFINITY ? 0.0f : exp2f(p[n][r] - m);
        l += e;
        pf[4 * n + r] = static_cast<__bf16>(e);
      }
    // V^T fragments; keys past the sequence read as zero (their P is 0,
    // and the padding bytes there need not be finite).
    const bool in_seq = k0 + kAttnKeys <= T;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      uint2 lo = vc[t][0], hi = vc[t][1];
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
  }
  l = query_sum(l);

  // Merge the wavefronts' states in wavefront order.
  if (g == 0) {
    m_s[wave][c] = m;
    l_s[wave][c] = l;
  }
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) o_s[wave][16 * t + 4 * g + r][c] = o[t][r];
  __syncthreads();
  for (int i = threadIdx.x; i < kAttnRows * D; i += 64 * kAttnWaves) {
    const int qq = i / D, d = i - qq * D;
    const int row = q0 + qq;
    if (row >= T) continue;
    float mt = m_s[0][qq];
#pragma unroll
    for (int w = 1; w < kAttnWaves; ++w) mt = fmaxf(mt, m_s[w][qq]);
    float lt = 0.0f, ot = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      const float f = m_s[w][qq] == -INFINITY ? 0.0f : exp2f(m_s[w][qq] - mt);
      lt += l_s[w][qq] * f;
      ot += o_s[w][d][qq] * f;
    }
    a.out[((static_cast<int64_t>(b) * T + row) * a.heads + h) * D + d] = f32_to_bf16(ot / lt);
  }
}

}  // namespace

bool attention_head_dim_supported(int head_dim) {
  return head_dim == 64 || head_dim == 96 || head_dim == 128;
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
  for (int i = 0; i < 3; ++i) {
    a.qs[i] = q_strides[i];
    a.ks[i] = k_strides[i];
    a.vs[i] = vt_strides[i];
  }
  a.seq = seq;
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.window = window;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out = out;
  const dim3 grid((seq + kAttnRows - 1) / kAttnRows, heads, batch);
  switch (head_dim) {
    case 64: causal_attention_kernel<64><<<grid, 64 * kAttnWaves, 0, s>>>(a); break;
    case 96: causal_attention_kernel<96><<<grid, 64 * kAttnWaves, 0, s>>>(a); break;
    case 128: causal_attention_kernel<128><<<grid, 64 * kAttnWaves, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace parrot
