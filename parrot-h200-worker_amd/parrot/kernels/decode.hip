// Single-token attention over the generation caches (decode steps).
//
// Reference semantics:
//   * sliding-window GQA decode (parrot/model.py:239-262): the new key and
//     value (RoPE applied) are stored at cache position p, and each query
//     head attends over keys max(0, p - W + 1) .. p of its kv head,
//     softmax(q k^T * scale) v with scale 1/sqrt(head_dim);
//   * MLA decode with absorbed weights (parrot/model.py:362-432): the new
//     latent is stored at p and each head's fp32 query attends over latents
//     0 .. p, which serve as both keys and values, scale head_dim^-0.5; the
//     context stays fp32 for the absorbed output map.
// p is read from device memory, so a decode step has static shapes and can
// be captured once in a HIP graph and replayed as the position advances.
//
// One workgroup per (query head, sequence).  Scores: one key per thread
// (16-byte loads of the key row, fp32 dot with the query in LDS); softmax in
// fp32 over the scores kept in LDS; values: wavefront w takes keys w, w + 4,
// ... and lane u accumulates dims 2u, 2u + 1; the four wavefront partials are
// added in a fixed order.  The key and value at p are read from the new rows
// (not from the cache being written), so no workgroup waits for another.
#include "common.h"

namespace parrot {

namespace {

__device__ __forceinline__ float to_f32(uint16_t v) { return __uint_as_float(uint32_t(v) << 16); }
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ void store_out(uint16_t* p, float v) { *p = f32_to_bf16(v); }
__device__ __forceinline__ void store_out(float* p, float v) { *p = v; }

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0xb1>(v));
  v = fmaxf(v, dpp<0x4e>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Workgroup (4 wavefronts) reductions through `red` [4], fixed order.
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return r;
}

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float r = ((red[0] + red[1]) + red[2]) + red[3];
  __syncthreads();
  return r;
}

template <typename QT, typename OT>
__global__ __launch_bounds__(256) void decode_attention_kernel(
    const QT* __restrict__ q, const uint16_t* __restrict__ k_new,
    const uint16_t* __restrict__ v_new, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache, const int32_t* __restrict__ position, int heads,
    int kv_heads, int head_dim, int max_pos, int window, float scale, OT* __restrict__ out) {
  extern __shared__ float smem[];
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int D = head_dim;
  const int rep = heads / kv_heads;
  const int kvh = h / rep;
  const int lcap = min(window, max_pos);
  float* s = smem;           // [lcap] scores, then probabilities
  float* qs = s + lcap;      // [D]
  float* part = qs + D;      // [4][D]
  float* red = part + 4 * D; // [4]

  const int pos = *position;
  if (pos < 0 || pos >= max_pos) return;  // uniform: nothing to attend to
  const int lo = max(0, pos - window + 1);
  const int L = pos - lo + 1;
  const int64_t kv_index = static_cast<int64_t>(b) * kv_heads + kvh;
  const uint16_t* kn = k_new + kv_index * D;
  const uint16_t* vn = v_new + kv_index * D;
  const uint16_t* kc = k_cache + kv_index * max_pos * D;
  const uint16_t* vc = v_cache + kv_index * max_pos * D;

  // The first head of each kv group stores the new key / value row.
  if (h % rep == 0) {
    for (int i = tid; i < D; i += 256) {
      k_cache[(kv_index * max_pos + pos) * D + i] = kn[i];
      if (v_cache != k_cache) v_cache[(kv_index * max_pos + pos) * D + i] = vn[i];
    }
  }
  for (int i = tid; i < D; i += 256) qs[i] = to_f32(q[(static_cast<int64_t>(b) * heads + h) * D + i]);
  __syncthreads();

  // Scores, one key per thread.
  float mx = -INFINITY;
  for (int j = tid; j < L; j += 256) {
    const int key = lo + j;
    const uint16_t* row = key == pos ? kn : kc + static_cast<int64_t>(key) * D;
    float acc = 0.0f;
    for (int c = 0; c < D; c += 8) {
      const uint4 v = *reinterpret_cast<const uint4*>(row + c);
      acc += lo_bf16(v.x) * qs[c] + hi_bf16(v.x) * qs[c + 1] + lo_bf16(v.y) * qs[c + 2] +
             hi_bf16(v.y) * qs[c + 3] + lo_bf16(v.z) * qs[c + 4] + hi_bf16(v.z) * qs[c + 5] +
             lo_bf16(v.w) * qs[c + 6] + hi_bf16(v.w) * qs[c + 7];
    }
    acc *= scale;
    s[j] = acc;
    mx = fmaxf(mx, acc);
  }
  mx = block_max(mx, red);
  float sum = 0.0f;
  for (int j = tid; j < L; j += 256) {
    const float e = __expf(s[j] - mx);
    s[j] = e;
    sum += e;
  }
  sum = block_sum(sum, red);  // also orders the probability writes before the reads below

  // Values: wavefront w takes keys w, w + 4, ...; lane u dims 2u, 2u + 1
  // (and 2u + 128, 2u + 129 when D > 128; D <= kMaxDecodeHeadDim).
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  const int pairs = D / 2;
  for (int j = wave; j < L; j += 4) {
    const int key = lo + j;
    const uint32_t* row = reinterpret_cast<const uint32_t*>(
        key == pos ? vn : vc + static_cast<int64_t>(key) * D);
    const float p = s[j];
    if (lane < pairs) {
      const uint32_t w = row[lane];
      a0 += p * lo_bf16(w);
      a1 += p * hi_bf16(w);
    }
    if (lane + kWave < pairs) {
      const uint32_t w = row[lane + kWave];
      a2 += p * lo_bf16(w);
      a3 += p * hi_bf16(w);
    }
  }
  if (lane < pairs) {
    part[wave * D + 2 * lane] = a0;
    part[wave * D + 2 * lane + 1] = a1;
  }
  if (lane + kWave < pairs) {
    part[wave * D + 2 * (lane + kWave)] = a2;
    part[wave * D + 2 * (lane + kWave) + 1] = a3;
  }
  __syncthreads();
  const float inv = 1.0f / sum;
  for (int i = tid; i < D; i += 256) {
    const float o = ((part[i] + part[D + i]) + part[2 * D + i]) + part[3 * D + i];
    store_out(out + (static_cast<int64_t>(b) * heads + h) * D + i, o * inv);
  }
}

}  // namespace

size_t decode_attention_lds_bytes(int window, int max_pos, int head_dim) {
  const int lcap = window < max_pos ? window : max_pos;
  return (static_cast<size_t>(lcap) + 5 * head_dim + 4) * sizeof(float);
}

hipError_t launch_decode_attention(const uint16_t* q, const uint16_t* k_new,
                                   const uint16_t* v_new, uint16_t* k_cache, uint16_t* v_cache,
                                   const int32_t* position, int batch, int heads, int kv_heads,
                                   int head_dim, int max_pos, int window, float scale,
                                   uint16_t* out, hipStream_t s) {
  if (batch == 0) return hipSuccess;
  const size_t lds = decode_attention_lds_bytes(window, max_pos, head_dim);
  decode_attention_kernel<uint16_t, uint16_t><<<dim3(heads, batch), 256, lds, s>>>(
      q, k_new, v_new, k_cache, v_cache, position, heads, kv_heads, head_dim, max_pos, window,
      scale, out);
  return hipGetLastError();
}

hipError_t launch_decode_attention_latent(const float* q, const uint16_t* latent_new,
                                          uint16_t* latent_cache, const int32_t* position,
                                          int batch, int heads, int latent_dim, int max_pos,
                                          float scale, float* out, hipStream_t s) {
  if (batch == 0) return hipSuccess;
  const size_t lds = decode_attention_lds_bytes(max_pos, max_pos, latent_dim);
  decode_attention_kernel<float, float><<<dim3(heads, batch), 256, lds, s>>>(
      q, latent_new, latent_new, latent_cache, latent_cache, position, heads, 1, latent_dim,
      max_pos, max_pos, scale, out);
  return hipGetLastError();
}

}  // namespace parrot
