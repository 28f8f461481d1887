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
// One workgroup per (query head, sequence).  Scores: one key per thread,
// all 16-byte chunks of its row loaded at once, fp32 dot with the query in
// LDS; softmax in fp32 over the scores kept in LDS; values: each thread owns
// one 16-byte chunk of the rows of a key slot, and the slot partials are
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

constexpr int kVPre = 8;  // value rows per thread loaded at kernel entry

// Output-projection operands of decode_attention_kernel with Q > 0: the
// [dim, heads x head_dim] bf16 weight and the fp32 per-head contributions
// [batch, heads, dim] it writes.
struct HeadsOut {
  const uint16_t* weight;
  int dim;
  float* contributions;
};

// CH = head_dim / 8 16-byte chunks per key / value row.
//
// Q = 0: one workgroup per (head, sequence) writes the head's output row.
// Q > 0 (bf16 query and output, the deferred residual): Q workgroups per
// (head, sequence) each attend over the window (the same arithmetic, so the
// same bits) and project the head's bf16-rounded output onto a Q-th of the
// output width: contributions[b, h, n] = sum_i out[i] * W[n, h D + i] in
// index order.  Each thread's weight row piece is loaded at entry, so the
// projection's operands arrive during the attention.  The contributions'
// sum over heads is left to the consumer (the reference's PendingResidual).
template <typename QT, typename OT, int CH, int Q>
__global__ __launch_bounds__(256) void decode_attention_kernel(
    const QT* __restrict__ q, const uint16_t* __restrict__ k_new,
    const uint16_t* __restrict__ v_new, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache, const int32_t* __restrict__ position, int heads,
    int kv_heads, int max_pos, int window, float scale, OT* __restrict__ out, HeadsOut ho) {
  constexpr int D = CH * 8;
  constexpr int kSlots = 256 / CH;  // value pass: key slots x chunks
  static_assert(D <= 256, "one query element per thread");
  extern __shared__ float smem[];
  // The kernel arguments in one batch of scalar loads, before any use.
  asm volatile("" ::"s"(q), "s"(k_new), "s"(v_new), "s"(k_cache), "s"(v_cache), "s"(position),
               "s"(heads), "s"(kv_heads), "s"(max_pos), "s"(window), "s"(scale));
  if constexpr (Q > 0) asm volatile("" ::"s"(ho.weight), "s"(ho.dim), "s"(ho.contributions));
  // The device position first, read through the constant address space (it
  // does not change during the launch) so that it is a scalar load: the
  // cache rows' addresses wait for it alone, not for the element loads below
  // (a vector load's wait would cover those too).
  using const_i32 = const __attribute__((address_space(4))) int32_t;
  const int pos = *(const_i32*)(reinterpret_cast<uintptr_t>(position));
  __builtin_amdgcn_sched_barrier(0);
  const int h = Q > 0 ? static_cast<int>(blockIdx.x) / Q : static_cast<int>(blockIdx.x);
  const int part_n = Q > 0 ? static_cast<int>(blockIdx.x) % Q : 0;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int rep = heads / kv_heads;
  const int kvh = h / rep;
  const int lcap = min(window, max_pos);
  float* s = smem;                 // [lcap] scores, then probabilities
  float* qs = s + lcap;            // [D]
  float* part = qs + D;            // [kSlots][D]
  float* red = part + kSlots * D;  // [4]
  float* ob = red + 4;             // [D] (Q > 0) the head's rounded output

  // Q > 0: thread t < dim / Q owns output column n = part_n dim / Q + t.
  const int nq = Q > 0 ? ho.dim / Q : 0;

  // This thread's elements of the new key / value rows (stored below) and
  // of the query (D <= 256), then the device position: none depends on the
  // position, so they are in flight together, and the cache rows behind
  // them wait for one round trip.  These loads go first, so their uses wait
  // for none of the row loads behind them (loads complete in order).
  const int64_t kv_index = static_cast<int64_t>(b) * kv_heads + kvh;
  const uint16_t* kn = k_new + kv_index * D;
  const uint16_t* vn = v_new + kv_index * D;
  const int ie = min(tid, D - 1);
  const uint16_t kne = kn[ie], vne = vn[ie];
  const float qv = to_f32(q[(static_cast<int64_t>(b) * heads + h) * D + ie]);
  asm volatile("" ::: "memory");
  if (pos < 0 || pos >= max_pos) return;  // uniform: nothing to attend to
  const int lo = max(0, pos - window + 1);
  const int L = pos - lo + 1;
  const uint16_t* kc = k_cache + kv_index * max_pos * D;
  const uint16_t* vc = v_cache + kv_index * max_pos * D;

  // The first pass of key rows (key lo + tid) and the first kVPre value rows
  // of this thread's (slot, chunk) are loaded here, together with the query:
  // none of them depends on another, so the scores and the value pass do not
  // each wait for a memory round trip of their own.
  auto key_row = [&](int key) -> const uint4* {
    return reinterpret_cast<const uint4*>(key == pos ? kn : kc + static_cast<int64_t>(key) * D);
  };
  auto value_row = [&](int key) -> const uint4* {
    return reinterpret_cast<const uint4*>(key == pos ? vn : vc + static_cast<int64_t>(key) * D);
  };
  uint4 kr0[CH];
  {
    const uint4* row = key_row(lo + min(tid, L - 1));
#pragma unroll
    for (int c = 0; c < CH; ++c) kr0[c] = row[c];
  }
  const int chunk = tid % CH;
  const int slot = tid / CH;
  uint4 vpre[kVPre];
#pragma unroll
  for (int u = 0; u < kVPre; ++u)
    vpre[u] = value_row(lo + min(slot + u * kSlots, L - 1))[chunk];

  // Q > 0: the D weights W[n, h D .. h D + D) (16-byte aligned) of this
  // thread's output column, issued after every load the attention waits
  // for, so they arrive during it.
  uint4 wo[Q > 0 ? CH : 1];
  if constexpr (Q > 0) {
    asm volatile("" ::: "memory");
    const uint4* wrow = reinterpret_cast<const uint4*>(
        ho.weight + static_cast<int64_t>(part_n * nq + min(tid, nq - 1)) * heads * D + h * D);
#pragma unroll
    for (int c = 0; c < CH; ++c) wo[c] = wrow[c];
  }
  // The first head of each kv group stores the new key / value row.
  if (h % rep == 0 && part_n == 0 && tid < D) {
    k_cache[(kv_index * max_pos + pos) * D + tid] = kne;
    if (v_cache != k_cache) v_cache[(kv_index * max_pos + pos) * D + tid] = vne;
  }
  if (tid < D) qs[tid] = qv;
  __syncthreads();

  auto score = [&](const uint4 (&kr)[CH]) -> float {
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const float* qc = qs + c * 8;
      acc += lo_bf16(kr[c].x) * qc[0] + hi_bf16(kr[c].x) * qc[1] + lo_bf16(kr[c].y) * qc[2] +
             hi_bf16(kr[c].y) * qc[3] + lo_bf16(kr[c].z) * qc[4] + hi_bf16(kr[c].z) * qc[5] +
             lo_bf16(kr[c].w) * qc[6] + hi_bf16(kr[c].w) * qc[7];
    }
    return acc * scale;
  };

  // Scores: one key per thread per pass, every chunk of its row in flight.
  float mx = -INFINITY;
  if (tid < L) {
    const float acc = score(kr0);
    s[tid] = acc;
    mx = acc;
  }
  for (int j = tid + 256; j < L; j += 256) {
    const uint4* row = key_row(lo + j);
    uint4 kr[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) kr[c] = row[c];
    const float acc = score(kr);
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

  // Values: thread = (key slot, 16-byte chunk); slot k takes keys k,
  // k + kSlots, ...: the first kVPre from the rows loaded at entry, then
  // four rows in flight at a time.  Partials per slot are added in slot
  // order below.
  float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  auto accumulate = [&](const uint4& vr, float p) {
    a[0] += p * lo_bf16(vr.x);
    a[1] += p * hi_bf16(vr.x);
    a[2] += p * lo_bf16(vr.y);
    a[3] += p * hi_bf16(vr.y);
    a[4] += p * lo_bf16(vr.z);
    a[5] += p * hi_bf16(vr.z);
    a[6] += p * lo_bf16(vr.w);
    a[7] += p * hi_bf16(vr.w);
  };
  if (slot < kSlots) {
#pragma unroll
    for (int u = 0; u < kVPre; ++u) {
      const int j = slot + u * kSlots;
      accumulate(vpre[u], j < L ? s[min(j, L - 1)] : 0.0f);
    }
    for (int j0 = slot + kVPre * kSlots; j0 < L; j0 += 4 * kSlots) {
      uint4 vr[4];
      float p[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int j = min(j0 + u * kSlots, L - 1);
        const int key = lo + j;
        vr[u] = value_row(key)[chunk];
        p[u] = j0 + u * kSlots < L ? s[j] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) accumulate(vr[u], p[u]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) part[slot * D + chunk * 8 + i] = a[i];
  }
  __syncthreads();
  const float inv = 1.0f / sum;
  if constexpr (Q == 0) {
    for (int i = tid; i < D; i += 256) {
      float o = 0.0f;
      for (int k = 0; k < kSlots; ++k) o += part[k * D + i];
      store_out(out + (static_cast<int64_t>(b) * heads + h) * D + i, o * inv);
    }
  } else {
    // The head's output rounded to bf16, as the output projection of the
    // undeferred path reads it, then this workgroup's output columns.
    for (int i = tid; i < D; i += 256) {
      float o = 0.0f;
      for (int k = 0; k < kSlots; ++k) o += part[k * D + i];
      ob[i] = to_f32(f32_to_bf16(o * inv));
    }
    __syncthreads();
    if (tid < nq) {
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const float* oc = ob + c * 8;
        acc += lo_bf16(wo[c].x) * oc[0] + hi_bf16(wo[c].x) * oc[1] + lo_bf16(wo[c].y) * oc[2] +
               hi_bf16(wo[c].y) * oc[3] + lo_bf16(wo[c].z) * oc[4] + hi_bf16(wo[c].z) * oc[5] +
               lo_bf16(wo[c].w) * oc[6] + hi_bf16(wo[c].w) * oc[7];
      }
      ho.contributions[(static_cast<int64_t>(b) * heads + h) * ho.dim + part_n * nq + tid] = acc;
    }
  }
}

template <typename QT, typename OT, int Q = 0>
hipError_t launch_decode(const QT* q, const uint16_t* k_new, const uint16_t* v_new,
                         uint16_t* k_cache, uint16_t* v_cache, const int32_t* position, int batch,
                         int heads, int kv_heads, int head_dim, int max_pos, int window,
                         float scale, OT* out, hipStream_t s, HeadsOut ho = HeadsOut{}) {
  const size_t lds = decode_attention_lds_bytes(window, max_pos, head_dim) +
                     (Q > 0 ? static_cast<size_t>(head_dim) * sizeof(float) : 0);
  const dim3 grid(heads * (Q > 0 ? Q : 1), batch);
#define PARROT_DECODE(CH)                                                                   \
  decode_attention_kernel<QT, OT, CH, Q><<<grid, 256, lds, s>>>(                            \
      q, k_new, v_new, k_cache, v_cache, position, heads, kv_heads, max_pos, window, scale, \
      out, ho)
  switch (head_dim / 8) {
    case 1: PARROT_DECODE(1); break;
    case 2: PARROT_DECODE(2); break;
    case 4: PARROT_DECODE(4); break;
    case 8: PARROT_DECODE(8); break;
    case 12: PARROT_DECODE(12); break;
    case 16: PARROT_DECODE(16); break;
    case 24: PARROT_DECODE(24); break;
    case 32: PARROT_DECODE(32); break;
    default: return hipErrorInvalidValue;
  }
#undef PARROT_DECODE
  return hipGetLastError();
}

}  // namespace

bool decode_head_dim_supported(int head_dim) {
  switch (head_dim) {
    case 8: case 16: case 32: case 64: case 96: case 128: case 192: case 256: return true;
    default: return false;
  }
}

size_t decode_attention_lds_bytes(int window, int max_pos, int head_dim) {
  const int lcap = window < max_pos ? window : max_pos;
  const int slots = 256 / (head_dim / 8 > 0 ? head_dim / 8 : 1);
  return (static_cast<size_t>(lcap) + head_dim + static_cast<size_t>(slots) * head_dim + 4) *
         sizeof(float);
}

hipError_t launch_decode_attention(const uint16_t* q, const uint16_t* k_new,
                                   const uint16_t* v_new, uint16_t* k_cache, uint16_t* v_cache,
                                   const int32_t* position, int batch, int heads, int kv_heads,
                                   int head_dim, int max_pos, int window, float scale,
                                   uint16_t* out, hipStream_t s) {
  if (batch == 0) return hipSuccess;
  return launch_decode(q, k_new, v_new, k_cache, v_cache, position, batch, heads, kv_heads,
                       head_dim, max_pos, window, scale, out, s);
}

hipError_t launch_decode_attention_heads(const uint16_t* q, const uint16_t* k_new,
                                         const uint16_t* v_new, uint16_t* k_cache,
                                         uint16_t* v_cache, const int32_t* position, int batch,
                                         int heads, int kv_heads, int head_dim, int max_pos,
                                         int window, float scale, const uint16_t* out_weight,
                                         int dim, float* contributions, hipStream_t s) {
  if (batch == 0) return hipSuccess;
  if (dim % kDecodeHeadsParts != 0 || dim / kDecodeHeadsParts > 256)
    return hipErrorInvalidValue;
  return launch_decode<uint16_t, uint16_t, kDecodeHeadsParts>(
      q, k_new, v_new, k_cache, v_cache, position, batch, heads, kv_heads, head_dim, max_pos,
      window, scale, nullptr, s, HeadsOut{out_weight, dim, contributions});
}

hipError_t launch_decode_attention_latent(const float* q, const uint16_t* latent_new,
                                          uint16_t* latent_cache, const int32_t* position,
                                          int batch, int heads, int latent_dim, int max_pos,
                                          float scale, float* out, hipStream_t s) {
  if (batch == 0) return hipSuccess;
  return launch_decode(q, latent_new, latent_new, latent_cache, latent_cache, position, batch,
                       heads, 1, latent_dim, max_pos, max_pos, scale, out, s);
}

}  // namespace parrot
