// Rotary position embedding for the sliding-window GQA layers, fused with
// the split of the packed q|k|v projection into head-major tensors.
//
// Reference semantics (parrot/model.py:176-230): for query and key heads,
// pair i of the head width rotates as
//   out[2i] = x[2i] cos(p w_i) - x[2i+1] sin(p w_i)
//   out[2i+1] = x[2i] sin(p w_i) + x[2i+1] cos(p w_i),   w_i = theta^(-2i/d),
// at model position p = start + row (+ a position read from device memory,
// for graph-captured decode steps); values are not rotated.  The angle
// tables are fp32 here and each output is rounded to bf16 once.
// Input: qkv [rows = batch * seq, (H + 2 Hk) * d] (one packed projection).
// Output: q [batch, H, seq, d], k and v [batch, Hk or H, seq, d]; with
// expand_kv each key/value head is written once for each of the H / Hk
// query heads that share it; with vt_keys > 0 v is written transposed,
// [batch, Hk, d, vt_keys], the value layout the attention kernel reads.
#include "common.h"

namespace parrot {

namespace {

__global__ __launch_bounds__(256) void rope_qkv_kernel(
    const uint2* __restrict__ qkv, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, int64_t rows, int seq, int start,
    const int32_t* __restrict__ start_device, int max_positions, int heads, int kv_heads,
    int head_dim, int expand, int vt_keys, uint16_t* __restrict__ q, uint16_t* __restrict__ k,
    uint16_t* __restrict__ v) {
  const int quads = (heads + 2 * kv_heads) * head_dim / 4;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= rows * quads) return;
  const int64_t row = i / quads;
  const int col = static_cast<int>(i - row * quads) * 4;
  const int head = col / head_dim;
  const int w = col - head * head_dim;  // multiple of 4: two rotation pairs
  const int64_t b = row / seq;
  const int tp = static_cast<int>(row - b * seq);
  uint2 x = qkv[i];
  if (head < heads + kv_heads) {
    const int half = head_dim / 2;
    int p = start + tp + (start_device != nullptr ? *start_device : 0);
    p = min(max(p, 0), max_positions - 1);  // a device position is not validated on the host
    const int64_t pos = static_cast<int64_t>(p) * half + w / 2;
    const float c0 = cos_t[pos], s0 = sin_t[pos];
    const float c1 = cos_t[pos + 1], s1 = sin_t[pos + 1];
    const float e0 = lo_bf16(x.x), o0 = hi_bf16(x.x);
    const float e1 = lo_bf16(x.y), o1 = hi_bf16(x.y);
    x.x = pack_bf16x2(rope_even(e0, o0, c0, s0), rope_odd(e0, o0, c0, s0));
    x.y = pack_bf16x2(rope_even(e1, o1, c1, s1), rope_odd(e1, o1, c1, s1));
  }
  const int kv_out = expand ? heads : kv_heads;
  const int rep = heads / kv_heads;
  if (head < heads) {
    *reinterpret_cast<uint2*>(q + ((b * heads + head) * seq + tp) * head_dim + w) = x;
    return;
  }
  const bool is_k = head < heads + kv_heads;
  const int kvh = head - heads - (is_k ? 0 : kv_heads);
  if (!is_k && vt_keys > 0) {  // transposed values: [b, Hk, d, vt_keys]
    uint16_t* col = v + ((b * kv_heads + kvh) * head_dim + w) * vt_keys + tp;
    col[0] = static_cast<uint16_t>(x.x & 0xffffu);
    col[vt_keys] = static_cast<uint16_t>(x.x >> 16);
    col[2 * vt_keys] = static_cast<uint16_t>(x.y & 0xffffu);
    col[3 * vt_keys] = static_cast<uint16_t>(x.y >> 16);
    return;
  }
  uint16_t* dst = is_k ? k : v;
  if (!expand) {
    *reinterpret_cast<uint2*>(dst + ((b * kv_out + kvh) * seq + tp) * head_dim + w) = x;
  } else {
    for (int r = 0; r < rep; ++r) {
      const int oh = kvh * rep + r;
      *reinterpret_cast<uint2*>(dst + ((b * kv_out + oh) * seq + tp) * head_dim + w) = x;
    }
  }
}

}  // namespace

hipError_t launch_rope_qkv(const uint16_t* qkv, const float* cos_t, const float* sin_t,
                           int64_t batch, int seq, int start, const int32_t* start_device,
                           int max_positions, int heads, int kv_heads, int head_dim,
                           int expand_kv, int vt_keys, uint16_t* q, uint16_t* k, uint16_t* v,
                           hipStream_t s) {
  const int64_t rows = batch * seq;
  const int64_t total = rows * (heads + 2 * kv_heads) * head_dim / 4;
  if (total == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  rope_qkv_kernel<<<grid, 256, 0, s>>>(reinterpret_cast<const uint2*>(qkv), cos_t, sin_t, rows,
                                       seq, start, start_device, max_positions, heads, kv_heads,
                                       head_dim, expand_kv, vt_keys, q, k, v);
  return hipGetLastError();
}

}  // namespace parrot
