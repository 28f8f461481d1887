// Weighted combine of the two routed expert rows and the shared expert row.
//
// out[t] = bf16(shared[t] + y[2t] + y[2t+1]) where y already carries the
// route weight: the bf16 rows the down projection wrote (each contribution
// rounded once, as parrot/model.py:550 rounds expert(x) * weight), added in
// fp32 with one rounding as in parrot/kernels/moe_bf16.metal:752-776; the
// oracle order is the shared expert first, then the experts' contributions
// (parrot/model.py:546-551).
// With an addend (the open AttnRes partial sum) the result is
// bf16(addend + bf16(delta)), the same two roundings as `partial + delta`
// in parrot/model.py:702.  Non-atomic: every token's three rows are read by
// the thread that writes it, as in parrot/cuda_training.py:33-37.
#include "common.h"

namespace parrot {

namespace {

__global__ __launch_bounds__(256) void combine_kernel(
    const uint2* __restrict__ y_routed, const uint2* __restrict__ y_shared,
    const uint2* __restrict__ addend, int64_t tokens, int quads_per_row,
    uint2* __restrict__ out) {
  // The kernel arguments in one batch of scalar loads before any use.
  asm volatile("" ::"s"(y_routed), "s"(y_shared), "s"(addend), "s"(tokens), "s"(quads_per_row),
               "s"(out));
  __builtin_amdgcn_sched_barrier(0);
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= tokens * quads_per_row) return;
  const int64_t t = i / quads_per_row;
  const int64_t q = i - t * quads_per_row;
  const uint2 s = y_shared[i];
  const uint2 a = y_routed[(2 * t) * quads_per_row + q];
  const uint2 b = y_routed[(2 * t + 1) * quads_per_row + q];
  // The addend's load goes out with the rows' (uniform branch), not after
  // their sum.
  const uint2 p = addend != nullptr ? addend[i] : make_uint2(0u, 0u);
  asm volatile("" ::: "memory");
  const float v0 = lo_bf16(s.x) + lo_bf16(a.x) + lo_bf16(b.x);
  const float v1 = hi_bf16(s.x) + hi_bf16(a.x) + hi_bf16(b.x);
  const float v2 = lo_bf16(s.y) + lo_bf16(a.y) + lo_bf16(b.y);
  const float v3 = hi_bf16(s.y) + hi_bf16(a.y) + hi_bf16(b.y);
  uint2 o;
  o.x = pack_bf16x2(v0, v1);
  o.y = pack_bf16x2(v2, v3);
  if (addend != nullptr) {
    o.x = pack_bf16x2(lo_bf16(p.x) + lo_bf16(o.x), hi_bf16(p.x) + hi_bf16(o.x));
    o.y = pack_bf16x2(lo_bf16(p.y) + lo_bf16(o.y), hi_bf16(p.y) + hi_bf16(o.y));
  }
  store_stream(out + i, o);
}

}  // namespace

hipError_t launch_combine(const uint16_t* y_routed, const uint16_t* y_shared,
                          const uint16_t* addend, int64_t tokens, int dim,
                          uint16_t* out, hipStream_t s) {
  if (tokens == 0) return hipSuccess;
  const int quads = dim / 4;
  const int64_t total = tokens * quads;
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  combine_kernel<<<grid, 256, 0, s>>>(reinterpret_cast<const uint2*>(y_routed),
                                      reinterpret_cast<const uint2*>(y_shared),
                                      reinterpret_cast<const uint2*>(addend), tokens, quads,
                                      reinterpret_cast<uint2*>(out));
  return hipGetLastError();
}

}  // namespace parrot
