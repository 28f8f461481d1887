// Attained-peak microkernels: the MFMA issue rate and the HBM copy rate this
// GPU actually reaches, measured beside the vendor peaks so every roofline
// fraction can be stated against both.  No counterpart in the reference.
//
//   mfma_loop_kernel: every wavefront runs `iters` rounds of kChains
//     independent bf16 MFMA chains on register operands (16x16x32 or
//     32x32x16), so the SIMDs issue MFMAs back to back and nothing else.
//     The MFMAs are inline asm on accumulators pinned to AGPRs ("+a"): with
//     the builtins the compiler rotated the 16x16x32 accumulators through
//     ~45 AGPR moves per 8 MFMAs, measuring its register copies instead of
//     the MFMA rate.
//   copy_kernel: grid-stride 16-byte copy with kCopyUnroll loads in flight
//     per lane before the stores.
#include "common.h"

namespace parrot {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kChains16 = 8;  // independent 16x16x32 accumulators per wavefront
constexpr int kChains32 = 4;  // independent 32x32x16 accumulators per wavefront

// The compiler does not see the asm MFMAs' latency: wait it out (longer
// than a 16-pass MFMA) before the accumulators are read back.
__device__ __forceinline__ void drain_mfma() {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7");
}

template <bool WIDE>
__global__ __launch_bounds__(256) void mfma_loop_kernel(int iters, float* __restrict__ out) {
  const int tid = threadIdx.x;
  // Operands depend on the thread so the compiler cannot fold the chains.
  bf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = static_cast<__bf16>(0.001f * static_cast<float>((tid + i) & 7));
    b[i] = static_cast<__bf16>(0.002f * static_cast<float>((tid * 3 + i) & 7));
  }
  float sum = 0.f;
  if constexpr (WIDE) {
    f32x16 acc[kChains32];
#pragma unroll
    for (int c = 0; c < kChains32; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[c][r] = 0.f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int c = 0; c < kChains32; ++c)
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc[c]) : "v"(a), "v"(b));
    }
    drain_mfma();
#pragma unroll
    for (int c = 0; c < kChains32; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) sum += acc[c][r];
  } else {
    f32x4 acc[kChains16];
#pragma unroll
    for (int c = 0; c < kChains16; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int c = 0; c < kChains16; ++c)
        asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc[c]) : "v"(a), "v"(b));
    }
    drain_mfma();
#pragma unroll
    for (int c = 0; c < kChains16; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) sum += acc[c][r];
  }
  out[static_cast<int64_t>(blockIdx.x) * 256 + tid] = sum;
}

constexpr int kCopyUnroll = 4;

__global__ __launch_bounds__(256) void copy_kernel(const uint4* __restrict__ src,
                                                   uint4* __restrict__ dst, int64_t n16) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  for (; i + (kCopyUnroll - 1) * stride < n16; i += kCopyUnroll * stride) {
    uint4 v[kCopyUnroll];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) v[u] = src[i + u * stride];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) dst[i + u * stride] = v[u];
  }
  for (; i < n16; i += stride) dst[i] = src[i];
}

}  // namespace

hipError_t launch_peak_mfma(int wide, int64_t blocks, int iters, float* out, hipStream_t s) {
  if (wide) mfma_loop_kernel<true><<<static_cast<unsigned>(blocks), 256, 0, s>>>(iters, out);
  else mfma_loop_kernel<false><<<static_cast<unsigned>(blocks), 256, 0, s>>>(iters, out);
  return hipGetLastError();
}

int64_t peak_mfma_flops_per_block(int wide, int iters) {
  // 4 wavefronts; 16x16x32 and 32x32x16 MFMAs do 2 * 16 * 16 * 32 and
  // 2 * 32 * 32 * 16 flops.
  const int64_t per_op = wide ? 2 * 32 * 32 * 16 : 2 * 16 * 16 * 32;
  const int64_t chains = wide ? kChains32 : kChains16;
  return 4 * per_op * chains * static_cast<int64_t>(iters);
}

hipError_t launch_peak_copy(const void* src, void* dst, int64_t bytes, int64_t blocks,
                            hipStream_t s) {
  copy_kernel<<<static_cast<unsigned>(blocks), 256, 0, s>>>(
      static_cast<const uint4*>(src), static_cast<uint4*>(dst), bytes / 16);
  return hipGetLastError();
}

}  // namespace parrot
