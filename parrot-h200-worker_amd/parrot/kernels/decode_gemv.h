// Decode GEMV building blocks: a workgroup of 256 lanes owns 16 output rows,
// one per 16-lane DPP row; lane p of a row holds the row's 16-byte weight
// chunks p, p + 16, ... (256 contiguous bytes per instruction across the
// row), and the row's 16 partial sums are added by four DPP steps in a fixed
// order.  Used by the MLA decode projections and the decode q|k|v
// projection.
#pragma once
#include <type_traits>

#include "common.h"

namespace parrot {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kGemvRows = 16;        // output rows per workgroup
constexpr int kGemvMaxChunks = 16;   // 16-byte weight chunks per lane: K <= 2048

__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0xb1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp<0x4e>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp<0x141>(v);  // row_half_mirror
  v += dpp<0x140>(v);  // row_mirror
  return v;
}

// Dot product of 8 bf16 pairs in fp32 on four v_dot2c_f32_bf16 (each adds two
// exact bf16 products to the running sum; within one fp32 rounding of the
// exactly rounded sum, as the decode MoE's dot8).
typedef __bf16 gemv_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float gemv_dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(gemv_bf16x2, a),
                                         __builtin_bit_cast(gemv_bf16x2, b), c, false);
}
__device__ __forceinline__ float dot_bf16x8(uint4 w, uint4 x) {
  return gemv_dot2(w.w, x.w, gemv_dot2(w.z, x.z, gemv_dot2(w.y, x.y, gemv_dot2(w.x, x.x, 0.0f))));
}

__device__ __forceinline__ float dot_f32x8(uint4 w, float4 x0, float4 x1) {
  float s = lo_bf16(w.x) * x0.x;
  s += hi_bf16(w.x) * x0.y;
  s += lo_bf16(w.y) * x0.z;
  s += hi_bf16(w.y) * x0.w;
  s += lo_bf16(w.z) * x1.x;
  s += hi_bf16(w.z) * x1.y;
  s += lo_bf16(w.w) * x1.z;
  s += hi_bf16(w.w) * x1.w;
  return s;
}

// Lane p's weight chunks of row `row` ([rows, K] bf16), issued at once.
__device__ __forceinline__ void load_row_chunks(const uint16_t* w, int row, int K, int p,
                                                uint4 (&wr)[kGemvMaxChunks]) {
  const int nch = K / 128;
  const uint4* src = reinterpret_cast<const uint4*>(w + static_cast<int64_t>(row) * K);
#pragma unroll
  for (int c = 0; c < kGemvMaxChunks; ++c)
    wr[c] = c < nch ? src[c * 16 + p] : make_uint4(0u, 0u, 0u, 0u);
}

// The same for kernels instantiated per chunk count NCH >= K / 128: every
// load is unconditional (chunks past K / 128 reread the last one and are
// left out of the sums), so a kernel can issue other loads before and after
// these and the compiler's waits still count them exactly.
template <int NCH>
__device__ __forceinline__ void load_row_chunks_n(const uint16_t* w, int row, int K, int p,
                                                  uint4 (&wr)[NCH]) {
  const int last = K / 128 - 1;
  const uint4* src = reinterpret_cast<const uint4*>(w + static_cast<int64_t>(row) * K);
#pragma unroll
  for (int c = 0; c < NCH; ++c) wr[c] = src[min(c, last) * 16 + p];
}

// The chunk counts those kernels are instantiated for, up to MAX; K / 128
// rounds up to the next, and K past 128 MAX is rejected.  `launch` is
// called with std::integral_constant<int, NCH>.
template <int MAX = kGemvMaxChunks, typename F>
__host__ hipError_t with_gemv_chunks(int K, F&& launch) {
  const int nch = K / 128;
  if (nch <= 2) return launch(std::integral_constant<int, 2>{});
  if (nch <= 4) return launch(std::integral_constant<int, 4>{});
  if (nch <= 6) return launch(std::integral_constant<int, 6>{});
  if (nch <= 8) return launch(std::integral_constant<int, 8>{});
  if constexpr (MAX > 8) {
    if (nch <= 12) return launch(std::integral_constant<int, 12>{});
    if (nch <= 16) return launch(std::integral_constant<int, 16>{});
  }
  return hipErrorInvalidValue;
}

// Copies `bytes` (a multiple of 16) from global memory into LDS.
__device__ __forceinline__ void stage(const void* src, void* lds, int bytes) {
  const uint4* s = static_cast<const uint4*>(src);
  uint4* d = static_cast<uint4*>(lds);
  for (int i = threadIdx.x; i < bytes / 16; i += blockDim.x) d[i] = s[i];
}

}  // namespace parrot
