// Grouped SwiGLU expert GEMMs on v_mfma_f32_16x16x32_bf16.
//
// Reference semantics: every routed assignment (token t, slot k) computes
// h = silu(x Wg^T) * (x Wu^T) rounded to bf16 and y = h Wd^T, and the shared
// expert does the same for every token (parrot/model.py:443-448, 546-551;
// parrot/kernels/moe_bf16.metal:662-676 for the bf16 rounding of h;
// parrot/metal_moe.py:392-416 for the grouped + overflow organisation).
//
// One launch per projection covers E + 1 row segments: segment E is the
// shared expert over all T tokens, segment e < E is expert e over its
// counts[e] assignments in stable order -- the in-capacity slots
// perm[e, 0..C) followed by the expert's part of the overflow list, so
// overflow rows run through the same MFMA tiles as in-capacity rows.  The
// M-tile -> segment mapping is decoded on device from `counts`, so nothing
// waits for the host; the grid is sized for the worst case and surplus
// workgroups exit at once.
//
// Phase 1 (gate/up): A rows are gathered straight from x through the index
// map, B is the packed [2H, dim] gate/up matrix whose rows alternate 16 gate
// rows and 16 up rows, so each wavefront owns matching gate and up columns
// and applies SwiGLU in its epilogue.  Output: bf16 hidden rows, compact in
// sorted-assignment order (routed rows [0, 2T), shared rows [2T, 3T)).
// Phase 2 (down): A = hidden rows (contiguous per segment), B = [dim, H];
// the epilogue scales routed rows by their route weight and scatters them
// to assignment order (fp32), shared rows go to token order (fp32).
#include "common.h"

namespace parrot {

namespace {

constexpr int kBK = 64;        // k per pipeline stage
constexpr int kLdsPad = 8;     // bf16 padding per LDS row (keeps b128 reads conflict-free)
constexpr int kLdsStride = kBK + kLdsPad;

struct GemmArgs {
  const uint16_t* a_src;      // phase 1: x [T, dim]; phase 2: hidden [3T, hstride]
  int64_t tokens;
  int dim, experts, hidden_dim, shared_dim, capacity, hstride;
  const int32_t* counts;
  const int32_t* offsets;
  const int32_t* perm;
  const int32_t* overflow;
  const float* weights;
  const uint16_t* w_routed;   // phase 1: [E, 2H, dim]; phase 2: [E, dim, H]
  const uint16_t* w_shared;   // phase 1: [2Hs, dim];  phase 2: [dim, Hs]
  uint16_t* hidden_out;       // phase 1 output
  float* y_routed;            // phase 2 output [2T, dim]
  float* y_shared;            // phase 2 output [T, dim]
};

// Raw buffer loads: the per-lane byte offset is fixed for the whole k loop
// and the stage offset travels in an SGPR, so the loop carries no 64-bit
// address arithmetic; reads past `bytes` return zero instead of faulting.
constexpr int kBufferWord3 = 0x00020000;  // gfx9-family buffer resource word 3

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kBufferWord3);
}

__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t voffset,
                                               uint32_t soffset) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset, 0));
}

template <int BM>
struct WaveLayout {
  static constexpr int kWavesM = BM >= 64 ? 2 : 1;
  static constexpr int kWavesN = 4 / kWavesM;
};

// Occupancy is bounded by LDS (two workgroups per CU), so let each wave
// use up to 256 VGPRs rather than squeezing registers for occupancy.
template <int BM, int BN, int PHASE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2)))
void grouped_gemm_kernel(GemmArgs p) {
  constexpr int kWavesM = WaveLayout<BM>::kWavesM;
  constexpr int kWavesN = WaveLayout<BM>::kWavesN;
  constexpr int kWaveM = BM / kWavesM;
  constexpr int kWaveN = BN / kWavesN;
  constexpr int kTilesM = kWaveM / 16;
  constexpr int kTilesN = kWaveN / 16;
  constexpr int kAVec = BM * (kBK / 8);  // 16-byte vectors per A stage
  constexpr int kBVec = BN * (kBK / 8);
  constexpr int kAPer = (kAVec + 255) / 256;
  constexpr int kBPer = kBVec / 256;
  static_assert(PHASE != 1 || kWaveN % 32 == 0, "gate/up pairs need 32-column wave tiles");
  static_assert(kBVec % 256 == 0, "B stage must split evenly over 256 threads");
  static_assert(kAPer <= 4, "A stage holds at most 4 vectors per thread");

  __shared__ __attribute__((aligned(16))) uint16_t a_lds[2][BM][kLdsStride];
  __shared__ __attribute__((aligned(16))) uint16_t b_lds[2][BN][kLdsStride];
  __shared__ int row_src[BM];
  __shared__ int row_dst[BM];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int T = static_cast<int>(p.tokens);

  // ---- which segment / M-tile does this workgroup own? (uniform) ----------
  int seg = -1, mt = 0, rows = 0;
  {
    const int shared_tiles = (T + BM - 1) / BM;
    int m = static_cast<int>(blockIdx.y);
    if (m < shared_tiles) {
      seg = p.experts; mt = m; rows = T;
    } else {
      m -= shared_tiles;
      for (int e = 0; e < p.experts; ++e) {
        const int c = p.counts[e];
        const int te = (c + BM - 1) / BM;
        if (m < te) { seg = e; mt = m; rows = c; break; }
        m -= te;
      }
    }
  }
  if (seg < 0) return;
  const bool shared = seg == p.experts;
  const int N = PHASE == 1 ? 2 * (shared ? p.shared_dim : p.hidden_dim) : p.dim;
  const int K = PHASE == 1 ? p.dim : (shared ? p.shared_dim : p.hidden_dim);
  const int n0 = static_cast<int>(blockIdx.x) * BN;
  if (n0 >= N) return;

  // ---- per-row source / destination ---------------------------------------
  if (tid < BM) {
    const int s = mt * BM + tid;
    const bool valid = s < rows;
    const int sc = valid ? s : mt * BM;  // clamp padding rows onto a real row
    int tok, hrow, asg = -1;
    if (shared) {
      tok = sc;
      hrow = 2 * T + sc;
    } else {
      asg = sc < p.capacity
                ? p.perm[static_cast<int64_t>(seg) * p.capacity + sc]
                : p.overflow[p.offsets[p.experts + 1 + seg] + sc - p.capacity];
      tok = asg >> 1;
      hrow = p.offsets[seg] + sc;
    }
    if (PHASE == 1) {
      row_src[tid] = tok;
      row_dst[tid] = valid ? hrow : -1;
    } else {
      row_src[tid] = hrow;
      row_dst[tid] = valid ? (shared ? tok : asg) : -1;
    }
  }
  __syncthreads();

  // Thread -> 16-byte vector of a stage: vector v = tid + 256 i covers row
  // v / 8, k-columns 8 (v % 8) .. +8, so 8 neighbouring threads read one
  // 128-byte row segment.  Threads beyond the A stage (BM = 16) load a
  // duplicate vector so every load is unconditional; only the owning threads
  // store it to LDS.
  const int a_ld = PHASE == 1 ? p.dim : p.hstride;
  const int64_t a_rows = PHASE == 1 ? p.tokens : 3 * p.tokens;
  const __amdgpu_buffer_rsrc_t a_rsrc =
      make_rsrc(p.a_src, static_cast<uint32_t>(a_rows * a_ld * 2));
  const uint16_t* wbase = shared ? p.w_shared
                                 : p.w_routed + static_cast<int64_t>(seg) * N * K;
  const __amdgpu_buffer_rsrc_t b_rsrc =
      make_rsrc(wbase, static_cast<uint32_t>(static_cast<int64_t>(N) * K * 2));
  const uint32_t col_bytes = (tid & 7) * 16;
  const uint32_t a_off0 = row_src[(tid % kAVec) >> 3] * a_ld * 2 + col_bytes;
  const uint32_t a_off1 = row_src[((tid + 256) % kAVec) >> 3] * a_ld * 2 + col_bytes;
  const uint32_t a_off2 = row_src[((tid + 512) % kAVec) >> 3] * a_ld * 2 + col_bytes;
  const uint32_t a_off3 = row_src[((tid + 768) % kAVec) >> 3] * a_ld * 2 + col_bytes;
  // B rows past N (a partial N tile) lie past the buffer end and read zero.
  const uint32_t b_off0 = static_cast<uint32_t>(n0 + (tid >> 3)) * K * 2 + col_bytes;
  const uint32_t b_step = 32u * K * 2;  // 32 rows further per extra vector
  const int b_row0 = tid >> 3;
  const int col8 = (tid & 7) * 8;

  static_assert(kBPer <= 4, "B stage holds at most 4 vectors per thread");
  // Two register stages (P, Q) of global loads are in flight while the
  // MFMAs consume the current LDS stage; LDS is double-buffered, one
  // barrier per 64-wide k step.
  uint4 pa0, pa1, pa2, pa3, pb0, pb1, pb2, pb3;
  uint4 qa0, qa1, qa2, qa3, qb0, qb1, qb2, qb3;
#define PARROT_LOAD_STAGE(R, kt)                                                            \
  do {                                                                                      \
    const uint32_t ko = static_cast<uint32_t>(kt) * (kBK * 2);                              \
    R##a0 = buffer_load16(a_rsrc, a_off0, ko);                                              \
    if (kAPer > 1) R##a1 = buffer_load16(a_rsrc, a_off1, ko);                               \
    if (kAPer > 2) R##a2 = buffer_load16(a_rsrc, a_off2, ko);                               \
    if (kAPer > 3) R##a3 = buffer_load16(a_rsrc, a_off3, ko);                               \
    R##b0 = buffer_load16(b_rsrc, b_off0, ko);                                              \
    if (kBPer > 1) R##b1 = buffer_load16(b_rsrc, b_off0 + b_step, ko);                      \
    if (kBPer > 2) R##b2 = buffer_load16(b_rsrc, b_off0 + 2 * b_step, ko);                  \
    if (kBPer > 3) R##b3 = buffer_load16(b_rsrc, b_off0 + 3 * b_step, ko);                  \
  } while (0)
#define PARROT_STORE_STAGE(R, buf)                                                          \
  do {                                                                                      \
    if (kAVec >= 256 || tid < kAVec)                                                        \
      *reinterpret_cast<uint4*>(&a_lds[buf][(tid % kAVec) >> 3][col8]) = R##a0;             \
    if (kAPer > 1) *reinterpret_cast<uint4*>(&a_lds[buf][(tid + 256) >> 3][col8]) = R##a1;  \
    if (kAPer > 2) *reinterpret_cast<uint4*>(&a_lds[buf][(tid + 512) >> 3][col8]) = R##a2;  \
    if (kAPer > 3) *reinterpret_cast<uint4*>(&a_lds[buf][(tid + 768) >> 3][col8]) = R##a3;  \
    *reinterpret_cast<uint4*>(&b_lds[buf][b_row0][col8]) = R##b0;                           \
    if (kBPer > 1) *reinterpret_cast<uint4*>(&b_lds[buf][b_row0 + 32][col8]) = R##b1;       \
    if (kBPer > 2) *reinterpret_cast<uint4*>(&b_lds[buf][b_row0 + 64][col8]) = R##b2;       \
    if (kBPer > 3) *reinterpret_cast<uint4*>(&b_lds[buf][b_row0 + 96][col8]) = R##b3;       \
  } while (0)

  const int wm0 = (wave / kWavesN) * kWaveM;
  const int wn0 = (wave % kWavesN) * kWaveN;
  f32x4 acc[kTilesM][kTilesN];
#pragma unroll
  for (int i = 0; i < kTilesM; ++i)
#pragma unroll
    for (int j = 0; j < kTilesN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

#define PARROT_COMPUTE(buf)                                                                 \
  do {                                                                                      \
    _Pragma("unroll") for (int kk = 0; kk < kBK / 32; ++kk) {                               \
      bf16x8 af[kTilesM], bfr[kTilesN];                                                     \
      _Pragma("unroll") for (int i = 0; i < kTilesM; ++i)                                   \
        af[i] = *reinterpret_cast<const bf16x8*>(                                           \
            &a_lds[buf][wm0 + i * 16 + (lane & 15)][kk * 32 + (lane >> 4) * 8]);            \
      _Pragma("unroll") for (int j = 0; j < kTilesN; ++j)                                   \
        bfr[j] = *reinterpret_cast<const bf16x8*>(                                          \
            &b_lds[buf][wn0 + j * 16 + (lane & 15)][kk * 32 + (lane >> 4) * 8]);            \
      _Pragma("unroll") for (int i = 0; i < kTilesM; ++i)                                   \
        _Pragma("unroll") for (int j = 0; j < kTilesN; ++j)                                 \
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0); \
    }                                                                                       \
  } while (0)

  // Every load is issued unconditionally (stage index clamped to the last
  // stage) so the compiler can wait for exactly the stage being stored
  // while the next one stays in flight.
  const int KT = K / kBK;
  PARROT_LOAD_STAGE(p, 0);
  PARROT_LOAD_STAGE(q, min(1, KT - 1));
  PARROT_STORE_STAGE(p, 0);
  __syncthreads();
  for (int kt = 0; kt < KT; kt += 2) {
    // even step: LDS buffer 0 holds stage kt, registers q hold stage kt + 1
    PARROT_LOAD_STAGE(p, min(kt + 2, KT - 1));
    __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the MFMAs
    PARROT_COMPUTE(0);
    PARROT_STORE_STAGE(q, 1);
    __syncthreads();
    if (kt + 1 >= KT) break;
    // odd step: LDS buffer 1 holds stage kt + 1, registers p hold stage kt + 2
    PARROT_LOAD_STAGE(q, min(kt + 3, KT - 1));
    __builtin_amdgcn_sched_barrier(0);
    PARROT_COMPUTE(1);
    PARROT_STORE_STAGE(p, 0);
    __syncthreads();
  }
#undef PARROT_LOAD_STAGE
#undef PARROT_STORE_STAGE
#undef PARROT_COMPUTE

  // ---- epilogue --------------------------------------------------------------
  // C fragment: lane holds column (lane & 15) of rows 4 * (lane >> 4) + r.
  if (PHASE == 1) {
#pragma unroll
    for (int jp = 0; jp < kTilesN / 2; ++jp) {
      const int ng = n0 + wn0 + jp * 32;  // first gate column of the pair
      if (ng >= N) continue;
      const int h = (ng >> 1) + (lane & 15);
#pragma unroll
      for (int i = 0; i < kTilesM; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = wm0 + i * 16 + 4 * (lane >> 4) + r;
          const int dst = row_dst[row];
          if (dst >= 0)
            p.hidden_out[static_cast<int64_t>(dst) * p.hstride + h] =
                f32_to_bf16(swiglu(acc[i][2 * jp][r], acc[i][2 * jp + 1][r]));
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < kTilesN; ++j) {
      const int n = n0 + wn0 + j * 16 + (lane & 15);
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < kTilesM; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = wm0 + i * 16 + 4 * (lane >> 4) + r;
          const int dst = row_dst[row];
          if (dst < 0) continue;
          if (shared) p.y_shared[static_cast<int64_t>(dst) * p.dim + n] = acc[i][j][r];
          else p.y_routed[static_cast<int64_t>(dst) * p.dim + n] = p.weights[dst] * acc[i][j][r];
        }
      }
    }
  }
}

template <int BM, int BN>
hipError_t launch_phase(int phase, const GemmArgs& args, int n_max, hipStream_t s) {
  const int T = static_cast<int>(args.tokens);
  const int m_tiles = (T + BM - 1) / BM + (2 * T) / BM + args.experts;
  const dim3 grid((n_max + BN - 1) / BN, m_tiles);
  if (phase == 1) grouped_gemm_kernel<BM, BN, 1><<<grid, 256, 0, s>>>(args);
  else grouped_gemm_kernel<BM, BN, 2><<<grid, 256, 0, s>>>(args);
  return hipGetLastError();
}

template <int BM>
hipError_t run_phase(int phase, GemmArgs args, const ExpertWeights& w, uint16_t* hidden,
                     hipStream_t s) {
  constexpr int BN = 128;
  if (phase == 1) {
    args.w_routed = w.gate_up;
    args.w_shared = w.shared_gate_up;
    args.hidden_out = hidden;
    return launch_phase<BM, BN>(1, args, 2 * max(args.hidden_dim, args.shared_dim), s);
  }
  args.a_src = hidden;
  args.w_routed = w.down;
  args.w_shared = w.shared_down;
  return launch_phase<BM, BN>(2, args, args.dim, s);
}

}  // namespace

int experts_tile_m(int64_t tokens, int experts) {
  const int64_t per_expert = (2 * tokens + experts - 1) / experts;
  if (tokens <= 16) return 16;
  if (per_expert <= 32) return 32;
  if (per_expert >= 512) return 128;
  return 64;
}

hipError_t launch_expert_gemm(int phase, const uint16_t* x, int64_t tokens, int dim,
                              int experts, int hidden_dim, int shared_dim, int capacity,
                              const GroupMap& map, const ExpertWeights& w, uint16_t* hidden,
                              float* y_routed, float* y_shared, hipStream_t s) {
  if (tokens == 0) return hipSuccess;
  GemmArgs args{};
  args.a_src = x;
  args.tokens = tokens;
  args.dim = dim;
  args.experts = experts;
  args.hidden_dim = hidden_dim;
  args.shared_dim = shared_dim;
  args.capacity = capacity;
  args.hstride = max(hidden_dim, shared_dim);
  args.counts = map.counts;
  args.offsets = map.offsets;
  args.perm = map.perm;
  args.overflow = map.overflow;
  args.weights = map.weights;
  args.y_routed = y_routed;
  args.y_shared = y_shared;
  switch (experts_tile_m(tokens, experts)) {
    case 16: return run_phase<16>(phase, args, w, hidden, s);
    case 32: return run_phase<32>(phase, args, w, hidden, s);
    case 128: return run_phase<128>(phase, args, w, hidden, s);
    default: return run_phase<64>(phase, args, w, hidden, s);
  }
}

}  // namespace parrot
