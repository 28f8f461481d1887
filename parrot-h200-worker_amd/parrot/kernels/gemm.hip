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

// Which row segment and M-tile does this workgroup own?  One vector load of
// the expert counts (lane e holds counts[e]), then a uniform scan over the
// lanes' tile counts with readlane -- no chain of dependent memory loads.
// Segment E (the shared expert, all T tokens) comes first.
template <int BM>
__device__ __forceinline__ bool find_tile(const GemmArgs& p, int T, int& seg, int& mt,
                                          int& rows) {
  const int lane = threadIdx.x & (kWave - 1);
  const int count = lane < p.experts ? p.counts[lane] : 0;
  const int tiles = (count + BM - 1) / BM;
  const int shared_tiles = (T + BM - 1) / BM;
  int m = static_cast<int>(blockIdx.y);
  if (m < shared_tiles) {
    seg = p.experts; mt = m; rows = T;
    return true;
  }
  m -= shared_tiles;
  for (int e = 0; e < p.experts; ++e) {
    const int te = __builtin_amdgcn_readlane(tiles, e);
    if (m < te) {
      seg = e; mt = m; rows = __builtin_amdgcn_readlane(count, e);
      return true;
    }
    m -= te;
  }
  return false;
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

  int seg = -1, mt = 0, rows = 0;
  if (!find_tile<BM>(p, T, seg, mt, rows)) return;
  const bool shared = seg == p.experts;
  const int N = PHASE == 1 ? 2 * (shared ? p.shared_dim : p.hidden_dim) : p.dim;
  const int K = PHASE == 1 ? p.dim : (shared ? p.shared_dim : p.hidden_dim);
  const int n0 = static_cast<int>(blockIdx.x) * BN;
  if (n0 >= N) return;

  // ---- weights: the first two stages go out before the row lookups --------
  const uint16_t* wbase = shared ? p.w_shared
                                 : p.w_routed + static_cast<int64_t>(seg) * N * K;
  const __amdgpu_buffer_rsrc_t b_rsrc =
      make_rsrc(wbase, static_cast<uint32_t>(static_cast<int64_t>(N) * K * 2));
  // B arrives in MFMA fragment order (1 KB blocks of 16 rows x 32 k, lane l's
  // 16 bytes at 16 l).  Vector v = tid + 256 i of a stage is lane v % 64 of
  // block v / 64 = (16-row group (v / 64) / 2, 32-k half (v / 64) % 2); it
  // lands in LDS row 16 group + lane % 16, k chunk 4 half + lane / 16.
  // Rows past N lie past the buffer end and read zero.
  const int ksteps32 = K / 32;
  uint32_t b_off[4];
  int b_lrow[4], b_lcol[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int v = tid + 256 * i;
    const int blk = v >> 6, l = v & 63;
    const int grp = blk >> 1, half = blk & 1;
    b_off[i] = static_cast<uint32_t>(((n0 / 16 + grp) * ksteps32 + half) * 64 + l) * 16;
    b_lrow[i] = grp * 16 + (l & 15);
    b_lcol[i] = (half * 4 + (l >> 4)) * 8;
  }
  static_assert(kBPer == 4, "B stage is 1024 vectors: 4 per thread");
  // Two register stages (P, Q) of global loads are in flight while the
  // MFMAs consume the current LDS stage; LDS is double-buffered, one
  // barrier per 64-wide k step.  Every load is issued unconditionally (stage
  // index clamped to the last stage) so the compiler can wait for exactly
  // the stage being stored while the next one stays in flight.
  uint4 pa0, pa1, pa2, pa3, pb0, pb1, pb2, pb3;
  uint4 qa0, qa1, qa2, qa3, qb0, qb1, qb2, qb3;
#define PARROT_LOAD_B(R, kt)                                                                \
  do {                                                                                      \
    const uint32_t kb = static_cast<uint32_t>(kt) * 2048;  /* two 1 KB blocks per stage */ \
    R##b0 = buffer_load16(b_rsrc, b_off[0], kb);                                            \
    R##b1 = buffer_load16(b_rsrc, b_off[1], kb);                                            \
    R##b2 = buffer_load16(b_rsrc, b_off[2], kb);                                            \
    R##b3 = buffer_load16(b_rsrc, b_off[3], kb);                                            \
  } while (0)
  const int KT = K / kBK;
  PARROT_LOAD_B(p, 0);
  PARROT_LOAD_B(q, min(1, KT - 1));

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

  // Thread -> 16-byte vector of an A stage: vector v = tid + 256 i covers
  // row v / 8, k-columns 8 (v % 8) .. +8, so 8 neighbouring threads read one
  // 128-byte row segment.  Threads beyond the A stage (BM = 16) load a
  // duplicate vector so every load is unconditional; only the owning threads
  // store it to LDS.
  const int a_ld = PHASE == 1 ? p.dim : p.hstride;
  const int64_t a_rows = PHASE == 1 ? p.tokens : 3 * p.tokens;
  const __amdgpu_buffer_rsrc_t a_rsrc =
      make_rsrc(p.a_src, static_cast<uint32_t>(a_rows * a_ld * 2));
  const uint32_t col_bytes = (tid & 7) * 16;
  const uint32_t a_off0 = row_src[(tid % kAVec) >> 3] * a_ld * 2 + col_bytes;
  const uint32_t a_off1 = row_src[((tid + 256) % kAVec) >> 3] * a_ld * 2 + col_bytes;
  const uint32_t a_off2 = row_src[((tid + 512) % kAVec) >> 3] * a_ld * 2 + col_bytes;
  const uint32_t a_off3 = row_src[((tid + 768) % kAVec) >> 3] * a_ld * 2 + col_bytes;
  const int col8 = (tid & 7) * 8;
#define PARROT_LOAD_A(R, kt)                                                                \
  do {                                                                                      \
    const uint32_t ko = static_cast<uint32_t>(kt) * (kBK * 2);                              \
    R##a0 = buffer_load16(a_rsrc, a_off0, ko);                                              \
    if (kAPer > 1) R##a1 = buffer_load16(a_rsrc, a_off1, ko);                               \
    if (kAPer > 2) R##a2 = buffer_load16(a_rsrc, a_off2, ko);                               \
    if (kAPer > 3) R##a3 = buffer_load16(a_rsrc, a_off3, ko);                               \
  } while (0)
#define PARROT_STORE_STAGE(R, buf)                                                          \
  do {                                                                                      \
    if (kAVec >= 256 || tid < kAVec)                                                        \
      *reinterpret_cast<uint4*>(&a_lds[buf][(tid % kAVec) >> 3][col8]) = R##a0;             \
    if (kAPer > 1) *reinterpret_cast<uint4*>(&a_lds[buf][(tid + 256) >> 3][col8]) = R##a1;  \
    if (kAPer > 2) *reinterpret_cast<uint4*>(&a_lds[buf][(tid + 512) >> 3][col8]) = R##a2;  \
    if (kAPer > 3) *reinterpret_cast<uint4*>(&a_lds[buf][(tid + 768) >> 3][col8]) = R##a3;  \
    *reinterpret_cast<uint4*>(&b_lds[buf][b_lrow[0]][b_lcol[0]]) = R##b0;                   \
    *reinterpret_cast<uint4*>(&b_lds[buf][b_lrow[1]][b_lcol[1]]) = R##b1;                   \
    *reinterpret_cast<uint4*>(&b_lds[buf][b_lrow[2]][b_lcol[2]]) = R##b2;                   \
    *reinterpret_cast<uint4*>(&b_lds[buf][b_lrow[3]][b_lcol[3]]) = R##b3;                   \
  } while (0)
#define PARROT_LOAD_STAGE(R, kt)                                                            \
  do {                                                                                      \
    PARROT_LOAD_A(R, kt);                                                                   \
    PARROT_LOAD_B(R, kt);                                                                   \
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

  PARROT_LOAD_A(p, 0);
  PARROT_LOAD_A(q, min(1, KT - 1));
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
#undef PARROT_LOAD_A
#undef PARROT_LOAD_B
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

// ---------------------------------------------------------------------------
// Streaming variant for small row tiles (BM <= 64, K <= kStreamKCap): the
// weight-streaming regime of prefill and decode.
//
// The workgroup's whole A tile (BM gathered rows x K) is copied into LDS once
// with direct-to-LDS loads (global_load_lds_dwordx4: lane l of a wavefront
// writes 16 bytes at base + 16 l, from any global address), stored as 16-byte
// chunks XOR-swizzled within groups of 16 (or 8) so the MFMA fragment reads
// of 16 consecutive rows hit distinct banks.  Weights never touch LDS: each
// lane loads its B fragments (16 bytes per 32-wide k step) straight into a
// ring of PF register stages with raw buffer loads, refilling a slot as soon
// as its MFMAs have consumed it.  The k loop has no barrier.
// Wavefront w owns output columns [w WN, w WN + WN) of the 4 WN-wide tile.
constexpr int kStreamKCap = 768;  // largest K whose A tile fits the LDS budget

typedef __attribute__((address_space(3))) void lds_void_t;

template <int BM, int WN, int PF, int PHASE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2)))
void grouped_gemm_stream_kernel(GemmArgs p) {
  constexpr int kTilesM = BM / 16;
  constexpr int kTilesN = WN / 16;
  constexpr int BN = 4 * WN;
  static_assert(PHASE != 1 || WN == 32, "gate/up pairs need 32 columns per wavefront");

  __shared__ __attribute__((aligned(16))) uint16_t a_lds[BM * kStreamKCap];
  __shared__ int row_src[BM];
  __shared__ int row_dst[BM];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int T = static_cast<int>(p.tokens);

  int seg = -1, mt = 0, rows = 0;
  if (!find_tile<BM>(p, T, seg, mt, rows)) return;
  const bool shared = seg == p.experts;
  const int N = PHASE == 1 ? 2 * (shared ? p.shared_dim : p.hidden_dim) : p.dim;
  const int K = PHASE == 1 ? p.dim : (shared ? p.shared_dim : p.hidden_dim);
  const int n0 = static_cast<int>(blockIdx.x) * BN;
  if (n0 >= N) return;

  const int chunks = K / 8;                       // 16-byte chunks per A row
  const int swz = (chunks & 15) == 0 ? 15 : 7;   // XOR group size - 1
  const int ksteps = K / 32;

  // ---- B: first PF k steps of this lane's fragments -------------------------
  const uint16_t* wbase = shared ? p.w_shared
                                 : p.w_routed + static_cast<int64_t>(seg) * N * K;
  const __amdgpu_buffer_rsrc_t b_rsrc =
      make_rsrc(wbase, static_cast<uint32_t>(static_cast<int64_t>(N) * K * 2));
  // Fragment order: the 1 KB block of (16-row group g, 32-k step) starts at
  // (g * ksteps + step) KB and holds lane l's 16 bytes at 16 l, so one
  // wavefront load is 1 KB contiguous.  Groups past N read zero.
  uint32_t b_off[kTilesN];
#pragma unroll
  for (int j = 0; j < kTilesN; ++j)
    b_off[j] = static_cast<uint32_t>(((n0 + wave * WN + j * 16) / 16) * ksteps * 64 + lane) * 16;
  uint4 bq[PF][kTilesN];
#pragma unroll
  for (int i = 0; i < PF; ++i)
#pragma unroll
    for (int j = 0; j < kTilesN; ++j)
      bq[i][j] = buffer_load16(b_rsrc, b_off[j], static_cast<uint32_t>(min(i, ksteps - 1)) * 1024);

  if (tid < BM) {
    const int s = mt * BM + tid;
    const bool valid = s < rows;
    const int sc = valid ? s : mt * BM;  // padding rows read a real row
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

  // ---- A: the whole tile, direct to LDS ------------------------------------
  {
    const int a_ld = PHASE == 1 ? p.dim : p.hstride;
    const int slots = BM * chunks;  // multiple of 64 (BM >= 16, chunks >= 8)
    for (int i = wave; i < slots / kWave; i += 4) {
      const int slot = i * kWave + lane;
      const int r = slot / chunks;
      const int pc = slot - r * chunks;
      const int c = (pc & ~swz) | ((pc ^ r) & swz);
      const uint16_t* g = p.a_src + static_cast<int64_t>(row_src[r]) * a_ld + c * 8;
      __builtin_amdgcn_global_load_lds(g, (lds_void_t*)(a_lds + i * kWave * 8), 16, 0, 0);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  f32x4 acc[kTilesM][kTilesN];
#pragma unroll
  for (int i = 0; i < kTilesM; ++i)
#pragma unroll
    for (int j = 0; j < kTilesN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int s0 = 0; s0 < ksteps; s0 += PF) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int step = s0 + i;  // ksteps is a multiple of PF
      bf16x8 af[kTilesM];
#pragma unroll
      for (int mi = 0; mi < kTilesM; ++mi) {
        const int r = mi * 16 + (lane & 15);
        const int c = step * 4 + (lane >> 4);
        const int pc = (c & ~swz) | ((c ^ r) & swz);
        af[mi] = *reinterpret_cast<const bf16x8*>(&a_lds[(r * chunks + pc) * 8]);
      }
#pragma unroll
      for (int mi = 0; mi < kTilesM; ++mi)
#pragma unroll
        for (int j = 0; j < kTilesN; ++j)
          acc[mi][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              af[mi], __builtin_bit_cast(bf16x8, bq[i][j]), acc[mi][j], 0, 0, 0);
      const uint32_t next = static_cast<uint32_t>(min(step + PF, ksteps - 1)) * 1024;
#pragma unroll
      for (int j = 0; j < kTilesN; ++j) bq[i][j] = buffer_load16(b_rsrc, b_off[j], next);
    }
  }

  // ---- epilogue (as in grouped_gemm_kernel) ----------------------------------
  if (PHASE == 1) {
    const int ng = n0 + wave * WN;  // first gate column of this wavefront's pair
    if (ng < N) {
      const int h = (ng >> 1) + (lane & 15);
#pragma unroll
      for (int mi = 0; mi < kTilesM; ++mi) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = mi * 16 + 4 * (lane >> 4) + r;
          const int dst = row_dst[row];
          if (dst >= 0)
            p.hidden_out[static_cast<int64_t>(dst) * p.hstride + h] =
                f32_to_bf16(swiglu(acc[mi][0][r], acc[mi][1][r]));
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < kTilesN; ++j) {
      const int n = n0 + wave * WN + j * 16 + (lane & 15);
      if (n >= N) continue;
#pragma unroll
      for (int mi = 0; mi < kTilesM; ++mi) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = mi * 16 + 4 * (lane >> 4) + r;
          const int dst = row_dst[row];
          if (dst < 0) continue;
          if (shared) p.y_shared[static_cast<int64_t>(dst) * p.dim + n] = acc[mi][j][r];
          else p.y_routed[static_cast<int64_t>(dst) * p.dim + n] = p.weights[dst] * acc[mi][j][r];
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

template <int BM, int WN, int PF>
hipError_t launch_stream(int phase, const GemmArgs& args, int n_max, hipStream_t s) {
  const int T = static_cast<int>(args.tokens);
  const int m_tiles = (T + BM - 1) / BM + (2 * T) / BM + args.experts;
  const dim3 grid((n_max + 4 * WN - 1) / (4 * WN), m_tiles);
  if (phase == 1) grouped_gemm_stream_kernel<BM, 32, PF, 1><<<grid, 256, 0, s>>>(args);
  else grouped_gemm_stream_kernel<BM, WN, PF, 2><<<grid, 256, 0, s>>>(args);
  return hipGetLastError();
}

// Register-ring depth: the largest of 8 / 4 / 2 / 1 dividing every segment's
// number of 32-wide k steps in this phase.
int stream_depth(int phase, const GemmArgs& a) {
  const int k0 = phase == 1 ? a.dim : a.hidden_dim;
  const int k1 = phase == 1 ? a.dim : a.shared_dim;
  for (int pf = 8; pf > 1; pf >>= 1)
    if ((k0 / 32) % pf == 0 && (k1 / 32) % pf == 0) return pf;
  return 1;
}

template <int BM>
hipError_t run_stream(int phase, GemmArgs args, int n_max, hipStream_t s) {
  // Down projection: 16 columns per wavefront doubles the workgroups when
  // the row tiles are few.
  switch (stream_depth(phase, args)) {
    case 8: return phase == 1 ? launch_stream<BM, 32, 8>(1, args, n_max, s)
                              : launch_stream<BM, 16, 8>(2, args, n_max, s);
    case 4: return phase == 1 ? launch_stream<BM, 32, 4>(1, args, n_max, s)
                              : launch_stream<BM, 16, 4>(2, args, n_max, s);
    case 2: return phase == 1 ? launch_stream<BM, 32, 2>(1, args, n_max, s)
                              : launch_stream<BM, 16, 2>(2, args, n_max, s);
    default: return phase == 1 ? launch_stream<BM, 32, 1>(1, args, n_max, s)
                               : launch_stream<BM, 16, 1>(2, args, n_max, s);
  }
}

template <int BM, bool STREAM>
hipError_t run_phase(int phase, GemmArgs args, const ExpertWeights& w, uint16_t* hidden,
                     hipStream_t s) {
  constexpr int BN = 128;
  int n_max;
  if (phase == 1) {
    args.w_routed = w.gate_up;
    args.w_shared = w.shared_gate_up;
    args.hidden_out = hidden;
    n_max = 2 * max(args.hidden_dim, args.shared_dim);
  } else {
    args.a_src = hidden;
    args.w_routed = w.down;
    args.w_shared = w.shared_down;
    n_max = args.dim;
  }
  const int k_max = phase == 1 ? args.dim : max(args.hidden_dim, args.shared_dim);
  if (STREAM && k_max <= kStreamKCap) return run_stream<BM>(phase, args, n_max, s);
  return launch_phase<BM, BN>(phase, args, n_max, s);
}

// Kernel and row tile per launch, chosen from T and E only (the per-expert
// counts stay on the device).  While an expert's rows fit one small tile the
// launch is weight-streaming bound and the streaming kernel wins (every extra
// row tile re-streams that expert's weights); with more rows per expert the
// LDS-tiled kernel with 64-row tiles, which shares each staged weight tile
// across four wavefronts, is faster.
enum class TilePlan { kStream16, kStream32, kStream64, kTiled64 };

TilePlan experts_tile_plan(int64_t tokens, int experts) {
  const int64_t per_expert = (2 * tokens + experts - 1) / experts;
  if (tokens <= 16) return TilePlan::kStream16;
  if (per_expert <= 24) return TilePlan::kStream32;
  if (per_expert <= 48) return TilePlan::kStream64;
  return TilePlan::kTiled64;
}

}  // namespace

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
  switch (experts_tile_plan(tokens, experts)) {
    case TilePlan::kStream16: return run_phase<16, true>(phase, args, w, hidden, s);
    case TilePlan::kStream32: return run_phase<32, true>(phase, args, w, hidden, s);
    case TilePlan::kStream64: return run_phase<64, true>(phase, args, w, hidden, s);
    default: return run_phase<64, false>(phase, args, w, hidden, s);
  }
}

}  // namespace parrot
