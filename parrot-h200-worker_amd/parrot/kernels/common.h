// Shared device helpers and the internal launcher API of the Parrot HIP
// inference path (gfx950 / CDNA4, 64-wide wavefronts).
//
// Storage type for bf16 is uint16_t; conversions are bit-exact
// round-to-nearest-even, so every rounding point is explicit in the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace parrot {

constexpr int kWave = 64;
constexpr int kMaxExperts = 32;
constexpr int kMaxDepthSources = 9;
// Assignments (token, k) handled by one route workgroup: 16 tokens x top-2.
constexpr int kRouteTokensPerBlock = 16;
constexpr int kRouteAssignPerBlock = 2 * kRouteTokensPerBlock;
constexpr int kScanChunk = 256;  // route blocks per chunk of the two-level histogram scan
// A route block's row of the block table (launch_route's `block_rows`, read
// by the gate/up launch that groups in-kernel): bytes 0-31 the block's 32
// expert ids in assignment order (kNoExpert for padding tokens), bytes
// 32-63 its number of assignments to each expert (0 past E).
constexpr int kRouteBlockRowBytes = 64;
constexpr uint32_t kNoExpert = 0xff;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// A streaming store of 4 bf16: the nt hint keeps a long output's lines from
// displacing cached inputs and lets HBM take the writes in larger bursts.
__device__ __forceinline__ void store_stream(uint2* dst, uint2 v) {
  u32x2 t;
  t.x = v.x;
  t.y = v.y;
  __builtin_nontemporal_store(t, reinterpret_cast<u32x2*>(dst));
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// IEEE round-to-nearest-even fp32 -> bf16; NaN stays NaN.  gfx950's
// v_cvt_pk_bf16_f32, first operand only: over all 2^32 fp32 patterns its low
// half equals the integer rounding u + 0x7fff + ((u >> 16) & 1) for every
// non-NaN input, denormals included, and keeps NaNs NaN (checked on MI355X).
// The second operand's half rounds fp32 denormals whose discarded bits are
// just above one half (0x00XX8001) down on this part, so the instruction is
// written out here: two conversions the compiler merged into one packed
// instruction would route one of them through that half.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t r;
  asm("v_cvt_pk_bf16_f32 %0, %1, 0" : "=v"(r) : "v"(f));
  return static_cast<uint16_t>(r);
}

// v rounded to bf16 (round to nearest even), as fp32.
__device__ __forceinline__ float bf16_round(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) |
         (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Raw buffer loads: the per-lane byte offset stays fixed over a k loop and
// the step offset travels in an SGPR, so the loop carries no 64-bit address
// arithmetic; reads past `bytes` return zero instead of faulting.
constexpr int kBufferWord3 = 0x00020000;  // gfx9-family buffer resource word 3

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kBufferWord3);
}

__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t voffset,
                                               uint32_t soffset) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset, 0));
}

typedef __attribute__((address_space(3))) void lds_void_t;

// 16 bytes per lane from a buffer straight into LDS: lane l's bytes land at
// lds + 16 l (buffer_load_dwordx4 ... lds).  Reads past the buffer end
// return zero.  (The global_load_lds form is a FLAT-family instruction that
// touches two address spaces, after which the compiler turns every
// vector-memory wait it places into vmcnt(0); the buffer form is not.)
__device__ __forceinline__ void buffer_to_lds16(__amdgpu_buffer_rsrc_t r, void* lds,
                                                uint32_t voffset, uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 16, voffset, soffset, 0, 0);
}

// Waits until at most N vector-memory operations of this wavefront are
// outstanding, then joins the workgroup barrier.  Written out because
// __syncthreads() would also wait for every in-flight direct-to-LDS load
// (vmcnt(0)), which drains a ring of stages on every step.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"i"(N) : "memory");
}

// One RoPE rotation pair (x[2i], x[2i+1]) by angle (c, s), in fp32 with the
// products contracted the same way wherever it is applied, so the fused and
// the stand-alone RoPE paths round identically.
__device__ __forceinline__ float rope_even(float e, float o, float c, float s) {
  return __builtin_fmaf(e, c, -(o * s));
}
__device__ __forceinline__ float rope_odd(float e, float o, float c, float s) {
  return __builtin_fmaf(e, s, o * c);
}

// Attention K and V in MFMA fragment order, per (batch, kv head), in blocks
// of 32 keys, so that every fragment of a key block is one 1 KB contiguous
// wavefront load:
//   K: [blocks][n = 2][s = d / 32][lane = 16 g + c][8]: key 32 blk + 16 n + c,
//      dims 32 s + 8 g .. + 7 (the A operand of S^T = K Q^T);
//   V: [blocks][t = d / 16][lane = 16 g + c][8]: dim 16 t + c, keys
//      32 blk + {4 g .. 4 g + 3, 16 + 4 g .. 16 + 4 g + 3} (the A operand of
//      O^T += V^T P^T with P^T's k order).
// bh = batch * kv_heads + kv head; nblk = ceil(seq / 32); element indices.
__device__ __forceinline__ int64_t kfrag_index(int64_t bh, int nblk, int key, int w, int ks) {
  const int blk = key >> 5, n = (key >> 4) & 1, c = key & 15;
  const int s = w >> 5, g = (w >> 3) & 3, e = w & 7;
  return ((((bh * nblk + blk) * 2 + n) * ks + s) * 64 + 16 * g + c) * 8 + e;
}
__device__ __forceinline__ int64_t vfrag_index(int64_t bh, int nblk, int key, int w, int nt) {
  const int blk = key >> 5, half = (key >> 4) & 1, g = (key >> 2) & 3, j = key & 3;
  const int t = w >> 4, c = w & 15;
  return (((bh * nblk + blk) * nt + t) * 64 + 16 * g + c) * 8 + 4 * half + j;
}

// DPP lane exchange inside rows of 16 lanes (VALU latency, no LDS trip).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the 64 lanes of a wavefront, returned to every lane.  Within each
// row of 16 lanes: quad_perm [1,0,3,2] and [2,3,0,1] (xor 1, xor 2), then
// row_half_mirror and row_mirror fold the quads and half-rows; the four row
// totals are then read from lanes 0, 16, 32, 48 and added in that order.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xb1>(v);
  v += dpp<0x4e>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return ((r0 + r1) + r2) + r3;
}

// ---------------------------------------------------------------------------
// Top-2 across a row of 16 lanes (route.hip, decode_moe.hip)
// ---------------------------------------------------------------------------
// A token's logits are spread over one DPP row: lane j holds experts j and
// j + 16.  Selection is a max-reduction of 64-bit keys (order-preserving
// float bits, then the complemented expert index), so equal logits go to
// the lower expert index: the strict '>' scan in expert order of the
// reference.

// Order-preserving map of a float to uint32 (-0 canonicalised to +0, so it
// ties with +0 as it does under '>').
__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t u = __float_as_uint(v + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t expert_key(float v, int e) {
  return (static_cast<uint64_t>(order_key(v)) << 32) | (0xffffffffu - static_cast<uint32_t>(e));
}

// Inverse of order_key on the high word of a key.
__device__ __forceinline__ float key_value(uint64_t k) {
  const uint32_t o = static_cast<uint32_t>(k >> 32);
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

__device__ __forceinline__ int key_expert(uint64_t k) {
  return static_cast<int>(0xffffffffu - static_cast<uint32_t>(k));
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_max_key(uint64_t k) {
  const int lo = static_cast<int>(static_cast<uint32_t>(k));
  const int hi = static_cast<int>(static_cast<uint32_t>(k >> 32));
  const uint32_t olo = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(lo, lo, CTRL, 0xf, 0xf, false));
  const uint32_t ohi = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(hi, hi, CTRL, 0xf, 0xf, false));
  const uint64_t o = (static_cast<uint64_t>(ohi) << 32) | olo;
  return o > k ? o : k;
}

// Max over the 16 lanes of a DPP row, returned to every lane of the row
// (xor 1, xor 2 inside quads, then half-row and row mirrors).
__device__ __forceinline__ uint64_t row_max_key(uint64_t k) {
  k = dpp_max_key<0xb1>(k);
  k = dpp_max_key<0x4e>(k);
  k = dpp_max_key<0x141>(k);
  return dpp_max_key<0x140>(k);
}

__device__ __forceinline__ float row_sum(float v) {
  v += dpp<0xb1>(v);
  v += dpp<0x4e>(v);
  v += dpp<0x141>(v);
  return v + dpp<0x140>(v);
}

// Top-2 of the logits a DPP row holds (lane j: experts j -> l0 and j + 16 ->
// l1, the latter ignored unless experts > 16): the two expert ids and their
// logits, returned to every lane of the row.
__device__ __forceinline__ void row_top2(float l0, float l1, int experts, int& first,
                                         int& second, float& best_logit, float& runner_logit) {
  const int j = threadIdx.x & 15;
  constexpr uint64_t kNone = 0;  // below every real key
  const uint64_t k0 = j < experts ? expert_key(l0, j) : kNone;
  const uint64_t k1 = j + 16 < experts ? expert_key(l1, j + 16) : kNone;
  const uint64_t mine = k1 > k0 ? k1 : k0;  // k0 wins ties: lower index
  const uint64_t other = k1 > k0 ? k0 : k1;
  const uint64_t best = row_max_key(mine);
  const uint64_t runner = row_max_key(mine == best ? other : mine);
  first = key_expert(best);
  second = key_expert(runner);
  best_logit = key_value(best);
  runner_logit = key_value(runner);
}

// Top-2 of the token whose logits lane j of this DPP row holds for experts
// j (l0) and j + 16 (l1; ignored unless experts > 16), route weights
// renormalised over the two selected exponentials, and the optional logits
// and probabilities.  Every lane of the row calls it; lane 0 of the row
// writes the per-token outputs and returns the two ids in `ids`.
__device__ __forceinline__ void select_top2(float l0, float l1, int experts, int64_t t,
                                            bool valid, float* out_logits, float* probs,
                                            float* weights, int64_t* indices, int* ids) {
  const int j = threadIdx.x & 15;
  const bool has0 = j < experts, has1 = j + 16 < experts;
  int first, second;
  float vb, vr;
  row_top2(l0, l1, experts, first, second, vb, vr);
  if (valid) {
    if (out_logits != nullptr) {
      if (has0) out_logits[t * experts + j] = l0;
      if (has1) out_logits[t * experts + j + 16] = l1;
    }
    if (probs != nullptr) {
      const float p0 = has0 ? __expf(l0 - vb) : 0.0f;
      const float p1 = has1 ? __expf(l1 - vb) : 0.0f;
      const float inv = 1.0f / row_sum(p0 + p1);
      if (has0) probs[t * experts + j] = p0 * inv;
      if (has1) probs[t * experts + j + 16] = p1 * inv;
    }
  }
  if (j == 0) {
    if (valid) {
      const float e2 = __expf(vr - vb);
      const float sel = 1.0f + e2;
      indices[2 * t] = first;
      indices[2 * t + 1] = second;
      weights[2 * t] = 1.0f / sel;
      weights[2 * t + 1] = e2 / sel;
    }
    ids[0] = valid ? first : -1;
    ids[1] = valid ? second : -1;
  }
}

// silu(g) * u with silu(g) = g / (1 + e^-g), evaluated in fp32.
__device__ __forceinline__ float swiglu(float g, float u) {
  return (g / (1.0f + __expf(-g))) * u;
}

// ---------------------------------------------------------------------------
// Launchers (host side, defined next to their kernels).  All return a
// hipError_t; shapes are validated by the C-ABI layer before these run.
// ---------------------------------------------------------------------------

hipError_t launch_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* out,
                           int64_t rows, int dim, float eps, hipStream_t s);

struct DepthSources {
  const uint16_t* src[kMaxDepthSources];
};

// The MoE combine folded into a depth mix: the combined row (as
// launch_combine computes it) is produced in the kernel, written to `out`
// and used as the last of the n_sources depth sources.
struct CombineSource {
  const uint16_t* y_routed;  // bf16 [2 T, dim], route weights applied
  const uint16_t* y_shared;  // bf16 [T, dim]
  const uint16_t* addend;  // optional [T, dim]
  uint16_t* out;           // [T, dim]
};

// An attention output whose sum over heads is deferred to the depth mix
// that reads it (the output projection's per-head contributions of
// launch_causal_attention_out): the mix's last source is made in the kernel
// as bf16(base + bf16(sum over the kPendingHeads heads of contrib)), summed
// in head order, written to `out`.
constexpr int kPendingHeads = 8;
struct PendingSum {
  const float* contrib;    // fp32 [T, kPendingHeads, dim]
  const uint16_t* base;    // optional [T, dim]
  uint16_t* out;           // [T, dim]
};

// Router top-2 computed inside the depth mix whose normalised output is the
// MoE input (route_kernel's results, bit for bit).
struct RouteOut {
  const uint16_t* router_w;  // [E, dim]
  const float* bias;         // optional [E]
  int experts;
  float* weights;            // [T, 2]
  int64_t* indices;          // [T, 2]
};

// comb: optional (nullptr: every source is read from srcs).  route:
// optional; needs out_norm.
// The forward's first launch: embedding rows by id (written to rows_out) and
// their single-source depth mix + RMSNorm (out_norm); zero-fills n_zeros
// floats at zeros (see norm.hip).
hipError_t launch_embed_mix(const int64_t* ids, const uint16_t* table, int64_t vocab,
                            const uint16_t* query, const uint16_t* score_w, float score_eps,
                            const uint16_t* out_norm_w, float out_eps, int64_t tokens, int dim,
                            uint16_t* rows_out, uint16_t* out_norm, float* zeros, int n_zeros,
                            hipStream_t s);

hipError_t launch_depth_mix(const DepthSources& srcs, int n_sources,
                            const uint16_t* query, const uint16_t* score_w,
                            float score_eps, const uint16_t* out_norm_w,
                            float out_eps, int64_t tokens, int dim,
                            uint16_t* out_mix, uint16_t* out_norm, const CombineSource* comb,
                            const RouteOut* route, hipStream_t s,
                            const PendingSum* pend = nullptr);

// Routing: router projection (or given fp32 logits) + top-2 + per-block
// stable ranks.  Writes block-local ranks into `positions` and per-block
// expert histograms into `block_counts` [n_blocks, experts]; with
// `block_rows` (tokens below kWideRouteTokens), the block table
// [n_blocks, kRouteBlockRowBytes].
hipError_t launch_route(const uint16_t* x, const uint16_t* router_w,
                        const float* given_logits, const float* bias,
                        int64_t tokens, int dim, int experts, float* out_logits,
                        float* probs, float* weights, int64_t* indices,
                        int32_t* positions, int32_t* block_counts, uint8_t* block_rows,
                        hipStream_t s);

// Whether launch_route writes `block_rows` for this many tokens.
bool route_block_rows_supported(int64_t tokens);

// Number of 16-token route blocks (= rows of block_counts) for `tokens`.
int route_blocks(int64_t tokens);

// Rows of the chunk-total table the group step needs beside block_counts
// (0 when one chunk holds every route block).
int route_chunks(int64_t tokens);

// Block-local ranks for externally supplied top-2 indices.
hipError_t launch_rank_indices(const int64_t* indices, int64_t tokens, int experts,
                               int32_t* positions, int32_t* block_counts,
                               hipStream_t s);

// Turns block-local ranks into global stable positions and writes the
// fixed-capacity map, the expert-contiguous overflow list and the offsets
// table: offsets[0..E] = exclusive prefix of counts, offsets[E+1..2E+1] =
// exclusive prefix of per-expert overflow counts.
// `chunk_totals` [route_chunks(tokens), experts] is scratch (unused when
// route_chunks is 0).
hipError_t launch_group(const int64_t* indices, int64_t tokens, int experts,
                        int capacity, const int32_t* block_counts, int32_t* chunk_totals,
                        int32_t* positions, int32_t* counts, int32_t* offsets,
                        int32_t* perm, int32_t* overflow, hipStream_t s);

struct ExpertWeights {
  const uint16_t* gate_up;         // [E, 2H, dim], gate/up interleaved per 16 rows
  const uint16_t* down;            // [E, dim, H]
  const uint16_t* shared_gate_up;  // [2Hs, dim], interleaved the same way
  const uint16_t* shared_down;     // [dim, Hs]
};

struct GroupMap {
  const int32_t* counts;    // [E]
  const int32_t* offsets;   // [2E+2]
  const int32_t* perm;      // [E, C]
  const int32_t* overflow;  // [2T]
  const float* weights;     // [2T] route weights
  // Grouping inside the gate/up launch (experts_group_in_kernel): phase 1
  // reads the top-2 `indices` instead of counts / offsets / perm / overflow
  // and writes `counts_out`, `offsets_out` and `sorted` (the assignment id of
  // each hidden row); phase 2 then reads counts / offsets / sorted.
  const int64_t* indices = nullptr;  // [2T]
  // ... or the route's block table (launch_route's block_rows) instead of
  // the indices, past the assignments the indices form takes.
  const uint8_t* route_blocks = nullptr;  // [ceil(T / 16), kRouteBlockRowBytes]
  int32_t* counts_out = nullptr;     // [E]
  int32_t* offsets_out = nullptr;    // [2E+2]
  const int32_t* sorted = nullptr;   // [2T], phase 2
  int32_t* sorted_out = nullptr;     // [2T], phase 1
};

// Whether a gate/up launch can group its assignments itself (the streaming
// kernel's shapes): kGroupFromIds from the top-2 indices (at most 2048
// assignments, ~3 x 32 rows per expert), kGroupFromBlocks from the route's
// block table (at most 256 route blocks), else kGroupNone.
enum GroupInKernel { kGroupNone = 0, kGroupFromIds = 1, kGroupFromBlocks = 2 };
GroupInKernel experts_group_in_kernel(int64_t tokens, int dim, int experts, int hidden_dim,
                                      int shared_dim);

// Grouped SwiGLU expert GEMM over every routed assignment plus the shared
// expert.  Phase 1 (gate/up + SwiGLU) reads x and writes hidden
// [3T, max(H, Hs)] bf16; phase 2 (down) reads hidden and writes y_routed
// [2T, dim] (route-weighted, assignment order) and y_shared [T, dim], each
// value the bf16 rounding of its fp32 result.
hipError_t launch_expert_gemm(int phase, const uint16_t* x, int64_t tokens, int dim,
                              int experts, int hidden_dim, int shared_dim, int capacity,
                              const GroupMap& map, const ExpertWeights& w, uint16_t* hidden,
                              uint16_t* y_routed, uint16_t* y_shared, hipStream_t s);

// RoPE + head-major split of a packed q|k|v projection (see rope.hip).
// The first position is start (+ *start_device when non-null); positions
// past the table are clamped to its last row.
// With vt_keys > 0, v is written transposed: [batch, Hk, head_dim, vt_keys].
hipError_t launch_rope_qkv(const uint16_t* qkv, const float* cos_t, const float* sin_t,
                           int64_t batch, int seq, int start, const int32_t* start_device,
                           int max_positions, int heads, int kv_heads, int head_dim,
                           int expand_kv, int vt_keys, uint16_t* q, uint16_t* k, uint16_t* v,
                           hipStream_t s);

// Decode-step attention over the generation caches (see decode.hip); the
// position is read from device memory.
constexpr size_t kMaxDecodeLds = 64 * 1024;  // dynamic LDS without an opt-in
bool decode_head_dim_supported(int head_dim);  // 8, 16, 32, 64, 96, 128, 192, 256
size_t decode_attention_lds_bytes(int window, int max_pos, int head_dim);
hipError_t launch_decode_attention(const uint16_t* q, const uint16_t* k_new,
                                   const uint16_t* v_new, uint16_t* k_cache, uint16_t* v_cache,
                                   const int32_t* position, int batch, int heads, int kv_heads,
                                   int head_dim, int max_pos, int window, float scale,
                                   uint16_t* out, hipStream_t s);
// The deferred form for bf16 queries: per-head contributions of the output
// projection, contributions [batch, heads, dim] fp32 = the head's output
// (rounded to bf16) times its [dim, head_dim] slice of out_weight [dim,
// heads x head_dim]; kDecodeHeadsParts workgroups per head split the
// output columns (dim / kDecodeHeadsParts <= 256).  The launch's LDS is
// decode_attention_lds_bytes + head_dim floats.
constexpr int kDecodeHeadsParts = 16;
hipError_t launch_decode_attention_heads(const uint16_t* q, const uint16_t* k_new,
                                         const uint16_t* v_new, uint16_t* k_cache,
                                         uint16_t* v_cache, const int32_t* position, int batch,
                                         int heads, int kv_heads, int head_dim, int max_pos,
                                         int window, float scale, const uint16_t* out_weight,
                                         int dim, float* contributions, hipStream_t s);
size_t mla_decode_lds_bytes(int tokens, int k, int elem_bytes);
hipError_t launch_decode_linear(const uint16_t* x, int tokens, int k, const uint16_t* w, int n,
                                const uint16_t* addend, uint16_t* out, hipStream_t s);
hipError_t launch_mla_decode_out(const float* ctx, int tokens, int width, const uint16_t* wo,
                                 int dim, const uint16_t* addend, uint16_t* out, hipStream_t s);
hipError_t launch_decode_attention_latent(const float* q, const uint16_t* latent_new,
                                          uint16_t* latent_cache, const int32_t* position,
                                          int batch, int heads, int latent_dim, int max_pos,
                                          float scale, float* out, hipStream_t s);

// Fused MoE layer for T <= decode_moe_max_tokens() tokens (see
// decode_moe.hip): route + gate/up + SwiGLU, then down + weighted combine
// (+ addend).  `hidden` is scratch [3T, max(H, Hs)] bf16.
int decode_moe_max_tokens();
// The depth mix + RMSNorm that makes a decode MoE's input row per token
// (n_sources == 0: the input x is given instead); dim <= 1024.
//
// A pending last source (pend != nullptr; decode MoE only) is resolved in
// the launch, as the reference's depth_mix_norm_pending_bf16: row t of
// source n_sources - 1 is bf16(base + bf16(sum over lanes l in order of
// pend[t, l, :])) (just the rounded sum without a base), and the launch
// writes that row to pend_out [tokens, dim].
struct DecodeMix {
  DepthSources srcs;
  int n_sources;
  const uint16_t* query;
  const uint16_t* score_w;
  float score_eps;
  const uint16_t* out_w;
  float out_eps;
  const float* pend;          // [tokens, pend_lanes, dim] fp32
  int pend_lanes;             // 1 .. kMaxPendingLanes
  const uint16_t* pend_base;  // [tokens, dim] or nullptr
  uint16_t* pend_out;         // [tokens, dim]
};
constexpr int kMaxPendingLanes = 16;

// The decode step's q|k|v projection + RoPE of a local layer (decode_qkv.hip).
struct DecodeQkvArgs {
  DecodeMix mix;            // n_sources > 0: the input rows are mixed in the launch
  const uint16_t* x;        // else the input rows [tokens, dim]
  int tokens, dim;
  const uint16_t* w;        // q|k|v weight [(H + 2 Hk) d, dim], row-major bf16
  int heads, kv_heads, head_dim;
  const float* cos_t;       // [max_positions, d / 2]
  const float* sin_t;
  int max_positions;
  const int32_t* position;  // device position of the new token
  uint16_t* q;              // [tokens, H, 1, d]
  uint16_t* k;              // [tokens, Hk, 1, d]
  uint16_t* v;              // [tokens, Hk, 1, d]
  // With gather_ids, the mix's single source is gathered in the launch:
  // row gather_ids[t] (clamped into [0, gather_rows)) of gather_table
  // [gather_rows, dim], also stored to gather_out [tokens, dim].
  const int64_t* gather_ids;
  const uint16_t* gather_table;
  int gather_rows;
  uint16_t* gather_out;
};
int decode_qkv_max_dim();
hipError_t launch_mla_decode_in(const uint16_t* x, const DecodeMix* mix, int tokens, int dim,
                                const uint16_t* wq, int nq, const uint16_t* wkv, int nl,
                                float* q_out, uint16_t* lat_out, hipStream_t s);
hipError_t launch_decode_qkv(const DecodeQkvArgs& a, hipStream_t s);

hipError_t launch_decode_moe(const uint16_t* x, const DecodeMix* mix, int tokens, int dim,
                             int experts, int hidden_dim, int shared_dim,
                             const uint16_t* router_w, const float* bias, const ExpertWeights& w,
                             const uint16_t* addend, uint16_t* out, int64_t* indices,
                             float* weights, uint16_t* hidden, hipStream_t s);

// Greedy token per row of h [rows <= vocab_argmax_max_rows(), dim] over a
// [vocab, dim] head, fp32 logits (see vocab.hip); part_v / part_i hold
// rows x vocab_argmax_groups(vocab) partials.
int vocab_argmax_max_rows();
int vocab_argmax_groups(int vocab);
hipError_t launch_vocab_argmax(const uint16_t* h, int rows, int dim, const uint16_t* w, int vocab,
                               float* part_v, int32_t* part_i, int64_t* out, int32_t* advance, hipStream_t s);

// Causal / sliding-window attention (see attention.hip).  Strides are in
// elements: [batch, head, row] for q and k (unit stride along head_dim),
// [batch, head, dim row] for the transposed values vt (unit stride along the
// keys, rows of at least roundup(seq, 32) keys); out [batch, seq, heads,
// head_dim].
bool attention_head_dim_supported(int head_dim);  // 64, 96, 128
// k_strides == vt_strides == nullptr: k and vt are K and V in fragment order
// (kfrag_index / vfrag_index).
hipError_t launch_causal_attention(const uint16_t* q, const uint16_t* k, const uint16_t* vt,
                                   const int64_t* q_strides, const int64_t* k_strides,
                                   const int64_t* vt_strides, int batch, int seq, int heads,
                                   int kv_heads, int head_dim, int window, float scale,
                                   uint16_t* out, hipStream_t s);
// Fragment-order K and V; instead of the output, each head's share of the
// output projection: contrib [batch, seq, heads, n_out] fp32 = y_h W_h^T
// with w_out packed as parrot_proj_bf16's weights (n_out rows, heads *
// head_dim columns).  n_out from attention_out_width_supported.
bool attention_out_width_supported(int n_out);  // 512, 768, 1024
hipError_t launch_causal_attention_out(const uint16_t* q, const uint16_t* k_frag,
                                       const uint16_t* v_frag, const int64_t* q_strides, int batch,
                                       int seq, int heads, int kv_heads, int head_dim, int window,
                                       float scale, const uint16_t* w_out, int n_out,
                                       float* contrib, hipStream_t s);

hipError_t launch_combine(const uint16_t* y_routed, const uint16_t* y_shared,
                          const uint16_t* addend, int64_t tokens, int dim,
                          uint16_t* out, hipStream_t s);

// Dense projections y = x W^T, W packed in MFMA fragment order (proj.hip).
bool proj_shape_supported(int k, int n);  // k % 64 == 0, k <= 2048, n % 16 == 0
hipError_t launch_proj_store(const uint16_t* x, int rows, int k, int64_t lda, const uint16_t* w,
                             int n, const uint16_t* addend, int64_t ld_addend, uint16_t* out,
                             int64_t ldo, hipStream_t s);
hipError_t launch_proj_transposed(const uint16_t* x, int rows, int seq, int k, const uint16_t* w,
                                  int n, int ld_keys, uint16_t* out, hipStream_t s);
hipError_t launch_proj_rope_qkv(const uint16_t* x, int rows, int seq, int dim, const uint16_t* w,
                                const float* cos_t, const float* sin_t, int start,
                                const int32_t* start_device, int max_positions, int heads,
                                int kv_heads, int head_dim, int vt_keys, uint16_t* q,
                                uint16_t* k, uint16_t* v, uint16_t* kf, uint16_t* vf,
                                hipStream_t s);
// kf and/or vf; with both, w is [Wk; Wv] and n counts both halves.
hipError_t launch_proj_frag(const uint16_t* x, int rows, int seq, int k, int64_t lda,
                            const uint16_t* w, int n, int head_dim, uint16_t* kf, uint16_t* vf,
                            hipStream_t s);

// Attained-peak microkernels (peak.hip).
hipError_t launch_peak_mfma(int wide, int64_t blocks, int iters, float* out, hipStream_t s);
int64_t peak_mfma_flops_per_block(int wide, int iters);
hipError_t launch_peak_copy(const void* src, void* dst, int64_t bytes, int64_t blocks,
                            hipStream_t s);

}  // namespace parrot
