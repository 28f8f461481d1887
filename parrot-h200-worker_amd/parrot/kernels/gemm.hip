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
  uint16_t* y_routed;         // phase 2 output bf16 [2T, dim]
  uint16_t* y_shared;         // phase 2 output bf16 [T, dim]
  // Grouping inside phase 1 (group_find, group_rows): top-2 ids in; counts,
  // offsets and the hidden rows' assignment ids out.  Phase 2 with `sorted`
  // reads a row's assignment id there instead of perm / overflow.
  const int64_t* indices;
  const uint8_t* route_blocks;  // or the route's block table (group_find_blocks)
  int32_t* counts_out;
  int32_t* offsets_out;
  int32_t* sorted_out;
  const int32_t* sorted;
  // Tile order (streaming kernel): 0 = the grid's own (XCD x gets column tile
  // x of every row tile), 1 = row-major per XCD (every column tile of row
  // tiles x, x + 8, ...); see xcd_tile.
  int rows_per_xcd;
};

// (row tile, column tile) of this workgroup.  Workgroups are dispatched
// round-robin over the 8 XCDs by linear id; with `rows_per_xcd` the workgroups
// of XCD x take row tiles x, x + 8, ... with all their column tiles in turn
// (the grid's row count is then a multiple of 8), so an XCD's L2 holds a few
// row tiles' A rows and the weights of their experts, instead of every row
// tile's A rows and one column tile of every expert's weights.
struct TileIndex {
  int m, n;
};

__device__ __forceinline__ TileIndex xcd_tile(bool rows_per_xcd) {
  if (!rows_per_xcd) return TileIndex{static_cast<int>(blockIdx.y), static_cast<int>(blockIdx.x)};
  const int nx = static_cast<int>(gridDim.x);
  const int id = static_cast<int>(blockIdx.y) * nx + static_cast<int>(blockIdx.x);
  const int pos = id >> 3;
  const int q = pos / nx;
  return TileIndex{q * 8 + (id & 7), pos - q * nx};
}

// Every kernel argument a GEMM prologue reads (and the grid width), in one
// batch of scalar loads before any use: a field first read inside a branch
// costs a scalar round trip of its own.
__device__ __forceinline__ void load_gemm_args(const GemmArgs& p) {
  asm volatile("" ::"s"(p.tokens), "s"(p.dim), "s"(p.experts), "s"(p.hidden_dim),
               "s"(p.shared_dim), "s"(p.capacity), "s"(p.hstride), "s"(p.counts),
               "s"(p.offsets), "s"(p.perm), "s"(p.overflow), "s"(p.sorted), "s"(p.indices),
               "s"(p.w_routed), "s"(p.w_shared), "s"(p.a_src), "s"(p.weights),
               "s"(p.hidden_out), "s"(p.y_routed), "s"(p.y_shared), "s"(p.counts_out),
               "s"(p.offsets_out), "s"(p.sorted_out), "s"(p.rows_per_xcd), "s"(gridDim.x),
               "s"(p.route_blocks));
  __builtin_amdgcn_sched_barrier(0);
}

// The row tile a workgroup owns: segment `seg` (E = the shared expert),
// M-tile `mt` of its `rows` rows; the segment's hidden rows start at `hbase`
// and its part of the overflow list at `obase`.
struct Tile {
  int seg, mt, rows, hbase, obase;
};

// Which tile does this workgroup own?  The shared expert's tiles come first
// and need no load.  For routed tiles one batch of vector loads fetches the
// expert counts and both offset tables (lane e holds expert e's entries),
// then a uniform scan over the lanes' tile counts with readlane picks the
// segment -- one memory hop, no chain of dependent loads.
template <int BM>
__device__ __forceinline__ bool find_tile(const GemmArgs& p, int T, Tile& t,
                                          int m = static_cast<int>(blockIdx.y)) {
  const int shared_tiles = (T + BM - 1) / BM;
  if (m < shared_tiles) {
    t = Tile{p.experts, m, T, 2 * T, 0};
    return true;
  }
  const int lane = threadIdx.x & (kWave - 1);
  const bool mine = lane < p.experts;  // experts <= kMaxExperts < kWave
  const int count = mine ? p.counts[lane] : 0;
  const int hoff = mine ? p.offsets[lane] : 0;
  const int ooff = mine ? p.offsets[p.experts + 1 + lane] : 0;
  const int tiles = (count + BM - 1) / BM;
  m -= shared_tiles;
  for (int e = 0; e < p.experts; ++e) {
    const int te = __builtin_amdgcn_readlane(tiles, e);
    if (m < te) {
      t = Tile{e, m, __builtin_amdgcn_readlane(count, e), __builtin_amdgcn_readlane(hoff, e),
               __builtin_amdgcn_readlane(ooff, e)};
      return true;
    }
    m -= te;
  }
  return false;
}

// The tile's fields are wavefront-uniform by construction; readfirstlane
// lets the compiler see it, so the weight buffer descriptor built from them
// stays in SGPRs (a descriptor it cannot prove uniform costs a readfirstlane
// loop around every buffer load).
__device__ __forceinline__ Tile uniform_tile(const Tile& t) {
  return Tile{__builtin_amdgcn_readfirstlane(t.seg), __builtin_amdgcn_readfirstlane(t.mt),
              __builtin_amdgcn_readfirstlane(t.rows), __builtin_amdgcn_readfirstlane(t.hbase),
              __builtin_amdgcn_readfirstlane(t.obase)};
}

// Segment row of tile row r; padding rows past the segment's end clamp onto
// the tile's first row (they are computed but never stored).
__device__ __forceinline__ int segment_row(const Tile& t, int BM, int r) {
  const int s = t.mt * BM + r;
  return s < t.rows ? s : t.mt * BM;
}

// Assignment id of routed segment row s: in-capacity rows from the slot
// map, the rest from the expert's part of the overflow list (or, after a
// phase 1 that grouped in-kernel, the hidden rows' id list).
__device__ __forceinline__ int assignment_of(const GemmArgs& p, const Tile& t, int s) {
  if (p.sorted != nullptr) return p.sorted[t.hbase + s];
  return s < p.capacity ? p.perm[static_cast<int64_t>(t.seg) * p.capacity + s]
                        : p.overflow[t.obase + s - p.capacity];
}

// ---------------------------------------------------------------------------
// Grouping inside the gate/up launch, for up to kGroupMaxAssign assignments:
// the tile, its rows and the grouping outputs straight from the top-2 ids,
// with the same results as the route + group kernels (stable slot order:
// segment row s of expert e is e's assignment of rank s in ascending
// assignment order, in-capacity slots then overflow; ids outside
// [0, experts) take no row).  Every routed workgroup
//   1. (group_find) loads all 2T ids (one memory hop; wavefront w owns the
//      64-id chunks w, w + 4, ...), histograms them with LDS atomics (one
//      histogram per wavefront), and finds its tile from prefix sums of the
//      counts over lanes;
//   2. (group_rows, once its weight loads are in flight) ranks its expert's
//      ids: a ballot per chunk gives the chunk's count (exchanged through
//      LDS, prefix-summed over lanes) and each id's rank within the chunk
//      (mbcnt).
// Rows of the tile land in row_src (token) / row_dst (hidden row); padding
// rows read token 0 and store nothing.  The workgroup of the first routed
// tile row, column 0, writes counts and both offset tables; column-0
// workgroups write the hidden rows' assignment ids.
constexpr int kGroupChunksPerWave = 8;
constexpr int kGroupMaxAssign = 4 * kGroupChunksPerWave * kWave;  // 2048

// Inclusive prefix sum over lanes 0-31 (lanes 32-63: unspecified): row
// shifts by 1, 2, 4, 8 within each 16-lane row, then lane 15 broadcast into
// the second row.  Lanes shifted in from outside a row add 0.
__device__ __forceinline__ int scan32(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  return v;
}

struct GroupIds {
  // group_find: this lane's ids, chunk w + 4 j (-1: none); group_find_blocks:
  // the count words of this thread's route block (zero past the last).
  int ids[kGroupChunksPerWave];
};

// The routed tile of row tile m (counted past the shared expert's tiles)
// from lane e's count of expert e: its tiles and overflow rows, and their
// exclusive prefixes over the experts before it.  The first routed
// workgroup of column 0 writes counts and both offset tables.  False
// (uniform) when no expert has tile m.
template <int BM>
__device__ __forceinline__ bool locate_tile(const GemmArgs& p, int count, int m, TileIndex ti,
                                            Tile& t) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int E = p.experts;
  const int tiles = (count + BM - 1) / BM;
  const int ovf = max(0, count - p.capacity);
  const int tile0 = scan32(tiles) - tiles;
  const int h_end = scan32(count);
  const int o_end = scan32(ovf);
  if (ti.n == 0 && m == 0 && wave == 0) {
    const int h_total = __builtin_amdgcn_readlane(h_end, E - 1);
    const int o_total = __builtin_amdgcn_readlane(o_end, E - 1);
    if (lane < E) {
      p.counts_out[lane] = count;
      p.offsets_out[lane] = h_end - count;
      p.offsets_out[E + 1 + lane] = o_end - ovf;
    }
    if (lane == E) {
      p.offsets_out[E] = h_total;
      p.offsets_out[2 * E + 1] = o_total;
    }
  }
  const uint64_t hit = __ballot(lane < E && m >= tile0 && m < tile0 + tiles);
  if (hit == 0) return false;  // uniform: no tile for this workgroup
  const int seg = static_cast<int>(__builtin_ctzll(hit));
  t = Tile{seg, m - __builtin_amdgcn_readlane(tile0, seg), __builtin_amdgcn_readlane(count, seg),
           __builtin_amdgcn_readlane(h_end - count, seg),
           __builtin_amdgcn_readlane(o_end - ovf, seg)};
  return true;
}

template <int BM>
__device__ __forceinline__ bool group_find(const GemmArgs& p, int T, Tile& t, GroupIds& g,
                                           int* row_src, int* row_dst,
                                           int (*hist_s)[kMaxExperts], TileIndex ti) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int shared_tiles = (T + BM - 1) / BM;
  int m = ti.m;
  if (m < shared_tiles) {
    t = Tile{p.experts, m, T, 2 * T, 0};
    return true;
  }
  const int E = p.experts;
  const int n_assign = 2 * T;
#pragma unroll
  for (int j = 0; j < kGroupChunksPerWave; ++j) {
    const int a = (wave + 4 * j) * kWave + lane;
    const int64_t e = a < n_assign ? p.indices[a] : -1;
    g.ids[j] = e >= 0 && e < E ? static_cast<int>(e) : -1;
  }
  // One histogram per wavefront: its zeroing and its atomics are one
  // wavefront's LDS operations, which execute in order.
  if (lane < kMaxExperts) hist_s[wave][lane] = 0;
#pragma unroll
  for (int j = 0; j < kGroupChunksPerWave; ++j)
    if (g.ids[j] >= 0) atomicAdd(&hist_s[wave][g.ids[j]], 1);
  if (tid < BM) {
    row_src[tid] = 0;
    row_dst[tid] = -1;
  }
  __syncthreads();

  // Lane e: expert e's count.
  const int count =
      lane < E ? hist_s[0][lane] + hist_s[1][lane] + hist_s[2][lane] + hist_s[3][lane] : 0;
  return locate_tile<BM>(p, count, m - shared_tiles, ti, t);
}

template <int BM>
__device__ __forceinline__ void group_rows(const GemmArgs& p, int T, const Tile& t,
                                           const GroupIds& g, int* row_src, int* row_dst,
                                           int* chunk_s, bool first_column) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nchunks = (2 * T + kWave - 1) / kWave;
  uint64_t mask[kGroupChunksPerWave];
#pragma unroll
  for (int j = 0; j < kGroupChunksPerWave; ++j) {
    mask[j] = __ballot(g.ids[j] == t.seg);
    const int c = wave + 4 * j;
    if (lane == 0 && c < nchunks) chunk_s[c] = __popcll(mask[j]);
  }
  __syncthreads();
  // Lane c: the expert's ids in chunks before c.
  const int per_chunk = lane < nchunks ? chunk_s[lane] : 0;
  const int before = scan32(per_chunk) - per_chunk;
#pragma unroll
  for (int j = 0; j < kGroupChunksPerWave; ++j) {
    const int c = wave + 4 * j;
    if (c < nchunks && g.ids[j] == t.seg) {
      const uint64_t mk = mask[j];
      const int rank = __builtin_amdgcn_readlane(before, c) +
                       static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                           static_cast<uint32_t>(mk >> 32),
                           __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mk), 0u)));
      const int r = rank - t.mt * BM;
      if (r >= 0 && r < BM) {
        const int a = c * kWave + lane;
        row_src[r] = a >> 1;
        row_dst[r] = t.hbase + rank;
        if (first_column) p.sorted_out[t.hbase + rank] = a;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Grouping inside the gate/up launch from the route's block table (up to
// kGroupMaxRouteBlocks route blocks, one per thread): the same tile, rows
// and outputs as group_find / group_rows, without reading all 2T ids.
//   1. (group_find_blocks) thread b loads the count half of route block b's
//      table row; the per-expert counts are those bytes summed over the
//      workgroup, as 16-bit pairs (a wavefront's sums stay below 2^16);
//   2. (group_rows_blocks) thread b takes block b's count of its tile's
//      expert from the same bytes, an exclusive scan over the blocks gives
//      the block's first rank, and only the threads whose ranks meet the
//      tile load their block's ids and place those rows in assignment
//      order.  Reading the id half only there keeps the table traffic of a
//      launch (every workgroup reads every block's counts) at 32 bytes per
//      block per workgroup.
constexpr int kGroupMaxRouteBlocks = 256;

// Inclusive prefix sum over the 64 lanes: row shifts by 1, 2, 4, 8, then
// lane 15 broadcast into the next row and lane 31 into rows 2 and 3.
__device__ __forceinline__ uint32_t scan64(uint32_t v) {
  v += __builtin_amdgcn_update_dpp(0u, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0u, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0u, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0u, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0u, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0u, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

template <int BM>
__device__ __forceinline__ bool group_find_blocks(const GemmArgs& p, int T, Tile& t, GroupIds& g,
                                                  int* row_src, int* row_dst,
                                                  int (*hist_s)[kMaxExperts], TileIndex ti) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int shared_tiles = (T + BM - 1) / BM;
  const int m = ti.m;
  if (m < shared_tiles) {
    t = Tile{p.experts, m, T, 2 * T, 0};
    return true;
  }
  const int E = p.experts;
  const int n_blocks = (T + kRouteTokensPerBlock - 1) / kRouteTokensPerBlock;
  const bool mine = tid < n_blocks;
  const uint4* row = reinterpret_cast<const uint4*>(
      p.route_blocks + static_cast<int64_t>(mine ? tid : 0) * kRouteBlockRowBytes);
  const uint4 cnt0 = row[2], cnt1 = row[3];
  const uint32_t cw[8] = {cnt0.x, cnt0.y, cnt0.z, cnt0.w, cnt1.x, cnt1.y, cnt1.z, cnt1.w};
  // Kept for group_rows_blocks: this block's count words (zero past the end).
#pragma unroll
  for (int k = 0; k < 8; ++k) g.ids[k] = static_cast<int>(mine ? cw[k] : 0u);
  if (tid < BM) {
    row_src[tid] = 0;
    row_dst[tid] = -1;
  }
  // Count word k holds experts 4k .. 4k + 3 (byte r = expert 4k + r): its
  // even bytes (experts 4k, 4k + 2) and odd bytes (4k + 1, 4k + 3) as
  // 16-bit pairs, summed over the wavefront into lane 63.
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t w = static_cast<uint32_t>(g.ids[k]);
    const uint32_t even = scan64(w & 0x00ff00ffu);
    const uint32_t odd = scan64((w >> 8) & 0x00ff00ffu);
    if (lane == kWave - 1) {
      hist_s[wave][2 * k] = static_cast<int>(even);
      hist_s[wave][2 * k + 1] = static_cast<int>(odd);
    }
  }
  __syncthreads();
  // Lane e: expert e's count, from pair 2 (e / 4) + (e % 2), half (e / 2) % 2.
  int count = 0;
  if (lane < E) {
    const int w = 2 * (lane >> 2) + (lane & 1);
    const int sh = (lane & 2) ? 16 : 0;
#pragma unroll
    for (int v = 0; v < 4; ++v) count += (static_cast<uint32_t>(hist_s[v][w]) >> sh) & 0xffffu;
  }
  return locate_tile<BM>(p, count, m - shared_tiles, ti, t);
}

template <int BM>
__device__ __forceinline__ void group_rows_blocks(const GemmArgs& p, const Tile& t,
                                                  const GroupIds& g, int* row_src, int* row_dst,
                                                  int* scan_s, bool first_column) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Block tid's count of expert t.seg: byte seg % 4 of count word seg / 4.
  uint32_t word = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) word = k == (t.seg >> 2) ? static_cast<uint32_t>(g.ids[k]) : word;
  const int c = static_cast<int>((word >> (8 * (t.seg & 3))) & 0xffu);
  const int inc = static_cast<int>(scan64(static_cast<uint32_t>(c)));
  if (lane == kWave - 1) scan_s[wave] = inc;
  __syncthreads();
  int base = inc - c;
#pragma unroll
  for (int v = 0; v < 3; ++v) base += v < wave ? scan_s[v] : 0;
  const int r_lo = t.mt * BM;
  if (c > 0 && base < r_lo + BM && base + c > r_lo) {
    const uint4* row =
        reinterpret_cast<const uint4*>(p.route_blocks + static_cast<int64_t>(tid) * kRouteBlockRowBytes);
    const uint4 id0 = row[0], id1 = row[1];
    const uint32_t ids[8] = {id0.x, id0.y, id0.z, id0.w, id1.x, id1.y, id1.z, id1.w};
    int rank = base;
#pragma unroll
    for (int j = 0; j < kRouteAssignPerBlock; ++j) {
      const int id = static_cast<int>((ids[j >> 2] >> (8 * (j & 3))) & 0xffu);
      if (id == t.seg) {
        const int r = rank - r_lo;
        if (r >= 0 && r < BM) {
          const int a = tid * kRouteAssignPerBlock + j;
          row_src[r] = a >> 1;
          row_dst[r] = t.hbase + rank;
          if (first_column) p.sorted_out[t.hbase + rank] = a;
        }
        ++rank;
      }
    }
  }
}

template <int BM>
struct WaveLayout {
  static constexpr int kWavesM = BM >= 64 ? 2 : 1;
  static constexpr int kWavesN = 4 / kWavesM;
};

// One 16-byte MFMA fragment from LDS, read with inline asm so the compiler
// does not treat it as an LDS access: otherwise it cannot tell the ring slot
// being read from the slots the in-flight direct-to-LDS loads fill, and
// waits for all of them (vmcnt(0)), draining the pipeline every step.  The
// ring's ordering is explicit instead (wait_vm_barrier), and the caller waits
// for the reads with lds_wait before using the fragments.
__device__ __forceinline__ bf16x8 lds_read_frag(const uint16_t* p) {
  const uint32_t addr = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint16_t*)p));
  bf16x8 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}

// Waits until at most N LDS operations of this wavefront are outstanding
// (they complete in order), then ties the fragments read before those N to
// the wait so no use of them is scheduled before it.
template <int N, int NA, int NB>
__device__ __forceinline__ void lds_wait_upto(bf16x8 (&a)[NA], bf16x8 (&b)[NB]) {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N));
#pragma unroll
  for (int i = 0; i < NA; ++i) asm volatile("" : "+v"(a[i]));
#pragma unroll
  for (int i = 0; i < NB; ++i) asm volatile("" : "+v"(b[i]));
}

// Waits for every outstanding LDS read of this wavefront, then ties the
// fragments to the wait so no use of them is scheduled before it.
template <int NA, int NB>
__device__ __forceinline__ void lds_wait(bf16x8 (&a)[NA], bf16x8 (&b)[NB]) {
  asm volatile("s_waitcnt lgkmcnt(0)");
#pragma unroll
  for (int i = 0; i < NA; ++i) asm volatile("" : "+v"(a[i]));
#pragma unroll
  for (int i = 0; i < NB; ++i) asm volatile("" : "+v"(b[i]));
}

// ---------------------------------------------------------------------------
// LDS-pipelined grouped GEMM: a ring of S k-stages (BK = 64) in LDS, filled
// by direct-to-LDS buffer loads with S - 1 stages in flight while the MFMAs
// consume the oldest; one barrier per k step.
//
// Every operand tile is stored in LDS in MFMA fragment order: 1 KB blocks of
// 16 rows x 32 k where lane l's 16 bytes (row l % 16, k 8 (l / 16) .. +8) sit
// at byte 16 l.  A direct-to-LDS load writes lane l's 16 bytes at 16 l, so
// one wavefront load fills one block, and one ds_read_b128 per lane reads a
// whole fragment without bank conflicts.  The packed weights are already in
// this order in HBM (each block is 1 KB contiguous); A blocks are gathered
// row by row through the index map.
//
// Stage layout: A blocks (m-tile i, k half h) at block 2 i + h, then B
// blocks (16-column group g, k half h) at block BM / 8 + 2 g + h.  Wavefront w
// loads blocks [w P, w P + P) of every stage, P = (BM + BN) / 32.
template <int BM, int BN, int S, int PHASE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2)))
void grouped_gemm_kernel(GemmArgs p) {
  constexpr int kWavesM = WaveLayout<BM>::kWavesM;
  constexpr int kWavesN = WaveLayout<BM>::kWavesN;
  constexpr int kWaveM = BM / kWavesM;
  constexpr int kWaveN = BN / kWavesN;
  constexpr int kTilesM = kWaveM / 16;
  constexpr int kTilesN = kWaveN / 16;
  constexpr int kABlocks = BM / 8;                      // 16-row tiles x 2 k halves
  constexpr int kBlocks = (BM + BN) / 8;
  constexpr int P = kBlocks / 4;                        // loads per wavefront per stage
  constexpr int kStageElems = kBlocks * 512;
  static_assert(kBlocks % 4 == 0, "stage blocks must split evenly over 4 wavefronts");
  static_assert(PHASE != 1 || kWaveN % 32 == 0, "gate/up pairs need 32-column wave tiles");
  static_assert(S >= 2, "the ring needs at least two stages");

  __shared__ __attribute__((aligned(16))) uint16_t ring[S][kStageElems];
  __shared__ int row_src[BM];
  __shared__ int row_dst[BM];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  // Uniform by construction; readfirstlane lets the compiler keep the
  // per-wavefront load choice (A or B buffer, LDS block) in SGPRs.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  load_gemm_args(p);
  const int T = static_cast<int>(p.tokens);

  Tile t;
  if (!find_tile<BM>(p, T, t)) return;
  const bool shared = t.seg == p.experts;
  const int N = PHASE == 1 ? 2 * (shared ? p.shared_dim : p.hidden_dim) : p.dim;
  const int K = PHASE == 1 ? p.dim : (shared ? p.shared_dim : p.hidden_dim);
  const int n0 = static_cast<int>(blockIdx.x) * BN;
  if (n0 >= N) return;
  const int KT = K / 64;

  // ---- per-row source / destination ---------------------------------------
  // Phase 1 gathers x rows by token (through the slot map) and writes hidden
  // row hbase + s.  Phase 2 reads hidden row hbase + s, known without a load,
  // so its A loads start at once; the assignment ids it scatters to are
  // needed only by the epilogue.
  const int sc = segment_row(t, BM, tid);
  const int asg = tid < BM && !shared ? assignment_of(p, t, sc) : 0;
  if (PHASE == 1) {
    if (tid < BM) {
      row_src[tid] = shared ? sc : asg >> 1;
      row_dst[tid] = t.mt * BM + tid < t.rows ? t.hbase + sc : -1;
    }
    __syncthreads();
  }
  asm volatile("" ::: "memory");  // issue the id loads before the A loads

  // ---- this lane's loads: one 16-byte piece of each of its P blocks -------
  const int a_ld = PHASE == 1 ? p.dim : p.hstride;
  const int64_t a_rows = PHASE == 1 ? p.tokens : 3 * p.tokens;
  const __amdgpu_buffer_rsrc_t a_rsrc =
      make_rsrc(p.a_src, static_cast<uint32_t>(a_rows * a_ld * 2));
  const uint16_t* wbase = shared ? p.w_shared
                                 : p.w_routed + static_cast<int64_t>(t.seg) * N * K;
  const __amdgpu_buffer_rsrc_t b_rsrc =
      make_rsrc(wbase, static_cast<uint32_t>(static_cast<int64_t>(N) * K * 2));
  const int ksteps32 = K / 32;
  uint32_t voff[P];
  bool is_a[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int b = wave * P + i;
    is_a[i] = b < kABlocks;
    if (b < kABlocks) {
      // A block (m-tile b / 2, k half b % 2): row 16 (b / 2) + l % 16,
      // k 32 (b % 2) + 8 (l / 16); the stage adds 128 bytes of k.
      const int ar = (b >> 1) * 16 + (lane & 15);
      const int r = PHASE == 1 ? row_src[ar] : t.hbase + segment_row(t, BM, ar);
      voff[i] = static_cast<uint32_t>(r * a_ld + (b & 1) * 32 + (lane >> 4) * 8) * 2;
    } else {
      // B block (group g, k half h) = packed block (n0 / 16 + g, 2 kt + h);
      // the stage adds two blocks (2 KB).  Groups past N read zero.
      const int g = (b - kABlocks) >> 1, h = (b - kABlocks) & 1;
      voff[i] = static_cast<uint32_t>(((n0 / 16 + g) * ksteps32 + h) * 1024 + lane * 16);
    }
  }
  auto issue = [&](uint16_t* stage, int kt) {
    const int ks = min(kt, KT - 1);
#pragma unroll
    for (int i = 0; i < P; ++i) {
      uint16_t* dst = stage + (wave * P + i) * 512;
      if (is_a[i]) buffer_to_lds16(a_rsrc, dst, voff[i], static_cast<uint32_t>(ks) * 128);
      else buffer_to_lds16(b_rsrc, dst, voff[i], static_cast<uint32_t>(ks) * 2048);
    }
  };

  const int wm = wave / kWavesN, wn = wave % kWavesN;
  f32x4 acc[kTilesM][kTilesN];
#pragma unroll
  for (int i = 0; i < kTilesM; ++i)
#pragma unroll
    for (int j = 0; j < kTilesN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Fragment reads go through lds_read_frag (see there); the k half h = 1
  // reads are in flight while the h = 0 MFMAs run.
  auto compute = [&](const uint16_t* stage) {
    bf16x8 a0[kTilesM], b0[kTilesN], a1[kTilesM], b1[kTilesN];
#pragma unroll
    for (int i = 0; i < kTilesM; ++i)
      a0[i] = lds_read_frag(stage + ((wm * kTilesM + i) * 2) * 512 + lane * 8);
#pragma unroll
    for (int j = 0; j < kTilesN; ++j)
      b0[j] = lds_read_frag(stage + (kABlocks + (wn * kTilesN + j) * 2) * 512 + lane * 8);
    lds_wait(a0, b0);
#pragma unroll
    for (int i = 0; i < kTilesM; ++i)
      a1[i] = lds_read_frag(stage + ((wm * kTilesM + i) * 2 + 1) * 512 + lane * 8);
#pragma unroll
    for (int j = 0; j < kTilesN; ++j)
      b1[j] = lds_read_frag(stage + (kABlocks + (wn * kTilesN + j) * 2 + 1) * 512 + lane * 8);
#pragma unroll
    for (int i = 0; i < kTilesM; ++i)
#pragma unroll
      for (int j = 0; j < kTilesN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0[i], b0[j], acc[i][j], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    lds_wait(a1, b1);
#pragma unroll
    for (int i = 0; i < kTilesM; ++i)
#pragma unroll
      for (int j = 0; j < kTilesN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[i], b1[j], acc[i][j], 0, 0, 0);
  };

  // k step kt computes slot kt % S and refills slot (kt - 1) % S with stage
  // kt + S - 1.  Stages past the last are reloads of the last one into
  // slots that are never read again, so every step issues the same P loads
  // and waits for the same count: stage kt has landed for every wavefront,
  // and every wavefront is done reading stage kt - 1, whose slot gets
  // refilled.
#pragma unroll
  for (int st = 0; st < S - 1; ++st) issue(ring[st], st);
  if (PHASE == 2) {
    // The k loop's first barrier publishes these; wait for the LDS writes
    // first, as that barrier is written out without one.
    if (tid < BM) row_dst[tid] = t.mt * BM + tid < t.rows ? (shared ? sc : asg) : -1;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
  for (int kt = 0; kt < KT; ++kt) {
    wait_vm_barrier<P * (S - 2)>();
    issue(ring[(kt + S - 1) % S], kt + S - 1);
    compute(ring[kt % S]);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- epilogue --------------------------------------------------------------
  // C fragment: lane holds column (lane & 15) of rows 4 * (lane >> 4) + r.
  const int wm0 = wm * kWaveM, wn0 = wn * kWaveN;
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
#pragma unroll
      for (int i = 0; i < kTilesM; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = wm0 + i * 16 + 4 * (lane >> 4) + r;
          const int dst = row_dst[row];
          const int64_t at = static_cast<int64_t>(max(dst, 0)) * p.dim + n;
          const float v = shared ? acc[i][j][r] : p.weights[max(dst, 0)] * acc[i][j][r];
          if (dst >= 0 && n < N) (shared ? p.y_shared : p.y_routed)[at] = f32_to_bf16(v);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Wide-MFMA tiles for large segments (hundreds to thousands of rows per
// expert): the same LDS ring as grouped_gemm_kernel (direct-to-LDS stages of
// 1 KB fragment-order blocks, BK = 64, one barrier per k step), with a
// 128 x 128 workgroup tile computed on v_mfma_f32_32x32x16_bf16.  Measured
// on MI355X, that MFMA keeps 92 % of the bf16 peak issuing from one
// wavefront per SIMD where 16x16x32 keeps 70 %, and a 64 x 64 wavefront
// tile reads 4 fragments from LDS per 4 MFMAs of 32 K flops each.
// WAVES_M x WAVES_N wavefronts share the tile: 2 x 2 for 128 x 128 tiles
// (64 x 64 per wavefront), 2 x 4 for 256 x 256 ones (128 x 64 per wavefront:
// 6 fragment reads per 8 MFMAs, and half the stage bytes per flop, at one
// workgroup per CU).  The 256 x 256 tile's route weights go through LDS:
// its 128 accumulators per lane leave no registers for them.
//
// 32x32x16 operands: lane l holds row (or column) l % 32, k 8 (l / 32) .. +7
// of a 16-wide k step.  In the 16 x 32 fragment-order blocks that is block
// (16-row group (l % 32) / 16, 32-k half u / 2), slot 2 (u % 2) + l / 32,
// row l % 16: 16 lanes read 256 contiguous bytes, so the reads do not
// conflict.  The C fragment gives lane l column l % 32 and rows
// 8 (e / 4) + 4 (l / 32) + e % 4 of element e.
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int BM, int BN, int BK, int S, int PHASE, int WAVES_M = 2, int WAVES_N = 2>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N)
void grouped_gemm_wide_kernel(GemmArgs p) {
  constexpr int kWaves = WAVES_M * WAVES_N;
  constexpr int kThreads = 64 * kWaves;
  constexpr int kWaveM = BM / WAVES_M, kWaveN = BN / WAVES_N;  // wavefront tile
  constexpr int kTilesM = kWaveM / 32, kTilesN = kWaveN / 32;
  constexpr int KH = BK / 32;                           // 32-wide k halves per stage
  constexpr int kSteps = BK / 16;                       // MFMA k steps per stage
  constexpr int kABlocks = BM / 16 * KH;                // 16-row groups x k halves
  constexpr int kBlocks = (BM + BN) / 16 * KH;
  constexpr int P = kBlocks / kWaves;                   // loads per wavefront per stage
  constexpr int kStageElems = kBlocks * 512;
  static_assert(kBlocks % kWaves == 0 && kTilesM >= 1 && kTilesN >= 1, "tile shape");
  static_assert(BM <= kThreads, "one thread per tile row sets up the row ids");
  static_assert(BK == 32 || BK == 64, "stages of one or two 32-wide k blocks");
  static_assert(S >= 2, "the ring needs at least two stages");

  __shared__ __attribute__((aligned(16))) uint16_t ring[S][kStageElems];
  __shared__ int row_src[BM];
  __shared__ int row_dst[BM];
  // Route weights of the tile's rows, for wavefront tiles whose registers
  // cannot also hold them (kRouteInLds).
  constexpr bool kRouteInLds = kTilesM * kTilesN * 16 > 64;
  __shared__ float row_w[kRouteInLds ? BM : 1];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  load_gemm_args(p);
  const int T = static_cast<int>(p.tokens);

  // XCD-aware tile order.  Workgroups are dispatched round-robin over the 8
  // XCDs by linear id, so the grid's own order would give XCD x column tile x
  // of every row tile: every XCD's L2 would stream all of A.  Instead the
  // workgroups of XCD x take row tiles x, x + 8, ... with all their column
  // tiles in turn: the ~32 workgroups an XCD runs at once share 4 row tiles'
  // A rows and the expert's weights in its L2.  The grid's row count is a
  // multiple of 8 (launch_wide), so every (row, column) tile is taken once.
  const int nx = static_cast<int>(gridDim.x);
  const int id = static_cast<int>(blockIdx.y) * nx + static_cast<int>(blockIdx.x);
  const int pos = id >> 3;
  const int m_tile = (pos / nx) * 8 + (id & 7);
  const int n_tile = pos - (pos / nx) * nx;

  Tile t;
  if (!find_tile<BM>(p, T, t, m_tile)) return;
  t = uniform_tile(t);
  const bool shared = t.seg == p.experts;
  const int N = PHASE == 1 ? 2 * (shared ? p.shared_dim : p.hidden_dim) : p.dim;
  const int K = PHASE == 1 ? p.dim : (shared ? p.shared_dim : p.hidden_dim);
  const int n0 = n_tile * BN;
  if (n0 >= N) return;
  const int KT = K / BK;

  // ---- per-row source / destination (as in grouped_gemm_kernel) -----------
  const int sc = segment_row(t, BM, tid < BM ? tid : 0);
  const int asg = tid < BM && !shared ? assignment_of(p, t, sc) : 0;
  if (tid < BM) {
    row_src[tid] = PHASE == 1 ? (shared ? sc : asg >> 1) : t.hbase + sc;
    const bool live = t.mt * BM + tid < t.rows;
    row_dst[tid] = !live ? -1 : PHASE == 1 ? t.hbase + sc : (shared ? sc : asg);
    if (kRouteInLds && PHASE == 2) row_w[tid] = live && !shared ? p.weights[asg] : 0.0f;
  }
  __syncthreads();

  // ---- this lane's loads: one 16-byte piece of each of its P blocks -------
  const int a_ld = PHASE == 1 ? p.dim : p.hstride;
  const int64_t a_rows = PHASE == 1 ? p.tokens : 3 * p.tokens;
  const __amdgpu_buffer_rsrc_t a_rsrc =
      make_rsrc(p.a_src, static_cast<uint32_t>(a_rows * a_ld * 2));
  const uint16_t* wbase = shared ? p.w_shared
                                 : p.w_routed + static_cast<int64_t>(t.seg) * N * K;
  const __amdgpu_buffer_rsrc_t b_rsrc =
      make_rsrc(wbase, static_cast<uint32_t>(static_cast<int64_t>(N) * K * 2));
  const int ksteps32 = K / 32;
  uint32_t voff[P];
  bool is_a[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int b = wave * P + i;
    is_a[i] = b < kABlocks;
    if (b < kABlocks) {
      // A block (16-row group b / KH, k half b % KH): row 16 (b / KH) + l % 16,
      // k 32 (b % KH) + 8 (l / 16); the stage adds 2 BK bytes of k.
      const int r = row_src[(b / KH) * 16 + (lane & 15)];
      voff[i] = static_cast<uint32_t>(r * a_ld + (b % KH) * 32 + (lane >> 4) * 8) * 2;
    } else {
      // B block (16-column group g, k half h) = packed block (n0 / 16 + g,
      // KH kt + h); the stage adds KH blocks.  Groups past N read zero.
      const int g = (b - kABlocks) / KH, h = (b - kABlocks) % KH;
      voff[i] = static_cast<uint32_t>(((n0 / 16 + g) * ksteps32 + h) * 1024 + lane * 16);
    }
  }
  auto issue = [&](uint16_t* stage, int kt) {
    const int ks = min(kt, KT - 1);
#pragma unroll
    for (int i = 0; i < P; ++i) {
      uint16_t* dst = stage + (wave * P + i) * 512;
      if (is_a[i]) buffer_to_lds16(a_rsrc, dst, voff[i], static_cast<uint32_t>(ks) * (2 * BK));
      else buffer_to_lds16(b_rsrc, dst, voff[i], static_cast<uint32_t>(ks) * (KH * 1024));
    }
  };

  // ---- fragment addresses (elements) within a stage, for k step u = 0 -----
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int lane_part = (lane >> 5) * 128 + (lane & 15) * 8;
  int a_frag[kTilesM], b_frag[kTilesN];
#pragma unroll
  for (int i = 0; i < kTilesM; ++i) {
    const int rb = wm * (kWaveM / 16) + 2 * i + ((lane & 31) >> 4);
    a_frag[i] = KH * rb * 512 + lane_part;
  }
#pragma unroll
  for (int j = 0; j < kTilesN; ++j) {
    const int g = wn * (kWaveN / 16) + 2 * j + ((lane & 31) >> 4);
    b_frag[j] = (kABlocks + KH * g) * 512 + lane_part;
  }

  f32x16 acc[kTilesM][kTilesN];
#pragma unroll
  for (int i = 0; i < kTilesM; ++i)
#pragma unroll
    for (int j = 0; j < kTilesN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Route weights of this lane's output rows (phase 2, routed): issued here,
  // they land while the k loop runs instead of stalling the epilogue.
  float route_w[kRouteInLds ? 1 : kTilesM][16];
  if (!kRouteInLds && PHASE == 2 && !shared) {
#pragma unroll
    for (int i = 0; i < kTilesM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = wm * kWaveM + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        route_w[i][e] = p.weights[max(row_dst[row], 0)];
      }
  }

  // kSteps 16-wide k steps per stage.  Fragment reads run two steps ahead of
  // the MFMAs: a wavefront's LDS reads complete in order, so waiting until at
  // most one step's reads are outstanding means step u's fragments have
  // landed while step u + 1's are still in flight.
  constexpr int kReads = kTilesM + kTilesN;  // LDS reads per k step
  auto read_step = [&](const uint16_t* stage, int u, bf16x8 (&a)[kTilesM],
                       bf16x8 (&b)[kTilesN]) {
    const int du = (u >> 1) * 512 + (u & 1) * 256;
#pragma unroll
    for (int i = 0; i < kTilesM; ++i) a[i] = lds_read_frag(stage + a_frag[i] + du);
#pragma unroll
    for (int j = 0; j < kTilesN; ++j) b[j] = lds_read_frag(stage + b_frag[j] + du);
  };
  auto compute = [&](const uint16_t* stage) {
    bf16x8 a[3][kTilesM], b[3][kTilesN];
    read_step(stage, 0, a[0], b[0]);
    read_step(stage, 1, a[1], b[1]);
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      const int c = u % 3;
      if (u + 1 < kSteps) lds_wait_upto<kReads>(a[c], b[c]);
      else lds_wait_upto<0>(a[c], b[c]);
      if (u + 2 < kSteps) read_step(stage, u + 2, a[(u + 2) % 3], b[(u + 2) % 3]);
#pragma unroll
      for (int i = 0; i < kTilesM; ++i)
#pragma unroll
        for (int j = 0; j < kTilesN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[c][i], b[c][j], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

#pragma unroll
  for (int st = 0; st < S - 1; ++st) issue(ring[st], st);
  for (int kt = 0; kt < KT; ++kt) {
    wait_vm_barrier<P * (S - 2)>();
    issue(ring[(kt + S - 1) % S], kt + S - 1);
    compute(ring[kt % S]);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- epilogue ----------------------------------------------------------------
  const int wm0 = wm * kWaveM;
  if (PHASE == 1) {
    // Columns 32 c .. 32 c + 15 of the packed gate/up matrix are gate rows
    // 16 c .. 16 c + 15 and the next 16 the matching up rows: lane l < 16 of
    // each 32-lane half takes the up value of lane l + 16 (ds_swizzle,
    // xor 16 within 32 lanes).  The tile's BM x BN / 2 hidden values are
    // staged in LDS (the ring is free once every wavefront has passed the
    // barrier) and stored as 16-byte row pieces.
    constexpr int kHalf = BN / 2;
    constexpr int kOutLd = kHalf + 8;  // staged row stride, elements (shifts banks by 4 rows)
    static_assert(BM * kOutLd <= S * kStageElems, "staged hidden tile must fit the ring");
    uint16_t* out_s = &ring[0][0];
    __syncthreads();
    const bool gate_lane = (lane & 31) < 16;
#pragma unroll
    for (int j = 0; j < kTilesN; ++j) {
      const int hl = (wn * kWaveN + 32 * j) / 2 + (lane & 15);  // hidden column within the tile
#pragma unroll
      for (int i = 0; i < kTilesM; ++i) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float up = __int_as_float(
              __builtin_amdgcn_ds_swizzle(__float_as_int(acc[i][j][e]), 0x401F));
          const int row = wm0 + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
          if (gate_lane) out_s[row * kOutLd + hl] = f32_to_bf16(swiglu(acc[i][j][e], up));
        }
      }
    }
    __syncthreads();
    const int h0 = n0 / 2;
    constexpr int kPieces = kHalf / 8;  // 16-byte pieces per staged row
    for (int c = tid; c < BM * kPieces; c += kThreads) {
      const int row = c / kPieces, piece = c - row * kPieces;
      const int dst = row_dst[row];
      const int h = h0 + piece * 8;
      if (dst >= 0 && 2 * h < N)
        *reinterpret_cast<uint4*>(p.hidden_out + static_cast<int64_t>(dst) * p.hstride + h) =
            *reinterpret_cast<const uint4*>(out_s + row * kOutLd + piece * 8);
    }
  } else {
#pragma unroll
    for (int j = 0; j < kTilesN; ++j) {
      const int n = n0 + wn * kWaveN + 32 * j + (lane & 31);
#pragma unroll
      for (int i = 0; i < kTilesM; ++i) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = wm0 + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
          const int dst = row_dst[row];
          const int64_t at = static_cast<int64_t>(max(dst, 0)) * p.dim + n;
          const float w = shared ? 1.0f
                                 : (kRouteInLds ? row_w[row] : route_w[kRouteInLds ? 0 : i][e]);
          const float v = shared ? acc[i][j][e] : w * acc[i][j][e];
          if (dst >= 0 && n < N) (shared ? p.y_shared : p.y_routed)[at] = f32_to_bf16(v);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Streaming variant for small row tiles (BM <= 32, K <= kStreamKCap): the
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

// No amdgpu_waves_per_eu cap: with it ("1, 2") the hardware ran at most two
// of these workgroups per CU, so at the bs1 x 512 shapes the down launch
// started its last quarter of workgroups only when the first ones ended
// (measured on MI355X: last workgroup start 4.2 us after the first, launch
// 8.6 -> 7.2 us without the cap; LDS alone allows three per CU).
//
// KCH > 1 splits the A tile along k into KCH chunks that take turns in the
// same LDS buffer (K % (64 KCH) == 0): 64-row tiles then fit the 32-row
// tile's LDS budget, and every weight fragment loaded feeds twice the rows.
// At the chunk boundary the workgroup waits for the next chunk's rows while
// the weight ring keeps streaming.
template <int BM, int WN, int PF, int PHASE, int KCH = 1>
__global__ __launch_bounds__(256)
void grouped_gemm_stream_kernel(GemmArgs p) {
  constexpr int kTilesM = BM / 16;
  constexpr int kTilesN = WN / 16;
  constexpr int BN = 4 * WN;
  static_assert(PHASE != 1 || WN == 32, "gate/up pairs need 32 columns per wavefront");

  __shared__ __attribute__((aligned(16))) uint16_t a_lds[BM * kStreamKCap / KCH];
  __shared__ int row_src[BM];
  __shared__ int row_dst[BM];
  __shared__ int hist_s[4][kMaxExperts];
  __shared__ int chunk_s[kGroupMaxAssign / kWave];

  load_gemm_args(p);
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int T = static_cast<int>(p.tokens);

  // Phase 1 groups in-kernel when given the top-2 ids or the route's block
  // table (uniform per launch).
  const bool from_blocks = PHASE == 1 && p.route_blocks != nullptr;
  const bool self_grouped = PHASE == 1 && (p.indices != nullptr || from_blocks);
  const TileIndex ti = xcd_tile(p.rows_per_xcd != 0);
  Tile t;
  GroupIds gids;
  if (self_grouped) {
    const bool found = from_blocks
                           ? group_find_blocks<BM>(p, T, t, gids, row_src, row_dst, hist_s, ti)
                           : group_find<BM>(p, T, t, gids, row_src, row_dst, hist_s, ti);
    if (!found) return;
  } else if (!find_tile<BM>(p, T, t, ti.m)) {
    return;
  }
  t = uniform_tile(t);
  const bool shared = t.seg == p.experts;
  const int N = PHASE == 1 ? 2 * (shared ? p.shared_dim : p.hidden_dim) : p.dim;
  const int K = PHASE == 1 ? p.dim : (shared ? p.shared_dim : p.hidden_dim);
  const int n0 = ti.n * BN;
  if (n0 >= N) return;

  const int chunks = K / 8 / KCH;                 // 16-byte chunks per A row (per k chunk)
  const int swz = (chunks & 15) == 0 ? 15 : 7;   // XOR group size - 1
  const int ksteps = K / 32;
  const int ksteps_c = ksteps / KCH;             // k steps per A chunk

  // ---- row ids: issued first, so waiting for them waits for no weight load
  // Phase 1 gathers x rows by token (through the slot map) and writes hidden
  // row hbase + s.  Phase 2 reads hidden row hbase + s, known without a load,
  // so its A gather starts at once; the assignment ids it scatters to are
  // needed only by the epilogue and arrive meanwhile.  With self_grouped,
  // group_rows places the routed rows instead.
  const int sc = segment_row(t, BM, tid);
  const int asg = tid < BM && !shared && !self_grouped ? assignment_of(p, t, sc) : 0;
  asm volatile("" ::: "memory");  // issue the id loads before the weight loads

  // ---- B: first PF k steps of this lane's fragments -------------------------
  const uint16_t* wbase = shared ? p.w_shared
                                 : p.w_routed + static_cast<int64_t>(t.seg) * N * K;
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

  // ---- per-row source / destination (the weight loads are in flight) -------
  if (self_grouped && !shared) {
    if (from_blocks) group_rows_blocks<BM>(p, t, gids, row_src, row_dst, chunk_s, ti.n == 0);
    else group_rows<BM>(p, T, t, gids, row_src, row_dst, chunk_s, ti.n == 0);
  }
  if (PHASE == 1) {
    if (tid < BM && (shared || !self_grouped)) {
      row_src[tid] = shared ? sc : asg >> 1;
      row_dst[tid] = t.mt * BM + tid < t.rows ? t.hbase + sc : -1;
    }
    __syncthreads();
  }

  // ---- A: the whole tile (or its first k chunk), direct to LDS -------------
  auto gather_a = [&](int kc) {
    const int a_ld = PHASE == 1 ? p.dim : p.hstride;
    const int slots = BM * chunks;  // multiple of 64 (BM >= 16, chunks >= 8)
    for (int i = wave; i < slots / kWave; i += 4) {
      const int slot = i * kWave + lane;
      const int r = slot / chunks;
      const int pc = slot - r * chunks;
      const int c = (pc & ~swz) | ((pc ^ r) & swz);
      const int src = PHASE == 1 ? row_src[r] : t.hbase + segment_row(t, BM, r);
      const uint16_t* g = p.a_src + static_cast<int64_t>(src) * a_ld + kc * (K / KCH) + c * 8;
      __builtin_amdgcn_global_load_lds(g, (lds_void_t*)(a_lds + i * kWave * 8), 16, 0, 0);
    }
  };
  gather_a(0);
  if (PHASE == 2 && tid < BM) row_dst[tid] = t.mt * BM + tid < t.rows ? (shared ? sc : asg) : -1;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // This lane's output rows (C fragment rows 4 (lane / 16) + r of each
  // 16-row tile), read once so the epilogue waits for no LDS read.
  int dst_row[kTilesM][4];
#pragma unroll
  for (int mi = 0; mi < kTilesM; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r) dst_row[mi][r] = row_dst[mi * 16 + 4 * (lane >> 4) + r];
  // Phase 2, routed rows: their route weights, loaded inside the first k
  // step, right after its weight refill (before the final pass when that is
  // the only one).  Loads retire in order, so issued before the loop they
  // would hold up its first MFMAs; issued there, the first wait that covers
  // them comes PF steps later.
  float route_w[kTilesM][4];
#pragma unroll
  for (int mi = 0; mi < kTilesM; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r) route_w[mi][r] = 0.f;
  auto load_route_weights = [&]() {
    if (PHASE == 2 && !shared) {
#pragma unroll
      for (int mi = 0; mi < kTilesM; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) route_w[mi][r] = p.weights[max(dst_row[mi][r], 0)];
    }
  };

  f32x4 acc[kTilesM][kTilesN];
#pragma unroll
  for (int i = 0; i < kTilesM; ++i)
#pragma unroll
    for (int j = 0; j < kTilesN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  int chunk_base = 0, chunk_end = ksteps_c;  // k steps of the A chunk in LDS
  // One k step on ring slot i: A fragments from LDS, the MFMAs, then the
  // slot's refill with step + PF unless the ring already holds the last
  // steps.  The final pass is peeled off so it issues no loads: refills of
  // steps past the end (reloads of the last one, to keep the loop uniform)
  // cost a full memory round trip before the kernel could finish.
  auto k_step = [&](int step, int i, bool refill) {
    if (KCH > 1 && step == chunk_end) {
      // Every wavefront is done with the A chunk in LDS: the next replaces it.
      chunk_base = chunk_end;
      chunk_end += ksteps_c;
      __syncthreads();
      gather_a(chunk_base / ksteps_c);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    }
    const int sl = step - chunk_base;  // k step within the A chunk in LDS
    bf16x8 af[kTilesM];
#pragma unroll
    for (int mi = 0; mi < kTilesM; ++mi) {
      const int r = mi * 16 + (lane & 15);
      const int c = sl * 4 + (lane >> 4);
      const int pc = (c & ~swz) | ((c ^ r) & swz);
      af[mi] = *reinterpret_cast<const bf16x8*>(&a_lds[(r * chunks + pc) * 8]);
    }
#pragma unroll
    for (int mi = 0; mi < kTilesM; ++mi)
#pragma unroll
      for (int j = 0; j < kTilesN; ++j)
        acc[mi][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            af[mi], __builtin_bit_cast(bf16x8, bq[i][j]), acc[mi][j], 0, 0, 0);
    if (refill) {
      const uint32_t next = static_cast<uint32_t>(step + PF) * 1024;
#pragma unroll
      for (int j = 0; j < kTilesN; ++j) bq[i][j] = buffer_load16(b_rsrc, b_off[j], next);
    }
    if (refill && step == 0) load_route_weights();
    // Keep the refill in its own step: left free, the scheduler sinks every
    // refill to the end of the loop body, and the next pass's first MFMAs
    // then wait on loads issued a few instructions earlier.  LDS reads and
    // SALU work may still cross (mask 0x104), so the next step's A
    // fragments are read while this step's MFMAs run.
    __builtin_amdgcn_sched_barrier(0x104);
  };
  const int last = ksteps - PF;  // first step of the final pass
  if (last == 0) load_route_weights();  // one pass only: no refilling step
  for (int s0 = 0; s0 < last; s0 += PF) {
#pragma unroll
    for (int i = 0; i < PF; ++i) k_step(s0 + i, i, true);
  }
#pragma unroll
  for (int i = 0; i < PF; ++i) k_step(last + i, i, false);

  // ---- epilogue (as in grouped_gemm_kernel) ----------------------------------
  if (PHASE == 1) {
    const int ng = n0 + wave * WN;  // first gate column of this wavefront's pair
    if (ng < N) {
      const int h = (ng >> 1) + (lane & 15);
#pragma unroll
      for (int mi = 0; mi < kTilesM; ++mi) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int dst = dst_row[mi][r];
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
#pragma unroll
      for (int mi = 0; mi < kTilesM; ++mi) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int dst = dst_row[mi][r];
          const int64_t at = static_cast<int64_t>(max(dst, 0)) * p.dim + n;
          const float v = shared ? acc[mi][j][r] : route_w[mi][r] * acc[mi][j][r];
          if (dst >= 0 && n < N) (shared ? p.y_shared : p.y_routed)[at] = f32_to_bf16(v);
        }
      }
    }
  }
}

template <int BM, int BN, int S>
hipError_t launch_phase(int phase, const GemmArgs& args, int n_max, hipStream_t s) {
  const int T = static_cast<int>(args.tokens);
  const int m_tiles = (T + BM - 1) / BM + (2 * T) / BM + args.experts;
  const dim3 grid((n_max + BN - 1) / BN, m_tiles);
  if (phase == 1) grouped_gemm_kernel<BM, BN, S, 1><<<grid, 256, 0, s>>>(args);
  else grouped_gemm_kernel<BM, BN, S, 2><<<grid, 256, 0, s>>>(args);
  return hipGetLastError();
}

template <int BM, int BN, int BK, int S, int WAVES_M = 2, int WAVES_N = 2>
hipError_t launch_wide(int phase, const GemmArgs& args, int n_max, hipStream_t s) {
  const int T = static_cast<int>(args.tokens);
  const int m_tiles = (T + BM - 1) / BM + (2 * T) / BM + args.experts;
  // Rows of tiles rounded up to a multiple of the 8 XCDs (the kernel's tile
  // order takes every eighth row tile per XCD).
  const dim3 grid((n_max + BN - 1) / BN, (m_tiles + 7) / 8 * 8);
  constexpr int kThreads = 64 * WAVES_M * WAVES_N;
  if (phase == 1)
    grouped_gemm_wide_kernel<BM, BN, BK, S, 1, WAVES_M, WAVES_N><<<grid, kThreads, 0, s>>>(args);
  else
    grouped_gemm_wide_kernel<BM, BN, BK, S, 2, WAVES_M, WAVES_N><<<grid, kThreads, 0, s>>>(args);
  return hipGetLastError();
}

template <int BM, int WN, int PF, int KCH>
hipError_t launch_stream(int phase, const GemmArgs& args, int n_max, hipStream_t s) {
  const int T = static_cast<int>(args.tokens);
  const int m_tiles = (T + BM - 1) / BM + (2 * T) / BM + args.experts;
  const dim3 grid((n_max + 4 * WN - 1) / (4 * WN),
                  args.rows_per_xcd ? (m_tiles + 7) / 8 * 8 : m_tiles);
  if (phase == 1) grouped_gemm_stream_kernel<BM, 32, PF, 1, KCH><<<grid, 256, 0, s>>>(args);
  else grouped_gemm_stream_kernel<BM, WN, PF, 2, KCH><<<grid, 256, 0, s>>>(args);
  return hipGetLastError();
}

// Register-ring depth: the largest of 8 / 4 / 2 / 1 dividing every segment's
// number of 32-wide k steps in this phase, at most 4 for gate/up (its two
// fragments per step double the registers per stage; measured on MI355X in
// the bs1 x 512 forward, 4 stages beat 8 for gate/up and 8 beat 4 for down).
int stream_depth(int phase, const GemmArgs& a) {
  const int k0 = phase == 1 ? a.dim : a.hidden_dim;
  const int k1 = phase == 1 ? a.dim : a.shared_dim;
  for (int pf = phase == 1 ? 4 : 8; pf > 1; pf >>= 1)
    if ((k0 / 32) % pf == 0 && (k1 / 32) % pf == 0) return pf;
  return 1;
}

template <int BM, int KCH>
hipError_t run_stream(int phase, GemmArgs args, int n_max, hipStream_t s) {
  // Down projection: 16 columns per wavefront doubles the workgroups when
  // the row tiles are few.
  switch (stream_depth(phase, args)) {
    case 8: return phase == 1 ? launch_stream<BM, 32, 8, KCH>(1, args, n_max, s)
                              : launch_stream<BM, 16, 8, KCH>(2, args, n_max, s);
    case 4: return phase == 1 ? launch_stream<BM, 32, 4, KCH>(1, args, n_max, s)
                              : launch_stream<BM, 16, 4, KCH>(2, args, n_max, s);
    case 2: return phase == 1 ? launch_stream<BM, 32, 2, KCH>(1, args, n_max, s)
                              : launch_stream<BM, 16, 2, KCH>(2, args, n_max, s);
    default: return phase == 1 ? launch_stream<BM, 32, 1, KCH>(1, args, n_max, s)
                               : launch_stream<BM, 16, 1, KCH>(2, args, n_max, s);
  }
}

// Tile plans.  kStreamBM: the streaming kernel with BM-row tiles when every
// K fits its LDS budget (64-row tiles in two k chunks, when every K splits
// into 128-element halves; else 32-row tiles), else the pipelined kernel
// with 32-row tiles.
enum class TilePlan { kStream16, kStream32, kStream64, kWide128, kWide256 };

// Average rows per expert from which the wide-MFMA tiles take over, per
// phase.  Measured on MI355X (E = 16 uniform, T = 4K ... 64K, and BASELINE
// config 3, E = 32 with 2 experts holding ~95 % of the rows): down is 18-31 %
// faster on wide tiles from 256 rows per expert; gate/up only from 512 --
// at config 3 its 30 small experts (~10 rows each) pay for whole 128 x 128
// tiles with 1 KB x 24 weight blocks each (wide 49.8 us vs streaming 41.2).
constexpr int64_t kWideRowsGateUp = 512;
constexpr int64_t kWideRowsDown = 256;
// Down on 256 x 256 tiles (eight wavefronts, one workgroup per CU) from this
// many rows per expert.  Measured on MI355X (E = 16, HIP events): down
// T = 32768 171 -> 163 us, T = 65536 327 -> 305 us; T = 16384 (2048 rows per
// expert) 75 -> 82 us.  Gate/up stays on 128 x 128 tiles: 256 x 256 measured
// 107 -> 156 us at T = 16384 and 385 -> 498 us at T = 65536 (with one
// workgroup per CU nothing overlaps a tile's prologue and its hidden-tile
// epilogue).
constexpr int64_t kWide256RowsDown = 4096;

template <TilePlan PLAN>
hipError_t run_phase(int phase, GemmArgs args, const ExpertWeights& w, uint16_t* hidden,
                     hipStream_t s) {
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
  if constexpr (PLAN == TilePlan::kWide128) return launch_wide<128, 128, 32, 3>(phase, args, n_max, s);
  if constexpr (PLAN == TilePlan::kWide256)
    return launch_wide<256, 256, 32, 4, 2, 4>(phase, args, n_max, s);
  const int k_max = phase == 1 ? args.dim : max(args.hidden_dim, args.shared_dim);
  if (k_max > kStreamKCap) return launch_phase<32, 128, 3>(phase, args, n_max, s);
  if constexpr (PLAN == TilePlan::kStream64) {
    const bool halves = phase == 1 ? args.dim % 128 == 0
                                   : args.hidden_dim % 128 == 0 && args.shared_dim % 128 == 0;
    if (halves) return run_stream<64, 2>(phase, args, n_max, s);
  }
  return run_stream<PLAN == TilePlan::kStream16 ? 16 : 32, 1>(phase, args, n_max, s);
}

// Kernel and row tile per launch, chosen from T and E only (the per-expert
// counts stay on the device).  Measured on MI355X (E = 16 and 32, T = 1024
// ... 16384, and BASELINE config 3): the streaming kernel beats the pipelined
// kernel with 64-row tiles at every size, by 10-35 % with 32-row tiles
// (config 3: gate/up 53.7 -> 46.2 us, down 41.8 -> 36.0 us); 128-row and
// 256-column pipelined tiles were slower still.  Past ~3 x 32 rows per
// expert the weight fragments' trips from L2 set the pace (each 32-row tile
// of an expert re-reads its weights), and 64-row tiles in two k chunks halve
// them.  From kWideRowsGateUp / kWideRowsDown rows per expert the wide-MFMA
// 128 x 128 tiles take over (grouped_gemm_wide_kernel).
TilePlan experts_tile_plan(int phase, int64_t tokens, int experts) {
  const int64_t per_expert = (2 * tokens + experts - 1) / experts;
  if (tokens <= 16) return TilePlan::kStream16;
  if (per_expert <= 96) return TilePlan::kStream32;
  const int64_t wide_from = phase == 1 ? kWideRowsGateUp : kWideRowsDown;
  if (per_expert < wide_from) return TilePlan::kStream64;
  return phase == 2 && per_expert >= kWide256RowsDown ? TilePlan::kWide256 : TilePlan::kWide128;
}

// Streaming-kernel tile order for gate/up: row-major per XCD once the
// gathered A rows (x) pass kXcdRowsABytes -- the grid's own order has every
// XCD read all of A, one column tile of weights at a time.  Measured on
// MI355X: config 3 (A 6.3 MB) gate/up 41.2 -> 32.6 us and E = 16 T = 2048
// (3.1 MB) 24.8 -> 23.0 us row-major; config 2 (0.4 MB) 11.9 -> 13.1 us and
// T = 512 (0.8 MB) 10.2 -> 14.0 us, where every XCD's L2 holds all of A and
// one column tile of every expert, the grid order wins.  Down (A = the
// hidden rows) measured no better row-major and keeps the grid order.
constexpr int64_t kXcdRowsABytes = int64_t{2} << 20;

int stream_rows_per_xcd(int phase, int64_t tokens, int dim, int, int, int) {
  return phase == 1 && tokens * dim * 2 > kXcdRowsABytes ? 1 : 0;
}

}  // namespace

GroupInKernel experts_group_in_kernel(int64_t tokens, int dim, int experts, int hidden_dim,
                                      int shared_dim) {
  if (tokens < 1 || experts > kMaxExperts) return kGroupNone;
  if (dim > kStreamKCap || max(hidden_dim, shared_dim) > kStreamKCap) return kGroupNone;
  // The streaming kernel groups; the wide tiles' plan does not.
  if (experts_tile_plan(1, tokens, experts) == TilePlan::kWide128) return kGroupNone;
  // From the ids: up to ~3 x 32 rows per expert on average (the shapes it
  // was measured at).
  if (2 * tokens <= kGroupMaxAssign && (2 * tokens + experts - 1) / experts <= 96)
    return kGroupFromIds;
  if (route_blocks(tokens) <= kGroupMaxRouteBlocks && route_block_rows_supported(tokens))
    return kGroupFromBlocks;
  return kGroupNone;
}

hipError_t launch_expert_gemm(int phase, const uint16_t* x, int64_t tokens, int dim,
                              int experts, int hidden_dim, int shared_dim, int capacity,
                              const GroupMap& map, const ExpertWeights& w, uint16_t* hidden,
                              uint16_t* y_routed, uint16_t* y_shared, hipStream_t s) {
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
  args.sorted = phase == 2 ? map.sorted : nullptr;
  args.rows_per_xcd = stream_rows_per_xcd(phase, tokens, dim, experts, hidden_dim, shared_dim);
  if (phase == 1 && (map.indices != nullptr || map.route_blocks != nullptr)) {
    const GroupInKernel mode = experts_group_in_kernel(tokens, dim, experts, hidden_dim,
                                                       shared_dim);
    if (mode == kGroupNone || (map.route_blocks == nullptr && mode != kGroupFromIds))
      return hipErrorInvalidValue;
    args.indices = map.route_blocks != nullptr ? nullptr : map.indices;
    args.route_blocks = map.route_blocks;
    args.counts_out = map.counts_out;
    args.offsets_out = map.offsets_out;
    args.sorted_out = map.sorted_out;
  }
  switch (experts_tile_plan(phase, tokens, experts)) {
    case TilePlan::kStream16: return run_phase<TilePlan::kStream16>(phase, args, w, hidden, s);
    case TilePlan::kStream32: return run_phase<TilePlan::kStream32>(phase, args, w, hidden, s);
    case TilePlan::kStream64: return run_phase<TilePlan::kStream64>(phase, args, w, hidden, s);
    case TilePlan::kWide128: return run_phase<TilePlan::kWide128>(phase, args, w, hidden, s);
    default: return run_phase<TilePlan::kWide256>(phase, args, w, hidden, s);
  }
}

}  // namespace parrot
