// Dense projections y = x W^T on v_mfma_f32_16x16x32_bf16: the linear maps of
// the attention layers (packed q|k|v, output, MLA latent and up maps).
//
// Reference semantics: bias-free nn.Linear in bf16 (parrot/model.py:167-230
// for the GQA layers, :331-432 for MLA), the output projection with its
// residual add as the reference's decode kernel computes it,
// bf16(addend + bf16(x W^T)) (parrot/kernels/moe_bf16.metal:1364-1389), and
// for the GQA layers RoPE of q and k plus the head split
// (parrot/model.py:176-230), applied here to the bf16-rounded projection
// exactly as the stand-alone RoPE kernel does.
//
// At prefill sizes (hundreds of rows, K <= 2048, a few MB of weights) a
// library GEMM spends most of its time in a k loop of global -> LDS -> MFMA
// round trips.  Here a workgroup owns 16 rows x 64 columns: the whole A tile
// (16 x K) is copied into LDS once with direct-to-LDS loads, XOR-swizzled as
// in the expert GEMMs, and each of the 4 wavefronts streams the B fragments
// of its 16 columns straight into registers with raw buffer loads from
// weights packed in MFMA fragment order (1 KB contiguous per wavefront
// load): for K = 32 KST with KST in {4, 8, 16, 24} every k step is loaded
// up front (the trip count is a template constant, so the compiler places
// exact per-step waits), for other K through a ring of PF registers.  The A
// loads are issued first and waited for alone (vmcnt(PF)), and the A
// fragments are read from LDS with inline asm so the compiler does not add
// a wait for the whole direct-to-LDS traffic; the k loop has no barrier.
// Measured on MI355X in the bs1 x 512 forward: 16-row tiles beat 32-row
// tiles (more workgroups in flight), and the up-front loads beat the ring.
//
// Workgroups are dispatched round-robin over the 8 XCDs; the tile index is
// remapped so each XCD takes a contiguous run of column-major tiles, and the
// row tiles that share a block of weight columns share that XCD's L2.
//
// Epilogues (the C fragment gives lane l column l % 16 and rows
// 4 (l / 16) + r):
//   kStore    out[row, col] = bf16(acc) or bf16(addend + bf16(acc));
//   kStoreT   per-sequence transpose, out[(b N + col) ld_keys + t], the value
//             layout the attention kernel reads (MLA values);
//   kRopeQkv  columns [0, H d) -> q [b, H, seq, d], [H d, (H + Hk) d) ->
//             k [b, Hk, seq, d], both rotated; the rest -> v, [b, Hk, seq, d]
//             or transposed [b, Hk, d, vt_keys]; and/or k and v in the
//             attention kernel's fragment order (kfrag_index, vfrag_index).
//             Rotation partners (2i, 2i + 1) sit in adjacent lanes: one DPP
//             quad_perm swap.
//   kFrag     the output as attention K or V in fragment order, columns
//             grouped into heads of head_dim, or both from one [Wk; Wv]
//             weight (the MLA up-projections).
#include "common.h"

namespace parrot {

namespace {

constexpr int kProjRows = 16;        // rows per workgroup
constexpr int kProjCols = 64;        // columns per workgroup: 4 wavefronts x 16
constexpr int kProjMaxK = 2048;      // A tile at most 64 KB of LDS

enum ProjEpilogue { kStore = 0, kStoreT = 1, kRopeQkv = 2, kFrag = 3 };

struct ProjArgs {
  const uint16_t* x;
  int64_t lda;
  int rows, K, N;
  const uint16_t* w;       // packed [N / 16][K / 32][64 lanes x 16 B]
  // kStore
  uint16_t* out;
  int64_t ldo;
  const uint16_t* addend;  // optional, [rows, ld_addend]
  int64_t ld_addend;
  // kStoreT and kRopeQkv
  int seq, ld_keys;
  // kRopeQkv
  const float* cos_t;
  const float* sin_t;
  int start, max_positions;
  const int32_t* start_device;
  int heads, kv_heads, head_dim;
  uint16_t* q;
  uint16_t* k;              // optional with kRopeQkv
  uint16_t* v;              // optional with kRopeQkv
  // fragment-order attention operands (kRopeQkv: optional; kFrag: one of them)
  uint16_t* kf;
  uint16_t* vf;
  int nblk;                 // ceil(seq / 32)
};

__device__ __forceinline__ float swap_pair(float v) {  // lanes 2i <-> 2i + 1
  return dpp<0xb1>(v);
}

// One 16-byte MFMA fragment from LDS, read with inline asm: the compiler then
// does not tie it to the direct-to-LDS loads (it would wait for every one of
// them, vmcnt(0), weight loads included); the kernel's own vmcnt wait and
// barrier order it after the A tile, and lds_frag_wait before its use.
__device__ __forceinline__ bf16x8 lds_frag(const uint16_t* p) {
  const uint32_t addr = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint16_t*)p));
  bf16x8 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}

// Stores one lane's 4 values (rows row0 .. row0 + 3, one column w of kv
// head kvh of kv_heads) as attention values: row-major p.v [b, kv_heads,
// seq, d] or transposed [b, kv_heads, d, ld_keys] when p.v is set, and in
// fragment order when p.vf is set.  When seq % 4 == 0 the 4 rows are
// consecutive positions of one sequence and the transposed and fragment
// stores take them in one 8-byte store.
__device__ __forceinline__ void store_values(const ProjArgs& p, const uint16_t (&bits)[4],
                                             int row0, int kvh, int kv_heads, int w) {
  const int d = p.head_dim;
  if ((p.seq & 3) == 0) {
    const int b = row0 / p.seq;
    const int t0 = row0 - b * p.seq;
    const int64_t bh = static_cast<int64_t>(b) * kv_heads + kvh;
    uint2 u;
    u.x = static_cast<uint32_t>(bits[0]) | (static_cast<uint32_t>(bits[1]) << 16);
    u.y = static_cast<uint32_t>(bits[2]) | (static_cast<uint32_t>(bits[3]) << 16);
    if (p.v != nullptr) {
      if (p.ld_keys > 0) {
        *reinterpret_cast<uint2*>(p.v + (bh * d + w) * p.ld_keys + t0) = u;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) p.v[(bh * p.seq + t0 + r) * d + w] = bits[r];
      }
    }
    if (p.vf != nullptr)
      *reinterpret_cast<uint2*>(p.vf + vfrag_index(bh, p.nblk, t0, w, d / 16)) = u;
    return;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = row0 + r;
    if (row >= p.rows) break;
    const int b = row / p.seq;
    const int tp = row - b * p.seq;
    const int64_t bh = static_cast<int64_t>(b) * kv_heads + kvh;
    if (p.v != nullptr) {
      if (p.ld_keys > 0) p.v[(bh * d + w) * p.ld_keys + tp] = bits[r];
      else p.v[(bh * p.seq + tp) * d + w] = bits[r];
    }
    if (p.vf != nullptr) p.vf[vfrag_index(bh, p.nblk, tp, w, d / 16)] = bits[r];
  }
}

// KST > 0: K == 32 KST and PF == KST (every k step loaded up front);
// KST == 0: a ring of PF stages over K / 32 steps (a multiple of PF).
template <int PF, int EPI, int KST>
__global__ __launch_bounds__(256) void proj_kernel(ProjArgs p) {
  constexpr int BM = kProjRows;
  constexpr int kTilesM = BM / 16;
  static_assert(KST == 0 || KST == PF, "the up-front mode loads every step at once");
  extern __shared__ __attribute__((aligned(16))) uint16_t a_lds[];  // [BM][K], swizzled

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // XCD-aware tile order: hardware id -> (XCD, slot) -> contiguous index j.
  const int total = static_cast<int>(gridDim.x);
  // The prologue's kernel arguments in one batch of scalar loads (a field
  // first read inside a branch or loop costs a scalar round trip of its own).
  asm volatile("" ::"s"(p.x), "s"(p.lda), "s"(p.rows), "s"(p.K), "s"(p.N), "s"(p.w), "s"(total));
  if constexpr (EPI == kStore) asm volatile("" ::"s"(p.addend), "s"(p.ld_addend));
  if constexpr (EPI == kRopeQkv)
    asm volatile("" ::"s"(p.cos_t), "s"(p.sin_t), "s"(p.start), "s"(p.start_device), "s"(p.seq),
                 "s"(p.max_positions), "s"(p.head_dim), "s"(p.heads), "s"(p.kv_heads));
  const int id = static_cast<int>(blockIdx.x);
  const int xcd = id & 7, slot = id >> 3;
  const int q8 = total >> 3, r8 = total & 7;
  const int j = xcd * q8 + min(xcd, r8) + slot;
  const int row_tiles = (p.rows + BM - 1) / BM;
  const int ct = j / row_tiles;
  const int m0 = (j - ct * row_tiles) * BM;
  const int nw = ct * kProjCols + wave * 16;  // this wavefront's first column

  const int K = p.K;
  const int chunks = K / 8;                      // 16-byte chunks per row (multiple of 8)
  const int swz = (chunks & 15) == 0 ? 15 : 7;   // XOR group size - 1
  const int ksteps = KST > 0 ? KST : K / 32;

  // ---- epilogue operands that depend only on this lane's rows and column,
  // loaded before the tile so their round trip overlaps it: read in the
  // epilogue they added one (the residual addend) or two (a device position,
  // then the RoPE tables).  The loads are unconditional (a value loaded
  // inside a branch is waited for at the branch's end): without an addend
  // they read the weights' first row, waves past N clamp their column, and
  // the table indices are clamped into the tables.
  const int ecol = min(nw, p.N - 16) + (lane & 15);
  uint16_t add_v[kTilesM][4];
  float rope_c[kTilesM][4], rope_s[kTilesM][4];
  if constexpr (EPI == kStore) {
    const bool has_addend = p.addend != nullptr;
    const uint16_t* ab = has_addend ? p.addend : p.w;
    const int64_t ald = has_addend ? p.ld_addend : 0;
#pragma unroll
    for (int mi = 0; mi < kTilesM; ++mi)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = min(m0 + mi * 16 + 4 * (lane >> 4) + r, p.rows - 1);
        add_v[mi][r] = ab[static_cast<int64_t>(row) * ald + ecol];
      }
  }
  if constexpr (EPI == kRopeQkv) {
    const int d = p.head_dim;
    const int w = ecol - (ecol / d) * d;
    const int shift = p.start + (p.start_device != nullptr ? *p.start_device : 0);
#pragma unroll
    for (int mi = 0; mi < kTilesM; ++mi)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = min(m0 + mi * 16 + 4 * (lane >> 4) + r, p.rows - 1);
        const int tp = row - (row / p.seq) * p.seq;
        const int pos = min(max(shift + tp, 0), p.max_positions - 1);
        const int64_t ti = static_cast<int64_t>(pos) * (d / 2) + w / 2;
        rope_c[mi][r] = p.cos_t[ti];
        rope_s[mi][r] = p.sin_t[ti];
      }
  }

  // ---- A: the whole tile, direct to LDS (rows past the end read the last
  // row).  Buffer loads, not global_load_lds: after a global_load_lds the
  // compiler cannot see that the wait below covered it and turns its own
  // wait for the first weight fragment into vmcnt(0), so no MFMA would start
  // before every weight load of the ring had landed.
  {
    const int tile_rows = min(BM, p.rows - m0);
    const __amdgpu_buffer_rsrc_t x_rsrc =
        make_rsrc(p.x + static_cast<int64_t>(m0) * p.lda,
                  static_cast<uint32_t>(static_cast<int64_t>(tile_rows) * p.lda * 2));
    const int slots = BM * chunks;  // multiple of 64
    for (int i = wave; i < slots / kWave; i += 4) {
      const int s = i * kWave + lane;
      const int r = s / chunks;
      const int pc = s - r * chunks;
      const int c = (pc & ~swz) | ((pc ^ r) & swz);
      const uint32_t off =
          static_cast<uint32_t>((static_cast<int64_t>(min(r, tile_rows - 1)) * p.lda + c * 8) * 2);
      buffer_to_lds16(x_rsrc, a_lds + i * kWave * 8, off, 0);
    }
  }

  asm volatile("" ::: "memory");  // every A load is issued before any B load

  // ---- B: first PF k steps of this lane's fragments (columns past N read 0)
  const __amdgpu_buffer_rsrc_t b_rsrc =
      make_rsrc(p.w, static_cast<uint32_t>(static_cast<int64_t>(p.N) * K * 2));
  const uint32_t b_off = static_cast<uint32_t>((nw / 16) * ksteps * 64 + lane) * 16;
  uint4 bq[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) bq[i] = buffer_load16(b_rsrc, b_off, static_cast<uint32_t>(i) * 1024);

  // The A tile is complete when at most the PF weight loads issued after it
  // are still in flight.
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"i"(PF) : "memory");

  f32x4 acc[kTilesM];
#pragma unroll
  for (int i = 0; i < kTilesM; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int s0 = 0; s0 < ksteps; s0 += PF) {  // ksteps is a multiple of PF
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int step = s0 + i;
      bf16x8 af[kTilesM];
#pragma unroll
      for (int mi = 0; mi < kTilesM; ++mi) {
        const int r = mi * 16 + (lane & 15);
        const int c = step * 4 + (lane >> 4);
        const int pc = (c & ~swz) | ((c ^ r) & swz);
        af[mi] = lds_frag(&a_lds[(r * chunks + pc) * 8]);
      }
      asm volatile("s_waitcnt lgkmcnt(0)");
#pragma unroll
      for (int mi = 0; mi < kTilesM; ++mi) asm volatile("" : "+v"(af[mi]));
#pragma unroll
      for (int mi = 0; mi < kTilesM; ++mi)
        acc[mi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            af[mi], __builtin_bit_cast(bf16x8, bq[i]), acc[mi], 0, 0, 0);
      if (step + PF < ksteps)
        bq[i] = buffer_load16(b_rsrc, b_off, static_cast<uint32_t>(step + PF) * 1024);
    }
  }

  // ---- epilogue --------------------------------------------------------------
  const int col = nw + (lane & 15);
  if (nw >= p.N) return;  // whole wavefront past the last column (N % 16 == 0)

  if (EPI == kStore) {
#pragma unroll
    for (int mi = 0; mi < kTilesM; ++mi)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + mi * 16 + 4 * (lane >> 4) + r;
        if (row >= p.rows) continue;
        uint16_t v = f32_to_bf16(acc[mi][r]);
        if (p.addend != nullptr) v = f32_to_bf16(bf16_to_f32(add_v[mi][r]) + bf16_to_f32(v));
        p.out[static_cast<int64_t>(row) * p.ldo + col] = v;
      }
    return;
  }

  if (EPI == kStoreT) {
    // rows 4 (l / 16) .. + 3 of a lane are consecutive positions of one
    // sequence when seq % 4 == 0: one 8-byte store.
#pragma unroll
    for (int mi = 0; mi < kTilesM; ++mi) {
      const int row0 = m0 + mi * 16 + 4 * (lane >> 4);
      if (row0 >= p.rows) continue;
      const int b = row0 / p.seq;
      const int t0 = row0 - b * p.seq;
      uint16_t* dst = p.out + (static_cast<int64_t>(b) * p.N + col) * p.ld_keys;
      if ((p.seq & 3) == 0) {
        uint2 w;
        w.x = pack_bf16x2(acc[mi][0], acc[mi][1]);
        w.y = pack_bf16x2(acc[mi][2], acc[mi][3]);
        *reinterpret_cast<uint2*>(dst + t0) = w;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = row0 + r;
          if (row >= p.rows) break;
          const int bb = row / p.seq;
          p.out[(static_cast<int64_t>(bb) * p.N + col) * p.ld_keys + (row - bb * p.seq)] =
              f32_to_bf16(acc[mi][r]);
        }
      }
    }
    return;
  }

  if (EPI == kFrag) {
    // With both outputs, columns [0, N / 2) are K and [N / 2, N) are V
    // (N / 2 is a multiple of 16: one side per wavefront).
    const int d = p.head_dim;
    const bool both = p.kf != nullptr && p.vf != nullptr;
    const int half = both ? p.N / 2 : p.N;
    const bool to_v = p.kf == nullptr || (both && nw >= half);
    const int c2 = both && to_v ? col - half : col;
    const int head = c2 / d;
    const int w = c2 - head * d;
    const int heads = half / d;
#pragma unroll
    for (int mi = 0; mi < kTilesM; ++mi) {
      const int row0 = m0 + mi * 16 + 4 * (lane >> 4);
      if (row0 >= p.rows) continue;
      uint16_t bits[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) bits[r] = f32_to_bf16(acc[mi][r]);
      if (!to_v) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = row0 + r;
          if (row >= p.rows) break;
          const int b = row / p.seq;
          p.kf[kfrag_index(static_cast<int64_t>(b) * heads + head, p.nblk, row - b * p.seq, w,
                           d / 32)] = bits[r];
        }
      } else {
        store_values(p, bits, row0, head, heads, w);
      }
    }
    return;
  }

  // kRopeQkv
  const int d = p.head_dim;
  const int head = col / d;  // per lane; a rotation pair never straddles heads (d even)
  const int w = col - head * d;
  const int H = p.heads, Hk = p.kv_heads;
  const bool rotate = head < H + Hk;
  const bool odd = (lane & 1) != 0;
#pragma unroll
  for (int mi = 0; mi < kTilesM; ++mi) {
    float val[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      // round as the projection output, then rotate (identical to the
      // stand-alone kernel applied to the stored projection)
      const float self = bf16_to_f32(f32_to_bf16(acc[mi][r]));
      const float other = swap_pair(self);
      val[r] = self;
      if (rotate) {
        const float c = rope_c[mi][r], s = rope_s[mi][r];
        val[r] = odd ? rope_odd(other, self, c, s) : rope_even(self, other, c, s);
      }
    }
    const int row0 = m0 + mi * 16 + 4 * (lane >> 4);
    if (row0 >= p.rows) continue;
    uint16_t bits[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) bits[r] = f32_to_bf16(val[r]);
    if (head < H) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = row0 + r;
        if (row >= p.rows) break;
        const int b = row / p.seq;
        const int tp = row - b * p.seq;
        p.q[((static_cast<int64_t>(b) * H + head) * p.seq + tp) * d + w] = bits[r];
      }
    } else if (head < H + Hk) {
      const int kvh = head - H;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = row0 + r;
        if (row >= p.rows) break;
        const int b = row / p.seq;
        const int tp = row - b * p.seq;
        if (p.k != nullptr) p.k[((static_cast<int64_t>(b) * Hk + kvh) * p.seq + tp) * d + w] = bits[r];
        if (p.kf != nullptr)
          p.kf[kfrag_index(static_cast<int64_t>(b) * Hk + kvh, p.nblk, tp, w, d / 32)] = bits[r];
      }
    } else {
      store_values(p, bits, row0, head - H - Hk, Hk, w);
    }
  }
}

int ring_depth(int ksteps) {
  for (int pf = 8; pf > 1; pf >>= 1)
    if (ksteps % pf == 0) return pf;
  return 1;
}

template <int EPI>
hipError_t launch_proj(const ProjArgs& a, hipStream_t s) {
  if (a.rows == 0 || a.N == 0) return hipSuccess;
  const int tiles = ((a.rows + kProjRows - 1) / kProjRows) * ((a.N + kProjCols - 1) / kProjCols);
  const size_t lds = static_cast<size_t>(kProjRows) * a.K * 2;
  switch (a.K / 32) {
    case 4: proj_kernel<4, EPI, 4><<<tiles, 256, lds, s>>>(a); break;
    case 8: proj_kernel<8, EPI, 8><<<tiles, 256, lds, s>>>(a); break;
    case 16: proj_kernel<16, EPI, 16><<<tiles, 256, lds, s>>>(a); break;
    case 24: proj_kernel<24, EPI, 24><<<tiles, 256, lds, s>>>(a); break;
    default:
      switch (ring_depth(a.K / 32)) {
        case 8: proj_kernel<8, EPI, 0><<<tiles, 256, lds, s>>>(a); break;
        case 4: proj_kernel<4, EPI, 0><<<tiles, 256, lds, s>>>(a); break;
        default: proj_kernel<2, EPI, 0><<<tiles, 256, lds, s>>>(a); break;
      }
  }
  return hipGetLastError();
}

}  // namespace

bool proj_shape_supported(int k, int n) {
  return k > 0 && k % 64 == 0 && k <= kProjMaxK && n > 0 && n % 16 == 0;
}

hipError_t launch_proj_store(const uint16_t* x, int rows, int k, int64_t lda, const uint16_t* w,
                             int n, const uint16_t* addend, int64_t ld_addend, uint16_t* out,
                             int64_t ldo, hipStream_t s) {
  ProjArgs a{};
  a.x = x; a.lda = lda; a.rows = rows; a.K = k; a.N = n; a.w = w;
  a.out = out; a.ldo = ldo; a.addend = addend; a.ld_addend = ld_addend;
  a.seq = 1;
  return launch_proj<kStore>(a, s);
}

hipError_t launch_proj_transposed(const uint16_t* x, int rows, int seq, int k, const uint16_t* w,
                                  int n, int ld_keys, uint16_t* out, hipStream_t s) {
  ProjArgs a{};
  a.x = x; a.lda = k; a.rows = rows; a.K = k; a.N = n; a.w = w;
  a.out = out; a.seq = seq; a.ld_keys = ld_keys;
  return launch_proj<kStoreT>(a, s);
}

hipError_t launch_proj_rope_qkv(const uint16_t* x, int rows, int seq, int dim, const uint16_t* w,
                                const float* cos_t, const float* sin_t, int start,
                                const int32_t* start_device, int max_positions, int heads,
                                int kv_heads, int head_dim, int vt_keys, uint16_t* q,
                                uint16_t* k, uint16_t* v, uint16_t* kf, uint16_t* vf,
                                hipStream_t s) {
  ProjArgs a{};
  a.kf = kf; a.vf = vf; a.nblk = (seq + 31) / 32;
  a.x = x; a.lda = dim; a.rows = rows; a.K = dim; a.N = (heads + 2 * kv_heads) * head_dim;
  a.w = w; a.seq = seq; a.ld_keys = vt_keys;
  a.cos_t = cos_t; a.sin_t = sin_t; a.start = start; a.start_device = start_device;
  a.max_positions = max_positions;
  a.heads = heads; a.kv_heads = kv_heads; a.head_dim = head_dim;
  a.q = q; a.k = k; a.v = v;
  return launch_proj<kRopeQkv>(a, s);
}

hipError_t launch_proj_frag(const uint16_t* x, int rows, int seq, int k, int64_t lda,
                            const uint16_t* w, int n, int head_dim, uint16_t* kf, uint16_t* vf,
                            hipStream_t s) {
  ProjArgs a{};
  a.x = x; a.lda = lda; a.rows = rows; a.K = k; a.N = n; a.w = w;
  a.seq = seq; a.head_dim = head_dim; a.nblk = (seq + 31) / 32;
  a.kf = kf; a.vf = vf;
  return launch_proj<kFrag>(a, s);
}

}  // namespace parrot
