// Greedy next token without materialising the logits: argmax over the
// vocabulary of fp32 logits h . W[v] for each row of h.
//
// Reference semantics: decode_next = argmax(F.linear(h, embedding.weight))
// (parrot/model.py:714-715, 922, 927-931), and the reference's Apple kernels
// vocab_argmax_partials_bf16 / vocab_argmax_reduce_bf16
// (parrot/kernels/moe_bf16.metal:1541-1621): fp32 accumulation of bf16
// products, ties to the lower vocabulary index.  Keeping the logits in fp32
// (the bf16 head of the eager path rounds them first) makes the pick follow
// the fp32 model more closely.
//
// vocab_argmax_partials_kernel: wavefront w of workgroup g scans vocabulary
// rows 16 g + 4 w .. + 3 for every row of h.  A whole wavefront reads one
// vocabulary row (lane l takes 16-byte chunks l, l + 64, ..., so one load
// instruction reads 1 KB contiguous), the loads of all 4 rows issued before
// any arithmetic; the rows of h come from LDS and each dot is a wavefront
// sum.  Measured on MI355X: 5.6 TB/s over the 50 MB head at one row of h.
// vocab_argmax_reduce_kernel picks the best of the per-wavefront partials.
#include "common.h"

namespace parrot {

namespace {

constexpr int kVocabRowsPerWave = 4;
constexpr int kVocabRowsPerGroup = 4 * kVocabRowsPerWave;
constexpr int kVocabMaxRows = 16;  // rows of h per launch

__device__ __forceinline__ float dot8v(uint4 a, uint4 b) {
  return lo_bf16(a.x) * lo_bf16(b.x) + hi_bf16(a.x) * hi_bf16(b.x) +
         lo_bf16(a.y) * lo_bf16(b.y) + hi_bf16(a.y) * hi_bf16(b.y) +
         lo_bf16(a.z) * lo_bf16(b.z) + hi_bf16(a.z) * hi_bf16(b.z) +
         lo_bf16(a.w) * lo_bf16(b.w) + hi_bf16(a.w) * hi_bf16(b.w);
}

// (value, index) keys: larger value wins, then the lower index.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// NCH = ceil(dim / 8 / 64) chunks per lane per vocabulary row; RB >= rows.
template <int NCH, int RB>
__global__ __launch_bounds__(256) void vocab_argmax_partials_kernel(
    const uint16_t* __restrict__ h, int rows, int dim, const uint16_t* __restrict__ w, int vocab,
    float* __restrict__ part_v, int32_t* __restrict__ part_i) {
  // The kernel arguments in one batch of scalar loads before any use.
  asm volatile("" ::"s"(h), "s"(rows), "s"(dim), "s"(w), "s"(vocab), "s"(part_v), "s"(part_i));
  __builtin_amdgcn_sched_barrier(0);
  extern __shared__ __attribute__((aligned(16))) uint16_t hs[];  // [rows][dim]
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int chunks = dim / 8;
  const int v0 = blockIdx.x * kVocabRowsPerGroup + wave * kVocabRowsPerWave;
  uint4 wr[kVocabRowsPerWave][NCH];
#pragma unroll
  for (int r = 0; r < kVocabRowsPerWave; ++r) {
    const uint4* row = reinterpret_cast<const uint4*>(
        w + static_cast<int64_t>(min(v0 + r, vocab - 1)) * dim);
#pragma unroll
    for (int c = 0; c < NCH; ++c) wr[r][c] = row[min(lane + 64 * c, chunks - 1)];
  }
  for (int i = tid; i < rows * chunks; i += 256)
    reinterpret_cast<uint4*>(hs)[i] = reinterpret_cast<const uint4*>(h)[i];
  __syncthreads();

  float bv[RB];
  int bi[RB];
#pragma unroll
  for (int b = 0; b < RB; ++b) {
    bv[b] = -INFINITY;
    bi[b] = 0x7fffffff;
  }
#pragma unroll
  for (int b = 0; b < RB; ++b) {
    if (b < rows) {
      uint4 hv[NCH];
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        hv[c] = reinterpret_cast<const uint4*>(hs + b * dim)[min(lane + 64 * c, chunks - 1)];
#pragma unroll
      for (int r = 0; r < kVocabRowsPerWave; ++r) {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c)
          if (lane + 64 * c < chunks) acc += dot8v(wr[r][c], hv[c]);
        acc = wave_sum(acc);  // uniform across the wavefront
        if (v0 + r < vocab && better(acc, v0 + r, bv[b], bi[b])) {
          bv[b] = acc;
          bi[b] = v0 + r;
        }
      }
    }
  }
  // rows ascend with the wavefront index, so a later wavefront only wins
  // with a strictly larger logit: the per-wavefront partials keep the order.
  const int64_t waves = static_cast<int64_t>(gridDim.x) * 4;
  if (lane == 0) {
#pragma unroll
    for (int b = 0; b < RB; ++b)
      if (b < rows) {
        part_v[b * waves + blockIdx.x * 4 + wave] = bv[b];
        part_i[b * waves + blockIdx.x * 4 + wave] = bi[b];
      }
  }
}

// Two or more rows of h: the dots are a GEMM [vocab x dim] . [dim x rows]
// on v_mfma_f32_16x16x32_bf16, so the VALU work per head byte no longer grows
// with the rows (the wavefront-sum kernel above runs 9.5 / 12 / 18 / 30 us
// at 1 / 2 / 4 / 8 rows).  Wavefront w of workgroup g takes vocabulary rows
// v0 = 64 g + 16 w .. v0 + 15 as the A operand (lane l: row l % 16) and the
// rows of h, staged in LDS with a padded stride, as B (lane l: h row l % 16,
// zero past `rows`).  The k order pairs the steps: steps 2j and 2j + 1 give
// lane group c = l / 16 the elements 64 j + 16 c .. + 7 and + 8 .. + 15, so
// each lane reads 32 contiguous bytes of its vocabulary row per pair and a
// pair of load instructions covers 128 contiguous bytes of every row.  The
// C fragment gives lane l the logits of h row l % 16 and vocabulary rows
// v0 + 4 (l / 16) + r; the best (value, lower index) of each h row is taken
// over r and then over the four lane groups, and lane n < rows writes h row
// n's partial for this wavefront.  The fp32 sums are MFMA sums over the
// same bf16 products, in another order than the wavefront sums.
constexpr int kVocabMfmaRows = 64;  // vocabulary rows per workgroup
constexpr int kVocabMfmaSteps = 24;  // k steps of head loads in flight per lane

__global__ __launch_bounds__(256) void vocab_argmax_mfma_kernel(
    const uint16_t* __restrict__ h, int rows, int dim, const uint16_t* __restrict__ w, int vocab,
    float* __restrict__ part_v, int32_t* __restrict__ part_i) {
  // The kernel arguments in one batch of scalar loads before any use.
  asm volatile("" ::"s"(h), "s"(rows), "s"(dim), "s"(w), "s"(vocab), "s"(part_v), "s"(part_i));
  __builtin_amdgcn_sched_barrier(0);
  extern __shared__ __attribute__((aligned(16))) uint16_t hs[];  // [rows][dim + 8]
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int c = lane >> 4;
  const int steps = dim / 32;  // even: dim % 64 == 0
  const int hstride = dim + 8;
  const int v0 = blockIdx.x * kVocabMfmaRows + wave * 16;
  const uint16_t* wrow =
      w + static_cast<int64_t>(min(v0 + (lane & 15), vocab - 1)) * dim + 16 * c;
  // Element offset (within a row) of this lane's 8 values at k step s.
  auto koff = [&](int s) { return 64 * (s >> 1) + 8 * (s & 1); };
  const int n = lane & 15;  // this lane's h row (B column)
  const bool live = n < rows;
  const uint16_t* hrow = hs + (live ? n : 0) * hstride + 16 * c;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < steps; s0 += kVocabMfmaSteps) {
    bf16x8 a[kVocabMfmaSteps];
#pragma unroll
    for (int i = 0; i < kVocabMfmaSteps; ++i)
      a[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(
                                            wrow + koff(min(s0 + i, steps - 1))));
    if (s0 == 0) {
      // h into LDS behind the first head loads (rows x dim / 8 chunks).
      const int chunks = dim / 8;
      for (int i = tid; i < rows * chunks; i += 256) {
        const int r = i / chunks;
        *reinterpret_cast<uint4*>(hs + r * hstride + (i - r * chunks) * 8) =
            reinterpret_cast<const uint4*>(h)[i];
      }
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < kVocabMfmaSteps; ++i) {
      const int st = s0 + i;
      if (st < steps) {
        const uint4 hv = live ? *reinterpret_cast<const uint4*>(hrow + koff(st))
                              : make_uint4(0u, 0u, 0u, 0u);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], __builtin_bit_cast(bf16x8, hv),
                                                      acc, 0, 0, 0);
      }
    }
  }
  float bv = -INFINITY;
  int bi = 0x7fffffff;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int v = v0 + 4 * c + r;
    if (v < vocab && better(acc[r], v, bv, bi)) {
      bv = acc[r];
      bi = v;
    }
  }
#pragma unroll
  for (int m = 16; m < kWave; m <<= 1) {
    const float ov = __shfl_xor(bv, m);
    const int oi = __shfl_xor(bi, m);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane < rows) {
    const int64_t groups = static_cast<int64_t>(gridDim.x) * 4;
    part_v[lane * groups + blockIdx.x * 4 + wave] = bv;
    part_i[lane * groups + blockIdx.x * 4 + wave] = bi;
  }
}

// One workgroup per row of h.  The row's partials are read as float4 / int4,
// every load of a lane issued before the first compare (a loop with a load,
// a wait and a compare per partial took ~11 us for 8192 partials), then
// reduced within each wavefront by xor shuffles and across the 4 wavefronts
// through LDS.  `better` is a total order (value, then the lower index), so
// the winner does not depend on the order of comparisons.
constexpr int kReduceLoads = 8;  // 16-byte loads of each kind in flight per lane

__device__ __forceinline__ void keep_better(float pv, int pi, float& v, int& i) {
  if (better(pv, pi, v, i)) {
    v = pv;
    i = pi;
  }
}

__global__ __launch_bounds__(256) void vocab_argmax_reduce_kernel(
    const float* __restrict__ part_v, const int32_t* __restrict__ part_i, int groups,
    int64_t* __restrict__ out, int32_t* __restrict__ advance) {
  // The kernel arguments in one batch of scalar loads before any use.
  asm volatile("" ::"s"(part_v), "s"(part_i), "s"(groups), "s"(out), "s"(advance));
  __builtin_amdgcn_sched_barrier(0);
  __shared__ float vs[4];
  __shared__ int is[4];
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  const int n4 = groups / 4;  // groups % 4 == 0
  const float4* pv4 = reinterpret_cast<const float4*>(part_v + static_cast<int64_t>(r) * groups);
  const int4* pi4 = reinterpret_cast<const int4*>(part_i + static_cast<int64_t>(r) * groups);
  float v = -INFINITY;
  int i = 0x7fffffff;
  for (int g0 = tid; g0 < n4; g0 += 256 * kReduceLoads) {
    float4 a[kReduceLoads];
    int4 b[kReduceLoads];
#pragma unroll
    for (int u = 0; u < kReduceLoads; ++u) {
      const int g = min(g0 + u * 256, n4 - 1);  // clamped: a repeat changes nothing
      a[u] = pv4[g];
      b[u] = pi4[g];
    }
#pragma unroll
    for (int u = 0; u < kReduceLoads; ++u) {
      keep_better(a[u].x, b[u].x, v, i);
      keep_better(a[u].y, b[u].y, v, i);
      keep_better(a[u].z, b[u].z, v, i);
      keep_better(a[u].w, b[u].w, v, i);
    }
  }
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const float ov = __shfl_xor(v, m);
    const int oi = __shfl_xor(i, m);
    keep_better(ov, oi, v, i);
  }
  if ((tid & (kWave - 1)) == 0) {
    vs[tid >> 6] = v;
    is[tid >> 6] = i;
  }
  __syncthreads();
  if (tid == 0) {
#pragma unroll
    for (int w = 1; w < 4; ++w) keep_better(vs[w], is[w], v, i);
    out[r] = i;
    // The decode step's last launch: it advances the device position the
    // step's attention kernels read (no kernel of this launch reads it).
    if (r == 0 && advance != nullptr) *advance += 1;
  }
}

}  // namespace

int vocab_argmax_max_rows() { return kVocabMaxRows; }

// Partials per row of h: one per wavefront.
int vocab_argmax_groups(int vocab) {
  return 4 * ((vocab + kVocabRowsPerGroup - 1) / kVocabRowsPerGroup);
}

hipError_t launch_vocab_argmax(const uint16_t* h, int rows, int dim, const uint16_t* w, int vocab,
                               float* part_v, int32_t* part_i, int64_t* out, int32_t* advance,
                               hipStream_t s) {
  if (rows == 0) return hipSuccess;
  // The MFMA kernel whenever the widest batch fits (16 rows of h staged in at
  // most 64 KB of LDS), at every row count: the kernel is chosen from dim
  // alone, so a row's logits are summed in the same order whether it is
  // decoded alone or in a batch, and its greedy token does not depend on
  // the batch it is in.  An MFMA output element depends only on its own
  // row and column; the unused B columns are zero.
  const size_t mfma_lds = static_cast<size_t>(rows) * (dim + 8) * sizeof(uint16_t);
  const size_t mfma_lds_max = static_cast<size_t>(kVocabMaxRows) * (dim + 8) * sizeof(uint16_t);
  if (dim % 64 == 0 && mfma_lds_max <= 65536) {
    const int blocks = (vocab + kVocabMfmaRows - 1) / kVocabMfmaRows;
    vocab_argmax_mfma_kernel<<<blocks, 256, mfma_lds, s>>>(h, rows, dim, w, vocab, part_v,
                                                           part_i);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    vocab_argmax_reduce_kernel<<<rows, 256, 0, s>>>(part_v, part_i, 4 * blocks, out, advance);
    return hipGetLastError();
  }
  const int blocks = (vocab + kVocabRowsPerGroup - 1) / kVocabRowsPerGroup;
  const size_t lds = static_cast<size_t>(rows) * dim * sizeof(uint16_t);
  const int nch = (dim / 8 + 63) / 64;
  const int rb = rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : rows <= 8 ? 8 : 16;
#define PARROT_VOCAB(NCH, RB)                                                             \
  vocab_argmax_partials_kernel<NCH, RB><<<blocks, 256, lds, s>>>(h, rows, dim, w, vocab, \
                                                                 part_v, part_i)
#define PARROT_VOCAB_RB(NCH)          \
  switch (rb) {                       \
    case 1: PARROT_VOCAB(NCH, 1); break; \
    case 2: PARROT_VOCAB(NCH, 2); break; \
    case 4: PARROT_VOCAB(NCH, 4); break; \
    case 8: PARROT_VOCAB(NCH, 8); break; \
    default: PARROT_VOCAB(NCH, 16); break; \
  }
  switch (nch) {
    case 1: PARROT_VOCAB_RB(1); break;
    case 2: PARROT_VOCAB_RB(2); break;
    case 3: PARROT_VOCAB_RB(3); break;
    default: PARROT_VOCAB_RB(4); break;
  }
#undef PARROT_VOCAB_RB
#undef PARROT_VOCAB
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  vocab_argmax_reduce_kernel<<<rows, 256, 0, s>>>(part_v, part_i, vocab_argmax_groups(vocab), out,
                                                  advance);
  return hipGetLastError();
}

}  // namespace parrot
