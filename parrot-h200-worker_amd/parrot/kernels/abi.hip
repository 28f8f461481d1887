// extern "C" entry points declared in include/parrot_hip.h.
//
// Every entry point validates its arguments on the host and returns a
// negative PARROT_ERR_* code before launching anything, or the hipError_t
// of its launches.  Nothing here allocates or synchronises.  The only
// global state is the per-device address of the static scratch array, set
// once per device by parrot_grouped_experts_static_bf16.
#include "../../../include/parrot_hip.h"

#include <atomic>

#include "common.h"

namespace {

using parrot::kMaxDepthSources;
using parrot::kMaxExperts;

constexpr size_t kAlign = 256;

size_t round_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int status(hipError_t e) { return e == hipSuccess ? PARROT_OK : static_cast<int>(e); }

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Route workspace: block histograms [route_blocks, E], then chunk totals
// [route_chunks, E] for the two-level scan of long inputs.
size_t route_hist_bytes(int64_t tokens, int32_t experts) {
  return round_up(static_cast<size_t>(parrot::route_blocks(tokens)) * experts * sizeof(int32_t));
}

size_t route_ws_bytes(int64_t tokens, int32_t experts) {
  return route_hist_bytes(tokens, experts) +
         round_up(static_cast<size_t>(parrot::route_chunks(tokens)) * experts * sizeof(int32_t));
}

int32_t* route_chunk_totals(void* workspace, int64_t tokens, int32_t experts) {
  return reinterpret_cast<int32_t*>(static_cast<char*>(workspace) +
                                    route_hist_bytes(tokens, experts));
}

struct ExpertsWorkspace {
  uint16_t* hidden;
  uint16_t* y_routed;  // bf16 [2T, dim], route-weighted expert outputs
  uint16_t* y_shared;  // bf16 [T, dim]
  size_t bytes;
};

ExpertsWorkspace experts_ws(void* base, int64_t tokens, int32_t dim, int32_t hidden_dim,
                            int32_t shared_dim) {
  const size_t hstride = static_cast<size_t>(hidden_dim > shared_dim ? hidden_dim : shared_dim);
  const size_t h_bytes = round_up(3 * static_cast<size_t>(tokens) * hstride * sizeof(uint16_t));
  const size_t yr_bytes = round_up(2 * static_cast<size_t>(tokens) * dim * sizeof(uint16_t));
  const size_t ys_bytes = round_up(static_cast<size_t>(tokens) * dim * sizeof(uint16_t));
  char* p = static_cast<char*>(base);
  ExpertsWorkspace ws;
  ws.hidden = reinterpret_cast<uint16_t*>(p);
  ws.y_routed = reinterpret_cast<uint16_t*>(p + h_bytes);
  ws.y_shared = reinterpret_cast<uint16_t*>(p + h_bytes + yr_bytes);
  ws.bytes = h_bytes + yr_bytes + ys_bytes;
  return ws;
}

int check_group_outputs(int32_t* positions, int32_t* counts, int32_t* offsets, int32_t* perm,
                        int32_t* overflow) {
  if (!positions || !counts || !offsets || !perm || !overflow) return PARROT_ERR_NULL_POINTER;
  return PARROT_OK;
}

int check_route_shape(int64_t tokens, int32_t experts, int32_t capacity) {
  if (tokens < 0 || tokens > (int64_t{1} << 29)) return PARROT_ERR_BAD_SHAPE;
  if (experts < 2 || experts > kMaxExperts) return PARROT_ERR_UNSUPPORTED;
  if (capacity < 1) return PARROT_ERR_BAD_SHAPE;
  if (static_cast<int64_t>(experts) * capacity > (int64_t{1} << 30)) return PARROT_ERR_BAD_SHAPE;
  return PARROT_OK;
}

}  // namespace

extern "C" {

int parrot_abi_version(void) { return PARROT_ABI_VERSION; }

const char* parrot_status_string(int s) {
  switch (s) {
    case PARROT_OK: return "ok";
    case PARROT_ERR_NULL_POINTER: return "a required pointer is NULL";
    case PARROT_ERR_BAD_SHAPE: return "invalid shape or size";
    case PARROT_ERR_UNSUPPORTED: return "shape outside the supported range of the HIP kernels";
    case PARROT_ERR_WORKSPACE: return "workspace missing or too small";
    case PARROT_ERR_ALIGNMENT: return "tensor pointer is not 16-byte aligned";
    case PARROT_ERR_SCRATCH_LIMIT:
      return "input needs more than the static scratch array (PARROT_STATIC_SCRATCH_BYTES)";
    default: break;
  }
  if (s > 0) return hipGetErrorString(static_cast<hipError_t>(s));
  return "unknown status";
}

int32_t parrot_capacity(int64_t tokens, int32_t experts) {
  if (experts <= 0 || tokens < 0) return 0;
  const int64_t assignments = 2 * tokens;
  const int64_t per = (2 * assignments + experts - 1) / experts;
  const int64_t c = (per + 7) / 8 * 8;
  return static_cast<int32_t>(c < 8 ? 8 : c);
}

int parrot_rms_norm_bf16(const void* x, const void* weight, void* out, int64_t rows,
                         int32_t dim, float eps, void* stream) {
  if (!x || !weight || !out) return PARROT_ERR_NULL_POINTER;
  if (rows < 0 || dim <= 0 || dim % 4) return PARROT_ERR_BAD_SHAPE;
  if (dim > 4096) return PARROT_ERR_UNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
       reinterpret_cast<uintptr_t>(out)) & 7u)
    return PARROT_ERR_ALIGNMENT;
  return status(parrot::launch_rms_norm(static_cast<const uint16_t*>(x),
                                        static_cast<const uint16_t*>(weight),
                                        static_cast<uint16_t*>(out), rows, dim, eps,
                                        as_stream(stream)));
}

static int depth_mix_entry(const void* const* sources, int32_t n_sources, const void* query,
                           const void* score_norm_weight, float score_eps,
                           const void* out_norm_weight, float out_eps, int64_t tokens,
                           int32_t dim, void* out_mix, void* out_norm,
                           const parrot::RouteOut* route, void* stream,
                           const parrot::PendingSum* pend = nullptr) {
  if (!sources || !query || !score_norm_weight) return PARROT_ERR_NULL_POINTER;
  if (!out_mix && !out_norm) return PARROT_ERR_NULL_POINTER;
  if (out_norm && !out_norm_weight) return PARROT_ERR_NULL_POINTER;
  if (n_sources < 1 || n_sources > kMaxDepthSources) return PARROT_ERR_UNSUPPORTED;
  if (tokens < 0 || dim <= 0 || dim % 4) return PARROT_ERR_BAD_SHAPE;
  if (dim > 2048) return PARROT_ERR_UNSUPPORTED;
  parrot::DepthSources srcs{};
  uintptr_t bits = reinterpret_cast<uintptr_t>(query) |
                   reinterpret_cast<uintptr_t>(score_norm_weight) |
                   reinterpret_cast<uintptr_t>(out_norm_weight) |
                   reinterpret_cast<uintptr_t>(out_mix) | reinterpret_cast<uintptr_t>(out_norm);
  for (int s = 0; s < kMaxDepthSources; ++s) {
    const void* p = sources[s < n_sources ? s : 0];
    if (!p) return PARROT_ERR_NULL_POINTER;
    bits |= reinterpret_cast<uintptr_t>(p);
    srcs.src[s] = static_cast<const uint16_t*>(p);
  }
  if (bits & 7u) return PARROT_ERR_ALIGNMENT;
  return status(parrot::launch_depth_mix(
      srcs, n_sources, static_cast<const uint16_t*>(query),
      static_cast<const uint16_t*>(score_norm_weight), score_eps,
      static_cast<const uint16_t*>(out_norm_weight), out_eps, tokens, dim,
      static_cast<uint16_t*>(out_mix), static_cast<uint16_t*>(out_norm), nullptr, route,
      as_stream(stream), pend));
}

int parrot_depth_mix_bf16(const void* const* sources, int32_t n_sources, const void* query,
                          const void* score_norm_weight, float score_eps,
                          const void* out_norm_weight, float out_eps, int64_t tokens,
                          int32_t dim, void* out_mix, void* out_norm, void* stream) {
  return depth_mix_entry(sources, n_sources, query, score_norm_weight, score_eps,
                         out_norm_weight, out_eps, tokens, dim, out_mix, out_norm, nullptr,
                         stream);
}

int parrot_embed_depth_mix_bf16(const int64_t* ids, int64_t tokens, const void* table,
                                int64_t vocab, int32_t dim, const void* query,
                                const void* score_norm_weight, float score_eps,
                                const void* out_norm_weight, float out_eps, void* rows_out,
                                void* out_norm, float* zeros, int32_t n_zeros, void* stream) {
  if (!table || !query || !score_norm_weight || !out_norm_weight) return PARROT_ERR_NULL_POINTER;
  if (tokens > 0 && (!ids || !rows_out || !out_norm)) return PARROT_ERR_NULL_POINTER;
  if (n_zeros > 0 && !zeros) return PARROT_ERR_NULL_POINTER;
  if (tokens < 0 || tokens > (int64_t{1} << 31) - 1 || vocab < 1 || n_zeros < 0 || dim <= 0 ||
      dim % 4)
    return PARROT_ERR_BAD_SHAPE;
  if (dim > 2048) return PARROT_ERR_UNSUPPORTED;
  const uintptr_t bits = reinterpret_cast<uintptr_t>(table) | reinterpret_cast<uintptr_t>(query) |
                         reinterpret_cast<uintptr_t>(score_norm_weight) |
                         reinterpret_cast<uintptr_t>(out_norm_weight) |
                         reinterpret_cast<uintptr_t>(rows_out) |
                         reinterpret_cast<uintptr_t>(out_norm);
  if (bits & 7u) return PARROT_ERR_ALIGNMENT;
  return status(parrot::launch_embed_mix(
      ids, static_cast<const uint16_t*>(table), vocab, static_cast<const uint16_t*>(query),
      static_cast<const uint16_t*>(score_norm_weight), score_eps,
      static_cast<const uint16_t*>(out_norm_weight), out_eps, tokens, dim,
      static_cast<uint16_t*>(rows_out), static_cast<uint16_t*>(out_norm), zeros, n_zeros,
      as_stream(stream)));
}

int parrot_depth_mix_route_bf16(const void* const* sources, int32_t n_sources,
                                const void* query, const void* score_norm_weight,
                                float score_eps, const void* out_norm_weight, float out_eps,
                                int64_t tokens, int32_t dim, void* out_mix, void* out_norm,
                                const void* router_weight, const float* logit_bias,
                                int32_t experts, float* out_weights, int64_t* out_indices,
                                void* stream) {
  if (!out_norm || !router_weight || !out_weights || !out_indices) return PARROT_ERR_NULL_POINTER;
  if (experts < 2 || experts > kMaxExperts) return PARROT_ERR_UNSUPPORTED;
  if (dim % 32) return PARROT_ERR_UNSUPPORTED;
  if (!aligned16(router_weight)) return PARROT_ERR_ALIGNMENT;
  const parrot::RouteOut route{static_cast<const uint16_t*>(router_weight), logit_bias, experts,
                               out_weights, out_indices};
  return depth_mix_entry(sources, n_sources, query, score_norm_weight, score_eps,
                         out_norm_weight, out_eps, tokens, dim, out_mix, out_norm, &route,
                         stream);
}

int parrot_depth_mix_route_pending_bf16(
    const void* const* sources, int32_t n_sources, const void* query,
    const void* score_norm_weight, float score_eps, const void* out_norm_weight, float out_eps,
    int64_t tokens, int32_t dim, void* out_norm, const void* router_weight,
    const float* logit_bias, int32_t experts, float* out_weights, int64_t* out_indices,
    const float* contributions, int32_t heads, const void* base, void* resolved, void* stream) {
  if (!out_norm || !router_weight || !out_weights || !out_indices || !contributions || !resolved)
    return PARROT_ERR_NULL_POINTER;
  if (experts < 2 || experts > kMaxExperts) return PARROT_ERR_UNSUPPORTED;
  if (dim % 32) return PARROT_ERR_UNSUPPORTED;
  if (heads != parrot::kPendingHeads || n_sources < 2) return PARROT_ERR_UNSUPPORTED;
  if (!aligned16(router_weight) || !aligned16(contributions)) return PARROT_ERR_ALIGNMENT;
  if ((reinterpret_cast<uintptr_t>(base) | reinterpret_cast<uintptr_t>(resolved)) & 7u)
    return PARROT_ERR_ALIGNMENT;
  const parrot::RouteOut route{static_cast<const uint16_t*>(router_weight), logit_bias, experts,
                               out_weights, out_indices};
  const parrot::PendingSum pend{contributions, static_cast<const uint16_t*>(base),
                                static_cast<uint16_t*>(resolved)};
  return depth_mix_entry(sources, n_sources, query, score_norm_weight, score_eps,
                         out_norm_weight, out_eps, tokens, dim, nullptr, out_norm, &route, stream,
                         &pend);
}

int parrot_rope_qkv_bf16(const void* qkv, const float* cos_table, const float* sin_table,
                         int64_t batch, int32_t seq, int32_t start, const int32_t* start_device,
                         int32_t max_positions, int32_t heads, int32_t kv_heads,
                         int32_t head_dim, int32_t expand_kv, int32_t vt_keys, void* q,
                         void* k, void* v, void* stream) {
  if (!qkv || !cos_table || !sin_table || !q || !k || !v) return PARROT_ERR_NULL_POINTER;
  if (batch < 0 || seq < 0 || start < 0 || heads <= 0 || kv_heads <= 0 || head_dim <= 0 ||
      max_positions <= 0 || vt_keys < 0)
    return PARROT_ERR_BAD_SHAPE;
  if (heads % kv_heads || head_dim % 4) return PARROT_ERR_UNSUPPORTED;
  if (static_cast<int64_t>(start) + seq > max_positions) return PARROT_ERR_BAD_SHAPE;
  if (vt_keys > 0 && (vt_keys < seq || expand_kv)) return PARROT_ERR_BAD_SHAPE;
  const uintptr_t bits = reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(q) |
                         reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v);
  if (bits & 7u) return PARROT_ERR_ALIGNMENT;
  return status(parrot::launch_rope_qkv(
      static_cast<const uint16_t*>(qkv), cos_table, sin_table, batch, seq, start, start_device,
      max_positions, heads, kv_heads, head_dim, expand_kv, vt_keys, static_cast<uint16_t*>(q),
      static_cast<uint16_t*>(k), static_cast<uint16_t*>(v), as_stream(stream)));
}

static int check_decode_shape(int32_t batch, int32_t heads, int32_t kv_heads, int32_t head_dim,
                              int32_t max_positions, int32_t window) {
  if (batch < 0 || heads <= 0 || kv_heads <= 0 || head_dim <= 0 || max_positions <= 0 ||
      window <= 0)
    return PARROT_ERR_BAD_SHAPE;
  if (heads % kv_heads || !parrot::decode_head_dim_supported(head_dim))
    return PARROT_ERR_UNSUPPORTED;
  if (parrot::decode_attention_lds_bytes(window, max_positions, head_dim) > parrot::kMaxDecodeLds)
    return PARROT_ERR_UNSUPPORTED;
  return PARROT_OK;
}

int parrot_decode_attention_bf16(const void* q, const void* k_new, const void* v_new,
                                 void* key_cache, void* value_cache, const int32_t* position,
                                 int32_t batch, int32_t heads, int32_t kv_heads,
                                 int32_t head_dim, int32_t max_positions, int32_t window,
                                 float scale, void* out, void* stream) {
  if (!q || !k_new || !v_new || !key_cache || !value_cache || !position || !out)
    return PARROT_ERR_NULL_POINTER;
  if (int rc = check_decode_shape(batch, heads, kv_heads, head_dim, max_positions, window))
    return rc;
  if (!aligned16(k_new) || !aligned16(v_new) || !aligned16(key_cache) || !aligned16(value_cache))
    return PARROT_ERR_ALIGNMENT;
  return status(parrot::launch_decode_attention(
      static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k_new),
      static_cast<const uint16_t*>(v_new), static_cast<uint16_t*>(key_cache),
      static_cast<uint16_t*>(value_cache), position, batch, heads, kv_heads, head_dim,
      max_positions, window, scale, static_cast<uint16_t*>(out), as_stream(stream)));
}

static int check_decode_heads_shape(int32_t batch, int32_t heads, int32_t kv_heads,
                                    int32_t head_dim, int32_t max_positions, int32_t window,
                                    int32_t dim) {
  if (int rc = check_decode_shape(batch, heads, kv_heads, head_dim, max_positions, window))
    return rc;
  if (dim <= 0) return PARROT_ERR_BAD_SHAPE;
  if (dim % parrot::kDecodeHeadsParts || dim / parrot::kDecodeHeadsParts > 256 ||
      parrot::decode_attention_lds_bytes(window, max_positions, head_dim) +
              static_cast<size_t>(head_dim) * sizeof(float) > parrot::kMaxDecodeLds)
    return PARROT_ERR_UNSUPPORTED;
  return PARROT_OK;
}

int parrot_decode_attention_heads_check(int32_t batch, int32_t heads, int32_t kv_heads,
                                        int32_t head_dim, int32_t max_positions, int32_t window,
                                        int32_t dim) {
  if (int rc = check_decode_heads_shape(batch, heads, kv_heads, head_dim, max_positions, window,
                                        dim))
    return rc;
  // The pending input mix of parrot_depth_mix_decode_moe_pending_bf16 takes
  // one lane per head.
  if (heads > parrot::kMaxPendingLanes || dim > 1024 || dim % 4) return PARROT_ERR_UNSUPPORTED;
  return PARROT_OK;
}

int parrot_decode_attention_heads_bf16(const void* q, const void* k_new, const void* v_new,
                                       void* key_cache, void* value_cache,
                                       const int32_t* position, int32_t batch, int32_t heads,
                                       int32_t kv_heads, int32_t head_dim, int32_t max_positions,
                                       int32_t window, float scale, const void* out_weight,
                                       int32_t dim, float* contributions, void* stream) {
  if (!q || !k_new || !v_new || !key_cache || !value_cache || !position || !out_weight ||
      !contributions)
    return PARROT_ERR_NULL_POINTER;
  if (int rc = check_decode_heads_shape(batch, heads, kv_heads, head_dim, max_positions, window,
                                        dim))
    return rc;
  if (!aligned16(k_new) || !aligned16(v_new) || !aligned16(key_cache) ||
      !aligned16(value_cache) || !aligned16(out_weight))
    return PARROT_ERR_ALIGNMENT;
  return status(parrot::launch_decode_attention_heads(
      static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k_new),
      static_cast<const uint16_t*>(v_new), static_cast<uint16_t*>(key_cache),
      static_cast<uint16_t*>(value_cache), position, batch, heads, kv_heads, head_dim,
      max_positions, window, scale, static_cast<const uint16_t*>(out_weight), dim, contributions,
      as_stream(stream)));
}

int parrot_decode_attention_latent_f32(const float* q, const void* latent_new, void* latent_cache,
                                       const int32_t* position, int32_t batch, int32_t heads,
                                       int32_t latent_dim, int32_t max_positions, float scale,
                                       float* out, void* stream) {
  if (!q || !latent_new || !latent_cache || !position || !out) return PARROT_ERR_NULL_POINTER;
  if (int rc = check_decode_shape(batch, heads, 1, latent_dim, max_positions, max_positions))
    return rc;
  if (!aligned16(latent_new) || !aligned16(latent_cache)) return PARROT_ERR_ALIGNMENT;
  return status(parrot::launch_decode_attention_latent(
      q, static_cast<const uint16_t*>(latent_new), static_cast<uint16_t*>(latent_cache),
      position, batch, heads, latent_dim, max_positions, scale, out, as_stream(stream)));
}

// The depth mix a decode launch makes its input rows with: checks and fills
// `mix` from the sources (as parrot_depth_mix_bf16 takes them) and the norms.
static int make_decode_mix(const void* const* sources, int32_t n_sources, const void* query,
                           const void* score_norm_weight, float score_eps,
                           const void* norm_weight, float norm_eps, parrot::DecodeMix& mix) {
  if (!sources || !query || !score_norm_weight || !norm_weight) return PARROT_ERR_NULL_POINTER;
  if (n_sources < 1 || n_sources > kMaxDepthSources) return PARROT_ERR_UNSUPPORTED;
  uintptr_t bits = reinterpret_cast<uintptr_t>(query) |
                   reinterpret_cast<uintptr_t>(score_norm_weight) |
                   reinterpret_cast<uintptr_t>(norm_weight);
  for (int s = 0; s < kMaxDepthSources; ++s) {
    const void* p = sources[s < n_sources ? s : 0];
    if (!p) return PARROT_ERR_NULL_POINTER;
    bits |= reinterpret_cast<uintptr_t>(p);
    mix.srcs.src[s] = static_cast<const uint16_t*>(p);
  }
  if (bits & 7u) return PARROT_ERR_ALIGNMENT;
  mix.n_sources = n_sources;
  mix.query = static_cast<const uint16_t*>(query);
  mix.score_w = static_cast<const uint16_t*>(score_norm_weight);
  mix.score_eps = score_eps;
  mix.out_w = static_cast<const uint16_t*>(norm_weight);
  mix.out_eps = norm_eps;
  return PARROT_OK;
}

int parrot_decode_qkv_bf16(const void* x, const void* const* sources, int32_t n_sources,
                           const void* query, const void* score_norm_weight, float score_eps,
                           const void* attention_norm_weight, float norm_eps, int32_t tokens,
                           int32_t dim, const void* qkv_weight, int32_t heads,
                           int32_t kv_heads, int32_t head_dim, const float* cos_table,
                           const float* sin_table, int32_t max_positions,
                           const int32_t* position, void* q, void* k, void* v, void* stream) {
  if ((!x && !sources) || !qkv_weight || !cos_table || !sin_table || !position || !q || !k ||
      !v)
    return PARROT_ERR_NULL_POINTER;
  if (tokens < 0 || dim <= 0 || heads <= 0 || kv_heads <= 0 || head_dim <= 0 ||
      max_positions <= 0)
    return PARROT_ERR_BAD_SHAPE;
  const int64_t n = static_cast<int64_t>(heads + 2 * kv_heads) * head_dim;
  if (tokens > 16 || dim % 128 || dim > parrot::decode_qkv_max_dim() || head_dim % 2 || n % 16)
    return PARROT_ERR_UNSUPPORTED;
  if ((x && !aligned16(x)) || !aligned16(qkv_weight)) return PARROT_ERR_ALIGNMENT;
  parrot::DecodeQkvArgs a{};
  if (!x) {
    if (int rc = make_decode_mix(sources, n_sources, query, score_norm_weight, score_eps,
                                 attention_norm_weight, norm_eps, a.mix))
      return rc;
  }
  a.x = static_cast<const uint16_t*>(x);
  a.tokens = tokens;
  a.dim = dim;
  a.w = static_cast<const uint16_t*>(qkv_weight);
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.head_dim = head_dim;
  a.cos_t = cos_table;
  a.sin_t = sin_table;
  a.max_positions = max_positions;
  a.position = position;
  a.q = static_cast<uint16_t*>(q);
  a.k = static_cast<uint16_t*>(k);
  a.v = static_cast<uint16_t*>(v);
  return status(parrot::launch_decode_qkv(a, as_stream(stream)));
}

int parrot_decode_qkv_embed_bf16(const int64_t* token_ids, const void* embedding, int32_t vocab,
                                 void* embedded, const void* query, const void* score_norm_weight,
                                 float score_eps, const void* attention_norm_weight,
                                 float norm_eps, int32_t tokens, int32_t dim,
                                 const void* qkv_weight, int32_t heads, int32_t kv_heads,
                                 int32_t head_dim, const float* cos_table,
                                 const float* sin_table, int32_t max_positions,
                                 const int32_t* position, void* q, void* k, void* v,
                                 void* stream) {
  if (!token_ids || !embedding || !embedded) return PARROT_ERR_NULL_POINTER;
  if (vocab <= 0) return PARROT_ERR_BAD_SHAPE;
  if (!aligned16(embedding) || !aligned16(embedded)) return PARROT_ERR_ALIGNMENT;
  // The single depth source is the gathered row (its slot names the output
  // buffer, which the launch writes and the later layers read).
  const void* sources[1] = {embedded};
  if (!qkv_weight || !cos_table || !sin_table || !position || !q || !k || !v)
    return PARROT_ERR_NULL_POINTER;
  if (tokens < 0 || dim <= 0 || heads <= 0 || kv_heads <= 0 || head_dim <= 0 ||
      max_positions <= 0)
    return PARROT_ERR_BAD_SHAPE;
  const int64_t n = static_cast<int64_t>(heads + 2 * kv_heads) * head_dim;
  if (tokens > 16 || dim % 128 || dim > parrot::decode_qkv_max_dim() || head_dim % 2 || n % 16)
    return PARROT_ERR_UNSUPPORTED;
  if (!aligned16(qkv_weight)) return PARROT_ERR_ALIGNMENT;
  parrot::DecodeQkvArgs a{};
  if (int rc = make_decode_mix(sources, 1, query, score_norm_weight, score_eps,
                               attention_norm_weight, norm_eps, a.mix))
    return rc;
  a.tokens = tokens;
  a.dim = dim;
  a.w = static_cast<const uint16_t*>(qkv_weight);
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.head_dim = head_dim;
  a.cos_t = cos_table;
  a.sin_t = sin_table;
  a.max_positions = max_positions;
  a.position = position;
  a.q = static_cast<uint16_t*>(q);
  a.k = static_cast<uint16_t*>(k);
  a.v = static_cast<uint16_t*>(v);
  a.gather_ids = token_ids;
  a.gather_table = static_cast<const uint16_t*>(embedding);
  a.gather_rows = vocab;
  a.gather_out = static_cast<uint16_t*>(embedded);
  return status(parrot::launch_decode_qkv(a, as_stream(stream)));
}

// Shapes of the MLA decode projections: up to 16 tokens, K a multiple of
// 128 up to 2048, row counts multiples of 16, the staged input within 64 KB.
static int check_mla_decode(int32_t tokens, int32_t k, int elem_bytes) {
  if (tokens < 0 || k <= 0) return PARROT_ERR_BAD_SHAPE;
  if (tokens > 16 || k % 128 || k > 2048) return PARROT_ERR_UNSUPPORTED;
  if (parrot::mla_decode_lds_bytes(tokens, k, elem_bytes) > 65536) return PARROT_ERR_UNSUPPORTED;
  return PARROT_OK;
}

int parrot_mla_decode_in_bf16(const void* x, const void* const* sources, int32_t n_sources,
                              const void* query, const void* score_norm_weight, float score_eps,
                              const void* attention_norm_weight, float norm_eps,
                              int32_t tokens, int32_t dim, const void* absorbed_query,
                              int32_t query_rows, const void* kv_down, int32_t latent_dim,
                              float* q_latent, void* latent, void* stream) {
  if ((!x && !sources) || !absorbed_query || !kv_down || !q_latent || !latent)
    return PARROT_ERR_NULL_POINTER;
  if (int rc = check_mla_decode(tokens, dim, 2)) return rc;
  if (query_rows <= 0 || latent_dim <= 0) return PARROT_ERR_BAD_SHAPE;
  if (query_rows % 16 || latent_dim % 16) return PARROT_ERR_UNSUPPORTED;
  if ((x && !aligned16(x)) || !aligned16(absorbed_query) || !aligned16(kv_down))
    return PARROT_ERR_ALIGNMENT;
  parrot::DecodeMix mix{};
  if (!x) {
    if (int rc = make_decode_mix(sources, n_sources, query, score_norm_weight, score_eps,
                                 attention_norm_weight, norm_eps, mix))
      return rc;
    if (dim > 1024) return PARROT_ERR_UNSUPPORTED;
  }
  return status(parrot::launch_mla_decode_in(
      static_cast<const uint16_t*>(x), x ? nullptr : &mix, tokens, dim,
      static_cast<const uint16_t*>(absorbed_query), query_rows,
      static_cast<const uint16_t*>(kv_down), latent_dim, q_latent,
      static_cast<uint16_t*>(latent), as_stream(stream)));
}

int parrot_decode_linear_bf16(const void* x, int32_t tokens, int32_t k, const void* weight,
                              int32_t n, const void* addend, void* out, void* stream) {
  if (!x || !weight || !out) return PARROT_ERR_NULL_POINTER;
  if (int rc = check_mla_decode(tokens, k, 2)) return rc;
  if (n <= 0) return PARROT_ERR_BAD_SHAPE;
  if (n % 16) return PARROT_ERR_UNSUPPORTED;
  if (!aligned16(x) || !aligned16(weight)) return PARROT_ERR_ALIGNMENT;
  return status(parrot::launch_decode_linear(
      static_cast<const uint16_t*>(x), tokens, k, static_cast<const uint16_t*>(weight), n,
      static_cast<const uint16_t*>(addend), static_cast<uint16_t*>(out), as_stream(stream)));
}

int parrot_mla_decode_out_bf16(const float* context, int32_t tokens, int32_t width,
                               const void* absorbed_output, int32_t dim, const void* addend,
                               void* out, void* stream) {
  if (!context || !absorbed_output || !out) return PARROT_ERR_NULL_POINTER;
  if (int rc = check_mla_decode(tokens, width, 4)) return rc;
  if (dim <= 0) return PARROT_ERR_BAD_SHAPE;
  if (dim % 16) return PARROT_ERR_UNSUPPORTED;
  if (!aligned16(context) || !aligned16(absorbed_output)) return PARROT_ERR_ALIGNMENT;
  return status(parrot::launch_mla_decode_out(
      context, tokens, width, static_cast<const uint16_t*>(absorbed_output), dim,
      static_cast<const uint16_t*>(addend), static_cast<uint16_t*>(out), as_stream(stream)));
}

size_t parrot_route_workspace_bytes(int64_t tokens, int32_t experts) {
  if (tokens < 0 || experts <= 0) return 0;
  return route_ws_bytes(tokens, experts);
}

static int route_common(const void* x, const void* router_weight, const float* logits,
                        const float* logit_bias, int64_t tokens, int32_t dim, int32_t experts,
                        int32_t capacity, float* out_logits, float* out_probs,
                        float* out_weights, int64_t* out_indices, int32_t* out_positions,
                        int32_t* out_counts, int32_t* out_offsets, int32_t* out_perm,
                        int32_t* out_overflow, void* workspace, size_t workspace_bytes,
                        void* stream) {
  if (int rc = check_route_shape(tokens, experts, capacity)) return rc;
  if (!out_weights || !out_indices) return PARROT_ERR_NULL_POINTER;
  if (int rc = check_group_outputs(out_positions, out_counts, out_offsets, out_perm, out_overflow))
    return rc;
  if (!workspace || workspace_bytes < route_ws_bytes(tokens, experts)) return PARROT_ERR_WORKSPACE;
  int32_t* block_counts = static_cast<int32_t*>(workspace);
  const hipStream_t s = as_stream(stream);
  hipError_t e = parrot::launch_route(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(router_weight), logits,
      logit_bias, tokens, dim, experts, out_logits, out_probs, out_weights, out_indices,
      out_positions, block_counts, nullptr, s);
  if (e != hipSuccess) return status(e);
  return status(parrot::launch_group(out_indices, tokens, experts, capacity, block_counts,
                                     route_chunk_totals(workspace, tokens, experts),
                                     out_positions, out_counts, out_offsets, out_perm,
                                     out_overflow, s));
}

int parrot_route_bf16(const void* x, const void* router_weight, const float* logit_bias,
                      int64_t tokens, int32_t dim, int32_t experts, int32_t capacity,
                      float* out_logits, float* out_probs, float* out_weights,
                      int64_t* out_indices, int32_t* out_positions, int32_t* out_counts,
                      int32_t* out_offsets, int32_t* out_perm, int32_t* out_overflow,
                      void* workspace, size_t workspace_bytes, void* stream) {
  if (!x || !router_weight) return PARROT_ERR_NULL_POINTER;
  if (dim <= 0 || dim % 32) return PARROT_ERR_UNSUPPORTED;
  if (!aligned16(x) || !aligned16(router_weight)) return PARROT_ERR_ALIGNMENT;
  return route_common(x, router_weight, nullptr, logit_bias, tokens, dim, experts, capacity,
                      out_logits, out_probs, out_weights, out_indices, out_positions,
                      out_counts, out_offsets, out_perm, out_overflow, workspace,
                      workspace_bytes, stream);
}

static int route_top2_common(const void* x, const void* router_weight, const float* logit_bias,
                             int64_t tokens, int32_t dim, int32_t experts, float* out_weights,
                             int64_t* out_indices, uint8_t* out_blocks, void* stream) {
  if (!x || !router_weight || !out_weights || !out_indices) return PARROT_ERR_NULL_POINTER;
  if (tokens < 0 || tokens > (int64_t{1} << 29)) return PARROT_ERR_BAD_SHAPE;
  if (experts < 2 || experts > kMaxExperts) return PARROT_ERR_UNSUPPORTED;
  if (dim <= 0 || dim % 32) return PARROT_ERR_UNSUPPORTED;
  if (!aligned16(x) || !aligned16(router_weight)) return PARROT_ERR_ALIGNMENT;
  return status(parrot::launch_route(static_cast<const uint16_t*>(x),
                                     static_cast<const uint16_t*>(router_weight), nullptr,
                                     logit_bias, tokens, dim, experts, nullptr, nullptr,
                                     out_weights, out_indices, nullptr, nullptr, out_blocks,
                                     as_stream(stream)));
}

int parrot_route_top2_bf16(const void* x, const void* router_weight, const float* logit_bias,
                           int64_t tokens, int32_t dim, int32_t experts, float* out_weights,
                           int64_t* out_indices, void* stream) {
  return route_top2_common(x, router_weight, logit_bias, tokens, dim, experts, out_weights,
                           out_indices, nullptr, stream);
}

int parrot_route_top2_blocks_bf16(const void* x, const void* router_weight,
                                  const float* logit_bias, int64_t tokens, int32_t dim,
                                  int32_t experts, float* out_weights, int64_t* out_indices,
                                  void* out_blocks, void* stream) {
  if (!out_blocks) return PARROT_ERR_NULL_POINTER;
  if (tokens > 0 && !parrot::route_block_rows_supported(tokens)) return PARROT_ERR_UNSUPPORTED;
  if (!aligned16(out_blocks)) return PARROT_ERR_ALIGNMENT;
  return route_top2_common(x, router_weight, logit_bias, tokens, dim, experts, out_weights,
                           out_indices, static_cast<uint8_t*>(out_blocks), stream);
}

int parrot_route_from_logits_f32(const float* logits, const float* logit_bias, int64_t tokens,
                                 int32_t experts, int32_t capacity, float* out_probs,
                                 float* out_weights, int64_t* out_indices,
                                 int32_t* out_positions, int32_t* out_counts,
                                 int32_t* out_offsets, int32_t* out_perm,
                                 int32_t* out_overflow, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  if (!logits) return PARROT_ERR_NULL_POINTER;
  return route_common(nullptr, nullptr, logits, logit_bias, tokens, 0, experts, capacity,
                      nullptr, out_probs, out_weights, out_indices, out_positions, out_counts,
                      out_offsets, out_perm, out_overflow, workspace, workspace_bytes, stream);
}

int parrot_group_indices(const int64_t* indices, int64_t tokens, int32_t experts,
                         int32_t capacity, int32_t* out_positions, int32_t* out_counts,
                         int32_t* out_offsets, int32_t* out_perm, int32_t* out_overflow,
                         void* workspace, size_t workspace_bytes, void* stream) {
  if (!indices) return PARROT_ERR_NULL_POINTER;
  if (int rc = check_route_shape(tokens, experts, capacity)) return rc;
  if (int rc = check_group_outputs(out_positions, out_counts, out_offsets, out_perm, out_overflow))
    return rc;
  if (!workspace || workspace_bytes < route_ws_bytes(tokens, experts)) return PARROT_ERR_WORKSPACE;
  int32_t* block_counts = static_cast<int32_t*>(workspace);
  const hipStream_t s = as_stream(stream);
  hipError_t e = parrot::launch_rank_indices(indices, tokens, experts, out_positions,
                                             block_counts, s);
  if (e != hipSuccess) return status(e);
  return status(parrot::launch_group(indices, tokens, experts, capacity, block_counts,
                                     route_chunk_totals(workspace, tokens, experts),
                                     out_positions, out_counts, out_offsets, out_perm,
                                     out_overflow, s));
}

size_t parrot_experts_workspace_bytes(int64_t tokens, int32_t dim, int32_t hidden_dim,
                                      int32_t shared_dim) {
  if (tokens < 0 || dim <= 0 || hidden_dim <= 0 || shared_dim <= 0) return 0;
  return experts_ws(nullptr, tokens, dim, hidden_dim, shared_dim).bytes;
}

}  // extern "C"

namespace {

struct ExpertsCall {
  parrot::GroupMap map;
  parrot::ExpertWeights w;
  ExpertsWorkspace ws;
};

// Validation shared by the expert entry points; weights / map pointers a
// stage does not read may be NULL (need_* = false).
int check_experts_shape(int64_t tokens, int32_t dim, int32_t experts, int32_t hidden_dim,
                        int32_t shared_dim, int32_t capacity, void* workspace,
                        size_t workspace_bytes, ExpertsWorkspace* ws) {
  if (int rc = check_route_shape(tokens, experts, capacity)) return rc;
  if (dim <= 0 || hidden_dim <= 0 || shared_dim <= 0) return PARROT_ERR_BAD_SHAPE;
  if (dim % 64 || hidden_dim % 64 || shared_dim % 64) return PARROT_ERR_UNSUPPORTED;
  *ws = experts_ws(workspace, tokens, dim, hidden_dim, shared_dim);
  if (!workspace || workspace_bytes < ws->bytes) return PARROT_ERR_WORKSPACE;
  if (!aligned16(workspace)) return PARROT_ERR_ALIGNMENT;
  return PARROT_OK;
}

int check_experts(int64_t tokens, int32_t dim, int32_t experts, int32_t hidden_dim,
                  int32_t shared_dim, int32_t capacity, const int32_t* counts,
                  const int32_t* offsets, const int32_t* perm, const int32_t* overflow,
                  void* workspace, size_t workspace_bytes, ExpertsWorkspace* ws) {
  if (!counts || !offsets || !perm || !overflow) return PARROT_ERR_NULL_POINTER;
  if (int rc = check_route_shape(tokens, experts, capacity)) return rc;
  if (dim <= 0 || hidden_dim <= 0 || shared_dim <= 0) return PARROT_ERR_BAD_SHAPE;
  if (dim % 64 || hidden_dim % 64 || shared_dim % 64) return PARROT_ERR_UNSUPPORTED;
  *ws = experts_ws(workspace, tokens, dim, hidden_dim, shared_dim);
  if (!workspace || workspace_bytes < ws->bytes) return PARROT_ERR_WORKSPACE;
  if (!aligned16(workspace)) return PARROT_ERR_ALIGNMENT;
  return PARROT_OK;
}

}  // namespace

extern "C" {

int parrot_experts_gate_up_bf16(const void* x, int64_t tokens, int32_t dim, int32_t experts,
                                int32_t hidden_dim, int32_t shared_dim, int32_t capacity,
                                const int32_t* counts, const int32_t* offsets,
                                const int32_t* perm, const int32_t* overflow,
                                const void* packed_gate_up, const void* shared_gate_up,
                                void* workspace, size_t workspace_bytes, void* stream) {
  if (!x || !packed_gate_up || !shared_gate_up) return PARROT_ERR_NULL_POINTER;
  ExpertsWorkspace ws;
  if (int rc = check_experts(tokens, dim, experts, hidden_dim, shared_dim, capacity, counts,
                             offsets, perm, overflow, workspace, workspace_bytes, &ws))
    return rc;
  if (!aligned16(x) || !aligned16(packed_gate_up) || !aligned16(shared_gate_up))
    return PARROT_ERR_ALIGNMENT;
  parrot::GroupMap map{counts, offsets, perm, overflow, nullptr};
  parrot::ExpertWeights w{static_cast<const uint16_t*>(packed_gate_up), nullptr,
                          static_cast<const uint16_t*>(shared_gate_up), nullptr};
  return status(parrot::launch_expert_gemm(1, static_cast<const uint16_t*>(x), tokens, dim,
                                           experts, hidden_dim, shared_dim, capacity, map, w,
                                           ws.hidden, ws.y_routed, ws.y_shared,
                                           as_stream(stream)));
}

int parrot_experts_group_in_kernel(int64_t tokens, int32_t dim, int32_t experts,
                                   int32_t hidden_dim, int32_t shared_dim) {
  if (experts < 2 || experts > kMaxExperts || dim <= 0 || hidden_dim <= 0 || shared_dim <= 0)
    return 0;
  return static_cast<int>(
      parrot::experts_group_in_kernel(tokens, dim, experts, hidden_dim, shared_dim));
}

// The gate/up launch that groups in-kernel, from the top-2 indices
// (kGroupFromIds shapes) or from the route's block table (kGroupFromIds or
// kGroupFromBlocks shapes).
static int gate_up_grouping_common(const void* x, int64_t tokens, int32_t dim, int32_t experts,
                                   int32_t hidden_dim, int32_t shared_dim, int32_t capacity,
                                   const int64_t* indices, const uint8_t* blocks,
                                   int32_t* out_counts, int32_t* out_offsets,
                                   int32_t* out_sorted, const void* packed_gate_up,
                                   const void* shared_gate_up, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  if (!x || (!indices && !blocks) || !out_counts || !out_offsets || !out_sorted ||
      !packed_gate_up || !shared_gate_up)
    return PARROT_ERR_NULL_POINTER;
  ExpertsWorkspace ws;
  if (int rc = check_experts_shape(tokens, dim, experts, hidden_dim, shared_dim, capacity,
                                   workspace, workspace_bytes, &ws))
    return rc;
  if (tokens == 0) return PARROT_OK;
  const parrot::GroupInKernel mode =
      parrot::experts_group_in_kernel(tokens, dim, experts, hidden_dim, shared_dim);
  if (mode == parrot::kGroupNone || (indices && mode != parrot::kGroupFromIds))
    return PARROT_ERR_UNSUPPORTED;
  if (!aligned16(x) || !aligned16(packed_gate_up) || !aligned16(shared_gate_up) ||
      (blocks && !aligned16(blocks)))
    return PARROT_ERR_ALIGNMENT;
  parrot::GroupMap map{nullptr, nullptr, nullptr, nullptr, nullptr};
  map.indices = indices;
  map.route_blocks = blocks;
  map.counts_out = out_counts;
  map.offsets_out = out_offsets;
  map.sorted_out = out_sorted;
  parrot::ExpertWeights w{static_cast<const uint16_t*>(packed_gate_up), nullptr,
                          static_cast<const uint16_t*>(shared_gate_up), nullptr};
  return status(parrot::launch_expert_gemm(1, static_cast<const uint16_t*>(x), tokens, dim,
                                           experts, hidden_dim, shared_dim, capacity, map, w,
                                           ws.hidden, ws.y_routed, ws.y_shared,
                                           as_stream(stream)));
}

int parrot_experts_gate_up_grouping_bf16(const void* x, int64_t tokens, int32_t dim,
                                         int32_t experts, int32_t hidden_dim,
                                         int32_t shared_dim, int32_t capacity,
                                         const int64_t* indices, int32_t* out_counts,
                                         int32_t* out_offsets, int32_t* out_sorted,
                                         const void* packed_gate_up, const void* shared_gate_up,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  if (!indices) return PARROT_ERR_NULL_POINTER;
  return gate_up_grouping_common(x, tokens, dim, experts, hidden_dim, shared_dim, capacity,
                                 indices, nullptr, out_counts, out_offsets, out_sorted,
                                 packed_gate_up, shared_gate_up, workspace, workspace_bytes,
                                 stream);
}

int parrot_experts_gate_up_grouping_blocks_bf16(
    const void* x, int64_t tokens, int32_t dim, int32_t experts, int32_t hidden_dim,
    int32_t shared_dim, int32_t capacity, const void* route_blocks, int32_t* out_counts,
    int32_t* out_offsets, int32_t* out_sorted, const void* packed_gate_up,
    const void* shared_gate_up, void* workspace, size_t workspace_bytes, void* stream) {
  if (!route_blocks) return PARROT_ERR_NULL_POINTER;
  return gate_up_grouping_common(x, tokens, dim, experts, hidden_dim, shared_dim, capacity,
                                 nullptr, static_cast<const uint8_t*>(route_blocks),
                                 out_counts, out_offsets, out_sorted, packed_gate_up,
                                 shared_gate_up, workspace, workspace_bytes, stream);
}

int parrot_experts_down_sorted_bf16(int64_t tokens, int32_t dim, int32_t experts,
                                    int32_t hidden_dim, int32_t shared_dim, int32_t capacity,
                                    const int32_t* counts, const int32_t* offsets,
                                    const int32_t* sorted, const float* route_weights,
                                    const void* down, const void* shared_down, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  if (!counts || !offsets || !sorted || !route_weights || !down || !shared_down)
    return PARROT_ERR_NULL_POINTER;
  ExpertsWorkspace ws;
  if (int rc = check_experts_shape(tokens, dim, experts, hidden_dim, shared_dim, capacity,
                                   workspace, workspace_bytes, &ws))
    return rc;
  if (!aligned16(down) || !aligned16(shared_down)) return PARROT_ERR_ALIGNMENT;
  parrot::GroupMap map{counts, offsets, nullptr, nullptr, route_weights};
  map.sorted = sorted;
  parrot::ExpertWeights w{nullptr, static_cast<const uint16_t*>(down), nullptr,
                          static_cast<const uint16_t*>(shared_down)};
  return status(parrot::launch_expert_gemm(2, nullptr, tokens, dim, experts, hidden_dim,
                                           shared_dim, capacity, map, w, ws.hidden, ws.y_routed,
                                           ws.y_shared, as_stream(stream)));
}

int parrot_experts_down_bf16(int64_t tokens, int32_t dim, int32_t experts, int32_t hidden_dim,
                             int32_t shared_dim, int32_t capacity, const int32_t* counts,
                             const int32_t* offsets, const int32_t* perm,
                             const int32_t* overflow, const float* route_weights,
                             const void* down, const void* shared_down, void* workspace,
                             size_t workspace_bytes, void* stream) {
  if (!route_weights || !down || !shared_down) return PARROT_ERR_NULL_POINTER;
  ExpertsWorkspace ws;
  if (int rc = check_experts(tokens, dim, experts, hidden_dim, shared_dim, capacity, counts,
                             offsets, perm, overflow, workspace, workspace_bytes, &ws))
    return rc;
  if (!aligned16(down) || !aligned16(shared_down)) return PARROT_ERR_ALIGNMENT;
  parrot::GroupMap map{counts, offsets, perm, overflow, route_weights};
  parrot::ExpertWeights w{nullptr, static_cast<const uint16_t*>(down), nullptr,
                          static_cast<const uint16_t*>(shared_down)};
  return status(parrot::launch_expert_gemm(2, nullptr, tokens, dim, experts, hidden_dim,
                                           shared_dim, capacity, map, w, ws.hidden, ws.y_routed,
                                           ws.y_shared, as_stream(stream)));
}

int parrot_experts_combine_bf16(int64_t tokens, int32_t dim, int32_t hidden_dim,
                                int32_t shared_dim, const void* addend, void* out,
                                void* workspace, size_t workspace_bytes, void* stream) {
  if (!out) return PARROT_ERR_NULL_POINTER;
  if (tokens < 0 || dim <= 0 || dim % 4 || hidden_dim <= 0 || shared_dim <= 0)
    return PARROT_ERR_BAD_SHAPE;
  const ExpertsWorkspace ws = experts_ws(workspace, tokens, dim, hidden_dim, shared_dim);
  if (!workspace || workspace_bytes < ws.bytes) return PARROT_ERR_WORKSPACE;
  if (!aligned16(workspace) || !aligned16(out) || (addend && !aligned16(addend)))
    return PARROT_ERR_ALIGNMENT;
  return status(parrot::launch_combine(ws.y_routed, ws.y_shared,
                                       static_cast<const uint16_t*>(addend), tokens, dim,
                                       static_cast<uint16_t*>(out), as_stream(stream)));
}

int parrot_experts_combine_depth_mix_bf16(
    int64_t tokens, int32_t dim, int32_t hidden_dim, int32_t shared_dim, const void* addend,
    void* out, void* workspace, size_t workspace_bytes, const void* const* sources,
    int32_t n_sources, const void* query, const void* score_norm_weight, float score_eps,
    const void* out_norm_weight, float out_eps, void* out_mix, void* out_norm, void* stream) {
  if (!out || !query || !score_norm_weight) return PARROT_ERR_NULL_POINTER;
  if (!out_mix && !out_norm) return PARROT_ERR_NULL_POINTER;
  if (out_norm && !out_norm_weight) return PARROT_ERR_NULL_POINTER;
  if (n_sources < 1 || n_sources > kMaxDepthSources) return PARROT_ERR_UNSUPPORTED;
  if (n_sources > 1 && !sources) return PARROT_ERR_NULL_POINTER;
  if (tokens < 0 || dim <= 0 || dim % 4 || hidden_dim <= 0 || shared_dim <= 0)
    return PARROT_ERR_BAD_SHAPE;
  if (dim > 2048) return PARROT_ERR_UNSUPPORTED;
  const ExpertsWorkspace ws = experts_ws(workspace, tokens, dim, hidden_dim, shared_dim);
  if (!workspace || workspace_bytes < ws.bytes) return PARROT_ERR_WORKSPACE;
  parrot::DepthSources srcs{};
  uintptr_t bits = reinterpret_cast<uintptr_t>(query) |
                   reinterpret_cast<uintptr_t>(score_norm_weight) |
                   reinterpret_cast<uintptr_t>(out_norm_weight) |
                   reinterpret_cast<uintptr_t>(out_mix) | reinterpret_cast<uintptr_t>(out_norm);
  for (int s = 0; s < kMaxDepthSources; ++s) {
    const void* p = s < n_sources - 1 ? sources[s] : out;  // unread slots: any valid row
    if (!p) return PARROT_ERR_NULL_POINTER;
    bits |= reinterpret_cast<uintptr_t>(p);
    srcs.src[s] = static_cast<const uint16_t*>(p);
  }
  if (bits & 7u) return PARROT_ERR_ALIGNMENT;
  if (!aligned16(workspace) || !aligned16(out) || (addend && !aligned16(addend)))
    return PARROT_ERR_ALIGNMENT;
  const parrot::CombineSource comb{ws.y_routed, ws.y_shared,
                                   static_cast<const uint16_t*>(addend),
                                   static_cast<uint16_t*>(out)};
  return status(parrot::launch_depth_mix(
      srcs, n_sources, static_cast<const uint16_t*>(query),
      static_cast<const uint16_t*>(score_norm_weight), score_eps,
      static_cast<const uint16_t*>(out_norm_weight), out_eps, tokens, dim,
      static_cast<uint16_t*>(out_mix), static_cast<uint16_t*>(out_norm), &comb, nullptr,
      as_stream(stream)));
}

size_t parrot_decode_moe_workspace_bytes(int64_t tokens, int32_t hidden_dim,
                                         int32_t shared_dim) {
  if (tokens < 0 || hidden_dim <= 0 || shared_dim <= 0) return 0;
  const size_t hstride = static_cast<size_t>(hidden_dim > shared_dim ? hidden_dim : shared_dim);
  return round_up(3 * static_cast<size_t>(tokens) * hstride * sizeof(uint16_t));
}

// Shared checks and launch of the two decode MoE entry points.
static int decode_moe_entry(const void* x, const parrot::DecodeMix* mix, int64_t tokens,
                            int32_t dim, int32_t experts, int32_t hidden_dim,
                            int32_t shared_dim, const void* router_weight,
                            const float* logit_bias, const void* packed_gate_up,
                            const void* packed_down, const void* shared_gate_up,
                            const void* shared_down, const void* addend, void* out,
                            int64_t* out_indices, float* out_weights, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if ((!x && !mix) || !router_weight || !packed_gate_up || !packed_down || !shared_gate_up ||
      !shared_down || !out || !out_indices || !out_weights)
    return PARROT_ERR_NULL_POINTER;
  if (tokens < 0 || dim <= 0 || hidden_dim <= 0 || shared_dim <= 0) return PARROT_ERR_BAD_SHAPE;
  if (tokens > parrot::decode_moe_max_tokens() || experts < 2 || experts > parrot::kMaxExperts ||
      dim % 64 || dim > 2048 || hidden_dim % 64 || shared_dim % 64)
    return PARROT_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < parrot_decode_moe_workspace_bytes(tokens, hidden_dim,
                                                                        shared_dim))
    return PARROT_ERR_WORKSPACE;
  if ((x && !aligned16(x)) || !aligned16(router_weight) || !aligned16(packed_gate_up) ||
      !aligned16(packed_down) || !aligned16(shared_gate_up) || !aligned16(shared_down) ||
      !aligned16(workspace))
    return PARROT_ERR_ALIGNMENT;
  parrot::ExpertWeights w{static_cast<const uint16_t*>(packed_gate_up),
                          static_cast<const uint16_t*>(packed_down),
                          static_cast<const uint16_t*>(shared_gate_up),
                          static_cast<const uint16_t*>(shared_down)};
  return status(parrot::launch_decode_moe(
      static_cast<const uint16_t*>(x), mix, static_cast<int>(tokens), dim, experts, hidden_dim,
      shared_dim, static_cast<const uint16_t*>(router_weight), logit_bias, w,
      static_cast<const uint16_t*>(addend), static_cast<uint16_t*>(out), out_indices,
      out_weights, static_cast<uint16_t*>(workspace), as_stream(stream)));
}

int parrot_decode_moe_bf16(const void* x, int64_t tokens, int32_t dim, int32_t experts,
                           int32_t hidden_dim, int32_t shared_dim, const void* router_weight,
                           const float* logit_bias, const void* packed_gate_up,
                           const void* packed_down, const void* shared_gate_up,
                           const void* shared_down, const void* addend, void* out,
                           int64_t* out_indices, float* out_weights, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (!x) return PARROT_ERR_NULL_POINTER;
  return decode_moe_entry(x, nullptr, tokens, dim, experts, hidden_dim, shared_dim,
                          router_weight, logit_bias, packed_gate_up, packed_down,
                          shared_gate_up, shared_down, addend, out, out_indices, out_weights,
                          workspace, workspace_bytes, stream);
}

int parrot_depth_mix_decode_moe_bf16(
    const void* const* sources, int32_t n_sources, const void* query,
    const void* score_norm_weight, float score_eps, const void* moe_norm_weight,
    float norm_eps, int64_t tokens, int32_t dim, int32_t experts, int32_t hidden_dim,
    int32_t shared_dim, const void* router_weight, const float* logit_bias,
    const void* packed_gate_up, const void* packed_down, const void* shared_gate_up,
    const void* shared_down, const void* addend, void* out, int64_t* out_indices,
    float* out_weights, void* workspace, size_t workspace_bytes, void* stream) {
  parrot::DecodeMix mix{};
  if (int rc = make_decode_mix(sources, n_sources, query, score_norm_weight, score_eps,
                               moe_norm_weight, norm_eps, mix))
    return rc;
  if (dim > 1024) return PARROT_ERR_UNSUPPORTED;
  return decode_moe_entry(nullptr, &mix, tokens, dim, experts, hidden_dim, shared_dim,
                          router_weight, logit_bias, packed_gate_up, packed_down,
                          shared_gate_up, shared_down, addend, out, out_indices, out_weights,
                          workspace, workspace_bytes, stream);
}

int parrot_depth_mix_decode_moe_pending_bf16(
    const void* const* sources, int32_t n_sources, const void* query,
    const void* score_norm_weight, float score_eps, const void* moe_norm_weight,
    float norm_eps, const float* contributions, int32_t lanes, const void* base,
    void* resolved, int64_t tokens, int32_t dim, int32_t experts, int32_t hidden_dim,
    int32_t shared_dim, const void* router_weight, const float* logit_bias,
    const void* packed_gate_up, const void* packed_down, const void* shared_gate_up,
    const void* shared_down, const void* addend, void* out, int64_t* out_indices,
    float* out_weights, void* workspace, size_t workspace_bytes, void* stream) {
  parrot::DecodeMix mix{};
  if (int rc = make_decode_mix(sources, n_sources, query, score_norm_weight, score_eps,
                               moe_norm_weight, norm_eps, mix))
    return rc;
  if (!contributions || !resolved) return PARROT_ERR_NULL_POINTER;
  if (lanes < 1 || lanes > parrot::kMaxPendingLanes || dim > 1024 || dim % 4)
    return PARROT_ERR_UNSUPPORTED;
  if (!aligned16(contributions) || reinterpret_cast<uintptr_t>(resolved) % 8 ||
      reinterpret_cast<uintptr_t>(base) % 8)
    return PARROT_ERR_ALIGNMENT;
  mix.pend = contributions;
  mix.pend_lanes = lanes;
  mix.pend_base = static_cast<const uint16_t*>(base);
  mix.pend_out = static_cast<uint16_t*>(resolved);
  return decode_moe_entry(nullptr, &mix, tokens, dim, experts, hidden_dim, shared_dim,
                          router_weight, logit_bias, packed_gate_up, packed_down,
                          shared_gate_up, shared_down, addend, out, out_indices, out_weights,
                          workspace, workspace_bytes, stream);
}

size_t parrot_vocab_argmax_workspace_bytes(int64_t rows, int32_t vocab) {
  if (rows < 0 || vocab <= 0) return 0;
  const size_t n = static_cast<size_t>(rows) * parrot::vocab_argmax_groups(vocab);
  return round_up(n * sizeof(float)) + round_up(n * sizeof(int32_t));
}

int parrot_vocab_argmax_bf16(const void* hidden, int64_t rows, int32_t dim, const void* weight,
                             int32_t vocab, int64_t* out_tokens, int32_t* advance_position,
                             void* workspace, size_t workspace_bytes, void* stream) {
  if (!hidden || !weight || !out_tokens) return PARROT_ERR_NULL_POINTER;
  if (rows < 0 || dim <= 0 || vocab <= 0) return PARROT_ERR_BAD_SHAPE;
  if (rows > parrot::vocab_argmax_max_rows() || dim % 8 || dim > 2048)
    return PARROT_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < parrot_vocab_argmax_workspace_bytes(rows, vocab))
    return PARROT_ERR_WORKSPACE;
  if (!aligned16(hidden) || !aligned16(weight) || !aligned16(workspace))
    return PARROT_ERR_ALIGNMENT;
  const size_t n = static_cast<size_t>(rows) * parrot::vocab_argmax_groups(vocab);
  float* part_v = static_cast<float*>(workspace);
  int32_t* part_i = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) +
                                               round_up(n * sizeof(float)));
  return status(parrot::launch_vocab_argmax(
      static_cast<const uint16_t*>(hidden), static_cast<int>(rows), dim,
      static_cast<const uint16_t*>(weight), vocab, part_v, part_i, out_tokens, advance_position,
      as_stream(stream)));
}

int parrot_causal_attention_bf16(const void* q, const void* k, const void* vt,
                                 const int64_t* q_strides, const int64_t* k_strides,
                                 const int64_t* vt_strides, int64_t batch, int32_t seq,
                                 int32_t heads, int32_t kv_heads, int32_t head_dim,
                                 int32_t window, float scale, void* out, void* stream) {
  if (!q || !k || !vt || !q_strides || !k_strides || !vt_strides || !out)
    return PARROT_ERR_NULL_POINTER;
  if (batch < 0 || seq < 0 || heads <= 0 || kv_heads <= 0 || head_dim <= 0 || window <= 0)
    return PARROT_ERR_BAD_SHAPE;
  if (heads % kv_heads || !parrot::attention_head_dim_supported(head_dim) ||
      batch > 65535 || heads > 65535)
    return PARROT_ERR_UNSUPPORTED;
  // V^T rows must hold roundup(seq, 32) keys (the kernel reads whole blocks).
  const int64_t padded = (static_cast<int64_t>(seq) + 31) / 32 * 32;
  if (vt_strides[2] < padded || vt_strides[1] < head_dim * vt_strides[2])
    return PARROT_ERR_BAD_SHAPE;
  // One kv head of K (seq rows) and of V^T (head_dim rows) is addressed with
  // 32-bit byte offsets.
  if (static_cast<int64_t>(seq) * k_strides[2] * 2 >= (int64_t{1} << 31) ||
      static_cast<int64_t>(head_dim) * vt_strides[2] * 2 >= (int64_t{1} << 31))
    return PARROT_ERR_UNSUPPORTED;
  for (int i = 0; i < 3; ++i)
    if (q_strides[i] % 8 || k_strides[i] % 8 || vt_strides[i] % 8 || q_strides[i] < 0 ||
        k_strides[i] < 0 || vt_strides[i] < 0)
      return PARROT_ERR_ALIGNMENT;
  if (!aligned16(q) || !aligned16(k) || !aligned16(vt)) return PARROT_ERR_ALIGNMENT;
  return status(parrot::launch_causal_attention(
      static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
      static_cast<const uint16_t*>(vt), q_strides, k_strides, vt_strides,
      static_cast<int>(batch), seq, heads, kv_heads, head_dim, window, scale,
      static_cast<uint16_t*>(out), as_stream(stream)));
}

int parrot_causal_attention_frag_bf16(const void* q, const int64_t* q_strides, const void* k_frag,
                                      const void* v_frag, int64_t batch, int32_t seq,
                                      int32_t heads, int32_t kv_heads, int32_t head_dim,
                                      int32_t window, float scale, void* out, void* stream) {
  if (!q || !q_strides || !k_frag || !v_frag || !out) return PARROT_ERR_NULL_POINTER;
  if (batch < 0 || seq < 0 || heads <= 0 || kv_heads <= 0 || head_dim <= 0 || window <= 0)
    return PARROT_ERR_BAD_SHAPE;
  if (heads % kv_heads || !parrot::attention_head_dim_supported(head_dim) ||
      batch > 65535 || heads > 65535)
    return PARROT_ERR_UNSUPPORTED;
  // One kv head's fragments are addressed with 32-bit byte offsets.
  const int64_t padded = (static_cast<int64_t>(seq) + 31) / 32 * 32;
  if (padded * head_dim * 2 >= (int64_t{1} << 31)) return PARROT_ERR_UNSUPPORTED;
  for (int i = 0; i < 3; ++i)
    if (q_strides[i] % 8 || q_strides[i] < 0) return PARROT_ERR_ALIGNMENT;
  if (!aligned16(q) || !aligned16(k_frag) || !aligned16(v_frag)) return PARROT_ERR_ALIGNMENT;
  return status(parrot::launch_causal_attention(
      static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k_frag),
      static_cast<const uint16_t*>(v_frag), q_strides, nullptr, nullptr,
      static_cast<int>(batch), seq, heads, kv_heads, head_dim, window, scale,
      static_cast<uint16_t*>(out), as_stream(stream)));
}

int parrot_causal_attention_frag_out_bf16(const void* q, const int64_t* q_strides,
                                          const void* k_frag, const void* v_frag, int64_t batch,
                                          int32_t seq, int32_t heads, int32_t kv_heads,
                                          int32_t head_dim, int32_t window, float scale,
                                          const void* out_weight_packed, int32_t dim,
                                          float* contributions, void* stream) {
  if (!q || !q_strides || !k_frag || !v_frag || !out_weight_packed || !contributions)
    return PARROT_ERR_NULL_POINTER;
  if (batch < 0 || seq < 0 || heads <= 0 || kv_heads <= 0 || head_dim <= 0 || window <= 0 ||
      dim <= 0)
    return PARROT_ERR_BAD_SHAPE;
  if (heads % kv_heads || !parrot::attention_head_dim_supported(head_dim) ||
      !parrot::attention_out_width_supported(dim) || batch > 65535 || heads > 65535)
    return PARROT_ERR_UNSUPPORTED;
  const int64_t padded = (static_cast<int64_t>(seq) + 31) / 32 * 32;
  if (padded * head_dim * 2 >= (int64_t{1} << 31) ||
      static_cast<int64_t>(heads) * head_dim * dim * 2 >= (int64_t{1} << 31))
    return PARROT_ERR_UNSUPPORTED;
  for (int i = 0; i < 3; ++i)
    if (q_strides[i] % 8 || q_strides[i] < 0) return PARROT_ERR_ALIGNMENT;
  if (!aligned16(q) || !aligned16(k_frag) || !aligned16(v_frag) ||
      !aligned16(out_weight_packed) || !aligned16(contributions))
    return PARROT_ERR_ALIGNMENT;
  return status(parrot::launch_causal_attention_out(
      static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k_frag),
      static_cast<const uint16_t*>(v_frag), q_strides, static_cast<int>(batch), seq, heads,
      kv_heads, head_dim, window, scale, static_cast<const uint16_t*>(out_weight_packed), dim,
      contributions, as_stream(stream)));
}

int parrot_proj_bf16(const void* x, int64_t rows, int32_t k, int64_t lda, const void* w_packed,
                     int32_t n, const void* addend, int64_t ld_addend, void* out, int64_t ldo,
                     void* stream) {
  if (!x || !w_packed || !out) return PARROT_ERR_NULL_POINTER;
  if (rows < 0 || k <= 0 || n <= 0 || lda < k || ldo < n || (addend && ld_addend < n))
    return PARROT_ERR_BAD_SHAPE;
  if (!parrot::proj_shape_supported(k, n) || rows > INT32_MAX) return PARROT_ERR_UNSUPPORTED;
  if (!aligned16(x) || !aligned16(w_packed) || lda % 8) return PARROT_ERR_ALIGNMENT;
  return status(parrot::launch_proj_store(
      static_cast<const uint16_t*>(x), static_cast<int>(rows), k, lda,
      static_cast<const uint16_t*>(w_packed), n, static_cast<const uint16_t*>(addend), ld_addend,
      static_cast<uint16_t*>(out), ldo, as_stream(stream)));
}

int parrot_proj_transposed_bf16(const void* x, int64_t batch, int32_t seq, int32_t k,
                                const void* w_packed, int32_t n, int32_t ld_keys, void* out,
                                void* stream) {
  if (!x || !w_packed || !out) return PARROT_ERR_NULL_POINTER;
  if (batch < 0 || seq < 0 || k <= 0 || n <= 0 || ld_keys < seq) return PARROT_ERR_BAD_SHAPE;
  if (!parrot::proj_shape_supported(k, n) || batch * seq > INT32_MAX)
    return PARROT_ERR_UNSUPPORTED;
  if (!aligned16(x) || !aligned16(w_packed) || (reinterpret_cast<uintptr_t>(out) & 7u) ||
      ld_keys % 4)
    return PARROT_ERR_ALIGNMENT;
  if (batch == 0 || seq == 0) return PARROT_OK;
  return status(parrot::launch_proj_transposed(
      static_cast<const uint16_t*>(x), static_cast<int>(batch * seq), seq, k,
      static_cast<const uint16_t*>(w_packed), n, ld_keys, static_cast<uint16_t*>(out),
      as_stream(stream)));
}

int parrot_proj_rope_qkv_bf16(const void* x, int64_t batch, int32_t seq, int32_t dim,
                              const void* w_packed, const float* cos_table,
                              const float* sin_table, int32_t start,
                              const int32_t* start_device, int32_t max_positions, int32_t heads,
                              int32_t kv_heads, int32_t head_dim, int32_t vt_keys, void* q,
                              void* k, void* v, void* stream) {
  if (!x || !w_packed || !cos_table || !sin_table || !q || !k || !v)
    return PARROT_ERR_NULL_POINTER;
  // The same shape rules as parrot_rope_qkv_bf16 (a device start on top of
  // `start` is clamped by the kernel).
  if (batch < 0 || seq < 0 || start < 0 || dim <= 0 || heads <= 0 || kv_heads <= 0 ||
      head_dim <= 0 || max_positions <= 0 || vt_keys < 0 || (vt_keys > 0 && vt_keys < seq) ||
      static_cast<int64_t>(start) + seq > max_positions)
    return PARROT_ERR_BAD_SHAPE;
  if (heads % kv_heads || head_dim % 4) return PARROT_ERR_UNSUPPORTED;
  const int64_t n = static_cast<int64_t>(heads + 2 * kv_heads) * head_dim;
  if (n > INT32_MAX || !parrot::proj_shape_supported(dim, static_cast<int>(n)) ||
      batch * seq > INT32_MAX)
    return PARROT_ERR_UNSUPPORTED;
  if (!aligned16(x) || !aligned16(w_packed) ||
      (vt_keys > 0 && ((reinterpret_cast<uintptr_t>(v) & 7u) || vt_keys % 4)))
    return PARROT_ERR_ALIGNMENT;
  if (batch == 0 || seq == 0) return PARROT_OK;
  return status(parrot::launch_proj_rope_qkv(
      static_cast<const uint16_t*>(x), static_cast<int>(batch * seq), seq, dim,
      static_cast<const uint16_t*>(w_packed), cos_table, sin_table, start, start_device,
      max_positions, heads, kv_heads, head_dim, vt_keys, static_cast<uint16_t*>(q),
      static_cast<uint16_t*>(k), static_cast<uint16_t*>(v), nullptr, nullptr, as_stream(stream)));
}

int parrot_proj_rope_qkv_frag_bf16(const void* x, int64_t batch, int32_t seq, int32_t dim,
                                   const void* w_packed, const float* cos_table,
                                   const float* sin_table, int32_t start,
                                   const int32_t* start_device, int32_t max_positions,
                                   int32_t heads, int32_t kv_heads, int32_t head_dim, void* q,
                                   void* k, void* v, void* k_frag, void* v_frag, void* stream) {
  if (!x || !w_packed || !cos_table || !sin_table || !q || !k_frag || !v_frag)
    return PARROT_ERR_NULL_POINTER;
  if (batch < 0 || seq < 0 || start < 0 || dim <= 0 || heads <= 0 || kv_heads <= 0 ||
      head_dim <= 0 || max_positions <= 0 || static_cast<int64_t>(start) + seq > max_positions)
    return PARROT_ERR_BAD_SHAPE;
  if (heads % kv_heads || !parrot::attention_head_dim_supported(head_dim))
    return PARROT_ERR_UNSUPPORTED;
  const int64_t n = static_cast<int64_t>(heads + 2 * kv_heads) * head_dim;
  if (n > INT32_MAX || !parrot::proj_shape_supported(dim, static_cast<int>(n)) ||
      batch * seq > INT32_MAX)
    return PARROT_ERR_UNSUPPORTED;
  if (!aligned16(x) || !aligned16(w_packed) || !aligned16(k_frag) || !aligned16(v_frag))
    return PARROT_ERR_ALIGNMENT;
  if (batch == 0 || seq == 0) return PARROT_OK;
  return status(parrot::launch_proj_rope_qkv(
      static_cast<const uint16_t*>(x), static_cast<int>(batch * seq), seq, dim,
      static_cast<const uint16_t*>(w_packed), cos_table, sin_table, start, start_device,
      max_positions, heads, kv_heads, head_dim, 0, static_cast<uint16_t*>(q),
      static_cast<uint16_t*>(k), static_cast<uint16_t*>(v), static_cast<uint16_t*>(k_frag),
      static_cast<uint16_t*>(v_frag), as_stream(stream)));
}

int parrot_proj_frag_bf16(const void* x, int64_t batch, int32_t seq, int32_t k,
                          const void* w_packed, int32_t n, int32_t head_dim, int32_t values,
                          void* out, void* stream) {
  if (!x || !w_packed || !out) return PARROT_ERR_NULL_POINTER;
  if (batch < 0 || seq < 0 || k <= 0 || n <= 0 || head_dim <= 0 || n % head_dim ||
      (values != 0 && values != 1))
    return PARROT_ERR_BAD_SHAPE;
  if (!parrot::proj_shape_supported(k, n) || !parrot::attention_head_dim_supported(head_dim) ||
      batch * seq > INT32_MAX)
    return PARROT_ERR_UNSUPPORTED;
  if (!aligned16(x) || !aligned16(w_packed) || !aligned16(out)) return PARROT_ERR_ALIGNMENT;
  if (batch == 0 || seq == 0) return PARROT_OK;
  return status(parrot::launch_proj_frag(
      static_cast<const uint16_t*>(x), static_cast<int>(batch * seq), seq, k, k,
      static_cast<const uint16_t*>(w_packed), n, head_dim,
      values ? nullptr : static_cast<uint16_t*>(out), values ? static_cast<uint16_t*>(out) : nullptr,
      as_stream(stream)));
}

int parrot_proj_kv_frag_bf16(const void* x, int64_t batch, int32_t seq, int32_t k, int64_t lda,
                             const void* w_packed, int32_t n, int32_t head_dim, void* k_frag,
                             void* v_frag, void* stream) {
  if (!x || !w_packed || !k_frag || !v_frag) return PARROT_ERR_NULL_POINTER;
  if (batch < 0 || seq < 0 || k <= 0 || n <= 0 || head_dim <= 0 || n % head_dim || lda < k)
    return PARROT_ERR_BAD_SHAPE;
  if (n > INT32_MAX / 2 || !parrot::proj_shape_supported(k, 2 * n) ||
      !parrot::attention_head_dim_supported(head_dim) || batch * seq > INT32_MAX)
    return PARROT_ERR_UNSUPPORTED;
  if (!aligned16(x) || lda % 8 || !aligned16(w_packed) || !aligned16(k_frag) ||
      !aligned16(v_frag))
    return PARROT_ERR_ALIGNMENT;
  if (batch == 0 || seq == 0) return PARROT_OK;
  return status(parrot::launch_proj_frag(
      static_cast<const uint16_t*>(x), static_cast<int>(batch * seq), seq, k, lda,
      static_cast<const uint16_t*>(w_packed), 2 * n, head_dim, static_cast<uint16_t*>(k_frag),
      static_cast<uint16_t*>(v_frag), as_stream(stream)));
}

int parrot_grouped_experts_bf16(const void* x, int64_t tokens, int32_t dim, int32_t experts,
                                int32_t hidden_dim, int32_t shared_dim, int32_t capacity,
                                const int32_t* counts, const int32_t* offsets,
                                const int32_t* perm, const int32_t* overflow,
                                const float* route_weights, const void* packed_gate_up,
                                const void* down, const void* shared_gate_up,
                                const void* shared_down, const void* addend, void* out,
                                void* workspace, size_t workspace_bytes, void* stream) {
  if (!out || !route_weights || !down || !shared_down) return PARROT_ERR_NULL_POINTER;
  ExpertsWorkspace ws;
  if (int rc = check_experts(tokens, dim, experts, hidden_dim, shared_dim, capacity, counts,
                             offsets, perm, overflow, workspace, workspace_bytes, &ws))
    return rc;
  if (!aligned16(down) || !aligned16(shared_down) || !aligned16(out) ||
      (addend && !aligned16(addend)))
    return PARROT_ERR_ALIGNMENT;
  int rc = parrot_experts_gate_up_bf16(x, tokens, dim, experts, hidden_dim, shared_dim,
                                       capacity, counts, offsets, perm, overflow,
                                       packed_gate_up, shared_gate_up, workspace,
                                       workspace_bytes, stream);
  if (rc != PARROT_OK) return rc;
  rc = parrot_experts_down_bf16(tokens, dim, experts, hidden_dim, shared_dim, capacity, counts,
                                offsets, perm, overflow, route_weights, down, shared_down,
                                workspace, workspace_bytes, stream);
  if (rc != PARROT_OK) return rc;
  return parrot_experts_combine_bf16(tokens, dim, hidden_dim, shared_dim, addend, out,
                                     workspace, workspace_bytes, stream);
}

}  // extern "C"

// ---- attained-peak measurements ---------------------------------------------

extern "C" {

int parrot_peak_mfma_bf16(int32_t wide, int64_t blocks, int32_t iters, float* out,
                          int64_t* flops, void* stream) {
  if (!out || !flops) return PARROT_ERR_NULL_POINTER;
  if (blocks < 1 || blocks > (int64_t{1} << 20) || iters < 1 || (wide != 0 && wide != 1))
    return PARROT_ERR_BAD_SHAPE;
  *flops = blocks * parrot::peak_mfma_flops_per_block(wide, iters);
  return status(parrot::launch_peak_mfma(wide, blocks, iters, out, as_stream(stream)));
}

int parrot_peak_copy(const void* src, void* dst, int64_t bytes, int64_t blocks, void* stream) {
  if (!src || !dst) return PARROT_ERR_NULL_POINTER;
  if (bytes < 0 || bytes % 16 || blocks < 1 || blocks > (int64_t{1} << 20))
    return PARROT_ERR_BAD_SHAPE;
  if (!aligned16(src) || !aligned16(dst)) return PARROT_ERR_ALIGNMENT;
  if (bytes == 0) return PARROT_OK;
  return status(parrot::launch_peak_copy(src, dst, bytes, blocks, as_stream(stream)));
}

}  // extern "C"

// ---- allocation-free grouped experts ----------------------------------------

namespace {

// The workspace of parrot_grouped_experts_static_bf16.  In host code the
// name is only a handle: kernels get the device address that
// hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) unsigned char scratch[PARROT_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_address[kMaxDevices];

// The current device's address of `scratch`, resolved on its first use on
// that device (concurrent first calls store the same address).
int static_scratch(void** address) {
  int device = 0;
  if (hipError_t e = hipGetDevice(&device); e != hipSuccess) return status(e);
  if (device < 0 || device >= kMaxDevices) return PARROT_ERR_UNSUPPORTED;
  void* p = g_scratch_address[device].load(std::memory_order_acquire);
  if (p == nullptr) {
    if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); e != hipSuccess)
      return status(e);
    if (p == nullptr) return PARROT_ERR_NULL_POINTER;
    g_scratch_address[device].store(p, std::memory_order_release);
  }
  *address = p;
  return PARROT_OK;
}

}  // namespace

extern "C" {

int parrot_grouped_experts_static_bf16(const void* x, int64_t tokens, int32_t dim,
                                       int32_t experts, int32_t hidden_dim, int32_t shared_dim,
                                       int32_t capacity, const int32_t* counts,
                                       const int32_t* offsets, const int32_t* perm,
                                       const int32_t* overflow, const float* route_weights,
                                       const void* packed_gate_up, const void* down,
                                       const void* shared_gate_up, const void* shared_down,
                                       const void* addend, void* out, void* stream) {
  if (tokens < 0 || dim <= 0 || hidden_dim <= 0 || shared_dim <= 0) return PARROT_ERR_BAD_SHAPE;
  const size_t need = experts_ws(nullptr, tokens, dim, hidden_dim, shared_dim).bytes;
  if (need > PARROT_STATIC_SCRATCH_BYTES) return PARROT_ERR_SCRATCH_LIMIT;
  void* workspace = nullptr;
  if (int rc = static_scratch(&workspace)) return rc;
  return parrot_grouped_experts_bf16(x, tokens, dim, experts, hidden_dim, shared_dim, capacity,
                                     counts, offsets, perm, overflow, route_weights,
                                     packed_gate_up, down, shared_gate_up, shared_down, addend,
                                     out, workspace, PARROT_STATIC_SCRATCH_BYTES, stream);
}

}  // extern "C"
