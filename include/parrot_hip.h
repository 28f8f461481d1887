/*
 * parrot_hip.h -- C ABI of the MI355X (gfx950) Parrot inference MoE path.
 *
 * Shared library: parrot-h200-worker_amd/parrot/_lib/libparrot_hip.so
 *
 * Conventions
 *   - Every pointer is a device pointer unless stated; tensors are dense and
 *     row-major.  bf16 tensors are 16-byte aligned.
 *   - `stream` is a hipStream_t (PyTorch-ROCm: torch.cuda.current_stream().cuda_stream).
 *     Every entry point only enqueues work on that stream: no host
 *     synchronisation, no allocation, no global mutable state.
 *   - The return value is a status: 0 on success, a negative PARROT_ERR_*
 *     code when an argument is rejected before anything is launched, or a
 *     positive hipError_t from the launch.
 *   - The caller owns every buffer, including the workspaces whose sizes the
 *     *_workspace_bytes functions report.
 *
 * Each entry point names the reference interface it replaces
 * (paths relative to the jkpdino/parrot-h200-worker checkout).
 */
#ifndef PARROT_HIP_H
#define PARROT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PARROT_ABI_VERSION 14

#define PARROT_OK 0
#define PARROT_ERR_NULL_POINTER (-1)
#define PARROT_ERR_BAD_SHAPE (-2)
#define PARROT_ERR_UNSUPPORTED (-3)
#define PARROT_ERR_WORKSPACE (-4)
#define PARROT_ERR_ALIGNMENT (-5)
#define PARROT_ERR_SCRATCH_LIMIT (-6)

/* Bytes of the library's static device scratch array (per GPU), the
 * workspace of parrot_grouped_experts_static_bf16: 4096 tokens at dim 768,
 * H 512, Hs 256 (7.5 KiB per token: the hidden rows and the bf16 expert
 * outputs). */
#define PARROT_STATIC_SCRATCH_BYTES ((size_t)30 << 20)

/* ABI version (PARROT_ABI_VERSION) of the loaded library. */
int parrot_abi_version(void);

/* Text for a status returned by any entry point (static storage). */
const char* parrot_status_string(int status);

/* Fixed expert capacity C = max(8, roundup8(ceil(2 * 2T / E))), top-2.
 * Replaces the capacity expression of grouped_mps_experts,
 * parrot/metal_moe.py:388-391. */
int32_t parrot_capacity(int64_t tokens, int32_t experts);

/* y = bf16(x * rsqrt(mean(x^2) + eps) * weight) per row; x, weight, out bf16.
 * dim % 4 == 0, dim <= 4096.
 * Replaces metal_rms_norm (parrot/metal_moe.py:37-55) with its kernels
 * rms_norm_bf16 / rms_norm_decode_bf16 (parrot/kernels/moe_bf16.metal:4-65). */
int parrot_rms_norm_bf16(const void* x, const void* weight, void* out, int64_t rows,
                         int32_t dim, float eps, void* stream);

/* Block AttnRes depth mix over 1..9 bf16 sources [tokens, dim]:
 *   score_s = <rmsnorm(v_s; score_norm_weight, score_eps), query>,
 *   mix = bf16(sum_s softmax(score)_s v_s).
 * Writes mix to out_mix when non-NULL, and rmsnorm(mix; out_norm_weight,
 * out_eps) to out_norm when non-NULL (at least one of them).
 * dim % 4 == 0, dim <= 2048.
 * Replaces metal_depth_mix (parrot/metal_moe.py:419-452; kernels
 * depth_scores_bf16, depth_mix_bf16, depth_mix_decode_bf16) and
 * metal_depth_mix_norm (parrot/metal_moe.py:455-477; kernel
 * depth_mix_norm_decode_bf16), for every token count. */
int parrot_depth_mix_bf16(const void* const* sources, int32_t n_sources, const void* query,
                          const void* score_norm_weight, float score_eps,
                          const void* out_norm_weight, float out_eps, int64_t tokens,
                          int32_t dim, void* out_mix, void* out_norm, void* stream);

/* The forward's first launch: rows_out[t] = table[ids[t]] (bf16 [tokens,
 * dim], the embedding rows that become the residual stream's first source)
 * and out_norm = rmsnorm(parrot_depth_mix_bf16 of that single source;
 * out_norm_weight, out_eps), the first module's input, with the same bits as
 * the separate gather and depth mix; also zero-fills n_zeros floats at zeros
 * (the forward's router-stat outputs when they are not collected; zeros may
 * be NULL when n_zeros is 0).  Ids outside [0, vocab) read the nearest row:
 * the caller validates them (nn.Embedding raises).  tokens may be 0 (only the
 * zero fill runs).  dim % 4 == 0, dim <= 2048; bf16 pointers 8-byte aligned.
 * Replaces self.embedding(input_ids) and the first depth_mix of
 * Parrot.forward (parrot/model.py:679, 685-687) and the router-stat zeros
 * (parrot/model.py:719-723) when bag_size is 1. */
int parrot_embed_depth_mix_bf16(const int64_t* ids, int64_t tokens, const void* table,
                                int64_t vocab, int32_t dim, const void* query,
                                const void* score_norm_weight, float score_eps,
                                const void* out_norm_weight, float out_eps, void* rows_out,
                                void* out_norm, float* zeros, int32_t n_zeros, void* stream);

/* parrot_depth_mix_bf16 (out_norm required) followed by the router of
 * parrot_route_bf16 on the normalised rows, in one launch: writes
 * out_weights fp32 [T, 2] and out_indices int64 [T, 2] exactly as
 * parrot_route_bf16 does for x = out_norm, at every token count (the same
 * logit arithmetic to the bit: four k-step chains by st % 4 summed in a
 * fixed order, the same top-2 and renormalised weights).  No grouping
 * outputs, no router stats.
 * router_weight bf16 [E, dim], 16-byte aligned; logit_bias optional fp32 [E];
 * 2 <= E <= 32; dim % 32 == 0, dim <= 2048.
 * Replaces, for a MoE layer's input, metal_depth_mix_norm
 * (parrot/metal_moe.py:455-477) followed by the router projection and top-2
 * of metal_route (parrot/metal_moe.py:58-81; parrot/model.py:520-527). */
int parrot_depth_mix_route_bf16(const void* const* sources, int32_t n_sources,
                                const void* query, const void* score_norm_weight,
                                float score_eps, const void* out_norm_weight, float out_eps,
                                int64_t tokens, int32_t dim, void* out_mix, void* out_norm,
                                const void* router_weight, const float* logit_bias,
                                int32_t experts, float* out_weights, int64_t* out_indices,
                                void* stream);

/* parrot_depth_mix_route_bf16 (no out_mix) whose last source is a pending
 * attention output: resolved = bf16(base + bf16(sum over the heads of
 * contributions[t, h, :])) (heads == 8, summed in head order; base optional,
 * else the rounded sum alone), written to `resolved` and mixed as source
 * n_sources - 1 (whose pointer in `sources` must still be a readable
 * [tokens, dim] row block; it is not used).  contributions fp32 [tokens,
 * heads, dim] as parrot_causal_attention_frag_out_bf16 writes them.
 * Replaces resolving the reference's PendingResidual inside the consumer's
 * mix (parrot/model.py:103-106, 832-860; metal_depth_mix_norm_pending,
 * parrot/metal_moe.py:480-500) for a MoE module's routed input. */
int parrot_depth_mix_route_pending_bf16(
    const void* const* sources, int32_t n_sources, const void* query,
    const void* score_norm_weight, float score_eps, const void* out_norm_weight, float out_eps,
    int64_t tokens, int32_t dim, void* out_norm, const void* router_weight,
    const float* logit_bias, int32_t experts, float* out_weights, int64_t* out_indices,
    const float* contributions, int32_t heads, const void* base, void* resolved, void* stream);

/* parrot_experts_combine_bf16 folded into the next module's depth mix: the
 * combined MoE row out (bf16(addend + bf16(shared + routed rows)), exactly
 * as parrot_experts_combine_bf16, written to out) is the last of n_sources
 * depth sources; sources holds the other n_sources - 1 ([tokens, dim] bf16,
 * in stream order), and the mix / normalised mix are written as by
 * parrot_depth_mix_bf16.  workspace is the one filled by
 * parrot_experts_down_bf16.  Replaces, for a layer whose MoE output feeds the
 * next attention layer, the combine of grouped_mps_experts
 * (parrot/metal_moe.py:372-416) followed by metal_depth_mix_norm
 * (parrot/metal_moe.py:455-477). */
int parrot_experts_combine_depth_mix_bf16(
    int64_t tokens, int32_t dim, int32_t hidden_dim, int32_t shared_dim, const void* addend,
    void* out, void* workspace, size_t workspace_bytes, const void* const* sources,
    int32_t n_sources, const void* query, const void* score_norm_weight, float score_eps,
    const void* out_norm_weight, float out_eps, void* out_mix, void* out_norm, void* stream);

/* Rotary embedding of the local-attention heads fused with the head-major
 * split of one packed projection qkv [batch * seq, (H + 2 Hk) * head_dim]
 * (bf16, row-major, columns q | k | v):
 *   q [batch, H, seq, head_dim]; k, v [batch, Hk, seq, head_dim], or
 *   [batch, H, seq, head_dim] with every kv head repeated H / Hk times when
 *   expand_kv != 0.
 * Pairs (2i, 2i+1) of q and k rotate by angle p * theta^(-2i/d) at position
 * p = start + s, plus *start_device when start_device (a device int32) is
 * non-NULL, read from fp32 tables cos_table / sin_table
 * [max_positions, head_dim / 2]; positions past the table are clamped to its
 * last row (a device position cannot be checked here).  v is copied.
 * With vt_keys > 0, v is written transposed instead: v [batch, Hk,
 * head_dim, vt_keys] (vt_keys >= seq; the layout parrot_causal_attention_bf16
 * reads; entries past seq are left untouched).
 * head_dim % 4 == 0, H % Hk == 0, start + seq <= max_positions.
 * Replaces LocalGQA._project / _project_decode / _rope
 * (parrot/model.py:206-262), which run RoPE as strided bf16 elementwise ops. */
int parrot_rope_qkv_bf16(const void* qkv, const float* cos_table, const float* sin_table,
                         int64_t batch, int32_t seq, int32_t start, const int32_t* start_device,
                         int32_t max_positions, int32_t heads, int32_t kv_heads,
                         int32_t head_dim, int32_t expand_kv, int32_t vt_keys, void* q,
                         void* k, void* v, void* stream);

/* Decode-step attention of the sliding-window GQA layers.  q [batch, H,
 * head_dim] and the new key / value rows k_new, v_new [batch, Hk, head_dim]
 * (RoPE applied, bf16); caches [batch, Hk, max_positions, head_dim] bf16.
 * With p = *position (device int32): stores k_new / v_new at cache position
 * p and writes out [batch, H, head_dim] (bf16) =
 * softmax(q . K^T * scale) V over positions max(0, p - window + 1) .. p of
 * each query head's kv head (head h uses kv head h / (H / Hk)); fp32 scores,
 * softmax and accumulation.  Nothing is written when p is outside
 * [0, max_positions).  head_dim in {8, 16, 32, 64, 96, 128, 192, 256},
 * (min(window, max_positions) + head_dim + 2048 + 4) * 4 <= 65536; caches
 * and new rows 16-byte aligned.  Reading p from device memory keeps the shapes
 * static, so a decode step can be captured in a HIP graph.
 * Replaces the cache update + scaled_dot_product_attention of
 * LocalGQA.decode (parrot/model.py:239-262) and the Metal kernel
 * local_attention_decode_bf16 (parrot/kernels/moe_bf16.metal:1203-1362). */
int parrot_decode_attention_bf16(const void* q, const void* k_new, const void* v_new,
                                 void* key_cache, void* value_cache, const int32_t* position,
                                 int32_t batch, int32_t heads, int32_t kv_heads,
                                 int32_t head_dim, int32_t max_positions, int32_t window,
                                 float scale, void* out, void* stream);

/* parrot_decode_attention_bf16 with the output projection of each head
 * deferred (the reference's defer_sum / PendingResidual, parrot/model.py:
 * 103-106, 301-316, 868-889, and the per-head output stage of
 * local_attention_decode_bf16, parrot/kernels/moe_bf16.metal:1203-1362):
 * instead of the attention output it writes contributions [batch, heads,
 * dim] fp32, contributions[b, h, n] = sum_i y[b, h, i] * out_weight[n,
 * h * head_dim + i] over i in order, where y is the head's attention output
 * rounded to bf16 and out_weight [dim, heads * head_dim] bf16 (16-byte
 * aligned) is the output projection.  Summed over heads (in head order),
 * rounded to bf16 and added to the addend they give the attention module's
 * output; parrot_depth_mix_decode_moe_pending_bf16 does that in its input
 * mix.  Each head runs in 16 workgroups, one per 1/16 of the output
 * columns: dim % 16 == 0, dim <= 4096; LDS as parrot_decode_attention_bf16
 * plus 4 * head_dim bytes; other limits as there. */
int parrot_decode_attention_heads_bf16(const void* q, const void* k_new, const void* v_new,
                                       void* key_cache, void* value_cache,
                                       const int32_t* position, int32_t batch, int32_t heads,
                                       int32_t kv_heads, int32_t head_dim, int32_t max_positions,
                                       int32_t window, float scale, const void* out_weight,
                                       int32_t dim, float* contributions, void* stream);

/* PARROT_OK when parrot_decode_attention_heads_bf16 takes this shape and its
 * contributions fit the pending input mix of
 * parrot_depth_mix_decode_moe_pending_bf16 (one lane per head: heads <= 16,
 * dim <= 1024, dim % 4 == 0); otherwise the status either call would return.
 * No pointer, no launch: the shape predicate of the deferred decode step
 * (LocalGQA.decode(defer_sum=True), parrot/model.py:301-316), which takes the
 * undeferred path when this fails. */
int parrot_decode_attention_heads_check(int32_t batch, int32_t heads, int32_t kv_heads,
                                        int32_t head_dim, int32_t max_positions, int32_t window,
                                        int32_t dim);

/* Decode-step attention of the MLA layers over the joint latent cache.
 * q [batch, H, latent_dim] fp32 (the query through the absorbed key
 * up-projection), latent_new [batch, latent_dim] bf16, latent_cache
 * [batch, max_positions, latent_dim] bf16.  With p = *position: stores
 * latent_new at position p and writes out [batch, H, latent_dim] (fp32) =
 * softmax(q . Lat^T * scale) Lat over positions 0 .. p, the latents serving
 * as both keys and values.  Limits as parrot_decode_attention_bf16 with
 * window = max_positions.  Replaces the cache update + attention of
 * GlobalMLA.decode (parrot/model.py:399-432) and the Metal kernel
 * mla_attention_decode_bf16 (parrot/kernels/moe_bf16.metal:1391-1518). */
int parrot_decode_attention_latent_f32(const float* q, const void* latent_new, void* latent_cache,
                                       const int32_t* position, int32_t batch, int32_t heads,
                                       int32_t latent_dim, int32_t max_positions, float scale,
                                       float* out, void* stream);

/* The decode step's q|k|v projection of a local (GQA) layer with RoPE, one
 * launch: for each token t, q|k|v = h_t W^T rounded to bf16 (qkv_weight
 * [(heads + 2 kv_heads) head_dim, dim] bf16 row-major, the q, k and v
 * weights stacked), then q and k rotated by RoPE at position *position
 * (cos_table / sin_table fp32 [max_positions, head_dim / 2], the position
 * clamped into them) and rounded again; q [tokens, heads, 1, head_dim], k
 * and v [tokens, kv_heads, 1, head_dim] bf16.  h is x [tokens, dim] bf16
 * when x is non-NULL, else the depth mix of `sources` normalised by the
 * attention norm (attention_norm_weight, norm_eps), exactly as
 * parrot_depth_mix_bf16 with out_norm computes it (sources, n_sources,
 * query, score_norm_weight, score_eps as there).  tokens <= 16, dim % 128 ==
 * 0 and dim <= 1024, head_dim even, (heads + 2 kv_heads) head_dim % 16 == 0;
 * x and qkv_weight 16-byte aligned.  The projection's fp32 sums run in
 * another order than a GEMM's, so its bf16 values may differ from those of
 * parrot_proj_rope_qkv_bf16 in the last place.  Replaces, for a decode step,
 * metal_depth_mix_norm (parrot/metal_moe.py:455-477) and the q/k/v
 * projections + _apply_rope of LocalGQA.decode (parrot/model.py:176-262). */
int parrot_decode_qkv_bf16(const void* x, const void* const* sources, int32_t n_sources,
                           const void* query, const void* score_norm_weight, float score_eps,
                           const void* attention_norm_weight, float norm_eps, int32_t tokens,
                           int32_t dim, const void* qkv_weight, int32_t heads,
                           int32_t kv_heads, int32_t head_dim, const float* cos_table,
                           const float* sin_table, int32_t max_positions,
                           const int32_t* position, void* q, void* k, void* v, void* stream);

/* parrot_decode_qkv_bf16 for the first layer of a decode step, with the
 * token embedding in the launch: h_t is the attention norm of the depth mix
 * of one source, row token_ids[t] of embedding [vocab, dim] bf16 (16-byte
 * aligned; an id outside [0, vocab) reads the nearest row, where the
 * reference's nn.Embedding raises), and that row is also stored to embedded
 * [tokens, dim] (16-byte aligned), the later layers' first depth source.
 * Replaces the embedding lookup of Parrot.decode_step (parrot/model.py:830,
 * nn.Embedding) and its launch; other limits and outputs as
 * parrot_decode_qkv_bf16. */
int parrot_decode_qkv_embed_bf16(const int64_t* token_ids, const void* embedding, int32_t vocab,
                                 void* embedded, const void* query, const void* score_norm_weight,
                                 float score_eps, const void* attention_norm_weight,
                                 float norm_eps, int32_t tokens, int32_t dim,
                                 const void* qkv_weight, int32_t heads, int32_t kv_heads,
                                 int32_t head_dim, const float* cos_table,
                                 const float* sin_table, int32_t max_positions,
                                 const int32_t* position, void* q, void* k, void* v,
                                 void* stream);

/* The MLA layers' decode-step projections before the latent attention, one
 * launch: q_latent [tokens, query_rows] fp32 = x . absorbed_query^T with x
 * [tokens, dim] bf16 and absorbed_query [query_rows, dim] bf16 (the absorbed
 * query map, H * latent_dim rows), products and sums in fp32; latent
 * [tokens, latent_dim] bf16 = bf16(x . kv_down^T), kv_down [latent_dim, dim]
 * bf16.  With x NULL the rows are the depth mix of `sources` normalised by
 * the attention norm, as parrot_decode_qkv_bf16 takes them (dim <= 1024).
 * tokens <= 16, dim % 128 == 0 and dim <= 2048, query_rows and latent_dim
 * multiples of 16; x, absorbed_query and kv_down 16-byte aligned.
 * Replaces F.linear(x.float(), absorbed_query.float()) and kv_down(x) in
 * GlobalMLA.decode (parrot/model.py:417-422), the projections that
 * metal_mla_attention_decode (parrot/metal_moe.py:293-326) fuses. */
int parrot_mla_decode_in_bf16(const void* x, const void* const* sources, int32_t n_sources,
                              const void* query, const void* score_norm_weight, float score_eps,
                              const void* attention_norm_weight, float norm_eps,
                              int32_t tokens, int32_t dim, const void* absorbed_query,
                              int32_t query_rows, const void* kv_down, int32_t latent_dim,
                              float* q_latent, void* latent, void* stream);

/* A decode step's bias-free linear map of up to 16 rows, one launch: out
 * [tokens, n] bf16 = bf16(x . weight^T), then bf16(addend + that) when
 * addend [tokens, n] bf16 is given; x [tokens, k] bf16, weight [n, k] bf16
 * row-major (nn.Linear), fp32 products and sums.  tokens <= 16, k % 128 ==
 * 0 and k <= 2048, tokens * k * 2 <= 65536, n % 16 == 0; x and weight
 * 16-byte aligned.  Replaces, at decode, the attention output projection of
 * LocalGQA with its residual add (parrot/model.py:167-230;
 * attention_output_decode_bf16, parrot/kernels/moe_bf16.metal:1364-1389). */
int parrot_decode_linear_bf16(const void* x, int32_t tokens, int32_t k, const void* weight,
                              int32_t n, const void* addend, void* out, void* stream);

/* The MLA layers' decode-step output projection after the latent attention:
 * out [tokens, dim] bf16 = bf16(context . absorbed_output^T), then
 * bf16(addend + that) when addend [tokens, dim] bf16 is given; context
 * [tokens, width] fp32, absorbed_output [dim, width] bf16, fp32 products and
 * sums.  tokens <= 16, width % 128 == 0, tokens * width * 4 <= 65536, dim %
 * 16 == 0; context and absorbed_output 16-byte aligned.  Replaces
 * F.linear(context, absorbed_output.float()).to(bf16) and the addend sum in
 * GlobalMLA.decode (parrot/model.py:430-431). */
int parrot_mla_decode_out_bf16(const float* context, int32_t tokens, int32_t width,
                               const void* absorbed_output, int32_t dim, const void* addend,
                               void* out, void* stream);

/* Workspace bytes of parrot_decode_moe_bf16: hidden rows [3T, max(H, Hs)]
 * bf16. */
size_t parrot_decode_moe_workspace_bytes(int64_t tokens, int32_t hidden_dim,
                                         int32_t shared_dim);

/* Whole MoE layer for a decode step of tokens <= 16 rows x [tokens, dim]
 * (bf16) in two launches: router logits (fp32, + logit_bias when non-NULL),
 * top-2 with ties to the lower expert index and weights renormalised over
 * the two (written to out_indices [tokens, 2] int64 / out_weights
 * [tokens, 2] fp32); SwiGLU of both routed experts and the shared expert
 * (hidden rounded to bf16); out = bf16(shared + w0 y0 + w1 y1), or
 * bf16(addend + bf16(...)) with an addend.  Packed weights as for
 * parrot_grouped_experts_bf16.  Every assignment is computed (capacity and
 * overflow do not apply at these sizes).  2 <= experts <= 32; dim, H, Hs
 * multiples of 64, dim <= 2048.  Replaces metal_experts_decode (parrot/metal_moe.py:
 * 182-221; kernels moe_decode_lanes_bf16 / moe_sum_decode_lanes_bf16,
 * parrot/kernels/moe_bf16.metal:894-1024, 1185-1201) and, for these sizes,
 * the route + grouped-experts path of MoE.inference (parrot/model.py:
 * 571-607). */
int parrot_decode_moe_bf16(const void* x, int64_t tokens, int32_t dim, int32_t experts,
                           int32_t hidden_dim, int32_t shared_dim, const void* router_weight,
                           const float* logit_bias, const void* packed_gate_up,
                           const void* packed_down, const void* shared_gate_up,
                           const void* shared_down, const void* addend, void* out,
                           int64_t* out_indices, float* out_weights, void* workspace,
                           size_t workspace_bytes, void* stream);

/* parrot_decode_moe_bf16 whose input rows it makes itself: x = the depth
 * mix of `sources` normalised by the MoE's RMSNorm (moe_norm_weight,
 * norm_eps), exactly as parrot_depth_mix_bf16 with out_norm computes it
 * (sources, n_sources, query, score_norm_weight and score_eps as there).
 * Saves that launch at decode.  dim <= 1024; other limits as
 * parrot_decode_moe_bf16.  Replaces, for a decode step's MoE layer,
 * metal_depth_mix_norm (parrot/metal_moe.py:455-477) followed by
 * metal_experts_decode (parrot/metal_moe.py:182-221). */
int parrot_depth_mix_decode_moe_bf16(
    const void* const* sources, int32_t n_sources, const void* query,
    const void* score_norm_weight, float score_eps, const void* moe_norm_weight,
    float norm_eps, int64_t tokens, int32_t dim, int32_t experts, int32_t hidden_dim,
    int32_t shared_dim, const void* router_weight, const float* logit_bias,
    const void* packed_gate_up, const void* packed_down, const void* shared_gate_up,
    const void* shared_down, const void* addend, void* out, int64_t* out_indices,
    float* out_weights, void* workspace, size_t workspace_bytes, void* stream);

/* parrot_depth_mix_decode_moe_bf16 whose last depth source is pending: row
 * t of source n_sources - 1 is resolved in the launch as bf16(base[t] +
 * bf16(sum over lanes l in order of contributions[t, l, :])) (without a
 * base: the rounded sum), the reference's depth_mix_norm_pending_bf16
 * (parrot/kernels/moe_bf16.metal:437-560, via metal_depth_mix_norm_pending,
 * parrot/metal_moe.py:480-500), and written to resolved [tokens, dim]; the
 * sources entry of that slot is only a placeholder (any valid row block).
 * contributions [tokens, lanes, dim] fp32 (16-byte aligned), 1 <= lanes <=
 * 16; base and resolved bf16, 8-byte aligned (base may be NULL).  The
 * addend may be `resolved` itself: the routed launch that stores it runs
 * before the one that adds the addend.  Other arguments and limits as
 * parrot_depth_mix_decode_moe_bf16. */
int parrot_depth_mix_decode_moe_pending_bf16(
    const void* const* sources, int32_t n_sources, const void* query,
    const void* score_norm_weight, float score_eps, const void* moe_norm_weight,
    float norm_eps, const float* contributions, int32_t lanes, const void* base,
    void* resolved, int64_t tokens, int32_t dim, int32_t experts, int32_t hidden_dim,
    int32_t shared_dim, const void* router_weight, const float* logit_bias,
    const void* packed_gate_up, const void* packed_down, const void* shared_gate_up,
    const void* shared_down, const void* addend, void* out, int64_t* out_indices,
    float* out_weights, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of parrot_vocab_argmax_bf16. */
size_t parrot_vocab_argmax_workspace_bytes(int64_t rows, int32_t vocab);

/* Greedy next token per row without materialising the logits:
 * out_tokens[r] = argmax_v sum_d hidden[r, d] * weight[v, d] for hidden
 * [rows, dim] and the tied head weight [vocab, dim] (bf16, row-major), fp32
 * logits, ties to the lower index.  rows <= 16, dim % 8 == 0, dim <= 2048.
 * Replaces argmax(F.linear(h, embedding.weight)) of decode_next
 * (parrot/model.py:714-715, 922, 927-931) and the Metal kernels
 * vocab_argmax_partials_bf16 / vocab_argmax_reduce_bf16
 * (parrot/kernels/moe_bf16.metal:1541-1621).
 * advance_position (optional, int32 on the device): incremented by one
 * after the argmax -- the decode step's position counter, advanced by the
 * step's last launch instead of a launch of its own. */
int parrot_vocab_argmax_bf16(const void* hidden, int64_t rows, int32_t dim, const void* weight,
                             int32_t vocab, int64_t* out_tokens, int32_t* advance_position,
                             void* workspace, size_t workspace_bytes, void* stream);

/* Causal attention with an optional sliding window, for prefill and full
 * forwards: out[b, i, h, :] = softmax_j(q[b,h,i] . k[b,h',j] * scale)
 * v[b,h',j] over keys i - window < j <= i (window >= seq: plain causal),
 * h' = h / (heads / kv_heads); fp32 scores, softmax and accumulation, P
 * rounded to bf16 for its product with V, one bf16 rounding of the output.
 * q [batch, heads, seq, head_dim] and k [batch, kv_heads, seq, head_dim]
 * given by element strides {batch, head, row} with unit stride along
 * head_dim; the values are given transposed, vt [batch, kv_heads, head_dim,
 * >= roundup(seq, 32)] by strides {batch, head, dim row} with unit stride
 * along the keys (entries past seq may hold anything).  Strides multiples of
 * 8, bases 16-byte aligned; out [batch, seq, heads, head_dim] contiguous.
 * head_dim in {64, 96, 128}; seq * k row stride and head_dim * vt row stride
 * below 2^30 elements.  Replaces scaled_dot_product_attention(...,
 * is_causal=True) and the masked chunk loop of LocalGQA.prefill
 * (parrot/model.py:264-295) and the causal SDPA of GlobalMLA.prefill
 * (parrot/model.py:350-360). */
int parrot_causal_attention_bf16(const void* q, const void* k, const void* vt,
                                 const int64_t* q_strides, const int64_t* k_strides,
                                 const int64_t* vt_strides, int64_t batch, int32_t seq,
                                 int32_t heads, int32_t kv_heads, int32_t head_dim,
                                 int32_t window, float scale, void* out, void* stream);

/* As parrot_causal_attention_bf16 with K and V given in MFMA fragment order,
 * the layout parrot_proj_rope_qkv_frag_bf16 and parrot_proj_frag_bf16 write:
 * per (batch, kv head), nblk = ceil(seq / 32) blocks of 32 keys, each block
 * a sequence of 1 KB wavefront fragments of 64 lanes x 8 bf16, lane
 * l = 16 g + c:
 *   k_frag [batch, kv_heads, nblk, 2 (n), head_dim / 32 (s), 64, 8]: key
 *     32 blk + 16 n + c, dims 32 s + 8 g .. 32 s + 8 g + 7;
 *   v_frag [batch, kv_heads, nblk, head_dim / 16 (t), 64, 8]: dim 16 t + c,
 *     keys 32 blk + 4 g .. + 3, then 32 blk + 16 + 4 g .. + 3.
 * Keys past seq in the last block may hold anything.  Every fragment of a
 * key block is then one contiguous 1 KB load (row-major K and V^T loads
 * touch 16 rows per instruction, which bounds the strided entry point at
 * prefill sizes).  Same results as parrot_causal_attention_bf16. */
int parrot_causal_attention_frag_bf16(const void* q, const int64_t* q_strides, const void* k_frag,
                                      const void* v_frag, int64_t batch, int32_t seq,
                                      int32_t heads, int32_t kv_heads, int32_t head_dim,
                                      int32_t window, float scale, void* out, void* stream);

/* parrot_causal_attention_frag_bf16 with the output projection deferred per
 * head, for whole sequences: instead of the output y it writes each head's
 * share of out(y), contributions[b, t, h, :] = y[b, t, h, :] (rounded to
 * bf16 as the output would be) times the head's head_dim columns of the
 * output weight, fp32 [batch, seq, heads, dim].  out_weight_packed is the
 * [dim, heads * head_dim] output weight packed as parrot_proj_bf16 takes it;
 * dim in {512, 768, 1024}.  bf16 of the sum over heads is
 * parrot_proj_bf16(y, out_weight) up to fp32 summation order.  Replaces the
 * attention + out projection of LocalGQA.prefill and GlobalMLA.prefill
 * (parrot/model.py:264-295, 350-360) where the next module's depth mix
 * takes the sum (parrot_depth_mix_route_pending_bf16), as the reference's
 * decode defers it (PendingResidual, parrot/model.py:103-106, 301-316). */
int parrot_causal_attention_frag_out_bf16(const void* q, const int64_t* q_strides,
                                          const void* k_frag, const void* v_frag, int64_t batch,
                                          int32_t seq, int32_t heads, int32_t kv_heads,
                                          int32_t head_dim, int32_t window, float scale,
                                          const void* out_weight_packed, int32_t dim,
                                          float* contributions, void* stream);

/* Dense projection y = x . W^T (bf16 in and out, fp32 accumulation) for the
 * attention layers' linear maps, with the weight pre-packed in MFMA fragment
 * order: w_packed holds W [n, k] as blocks of 16 rows x 32 k (1 KB), row
 * group major and k step minor; inside a block lane l = 16 g + r holds row r,
 * k = 8 g .. 8 g + 7 (16 bytes at 16 l).  x [rows, k] with row stride lda;
 * out [rows, n] with row stride ldo; when addend [rows, n] (row stride
 * ld_addend) is non-NULL, out = bf16(addend + bf16(x W^T)) (addend may be
 * out itself).  k % 64 == 0, k <= 2048, n % 16 == 0, lda % 8 == 0, x
 * 16-byte aligned.
 * Replaces the bias-free nn.Linear maps of LocalGQA / GlobalMLA
 * (parrot/model.py:167-230, 331-432) with the residual add of the
 * attention output as in attention_output_decode_bf16
 * (parrot/kernels/moe_bf16.metal:1364-1389). */
int parrot_proj_bf16(const void* x, int64_t rows, int32_t k, int64_t lda, const void* w_packed,
                     int32_t n, const void* addend, int64_t ld_addend, void* out, int64_t ldo,
                     void* stream);

/* As parrot_proj_bf16 for x [batch * seq, k] (contiguous) without addend,
 * stored transposed per sequence: out[(b * n + j) * ld_keys + t] =
 * bf16(x W^T)[b * seq + t, j], ld_keys >= seq, ld_keys % 4 == 0, out 8-byte
 * aligned; entries t >= seq are not written.  Produces the transposed values
 * parrot_causal_attention_bf16 reads (v_up of GlobalMLA.prefill,
 * parrot/model.py:350-360). */
int parrot_proj_transposed_bf16(const void* x, int64_t batch, int32_t seq, int32_t k,
                                const void* w_packed, int32_t n, int32_t ld_keys, void* out,
                                void* stream);

/* The packed q|k|v projection of a local-attention layer fused with RoPE and
 * the head split: x [batch * seq, dim] (contiguous) times the packed
 * [(H + 2 Hk) * head_dim, dim] weight (as parrot_proj_bf16), each output
 * rounded to bf16, then exactly the transform of parrot_rope_qkv_bf16 with
 * expand_kv = 0 (q, k and v, or v transposed when vt_keys > 0).  Replaces
 * F.linear + parrot_rope_qkv_bf16, i.e. the projections, _apply_rope and
 * the head split of LocalGQA (parrot/model.py:176-230). */
int parrot_proj_rope_qkv_bf16(const void* x, int64_t batch, int32_t seq, int32_t dim,
                              const void* w_packed, const float* cos_table,
                              const float* sin_table, int32_t start,
                              const int32_t* start_device, int32_t max_positions, int32_t heads,
                              int32_t kv_heads, int32_t head_dim, int32_t vt_keys, void* q,
                              void* k, void* v, void* stream);

/* parrot_proj_rope_qkv_bf16 (vt_keys = 0) writing the attention operands in
 * fragment order as well: q [batch, H, seq, head_dim]; k, v [batch, Hk, seq,
 * head_dim] only when non-NULL (the KV cache of a prefill); k_frag, v_frag in
 * the layout of parrot_causal_attention_frag_bf16.  head_dim in
 * {64, 96, 128}. */
int parrot_proj_rope_qkv_frag_bf16(const void* x, int64_t batch, int32_t seq, int32_t dim,
                                   const void* w_packed, const float* cos_table,
                                   const float* sin_table, int32_t start,
                                   const int32_t* start_device, int32_t max_positions,
                                   int32_t heads, int32_t kv_heads, int32_t head_dim, void* q,
                                   void* k, void* v, void* k_frag, void* v_frag, void* stream);

/* The projection x W^T of x [batch * seq, k] (as parrot_proj_bf16) stored as
 * attention K (values = 0) or V (values = 1) in fragment order for
 * n / head_dim heads (the layout of parrot_causal_attention_frag_bf16 with
 * kv_heads = n / head_dim).  head_dim in {64, 96, 128}.  Replaces k_up /
 * v_up of GlobalMLA.prefill (parrot/model.py:350-360). */
int parrot_proj_frag_bf16(const void* x, int64_t batch, int32_t seq, int32_t k,
                          const void* w_packed, int32_t n, int32_t head_dim, int32_t values,
                          void* out, void* stream);

/* Both MLA up-projections in one launch: w_packed is [Wk; Wv] ([2n, k],
 * packed as parrot_proj_bf16), x [batch * seq, k] with row stride lda; the
 * first n output columns are stored as k_frag and the last n as v_frag
 * (n / head_dim heads each, the layout of parrot_causal_attention_frag_bf16).
 * Replaces k_up(latent) and v_up(latent) of GlobalMLA.prefill
 * (parrot/model.py:350-360). */
int parrot_proj_kv_frag_bf16(const void* x, int64_t batch, int32_t seq, int32_t k, int64_t lda,
                             const void* w_packed, int32_t n, int32_t head_dim, void* k_frag,
                             void* v_frag, void* stream);

/* Workspace bytes for the routing / grouping entry points. */
size_t parrot_route_workspace_bytes(int64_t tokens, int32_t experts);

/* Router + top-2 + deterministic grouping.
 *   logits = x . router_weight^T (fp32) [+ logit_bias[e]], softmax top-2 with
 *   ties to the lower expert index, route weights renormalised over the pair.
 * Outputs (all required unless marked optional):
 *   out_logits  fp32 [T, E]   optional, the logits after the bias
 *   out_probs   fp32 [T, E]   optional, softmax probabilities (router stats)
 *   out_weights fp32 [T, 2], out_indices int64 [T, 2]
 *   out_positions int32 [2T]  stable slot of assignment a = 2t + k among the
 *                             expert's assignments (ascending a)
 *   out_counts  int32 [E]
 *   out_offsets int32 [2E + 2] exclusive prefix of counts (E + 1 entries),
 *                             then of max(0, counts - C) (E + 1 entries)
 *   out_perm    int32 [E, C]  assignment id in slot (e, s), -1 when empty
 *   out_overflow int32 [2T]   assignments with slot >= C, grouped by expert
 *                             then ascending a; valid entries:
 *                             out_offsets[2E + 1]
 * x, router_weight bf16; 2 <= E <= 32; dim % 32 == 0.
 * Replaces metal_route (parrot/metal_moe.py:58-81; kernel moe_route_bf16,
 * parrot/kernels/moe_bf16.metal:67-134) and the slot/scatter bookkeeping of
 * grouped_mps_experts (parrot/metal_moe.py:384-399). */
int parrot_route_bf16(const void* x, const void* router_weight, const float* logit_bias,
                      int64_t tokens, int32_t dim, int32_t experts, int32_t capacity,
                      float* out_logits, float* out_probs, float* out_weights,
                      int64_t* out_indices, int32_t* out_positions, int32_t* out_counts,
                      int32_t* out_offsets, int32_t* out_perm, int32_t* out_overflow,
                      void* workspace, size_t workspace_bytes, void* stream);

/* The router and top-2 of parrot_route_bf16 alone: out_weights fp32 [T, 2]
 * and out_indices int64 [T, 2], the same bits as parrot_route_bf16 gives, and
 * no grouping outputs (for callers whose expert launch groups the indices
 * itself, parrot_experts_gate_up_grouping_bf16).  Replaces metal_route
 * (parrot/metal_moe.py:58-81) where grouped_mps_experts then recounts the
 * slots itself (parrot/metal_moe.py:384-387). */
int parrot_route_top2_bf16(const void* x, const void* router_weight, const float* logit_bias,
                           int64_t tokens, int32_t dim, int32_t experts, float* out_weights,
                           int64_t* out_indices, void* stream);

/* parrot_route_top2_bf16 that also writes the route block table out_blocks
 * uint8 [ceil(T / 16), 64] (16-byte aligned), one row per 16 tokens: bytes
 * 0-31 the block's 32 expert ids in assignment order (assignment 2t + k;
 * 255 for the padding tokens of the last block), bytes 32-63 the block's
 * number of assignments to each expert (0 past E).  The table is what
 * parrot_experts_gate_up_grouping_blocks_bf16 groups from; T < 32768
 * (PARROT_ERR_UNSUPPORTED above).  Replaces metal_route
 * (parrot/metal_moe.py:58-81) with moe_count_assignments' per-expert counts
 * (parrot/kernels/moe_bf16.metal:650-660) taken per 16 tokens. */
int parrot_route_top2_blocks_bf16(const void* x, const void* router_weight,
                                  const float* logit_bias, int64_t tokens, int32_t dim,
                                  int32_t experts, float* out_weights, int64_t* out_indices,
                                  void* out_blocks, void* stream);

/* As parrot_route_bf16, starting from given fp32 logits [T, E] (the
 * "identical router logits" entry of the parity contract). */
int parrot_route_from_logits_f32(const float* logits, const float* logit_bias, int64_t tokens,
                                 int32_t experts, int32_t capacity, float* out_probs,
                                 float* out_weights, int64_t* out_indices,
                                 int32_t* out_positions, int32_t* out_counts,
                                 int32_t* out_offsets, int32_t* out_perm,
                                 int32_t* out_overflow, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* Grouping for caller-supplied top-2 indices int64 [T, 2], values in [0, E).
 * Outputs as parrot_route_bf16.
 * Replaces moe_count_assignments (parrot/kernels/moe_bf16.metal:650-660,
 * called from parrot/metal_moe.py:384-387). */
int parrot_group_indices(const int64_t* indices, int64_t tokens, int32_t experts,
                         int32_t capacity, int32_t* out_positions, int32_t* out_counts,
                         int32_t* out_offsets, int32_t* out_perm, int32_t* out_overflow,
                         void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes for parrot_grouped_experts_bf16. */
size_t parrot_experts_workspace_bytes(int64_t tokens, int32_t dim, int32_t hidden_dim,
                                      int32_t shared_dim);

/* The three stages of parrot_grouped_experts_bf16, for callers that schedule
 * them separately.  They share one workspace of
 * parrot_experts_workspace_bytes() bytes that carries the intermediate
 * results from stage to stage (hidden rows, then bf16 expert outputs), so
 * the same workspace must be passed to all three, in order, on one stream.
 *   gate_up: h = bf16(silu(x Wg^T) * (x Wu^T)) for every routed assignment
 *            (in-capacity slots and overflow list alike) and every token of
 *            the shared expert, one grouped MFMA launch;
 *   down:    y = bf16(w[a] * (h Wd^T)) per routed assignment, bf16(h Ws^T)
 *            per token (fp32 products and sums, one rounding each);
 *   combine: out[t] = bf16(y_shared[t] + y[2t] + y[2t+1]) in fp32 (+ addend).
 * Replace the torch.bmm / swiglu_from_gate_up_bf16 / moe_overflow_hidden_bf16
 * (gate_up), torch.bmm + overflow dot (down) and moe_gather_grouped_bf16
 * (combine) steps of grouped_mps_experts, parrot/metal_moe.py:400-415. */
int parrot_experts_gate_up_bf16(const void* x, int64_t tokens, int32_t dim, int32_t experts,
                                int32_t hidden_dim, int32_t shared_dim, int32_t capacity,
                                const int32_t* counts, const int32_t* offsets,
                                const int32_t* perm, const int32_t* overflow,
                                const void* packed_gate_up, const void* shared_gate_up,
                                void* workspace, size_t workspace_bytes, void* stream);

int parrot_experts_down_bf16(int64_t tokens, int32_t dim, int32_t experts, int32_t hidden_dim,
                             int32_t shared_dim, int32_t capacity, const int32_t* counts,
                             const int32_t* offsets, const int32_t* perm,
                             const int32_t* overflow, const float* route_weights,
                             const void* down, const void* shared_down, void* workspace,
                             size_t workspace_bytes, void* stream);

int parrot_experts_combine_bf16(int64_t tokens, int32_t dim, int32_t hidden_dim,
                                int32_t shared_dim, const void* addend, void* out,
                                void* workspace, size_t workspace_bytes, void* stream);

/* Whether the gate/up launch can group in-kernel at this shape (dim, H,
 * Hs <= 768 and the streaming tiles' plan): 1 from the top-2 indices
 * (parrot_experts_gate_up_grouping_bf16: 2T <= 2048 assignments, at most
 * 96 rows per expert on average), 2 from the route block table only
 * (parrot_experts_gate_up_grouping_blocks_bf16: T <= 4096), else 0.  The
 * block table form also takes every shape that answers 1. */
int parrot_experts_group_in_kernel(int64_t tokens, int32_t dim, int32_t experts,
                                   int32_t hidden_dim, int32_t shared_dim);

/* parrot_group_indices and parrot_experts_gate_up_bf16 in one launch: the
 * gate/up stage groups the top-2 indices int64 [T, 2] itself (stable slot
 * order, as parrot_group_indices) and writes
 *   out_counts  int32 [E], out_offsets int32 [2E + 2] (as parrot_route_bf16),
 *   out_sorted  int32 [2T]  assignment id of each routed hidden row: the
 *               expert-contiguous slot order, in-capacity slots then
 *               overflow (out_sorted[offsets[e] + s] = slot s of expert e);
 * positions / perm / overflow are not materialised.  Follow it with
 * parrot_experts_down_sorted_bf16 and parrot_experts_combine_bf16 (or its
 * depth-mix form) on the same workspace.  PARROT_ERR_UNSUPPORTED outside
 * parrot_experts_group_in_kernel's shapes.
 * Replaces moe_count_assignments (parrot/kernels/moe_bf16.metal:650-660) and
 * the gate/up steps of grouped_mps_experts (parrot/metal_moe.py:384-408). */
int parrot_experts_gate_up_grouping_bf16(const void* x, int64_t tokens, int32_t dim,
                                         int32_t experts, int32_t hidden_dim,
                                         int32_t shared_dim, int32_t capacity,
                                         const int64_t* indices, int32_t* out_counts,
                                         int32_t* out_offsets, int32_t* out_sorted,
                                         const void* packed_gate_up, const void* shared_gate_up,
                                         void* workspace, size_t workspace_bytes, void* stream);

/* parrot_experts_gate_up_grouping_bf16 grouping from the route block table
 * of parrot_route_top2_blocks_bf16 (route_blocks, 16-byte aligned) instead
 * of the indices, with the same outputs; for the shapes where
 * parrot_experts_group_in_kernel answers 1 or 2.  Replaces
 * moe_count_assignments (parrot/kernels/moe_bf16.metal:650-660) and the
 * gate/up steps of grouped_mps_experts (parrot/metal_moe.py:384-408). */
int parrot_experts_gate_up_grouping_blocks_bf16(
    const void* x, int64_t tokens, int32_t dim, int32_t experts, int32_t hidden_dim,
    int32_t shared_dim, int32_t capacity, const void* route_blocks, int32_t* out_counts,
    int32_t* out_offsets, int32_t* out_sorted, const void* packed_gate_up,
    const void* shared_gate_up, void* workspace, size_t workspace_bytes, void* stream);

/* parrot_experts_down_bf16 with the grouping written by
 * parrot_experts_gate_up_grouping_bf16 or ..._blocks_bf16 (counts,
 * offsets, sorted).
 * Replaces the down steps of grouped_mps_experts
 * (parrot/metal_moe.py:409-415). */
int parrot_experts_down_sorted_bf16(int64_t tokens, int32_t dim, int32_t experts,
                                    int32_t hidden_dim, int32_t shared_dim, int32_t capacity,
                                    const int32_t* counts, const int32_t* offsets,
                                    const int32_t* sorted, const float* route_weights,
                                    const void* down, const void* shared_down, void* workspace,
                                    size_t workspace_bytes, void* stream);

/* Routed + shared SwiGLU experts and the weighted combine:
 *   out[t] = bf16(shared(x_t) + sum_k w[t,k] * expert_{i[t,k]}(x_t))
 *   (then bf16(addend[t] + out[t]) when addend is non-NULL).
 * counts/offsets/perm/overflow/route_weights come from the routing entry
 * points above.  Weights (bf16), each matrix [N, K] stored in MFMA fragment
 * order: 1 KB blocks of 16 rows x 32 k, block (g, s) at byte
 * (g * K/32 + s) * 1024, holding row 16 g + r, k = 32 s + 8 c .. + 7 at byte
 * 16 (16 c + r) of the block:
 *   packed_gate_up [E, 2H, dim]  rows 32g..32g+15 = gate rows 16g..16g+15,
 *                                rows 32g+16..32g+31 = up rows 16g..16g+15
 *                                (before the fragment ordering)
 *   down           [E, dim, H]
 *   shared_gate_up [2Hs, dim]    interleaved the same way
 *   shared_down    [dim, Hs]
 * dim, H and Hs multiples of 64; E <= 32.
 * Replaces grouped_mps_experts (parrot/metal_moe.py:372-416): the zero-fill
 * and scatter into [E, C, dim], moe_overflow_hidden_bf16, the two torch.bmm,
 * swiglu_from_gate_up_bf16, the shared expert (_fused_shared, :145-148) and
 * moe_gather_grouped_bf16 (parrot/kernels/moe_bf16.metal:662-777). */
int parrot_grouped_experts_bf16(const void* x, int64_t tokens, int32_t dim, int32_t experts,
                                int32_t hidden_dim, int32_t shared_dim, int32_t capacity,
                                const int32_t* counts, const int32_t* offsets,
                                const int32_t* perm, const int32_t* overflow,
                                const float* route_weights, const void* packed_gate_up,
                                const void* down, const void* shared_gate_up,
                                const void* shared_down, const void* addend, void* out,
                                void* workspace, size_t workspace_bytes, void* stream);

/* Attained-peak measurements (no counterpart in the reference; they state
 * every roofline fraction against what this GPU reaches as well as against
 * the vendor peak).
 * parrot_peak_mfma_bf16: `blocks` workgroups of 4 wavefronts, each running
 * `iters` rounds of independent bf16 MFMA chains on register operands
 * (wide = 0: v_mfma_f32_16x16x32_bf16, 8 chains; wide = 1:
 * v_mfma_f32_32x32x16_bf16, 4 chains); writes one float per thread to out
 * [blocks * 256] and the flops of the launch to *flops.
 * parrot_peak_copy: copies `bytes` (a multiple of 16, 16-byte aligned) from
 * src to dst with `blocks` workgroups. */
int parrot_peak_mfma_bf16(int32_t wide, int64_t blocks, int32_t iters, float* out,
                          int64_t* flops, void* stream);
int parrot_peak_copy(const void* src, void* dst, int64_t bytes, int64_t blocks, void* stream);

/* parrot_grouped_experts_bf16 without a workspace argument and without any
 * allocation: its intermediate rows live in a static device array of
 * PARROT_STATIC_SCRATCH_BYTES bytes that every GPU the library runs on
 * holds until the process ends.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops that forbid hipMalloc).  Same arguments, semantics and
 * results as parrot_grouped_experts_bf16 (the same kernels).  Returns
 * PARROT_ERR_SCRATCH_LIMIT when parrot_experts_workspace_bytes(tokens, dim,
 * hidden_dim, shared_dim) exceeds PARROT_STATIC_SCRATCH_BYTES.  The first
 * call on a device resolves the array's address for that device (the stream
 * must belong to the calling thread's current device).  Nothing in the array
 * needs to start at zero.  All calls on one GPU share the array: calls whose
 * launches overlap on that GPU (several streams, or several threads) race
 * and must be serialised by the caller. */
int parrot_grouped_experts_static_bf16(const void* x, int64_t tokens, int32_t dim,
                                       int32_t experts, int32_t hidden_dim, int32_t shared_dim,
                                       int32_t capacity, const int32_t* counts,
                                       const int32_t* offsets, const int32_t* perm,
                                       const int32_t* overflow, const float* route_weights,
                                       const void* packed_gate_up, const void* down,
                                       const void* shared_gate_up, const void* shared_down,
                                       const void* addend, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PARROT_HIP_H */
