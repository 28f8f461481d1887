/*
 * TEST INFRASTRUCTURE ONLY -- the CPU oracle for routing and grouping.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, as the checker; the product path never does.
 *
 * Plain-C restatement of the reference's routing/grouping semantics
 * (paths relative to the jkpdino/parrot-h200-worker checkout):
 *   - softmax top-2 with renormalised weights: parrot/model.py:520-527
 *   - selection by strict '>' in expert order (ties -> lower index):
 *     parrot/kernels/moe_bf16.metal:104-118
 *   - slot order of an expert's assignments = ascending assignment index
 *     a = 2t + k, the order torch.where(indices == e) yields:
 *     parrot/model.py:547-551
 *   - capacity C = max(8, roundup8(ceil(2 * 2T / E))): parrot/metal_moe.py:388-391
 *   - an assignment with slot >= C takes the overflow path and is never
 *     dropped: parrot/metal_moe.py:400-416, moe_bf16.metal:698-777
 * Build: make -C oracle  (writes oracle/build/liboracle.so)
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

int32_t oracle_capacity(int64_t tokens, int32_t experts) {
  int64_t assignments = 2 * tokens;
  int64_t per = (2 * assignments + experts - 1) / experts;
  int64_t c = (per + 7) / 8 * 8;
  return (int32_t)(c < 8 ? 8 : c);
}

/* logits [T, E] (+ bias [E] when non-NULL) -> indices [T, 2], weights [T, 2],
 * probs [T, E] (when non-NULL).  Probabilities are fp32 softmax; weights are
 * p_k / (p_first + p_second). */
void oracle_top2(const float* logits, const float* bias, int64_t tokens, int32_t experts,
                 int64_t* indices, float* weights, float* probs) {
  float row[64];
  for (int64_t t = 0; t < tokens; ++t) {
    for (int32_t e = 0; e < experts; ++e)
      row[e] = logits[t * experts + e] + (bias ? bias[e] : 0.0f);
    int32_t first = 0, second = 1;
    if (row[1] > row[0]) { first = 1; second = 0; }
    for (int32_t e = 2; e < experts; ++e) {
      if (row[e] > row[first]) { second = first; first = e; }
      else if (row[e] > row[second]) { second = e; }
    }
    float mx = row[first];
    float denom = 0.0f;
    for (int32_t e = 0; e < experts; ++e) denom += expf(row[e] - mx);
    float p1 = expf(row[first] - mx) / denom;
    float p2 = expf(row[second] - mx) / denom;
    indices[2 * t] = first;
    indices[2 * t + 1] = second;
    weights[2 * t] = p1 / (p1 + p2);
    weights[2 * t + 1] = p2 / (p1 + p2);
    if (probs)
      for (int32_t e = 0; e < experts; ++e) probs[t * experts + e] = expf(row[e] - mx) / denom;
  }
}

/* positions[a] = #{a' < a : indices[a'] == indices[a]}; counts[e]. */
void oracle_positions(const int64_t* indices, int64_t assignments, int32_t experts,
                      int32_t* positions, int32_t* counts) {
  memset(counts, 0, sizeof(int32_t) * (size_t)experts);
  for (int64_t a = 0; a < assignments; ++a) positions[a] = counts[indices[a]]++;
}

/* perm [E, C]: assignment in slot s < C of expert e, -1 when empty.
 * overflow: assignments with slot >= C ordered by expert, then ascending a.
 * offsets [2E + 2]: exclusive prefix of counts (E + 1 entries) followed by
 * the exclusive prefix of max(0, counts - C) (E + 1 entries). */
void oracle_group(const int64_t* indices, const int32_t* positions, const int32_t* counts,
                  int64_t assignments, int32_t experts, int32_t capacity, int32_t* perm,
                  int32_t* overflow, int32_t* offsets) {
  int32_t o = 0, v = 0;
  for (int32_t e = 0; e < experts; ++e) {
    offsets[e] = o;
    offsets[experts + 1 + e] = v;
    o += counts[e];
    v += counts[e] > capacity ? counts[e] - capacity : 0;
  }
  offsets[experts] = o;
  offsets[2 * experts + 1] = v;
  for (int64_t i = 0; i < (int64_t)experts * capacity; ++i) perm[i] = -1;
  for (int64_t a = 0; a < assignments; ++a) {
    int32_t e = (int32_t)indices[a];
    int32_t p = positions[a];
    if (p < capacity) perm[(int64_t)e * capacity + p] = (int32_t)a;
    else overflow[offsets[experts + 1 + e] + p - capacity] = (int32_t)a;
  }
}
