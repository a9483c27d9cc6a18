/*
 * Router logits in the fixed fp32 order the HIP route kernel uses
 * (TEST INFRASTRUCTURE: only tests/, smoke() and bench.py's cpu_baseline
 * leg load this library).
 *
 * Restates router_logits = x @ W_gate^T of QuantFused*MoEBlock
 * (gemq/inference/moe_block.py:790, :1020, :243; fp32 gate :549 / :591) with
 * the summation order pinned so that GPU and CPU agree bit for bit:
 *
 *   chain l (l = 0..63) = fmaf over k = 512*i + 8*l + j  (i ascending, then
 *                         j = 0..7 ascending, k < H), starting from +0.0f
 *   then for o = 32, 16, 8, 4, 2, 1:  v[l] <- v[l] + v[l ^ o]
 *   logit = v[0]
 *
 * Inputs are fp32 (fp16 / bf16 values widen exactly).  Built with
 * -ffp-contract=off so the compiler adds no fusion of its own; fmaf() is the
 * correctly rounded C99 fused multiply-add.
 */
#include <math.h>
#include <stdint.h>

static float dot_fixed(const float *x, const float *w, int H) {
  float v[64];
  for (int l = 0; l < 64; ++l) v[l] = 0.0f;
  for (int base = 0; base < H; base += 512)
    for (int l = 0; l < 64; ++l)
      for (int j = 0; j < 8; ++j) {
        int k = base + 8 * l + j;
        if (k < H) v[l] = fmaf(x[k], w[k], v[l]);
      }
  for (int o = 32; o >= 1; o >>= 1) {
    float n[64];
    for (int l = 0; l < 64; ++l) n[l] = v[l] + v[l ^ o];
    for (int l = 0; l < 64; ++l) v[l] = n[l];
  }
  return v[0];
}

void oracle_router_logits(const float *x, const float *w, int64_t T, int H,
                          int E, float *out) {
  for (int64_t t = 0; t < T; ++t)
    for (int e = 0; e < E; ++e)
      out[t * E + e] = dot_fixed(x + t * H, w + (int64_t)e * H, H);
}
