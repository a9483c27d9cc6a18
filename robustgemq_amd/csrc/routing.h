// Router helpers shared by the logits / top-k kernels (route.hip) and the
// single-work-group top-k + permute kernel (permute.hip).
#pragma once

#include <float.h>

#include "common.h"

namespace moeq {

constexpr int kMaxTopK = 16;

struct RouteArgs {
  const void *x;
  int x_dtype;
  int64_t T;
  int H;
  const void *wg;
  int wg_dtype;
  const float *bias;  // may be null
  int E, k, norm;
  void *logits;      // rounded logits [T, E]
  int logits_dtype;  // rounding target of the logits
  int store_dtype;   // element type of `logits` (logits_dtype, or F32 scratch)
  int32_t *idx;
  float *w;
  uint16_t *x16 = nullptr;  // optional [T, H] fp16 copy of x, written by the expert-0 waves
  // MOEQ_F32: rank the logits, fp32 softmax weights (every family's
  // forward_n_tokens).  MOEQ_F16 / MOEQ_BF16: softmax probabilities rounded
  // to that type are ranked and renormalised in it (Mixtral's
  // forward_one_token); only the one-token kernel (route1) honours it.
  int prob_dtype = MOEQ_F32;
};

__device__ __forceinline__ float round_logit(float v, int dtype) {
  if (dtype == MOEQ_F16) return (float)(f16)v;
  if (dtype == MOEQ_BF16) return bf16_to_f32(f32_to_bf16(v));
  return v;
}

__device__ __forceinline__ void store_logit(void *p, int dtype, int64_t i, float v) {
  if (dtype == MOEQ_F32)
    static_cast<float *>(p)[i] = v;
  else if (dtype == MOEQ_BF16)
    static_cast<uint16_t *>(p)[i] = f32_to_bf16(v);
  else
    static_cast<uint16_t *>(p)[i] = f32_to_f16_bits(v);
}

// Loads 8 consecutive elements starting at element i and widens them to fp32.
__device__ __forceinline__ void load8(const void *p, int dtype, int64_t i, float (&o)[8]) {
  if (dtype == MOEQ_F32) {
    const float4 *q = reinterpret_cast<const float4 *>(static_cast<const float *>(p) + i);
    float4 a = q[0], b = q[1];
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  } else {
    uint4 u = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(p) + i);
    uint32_t ws[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint16_t lo = uint16_t(ws[j] & 0xffffu), hi = uint16_t(ws[j] >> 16);
      if (dtype == MOEQ_BF16) {
        o[2 * j] = bf16_to_f32(lo);
        o[2 * j + 1] = bf16_to_f32(hi);
      } else {
        o[2 * j] = f16_bits_to_f32(lo);
        o[2 * j + 1] = f16_bits_to_f32(hi);
      }
    }
  }
}

// Maximum over the 64 lanes, returned in every lane (no NaN inputs): lane
// pairs (xor 1, xor 2), the two quads of each half-row (half-row mirror), the
// two halves of each row (row mirror), then row pairs and wave halves by
// swapping them between two copies (v_permlane16/32_swap).
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false)));
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Sum over the 64 lanes, the same value in every lane: the pairing of
// wave_max, each level adding two partial sums (commutative, so both lanes
// of a pair hold the identical result).
__device__ __forceinline__ float wave_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false));
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Top-k of the logits held by one wave (expert e = 64 r + lane in vals[r]),
// ranked by value with ties to the lower index (NaN ranks last); softmax
// weights over all E experts; optional renormalisation over the selected k.
// topk_ranks leaves each expert's rank and routing weight in the lane that
// holds it; select_topk writes row t.  The k selected experts are found by k
// wave-wide argmax rounds (a DPP / permlane reduction each), so the cost
// grows with k, not with E, and no register is indexed dynamically.  Every
// round places one expert (k <= E), so all k slots of the row are written.
//
// prob_dtype F16 / BF16 restates a router that runs softmax on a 16-bit
// tensor (F.softmax computes in fp32 and rounds its output), ranks those
// rounded probabilities with torch.topk and renormalises in the same type
// (gemq/inference/moe_block.py:280-283): p = rnd(exp(l - max) / sum),
// ranked by p (equal p: lower index first), w = rnd(p / rnd(sum_sel p)).
// The selected sum is exact in fp32 for k = 2 (two 16-bit values), so its
// order does not matter there.
template <int EREG>
__device__ void topk_ranks(float (&vals)[EREG], int E, int k, int norm, int (&rank)[EREG],
                           float (&wsel)[EREG], int prob_dtype = MOEQ_F32) {
  const int lane = lane_id();
#pragma unroll
  for (int r = 0; r < EREG; ++r) {
    const int e = 64 * r + lane;
    if (e >= E || vals[r] != vals[r]) vals[r] = -INFINITY;  // NaN ranks last
  }
  if (prob_dtype != MOEQ_F32) {
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < EREG; ++r) mx = fmaxf(mx, vals[r]);
    mx = wave_max(mx);
    float den = 0.f;
#pragma unroll
    for (int r = 0; r < EREG; ++r)
      if (64 * r + lane < E) den += expf(vals[r] - mx);
    den = wave_sum(den);
#pragma unroll
    for (int r = 0; r < EREG; ++r)
      vals[r] = 64 * r + lane < E ? round_logit(expf(vals[r] - mx) / den, prob_dtype) : -INFINITY;
#pragma unroll
    for (int r = 0; r < EREG; ++r)
      if (vals[r] != vals[r]) vals[r] = -INFINITY;  // every logit -inf: NaN probabilities, rank last
  }
  // k rounds of a wave-wide argmax over the experts not yet taken: round s
  // takes the largest value, the lowest expert index among equal ones (the
  // order of a stable descending sort), and gives it rank s; the others keep
  // rank k.  +0 and -0 compare equal, as in the sort.
#pragma unroll
  for (int r = 0; r < EREG; ++r) rank[r] = k;
  float m = -INFINITY;  // the top value
  for (int s = 0; s < k; ++s) {
    float c = -INFINITY;
#pragma unroll
    for (int r = 0; r < EREG; ++r)
      if (rank[r] == k && 64 * r + lane < E) c = fmaxf(c, vals[r]);
    const float top = wave_max(c);
    if (s == 0) m = top;
    bool placed = false;
#pragma unroll
    for (int r = 0; r < EREG; ++r) {
      const uint64_t b = __builtin_amdgcn_ballot_w64(rank[r] == k && 64 * r + lane < E && vals[r] == top);
      if (!placed && b != 0) {
        placed = true;
        if (lane == __builtin_ctzll(b)) rank[r] = s;
      }
    }
  }
  if (prob_dtype != MOEQ_F32) {
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < EREG; ++r)
      if (64 * r + lane < E && rank[r] < k) psum += vals[r];
    psum = wave_sum(psum);
    const float s = round_logit(psum, prob_dtype);
#pragma unroll
    for (int r = 0; r < EREG; ++r) wsel[r] = norm ? round_logit(vals[r] / s, prob_dtype) : vals[r];
    return;
  }
  // m is the top value (sel 0) unless every logit is -inf / NaN
  float den = 0.f;
#pragma unroll
  for (int r = 0; r < EREG; ++r)
    if (64 * r + lane < E) den += __expf(vals[r] - m);
  den = wave_sum(den);
  float p[EREG];
  float psum = 0.f;
#pragma unroll
  for (int r = 0; r < EREG; ++r) {
    p[r] = __expf(vals[r] - m) / den;
    if (64 * r + lane < E && rank[r] < k) psum += p[r];
  }
  psum = wave_sum(psum);
#pragma unroll
  for (int r = 0; r < EREG; ++r) wsel[r] = norm ? p[r] / psum : p[r];
}

template <int EREG>
__device__ void select_topk(float (&vals)[EREG], int E, int k, int norm,
                            int64_t t, int32_t *idx_out, float *w_out) {
  const int lane = lane_id();
  int rank[EREG];
  float wsel[EREG];
  topk_ranks<EREG>(vals, E, k, norm, rank, wsel);
#pragma unroll
  for (int r = 0; r < EREG; ++r) {
    const int e = 64 * r + lane;
    if (e < E && rank[r] < k) {
      idx_out[t * k + rank[r]] = e;
      w_out[t * k + rank[r]] = wsel[r];
    }
  }
}

// Logits of a TT-token x EE-expert tile per wave.  Lane l runs the TT*EE
// fused multiply-add chains over its k set (k = 512 i + 8 l + j), then every
// chain is reduced with the xor butterfly; the order per logit is exactly the
// one documented at the top of this file whatever the tiling.
template <int TT, int EE, int MAXCH>
__device__ void logit_tile(const RouteArgs &a, int64_t t0, int e0) {
  const int lane = lane_id();
  if (t0 >= a.T) return;
  float ch[TT][EE];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int ee = 0; ee < EE; ++ee) ch[tt][ee] = 0.f;
  if constexpr (TT == 1 && EE == 1) {
    // one logit per wave (decode): every k step's loads are issued before
    // the first multiply-add, so the wave waits for memory once.  Lanes past
    // H load the row's last 8 values and skip the multiply-adds.
    const int64_t xr = min(t0, a.T - 1) * a.H;
    const int64_t wr = int64_t(min(e0, a.E - 1)) * a.H;
    float xv[MAXCH][8], wv[MAXCH][8];
#pragma unroll
    for (int i = 0; i < MAXCH; ++i) {
      const int kc = min(512 * i + 8 * lane, a.H - 8);
      load8(a.x, a.x_dtype, xr + kc, xv[i]);
      load8(a.wg, a.wg_dtype, wr + kc, wv[i]);
    }
#pragma unroll
    for (int i = 0; i < MAXCH; ++i) {
      const int k0 = 512 * i + 8 * lane;
      if (k0 < a.H) {
        if (a.x16 && e0 == 0) {  // the activations the expert GEMMs read, converted once
          uint32_t h[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            h[j] = uint32_t(f32_to_f16_bits(xv[i][2 * j])) | (uint32_t(f32_to_f16_bits(xv[i][2 * j + 1])) << 16);
          *reinterpret_cast<uint4 *>(a.x16 + t0 * a.H + k0) = (uint4){h[0], h[1], h[2], h[3]};
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) ch[0][0] = __builtin_fmaf(xv[i][j], wv[i][j], ch[0][0]);
      }
    }
  } else
#pragma unroll
  for (int i = 0; i < MAXCH; ++i) {
    const int k0 = 512 * i + 8 * lane;
    if (k0 < a.H) {
      float xv[TT][8], wv[EE][8];
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        if (t0 + tt < a.T) {
          load8(a.x, a.x_dtype, (t0 + tt) * a.H + k0, xv[tt]);
          if (a.x16 && e0 == 0) {  // the activations the expert GEMMs read, converted once
            uint32_t h[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
              h[j] = uint32_t(f32_to_f16_bits(xv[tt][2 * j])) | (uint32_t(f32_to_f16_bits(xv[tt][2 * j + 1])) << 16);
            *reinterpret_cast<uint4 *>(a.x16 + (t0 + tt) * a.H + k0) = (uint4){h[0], h[1], h[2], h[3]};
          }
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) xv[tt][j] = 0.f;
        }
      }
#pragma unroll
      for (int ee = 0; ee < EE; ++ee) {
        if (e0 + ee < a.E) {
          load8(a.wg, a.wg_dtype, int64_t(e0 + ee) * a.H + k0, wv[ee]);
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) wv[ee][j] = 0.f;
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
#pragma unroll
          for (int ee = 0; ee < EE; ++ee) ch[tt][ee] = __builtin_fmaf(xv[tt][j], wv[ee][j], ch[tt][ee]);
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1)
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int ee = 0; ee < EE; ++ee) ch[tt][ee] = ch[tt][ee] + __shfl_xor(ch[tt][ee], o);
  // every lane now holds all TT*EE logits; lane j stores logit j
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int ee = 0; ee < EE; ++ee) {
      const int64_t t = t0 + tt;
      const int e = e0 + ee;
      if (lane == tt * EE + ee && t < a.T && e < a.E) {
        float v = ch[tt][ee];
        if (a.bias) v = v + a.bias[e];
        store_logit(a.logits, a.store_dtype, t * a.E + e, round_logit(v, a.logits_dtype));
      }
    }
}

__host__ __device__ inline int ereg_for(int E) { return E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : 8; }

// Logits of every (token, expert) pair (rounded as RouteArgs asks), without
// the selection; defined in route.hip.
int launch_route_logits(const RouteArgs &a, hipStream_t s);

// Logits (stored only when a.logits is set) and top-k in one launch, for
// T * E > 16384 and the dtype pairs (x, gate) f16/f16, f16/f32, bf16/bf16,
// bf16/f32, f32/f32; returns false without launching otherwise.  Needs
// H % 8 == 0 and H <= 4096, E <= 512 (route.hip).
bool launch_logits_topk(const RouteArgs &a, hipStream_t s);

// Top-k of T rows of logits followed by the token -> expert permutation, in
// one work-group; valid when T * k <= 4096, E + n_shared <= 256 and
// k <= kMaxTopK (permute.hip).
int launch_topk_permute(const void *logits, int dtype, int64_t T, int E, int k, int norm, int32_t *idx,
                        float *w, int n_shared, int bm, int32_t *counts, int32_t *offsets,
                        int32_t *row_token, int32_t *row_pair, int32_t *inv_perm, int32_t *tiles,
                        int32_t *n_tiles, hipStream_t s);
bool topk_permute_fits(int64_t T, int k, int E, int n_shared);

// Outputs of the token -> expert permutation (moeq_permute's arrays).
struct PermOut {
  int n_shared, max_tiles;
  int32_t *counts, *offsets, *row_token, *row_pair, *inv_perm, *tiles, *n_tiles;
};

// One token (decode): logits, top-k and the permutation in one work-group.
// With a single token every selected expert holds one row, so the stable
// grouping is the selected experts in id order, one 1-row tile each, then
// the shared experts' rows: exactly moeq_permute's output for T = 1.  Needs
// T == 1, E <= 256, k <= kMaxTopK, H % 8 == 0, H <= 4096 and the dtype pairs
// (x, gate) f16/f16, f16/f32, bf16/bf16, bf16/f32; returns false without
// launching otherwise (route.hip).
bool launch_route1(const RouteArgs &a, const PermOut &po, hipStream_t s);

// One token's top-k and grouping as route1_kernel writes them, from E logits
// already in memory (`dtype`), in one wave (route.hip).
int launch_topk1(const void *logits, int dtype, const RouteArgs &a, const PermOut &po, hipStream_t s);

}  // namespace moeq
