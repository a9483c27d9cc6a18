// Router: logits in a pinned fp32 order, softmax, top-k, renormalisation.
//
// Logit (t, e) = butterfly over 64 lanes of per-lane fused multiply-add
// chains; lane l covers k = 512 i + 8 l + j (i ascending, then j = 0..7).
// The xor butterfly (o = 32 .. 1, v <- v + v[l ^ o]) gives every lane the
// same value because fp32 addition is commutative.  oracle/router_exact.c
// replays exactly this order, so routing is bit-reproducible on the CPU.
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

// Top-k of the logits held by one wave (expert e = 64 r + lane in vals[r]),
// ranked by value with ties to the lower index; softmax weights over all E
// experts; optional renormalisation over the selected k.  Writes row t.
template <int EREG>
__device__ void select_topk(float (&vals)[EREG], int E, int k, int norm,
                            int64_t t, int32_t *idx_out, float *w_out) {
  const int lane = lane_id();
  bool avail[EREG];
#pragma unroll
  for (int r = 0; r < EREG; ++r) {
    int e = 64 * r + lane;
    avail[r] = e < E;
    if (!avail[r] || vals[r] != vals[r]) vals[r] = -INFINITY;  // NaN ranks last
  }
  int sel_i[kMaxTopK];
  float sel_v[kMaxTopK];
  for (int s = 0; s < k; ++s) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int r = 0; r < EREG; ++r) {
      int e = 64 * r + lane;
      if (avail[r] && (vals[r] > bv || (vals[r] == bv && e < bi))) {
        bv = vals[r];
        bi = e;
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      float ov = __shfl_xor(bv, o);
      int oi = __shfl_xor(bi, o);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    sel_i[s] = bi;
    sel_v[s] = bv;
#pragma unroll
    for (int r = 0; r < EREG; ++r)
      if (64 * r + lane == bi) avail[r] = false;
  }
  const float m = sel_v[0];
  float den = 0.f;
#pragma unroll
  for (int r = 0; r < EREG; ++r)
    if (64 * r + lane < E) den += __expf(vals[r] - m);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) den += __shfl_xor(den, o);
  float p[kMaxTopK];
  float psum = 0.f;
  for (int s = 0; s < k; ++s) {
    p[s] = __expf(sel_v[s] - m) / den;
    psum += p[s];
  }
  for (int s = 0; s < k; ++s) {
    if (lane == s) {
      idx_out[t * k + s] = sel_i[s];
      w_out[t * k + s] = norm ? p[s] / psum : p[s];
    }
  }
}

// Logits of a TT-token x EE-expert tile per wave.  Lane l runs the TT*EE
// fused multiply-add chains over its k set (k = 512 i + 8 l + j), then every
// chain is reduced with the xor butterfly; the order per logit is exactly the
// one documented at the top of this file whatever the tiling.
template <int TT, int EE, int MAXCH>
__global__ __launch_bounds__(256) void logits_kernel(RouteArgs a, int n_et) {
  const int lane = lane_id();
  const int64_t wave = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t tt_tile = wave / n_et;
  const int e0 = int(wave % n_et) * EE;
  const int64_t t0 = tt_tile * TT;
  if (t0 >= a.T) return;
  float ch[TT][EE];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int ee = 0; ee < EE; ++ee) ch[tt][ee] = 0.f;
#pragma unroll
  for (int i = 0; i < MAXCH; ++i) {
    const int k0 = 512 * i + 8 * lane;
    if (k0 < a.H) {
      float xv[TT][8], wv[EE][8];
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        if (t0 + tt < a.T) {
          load8(a.x, a.x_dtype, (t0 + tt) * a.H + k0, xv[tt]);
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

template <int EREG>
__global__ __launch_bounds__(256) void topk_from_logits_kernel(
    const void *logits, int dtype, int64_t T, int E, int k, int norm,
    int32_t *idx, float *w) {
  const int lane = lane_id();
  const int64_t t = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  float vals[EREG];
#pragma unroll
  for (int r = 0; r < EREG; ++r) {
    int e = 64 * r + lane;
    vals[r] = e < E ? load_as_f32(logits, dtype, t * E + e) : -INFINITY;
  }
  select_topk<EREG>(vals, E, k, norm, t, idx, w);
}

static int ereg_for(int E) { return E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : 8; }

template <int TT, int EE>
static void launch_logits(const RouteArgs &a, int maxch, hipStream_t s) {
  const int n_et = int(cdiv(a.E, EE));
  const int64_t waves = cdiv(a.T, TT) * n_et;
  dim3 grid(unsigned(cdiv(waves, 4))), block(256);
  switch (maxch) {
    case 1: logits_kernel<TT, EE, 1><<<grid, block, 0, s>>>(a, n_et); break;
    case 2: logits_kernel<TT, EE, 2><<<grid, block, 0, s>>>(a, n_et); break;
    case 4: logits_kernel<TT, EE, 4><<<grid, block, 0, s>>>(a, n_et); break;
    default: logits_kernel<TT, EE, 8><<<grid, block, 0, s>>>(a, n_et); break;
  }
}

static int launch_topk(const void *logits, int dtype, int64_t T, int E, int k, int norm, int32_t *idx,
                       float *w, hipStream_t s) {
  dim3 grid(unsigned(cdiv(T, 4))), block(256);
  switch (ereg_for(E)) {
    case 1: topk_from_logits_kernel<1><<<grid, block, 0, s>>>(logits, dtype, T, E, k, norm, idx, w); break;
    case 2: topk_from_logits_kernel<2><<<grid, block, 0, s>>>(logits, dtype, T, E, k, norm, idx, w); break;
    case 4: topk_from_logits_kernel<4><<<grid, block, 0, s>>>(logits, dtype, T, E, k, norm, idx, w); break;
    default: topk_from_logits_kernel<8><<<grid, block, 0, s>>>(logits, dtype, T, E, k, norm, idx, w); break;
  }
  return check_launch("route/topk");
}


static bool valid_dtype(int d) { return d == MOEQ_F16 || d == MOEQ_BF16 || d == MOEQ_F32; }

}  // namespace moeq

using namespace moeq;

extern "C" size_t moeq_route_workspace_size(int64_t T, int E) {
  if (T <= 0 || E <= 0) return 0;
  return align256(size_t(T) * size_t(E) * sizeof(float));
}

extern "C" int moeq_route(const void *x, int x_dtype, int64_t T, int H,
                          const void *gate_w, int gate_dtype, const float *logit_bias,
                          int E, int top_k, int norm_topk, void *logits_out,
                          int32_t *idx_out, float *w_out, void *ws, size_t ws_bytes,
                          void *stream) {
  if (!x || !gate_w || !idx_out || !w_out) return fail(MOEQ_ERR_INVALID, "route: null pointer");
  if (!valid_dtype(x_dtype) || !valid_dtype(gate_dtype))
    return fail(MOEQ_ERR_INVALID, "route: dtype x=%d gate=%d", x_dtype, gate_dtype);
  if (T <= 0) return fail(MOEQ_ERR_INVALID, "route: T=%lld", (long long)T);
  if (H <= 0 || H % 8) return fail(MOEQ_ERR_INVALID, "route: hidden=%d must be a positive multiple of 8", H);
  if (H > 4096) return fail(MOEQ_ERR_UNSUPPORTED, "route: hidden=%d > 4096", H);
  if (E <= 0 || E > 512) return fail(MOEQ_ERR_UNSUPPORTED, "route: n_experts=%d not in 1..512", E);
  if (top_k <= 0 || top_k > E || top_k > kMaxTopK)
    return fail(MOEQ_ERR_INVALID, "route: top_k=%d must be in 1..min(n_experts=%d, %d)", top_k, E, kMaxTopK);
  const int ldt = gate_dtype == MOEQ_F32 ? MOEQ_F32 : x_dtype;
  void *lg = logits_out;
  int lg_dt = ldt;
  if (!lg) {
    if (!ws || ws_bytes < moeq_route_workspace_size(T, E))
      return fail(MOEQ_ERR_WORKSPACE, "route: logits_out is NULL and workspace %zu < %zu bytes", ws_bytes,
                  moeq_route_workspace_size(T, E));
    lg = ws;  // rounded logits kept as fp32 (exact)
    lg_dt = MOEQ_F32;
  }
  RouteArgs a{x, x_dtype, T, H, gate_w, gate_dtype, logit_bias, E, top_k, norm_topk ? 1 : 0,
              lg, ldt, lg_dt, idx_out, w_out};
  hipStream_t s = as_stream(stream);
  const int maxch = H <= 512 ? 1 : H <= 1024 ? 2 : H <= 2048 ? 4 : 8;
  if (T <= 2)
    launch_logits<1, 4>(a, maxch, s);
  else
    launch_logits<4, 4>(a, maxch, s);
  int rc = check_launch("route/logits");
  if (rc) return rc;
  // the selection reads the rounded logits (stored as ldt, or exactly as fp32)
  return launch_topk(lg, lg_dt, T, E, top_k, norm_topk ? 1 : 0, idx_out, w_out, s);
}

extern "C" int moeq_route_from_logits(const void *logits, int dtype, int64_t T,
                                      int E, int top_k, int norm_topk,
                                      int32_t *idx_out, float *w_out, void *stream) {
  if (!logits || !idx_out || !w_out) return fail(MOEQ_ERR_INVALID, "route_from_logits: null pointer");
  if (!valid_dtype(dtype)) return fail(MOEQ_ERR_INVALID, "route_from_logits: dtype=%d", dtype);
  if (T <= 0) return fail(MOEQ_ERR_INVALID, "route_from_logits: T=%lld", (long long)T);
  if (E <= 0 || E > 512) return fail(MOEQ_ERR_UNSUPPORTED, "route_from_logits: n_experts=%d not in 1..512", E);
  if (top_k <= 0 || top_k > E || top_k > kMaxTopK)
    return fail(MOEQ_ERR_INVALID, "route_from_logits: top_k=%d must be in 1..min(n_experts=%d, %d)", top_k, E, kMaxTopK);
  return launch_topk(logits, dtype, T, E, top_k, norm_topk ? 1 : 0, idx_out, w_out, as_stream(stream));
}
