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
  void *logits;      // may be null
  int logits_dtype;  // rounding target of the logits
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

template <int MAXCH, int TT, int EREG>
__global__ __launch_bounds__(256) void route_kernel(RouteArgs a) {
  const int lane = lane_id();
  const int64_t wave = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t t0 = wave * TT;
  if (t0 >= a.T) return;

  float xr[TT][MAXCH][8];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int i = 0; i < MAXCH; ++i) {
      int k0 = 512 * i + 8 * lane;
      if (t0 + tt < a.T && k0 < a.H) {
        load8(a.x, a.x_dtype, (t0 + tt) * a.H + k0, xr[tt][i]);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) xr[tt][i][j] = 0.f;
      }
    }

  float lg[TT][EREG];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int r = 0; r < EREG; ++r) lg[tt][r] = 0.f;

  for (int e = 0; e < a.E; ++e) {
    float v[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) v[tt] = 0.f;
#pragma unroll
    for (int i = 0; i < MAXCH; ++i) {
      int k0 = 512 * i + 8 * lane;
      if (k0 < a.H) {
        float wr[8];
        load8(a.wg, a.wg_dtype, int64_t(e) * a.H + k0, wr);
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
#pragma unroll
          for (int j = 0; j < 8; ++j) v[tt] = __builtin_fmaf(xr[tt][i][j], wr[j], v[tt]);
      }
    }
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      float s = v[tt];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) s = s + __shfl_xor(s, o);
      if (a.bias) s = s + a.bias[e];
      s = round_logit(s, a.logits_dtype);
      if ((e & 63) == lane) lg[tt][e >> 6] = s;
    }
  }

#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    const int64_t t = t0 + tt;
    if (t >= a.T) break;
    if (a.logits) {
#pragma unroll
      for (int r = 0; r < EREG; ++r) {
        int e = 64 * r + lane;
        if (e < a.E) store_logit(a.logits, a.logits_dtype, t * a.E + e, lg[tt][r]);
      }
    }
    select_topk<EREG>(lg[tt], a.E, a.k, a.norm, t, a.idx, a.w);
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

template <int MAXCH, int TT>
static void launch_route_e(const RouteArgs &a, int ereg, hipStream_t s) {
  int64_t waves = cdiv(a.T, TT);
  dim3 grid(unsigned(cdiv(waves, 4))), block(256);
  switch (ereg) {
    case 1: route_kernel<MAXCH, TT, 1><<<grid, block, 0, s>>>(a); break;
    case 2: route_kernel<MAXCH, TT, 2><<<grid, block, 0, s>>>(a); break;
    case 4: route_kernel<MAXCH, TT, 4><<<grid, block, 0, s>>>(a); break;
    default: route_kernel<MAXCH, TT, 8><<<grid, block, 0, s>>>(a); break;
  }
}

static int ereg_for(int E) { return E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : 8; }

static bool valid_dtype(int d) { return d == MOEQ_F16 || d == MOEQ_BF16 || d == MOEQ_F32; }

}  // namespace moeq

using namespace moeq;

extern "C" int moeq_route(const void *x, int x_dtype, int64_t T, int H,
                          const void *gate_w, int gate_dtype, const float *logit_bias,
                          int E, int top_k, int norm_topk, void *logits_out,
                          int32_t *idx_out, float *w_out, void *stream) {
  if (!x || !gate_w || !idx_out || !w_out) return fail(MOEQ_ERR_INVALID, "route: null pointer");
  if (!valid_dtype(x_dtype) || !valid_dtype(gate_dtype))
    return fail(MOEQ_ERR_INVALID, "route: dtype x=%d gate=%d", x_dtype, gate_dtype);
  if (T <= 0) return fail(MOEQ_ERR_INVALID, "route: T=%lld", (long long)T);
  if (H <= 0 || H % 8) return fail(MOEQ_ERR_INVALID, "route: hidden=%d must be a positive multiple of 8", H);
  if (H > 4096) return fail(MOEQ_ERR_UNSUPPORTED, "route: hidden=%d > 4096", H);
  if (E <= 0 || E > 512) return fail(MOEQ_ERR_UNSUPPORTED, "route: n_experts=%d not in 1..512", E);
  if (top_k <= 0 || top_k > E || top_k > kMaxTopK)
    return fail(MOEQ_ERR_INVALID, "route: top_k=%d must be in 1..min(n_experts=%d, %d)", top_k, E, kMaxTopK);
  RouteArgs a{x, x_dtype, T, H, gate_w, gate_dtype, logit_bias, E, top_k, norm_topk ? 1 : 0,
              logits_out, gate_dtype == MOEQ_F32 ? MOEQ_F32 : x_dtype, idx_out, w_out};
  hipStream_t s = as_stream(stream);
  int ereg = ereg_for(E);
  if (H <= 512)
    launch_route_e<1, 8>(a, ereg, s);
  else if (H <= 1024)
    launch_route_e<2, 8>(a, ereg, s);
  else if (H <= 2048)
    launch_route_e<4, 4>(a, ereg, s);
  else
    launch_route_e<8, 2>(a, ereg, s);
  return check_launch("route");
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
  dim3 grid(unsigned(cdiv(T, 4))), block(256);
  hipStream_t s = as_stream(stream);
  int n = norm_topk ? 1 : 0;
  switch (ereg_for(E)) {
    case 1: topk_from_logits_kernel<1><<<grid, block, 0, s>>>(logits, dtype, T, E, top_k, n, idx_out, w_out); break;
    case 2: topk_from_logits_kernel<2><<<grid, block, 0, s>>>(logits, dtype, T, E, top_k, n, idx_out, w_out); break;
    case 4: topk_from_logits_kernel<4><<<grid, block, 0, s>>>(logits, dtype, T, E, top_k, n, idx_out, w_out); break;
    default: topk_from_logits_kernel<8><<<grid, block, 0, s>>>(logits, dtype, T, E, top_k, n, idx_out, w_out); break;
  }
  return check_launch("route_from_logits");
}
