// Router: logits in a pinned fp32 order, softmax, top-k, renormalisation.
//
// Logit (t, e) = butterfly over 64 lanes of per-lane fused multiply-add
// chains; lane l covers k = 512 i + 8 l + j (i ascending, then j = 0..7).
// The xor butterfly (o = 32 .. 1, v <- v + v[l ^ o]) gives every lane the
// same value because fp32 addition is commutative.  oracle/router_exact.c
// replays exactly this order, so routing is bit-reproducible on the CPU.
#include "routing.h"

namespace moeq {

template <int TT, int EE, int MAXCH>
__global__ __launch_bounds__(256) void logits_kernel(RouteArgs a, int n_et) {
  const int64_t wave = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  logit_tile<TT, EE, MAXCH>(a, (wave / n_et) * TT, int(wave % n_et) * EE);
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


// Small batches take one logit per wave (up to 16384 waves) so enough waves
// read the router weights at once; larger ones share loads over 4 x 4 tiles.
// The summation order of a logit is the same for every tiling.
int launch_route_logits(const RouteArgs &a, hipStream_t s) {
  const int maxch = a.H <= 512 ? 1 : a.H <= 1024 ? 2 : a.H <= 2048 ? 4 : 8;
  if (a.T * a.E <= 16384)
    launch_logits<1, 1>(a, maxch, s);
  else
    launch_logits<4, 4>(a, maxch, s);
  return check_launch("route/logits");
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
  int rc = launch_route_logits(a, s);
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
