// Error reporting, version, and the whole-layer driver moeq_moe_forward.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>

#include "gemm_impl.h"
#include "routing.h"

extern "C" int moeq_gemm_tile_n(int bm, int epilogue);

namespace moeq {

// One-token layers whose gate matrix is at least this large route in two
// launches (logits over the whole GPU, then a one-wave top-k).  Measured per
// layer: Qwen3-shaped (512 KB) 32.7 -> 28.5 us; OLMoE-shaped (256 KB) 26.0 ->
// 27.0 and Mixtral-shaped (64 KB) 61.2 -> 67.9 us, so those keep route1.
constexpr int64_t kSplitRoute1Bytes = 512 * 1024;

static thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MOEQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return MOEQ_OK;
}

static int hip_ok(hipError_t e, const char *what) {
  if (e != hipSuccess) return fail(MOEQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return MOEQ_OK;
}

// Launch plan of one layer forward; a pure function of (layer, T) so the
// workspace query and the forward agree.
struct Plan {
  int bm, splits, max_tiles, y_dtype;
  int64_t T, pairs, rows;
  size_t off_idx, off_w, off_counts, off_offsets, off_row_token, off_row_pair, off_inv,
      off_tiles, off_ntiles, off_perm, off_route, off_x16, off_h, off_y, total;
};

static Plan make_plan(const moeq_moe *m, int64_t T) {
  Plan p{};
  p.T = T;
  p.pairs = T * m->top_k;
  p.rows = p.pairs + int64_t(m->n_shared) * T;
  const double avg = double(p.pairs) / double(m->n_experts);
  p.bm = avg <= 16 ? 16 : avg <= 32 ? 32 : avg <= 64 ? 64 : 128;
  // From 10 rows per expert many experts need a second 16-row tile, which
  // streams their weights again; the 48-row class streams each expert once
  // and wins when its down launch still has a work-group per CU (OLMoE
  // T = 128: 64 experts x 8 column tiles, 1.04 -> 1.64 M tokens/s).  Few
  // large experts keep the 16-row kernel's K split and deeper fetch ring
  // (Mixtral B = 64 has 8 x 16 and was 9% slower in the 48-row class).
  if (p.bm == 16 && avg > 10 && std::min<int64_t>(m->n_experts, p.pairs) * cdiv(m->hidden, 256) >= 256) p.bm = 32;
  p.max_tiles = moeq_max_tiles(T, m->top_k, m->n_experts, m->n_shared, p.bm);
  // 16-row (decode) down projections with few blocks also split K over
  // work-groups (fp32 slices the combine adds in order), so enough waves keep
  // weight fetches in flight: a K-split block of that shape covers 32 columns.
  p.splits = 1;
  if (p.bm == 16) {
    const int64_t blocks = int64_t(p.max_tiles) * cdiv(m->hidden, 32);
    const int64_t nchunks = m->inter / 128;
    if (blocks < 512) p.splits = int(std::max<int64_t>(1, std::min<int64_t>(cdiv(512, blocks), nchunks / 8)));
  }
  p.y_dtype = p.splits > 1 ? MOEQ_F32 : MOEQ_F16;
  const int Et = m->n_experts + m->n_shared;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    size_t at = o;
    o += align256(bytes);
    return at;
  };
  p.off_idx = take(size_t(p.pairs) * 4);
  p.off_w = take(size_t(p.pairs) * 4);
  p.off_counts = take(size_t(Et) * 4);
  p.off_offsets = take(size_t(Et + 1) * 4);
  p.off_row_token = take(size_t(p.rows) * 4);
  p.off_row_pair = take(size_t(p.pairs) * 4);
  p.off_inv = take(size_t(p.pairs) * 4);
  p.off_tiles = take(size_t(p.max_tiles) * 16);
  p.off_ntiles = take(4);
  p.off_perm = take(moeq_permute_workspace_size(T, m->top_k, m->n_experts, m->n_shared));
  p.off_route = take(moeq_route_workspace_size(T, m->n_experts));
  // the LDS-staged GEMM tiles (bm >= 32) read F16 rows
  // the expert GEMMs read F16 activations
  p.off_x16 = take(m->act_dtype == MOEQ_BF16 ? size_t(T) * m->hidden * 2 : 0);
  p.off_h = take(size_t(p.rows) * m->inter * 2);
  p.off_y = take(size_t(p.splits) * p.rows * m->hidden * (p.y_dtype == MOEQ_F32 ? 4 : 2));
  p.total = o;
  return p;
}

__global__ void bf16_to_f16_kernel(const uint16_t *x, int64_t n, uint16_t *y) {
  const int64_t i = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
  if (i >= n) return;  // n is a multiple of 8
  const uint4 u = *reinterpret_cast<const uint4 *>(x + i);
  const uint32_t ws[4] = {u.x, u.y, u.z, u.w};
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    o[j] = uint32_t(f32_to_f16_bits(__uint_as_float(ws[j] << 16))) |
           (uint32_t(f32_to_f16_bits(__uint_as_float(ws[j] & 0xffff0000u))) << 16);
  *reinterpret_cast<uint4 *>(y + i) = (uint4){o[0], o[1], o[2], o[3]};
}

static int check_layer(const moeq_moe *m) {
  if (!m) return fail(MOEQ_ERR_INVALID, "moe: null layer");
  if (m->hidden <= 0 || m->inter <= 0 || m->n_experts <= 0 || m->top_k <= 0 || m->n_shared < 0)
    return fail(MOEQ_ERR_INVALID, "moe: hidden=%d inter=%d n_experts=%d top_k=%d n_shared=%d", m->hidden,
                m->inter, m->n_experts, m->top_k, m->n_shared);
  if (m->top_k > m->n_experts) return fail(MOEQ_ERR_INVALID, "moe: top_k=%d > n_experts=%d", m->top_k, m->n_experts);
  if (m->act_dtype != MOEQ_F16 && m->act_dtype != MOEQ_BF16) return fail(MOEQ_ERR_INVALID, "moe: act_dtype=%d", m->act_dtype);
  if (m->gate_dtype != MOEQ_F16 && m->gate_dtype != MOEQ_BF16 && m->gate_dtype != MOEQ_F32)
    return fail(MOEQ_ERR_INVALID, "moe: gate_dtype=%d", m->gate_dtype);
  if (!m->gate_w) return fail(MOEQ_ERR_INVALID, "moe: gate_w is null");
  if (m->w1.K != m->hidden || m->w1.N != m->inter || m->w3.K != m->hidden || m->w3.N != m->inter)
    return fail(MOEQ_ERR_INVALID, "moe: gate/up projections must be [hidden=%d -> inter=%d]", m->hidden, m->inter);
  if (m->w2.K != m->inter || m->w2.N != m->hidden)
    return fail(MOEQ_ERR_INVALID, "moe: down projection must be [inter=%d -> hidden=%d]", m->inter, m->hidden);
  return MOEQ_OK;
}

}  // namespace moeq

using namespace moeq;

extern "C" const char *moeq_last_error(void) { return g_err; }

extern "C" int moeq_version(void) { return 1; }

extern "C" size_t moeq_moe_workspace_size(const moeq_moe *m, int64_t T) {
  if (check_layer(m) || T <= 0) return 0;
  return make_plan(m, T).total;
}

// The layer forward; ev0 / ev1 (may be null) are recorded on the stream
// just before and just after the gate/up launch.
static int moe_forward(const moeq_moe *m, const void *x, int64_t T, void *out, int out_dtype,
                       void *logits_out, void *ws, size_t ws_bytes, void *stream, hipEvent_t ev0,
                       hipEvent_t ev1) {
  int rc = check_layer(m);
  if (rc) return rc;
  if (!x || !out) return fail(MOEQ_ERR_INVALID, "moe: null x/out");
  if (T <= 0) return fail(MOEQ_ERR_INVALID, "moe: T=%lld", (long long)T);
  if (out_dtype != m->act_dtype && out_dtype != MOEQ_F32)
    return fail(MOEQ_ERR_INVALID, "moe: out_dtype=%d must be act_dtype or F32", out_dtype);
  // the LDS-staged GEMM tiles address activation rows with 32-bit offsets
  if (T * int64_t(m->hidden) * 2 >= (int64_t(1) << 31) ||
      T * int64_t(m->top_k + m->n_shared) * m->inter * 2 >= (int64_t(1) << 31))
    return fail(MOEQ_ERR_UNSUPPORTED, "moe: T=%lld too large (activations must stay below 2 GiB)", (long long)T);
  const Plan p = make_plan(m, T);
  if (!ws || ws_bytes < p.total)
    return fail(MOEQ_ERR_WORKSPACE, "moe: workspace %zu < %zu bytes", ws_bytes, p.total);
  char *base = static_cast<char *>(ws);
  auto at = [&](size_t off) { return static_cast<void *>(base + off); };
  int32_t *idx = static_cast<int32_t *>(at(p.off_idx));
  float *w = static_cast<float *>(at(p.off_w));
  int32_t *counts = static_cast<int32_t *>(at(p.off_counts));
  int32_t *offsets = static_cast<int32_t *>(at(p.off_offsets));
  int32_t *row_token = static_cast<int32_t *>(at(p.off_row_token));
  int32_t *row_pair = static_cast<int32_t *>(at(p.off_row_pair));
  int32_t *inv = static_cast<int32_t *>(at(p.off_inv));
  int32_t *tiles = static_cast<int32_t *>(at(p.off_tiles));
  int32_t *n_tiles = static_cast<int32_t *>(at(p.off_ntiles));

  bool x16_done = false;
  // The fused top-k + permutation work-group ranks its tokens one per wave,
  // 16 at a time, one after another; past one token per wave the top-k of
  // every token at once over the GPU plus a separate permutation launch is
  // faster (Qwen3-shaped, 64 tokens: 22 us fused, about 11 us split; the
  // OLMoE-shaped 32-token layer 78.7 -> 76.2 us).
  constexpr int64_t kFusedTopkTokens = 16;
  if (T <= 64 && m->hidden % 8 == 0 && m->hidden <= 4096 &&
      topk_permute_fits(T, m->top_k, m->n_experts, m->n_shared)) {
    // small batches: logits, then top-k and the permutation in one work-group
    const int ldt = m->gate_dtype == MOEQ_F32 ? MOEQ_F32 : m->act_dtype;
    void *lg = logits_out ? logits_out : at(p.off_route);
    const int lg_dt = logits_out ? ldt : MOEQ_F32;
    RouteArgs ra{x, m->act_dtype, T, m->hidden, m->gate_w, m->gate_dtype, m->logit_bias, m->n_experts,
                 m->top_k, m->norm_topk ? 1 : 0, lg, ldt, lg_dt, idx, w,
                 m->act_dtype == MOEQ_BF16 ? static_cast<uint16_t *>(at(p.off_x16)) : nullptr};
    x16_done = m->act_dtype == MOEQ_BF16;
    hipStream_t s = as_stream(stream);
    // one token: logits, top-k and the (trivial) grouping in one launch
    const PermOut po{m->n_shared, p.max_tiles, counts, offsets, row_token, row_pair, inv, tiles, n_tiles};
    RouteArgs r1 = ra;  // its logits stay in LDS unless asked for
    r1.logits = logits_out;
    r1.store_dtype = ldt;
    // Mixtral's one-token router ranks and renormalises 16-bit probabilities
    const bool act_softmax = T == 1 && m->one_token_act_softmax;
    if (act_softmax) r1.prob_dtype = m->act_dtype;
    // A large gate matrix is read faster by one logit per wave over the whole
    // GPU and a one-wave top-k after it than by route1's single work-group.
    const int64_t gate_bytes = int64_t(m->n_experts) * m->hidden * (m->gate_dtype == MOEQ_F32 ? 4 : 2);
    if (T == 1 && gate_bytes >= kSplitRoute1Bytes && m->n_experts <= 256 && m->top_k <= kMaxTopK) {
      if ((rc = launch_route_logits(ra, s))) return rc;
      if ((rc = launch_topk1(lg, lg_dt, r1, po, s))) return rc;
    } else if (launch_route1(r1, po, s)) {
      if ((rc = check_launch("moe/route1"))) return rc;
    } else if (act_softmax) {
      return fail(MOEQ_ERR_UNSUPPORTED, "moe: one_token_act_softmax needs the one-token router "
                  "(n_experts <= 256, top_k <= 16, hidden %% 8 == 0 and <= 4096)");
    } else if (T <= kFusedTopkTokens) {
      if ((rc = launch_route_logits(ra, s))) return rc;
      rc = launch_topk_permute(lg, lg_dt, T, m->n_experts, m->top_k, m->norm_topk ? 1 : 0, idx, w, m->n_shared,
                               p.bm, counts, offsets, row_token, row_pair, inv, tiles, n_tiles, s);
      if (rc) return rc;
    } else {
      if ((rc = launch_route_logits(ra, s))) return rc;
      if ((rc = moeq_route_from_logits(lg, lg_dt, T, m->n_experts, m->top_k, m->norm_topk, idx, w, stream)))
        return rc;
      rc = moeq_permute(idx, T, m->top_k, m->n_experts, m->n_shared, p.bm, counts, offsets, row_token,
                        row_pair, inv, tiles, n_tiles, at(p.off_perm),
                        moeq_permute_workspace_size(T, m->top_k, m->n_experts, m->n_shared), stream);
      if (rc) return rc;
    }
  } else {
    // larger batches: fused logits + top-k (writing the fp16 copy of bf16
    // activations on the way) where it covers the dtypes, else moeq_route
    const int ldt = m->gate_dtype == MOEQ_F32 ? MOEQ_F32 : m->act_dtype;
    RouteArgs ra{x, m->act_dtype, T, m->hidden, m->gate_w, m->gate_dtype, m->logit_bias, m->n_experts,
                 m->top_k, m->norm_topk ? 1 : 0, logits_out, ldt, ldt, idx, w,
                 m->act_dtype == MOEQ_BF16 ? static_cast<uint16_t *>(at(p.off_x16)) : nullptr};
    if (m->hidden % 8 == 0 && m->hidden <= 4096 && launch_logits_topk(ra, as_stream(stream))) {
      if ((rc = check_launch("moe/logits_topk"))) return rc;
      x16_done = m->act_dtype == MOEQ_BF16;
    } else {
      rc = moeq_route(x, m->act_dtype, T, m->hidden, m->gate_w, m->gate_dtype, m->logit_bias, m->n_experts,
                      m->top_k, m->norm_topk, logits_out, idx, w, at(p.off_route),
                      moeq_route_workspace_size(T, m->n_experts), stream);
      if (rc) return rc;
    }
    rc = moeq_permute(idx, T, m->top_k, m->n_experts, m->n_shared, p.bm, counts, offsets, row_token,
                      row_pair, inv, tiles, n_tiles, at(p.off_perm),
                      moeq_permute_workspace_size(T, m->top_k, m->n_experts, m->n_shared), stream);
    if (rc) return rc;
  }

  const void *xa = x;
  int xa_dtype = m->act_dtype;
  if (m->act_dtype == MOEQ_BF16) {
    if (!x16_done) {
      const int64_t n = T * m->hidden;
      bf16_to_f16_kernel<<<dim3(unsigned(cdiv(n / 8, 256))), dim3(256), 0, as_stream(stream)>>>(
          static_cast<const uint16_t *>(x), n, static_cast<uint16_t *>(at(p.off_x16)));
      if ((rc = check_launch("moe/bf16_to_f16"))) return rc;
    }
    xa = at(p.off_x16);
    xa_dtype = MOEQ_F16;
  }

  moeq_gemm gu{};
  gu.a = xa;
  gu.a_dtype = xa_dtype;
  gu.lda = m->hidden;
  gu.row_src = row_token;
  gu.tiles = tiles;
  gu.n_tiles = n_tiles;
  gu.max_tiles = p.max_tiles;
  gu.bm = p.bm;
  gu.epilogue = MOEQ_EPI_SILU_MUL;
  gu.out = at(p.off_h);
  gu.out_dtype = MOEQ_F16;
  gu.ldo = m->inter;
  gu.splits = 1;
  gu.split_stride = 0;
  if (ev0 && (rc = hip_ok(hipEventRecord(ev0, as_stream(stream)), "moe: event record"))) return rc;
  // a token picks an expert at most once: no tile holds more than T rows
  const int max_rows = int(std::min<int64_t>(T, tile_rows(p.bm)));
  // average rows per routed expert if the pairs spread over as many experts as they can
  const int rows_hint = int(T * m->top_k / std::max<int64_t>(1, std::min<int64_t>(m->n_experts, T * m->top_k)));
  // one token: each selected expert and each shared expert one 1-row tile
  const int known_tiles = T == 1 ? m->top_k + m->n_shared : 0;
  rc = grouped_gemm_rows(&gu, &m->w1, &m->w3, max_rows, rows_hint, known_tiles, stream);
  if (rc) return rc;
  if (ev1 && (rc = hip_ok(hipEventRecord(ev1, as_stream(stream)), "moe: event record"))) return rc;

  // one token: down projection and combine in one launch
  if (T == 1 && m->top_k + m->n_shared <= 32)
    return launch_down_combine1(&m->w2, static_cast<const uint16_t *>(at(p.off_h)), tiles, inv, w, m->top_k,
                                m->n_shared, out, out_dtype, as_stream(stream));

  moeq_gemm dn = gu;
  dn.a = at(p.off_h);
  dn.a_dtype = MOEQ_F16;
  dn.lda = m->inter;
  dn.row_src = nullptr;
  dn.epilogue = MOEQ_EPI_STORE;
  dn.out = at(p.off_y);
  dn.out_dtype = p.y_dtype;
  dn.ldo = m->hidden;
  dn.splits = p.splits;
  dn.split_stride = p.rows * m->hidden;
  rc = grouped_gemm_rows(&dn, &m->w2, nullptr, max_rows, rows_hint, known_tiles, stream);
  if (rc) return rc;

  return moeq_combine(at(p.off_y), p.y_dtype, p.splits, p.rows * m->hidden, m->hidden, inv, w, T,
                      m->top_k, m->n_shared, m->hidden, out, out_dtype, stream);
}

extern "C" int moeq_moe_forward(const moeq_moe *m, const void *x, int64_t T, void *out,
                                int out_dtype, void *logits_out, void *ws, size_t ws_bytes,
                                void *stream) {
  return moe_forward(m, x, T, out, out_dtype, logits_out, ws, ws_bytes, stream, nullptr, nullptr);
}

// Benchmark introspection (not a reference interface): moeq_moe_forward that
// also records two HIP events around its gate/up launch.
extern "C" int moeq_moe_forward_timed(const moeq_moe *m, const void *x, int64_t T, void *out,
                                      int out_dtype, void *logits_out, void *ws, size_t ws_bytes,
                                      void *stream, void *ev_gate_up_begin, void *ev_gate_up_end) {
  if (!ev_gate_up_begin || !ev_gate_up_end) return fail(MOEQ_ERR_INVALID, "moe_forward_timed: null event");
  return moe_forward(m, x, T, out, out_dtype, logits_out, ws, ws_bytes, stream,
                     static_cast<hipEvent_t>(ev_gate_up_begin), static_cast<hipEvent_t>(ev_gate_up_end));
}

// Workspace introspection for tests (not a reference interface): byte
// offsets in the forward's workspace of {idx, w, counts, offsets, row_token,
// row_pair, inv_perm, tiles, n_tiles}, the routing and permutation the
// forward leaves there.
extern "C" int moeq_moe_workspace_layout(const moeq_moe *m, int64_t T, int64_t *out9) {
  int rc = check_layer(m);
  if (rc) return rc;
  if (T <= 0 || !out9) return fail(MOEQ_ERR_INVALID, "moe_workspace_layout: T=%lld", (long long)T);
  const Plan p = make_plan(m, T);
  const size_t offs[9] = {p.off_idx, p.off_w, p.off_counts, p.off_offsets, p.off_row_token,
                          p.off_row_pair, p.off_inv, p.off_tiles, p.off_ntiles};
  for (int i = 0; i < 9; ++i) out9[i] = int64_t(offs[i]);
  return MOEQ_OK;
}

// Launch plan introspection for tests and the benchmark (not a reference
// interface): writes {bm, splits, max_tiles, y_dtype}.
extern "C" int moeq_moe_plan(const moeq_moe *m, int64_t T, int32_t *out4) {
  int rc = check_layer(m);
  if (rc) return rc;
  if (T <= 0 || !out4) return fail(MOEQ_ERR_INVALID, "moe_plan: T=%lld", (long long)T);
  Plan p = make_plan(m, T);
  out4[0] = p.bm;
  out4[1] = p.splits;
  out4[2] = p.max_tiles;
  out4[3] = p.y_dtype;
  return MOEQ_OK;
}
