// Entry point of the grouped GEMM: argument checks and dispatch to the
// row-tile height instantiated in gemm_bm<BM>.hip (kernel: gemm_impl.h).
#include <algorithm>

#include "gemm_impl.h"

using namespace moeq;

static int check_proj(const moeq_proj *p, const char *name) {
  if (!p) return fail(MOEQ_ERR_INVALID, "grouped_gemm: %s is null", name);
  if (!p->words || !p->word_off || !p->sz || !p->sz_off || !p->nbits)
    return fail(MOEQ_ERR_INVALID, "grouped_gemm: %s has a null pointer", name);
  if (p->K <= 0 || p->K % 128) return fail(MOEQ_ERR_UNSUPPORTED, "grouped_gemm: %s K=%d must be a positive multiple of 128", name, p->K);
  if (p->N <= 0 || p->N % 16) return fail(MOEQ_ERR_UNSUPPORTED, "grouped_gemm: %s N=%d must be a positive multiple of 16", name, p->N);
  if (p->group_size < 32 || p->group_size % 32 || p->K % p->group_size)
    return fail(MOEQ_ERR_UNSUPPORTED, "grouped_gemm: %s group_size=%d must be a multiple of 32 dividing K=%d", name, p->group_size, p->K);
  if (int64_t(p->K) * p->N / 2 >= (int64_t(1) << 31))
    return fail(MOEQ_ERR_UNSUPPORTED, "grouped_gemm: %s K*N=%lld too large (one expert's words must stay below 2 GiB)",
                name, (long long)(int64_t(p->K) * p->N));
  if (p->dq_mode != MOEQ_DQ_HQQ && p->dq_mode != MOEQ_DQ_AFFINE && p->dq_mode != MOEQ_DQ_HQQ_INT)
    return fail(MOEQ_ERR_INVALID, "grouped_gemm: %s dq_mode=%d", name, p->dq_mode);
  return MOEQ_OK;
}

int moeq::grouped_gemm_rows(const moeq_gemm *gm, const moeq_proj *p0, const moeq_proj *p1, int max_rows, int rows_hint,
                            int known_tiles, void *stream) {
  if (!gm) return fail(MOEQ_ERR_INVALID, "grouped_gemm: null descriptor");
  if (!gm->a || !gm->tiles || !gm->n_tiles || !gm->out) return fail(MOEQ_ERR_INVALID, "grouped_gemm: null pointer");
  int rc = check_proj(p0, "p0");
  if (rc) return rc;
  if (gm->epilogue == MOEQ_EPI_SILU_MUL) {
    if ((rc = check_proj(p1, "p1"))) return rc;
    if (p1->K != p0->K || p1->N != p0->N || p1->group_size != p0->group_size || p1->dq_mode != p0->dq_mode)
      return fail(MOEQ_ERR_INVALID, "grouped_gemm: gate/up projections differ in shape or convention");
    if (gm->out_dtype != MOEQ_F16) return fail(MOEQ_ERR_INVALID, "grouped_gemm: SILU_MUL writes F16");
    if (gm->splits != 1) return fail(MOEQ_ERR_INVALID, "grouped_gemm: SILU_MUL cannot split K");
  } else if (gm->epilogue == MOEQ_EPI_STORE) {
    if (p1) return fail(MOEQ_ERR_INVALID, "grouped_gemm: STORE takes one projection");
  } else {
    return fail(MOEQ_ERR_INVALID, "grouped_gemm: epilogue=%d", gm->epilogue);
  }
  if (gm->a_dtype != MOEQ_F16 && gm->a_dtype != MOEQ_BF16) return fail(MOEQ_ERR_INVALID, "grouped_gemm: a_dtype=%d", gm->a_dtype);
  if (gm->out_dtype != MOEQ_F16 && gm->out_dtype != MOEQ_F32) return fail(MOEQ_ERR_INVALID, "grouped_gemm: out_dtype=%d", gm->out_dtype);
  if (gm->lda < p0->K || gm->lda % 8) return fail(MOEQ_ERR_INVALID, "grouped_gemm: lda=%lld (K=%d, multiple of 8)", (long long)gm->lda, p0->K);
  if (gm->ldo < p0->N) return fail(MOEQ_ERR_INVALID, "grouped_gemm: ldo=%lld < N=%d", (long long)gm->ldo, p0->N);
  if (gm->max_tiles <= 0) return fail(MOEQ_ERR_INVALID, "grouped_gemm: max_tiles=%d", gm->max_tiles);
  const int nchunks = p0->K / 128;
  if (gm->splits < 1 || gm->splits > nchunks) return fail(MOEQ_ERR_INVALID, "grouped_gemm: splits=%d not in 1..%d", gm->splits, nchunks);
  if (gm->splits > 1 && gm->out_dtype != MOEQ_F32) return fail(MOEQ_ERR_INVALID, "grouped_gemm: split-K writes F32");

  GemmArgs g{};
  g.a = gm->a;
  g.lda = gm->lda;
  g.row_src = gm->row_src;
  g.tiles = gm->tiles;
  g.n_tiles = gm->n_tiles;
  g.K = p0->K;
  g.N = p0->N;
  g.group_size = p0->group_size;
  g.gshift = (p0->group_size & (p0->group_size - 1)) ? -1 : __builtin_ctz(unsigned(p0->group_size));
  g.dq_mode = p0->dq_mode;
  g.p[0] = ProjDev{p0->words, p0->word_off, p0->sz, p0->sz_off, p0->nbits};
  g.p[1] = p1 ? ProjDev{p1->words, p1->word_off, p1->sz, p1->sz_off, p1->nbits} : g.p[0];
  g.out = gm->out;
  g.ldo = gm->ldo;
  g.split_stride = gm->split_stride;
  g.nchunks = nchunks;
  g.chunks_per_split = int(cdiv(nchunks, gm->splits));
  g.max_rows = max_rows;
  g.rows_hint = rows_hint;
  g.known_tiles = known_tiles > 0 && known_tiles <= gm->max_tiles ? known_tiles : 0;
  hipStream_t s = as_stream(stream);
  const int mt = gm->max_tiles, sp = gm->splits;
  const bool silu = gm->epilogue == MOEQ_EPI_SILU_MUL;
  switch (gm->bm) {
    case 16: return launch_grouped_gemm<16>(g, silu, gm->a_dtype, gm->out_dtype, mt, sp, s);
    case 32: return launch_grouped_gemm<32>(g, silu, gm->a_dtype, gm->out_dtype, mt, sp, s);
    case 64: return launch_grouped_gemm<64>(g, silu, gm->a_dtype, gm->out_dtype, mt, sp, s);
    case 128: return launch_grouped_gemm<128>(g, silu, gm->a_dtype, gm->out_dtype, mt, sp, s);
    case 256: return launch_grouped_gemm<256>(g, silu, gm->a_dtype, gm->out_dtype, mt, sp, s);
    default: return fail(MOEQ_ERR_INVALID, "grouped_gemm: bm=%d not in {16, 32, 64, 128, 256}", gm->bm);
  }
}

extern "C" int moeq_grouped_gemm(const moeq_gemm *gm, const moeq_proj *p0,
                                 const moeq_proj *p1, void *stream) {
  return grouped_gemm_rows(gm, p0, p1, 0, 0, 0, stream);
}

// Column tile width the kernels use for a given (bm, epilogue); the layer
// driver sizes its launches with it.
template <int BM>
static int tile_n(bool silu) {
  return silu ? tile_cols<Shape<BM, true>, false>() : tile_cols<Shape<BM, false>, false>();
}

extern "C" int moeq_gemm_tile_n(int bm, int epilogue) {
  const bool silu = epilogue == MOEQ_EPI_SILU_MUL;
  switch (bm) {
    case 16: return tile_n<16>(silu);
    case 32: return tile_n<32>(silu);
    case 64: return tile_n<64>(silu);
    case 128: return tile_n<128>(silu);
    case 256: return tile_n<256>(silu);
    default: return 0;
  }
}
