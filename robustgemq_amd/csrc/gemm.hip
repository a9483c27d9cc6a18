// Persistent-tile grouped GEMM over all experts of a MoE layer with mixed
// 1/2/3/4-bit weights, on v_mfma_f32_16x16x32_f16.
//
// One launch covers every (row tile, column tile) of every expert; the row
// tiles come from the device-side schedule written by moeq_permute, so no
// host synchronisation is needed.  Per 128-deep K chunk:
//   A (activations, gathered rows): staged through LDS, 16-byte units XOR-
//      swizzled by row so the 16 rows read by one MFMA fragment hit disjoint
//      banks (BM >= 32), or loaded straight into registers (BM == 16, decode).
//   B (weights): each lane loads its own lane slice (`bits` words of one
//      column, 32 consecutive k) with one vector load and dequantizes it in
//      registers straight into the MFMA B-fragment layout:
//        raw pair -> | 0x6400 per half (1024 + q, exact) -> - 1024 (q, exact)
//        HQQ:    (q + (-z)) * s   two fp16 roundings = fp16(fp16(q - z) * s)
//        AFFINE: fma(q, s, z')    one rounding       = GemLite's q * s + z'
//      so the weight fed to the MFMA equals the reference's dequantized weight
//      bit for bit.
// Accumulation is fp32.  Epilogues: store (f16 / f32, optional split-K
// slices), or silu(gate) * up for the fused gate/up projection.
#include <algorithm>

#include "common.h"

namespace moeq {

struct ProjDev {
  const uint32_t *words;
  const int64_t *word_off;
  const uint32_t *sz;
  const int64_t *sz_off;
  const int32_t *nbits;
};

struct GemmArgs {
  const void *a;
  int64_t lda;
  const int32_t *row_src;
  const int32_t *tiles;
  const int32_t *n_tiles;
  int K, N, group_size, dq_mode;
  ProjDev p[2];
  void *out;
  int64_t ldo, split_stride;
  int n_ntiles, nchunks, chunks_per_split;
};

// The two codes of MFMA step t, pair d of a lane slice, at bits [0, b) of
// each 16-bit half (layout written by repack_kernel).
template <int BITS>
__device__ __forceinline__ uint32_t raw_pair(const uint32_t (&w)[BITS], int t, int d) {
  if constexpr (BITS == 4) {
    return (w[t] >> (4 * d)) & 0x000f000fu;
  } else if constexpr (BITS == 2) {
    return (w[t >> 1] >> (8 * (t & 1) + 2 * d)) & 0x00030003u;
  } else if constexpr (BITS == 1) {
    return (w[0] >> (4 * t + d)) & 0x00010001u;
  } else {
    return ((w[t >> 1] >> (8 * (t & 1) + 2 * d)) & 0x00030003u) |
           (((w[2] >> (4 * t + d)) & 0x00010001u) << 2);
  }
}

template <int BITS, int DQ>
__device__ __forceinline__ f16x8 deq_frag(const uint32_t (&w)[BITS], uint32_t sz, int t) {
  const f16 sh = __builtin_bit_cast(f16, uint16_t(sz & 0xffffu));
  const f16 zh = __builtin_bit_cast(f16, uint16_t(sz >> 16));
  const f16x2 s2 = {sh, sh}, z2 = {zh, zh};
  const f16x2 k1024 = {(f16)1024.0f, (f16)1024.0f};
  f16x8 r;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    f16x2 v = __builtin_bit_cast(f16x2, raw_pair<BITS>(w, t, d) | 0x64006400u);
    f16x2 q = v - k1024;
    f16x2 o;
    if constexpr (DQ == MOEQ_DQ_HQQ)
      o = (q + z2) * s2;
    else
      o = __builtin_elementwise_fma(q, s2, z2);
    r[2 * d] = o[0];
    r[2 * d + 1] = o[1];
  }
  return r;
}

template <int BITS>
__device__ __forceinline__ void load_slice(const uint32_t *p, uint32_t (&w)[BITS]) {
  if constexpr (BITS == 4) {
    uint4 v = *reinterpret_cast<const uint4 *>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else if constexpr (BITS == 2) {
    uint2 v = *reinterpret_cast<const uint2 *>(p);
    w[0] = v.x; w[1] = v.y;
  } else if constexpr (BITS == 1) {
    w[0] = *p;
  } else {
    w[0] = p[0]; w[1] = p[1]; w[2] = p[2];
  }
}

// 8 activations (16 bytes) of type ADT -> f16x8.  bf16 -> f16 is exact for
// |x| in the fp16 normal range; smaller values round to fp16 subnormals.
template <int ADT>
__device__ __forceinline__ f16x8 to_f16x8(uint4 u) {
  if constexpr (ADT == MOEQ_F16) {
    return __builtin_bit_cast(f16x8, u);
  } else {
    uint32_t ws[4] = {u.x, u.y, u.z, u.w};
    f16x8 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      r[2 * j] = (f16)__uint_as_float(ws[j] << 16);
      r[2 * j + 1] = (f16)__uint_as_float(ws[j] & 0xffff0000u);
    }
    return r;
  }
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  return g / (1.0f + __expf(-g)) * u;
}

template <int BM, int NW, int NB, int NP, int EPI, int ADT, int ODT, int BITS, int DQ>
__device__ __forceinline__ void gemm_tile(const GemmArgs &g, int e, int row0, int mcount,
                                          int nt, int c0, int c1, uint4 (*As)[BM][16]) {
  constexpr int MB = BM / 16;
  constexpr int NT = NW * 64;
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int l16 = lane & 15, kb = lane >> 4;
  const int N = g.N;
  const int n_wave = nt * (NW * NB * 16) + wave * NB * 16;

  // per projection: expert block base pointers
  const uint32_t *wbase[NP];
  const uint32_t *sbase[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    wbase[p] = g.p[p].words + g.p[p].word_off[e];
    sbase[p] = g.p[p].sz + g.p[p].sz_off[e];
  }
  bool col_ok[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) col_ok[nb] = n_wave + nb * 16 < N;

  f32x4 acc[NP][MB][NB];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[p][mb][nb] = (f32x4){0.f, 0.f, 0.f, 0.f};

  uint32_t wcur[NP][NB][BITS], wnxt[NP][NB][BITS];
  uint32_t scur[NP][NB], snxt[NP][NB];

  auto load_b = [&](int c, uint32_t (&w)[NP][NB][BITS], uint32_t (&s)[NP][NB]) {
    const int grp = (c * 128 + 32 * kb) / g.group_size;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if (col_ok[nb]) {
          const int n = n_wave + nb * 16 + l16;
          load_slice<BITS>(wbase[p] + ((int64_t(c) * N + n) * 4 + kb) * BITS, w[p][nb]);
          s[p][nb] = sbase[p][int64_t(grp) * N + n];
        } else {
#pragma unroll
          for (int j = 0; j < BITS; ++j) w[p][nb][j] = 0;
          s[p][nb] = 0;
        }
      }
  };

  const char *abytes = static_cast<const char *>(g.a);
  constexpr int AES = ADT == MOEQ_F32 ? 4 : 2;

  if constexpr (BM == 16) {
    // ---------------- decode shape: A fragments straight from global memory
    const bool row_ok = l16 < mcount;
    int64_t src = 0;
    if (row_ok) src = g.row_src ? g.row_src[row0 + l16] : int64_t(row0 + l16);
    const char *arow = abytes + src * g.lda * AES;
    uint4 acur[4], anxt[4];
    auto load_a = [&](int c, uint4 (&av)[4]) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (row_ok)
          av[t] = *reinterpret_cast<const uint4 *>(arow + (int64_t(c) * 128 + 32 * kb + 8 * t) * AES);
        else
          av[t] = (uint4){0u, 0u, 0u, 0u};
      }
    };
    if (c0 < c1) {
      load_a(c0, acur);
      load_b(c0, wcur, scur);
    }
    for (int c = c0; c < c1; ++c) {
      if (c + 1 < c1) {
        load_a(c + 1, anxt);
        load_b(c + 1, wnxt, snxt);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        f16x8 A = to_f16x8<ADT>(acur[t]);
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            if (!col_ok[nb]) continue;
            f16x8 B = deq_frag<BITS, DQ>(wcur[p][nb], scur[p][nb], t);
            acc[p][0][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, acc[p][0][nb], 0, 0, 0);
          }
      }
      if (c + 1 < c1) {
#pragma unroll
        for (int t = 0; t < 4; ++t) acur[t] = anxt[t];
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            scur[p][nb] = snxt[p][nb];
#pragma unroll
            for (int j = 0; j < BITS; ++j) wcur[p][nb][j] = wnxt[p][nb][j];
          }
      }
    }
  } else {
    // ---------------- prefill shape: A staged through LDS (double buffered)
    // As[buf][row][unit]: 128 halves per row as 16 units of 8; unit u of row
    // r is stored at u ^ (r & 15).
    constexpr int SEGS = BM * 16 / NT;  // 16-byte units per thread per chunk
    static_assert(SEGS >= 1 && (BM * 16) % NT == 0, "A staging split");
    uint4 areg[SEGS];
    int64_t asrc[SEGS];
#pragma unroll
    for (int i = 0; i < SEGS; ++i) {
      int seg = threadIdx.x + i * NT;
      int r = seg >> 4;
      asrc[i] = -1;
      if (r < mcount) asrc[i] = g.row_src ? g.row_src[row0 + r] : int64_t(row0 + r);
    }
    auto load_a = [&](int c) {
#pragma unroll
      for (int i = 0; i < SEGS; ++i) {
        int seg = threadIdx.x + i * NT;
        int u = seg & 15;
        if (asrc[i] >= 0) {
          const char *p = abytes + (asrc[i] * g.lda + int64_t(c) * 128 + u * 8) * AES;
          areg[i] = *reinterpret_cast<const uint4 *>(p);
        } else {
          areg[i] = (uint4){0u, 0u, 0u, 0u};
        }
      }
    };
    auto store_a = [&](int buf) {
#pragma unroll
      for (int i = 0; i < SEGS; ++i) {
        int seg = threadIdx.x + i * NT;
        int r = seg >> 4, u = seg & 15;
        f16x8 h = to_f16x8<ADT>(areg[i]);
        As[buf][r][u ^ (r & 15)] = __builtin_bit_cast(uint4, h);
      }
    };
    if (c0 < c1) {
      load_a(c0);
      load_b(c0, wcur, scur);
      store_a(0);
    }
    __syncthreads();
    for (int c = c0; c < c1; ++c) {
      const int buf = (c - c0) & 1;
      const bool more = c + 1 < c1;
      if (more) {
        load_a(c + 1);
        load_b(c + 1, wnxt, snxt);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        f16x8 B[NP][NB];
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) B[p][nb] = deq_frag<BITS, DQ>(wcur[p][nb], scur[p][nb], t);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          if (mb * 16 >= mcount) break;
          const int r = mb * 16 + l16;
          f16x8 A = __builtin_bit_cast(f16x8, As[buf][r][(4 * kb + t) ^ (r & 15)]);
#pragma unroll
          for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
              if (!col_ok[nb]) continue;
              acc[p][mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B[p][nb], acc[p][mb][nb], 0, 0, 0);
            }
        }
      }
      if (more) {
        store_a(buf ^ 1);
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            scur[p][nb] = snxt[p][nb];
#pragma unroll
            for (int j = 0; j < BITS; ++j) wcur[p][nb][j] = wnxt[p][nb][j];
          }
      }
      __syncthreads();
    }
  }

  // ---------------- epilogue: D[row = 4 * (lane / 16) + i][col = lane % 16]
  char *obytes = static_cast<char *>(g.out);
  const int split = blockIdx.z;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    if (mb * 16 >= mcount) break;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if (!col_ok[nb]) continue;
      const int col = n_wave + nb * 16 + l16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = mb * 16 + 4 * kb + i;
        if (r >= mcount) continue;
        const int64_t o = int64_t(row0 + r) * g.ldo + col;
        if constexpr (EPI == MOEQ_EPI_SILU_MUL) {
          float h = silu_mul(acc[0][mb][nb][i], acc[NP - 1][mb][nb][i]);
          reinterpret_cast<uint16_t *>(obytes)[o] = f32_to_f16_bits(h);
        } else if constexpr (ODT == MOEQ_F32) {
          reinterpret_cast<float *>(obytes)[split * g.split_stride + o] = acc[0][mb][nb][i];
        } else {
          reinterpret_cast<uint16_t *>(obytes)[split * g.split_stride + o] =
              f32_to_f16_bits(acc[0][mb][nb][i]);
        }
      }
    }
  }
}

template <int BM, int NW, int NB, int NP, int EPI, int ADT, int ODT>
__global__ __launch_bounds__(NW * 64) void grouped_gemm_kernel(GemmArgs g) {
  // The grid is sized for the host-side bound on row tiles; blocks past the
  // real count (read from the device schedule) exit together.  Work-groups
  // are dealt to the 8 XCDs round-robin, so the live ones are renumbered to
  // give each XCD a contiguous run of tiles (same row tile with neighbouring
  // column tiles, then the next row tile of the same expert) sharing its L2.
  const unsigned V = unsigned(*g.n_tiles) * unsigned(g.n_ntiles);
  const unsigned b = blockIdx.x;
  if (b >= V) return;
  const unsigned V8 = V & ~7u;
  const unsigned L = b < V8 ? (b & 7u) * (V8 >> 3) + (b >> 3) : b;
  const int mt = int(L / unsigned(g.n_ntiles));
  const int nt = int(L % unsigned(g.n_ntiles));
  __shared__ uint4 As[BM == 16 ? 1 : 2][BM][16];
  const int32_t *tp = g.tiles + 4 * mt;
  const int e = tp[0], row0 = tp[1], mcount = tp[2];
  const int c0 = int(blockIdx.z) * g.chunks_per_split;
  const int c1 = min(c0 + g.chunks_per_split, g.nchunks);
  const int bits = g.p[0].nbits[e];
  const bool hqq = g.dq_mode == MOEQ_DQ_HQQ;
#define MOEQ_TILE(B, D) gemm_tile<BM, NW, NB, NP, EPI, ADT, ODT, B, D>(g, e, row0, mcount, nt, c0, c1, As)
  switch (bits) {
    case 1: if (hqq) MOEQ_TILE(1, MOEQ_DQ_HQQ); else MOEQ_TILE(1, MOEQ_DQ_AFFINE); break;
    case 2: if (hqq) MOEQ_TILE(2, MOEQ_DQ_HQQ); else MOEQ_TILE(2, MOEQ_DQ_AFFINE); break;
    case 3: if (hqq) MOEQ_TILE(3, MOEQ_DQ_HQQ); else MOEQ_TILE(3, MOEQ_DQ_AFFINE); break;
    default: if (hqq) MOEQ_TILE(4, MOEQ_DQ_HQQ); else MOEQ_TILE(4, MOEQ_DQ_AFFINE); break;
  }
#undef MOEQ_TILE
}

// Column tile width per configuration.
template <int NW, int NB>
constexpr int bn_of() { return NW * NB * 16; }

template <int BM, int NW, int NB, int NP, int EPI>
static int launch_cfg(const GemmArgs &g, int a_dtype, int out_dtype, int max_tiles, int splits,
                      hipStream_t s) {
  GemmArgs a = g;
  a.n_ntiles = int(cdiv(g.N, bn_of<NW, NB>()));
  dim3 grid(unsigned(int64_t(max_tiles) * a.n_ntiles), 1, unsigned(splits)), block(NW * 64);
  if (int64_t(max_tiles) * a.n_ntiles > 0x7fffffff) return fail(MOEQ_ERR_UNSUPPORTED, "grouped_gemm: grid too large");
#define MOEQ_L(ADT, ODT) grouped_gemm_kernel<BM, NW, NB, NP, EPI, ADT, ODT><<<grid, block, 0, s>>>(a)
  if (EPI == MOEQ_EPI_SILU_MUL) {
    if (a_dtype == MOEQ_BF16) MOEQ_L(MOEQ_BF16, MOEQ_F16); else MOEQ_L(MOEQ_F16, MOEQ_F16);
  } else if (out_dtype == MOEQ_F32) {
    if (a_dtype == MOEQ_BF16) MOEQ_L(MOEQ_BF16, MOEQ_F32); else MOEQ_L(MOEQ_F16, MOEQ_F32);
  } else {
    if (a_dtype == MOEQ_BF16) MOEQ_L(MOEQ_BF16, MOEQ_F16); else MOEQ_L(MOEQ_F16, MOEQ_F16);
  }
#undef MOEQ_L
  return check_launch("grouped_gemm");
}

}  // namespace moeq

using namespace moeq;

static int check_proj(const moeq_proj *p, const char *name) {
  if (!p) return fail(MOEQ_ERR_INVALID, "grouped_gemm: %s is null", name);
  if (!p->words || !p->word_off || !p->sz || !p->sz_off || !p->nbits)
    return fail(MOEQ_ERR_INVALID, "grouped_gemm: %s has a null pointer", name);
  if (p->K <= 0 || p->K % 128) return fail(MOEQ_ERR_UNSUPPORTED, "grouped_gemm: %s K=%d must be a positive multiple of 128", name, p->K);
  if (p->N <= 0 || p->N % 16) return fail(MOEQ_ERR_UNSUPPORTED, "grouped_gemm: %s N=%d must be a positive multiple of 16", name, p->N);
  if (p->group_size < 32 || p->group_size % 32 || p->K % p->group_size)
    return fail(MOEQ_ERR_UNSUPPORTED, "grouped_gemm: %s group_size=%d must be a multiple of 32 dividing K=%d", name, p->group_size, p->K);
  if (p->dq_mode != MOEQ_DQ_HQQ && p->dq_mode != MOEQ_DQ_AFFINE)
    return fail(MOEQ_ERR_INVALID, "grouped_gemm: %s dq_mode=%d", name, p->dq_mode);
  return MOEQ_OK;
}

extern "C" int moeq_grouped_gemm(const moeq_gemm *gm, const moeq_proj *p0,
                                 const moeq_proj *p1, void *stream) {
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
  g.dq_mode = p0->dq_mode;
  g.p[0] = ProjDev{p0->words, p0->word_off, p0->sz, p0->sz_off, p0->nbits};
  g.p[1] = p1 ? ProjDev{p1->words, p1->word_off, p1->sz, p1->sz_off, p1->nbits} : g.p[0];
  g.out = gm->out;
  g.ldo = gm->ldo;
  g.split_stride = gm->split_stride;
  g.nchunks = nchunks;
  g.chunks_per_split = int(cdiv(nchunks, gm->splits));
  hipStream_t s = as_stream(stream);
  const int mt = gm->max_tiles, sp = gm->splits;
  const bool silu = gm->epilogue == MOEQ_EPI_SILU_MUL;
  switch (gm->bm) {
    case 16:
      return silu ? launch_cfg<16, 4, 1, 2, MOEQ_EPI_SILU_MUL>(g, gm->a_dtype, gm->out_dtype, mt, sp, s)
                  : launch_cfg<16, 4, 2, 1, MOEQ_EPI_STORE>(g, gm->a_dtype, gm->out_dtype, mt, sp, s);
    case 32:
      return silu ? launch_cfg<32, 4, 2, 2, MOEQ_EPI_SILU_MUL>(g, gm->a_dtype, gm->out_dtype, mt, sp, s)
                  : launch_cfg<32, 4, 4, 1, MOEQ_EPI_STORE>(g, gm->a_dtype, gm->out_dtype, mt, sp, s);
    case 64:
      return silu ? launch_cfg<64, 4, 2, 2, MOEQ_EPI_SILU_MUL>(g, gm->a_dtype, gm->out_dtype, mt, sp, s)
                  : launch_cfg<64, 4, 4, 1, MOEQ_EPI_STORE>(g, gm->a_dtype, gm->out_dtype, mt, sp, s);
    case 128:
      return silu ? launch_cfg<128, 4, 2, 2, MOEQ_EPI_SILU_MUL>(g, gm->a_dtype, gm->out_dtype, mt, sp, s)
                  : launch_cfg<128, 4, 4, 1, MOEQ_EPI_STORE>(g, gm->a_dtype, gm->out_dtype, mt, sp, s);
    default:
      return fail(MOEQ_ERR_INVALID, "grouped_gemm: bm=%d not in {16, 32, 64, 128}", gm->bm);
  }
}

// Column tile width the kernels use for a given (bm, epilogue); the layer
// driver sizes its launches with it.
extern "C" int moeq_gemm_tile_n(int bm, int epilogue) {
  const bool silu = epilogue == MOEQ_EPI_SILU_MUL;
  switch (bm) {
    case 16: return silu ? bn_of<4, 1>() : bn_of<4, 2>();
    case 32: case 64: case 128: return silu ? bn_of<4, 2>() : bn_of<4, 4>();
    default: return 0;
  }
}
