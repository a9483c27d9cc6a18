// Grouped mixed-bit GEMM over all experts of a MoE layer on
// v_mfma_f32_16x16x32_f16 (gfx950).  Included by gemm_bm*.hip, each of which
// instantiates one row-tile height BM.
//
// One launch covers every (row tile, column tile) of every expert; the row
// tiles come from the device-side schedule written by moeq_permute (full BM
// tiles plus one remainder tile per expert), so no host synchronisation is
// needed.  A block has NW waves; wave w owns NB * 16 output columns and all
// active rows of the tile.  Per 128-deep K chunk:
//   A (activations, gathered rows): BM >= 32 -> copied global -> LDS with
//      global_load_lds_dwordx4 (no register staging), 16-byte units XOR-
//      swizzled by row so the 16 rows of one MFMA fragment hit disjoint banks;
//      BM == 16 -> loaded straight into registers (decode shapes).
//   B (weights): each lane loads its own lane slice (`BITS` words = 32 codes of
//      one column) with one vector load, one chunk ahead, and dequantizes it
//      in registers straight into the MFMA B-fragment layout:
//        pair of codes ORed into the mantissa of 1024 -> 1024 + q (exact)
//        HQQ_INT: (v - (1024 + z)) * s = fp16(fp16(q - z) * s), fake-quant weight
//        HQQ:     ((v - 1024) - z) * s  (same value, any fp16 zero)
//        AFFINE:  fma(v - 1024, s, z')  = GemLite's q * s + z'
// The inner loop is branch-free: the wave index is made uniform, columns past
// N load a valid column and are not stored, rows past the tile load a valid
// row and are not stored, and the number of active 16-row blocks (MBA) is a
// template parameter chosen per tile.  Accumulation is fp32.
#pragma once

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

typedef __attribute__((address_space(3))) void lds_void;

// (x & m) | c in one instruction (the compiler splits it into two when both
// constants would need the scalar constant bus).
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(m), "v"(c));
  return r;
}

// fp16 pair (1024 + q_lo, 1024 + q_hi) for MFMA step t, pair d of a lane
// slice: the two codes sit at the same bit offset of the two 16-bit halves
// (layout written by repack_kernel) and are ORed into the mantissa of 1024.
template <int BITS>
__device__ __forceinline__ uint32_t magic_pair(const uint32_t (&w)[BITS], int t, int d, uint32_t magic) {
  if constexpr (BITS == 4) {
    return and_or(w[t] >> (4 * d), 0x000f000fu, magic);
  } else if constexpr (BITS == 2) {
    return and_or(w[t >> 1] >> (8 * (t & 1) + 2 * d), 0x00030003u, magic);
  } else if constexpr (BITS == 1) {
    return and_or(w[0] >> (4 * t + d), 0x00010001u, magic);
  } else {
    const uint32_t lo = and_or(w[t >> 1] >> (8 * (t & 1) + 2 * d), 0x00030003u, magic);
    const int hb = 4 * t + d;  // bit of the high code bit in word 2, moved to bit 2
    const uint32_t hi = hb >= 2 ? (w[2] >> (hb - 2)) : (w[2] << (2 - hb));
    return and_or(hi, 0x00040004u, lo);
  }
}

// B fragment (8 fp16 weights) of MFMA step t from a lane slice and its
// group's half2 (scale, zero term):
//   MOEQ_DQ_HQQ_INT: (v + c) * s, c = -(1024 + z)   [z integer in 0..1023]
//   MOEQ_DQ_HQQ:     ((v - 1024) + (-z)) * s
//   MOEQ_DQ_AFFINE:  fma(v - 1024, s, z')
// v - 1024 = q and v + c = q - z are exact, so HQQ modes give
// fp16(fp16(q - z) * s), the fake-quant weight, and AFFINE GemLite's weight.
template <int BITS, int DQ>
__device__ __forceinline__ f16x8 deq_frag(const uint32_t (&w)[BITS], uint32_t sz, int t) {
  const f16 sh = __builtin_bit_cast(f16, uint16_t(sz & 0xffffu));
  const f16 zh = __builtin_bit_cast(f16, uint16_t(sz >> 16));
  const f16x2 s2 = {sh, sh}, z2 = {zh, zh};
  const f16x2 k1024 = {(f16)1024.0f, (f16)1024.0f};
  f16x8 r;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const f16x2 v = __builtin_bit_cast(f16x2, magic_pair<BITS>(w, t, d, 0x64006400u));
    f16x2 o;
    if constexpr (DQ == MOEQ_DQ_HQQ_INT)
      o = (v + z2) * s2;
    else if constexpr (DQ == MOEQ_DQ_HQQ)
      o = ((v - k1024) + z2) * s2;
    else
      o = __builtin_elementwise_fma(v - k1024, s2, z2);
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
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

template <int BM, int NW, int NB, int NP, int EPI, int ADT, int ODT, int BITS, int DQ, int MBA>
__device__ __forceinline__ void gemm_tile(const GemmArgs &g, int e, int row0, int mcount, int nt,
                                          int c0, int c1, uint4 (*As)[BM][16]) {
  constexpr int NT = NW * 64;
  static_assert(MBA * 16 <= BM, "active row blocks exceed the tile");
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, kb = lane >> 4;
  const int N = g.N;
  const int n_wave = nt * (NW * NB * 16) + wave * NB * 16;

  const uint32_t *wbase[NP];
  const uint32_t *sbase[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    wbase[p] = g.p[p].words + g.p[p].word_off[e];
    sbase[p] = g.p[p].sz + g.p[p].sz_off[e];
  }
  // columns past N read column N - 1 and are never stored
  int ncol[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) ncol[nb] = min(n_wave + nb * 16 + l16, N - 1);

  f32x4 acc[NP][MBA][NB];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int mb = 0; mb < MBA; ++mb)
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
        load_slice<BITS>(wbase[p] + ((int64_t(c) * N + ncol[nb]) * 4 + kb) * BITS, w[p][nb]);
        s[p][nb] = sbase[p][int64_t(grp) * N + ncol[nb]];
      }
  };
  auto advance = [&]() {
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        scur[p][nb] = snxt[p][nb];
#pragma unroll
        for (int j = 0; j < BITS; ++j) wcur[p][nb][j] = wnxt[p][nb][j];
      }
  };

  const char *abytes = static_cast<const char *>(g.a);

  if constexpr (BM == 16) {
    // ---------------- decode shapes: A fragments straight from global memory
    constexpr int AES = 2;
    const int rr = row0 + min(l16, mcount - 1);
    const int64_t src = g.row_src ? int64_t(g.row_src[rr]) : int64_t(rr);
    const char *arow = abytes + src * g.lda * AES;
    uint4 acur[4], anxt[4];
    auto load_a = [&](int c, uint4 (&av)[4]) {
      const uint4 *p = reinterpret_cast<const uint4 *>(arow + (int64_t(c) * 128 + 32 * kb) * AES);
#pragma unroll
      for (int t = 0; t < 4; ++t) av[t] = p[t];
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
        const f16x8 A = to_f16x8<ADT>(acur[t]);
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            const f16x8 B = deq_frag<BITS, DQ>(wcur[p][nb], scur[p][nb], t);
            acc[p][0][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, acc[p][0][nb], 0, 0, 0);
          }
      }
      if (c + 1 < c1) {
#pragma unroll
        for (int t = 0; t < 4; ++t) acur[t] = anxt[t];
        advance();
      }
    }
  } else {
    // ---------------- prefill shapes: A copied global -> LDS, double buffered.
    // Unit u (16 bytes) of row r lives at As[buf][r][u ^ (r & 15)]; one
    // global_load_lds_dwordx4 writes 64 consecutive units (4 rows).
    constexpr int UNITS = MBA * 16 * 16;
    constexpr int SEGS = UNITS / NT;
    static_assert(SEGS >= 1 && UNITS % NT == 0, "A staging split");
    // byte offsets of this lane's source units (activations are < 2 GiB)
    uint32_t aoff[SEGS];
#pragma unroll
    for (int j = 0; j < SEGS; ++j) {
      const int gu = (j * NW + wave) * 64 + lane;  // LDS unit written by this lane
      const int r = gu >> 4, pu = gu & 15, u = pu ^ (r & 15);
      const int rr = row0 + min(r, mcount - 1);
      const int64_t src = g.row_src ? int64_t(g.row_src[rr]) : int64_t(rr);
      aoff[j] = uint32_t((src * g.lda + u * 8) * 2);
    }
    auto load_a = [&](int c, int buf) {
#pragma unroll
      for (int j = 0; j < SEGS; ++j) {
        char *dst = reinterpret_cast<char *>(&As[buf][0][0]) + (j * NW + wave) * 64 * 16;
        __builtin_amdgcn_global_load_lds(abytes + aoff[j] + uint32_t(c) * 256u, (lds_void *)dst, 16, 0, 0);
      }
    };
    if (c0 < c1) {
      load_a(c0, 0);
      load_b(c0, wcur, scur);
    }
    __syncthreads();
    for (int c = c0; c < c1; ++c) {
      const int buf = (c - c0) & 1;
      const bool more = c + 1 < c1;
      if (more) {
        load_a(c + 1, buf ^ 1);
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
        for (int mb = 0; mb < MBA; ++mb) {
          const int r = mb * 16 + l16;
          const f16x8 A = __builtin_bit_cast(f16x8, As[buf][r][(4 * kb + t) ^ l16]);
#pragma unroll
          for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
              acc[p][mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B[p][nb], acc[p][mb][nb], 0, 0, 0);
        }
      }
      if (more) advance();
      __syncthreads();
    }
  }

  // ---------------- epilogue: D[row = 4 * (lane / 16) + i][col = lane % 16]
  char *obytes = static_cast<char *>(g.out);
  const int split = blockIdx.z;
#pragma unroll
  for (int mb = 0; mb < MBA; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int col = n_wave + nb * 16 + l16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = mb * 16 + 4 * kb + i;
        if (r >= mcount || col >= N) continue;
        const int64_t o = int64_t(row0 + r) * g.ldo + col;
        if constexpr (EPI == MOEQ_EPI_SILU_MUL) {
          const float h = silu_mul(acc[0][mb][nb][i], acc[NP - 1][mb][nb][i]);
          reinterpret_cast<uint16_t *>(obytes)[o] = f32_to_f16_bits(h);
        } else if constexpr (ODT == MOEQ_F32) {
          reinterpret_cast<float *>(obytes)[split * g.split_stride + o] = acc[0][mb][nb][i];
        } else {
          reinterpret_cast<uint16_t *>(obytes)[split * g.split_stride + o] = f32_to_f16_bits(acc[0][mb][nb][i]);
        }
      }
    }
}

template <int BM, int NW, int NB, int NP, int EPI, int ADT, int ODT, int BITS, int DQ>
__device__ __forceinline__ void gemm_tile_mba(const GemmArgs &g, int e, int row0, int mcount, int nt, int c0,
                                              int c1, uint4 (*As)[BM][16]) {
  const int mb_act = (mcount + 15) >> 4;
#define MOEQ_T(M) gemm_tile<BM, NW, NB, NP, EPI, ADT, ODT, BITS, DQ, M>(g, e, row0, mcount, nt, c0, c1, As)
  if constexpr (BM == 16) {
    MOEQ_T(1);
  } else if constexpr (BM == 32) {
    MOEQ_T(2);
  } else if constexpr (BM == 64) {
    if (mb_act <= 2) MOEQ_T(2); else MOEQ_T(4);
  } else {
    if (mb_act <= 2) MOEQ_T(2); else if (mb_act <= 4) MOEQ_T(4); else MOEQ_T(8);
  }
#undef MOEQ_T
}

// Two work-groups per CU for the LDS-staged shapes (2 waves per SIMD).
template <int BM, int NW, int NB, int NP, int EPI, int ADT, int ODT>
__global__ __launch_bounds__(NW * 64, BM == 16 ? 1 : 2) void grouped_gemm_kernel(GemmArgs g) {
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
  const int dq = g.dq_mode;
#define MOEQ_TILE(B, D) gemm_tile_mba<BM, NW, NB, NP, EPI, ADT, ODT, B, D>(g, e, row0, mcount, nt, c0, c1, As)
#define MOEQ_BITS(B)                                                   \
  if (dq == MOEQ_DQ_HQQ_INT) MOEQ_TILE(B, MOEQ_DQ_HQQ_INT);           \
  else if (dq == MOEQ_DQ_HQQ) MOEQ_TILE(B, MOEQ_DQ_HQQ);              \
  else MOEQ_TILE(B, MOEQ_DQ_AFFINE);
  switch (bits) {
    case 1: MOEQ_BITS(1) break;
    case 2: MOEQ_BITS(2) break;
    case 3: MOEQ_BITS(3) break;
    default: MOEQ_BITS(4) break;
  }
#undef MOEQ_BITS
#undef MOEQ_TILE
}

// Launch shapes: (NW waves, NB 16-column blocks per wave) for each BM and
// epilogue.  Column tile width = NW * NB * 16.
template <int BM, bool SILU>
struct Shape;
template <> struct Shape<16, true> { static constexpr int NW = 4, NB = 1; };
template <> struct Shape<16, false> { static constexpr int NW = 4, NB = 2; };
template <> struct Shape<32, true> { static constexpr int NW = 4, NB = 2; };
template <> struct Shape<32, false> { static constexpr int NW = 4, NB = 4; };
template <> struct Shape<64, true> { static constexpr int NW = 4, NB = 2; };
template <> struct Shape<64, false> { static constexpr int NW = 4, NB = 4; };
template <> struct Shape<128, true> { static constexpr int NW = 4, NB = 2; };
template <> struct Shape<128, false> { static constexpr int NW = 4, NB = 4; };

// Launches one configuration (defined in gemm_bm<BM>.hip).
template <int BM>
int launch_grouped_gemm(const GemmArgs &g, bool silu, int a_dtype, int out_dtype, int max_tiles, int splits,
                        hipStream_t s);

template <int BM, bool SILU, int ADT, int ODT>
inline int launch_one(const GemmArgs &g0, int max_tiles, int splits, hipStream_t s) {
  using S = Shape<BM, SILU>;
  GemmArgs g = g0;
  g.n_ntiles = int(cdiv(g.N, S::NW * S::NB * 16));
  const int64_t blocks = int64_t(max_tiles) * g.n_ntiles;
  if (blocks > 0x7fffffff) return fail(MOEQ_ERR_UNSUPPORTED, "grouped_gemm: grid too large");
  dim3 grid(unsigned(blocks), 1, unsigned(splits)), block(S::NW * 64);
  grouped_gemm_kernel<BM, S::NW, S::NB, SILU ? 2 : 1, SILU ? MOEQ_EPI_SILU_MUL : MOEQ_EPI_STORE, ADT, ODT>
      <<<grid, block, 0, s>>>(g);
  return check_launch("grouped_gemm");
}

}  // namespace moeq
