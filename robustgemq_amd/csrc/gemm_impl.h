// Grouped mixed-bit GEMM over all experts of a MoE layer on
// v_mfma_f32_16x16x32_f16 (gfx950).  Included by gemm_bm*.hip, each of which
// instantiates one row-tile height BM.
//
// One launch covers every (row tile, column tile) of every expert; the row
// tiles come from the device-side schedule written by moeq_permute (each
// expert's rows in tiles of at most tile_rows(BM) rows), so no
// host synchronisation is needed.  A block has NW waves; wave w owns NB * 16 output columns and all
// active rows of the tile.  Per 128-deep K chunk:
//   A (activations, gathered rows): BM >= 32 -> copied global -> LDS with
//      buffer_load_dwordx4 ... lds (no register staging), 16-byte units XOR-
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

#include <type_traits>

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
  int K, N, group_size, gshift, dq_mode;  // gshift = log2(group_size), or -1
  ProjDev p[2];
  void *out;
  int64_t ldo, split_stride;
  int n_ntiles, nchunks, chunks_per_split;
  // most rows any tile of this launch can hold (0: the class capacity);
  // 16-row launches at most 16 run the kernel without the two-block path
  int max_rows;
  // average rows per hit expert the caller expects (0: unknown); 16-row
  // launches of tall tiles take twice the columns per wave
  int rows_hint;
  // number of row tiles when the caller knows it (one-token forwards: k +
  // shared experts), or 0: the launch then need not read it from n_tiles
  // before its tile lookup
  int known_tiles;
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
__device__ __forceinline__ f16x2 deq_pair(const uint32_t (&w)[BITS], uint32_t sz, int t, int d) {
  const f16 sh = __builtin_bit_cast(f16, uint16_t(sz & 0xffffu));
  const f16 zh = __builtin_bit_cast(f16, uint16_t(sz >> 16));
  const f16x2 s2 = {sh, sh}, z2 = {zh, zh};
  const f16x2 k1024 = {(f16)1024.0f, (f16)1024.0f};
  const f16x2 v = __builtin_bit_cast(f16x2, magic_pair<BITS>(w, t, d, 0x64006400u));
  if constexpr (DQ == MOEQ_DQ_HQQ_INT)
    return (v + z2) * s2;
  else if constexpr (DQ == MOEQ_DQ_HQQ)
    return ((v - k1024) + z2) * s2;
  else
    return __builtin_elementwise_fma(v - k1024, s2, z2);
}

template <int BITS, int DQ>
__device__ __forceinline__ f16x8 deq_frag(const uint32_t (&w)[BITS], uint32_t sz, int t) {
  f16x8 r;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const f16x2 o = deq_pair<BITS, DQ>(w, sz, t, d);
    r[2 * d] = o[0];
    r[2 * d + 1] = o[1];
  }
  return r;
}

// Build-layout addressing (moeq_repack, moeq_prep_scales).  Panel p = n / 16
// holds the lane slices of its 16 columns chunk after chunk: slice (c, n, kb)
// at word ((p * nchunks + c) * 64 + (n % 16) * 4 + kb) * BITS, so the slices
// of chunk c + 1 follow those of chunk c (256 * BITS bytes on); the
// scale/zero pair of group g at dword (p * groups + g) * 16 + n % 16 (64 bytes
// from one group to the next).  Byte offsets of chunk / group 0; one expert's
// codes and pairs stay below 2 GiB (checked at launch).
template <int BITS>
__device__ __forceinline__ uint32_t slice_byte_off(int n, int kb, int nchunks) {
  return uint32_t(((int64_t(n >> 4) * nchunks * 64) + (n & 15) * 4 + kb) * BITS * 4);
}
template <int BITS>
constexpr int64_t chunk_step_bytes() { return 256 * BITS; }
__device__ __forceinline__ uint32_t sz_byte_off(int n, int groups) {
  return uint32_t((int64_t(n >> 4) * groups * 16 + (n & 15)) * 4);
}
constexpr uint32_t kGroupStepBytes = 64;

// A buffer resource over `base` (wave-uniform): loads through it take a
// 32-bit lane offset and a scalar offset, so no 64-bit lane addresses are
// formed; offsets past 2 GiB read zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7fffffff, 0x00020000);
}

// One lane slice (BITS words) at byte offset voff + soff of a buffer.
template <int BITS>
__device__ __forceinline__ void load_slice_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                               uint32_t (&w)[BITS]) {
  if constexpr (BITS == 4) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, int(voff), int(soff), 0);
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
  } else if constexpr (BITS == 3) {
    const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(r, int(voff), int(soff), 0);
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2];
  } else if constexpr (BITS == 2) {
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, int(voff), int(soff), 0);
    w[0] = v[0]; w[1] = v[1];
  } else {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, int(voff), int(soff), 0);
  }
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

template <int BM, int NW, int NB, int NP, int EPI, int ADT, int ODT, int BITS, int DQ, int MBA, bool KS>
__device__ __forceinline__ void gemm_tile(const GemmArgs &g, int e, int row0, int mcount, int nt,
                                          int c0, int c1, uint4 (*As0)[16], uint4 (*As1)[16]) {
  constexpr int NT = NW * 64;
  static_assert(MBA * 16 <= tile_rows(BM), "active row blocks exceed the tile");
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, kb = lane >> 4;
  const int N = g.N;
  // KS (16-row blocks of small launches): all waves share the block's
  // columns and split K instead
  const int n_wave = KS ? nt * (NB * 16) : nt * (NW * NB * 16) + wave * NB * 16;

  // Expert bases are wave-uniform; each lane adds 32-bit byte offsets (one
  // expert's words and scales stay far below 2 GiB).
  const char *wbase[NP];
  const char *sbase[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    wbase[p] = reinterpret_cast<const char *>(g.p[p].words + g.p[p].word_off[e]);
    sbase[p] = reinterpret_cast<const char *>(g.p[p].sz + g.p[p].sz_off[e]);
  }
  // columns past N read column N - 1 and are never stored
  const int groups = g.gshift >= 0 ? g.K >> g.gshift : g.K / g.group_size;
  uint32_t woff[NB], soff[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int ncol = min(n_wave + nb * 16 + l16, N - 1);
    woff[nb] = slice_byte_off<BITS>(ncol, kb, g.nchunks);
    soff[nb] = sz_byte_off(ncol, groups);
  }
  constexpr int64_t chunk_bytes = chunk_step_bytes<BITS>();  // one 128-deep chunk of a panel
  constexpr uint32_t grp_bytes = kGroupStepBytes;            // one group of a panel

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
    const int k = c * 128 + 32 * kb;
    const uint32_t grp = uint32_t(g.gshift >= 0 ? k >> g.gshift : k / g.group_size);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const char *wc = wbase[p] + int64_t(c) * chunk_bytes;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        load_slice<BITS>(reinterpret_cast<const uint32_t *>(wc + woff[nb]), w[p][nb]);
        s[p][nb] = *reinterpret_cast<const uint32_t *>(sbase[p] + (grp * grp_bytes + soff[nb]));
      }
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
    // ---------------- decode shapes: A fragments straight from global memory.
    // KS (small launches): the NW waves share the block's columns and take
    // interleaved K chunks (wave w: chunks c0 + w, c0 + w + NW, ...), their
    // partial sums meeting in LDS afterwards; otherwise each wave owns NB * 16
    // columns and runs all chunks.  A wave with at most 8 chunks fetches all
    // of them at once, a longer one keeps a 4-chunk ring in flight.  Steps
    // past a wave's last chunk re-read a valid chunk and multiply it by a
    // zero A fragment, so every fetch and MFMA is unconditional (no joins for
    // the wait counts to merge).  A tile of two 16-row blocks (MBA = 2: an
    // expert with 17..32 rows, one pass over its weights instead of two)
    // fetches both blocks' fragments and keeps to the ring past 4 chunks.
    constexpr int AES = 2;
    const char *arow[MBA];
#pragma unroll
    for (int mb = 0; mb < MBA; ++mb) {
      const int rr = row0 + min(16 * mb + l16, mcount - 1);
      const int64_t src = g.row_src ? int64_t(g.row_src[rr]) : int64_t(rr);
      arow[mb] = abytes + src * g.lda * AES;
    }
    const int cfirst = KS ? c0 + wave : c0, cstep = KS ? NW : 1;
    const int nc = KS ? (c1 > c0 + wave ? (c1 - c0 - wave + NW - 1) / NW : 0) : max(c1 - c0, 0);
    auto fetch = [&](int j, uint4 (&av)[MBA][4], uint32_t (&w)[NP][NB][BITS], uint32_t (&sz)[NP][NB]) {
      // a K-split wave with no chunk of its own (fewer chunks than waves, or
      // an empty split) still fetches a valid chunk, c1 - 1, times zero
      const int c = max(min(cfirst + cstep * min(j, max(nc - 1, 0)), c1 - 1), 0);
#pragma unroll
      for (int mb = 0; mb < MBA; ++mb) {
        const uint4 *pa = reinterpret_cast<const uint4 *>(arow[mb] + (int64_t(c) * 128 + 32 * kb) * AES);
#pragma unroll
        for (int t = 0; t < 4; ++t) av[mb][t] = pa[t];
      }
      load_b(c, w, sz);
    };
    auto step = [&](bool live, const uint4 (&av)[MBA][4], const uint32_t (&w)[NP][NB][BITS],
                    const uint32_t (&sz)[NP][NB]) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        f16x8 A[MBA];
#pragma unroll
        for (int mb = 0; mb < MBA; ++mb) A[mb] = live ? to_f16x8<ADT>(av[mb][t]) : f16x8{};
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            const f16x8 B = deq_frag<BITS, DQ>(w[p][nb], sz[p][nb], t);
#pragma unroll
            for (int mb = 0; mb < MBA; ++mb)
              acc[p][mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[mb], B, acc[p][mb][nb], 0, 0, 0);
          }
      }
    };
    auto all_at_once = [&](auto slots) {
      constexpr int S = decltype(slots)::value;
      uint4 ar[S][MBA][4];
      uint32_t wr[S][NP][NB][BITS], sr[S][NP][NB];
#pragma unroll
      for (int j = 0; j < S; ++j) fetch(j, ar[j], wr[j], sr[j]);
#pragma unroll
      for (int j = 0; j < S; ++j) step(j < nc, ar[j], wr[j], sr[j]);
    };
    if (nc == 1) {
      all_at_once(std::integral_constant<int, 1>{});
    } else if (nc == 2) {
      all_at_once(std::integral_constant<int, 2>{});
    } else if (nc > 2 && nc <= 4) {
      all_at_once(std::integral_constant<int, 4>{});
    } else if (MBA == 1 && nc > 4 && nc <= 8) {
      all_at_once(std::integral_constant<int, 8>{});
    } else if (nc > 4) {
      constexpr int DEPTH = 4;
      uint4 ar[DEPTH][MBA][4];
      uint32_t wr[DEPTH][NP][NB][BITS], sr[DEPTH][NP][NB];
#pragma unroll
      for (int d = 0; d < DEPTH - 1; ++d) fetch(d, ar[d], wr[d], sr[d]);
      for (int j0 = 0; j0 < nc; j0 += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
          const int nx = (d + DEPTH - 1) % DEPTH;
          fetch(j0 + d + DEPTH - 1, ar[nx], wr[nx], sr[nx]);
          step(j0 + d < nc, ar[d], wr[d], sr[d]);
        }
      }
    }
    // KS: partial sums of the NW waves -> wave 0, added in wave order
    if constexpr (KS) {
      float *red = reinterpret_cast<float *>(&As0[0][0]);
      static_assert((NW - 1) * NP * MBA * NB * 4 * 64 * 4 <= 96 * 16 * 16, "K-split partials exceed As0");
      if (wave > 0) {
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int mb = 0; mb < MBA; ++mb)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
              for (int i = 0; i < 4; ++i)
                red[((((wave - 1) * NP + p) * MBA + mb) * NB * 4 + nb * 4 + i) * 64 + lane] = acc[p][mb][nb][i];
      }
      __syncthreads();
      if (wave > 0) return;
#pragma unroll
      for (int w = 1; w < NW; ++w)
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int mb = 0; mb < MBA; ++mb)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
              for (int i = 0; i < 4; ++i)
                acc[p][mb][nb][i] += red[((((w - 1) * NP + p) * MBA + mb) * NB * 4 + nb * 4 + i) * 64 + lane];
    }
  } else {
    // ---------------- prefill shapes: A copied global -> LDS, double buffered
    // in two separate arrays.  Unit u (16 bytes) of row r lives at
    // A[r][u ^ (r & 15)]; one buffer_load_dwordx4 ... lds writes 64
    // consecutive units (4 rows).  The chunk loop is unrolled by two so every
    // LDS access names its buffer at compile time: the copy into one buffer
    // then never makes the fragment reads of the other wait for it.
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
    // Buffer loads take the lane's 32-bit offset plus the chunk's scalar
    // offset, so no per-lane 64-bit addresses are kept.
    const __amdgpu_buffer_rsrc_t arsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(abytes), (short)0, 0x7fffffff, 0x00020000);
    auto load_a = [&](int c, uint4 (*dstA)[16]) {
#pragma unroll
      for (int j = 0; j < SEGS; ++j) {
        char *dst = reinterpret_cast<char *>(&dstA[0][0]) + (j * NW + wave) * 64 * 16;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (lds_void *)dst, 16, aoff[j], uint32_t(c) * 256u, 0, 0);
      }
    };
    auto chunk = [&](int c, uint4 (*Ard)[16], uint4 (*Awr)[16]) {
      // Fetch the next chunk unconditionally (the last chunk re-reads
      // itself into the idle buffer): a conditional fetch joins two paths,
      // and the wait counts merged at the join would wait for it at once.
      const int cn = min(c + 1, c1 - 1);
      load_a(cn, Awr);
      load_b(cn, wnxt, snxt);
      // A fragments in (step, row block) order, each read from LDS one row
      // block ahead: the scheduling groups pin every read before the MFMAs of
      // the previous fragment, so its latency runs under them (left to
      // itself the scheduler reads two fragments and waits for them at once)
      f16x8 Acur = __builtin_bit_cast(f16x8, Ard[l16][(4 * kb) ^ l16]);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        f16x8 B[NP][NB];
        if (t == 0) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) B[p][nb] = deq_frag<BITS, DQ>(wcur[p][nb], scur[p][nb], t);
#pragma unroll
        for (int mb = 0; mb < MBA; ++mb) {
          f16x8 Anext = Acur;
          if (mb + 1 < MBA) Anext = __builtin_bit_cast(f16x8, Ard[(mb + 1) * 16 + l16][(4 * kb + t) ^ l16]);
          else if (t < 3) Anext = __builtin_bit_cast(f16x8, Ard[l16][(4 * kb + t + 1) ^ l16]);
#pragma unroll
          for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
              acc[p][mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Acur, B[p][nb], acc[p][mb][nb], 0, 0, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);        // LDS read
          __builtin_amdgcn_sched_group_barrier(0x008, NP * NB, 0);  // MFMA
          Acur = Anext;
        }
      }
      advance();
      __syncthreads();
    };
    if (c0 < c1) {
      load_a(c0, As0);
      load_b(c0, wcur, scur);
    }
    __syncthreads();
    for (int c = c0; c < c1; c += 2) {
      chunk(c, As0, As1);
      if (c + 1 < c1) chunk(c + 1, As1, As0);
    }
  }

  // ---------------- epilogue: D[row = 16 mb + 4 (lane / 16) + i][col = lane % 16].
  // Each output row starts at a wave-uniform (scalar) address; the lane adds
  // a 32-bit offset.  Column blocks past N are skipped per wave (N % 16 == 0)
  // and only the tile's partial last row block tests rows per lane.
  constexpr int OES = (EPI == MOEQ_EPI_SILU_MUL || ODT != MOEQ_F32) ? 2 : 4;
  const int64_t ldo_b = g.ldo * OES;
  char *const tile_out =
      static_cast<char *>(g.out) + (int64_t(blockIdx.z) * g.split_stride + int64_t(row0) * g.ldo) * OES;
  const uint32_t lane_off = uint32_t(4 * kb) * uint32_t(ldo_b) + uint32_t((n_wave + l16) * OES);
  if constexpr (BM >= 32 && OES == 2) {
    // Prefill tiles with 16-bit outputs go out through LDS: the waves leave
    // their fp16 results in the two A buffers (row r of the tile at row
    // r % RPB of buffer r / RPB, 16-byte units XOR-swizzled by (r / 4) % 4 so
    // the four row groups of one store hit disjoint banks), then every thread
    // writes whole 16-byte row pieces, so each row's columns leave as full
    // cache lines instead of 2-byte stores per accumulator.  Needs 16-byte
    // aligned output rows (the layer's h and y are).
    constexpr int COLS = NW * NB * 16;
    constexpr int UPR = COLS / 8;                    // 16-byte units per staged row
    constexpr int RPB = tile_rows(BM) * 128 / COLS;  // staged rows per A buffer
    static_assert(UPR >= 8 && (UPR & (UPR - 1)) == 0, "staged rows: a power of two of at least 8 units");
    static_assert(2 * RPB >= MBA * 16, "staged tile exceeds the A buffers");
    if (((reinterpret_cast<uintptr_t>(tile_out) | uintptr_t(ldo_b)) & 15) == 0) {
      // the last chunk's repeated prefetch may still be landing in a buffer
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      char *const sb0 = reinterpret_cast<char *>(&As0[0][0]);
      char *const sb1 = reinterpret_cast<char *>(&As1[0][0]);
      auto srow = [&](int r) { return r < RPB ? sb0 + r * (COLS * 2) : sb1 + (r - RPB) * (COLS * 2); };
      auto swz = [](int r) { return ((r >> 2) & 3) << 1; };
      const int cw = wave * NB * 16;  // the wave's first column in the tile
#pragma unroll
      for (int mb = 0; mb < MBA; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 16 * mb + 4 * kb + i, c = cw + nb * 16 + l16;
            uint16_t v;
            if constexpr (EPI == MOEQ_EPI_SILU_MUL) v = f32_to_f16_bits(silu_mul(acc[0][mb][nb][i], acc[NP - 1][mb][nb][i]));
            else v = f32_to_f16_bits(acc[0][mb][nb][i]);
            *reinterpret_cast<uint16_t *>(srow(r) + (((c >> 3) ^ swz(r)) << 4) + (c & 7) * 2) = v;
          }
      __syncthreads();
      const int rows = min(MBA * 16, mcount);
      const int col0 = nt * COLS;
      for (int q = int(threadIdx.x); q < rows * UPR; q += NT) {
        const int r = q / UPR, u = q % UPR, col = col0 + u * 8;
        if (col < N)
          *reinterpret_cast<uint4 *>(tile_out + int64_t(r) * ldo_b + col * 2) =
              *reinterpret_cast<const uint4 *>(srow(r) + ((u ^ swz(r)) << 4));
      }
      return;
    }
  }
  auto put = [&](int mb, int nb, int i) {
    char *p = tile_out + int64_t(16 * mb + i) * ldo_b + (lane_off + uint32_t(nb * 16 * OES));
    if constexpr (EPI == MOEQ_EPI_SILU_MUL) {
      *reinterpret_cast<uint16_t *>(p) = f32_to_f16_bits(silu_mul(acc[0][mb][nb][i], acc[NP - 1][mb][nb][i]));
    } else if constexpr (ODT == MOEQ_F32) {
      *reinterpret_cast<float *>(p) = acc[0][mb][nb][i];
    } else {
      *reinterpret_cast<uint16_t *>(p) = f32_to_f16_bits(acc[0][mb][nb][i]);
    }
  };
#pragma unroll
  for (int mb = 0; mb < MBA; ++mb) {
    if (16 * (mb + 1) <= mcount) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if (n_wave + nb * 16 >= N) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) put(mb, nb, i);
      }
    } else if (16 * mb < mcount) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if (n_wave + nb * 16 >= N) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (16 * mb + 4 * kb + i < mcount) put(mb, nb, i);
      }
    }
  }
}

template <int BM, int NW, int NB, int NP, int EPI, int ADT, int ODT, int BITS, int DQ, bool KS, bool MB2>
__device__ __forceinline__ void gemm_tile_mba(const GemmArgs &g, int e, int row0, int mcount, int nt, int c0,
                                              int c1, uint4 (*As0)[16], uint4 (*As1)[16]) {
  const int mb_act = (mcount + 15) >> 4;
#define MOEQ_T(M) gemm_tile<BM, NW, NB, NP, EPI, ADT, ODT, BITS, DQ, M, KS>(g, e, row0, mcount, nt, c0, c1, As0, As1)
  if constexpr (BM == 16) {
    if constexpr (MB2) {
      if (mb_act <= 1) MOEQ_T(1); else MOEQ_T(2);
    } else {
      MOEQ_T(1);
    }
  } else if constexpr (BM == 32) {
    if (mb_act <= 2) MOEQ_T(2); else MOEQ_T(3);
  } else if constexpr (BM == 64) {
    if (mb_act <= 2) MOEQ_T(2); else if (mb_act <= 4) MOEQ_T(4); else MOEQ_T(6);
  } else {
    static_assert(BM == 128, "the 256-row class has its own kernel (gemm_wide.h)");
    if (mb_act <= 2) MOEQ_T(2); else if (mb_act <= 4) MOEQ_T(4); else if (mb_act <= 8) MOEQ_T(8); else MOEQ_T(10);
  }
#undef MOEQ_T
}

// Block b of a launch of V live blocks -> block L of the tile list (tile
// L / n_ntiles, column tile L % n_ntiles).  Work-groups are dealt to the 8
// XCDs round-robin, so XCD x = b % 8 takes its k-th block as block L: the
// list (first V8 = V & ~7 blocks) is cut into 64 segments of ln = V8 / 64
// blocks and XCD x gets segments x, x + 8, x + 16, ...  A segment keeps
// neighbouring tiles together (a row tile's column tiles, then the expert's
// next row tile), so they share the expert's weights and the activation rows
// through one L2, while tiles of different sizes (the list runs largest
// first) spread over the XCDs; the blocks left over go to the XCDs as equal
// runs after the segments.
__device__ __forceinline__ unsigned xcd_block(unsigned b, unsigned V, unsigned n_ntiles) {
  const unsigned V8 = V & ~7u;
  if (b >= V8) return b;
  constexpr unsigned XG = 8;
  const unsigned x = b & 7u, k = b >> 3, per = V8 >> 3, ln = per / XG;
  if (ln == 0) return x * per + k;
  return k < XG * ln ? ((k / ln) * 8u + x) * ln + k % ln : 8u * XG * ln + x * (per - XG * ln) + (k - XG * ln);
}

// Two work-groups per CU for the 32..128 classes (tiles of up to 48..160
// rows): 2 waves per SIMD.
template <int BM, int NW, int NB, int NP, int EPI, int ADT, int ODT, bool KS, bool MB2 = true>
__global__ __launch_bounds__(NW * 64, BM == 16 ? 1 : 2) void grouped_gemm_kernel(GemmArgs g) {
  // The grid is sized for the host-side bound on row tiles; blocks past the
  // real count (read from the device schedule) exit together; the live ones
  // are renumbered per XCD (xcd_block).
  const unsigned V = unsigned(g.known_tiles > 0 ? g.known_tiles : *g.n_tiles) * unsigned(g.n_ntiles);
  const unsigned b = blockIdx.x;
  if (b >= V) return;
  const unsigned L = xcd_block(b, V, unsigned(g.n_ntiles));
  const int mt = int(L / unsigned(g.n_ntiles));
  const int nt = int(L % unsigned(g.n_ntiles));
  // 16-row blocks use As0 for the cross-wave reduction: (NW - 1) * NP * MBA *
  // NB * 4 floats per lane, at most 24 KB.  The prefill classes hold tile_rows(BM)
  // rows per buffer (two 40 KB buffers for the 160-row class: two
  // work-groups fill the 160 KB of LDS).
  __shared__ uint4 As0[BM == 16 ? 96 : tile_rows(BM)][16];
  __shared__ uint4 As1[BM == 16 ? 1 : tile_rows(BM)][16];
  const int32_t *tp = g.tiles + 4 * mt;
  const int e = tp[0], row0 = tp[1], mcount = tp[2];
  const int c0 = int(blockIdx.z) * g.chunks_per_split;
  const int c1 = min(c0 + g.chunks_per_split, g.nchunks);
  const int bits = g.p[0].nbits[e];
  const int dq = g.dq_mode;
#define MOEQ_TILE(B, D) gemm_tile_mba<BM, NW, NB, NP, EPI, ADT, ODT, B, D, KS, MB2>(g, e, row0, mcount, nt, c0, c1, As0, As1)
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
// epilogue.  Column tile width = NW * NB * 16, except for 16-row blocks whose
// waves split K over the same NB * 16 columns.
template <int BM, bool SILU>
struct Shape;
template <class S, bool KS>
constexpr int tile_cols() { return KS ? S::NB * 16 : S::NW * S::NB * 16; }
template <> struct Shape<16, true> { static constexpr int NW = 4, NB = 1; };
template <> struct Shape<16, false> { static constexpr int NW = 4, NB = 2; };
template <> struct Shape<32, true> { static constexpr int NW = 4, NB = 2; };
template <> struct Shape<32, false> { static constexpr int NW = 4, NB = 4; };
template <> struct Shape<64, true> { static constexpr int NW = 4, NB = 2; };
template <> struct Shape<64, false> { static constexpr int NW = 4, NB = 4; };
template <> struct Shape<128, true> { static constexpr int NW = 4, NB = 2; };
template <> struct Shape<128, false> { static constexpr int NW = 4, NB = 4; };
// 256-row tiles (gemm_wide.h): 4 waves, one per SIMD, each with all rows and
// 32 + 32 (gate + up) or 64 columns: 256 accumulators per wave in the AGPRs.
template <> struct Shape<256, true> { static constexpr int NW = 4, NB = 2; };
template <> struct Shape<256, false> { static constexpr int NW = 4, NB = 4; };

// moeq_grouped_gemm for callers that know the most rows any tile holds
// (max_rows > 0; the layer forward: at most T per expert), which lets 16-row
// launches of at most 16 rows per tile skip the two-block kernel path.
int grouped_gemm_rows(const moeq_gemm *gm, const moeq_proj *p0, const moeq_proj *p1, int max_rows, int rows_hint,
                      int known_tiles, void *stream);

// One-token forwards: the down projection of the k routed rows plus the
// shared rows and the weighted combine in one launch (decode1.hip), given
// the one-token grouping (tiles, inv_perm, w) and the SiLU * up rows h.
int launch_down_combine1(const moeq_proj *w2, const uint16_t *h, const int32_t *tiles, const int32_t *inv_perm,
                         const float *w, int k, int n_shared, void *out, int out_dtype, hipStream_t s);

// Launches one configuration (defined in gemm_bm<BM>.hip).
template <int BM>
int launch_grouped_gemm(const GemmArgs &g, bool silu, int a_dtype, int out_dtype, int max_tiles, int splits,
                        hipStream_t s);

template <int BM, bool SILU, int ADT, int ODT, bool KS = false, bool MB2 = true, int NBW = Shape<BM, SILU>::NB>
inline int launch_one(const GemmArgs &g0, int max_tiles, int splits, hipStream_t s) {
  using S = Shape<BM, SILU>;
  static_assert(!KS || BM == 16, "K split over waves is a 16-row block variant");
  GemmArgs g = g0;
  g.n_ntiles = int(cdiv(g.N, KS ? NBW * 16 : S::NW * NBW * 16));
  const int64_t blocks = int64_t(max_tiles) * g.n_ntiles;
  if (blocks > 0x7fffffff) return fail(MOEQ_ERR_UNSUPPORTED, "grouped_gemm: grid too large");
  dim3 grid(unsigned(blocks), 1, unsigned(splits)), block(S::NW * 64);
  grouped_gemm_kernel<BM, S::NW, NBW, SILU ? 2 : 1, SILU ? MOEQ_EPI_SILU_MUL : MOEQ_EPI_STORE, ADT, ODT, KS, MB2>
      <<<grid, block, 0, s>>>(g);
  return check_launch("grouped_gemm");
}

}  // namespace moeq
