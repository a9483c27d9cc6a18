// 256-row prefill tile of the grouped GEMM: one wave per SIMD, accumulators
// resident in AGPRs.  Included by gemm_bm256.hip.
//
// The prefill tiles of gemm_impl.h run two waves per SIMD, so each wave has
// 256 registers; 160 of them hold accumulators and the dequantized B fragment
// of one MFMA step feeds at most 10 row blocks.  Here a work-group of four
// waves owns a CU (one wave per SIMD, 512 registers each): the 256
// accumulators of a wave (16 row blocks x 4 fragments of 16 columns) live in
// the AGPRs and the VGPRs hold the operands, so
//   * one dequantized B fragment feeds 16 row blocks (16 MFMAs per 14 or so
//     VALU instructions of unpacking instead of 10), and
//   * the fragments of step t + 1 are unpacked while step t's MFMAs run (two
//     register sets), with no register pressure pushing the unpacking back
//     into the MFMA stream.
// The MFMAs are written as inline asm with "+a" accumulator operands, the one
// way to keep the compiler from staging accumulators through VGPRs (with the
// builtin it parks them in AGPRs as spill slots and copies them back and
// forth).
//
// Issue order.  With one wave per SIMD nothing fills the MFMA pipe's gaps but
// the wave itself.  Measured on gfx950 (16x16x32 f16, one wave per SIMD):
// back-to-back MFMAs issue every 18 cycles, and up to two independent VALU
// instructions between consecutive MFMAs cost nothing, while a third doubles
// the gap.  So every MFMA is fenced by a scheduling barrier and the step's
// unpacking is cut into single instructions (pair_op) dealt evenly over the
// gaps: OPS = pairs x ops-per-pair over MBA * NP * NB MFMAs, one instruction
// per gap for 1/2/4-bit codes at 16 row blocks.
//
// Hazards the compiler cannot see, since it does not know the asm is an MFMA:
//   * a VALU write of a VGPR followed by an MFMA reading it needs two wait
//     states.  MFMA sources are A fragments (LDS loads) and the B fragments
//     of the previous step; the last unpacking instruction of a step may
//     directly precede the next step's first MFMA, so each step starts with
//     s_nop 1 (which also covers copies the compiler places at the loop's
//     back edge, and the accumulators' zero initialisation);
//   * an MFMA's result read by a VALU instruction (the epilogue's AGPR reads)
//     needs the MFMA's passes plus a few wait states: the k loop ends with 24
//     wait states behind scheduling barriers;
//   * consecutive MFMAs on one accumulator are at least 7 MFMAs apart (4
//     fragments x 2 row blocks), far more than the dependent-accumulate
//     latency.
// A rows are staged global -> LDS exactly as in gemm_impl.h (XOR-swizzled
// 16-byte units, two 64 KB buffers).
#pragma once

#include "gemm_impl.h"

namespace moeq {

__device__ __forceinline__ void mfma_agpr(f32x4 &acc, const f16x8 &a, const f16x8 &b) {
  asm("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// Unpacking one pair of codes (deq_pair's arithmetic) as a sequence of single
// VALU instructions: the code pair ORed into the mantissa of 1024 (2 ops; 4
// for 3-bit codes, whose high bit sits in a third word), then the dequant
// mode's 2 or 3 ops.  pair_op(k) runs op k; the result lands in B[2d..2d+1].
template <int BITS>
constexpr int magic_ops() { return BITS == 3 ? 4 : 2; }
template <int DQ>
constexpr int deq_ops() { return DQ == MOEQ_DQ_HQQ ? 3 : 2; }

struct PairState {
  uint32_t x, m;
  f16x2 v;
};

template <int BITS, int DQ>
__device__ __forceinline__ void pair_op(int k, PairState &st, const uint32_t (&w)[BITS], uint32_t sz, int t, int d,
                                        f16x8 &B) {
  constexpr uint32_t magic = 0x64006400u;
  const f16 sh = __builtin_bit_cast(f16, uint16_t(sz & 0xffffu));
  const f16 zh = __builtin_bit_cast(f16, uint16_t(sz >> 16));
  const f16x2 s2 = {sh, sh}, z2 = {zh, zh};
  const f16x2 k1024 = {(f16)1024.0f, (f16)1024.0f};
  constexpr int MO = magic_ops<BITS>();
  if (k < MO) {
    if constexpr (BITS == 4) {
      if (k == 0) st.x = w[t] >> (4 * d);
      else st.m = and_or(st.x, 0x000f000fu, magic);
    } else if constexpr (BITS == 2) {
      if (k == 0) st.x = w[t >> 1] >> (8 * (t & 1) + 2 * d);
      else st.m = and_or(st.x, 0x00030003u, magic);
    } else if constexpr (BITS == 1) {
      if (k == 0) st.x = w[0] >> (4 * t + d);
      else st.m = and_or(st.x, 0x00010001u, magic);
    } else {
      const int hb = 4 * t + d;
      if (k == 0) st.x = w[t >> 1] >> (8 * (t & 1) + 2 * d);
      else if (k == 1) st.m = and_or(st.x, 0x00030003u, magic);
      else if (k == 2) st.x = hb >= 2 ? (w[2] >> (hb - 2)) : (w[2] << (2 - hb));
      else st.m = and_or(st.x, 0x00040004u, st.m);
    }
    return;
  }
  const int j = k - MO;
  f16x2 r;
  if constexpr (DQ == MOEQ_DQ_HQQ_INT) {
    if (j == 0) { st.v = __builtin_bit_cast(f16x2, st.m) + z2; return; }
    r = st.v * s2;
  } else if constexpr (DQ == MOEQ_DQ_HQQ) {
    if (j == 0) { st.v = __builtin_bit_cast(f16x2, st.m) - k1024; return; }
    if (j == 1) { st.v = st.v + z2; return; }
    r = st.v * s2;
  } else {
    if (j == 0) { st.v = __builtin_bit_cast(f16x2, st.m) - k1024; return; }
    r = __builtin_elementwise_fma(st.v, s2, z2);
  }
  B[2 * d] = r[0];
  B[2 * d + 1] = r[1];
}

template <int NB, int NP, int EPI, int ODT, int BITS, int DQ, int MBA>
__device__ __forceinline__ void wide_tile(const GemmArgs &g, int e, int row0, int mcount, int nt, int c0, int c1,
                                          uint4 (*As0)[16], uint4 (*As1)[16]) {
  constexpr int NW = 4, NT = NW * 64;
  static_assert(MBA <= 16, "a wave holds at most 16 row blocks");
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, kb = lane >> 4;
  const int N = g.N;
  const int n_wave = nt * (NW * NB * 16) + wave * NB * 16;

  const char *wbase[NP];
  const char *sbase[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    wbase[p] = reinterpret_cast<const char *>(g.p[p].words + g.p[p].word_off[e]);
    sbase[p] = reinterpret_cast<const char *>(g.p[p].sz + g.p[p].sz_off[e]);
  }
  const int groups = g.gshift >= 0 ? g.K >> g.gshift : g.K / g.group_size;
  uint32_t woff[NB], soff[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int ncol = min(n_wave + nb * 16 + l16, N - 1);
    woff[nb] = slice_byte_off<BITS>(ncol, kb, g.nchunks);
    soff[nb] = sz_byte_off(ncol, groups);
  }
  constexpr int64_t chunk_bytes = chunk_step_bytes<BITS>();
  constexpr uint32_t grp_bytes = kGroupStepBytes;

  f32x4 acc[NP][MBA][NB];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int mb = 0; mb < MBA; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[p][mb][nb] = (f32x4){0.f, 0.f, 0.f, 0.f};

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

  // A staging: MBA * 256 units of 16 bytes per chunk, MBA per thread.
  constexpr int SEGS = MBA * 16 * 16 / NT;
  const char *abytes = static_cast<const char *>(g.a);
  uint32_t aoff[SEGS];
#pragma unroll
  for (int j = 0; j < SEGS; ++j) {
    const int gu = (j * NW + wave) * 64 + lane;
    const int r = gu >> 4, pu = gu & 15, u = pu ^ (r & 15);
    const int rr = row0 + min(r, mcount - 1);
    const int64_t src = g.row_src ? int64_t(g.row_src[rr]) : int64_t(rr);
    aoff[j] = uint32_t((src * g.lda + u * 8) * 2);
  }
  const __amdgpu_buffer_rsrc_t arsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(abytes), (short)0, 0x7fffffff, 0x00020000);
  auto load_a = [&](int c, uint4 (*dstA)[16]) {
#pragma unroll
    for (int j = 0; j < SEGS; ++j) {
      char *dst = reinterpret_cast<char *>(&dstA[0][0]) + (j * NW + wave) * 64 * 16;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (lds_void *)dst, 16, aoff[j], uint32_t(c) * 256u, 0, 0);
    }
  };

  uint32_t w0[NP][NB][BITS], w1[NP][NB][BITS], s0[NP][NB], s1[NP][NB];
  f16x8 Bc[NP][NB];
  // Each MFMA step issues its MBA * NP * NB MFMAs one per scheduling
  // region; region i also carries ops [i * OPS / S, (i + 1) * OPS / S) of the
  // next step's unpacking (NP * NB * 4 pairs, in order) and, at the start of
  // each row block, the LDS read of the A fragment two row blocks ahead (into
  // the next step while the chunk lasts; a chunk's first two are read after
  // its barrier).
  constexpr int S = MBA * NP * NB;
  constexpr int NOPS = magic_ops<BITS>() + deq_ops<DQ>();
  constexpr int OPS = NP * NB * 4 * NOPS;
  auto chunk = [&](int c, uint4 (*Ard)[16], uint4 (*Awr)[16], const uint32_t (&wc)[NP][NB][BITS],
                   const uint32_t (&sc)[NP][NB], uint32_t (&wn)[NP][NB][BITS], uint32_t (&sn)[NP][NB]) {
    // next chunk fetched unconditionally (the last chunk re-reads itself)
    const int cn = min(c + 1, c1 - 1);
    load_a(cn, Awr);
    load_b(cn, wn, sn);
    auto read_a = [&](int t, int mb) {
      return __builtin_bit_cast(f16x8, Ard[mb * 16 + l16][(4 * kb + t) ^ l16]);
    };
    f16x8 Aq[4 * MBA + 2];  // fragments in (step, row block) order
    Aq[0] = read_a(0, 0);
    if constexpr (MBA > 1) Aq[1] = read_a(0, 1);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      // the previous step's last unpacking op may write a B fragment this
      // step's first MFMA reads: two wait states
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_nop 1");
      __builtin_amdgcn_sched_barrier(0);
      f16x8 Bn[NP][NB];
      PairState st[NP * NB * 4];
#pragma unroll
      for (int i = 0; i < S; ++i) {
        const int mb = i / (NP * NB), f = i % (NP * NB), p = f / NB, nb = f % NB;
        if (f == 0) {
          const int q = t * MBA + mb + 2;  // fragment read two row blocks ahead
          if (q < 4 * MBA) Aq[q] = read_a(q / MBA, q % MBA);
        }
#pragma unroll
        for (int o = i * OPS / S; o < (i + 1) * OPS / S; ++o) {
          const int j = o / NOPS, k = o % NOPS;
          const int fj = j >> 2, d = j & 3, pj = fj / NB, nbj = fj % NB;
          if (t < 3)
            pair_op<BITS, DQ>(k, st[j], wc[pj][nbj], sc[pj][nbj], t + 1, d, Bn[pj][nbj]);
          else
            pair_op<BITS, DQ>(k, st[j], wn[pj][nbj], sn[pj][nbj], 0, d, Bn[pj][nbj]);
        }
        mfma_agpr(acc[p][mb][nb], Aq[t * MBA + mb], Bc[p][nb]);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) Bc[p][nb] = Bn[p][nb];
    }
    __syncthreads();
  };
  if (c0 < c1) {
    load_a(c0, As0);
    load_b(c0, w0, s0);
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) Bc[p][nb] = deq_frag<BITS, DQ>(w0[p][nb], s0[p][nb], 0);
  // pairs of chunks, then an odd last one: no branch inside the loop body,
  // whose join would have the accumulators copied out of the AGPRs and back
  int c = c0;
  for (; c + 1 < c1; c += 2) {
    chunk(c, As0, As1, w0, s0, w1, s1);
    chunk(c + 1, As1, As0, w1, s1, w0, s0);
  }
  if (c < c1) chunk(c, As0, As1, w0, s0, w1, s1);
  // the last MFMAs' results are read by VALU instructions below
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);

  // epilogue: D[row = 16 mb + 4 (lane / 16) + i][col = lane % 16], as gemm_tile's
  constexpr int OES = (EPI == MOEQ_EPI_SILU_MUL || ODT != MOEQ_F32) ? 2 : 4;
  const int64_t ldo_b = g.ldo * OES;
  char *const tile_out =
      static_cast<char *>(g.out) + (int64_t(blockIdx.z) * g.split_stride + int64_t(row0) * g.ldo) * OES;
  const uint32_t lane_off = uint32_t(4 * kb) * uint32_t(ldo_b) + uint32_t((n_wave + l16) * OES);
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

// Four waves per work-group and OCC work-groups per CU (OCC waves per SIMD,
// 512 / OCC registers each); tiles of up to MAXB row blocks, whose two A
// buffers take 2 * MAXB * 4 KB of LDS.
template <int NB, int NP, int EPI, int ODT, int MAXB, int OCC>
__global__ __launch_bounds__(256, OCC) void wide_gemm_kernel(GemmArgs g) {
  static_assert(NP * NB * MAXB * 4 <= 256 / OCC, "accumulators exceed the AGPRs of a wave");
  const unsigned V = unsigned(*g.n_tiles) * unsigned(g.n_ntiles);
  const unsigned b = blockIdx.x;
  if (b >= V) return;
  const unsigned L = xcd_block(b, V, unsigned(g.n_ntiles));
  const int mt = int(L / unsigned(g.n_ntiles));
  const int nt = int(L % unsigned(g.n_ntiles));
  __shared__ uint4 As0[MAXB * 16][16];
  __shared__ uint4 As1[MAXB * 16][16];
  const int32_t *tp = g.tiles + 4 * mt;
  const int e = tp[0], row0 = tp[1], mcount = tp[2];
  const int c0 = int(blockIdx.z) * g.chunks_per_split;
  const int c1 = min(c0 + g.chunks_per_split, g.nchunks);
  const int bits = g.p[0].nbits[e];
  const int dq = g.dq_mode;
  const int mb_act = (mcount + 15) >> 4;
#define MOEQ_W(B, D, M) wide_tile<NB, NP, EPI, ODT, B, D, M>(g, e, row0, mcount, nt, c0, c1, As0, As1)
#define MOEQ_WM(B, D)                                                   \
  if constexpr (MAXB == 16) {                                           \
    if (mb_act <= 2) MOEQ_W(B, D, 2);                                   \
    else if (mb_act <= 4) MOEQ_W(B, D, 4);                              \
    else if (mb_act <= 8) MOEQ_W(B, D, 8);                              \
    else if (mb_act <= 10) MOEQ_W(B, D, 10);                            \
    else MOEQ_W(B, D, 16);                                              \
  } else {                                                              \
    static_assert(MAXB == 8, "row-block variants for 8 or 16 blocks");  \
    if (mb_act <= 2) MOEQ_W(B, D, 2);                                   \
    else if (mb_act <= 4) MOEQ_W(B, D, 4);                              \
    else if (mb_act <= 6) MOEQ_W(B, D, 6);                              \
    else MOEQ_W(B, D, 8);                                               \
  }
#define MOEQ_WB(B)                                           \
  if (dq == MOEQ_DQ_HQQ_INT) { MOEQ_WM(B, MOEQ_DQ_HQQ_INT) } \
  else if (dq == MOEQ_DQ_HQQ) { MOEQ_WM(B, MOEQ_DQ_HQQ) }    \
  else { MOEQ_WM(B, MOEQ_DQ_AFFINE) }
  switch (bits) {
    case 1: MOEQ_WB(1) break;
    case 2: MOEQ_WB(2) break;
    case 3: MOEQ_WB(3) break;
    default: MOEQ_WB(4) break;
  }
#undef MOEQ_WB
#undef MOEQ_WM
#undef MOEQ_W
}

}  // namespace moeq
