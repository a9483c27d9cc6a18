// One-token layer tail: the down projection of the k routed rows and the
// shared experts' rows, and the top-k weighted combine, in one launch.
//
// For T = 1 the routed rows are the selected experts in id order, one row
// each, then the shared rows (the grouping route1_kernel writes).  A work-group
// owns 16 output columns of every row: its eight waves split the R * (F / 128)
// (row, chunk) units of the down projection into contiguous ranges, stream
// their weight slices through a fetch ring (unconditional fetches, clamped
// chunk indices, steps past a range multiplied by zero, as the grouped
// GEMM's decode tiles do), and leave one partial sum per (row, column) in
// LDS.  Wave 0 then adds the partials in wave order and forms
//   out[n] = sum_slot w[slot] * y[inv_perm[slot], n] + sum_v y[k + v, n]
// in fp32, slots ascending, shared rows last (the combine's order), rounding
// once to the output type.  No y buffer, no combine launch, no atomics.
//
// The activation row is the same for the 16 rows of the MFMA A fragment (one
// token), so every row of the 16 x 16 result holds y; lane l16 keeps column
// l16 in element 0.
#include "gemm_impl.h"
#include "routing.h"

namespace moeq {

constexpr int kD1Waves = 8;
constexpr int kD1MaxRows = 32;  // k + n_shared

struct Down1Args {
  const uint16_t *h;        // [R, K] fp16 (SiLU * up of the R rows)
  const int32_t *tiles;     // (expert, row, 1, 0) per row
  const int32_t *inv_perm;  // [k] row of each slot
  const float *w;           // [k] routing weights
  int R, k, K, N, group_size, gshift, dq_mode;
  uint32_t gmagic;  // ceil(2^32 / group_size)
  ProjDev p;                // down projection
  void *out;
  int out_dtype;
};

// Partial sums of row r over chunks [cb, ce) for the work-group's 16 columns.
template <int BITS, int DQ>
__device__ __forceinline__ float d1_segment(const Down1Args &a, int r, int cb, int ce, int n0) {
  const int lane = lane_id();
  const int l16 = lane & 15, kb = lane >> 4;
  const int e = a.tiles[4 * r];
  const char *wb = reinterpret_cast<const char *>(a.p.words + a.p.word_off[e]);
  const char *sb = reinterpret_cast<const char *>(a.p.sz + a.p.sz_off[e]);
  const int groups = a.gshift >= 0 ? a.K >> a.gshift : a.K / a.group_size;
  const uint32_t woff = slice_byte_off<BITS>(n0 + l16, kb, a.K / 128);
  const uint32_t soff = sz_byte_off(n0 + l16, groups);
  constexpr uint32_t chunk_bytes = uint32_t(chunk_step_bytes<BITS>());
  constexpr uint32_t grp_bytes = kGroupStepBytes;
  // buffer loads: the lane's 32-bit offset plus the chunk's scalar offset
  const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(wb), srs = buffer_rsrc(sb);
  const __amdgpu_buffer_rsrc_t ars = buffer_rsrc(reinterpret_cast<const char *>(a.h) + int64_t(r) * a.K * 2);
  const int nc = ce - cb;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  auto fetch = [&](int j, uint4 (&av)[4], uint32_t (&w)[BITS], uint32_t &sz) {
    const int c = cb + min(j, nc - 1);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(ars, int(64 * kb + 16 * t), c * 256, 0);
      av[t] = (uint4){v[0], v[1], v[2], v[3]};
    }
    load_slice_buf<BITS>(wrs, woff, uint32_t(c) * chunk_bytes, w);
    const uint32_t grp = __umulhi(uint32_t(c * 128 + 32 * kb), a.gmagic);
    sz = __builtin_amdgcn_raw_buffer_load_b32(srs, int(soff + grp * grp_bytes), 0, 0);
  };
  auto step = [&](bool live, const uint4 (&av)[4], const uint32_t (&w)[BITS], uint32_t sz) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const f16x8 A = live ? __builtin_bit_cast(f16x8, av[t]) : f16x8{};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, deq_frag<BITS, DQ>(w, sz, t), acc, 0, 0, 0);
    }
  };
  constexpr int DEPTH = 8;
  uint4 ar[DEPTH][4];
  uint32_t wr[DEPTH][BITS], sr[DEPTH];
  if (nc <= DEPTH) {
#pragma unroll
    for (int j = 0; j < DEPTH; ++j) fetch(j, ar[j], wr[j], sr[j]);
#pragma unroll
    for (int j = 0; j < DEPTH; ++j) step(j < nc, ar[j], wr[j], sr[j]);
  } else {
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
  return acc[0];
}

template <int DQ>
__device__ __forceinline__ float d1_dispatch(const Down1Args &a, int r, int cb, int ce, int n0) {
  switch (a.p.nbits[a.tiles[4 * r]]) {
    case 1: return d1_segment<1, DQ>(a, r, cb, ce, n0);
    case 2: return d1_segment<2, DQ>(a, r, cb, ce, n0);
    case 3: return d1_segment<3, DQ>(a, r, cb, ce, n0);
    default: return d1_segment<4, DQ>(a, r, cb, ce, n0);
  }
}

__global__ __launch_bounds__(kD1Waves * 64) void down_combine1_kernel(Down1Args a) {
  __shared__ float part[kD1Waves][kD1MaxRows][16];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15;
  const int n0 = blockIdx.x * 16;
  for (int r = 0; r < a.R; ++r)
    if (lane < 16) part[wave][r][lane] = 0.f;
  // this wave's contiguous range of the row-major (row, chunk) units
  const int nch = a.K / 128, units = a.R * nch;
  const int per = (units + kD1Waves - 1) / kD1Waves;
  const int u0 = wave * per, u1 = min(units, u0 + per);
  for (int u = u0; u < u1;) {
    const int r = u / nch, cb = u % nch, ce = min(nch, cb + (u1 - u));
    float v;
    if (a.dq_mode == MOEQ_DQ_HQQ_INT) v = d1_dispatch<MOEQ_DQ_HQQ_INT>(a, r, cb, ce, n0);
    else if (a.dq_mode == MOEQ_DQ_HQQ) v = d1_dispatch<MOEQ_DQ_HQQ>(a, r, cb, ce, n0);
    else v = d1_dispatch<MOEQ_DQ_AFFINE>(a, r, cb, ce, n0);
    if (lane < 16) part[wave][r][lane] = v;
    u += ce - cb;
  }
  __syncthreads();
  if (wave != 0 || lane >= 16) return;
  auto y = [&](int r) {
    float s = part[0][r][l16];
#pragma unroll
    for (int w = 1; w < kD1Waves; ++w) s += part[w][r][l16];
    return s;
  };
  float o = 0.f;
  for (int s = 0; s < a.k; ++s) o += a.w[s] * y(a.inv_perm[s]);
  for (int v = a.k; v < a.R; ++v) o += y(v);
  const int n = n0 + l16;
  if (a.out_dtype == MOEQ_F32) static_cast<float *>(a.out)[n] = o;
  else if (a.out_dtype == MOEQ_BF16) static_cast<uint16_t *>(a.out)[n] = f32_to_bf16(o);
  else static_cast<uint16_t *>(a.out)[n] = f32_to_f16_bits(o);
}

// Launches the fused tail for a one-token forward whose grouping (route1's:
// tiles, inv_perm, w) and SiLU * up rows h are in place.
int launch_down_combine1(const moeq_proj *w2, const uint16_t *h, const int32_t *tiles, const int32_t *inv_perm,
                         const float *w, int k, int n_shared, void *out, int out_dtype, hipStream_t s) {
  const int R = k + n_shared;
  if (R > kD1MaxRows) return fail(MOEQ_ERR_UNSUPPORTED, "down_combine1: %d rows > %d", R, kD1MaxRows);
  if (w2->N % 16 || w2->K % 128) return fail(MOEQ_ERR_UNSUPPORTED, "down_combine1: N=%d K=%d", w2->N, w2->K);
  Down1Args a{};
  a.h = h;
  a.tiles = tiles;
  a.inv_perm = inv_perm;
  a.w = w;
  a.R = R;
  a.k = k;
  a.K = w2->K;
  a.N = w2->N;
  a.group_size = w2->group_size;
  a.gshift = (w2->group_size & (w2->group_size - 1)) ? -1 : __builtin_ctz(unsigned(w2->group_size));
  a.gmagic = uint32_t(((uint64_t(1) << 32) + uint64_t(w2->group_size) - 1) / uint64_t(w2->group_size));
  a.dq_mode = w2->dq_mode;
  a.p = ProjDev{w2->words, w2->word_off, w2->sz, w2->sz_off, w2->nbits};
  a.out = out;
  a.out_dtype = out_dtype;
  down_combine1_kernel<<<dim3(unsigned(w2->N / 16)), dim3(kD1Waves * 64), 0, s>>>(a);
  return check_launch("down_combine1");
}

}  // namespace moeq
