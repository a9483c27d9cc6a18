// Load-time layout kernels: pack codes into the reference's int32 words,
// rewrite those words into the build layout, fuse scales and zeros.
#include "common.h"

namespace moeq {

// One thread per output word (r, n) of the [ceil(K/eps), N] result.
__global__ void pack_cols_kernel(const uint8_t *codes, int64_t N, int64_t K,
                                 int nbits, int32_t *out, int64_t rows) {
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * N) return;
  int64_t r = i / N, n = i % N;
  int eps = 32 / nbits;
  uint32_t mask = (1u << nbits) - 1u, w = 0;
  for (int j = 0; j < eps; ++j) {
    int64_t k = r * eps + j;
    if (k < K) w |= (uint32_t(codes[n * K + k]) & mask) << (j * nbits);
  }
  out[r * N + n] = int32_t(w);
}

// Build layout (see include/moeq.h, moeq_repack): lane slice (c, n, kb)
// holds the 32 codes k = 128c + 32kb + i, i = 8t + 2d + h, placed so that the
// pair (h = 0, 1) of MFMA step t, pair d sits at the same bit offset of the
// two 16-bit halves of one word.  Slices are stored panel-major: panel
// p = n / 16 holds its 16 columns' slices of chunk 0, then chunk 1, ...
// (memory order [p][c][n % 16][kb][word]), so one wave streaming a panel over
// K reads one contiguous run.  Bit positions inside a slice:
//   4-bit: word t,   bit 16h + 4d
//   2-bit: word t/2, bit 16h + 2(4(t%2) + d)
//   1-bit: word 0,   bit 16h + 4t + d
//   3-bit: low two bits as 2-bit in words 0..1, high bit as 1-bit in word 2.
template <int BITS>
__device__ __forceinline__ void place_code(uint32_t *w, int i, uint32_t q) {
  int t = i >> 3, d = (i & 7) >> 1, h = i & 1;
  if constexpr (BITS == 4) {
    w[t] |= q << (16 * h + 4 * d);
  } else if constexpr (BITS == 2) {
    w[t >> 1] |= q << (16 * h + 2 * (4 * (t & 1) + d));
  } else if constexpr (BITS == 1) {
    w[0] |= q << (16 * h + 4 * t + d);
  } else {
    w[t >> 1] |= (q & 3u) << (16 * h + 2 * (4 * (t & 1) + d));
    w[2] |= (q >> 2) << (16 * h + 4 * t + d);
  }
}

template <int BITS>
__global__ void repack_kernel(const int32_t *ref, int64_t K, int64_t N,
                              uint32_t *out) {
  int64_t s = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;  // slice id
  int64_t nslices = (K / 128) * N * 4;
  if (s >= nslices) return;
  int kb = int(s & 3);
  int64_t cn = s >> 2;
  int64_t n = cn % N, c = cn / N;
  // destination slice: [n / 16][c][n % 16][kb]
  const int64_t d = (((n >> 4) * (K / 128) + c) * 16 + (n & 15)) * 4 + kb;
  constexpr int eps = 32 / BITS;
  constexpr uint32_t mask = (1u << BITS) - 1u;
  uint32_t w[BITS];
#pragma unroll
  for (int j = 0; j < BITS; ++j) w[j] = 0;
  for (int i = 0; i < 32; ++i) {
    int64_t k = 128 * c + 32 * kb + i;
    uint32_t word = uint32_t(ref[(k / eps) * N + n]);
    uint32_t q = (word >> ((k % eps) * BITS)) & mask;
    place_code<BITS>(w, i, q);
  }
#pragma unroll
  for (int j = 0; j < BITS; ++j) out[d * BITS + j] = w[j];
}

// Element (g, n) of block b ([G, N] per block, one block per expert) goes to
// dword b * G * N + ((n / 16) * G + g) * 16 + n % 16: panel-major like the
// codes, so a panel's scale/zero pairs over all groups are one contiguous run.
__global__ void prep_scales_kernel(const uint16_t *s, const uint16_t *z, int64_t blocks, int64_t G,
                                   int64_t N, int mode, uint32_t *out) {
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= blocks * G * N) return;
  const int64_t b = i / (G * N), r = i % (G * N), g = r / N, n = r % N;
  uint32_t zb = z[i];
  if (mode == MOEQ_DQ_HQQ) zb ^= 0x8000u;  // -z: flip the fp16 sign bit
  if (mode == MOEQ_DQ_HQQ_INT) zb = f32_to_f16_bits(-(1024.0f + f16_bits_to_f32(uint16_t(zb))));
  out[b * G * N + ((n >> 4) * G + g) * 16 + (n & 15)] = uint32_t(s[i]) | (zb << 16);
}

}  // namespace moeq

using namespace moeq;

extern "C" int moeq_pack_cols(const uint8_t *codes, int64_t N, int64_t K,
                              int nbits, int32_t *out, void *stream) {
  if (!codes || !out) return fail(MOEQ_ERR_INVALID, "pack_cols: null pointer");
  if (nbits < 1 || nbits > 4) return fail(MOEQ_ERR_INVALID, "pack_cols: nbits=%d not in 1..4", nbits);
  if (N <= 0 || K <= 0) return fail(MOEQ_ERR_INVALID, "pack_cols: empty shape N=%lld K=%lld", (long long)N, (long long)K);
  int64_t rows = cdiv(K, 32 / nbits);
  int64_t total = rows * N;
  pack_cols_kernel<<<dim3(unsigned(cdiv(total, 256))), dim3(256), 0, as_stream(stream)>>>(
      codes, N, K, nbits, out, rows);
  return check_launch("pack_cols");
}

extern "C" int moeq_repack(const int32_t *ref_words, int64_t K, int64_t N,
                           int nbits, uint32_t *out, void *stream) {
  if (!ref_words || !out) return fail(MOEQ_ERR_INVALID, "repack: null pointer");
  if (K <= 0 || N <= 0 || K % 128) return fail(MOEQ_ERR_INVALID, "repack: K=%lld must be a positive multiple of 128", (long long)K);
  if (N % 16) return fail(MOEQ_ERR_INVALID, "repack: N=%lld must be a multiple of 16", (long long)N);
  int64_t slices = (K / 128) * N * 4;
  dim3 grid(unsigned(cdiv(slices, 256))), block(256);
  hipStream_t st = as_stream(stream);
  switch (nbits) {
    case 1: repack_kernel<1><<<grid, block, 0, st>>>(ref_words, K, N, out); break;
    case 2: repack_kernel<2><<<grid, block, 0, st>>>(ref_words, K, N, out); break;
    case 3: repack_kernel<3><<<grid, block, 0, st>>>(ref_words, K, N, out); break;
    case 4: repack_kernel<4><<<grid, block, 0, st>>>(ref_words, K, N, out); break;
    default: return fail(MOEQ_ERR_INVALID, "repack: nbits=%d not in 1..4", nbits);
  }
  return check_launch("repack");
}

extern "C" int moeq_prep_scales(const uint16_t *scales, const uint16_t *zeros, int64_t blocks,
                                int64_t groups, int64_t N, int dq_mode, uint32_t *out, void *stream) {
  if (!scales || !zeros || !out) return fail(MOEQ_ERR_INVALID, "prep_scales: null pointer");
  if (dq_mode != MOEQ_DQ_HQQ && dq_mode != MOEQ_DQ_AFFINE && dq_mode != MOEQ_DQ_HQQ_INT)
    return fail(MOEQ_ERR_INVALID, "prep_scales: dq_mode=%d", dq_mode);
  if (blocks <= 0 || groups <= 0 || N <= 0 || N % 16)
    return fail(MOEQ_ERR_INVALID, "prep_scales: blocks=%lld groups=%lld N=%lld (N a multiple of 16)",
                (long long)blocks, (long long)groups, (long long)N);
  const int64_t n = blocks * groups * N;
  prep_scales_kernel<<<dim3(unsigned(cdiv(n, 256))), dim3(256), 0, as_stream(stream)>>>(
      scales, zeros, blocks, groups, N, dq_mode, out);
  return check_launch("prep_scales");
}
