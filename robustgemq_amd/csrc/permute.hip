// Stable token->expert grouping without host synchronisation.
//
// The pairs (t, slot) are visited in slot-major order p = slot * T + t, the
// order torch.where walks the [k, T] expert mask in the reference, and stably
// sorted by expert:
//   1. hist:    one wave per chunk of kChunk positions counts experts (LDS).
//   2. scan:    one block turns the chunk counts into per-(chunk, expert)
//               start rows, expert offsets and the row-tile schedule, and
//               writes the rows of the shared experts.
//   3. scatter: one wave per chunk walks its positions in order, 64 at a
//               time; lanes with the same expert are found with one ballot
//               per key bit, ranked by lane order, and placed after the
//               rows already emitted for that expert.
#include <algorithm>

#include "common.h"

namespace moeq {

constexpr int kChunk = 512;
constexpr int kMaxExperts = 1024;  // routed + shared

__device__ __forceinline__ int pair_expert(const int32_t *idx, int64_t p, int64_t T, int k,
                                           int64_t *t_out, int *slot_out) {
  int slot = int(p / T);
  int64_t t = p - int64_t(slot) * T;
  *t_out = t;
  *slot_out = slot;
  return idx[t * k + slot];
}

__global__ __launch_bounds__(256) void hist_kernel(const int32_t *idx, int64_t T, int k, int E,
                                                   int64_t nchunks, int32_t *cc) {
  extern __shared__ int32_t smem[];
  const int w = threadIdx.x >> 6, lane = lane_id();
  const int64_t chunk = int64_t(blockIdx.x) * 4 + w;
  int32_t *cnt = smem + w * E;
  for (int e = lane; e < E; e += 64) cnt[e] = 0;
  __syncthreads();
  if (chunk < nchunks) {
    const int64_t P = T * k, p0 = chunk * kChunk;
    for (int it = 0; it < kChunk; it += 64) {
      int64_t p = p0 + it + lane;
      if (p < P) {
        int64_t t;
        int slot;
        int e = pair_expert(idx, p, T, k, &t, &slot);
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
      }
    }
  }
  __syncthreads();
  if (chunk < nchunks)
    for (int e = lane; e < E; e += 64) cc[chunk * E + e] = cnt[e];
}

// Single block.  cc[nchunks][E] (chunk counts) becomes the first row of each
// (chunk, expert) in place.
__global__ __launch_bounds__(1024) void scan_kernel(
    int32_t *cc, int64_t nchunks, int64_t T, int k, int E, int n_shared, int bm,
    int max_tiles, int32_t *counts, int32_t *offsets, int32_t *row_token, int32_t *tiles,
    int32_t *n_tiles) {
  __shared__ int32_t s_cnt[kMaxExperts];
  __shared__ int32_t s_off[kMaxExperts + 1];
  __shared__ int32_t s_ntile[kMaxExperts];
  __shared__ int32_t s_rt[kMaxExperts];
  __shared__ int32_t s_tbase[kMaxExperts + 1];
  const int Et = E + n_shared;
  for (int e = threadIdx.x; e < Et; e += blockDim.x) {
    int32_t c = 0;
    if (e < E)
      for (int64_t ch = 0; ch < nchunks; ++ch) c += cc[ch * E + e];
    else
      c = int32_t(T);
    s_cnt[e] = c;
    counts[e] = c;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t run = 0, trun = 0;
    for (int e = 0; e < Et; ++e) {
      s_off[e] = run;
      run += s_cnt[e];
      // ceil(m / bm) tiles of near-equal height, rounded up to 16 rows
      int32_t m = s_cnt[e], nt = 0, rt = 16;
      if (m > 0) {
        int32_t nmt = (m + bm - 1) / bm;
        rt = ((m + nmt - 1) / nmt + 15) / 16 * 16;
        nt = (m + rt - 1) / rt;
      }
      s_ntile[e] = nt;
      s_rt[e] = rt;
      s_tbase[e] = trun;
      trun += nt;
    }
    s_off[Et] = run;
    s_tbase[Et] = trun;
    // moeq_max_tiles bounds trun for any routing; the clamp only keeps a
    // corrupted idx from writing past the schedule buffer
    *n_tiles = min(trun, max_tiles);
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= Et; e += blockDim.x) offsets[e] = s_off[e];
  for (int e = threadIdx.x; e < Et; e += blockDim.x) {
    int32_t m = s_cnt[e], nt = s_ntile[e], rt = s_rt[e];
    if (nt > 0) {
      for (int32_t j = 0; j < nt && s_tbase[e] + j < max_tiles; ++j) {
        int32_t r0 = j * rt;
        int32_t rc = min(rt, m - r0);
        int32_t *tp = tiles + 4 * (s_tbase[e] + j);
        tp[0] = e;
        tp[1] = s_off[e] + r0;
        tp[2] = rc;
        tp[3] = 0;
      }
    }
    if (e < E) {
      int32_t run = s_off[e];
      for (int64_t ch = 0; ch < nchunks; ++ch) {
        int32_t c = cc[ch * E + e];
        cc[ch * E + e] = run;
        run += c;
      }
    }
  }
  // shared experts: T rows each, token order
  for (int v = 0; v < n_shared; ++v) {
    int32_t base = s_off[E + v];
    for (int64_t t = threadIdx.x; t < T; t += blockDim.x) row_token[base + t] = int32_t(t);
  }
}

__global__ __launch_bounds__(256) void scatter_kernel(const int32_t *idx, int64_t T, int k,
                                                      int E, int key_bits, int64_t nchunks,
                                                      const int32_t *base, int32_t *row_token,
                                                      int32_t *row_pair, int32_t *inv_perm) {
  extern __shared__ int32_t smem[];
  const int w = threadIdx.x >> 6, lane = lane_id();
  const int64_t chunk = int64_t(blockIdx.x) * 4 + w;
  if (chunk >= nchunks) return;  // no block-level barrier below
  int32_t *cnt = smem + w * E;
  for (int e = lane; e < E; e += 64) cnt[e] = base[chunk * E + e];
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  const int64_t P = T * k, p0 = chunk * kChunk;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int it = 0; it < kChunk; it += 64) {
    int64_t p = p0 + it + lane;
    bool valid = p < P;
    int64_t t = 0;
    int slot = 0, e = 0;
    if (valid) {
      e = pair_expert(idx, p, T, k, &t, &slot);
      valid = e >= 0 && e < E;  // out-of-range ids are dropped, never written
      if (!valid) e = 0;
    }
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < key_bits; ++b) {
      bool bit = (e >> b) & 1;
      uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    int rank = __popcll(peers & lt_mask);
    int32_t start = valid ? cnt[e] : 0;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    // the highest lane of each group publishes the new count
    if (valid && (peers >> lane) == 1ull) cnt[e] = start + __popcll(peers);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    if (valid) {
      int32_t pos = start + rank;
      int32_t pair = int32_t(t * k + slot);
      row_pair[pos] = pair;
      row_token[pos] = int32_t(t);
      inv_perm[pair] = pos;
    }
  }
}

}  // namespace moeq

using namespace moeq;

extern "C" int moeq_max_tiles(int64_t T, int top_k, int E, int n_shared, int bm) {
  if (T <= 0 || top_k <= 0 || E <= 0 || n_shared < 0 || bm <= 0) return 0;
  int64_t pairs = T * top_k;
  int64_t bound = pairs / bm + std::min<int64_t>(E, pairs) + int64_t(n_shared) * cdiv(T, bm);
  return int(bound);
}

extern "C" size_t moeq_permute_workspace_size(int64_t T, int top_k, int E, int n_shared) {
  (void)n_shared;
  if (T <= 0 || top_k <= 0 || E <= 0) return 0;
  return align256(size_t(cdiv(T * top_k, kChunk)) * size_t(E) * sizeof(int32_t));
}

extern "C" int moeq_permute(const int32_t *idx, int64_t T, int top_k, int E,
                            int n_shared, int bm, int32_t *counts, int32_t *offsets,
                            int32_t *row_token, int32_t *row_pair, int32_t *inv_perm,
                            int32_t *tiles, int32_t *n_tiles, void *ws, size_t ws_bytes,
                            void *stream) {
  if (!idx || !counts || !offsets || !row_token || !row_pair || !inv_perm || !tiles || !n_tiles)
    return fail(MOEQ_ERR_INVALID, "permute: null pointer");
  if (T <= 0 || top_k <= 0) return fail(MOEQ_ERR_INVALID, "permute: T=%lld top_k=%d", (long long)T, top_k);
  if (E <= 0 || n_shared < 0 || E + n_shared > kMaxExperts)
    return fail(MOEQ_ERR_UNSUPPORTED, "permute: n_experts=%d + n_shared=%d exceeds %d", E, n_shared, kMaxExperts);
  if (top_k > E) return fail(MOEQ_ERR_INVALID, "permute: top_k=%d > n_experts=%d", top_k, E);
  if (bm < 16 || bm % 16) return fail(MOEQ_ERR_INVALID, "permute: bm=%d must be a positive multiple of 16", bm);
  if (T * top_k > INT32_MAX / 2 || T * (top_k + n_shared) > INT32_MAX / 2)
    return fail(MOEQ_ERR_UNSUPPORTED, "permute: T=%lld too large", (long long)T);
  size_t need = moeq_permute_workspace_size(T, top_k, E, n_shared);
  if (!ws || ws_bytes < need)
    return fail(MOEQ_ERR_WORKSPACE, "permute: workspace %zu < %zu bytes", ws_bytes, need);
  int32_t *cc = static_cast<int32_t *>(ws);
  int64_t nchunks = cdiv(T * top_k, kChunk);
  int key_bits = 1;
  while ((1 << key_bits) < E) ++key_bits;
  hipStream_t s = as_stream(stream);
  dim3 grid(unsigned(cdiv(nchunks, 4))), block(256);
  size_t lds = size_t(4) * E * sizeof(int32_t);
  hist_kernel<<<grid, block, lds, s>>>(idx, T, top_k, E, nchunks, cc);
  int rc = check_launch("permute/hist");
  if (rc) return rc;
  const int max_tiles = moeq_max_tiles(T, top_k, E, n_shared, bm);
  scan_kernel<<<1, 1024, 0, s>>>(cc, nchunks, T, top_k, E, n_shared, bm, max_tiles, counts,
                                 offsets, row_token, tiles, n_tiles);
  rc = check_launch("permute/scan");
  if (rc) return rc;
  scatter_kernel<<<grid, block, lds, s>>>(idx, T, top_k, E, key_bits, nchunks, cc, row_token,
                                          row_pair, inv_perm);
  return check_launch("permute/scatter");
}
