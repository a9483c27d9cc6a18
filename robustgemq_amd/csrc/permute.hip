// Stable token->expert grouping without host synchronisation.
//
// The pairs (t, slot) are visited in slot-major order p = slot * T + t, the
// order torch.where walks the [k, T] expert mask in the reference, and stably
// sorted by expert.  Three paths by batch size (E + n_shared <= 256 for the
// first two):
//   * up to 1024 pairs: one work-group holds every expert id in registers,
//     counts, scans and places them (permute_block);
//   * up to 65536 pairs: one work-group per 512 positions counts its chunk
//     (chunk_hist), then every work-group sums the chunk counts itself and
//     places its chunk (chunk_scatter);
//   * beyond: hist (one wave per chunk), scan (one block turns the chunk
//     counts into per-(chunk, expert) start rows), scatter.
// Placing 64 pairs at a time: lanes with the same expert are found with one
// ballot per key bit, ranked by lane order, and put after the rows already
// emitted for that expert.
#include <algorithm>

#include "routing.h"

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

// Exclusive prefix sum of one int per thread over the whole block (blockDim
// a multiple of 64, <= 1024).  `sh` holds >= 17 ints of LDS; *total gets the
// block sum.  Contains barriers: every thread of the block must call it.
__device__ int block_exclusive_scan(int v, int *sh, int *total) {
  const int lane = lane_id(), w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int t = __shfl_up(incl, o);
    if (lane >= o) incl += t;
  }
  if (lane == 63) sh[w] = incl;
  __syncthreads();
  if (w == 0) {
    int tv = lane < nw ? sh[lane] : 0, ti = tv;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      int t = __shfl_up(ti, o);
      if (lane >= o) ti += t;
    }
    if (lane < nw) sh[lane] = ti - tv;
    if (lane == nw - 1) sh[16] = ti;
  }
  __syncthreads();
  const int r = sh[w] + incl - v;
  *total = sh[16];
  __syncthreads();
  return r;
}

// The same over one packed 64-bit value per thread (three 21-bit counts).
__device__ uint64_t block_exclusive_scan64(uint64_t v, uint64_t *sh, uint64_t *total) {
  const int lane = lane_id(), w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  uint64_t incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t t = __shfl_up(incl, o);
    if (lane >= o) incl += t;
  }
  if (lane == 63) sh[w] = incl;
  __syncthreads();
  if (w == 0) {
    const uint64_t tv = lane < nw ? sh[lane] : 0;
    uint64_t ti = tv;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t t = __shfl_up(ti, o);
      if (lane >= o) ti += t;
    }
    if (lane < nw) sh[lane] = ti - tv;
    if (lane == nw - 1) sh[16] = ti;
  }
  __syncthreads();
  const uint64_t r = sh[w] + incl - v;
  *total = sh[16];
  __syncthreads();
  return r;
}

// Given per-expert row counts (one per thread e < Et), writes counts,
// offsets, the tile schedule and the shared-expert rows; returns this
// expert's first row.  Every thread of the block must call it.
__device__ int schedule(int c, int E, int n_shared, int64_t T, int bm, int max_tiles,
                        int32_t *counts, int32_t *offsets, int32_t *row_token, int32_t *tiles,
                        int32_t *n_tiles, int *sh, int *s_off) {
  const int e = threadIdx.x, Et = E + n_shared;
  const int m = e < Et ? c : 0;
  // An expert's rows in ceil(m / cap) tiles cut at 16-row block boundaries.
  // A tile of b blocks runs the kernel variant with the smallest
  // block count >= b, so the first x tiles take the class's largest count
  // smax and the rest the next lower count s2, x being the fewest that hold
  // all B blocks: an expert of 17 blocks at smax = 10 runs 10 + 8 = 18
  // blocks, where two halves of 8.5 blocks would run 10 + 10.
  const int cap = tile_rows(bm);
  const int smax = cap / 16, s2 = tile_blocks_below(bm);
  const int B = (m + 15) / 16;
  const int nt = (B + smax - 1) / smax;
  const int x = smax == s2 ? nt : min(nt, max(0, (B - s2 * nt + (smax - s2) - 1) / (smax - s2)));
  // The list runs by kernel variant of each expert's first (largest) tile,
  // largest first: class 0 = more than s2 blocks (the largest variant),
  // class 1 = more than the variant below s2, class 2 = the rest; experts in
  // order within a class, and an expert's tiles together, so they run at the
  // same time and share the expert's weights through one L2 (listed by
  // their own classes, an expert's second tile ran a round later and fetched
  // the weights again).  The dispatcher starts the longest tiles first and
  // the short ones fill the end of the launch.
  const int below = tile_blocks_below2(bm);
  auto tile_blocks = [&](int j, int &b0) {
    b0 = j < x ? j * smax : x * smax + (j - x) * s2;
    return min(b0 + (j < x ? smax : s2), B) - b0;
  };
  auto cls = [&](int nb) { return nb > s2 ? 0 : nb > below ? 1 : 2; };
  int b00;
  const int ecls = nt > 0 ? cls(tile_blocks(0, b00)) : 0;
  const uint64_t mine = uint64_t(nt) << (21 * ecls);
  __shared__ uint64_t sh64[17];
  int tot_rows;
  uint64_t tot_cls;
  const int off = block_exclusive_scan(m, sh, &tot_rows);
  const uint64_t before = block_exclusive_scan64(mine, sh64, &tot_cls);
  constexpr uint64_t kF = (uint64_t(1) << 21) - 1;
  const int t0 = int(tot_cls & kF), t1 = int((tot_cls >> 21) & kF), t2 = int(tot_cls >> 42);
  int pos0 = int(before & kF), pos1 = t0 + int((before >> 21) & kF), pos2 = t0 + t1 + int(before >> 42);
  if (e < Et) {
    counts[e] = c;
    offsets[e] = off;
    s_off[e] = off;
  }
  if (e == 0) {
    offsets[Et] = tot_rows;
    // moeq_max_tiles bounds the count for any routing; the clamp only keeps
    // a corrupted idx from writing past the schedule buffer
    *n_tiles = min(t0 + t1 + t2, max_tiles);
  }
  for (int j = 0; j < nt; ++j) {
    // (nt - 1) * smax < B, so every tile before the last is full and the
    // last one holds at least one block
    int b0;
    const int nb = tile_blocks(j, b0);
    const int at = ecls == 0 ? pos0++ : ecls == 1 ? pos1++ : pos2++;
    if (at >= max_tiles) continue;
    const int r0 = 16 * b0, r1 = min(16 * (b0 + nb), m);
    int32_t *tp = tiles + 4 * at;
    tp[0] = e;
    tp[1] = off + r0;
    tp[2] = r1 - r0;
    tp[3] = 0;
  }
  __syncthreads();
  for (int v = 0; v < n_shared; ++v)
    for (int64_t t = threadIdx.x; t < T; t += blockDim.x) row_token[s_off[E + v] + t] = int32_t(t);
  return off;
}

// Single block of 1024 threads.  cc[nchunks][E] (chunk counts) becomes the
// first row of each (chunk, expert) in place.
__global__ __launch_bounds__(1024) void scan_kernel(
    int32_t *cc, int64_t nchunks, int64_t T, int k, int E, int n_shared, int bm,
    int max_tiles, int32_t *counts, int32_t *offsets, int32_t *row_token, int32_t *tiles,
    int32_t *n_tiles) {
  __shared__ int sh[17];
  __shared__ int s_off[kMaxExperts];
  const int e = threadIdx.x;
  int c = 0;
  if (e < E) {
#pragma unroll 8
    for (int64_t ch = 0; ch < nchunks; ++ch) c += cc[ch * E + e];
  } else if (e < E + n_shared) {
    c = int(T);
  }
  const int off = schedule(c, E, n_shared, T, bm, max_tiles, counts, offsets, row_token, tiles, n_tiles, sh,
                           s_off);
  if (e < E) {
    int run = off;
    for (int64_t ch = 0; ch < nchunks; ++ch) {
      const int v = cc[ch * E + e];
      cc[ch * E + e] = run;
      run += v;
    }
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


// Rank of this lane among the lanes of the wave holding the same key
// (valid lanes only), and the size of that group.
__device__ __forceinline__ void peer_rank(bool valid, int e, int key_bits, int *rank, int *group,
                                          bool *leader) {
  const int lane = lane_id();
  uint64_t peers = __ballot(valid);
  for (int b = 0; b < key_bits; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t m = __ballot(bit);
    peers &= bit ? m : ~m;
  }
  const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  *rank = __popcll(peers & lt);
  *group = __popcll(peers);
  *leader = valid && (peers >> lane) == 1ull;
}

// Everything in one work-group (16 waves) for up to kFusedPairs pairs: wave
// w owns the slice [w * 64 * PPL, (w + 1) * 64 * PPL) of the slot-major
// sequence and loads all its expert ids into registers at once (one memory
// round trip); it counts them, the block scans the counts into slice bases,
// then each wave places its slice in order, 64 pairs at a time.
constexpr int kFusedWaves = 16;
constexpr int kFusedMaxPPL = 4;
constexpr int kFusedPairs = kFusedWaves * 64 * kFusedMaxPPL;
constexpr int kFusedExperts = 256;
// moeq_permute keeps batches of at most this many pairs in one work-group
// and gives larger ones to the two chunked launches below: at 4096 pairs the
// single work-group's dozen dependent barrier steps took 12 us, the two
// launches 6-7 us less (the top-k + permutation work-group of small decode
// batches still takes up to kFusedPairs).
constexpr int kOneGroupPairs = kFusedWaves * 64;

template <int PPL>
__device__ void permute_block(
    const int32_t *idx, int64_t T, int k, int E, int n_shared, int bm, int max_tiles, int key_bits,
    int32_t *counts, int32_t *offsets, int32_t *row_token, int32_t *row_pair, int32_t *inv_perm,
    int32_t *tiles, int32_t *n_tiles) {
  __shared__ int cnt[kFusedWaves][kFusedExperts];
  __shared__ int sh[17];
  __shared__ int s_off[kFusedExperts + 8];
  const int w = threadIdx.x >> 6, lane = lane_id();
  const int P = int(T) * k;  // <= kFusedPairs
  const int Ti = int(T);
  for (int i = threadIdx.x; i < kFusedWaves * kFusedExperts; i += blockDim.x) (&cnt[0][0])[i] = 0;
  // expert of pair p = slot * T + t (-1: past the end or an id outside 0..E-1)
  int ex[PPL];
  const int p0 = w * 64 * PPL + lane;
#pragma unroll
  for (int j = 0; j < PPL; ++j) {
    const int p = p0 + 64 * j;
    const int sl = p / Ti, t = p - sl * Ti;
    const int e = p < P ? idx[int64_t(t) * k + sl] : -1;
    ex[j] = (e >= 0 && e < E) ? e : -1;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < PPL; ++j)
    if (ex[j] >= 0) atomicAdd(&cnt[w][ex[j]], 1);
  __syncthreads();
  const int e = threadIdx.x;
  int c = 0;
  if (e < E) {
    for (int ww = 0; ww < kFusedWaves; ++ww) c += cnt[ww][e];
  } else if (e < E + n_shared) {
    c = int(T);
  }
  const int off = schedule(c, E, n_shared, T, bm, max_tiles, counts, offsets, row_token, tiles, n_tiles, sh,
                           s_off);
  if (e < E) {
    int run = off;
    for (int ww = 0; ww < kFusedWaves; ++ww) {
      const int v = cnt[ww][e];
      cnt[ww][e] = run;
      run += v;
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < PPL; ++j) {
    const bool valid = ex[j] >= 0;
    const int exj = valid ? ex[j] : 0;
    int rank, group;
    bool leader;
    peer_rank(valid, exj, key_bits, &rank, &group, &leader);
    const int start = valid ? cnt[w][exj] : 0;
    __builtin_amdgcn_wave_barrier();
    if (leader) cnt[w][exj] = start + group;
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      const int p = p0 + 64 * j;
      const int sl = p / Ti, t = p - sl * Ti;
      const int pos = start + rank;
      const int pair = t * k + sl;
      row_pair[pos] = pair;
      row_token[pos] = t;
      inv_perm[pair] = pos;
    }
  }
}

// Mid-size batches (kOneGroupPairs < T * k <= kChunkedPairs, E + n_shared <=
// 256): two launches of one 256-thread work-group per kWgChunk positions.
// The first counts each chunk's experts; the second has every work-group sum
// the chunk counts itself (totals, and the prefix over earlier chunks), so no
// separate scan launch is needed, and place its chunk in order.  Work-group
// 0 also writes counts, offsets, the tile schedule and the shared rows.
constexpr int kWgChunk = 512;
constexpr int kChunkedPairs = 65536;

__global__ __launch_bounds__(256) void chunk_hist_kernel(const int32_t *idx, int64_t T, int k, int E,
                                                         int32_t *cc) {
  __shared__ int cnt[kFusedExperts];
  const int c = blockIdx.x, Ti = int(T), P = int(T) * k;
  for (int i = threadIdx.x; i < E; i += 256) cnt[i] = 0;
  int ex[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int p = c * kWgChunk + 256 * j + threadIdx.x;
    const int sl = p / Ti, t = p - sl * Ti;
    const int e = p < P ? idx[int64_t(t) * k + sl] : -1;
    ex[j] = (e >= 0 && e < E) ? e : -1;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j)
    if (ex[j] >= 0) atomicAdd(&cnt[ex[j]], 1);
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 256) cc[int64_t(c) * E + e] = cnt[e];
}

__global__ __launch_bounds__(256) void chunk_scatter_kernel(
    const int32_t *idx, int64_t T, int k, int E, int n_shared, int bm, int max_tiles, int key_bits,
    int nchunks, const int32_t *cc, int32_t *counts, int32_t *offsets, int32_t *row_token,
    int32_t *row_pair, int32_t *inv_perm, int32_t *tiles, int32_t *n_tiles) {
  __shared__ int sh[17];
  __shared__ int s_off[kFusedExperts + 8];
  __shared__ int wcnt[4][kFusedExperts];
  const int c = blockIdx.x, e = threadIdx.x, w = e >> 6, lane = lane_id();
  const int Ti = int(T), P = int(T) * k;
  // this chunk's pairs: wave w takes positions [128 w, 128 w + 128) of it
  // (loaded first, so their round trip overlaps the chunk counts' and the scan)
  int ex[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int p = c * kWgChunk + 128 * w + 64 * j + lane;
    const int sl = p / Ti, t = p - sl * Ti;
    ex[j] = p < P ? idx[int64_t(t) * k + sl] : -1;
  }
  // this expert's rows over all chunks, and over the chunks before this one
  int tot = 0, pre = 0;
  if (e < E) {
    // eight chunk counts in flight per trip (up to 128 chunks: one serial
    // load round trip per chunk would dominate the launch)
    int ch = 0;
    for (; ch + 8 <= nchunks; ch += 8) {
      int v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = cc[int64_t(ch + u) * E + e];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        tot += v[u];
        pre += ch + u < c ? v[u] : 0;
      }
    }
    for (; ch < nchunks; ++ch) {
      const int v = cc[int64_t(ch) * E + e];
      tot += v;
      pre += ch < c ? v : 0;
    }
  } else if (e < E + n_shared) {
    tot = Ti;
  }
  // the expert's first row (schedule() also writes the outputs; one block does)
  int off;
  if (c == 0) {
    off = schedule(tot, E, n_shared, T, bm, max_tiles, counts, offsets, row_token, tiles, n_tiles, sh, s_off);
  } else {
    int total;
    off = block_exclusive_scan(e < E + n_shared ? tot : 0, sh, &total);
  }
  for (int i = threadIdx.x; i < 4 * kFusedExperts; i += 256) (&wcnt[0][0])[i] = 0;
#pragma unroll
  for (int j = 0; j < 2; ++j) ex[j] = (ex[j] >= 0 && ex[j] < E) ? ex[j] : -1;  // -1: past the end or bad id
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j)
    if (ex[j] >= 0) atomicAdd(&wcnt[w][ex[j]], 1);
  __syncthreads();
  if (e < E) {
    int run = off + pre;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const int v = wcnt[ww][e];
      wcnt[ww][e] = run;
      run += v;
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const bool valid = ex[j] >= 0;
    const int exj = valid ? ex[j] : 0;
    int rank, group;
    bool leader;
    peer_rank(valid, exj, key_bits, &rank, &group, &leader);
    const int start = valid ? wcnt[w][exj] : 0;
    __builtin_amdgcn_wave_barrier();
    if (leader) wcnt[w][exj] = start + group;
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      const int p = c * kWgChunk + 128 * w + 64 * j + lane;
      const int sl = p / Ti, t = p - sl * Ti;
      const int pos = start + rank;
      const int pair = t * k + sl;
      row_pair[pos] = pair;
      row_token[pos] = t;
      inv_perm[pair] = pos;
    }
  }
}

template <int PPL>
__global__ __launch_bounds__(1024) void permute_fused_kernel(
    const int32_t *idx, int64_t T, int k, int E, int n_shared, int bm, int max_tiles, int key_bits,
    int32_t *counts, int32_t *offsets, int32_t *row_token, int32_t *row_pair, int32_t *inv_perm,
    int32_t *tiles, int32_t *n_tiles) {
  permute_block<PPL>(idx, T, k, E, n_shared, bm, max_tiles, key_bits, counts, offsets, row_token, row_pair,
                inv_perm, tiles, n_tiles);
}

// Top-k of every token (wave t % 16 takes token t), then the permutation of
// the selection by the same work-group: one launch instead of two for small
// batches.  The selected indices are read back after the barrier, which
// makes the waves' global stores visible to the whole work-group.
template <int EREG, int PPL>
__global__ __launch_bounds__(1024) void topk_permute_kernel(
    const void *logits, int dtype, int64_t T, int E, int k, int norm, int32_t *idx, float *w,
    int n_shared, int bm, int max_tiles, int key_bits, int32_t *counts, int32_t *offsets,
    int32_t *row_token, int32_t *row_pair, int32_t *inv_perm, int32_t *tiles, int32_t *n_tiles) {
  const int lane = lane_id();
  // token t + 16's logits are loaded while token t is ranked
  auto load_row = [&](int64_t t, float (&v)[EREG]) {
#pragma unroll
    for (int r = 0; r < EREG; ++r) {
      const int e = 64 * r + lane;
      v[r] = t < T && e < E ? load_as_f32(logits, dtype, t * E + e) : -INFINITY;
    }
  };
  float cur[EREG], nxt[EREG];
  load_row(threadIdx.x >> 6, cur);
  for (int64_t t = threadIdx.x >> 6; t < T; t += kFusedWaves) {
    load_row(t + kFusedWaves, nxt);
    select_topk<EREG>(cur, E, k, norm, t, idx, w);
#pragma unroll
    for (int r = 0; r < EREG; ++r) cur[r] = nxt[r];
  }
  __syncthreads();
  permute_block<PPL>(idx, T, k, E, n_shared, bm, max_tiles, key_bits, counts, offsets, row_token, row_pair,
                     inv_perm, tiles, n_tiles);
}

// Pairs per lane of the single-work-group permutation for P <= kFusedPairs.
static int fused_ppl(int64_t P) { return P <= kFusedWaves * 64 ? 1 : 4; }

bool topk_permute_fits(int64_t T, int k, int E, int n_shared) {
  return T * k <= kFusedPairs && E + n_shared <= kFusedExperts && k <= kMaxTopK;
}

static int key_bits_for(int E) {
  int b = 1;
  while ((1 << b) < E) ++b;
  return b;
}

int launch_topk_permute(const void *logits, int dtype, int64_t T, int E, int k, int norm, int32_t *idx,
                        float *w, int n_shared, int bm, int32_t *counts, int32_t *offsets,
                        int32_t *row_token, int32_t *row_pair, int32_t *inv_perm, int32_t *tiles,
                        int32_t *n_tiles, hipStream_t s) {
  if (!topk_permute_fits(T, k, E, n_shared)) return fail(MOEQ_ERR_UNSUPPORTED, "topk_permute: batch too large");
  const int max_tiles = moeq_max_tiles(T, k, E, n_shared, bm);
  const int kb = key_bits_for(E);
#define MOEQ_TP(R, Q)                                                                                       \
  topk_permute_kernel<R, Q><<<1, 1024, 0, s>>>(logits, dtype, T, E, k, norm, idx, w, n_shared, bm,          \
                                               max_tiles, kb, counts, offsets, row_token, row_pair, inv_perm, \
                                               tiles, n_tiles)
  const bool one = fused_ppl(T * k) == 1;
  switch (ereg_for(E)) {
    case 1: if (one) MOEQ_TP(1, 1); else MOEQ_TP(1, 4); break;
    case 2: if (one) MOEQ_TP(2, 1); else MOEQ_TP(2, 4); break;
    default: if (one) MOEQ_TP(4, 1); else MOEQ_TP(4, 4); break;  // E <= kFusedExperts = 256
  }
#undef MOEQ_TP
  return check_launch("route/topk_permute");
}

}  // namespace moeq

using namespace moeq;

extern "C" int moeq_tile_rows(int bm) { return tile_rows(bm); }

extern "C" int moeq_max_tiles(int64_t T, int top_k, int E, int n_shared, int bm) {
  const int cap = tile_rows(bm);
  if (T <= 0 || top_k <= 0 || E <= 0 || n_shared < 0 || cap <= 0) return 0;
  // sum over experts of ceil(m_e / cap) <= pairs / cap + (experts with rows)
  int64_t pairs = T * top_k;
  int64_t bound = pairs / cap + std::min<int64_t>(E, pairs) + int64_t(n_shared) * cdiv(T, cap);
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
  if (tile_rows(bm) == 0) return fail(MOEQ_ERR_INVALID, "permute: bm=%d not in {16, 32, 64, 128, 256}", bm);
  if (T * top_k > INT32_MAX / 2 || T * (top_k + n_shared) > INT32_MAX / 2)
    return fail(MOEQ_ERR_UNSUPPORTED, "permute: T=%lld too large", (long long)T);
  size_t need = moeq_permute_workspace_size(T, top_k, E, n_shared);
  if (!ws || ws_bytes < need)
    return fail(MOEQ_ERR_WORKSPACE, "permute: workspace %zu < %zu bytes", ws_bytes, need);
  const int key_bits = key_bits_for(E);
  hipStream_t s = as_stream(stream);
  const int max_tiles = moeq_max_tiles(T, top_k, E, n_shared, bm);
  if (T * top_k > kOneGroupPairs && T * top_k <= kChunkedPairs && E + n_shared <= kFusedExperts) {
    int32_t *cc = static_cast<int32_t *>(ws);
    const int nchunks = int(cdiv(T * top_k, kWgChunk));
    chunk_hist_kernel<<<nchunks, 256, 0, s>>>(idx, T, top_k, E, cc);
    int rc = check_launch("permute/chunk_hist");
    if (rc) return rc;
    chunk_scatter_kernel<<<nchunks, 256, 0, s>>>(idx, T, top_k, E, n_shared, bm, max_tiles, key_bits, nchunks, cc,
                                                 counts, offsets, row_token, row_pair, inv_perm, tiles, n_tiles);
    return check_launch("permute/chunk_scatter");
  }
  if (T * top_k <= kOneGroupPairs && E + n_shared <= kFusedExperts) {
    permute_fused_kernel<1><<<1, 1024, 0, s>>>(idx, T, top_k, E, n_shared, bm, max_tiles, key_bits, counts,
                                               offsets, row_token, row_pair, inv_perm, tiles, n_tiles);
    return check_launch("permute/fused");
  }
  int32_t *cc = static_cast<int32_t *>(ws);
  int64_t nchunks = cdiv(T * top_k, kChunk);
  dim3 grid(unsigned(cdiv(nchunks, 4))), block(256);
  size_t lds = size_t(4) * E * sizeof(int32_t);
  hist_kernel<<<grid, block, lds, s>>>(idx, T, top_k, E, nchunks, cc);
  int rc = check_launch("permute/hist");
  if (rc) return rc;
  scan_kernel<<<1, 1024, 0, s>>>(cc, nchunks, T, top_k, E, n_shared, bm, max_tiles, counts,
                                 offsets, row_token, tiles, n_tiles);
  rc = check_launch("permute/scan");
  if (rc) return rc;
  scatter_kernel<<<grid, block, lds, s>>>(idx, T, top_k, E, key_bits, nchunks, cc, row_token,
                                          row_pair, inv_perm);
  return check_launch("permute/scatter");
}
