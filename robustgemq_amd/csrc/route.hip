// Router: logits in a pinned fp32 order, softmax, top-k, renormalisation.
//
// Logit (t, e) = butterfly over 64 lanes of per-lane fused multiply-add
// chains; lane l covers k = 512 i + 8 l + j (i ascending, then j = 0..7).
// The xor butterfly (o = 32 .. 1, v <- v + v[l ^ o]) gives every lane the
// same value because fp32 addition is commutative.  oracle/router_exact.c
// replays exactly this order, so routing is bit-reproducible on the CPU.
#include <algorithm>
#include <type_traits>

#include "routing.h"

namespace moeq {

template <int TT, int EE, int MAXCH>
__global__ __launch_bounds__(256) void logits_kernel(RouteArgs a, int n_et) {
  const int64_t wave = int64_t(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  logit_tile<TT, EE, MAXCH>(a, (wave / n_et) * TT, int(wave % n_et) * EE);
}

template <int EREG>
__global__ __launch_bounds__(256) void topk_from_logits_kernel(
    const void *logits, int dtype, int64_t T, int E, int k, int norm,
    int32_t *idx, float *w) {
  const int lane = lane_id();
  const int64_t t = int64_t(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (t >= T) return;
  float vals[EREG];
#pragma unroll
  for (int r = 0; r < EREG; ++r) {
    int e = 64 * r + lane;
    vals[r] = e < E ? load_as_f32(logits, dtype, t * E + e) : -INFINITY;
  }
  select_topk<EREG>(vals, E, k, norm, t, idx, w);
}

// ---------------------------------------------------------------- prefill
// Logits and top-k of kTT tokens per work-group (8, or 4 for batches of at
// most 1024 tokens).  Wave w takes (64 / kTT)-expert blocks w, w + NWV, ...;
// each lane runs the 64 chains of a kTT x (64 / kTT) (token, expert) block
// over its k set, so every loaded x value feeds 64 / kTT and every w value
// kTT fused multiply-adds.  The 64 chains are then summed over the lanes by
// halving exchanges that pair the same lanes in the same order as the xor
// butterfly (o = 32 .. 1), leaving chain l in lane l with the identical
// value, whatever (token, expert) it holds.  The rounded logits of the kTT
// tokens meet in LDS, and one wave per token ranks them.


// One operand row: the 8 values of one k step, as loaded (fp16 / bf16: four
// packed words; fp32: eight words).
template <int DT>
struct Raw8 {
  static constexpr int W = DT == MOEQ_F32 ? 8 : 4;
  uint32_t u[W];
  // 8 values at byte offset voff (per lane) + soff (uniform) of the buffer
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, int(voff), int(soff), 0);
    u[0] = a[0]; u[1] = a[1]; u[2] = a[2]; u[3] = a[3];
    if constexpr (W == 8) {
      const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(r, int(voff + 16), int(soff), 0);
      u[4] = b[0]; u[5] = b[1]; u[6] = b[2]; u[7] = b[3];
    }
  }
  // value j widened to fp32 (exact)
  __device__ __forceinline__ float value(int j) const {
    if constexpr (DT == MOEQ_F32) return __uint_as_float(u[j]);
    else if constexpr (DT == MOEQ_BF16) return __uint_as_float((j & 1) ? (u[j >> 1] & 0xffff0000u) : (u[j >> 1] << 16));
    else return f16_bits_to_f32(uint16_t(u[j >> 1] >> (16 * (j & 1))));
  }
};

// fmaf(x_j, w_j, c) with one rounding.  fp16 operands go to v_fma_mix_f32
// straight from the packed word (the widening is exact); other operands are
// widened first (xf / wf: value j of the row, precomputed by the caller).
template <int XDT, int WDT>
__device__ __forceinline__ float fma_j(const Raw8<XDT> &x, float xf, const Raw8<WDT> &w, float wf, int j, float c) {
  float r;
  if constexpr (XDT == MOEQ_F16 && WDT == MOEQ_F16) {
    if (j & 1)
      asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,1,0] op_sel_hi:[1,1,0]" : "=v"(r) : "v"(x.u[j >> 1]), "v"(w.u[j >> 1]), "v"(c));
    else
      asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,1,0]" : "=v"(r) : "v"(x.u[j >> 1]), "v"(w.u[j >> 1]), "v"(c));
  } else if constexpr (XDT == MOEQ_F16 && WDT == MOEQ_F32) {
    if (j & 1)
      asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(x.u[j >> 1]), "v"(w.u[j]), "v"(c));
    else
      asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(x.u[j >> 1]), "v"(w.u[j]), "v"(c));
  } else {
    r = __builtin_fmaf(xf, wf, c);
  }
  return r;
}

// Sum of chain c[j] over the 64 lanes, for all 64 j at once; lane l returns
// the sum of chain l.  Level o keeps, in each lane, the half of the chains
// whose bit matches the lane's bit o and adds the partner's (lane ^ o) copy:
// the pairs are those of the butterfly v <- v + v[lane ^ o] (fp32 addition
// commutes), so every sum is identical to the butterfly's.  Levels 32 and 16
// are one v_permlane32/16_swap per pair of chains: after swapping c[j]'s
// upper half (odd rows) with c[j + o]'s lower half (even rows), the two
// registers hold, lane by lane, the kept value and its partner.
__device__ __forceinline__ float halving_sum(float (&c)[64]) {
  const int lane = lane_id();
  float a[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(c[j]), __float_as_uint(c[j + 32]), false, false);
    a[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[j]), __float_as_uint(a[j + 16]), false, false);
    a[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  // Levels 8 .. 1: the lane picks with an explicit v_cndmask on its own two
  // registers (a plain `up ? a[j] : a[j + o]` is folded by the compiler into
  // a lane-dependent index into a[], lowered as a 32-way select chain).
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) {
    const uint64_t up = __builtin_amdgcn_ballot_w64((lane & o) != 0);
#pragma unroll
    for (int j = 0; j < o; ++j) {
      float send, keep;
      asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(send) : "v"(a[j + o]), "v"(a[j]), "s"(up));
      asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(keep) : "v"(a[j]), "v"(a[j + o]), "s"(up));
      a[j] = keep + __shfl_xor(send, o);
    }
  }
  return a[0];
}

// Copies kTT activation rows (16-bit, from token t0 on) to LDS as units
// (tt, i, l) = the 8 values lane l multiplies at k step i: one 1 KB unit row
// per wave instruction (buffer_load ... lds), then waits for every wave's
// copies.  Rows past T and k steps past H copy a valid row, never read.
// (A device function: with this builtin or the inline wait directly in the
// kernel template's body, hipcc's host pass emitted no launch stub for it.)
template <int MAXCH, int kTT, int NWV>
__device__ __forceinline__ void stage_rows(uint4 *xs, __amdgpu_buffer_rsrc_t xrs, const RouteArgs &a, int64_t t0,
                                           int wave, int lane) {
  for (int q = wave; q < kTT * MAXCH; q += NWV) {
    const int tt = q / MAXCH, i = q % MAXCH;
    const uint32_t kc = uint32_t(min(512 * i + 8 * lane, a.H - 8));
    const uint32_t row = uint32_t(min(int64_t(tt), a.T - 1 - t0)) * uint32_t(a.H) * 2u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void *)&xs[q * 64], 16, kc * 2u,
                                             row, 0, 0);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

template <int XDT, int WDT, int NWV, int MAXCH, int kTT>
__global__ __launch_bounds__(NWV * 64) void logits_topk_kernel(RouteArgs a) {
  // kTT tokens x kEE experts per wave pass (64 chains per lane); the chain
  // order and the lane reduction do not depend on the split
  constexpr int kEE = 64 / kTT;
  __shared__ float lg[kTT][512];
  // 16-bit activations: the block's kTT rows are copied to LDS once, as
  // units (tt, i, l) = the 8 values lane l multiplies at k step i, so the k
  // loop waits only for gate rows (from L2), fetched one step ahead
  constexpr bool XL = XDT != MOEQ_F32;
  __shared__ uint4 xs[XL ? kTT * MAXCH * 64 : 1];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t0 = int64_t(blockIdx.x) * kTT;
  const int n_eb = (a.E + kEE - 1) / kEE;
  // Rows are read through buffer resources based at this block's first token
  // / expert: one 32-bit lane offset (the k position) serves all rows, whose
  // row offsets are uniform.  Rows past T or E, and k steps past H, load a
  // valid row (token T - 1, expert E - 1, k = H - 8) that is never used, so
  // the loads are unconditional.
  constexpr uint32_t XES = XDT == MOEQ_F32 ? 4 : 2, WES = WDT == MOEQ_F32 ? 4 : 2;
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char *>(static_cast<const char *>(a.x) + t0 * a.H * XES), (short)0, 0x7fffffff, 0x00020000);
  auto kcol = [&](int i) { return uint32_t(min(512 * i + 8 * lane, a.H - 8)); };
  auto xrow = [&](int tt) { return uint32_t(min(int64_t(tt), a.T - 1 - t0)) * uint32_t(a.H) * XES; };
  if constexpr (XL) stage_rows<MAXCH, kTT, NWV>(xs, xrs, a, t0, wave, lane);
  const uint4 *const xsp = xs;
  // gate rows of fp16 / bf16 gates two k steps in flight; fp32 gate rows
  // (twice the registers) and fp32 activations one
  constexpr int NBUF = (XL && WDT != MOEQ_F32) ? 2 : 1;
  for (int eb = wave; eb < n_eb; eb += NWV) {
    const int e0 = eb * kEE;
    float ch[kTT * kEE];
#pragma unroll
    for (int i = 0; i < kTT * kEE; ++i) ch[i] = 0.f;
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char *>(static_cast<const char *>(a.wg) + int64_t(e0) * a.H * WES), (short)0, 0x7fffffff,
        0x00020000);
    auto fetch_w = [&](int i, Raw8<WDT> (&wb)[kEE]) {
      const uint32_t kc = kcol(i);
#pragma unroll
      for (int ee = 0; ee < kEE; ++ee)
        wb[ee].load(wrs, kc * WES, uint32_t(min(ee, a.E - 1 - e0)) * uint32_t(a.H) * WES);
    };
    auto fetch_x = [&](int i, Raw8<XDT> (&xb)[kTT]) {
#pragma unroll
      for (int tt = 0; tt < kTT; ++tt) {
        if constexpr (XL) {
          const uint4 v = xsp[(tt * MAXCH + i) * 64 + lane];
          xb[tt].u[0] = v.x; xb[tt].u[1] = v.y; xb[tt].u[2] = v.z; xb[tt].u[3] = v.w;
        } else {
          xb[tt].load(xrs, kcol(i) * XES, xrow(tt));
        }
      }
    };
    auto step = [&](int i, const Raw8<XDT> (&xb)[kTT], const Raw8<WDT> (&wb)[kEE]) {
      const int k0 = 512 * i + 8 * lane;
      if (k0 >= a.H) return;
      if (a.x16 && eb == 0) {  // the activations the expert GEMMs read, converted once
#pragma unroll
        for (int tt = 0; tt < kTT; ++tt) {
          if (t0 + tt >= a.T) continue;
          uint32_t h[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            h[j] = uint32_t(f32_to_f16_bits(xb[tt].value(2 * j))) |
                   (uint32_t(f32_to_f16_bits(xb[tt].value(2 * j + 1))) << 16);
          *reinterpret_cast<uint4 *>(a.x16 + (t0 + tt) * a.H + k0) = (uint4){h[0], h[1], h[2], h[3]};
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float xf[kTT], wf[kEE];
#pragma unroll
        for (int tt = 0; tt < kTT; ++tt) xf[tt] = XDT == MOEQ_F16 ? 0.f : xb[tt].value(j);
#pragma unroll
        for (int ee = 0; ee < kEE; ++ee) wf[ee] = XDT == MOEQ_F16 ? 0.f : wb[ee].value(j);
        // rows past T / E hold data of another row: their chains are never stored
#pragma unroll
        for (int tt = 0; tt < kTT; ++tt)
#pragma unroll
          for (int ee = 0; ee < kEE; ++ee)
            ch[tt * kEE + ee] = fma_j<XDT, WDT>(xb[tt], xf[tt], wb[ee], wf[ee], j, ch[tt * kEE + ee]);
      }
    };
    if constexpr (NBUF == 2) {
      // k steps i (gate rows A) and i + 1 (rows B) per trip: the next step's
      // rows are in flight while one step is multiplied
      Raw8<WDT> wa[kEE], wb[kEE];
      fetch_w(0, wa);
#pragma unroll 1
      for (int i = 0; i < MAXCH; i += 2) {
        fetch_w(i + 1, wb);
        __builtin_amdgcn_sched_barrier(0);
        {
          Raw8<XDT> xa[kTT];
          fetch_x(i, xa);
          step(i, xa, wa);
        }
        __builtin_amdgcn_sched_barrier(0);
        fetch_w(i + 2, wa);
        __builtin_amdgcn_sched_barrier(0);
        if (i + 1 < MAXCH) {
          Raw8<XDT> xa[kTT];
          fetch_x(i + 1, xa);
          step(i + 1, xa, wb);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      Raw8<XDT> xa[kTT];
      Raw8<WDT> wa[kEE];
#pragma unroll 1
      for (int i = 0; i < MAXCH; ++i) {
        fetch_w(i, wa);
        fetch_x(i, xa);
        step(i, xa, wa);
      }
    }
    float v = halving_sum(ch);
    const int tt = lane / kEE, e = e0 + lane % kEE;
    const int64_t t = t0 + tt;
    if (e < a.E) {
      if (a.bias) v = v + a.bias[e];
      v = round_logit(v, a.logits_dtype);
      lg[tt][e] = v;
      if (a.logits && t < a.T) store_logit(a.logits, a.store_dtype, t * a.E + e, v);
    }
  }
  __syncthreads();
  for (int tt = wave; tt < kTT && t0 + tt < a.T; tt += NWV) {
    const int ereg = ereg_for(a.E);
#define MOEQ_SEL(R)                                                       \
  {                                                                       \
    float vals[R];                                                        \
    _Pragma("unroll") for (int r = 0; r < R; ++r) {                       \
      const int e = 64 * r + lane;                                        \
      vals[r] = e < a.E ? lg[tt][e] : -INFINITY;                          \
    }                                                                     \
    select_topk<R>(vals, a.E, a.k, a.norm, t0 + tt, a.idx, a.w);          \
  }
    if (ereg == 1) MOEQ_SEL(1) else if (ereg == 2) MOEQ_SEL(2) else if (ereg == 4) MOEQ_SEL(4) else MOEQ_SEL(8)
#undef MOEQ_SEL
  }
}

template <int XDT, int WDT, int NWV, int TT>
static void launch_logits_topk_nw(const RouteArgs &a, int maxch, hipStream_t s) {
  dim3 grid(unsigned(cdiv(a.T, TT))), block(NWV * 64);
  switch (maxch) {
    case 1: logits_topk_kernel<XDT, WDT, NWV, 1, TT><<<grid, block, 0, s>>>(a); break;
    case 2: logits_topk_kernel<XDT, WDT, NWV, 2, TT><<<grid, block, 0, s>>>(a); break;
    case 4: logits_topk_kernel<XDT, WDT, NWV, 4, TT><<<grid, block, 0, s>>>(a); break;
    default: logits_topk_kernel<XDT, WDT, NWV, 8, TT><<<grid, block, 0, s>>>(a); break;
  }
}

// 8 tokens x 8 experts per wave pass; up to 1024 tokens (at most 128
// work-groups of 8, half the CUs or fewer) 4 tokens x 16 experts, so twice
// as many work-groups share the launch.
template <int XDT, int WDT>
static void launch_logits_topk_dt(const RouteArgs &a, int maxch, hipStream_t s) {
  if (a.T <= 1024 && a.E > 8) {
    if (a.E <= 16) launch_logits_topk_nw<XDT, WDT, 1, 4>(a, maxch, s);
    else if (a.E <= 32) launch_logits_topk_nw<XDT, WDT, 2, 4>(a, maxch, s);
    else if (a.E <= 64) launch_logits_topk_nw<XDT, WDT, 4, 4>(a, maxch, s);
    else launch_logits_topk_nw<XDT, WDT, 8, 4>(a, maxch, s);
    return;
  }
  if (a.E <= 8) launch_logits_topk_nw<XDT, WDT, 1, 8>(a, maxch, s);
  else if (a.E <= 16) launch_logits_topk_nw<XDT, WDT, 2, 8>(a, maxch, s);
  else if (a.E <= 32) launch_logits_topk_nw<XDT, WDT, 4, 8>(a, maxch, s);
  // bf16 with more than 64 experts: four waves per work-group, so the two
  // work-groups on a CU run out of step (Qwen3-shaped T = 4096 routing
  // alone: 49.2 -> 46.1 us)
  else if (XDT == MOEQ_BF16 && a.E > 64) launch_logits_topk_nw<XDT, WDT, 4, 8>(a, maxch, s);
  else launch_logits_topk_nw<XDT, WDT, 8, 8>(a, maxch, s);
}

// ---------------------------------------------------------------- one token
// One token's top-k and grouping from its E rounded logits (one wave): ranks
// them (topk_ranks), writes idx / w and the permutation, which for one token
// is the selected experts in id order, one 1-row tile each, then the shared
// experts' rows (moeq_permute's output for T = 1).
__device__ __forceinline__ void one_token_grouping(const float *lg, const RouteArgs &a, const PermOut &po) {
  const int lane = lane_id();
  const int E = a.E, k = a.k;
  const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  auto finish = [&](auto regs) {
    constexpr int R = decltype(regs)::value;
    float vals[R];
    int rank[R];
    float wsel[R];
#pragma unroll
    for (int r = 0; r < R; ++r) vals[r] = 64 * r + lane < E ? lg[64 * r + lane] : -INFINITY;
    topk_ranks<R>(vals, E, k, a.norm, rank, wsel, a.prob_dtype);
    int before = 0;  // selected experts in earlier registers
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int e = 64 * r + lane;
      const bool sel = e < E && rank[r] < k;
      const uint64_t m = __builtin_amdgcn_ballot_w64(sel);
      const int pos = before + __popcll(m & lt);  // row = selected experts below e
      if (e < E) {
        po.counts[e] = sel ? 1 : 0;
        po.offsets[e] = pos;
      }
      if (sel) {
        a.idx[rank[r]] = e;
        a.w[rank[r]] = wsel[r];
        po.row_pair[pos] = rank[r];
        po.row_token[pos] = 0;
        po.inv_perm[rank[r]] = pos;
        *reinterpret_cast<int4 *>(po.tiles + 4 * pos) = (int4){e, pos, 1, 0};
      }
      before += __popcll(m);
    }
  };
  const int ereg = ereg_for(E);
  if (ereg == 1) finish(std::integral_constant<int, 1>{});
  else if (ereg == 2) finish(std::integral_constant<int, 2>{});
  else finish(std::integral_constant<int, 4>{});
  // shared experts: one row each after the k routed rows
  for (int v = lane; v < po.n_shared; v += 64) {
    po.counts[E + v] = 1;
    po.offsets[E + v] = k + v;
    po.row_token[k + v] = 0;
    *reinterpret_cast<int4 *>(po.tiles + 4 * (k + v)) = (int4){E + v, k + v, 1, 0};
  }
  if (lane == 0) {
    po.offsets[E + po.n_shared] = k + po.n_shared;
    *po.n_tiles = min(k + po.n_shared, po.max_tiles);
  }
}

// Eight waves; wave w computes the logits of experts w * EE .. w * EE + EE - 1,
// then (w + 8) * EE .., with every k step of the x row and of its EE gate
// rows loaded at once (one memory round trip per expert group).  Each logit
// is the same chain and butterfly as logit_tile's.  The rounded logits meet
// in LDS; wave 0 ranks them and writes idx / w and the permutation.
constexpr int kR1Waves = 8;

template <int XDT, int WDT, int EE, int MAXCH>
__global__ __launch_bounds__(kR1Waves * 64) void route1_kernel(RouteArgs a, PermOut po) {
  __shared__ float lg[256];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr uint32_t XES = XDT == MOEQ_F32 ? 4 : 2, WES = WDT == MOEQ_F32 ? 4 : 2;
  // k steps past H load the row's last 8 values and skip the multiply-adds
  uint32_t kc[MAXCH];
#pragma unroll
  for (int i = 0; i < MAXCH; ++i) kc[i] = uint32_t(min(512 * i + 8 * lane, a.H - 8));
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(a.x), (short)0, 0x7fffffff, 0x00020000);
  Raw8<XDT> xb[MAXCH];
#pragma unroll
  for (int i = 0; i < MAXCH; ++i) xb[i].load(xrs, kc[i] * XES, 0);
  for (int e0 = wave * EE; e0 < a.E; e0 += kR1Waves * EE) {
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char *>(static_cast<const char *>(a.wg) + int64_t(e0) * a.H * WES), (short)0, 0x7fffffff,
        0x00020000);
    Raw8<WDT> wb[MAXCH][EE];
#pragma unroll
    for (int i = 0; i < MAXCH; ++i)
#pragma unroll
      for (int ee = 0; ee < EE; ++ee)
        wb[i][ee].load(wrs, kc[i] * WES, uint32_t(min(ee, a.E - 1 - e0)) * uint32_t(a.H) * WES);
    if (a.x16 && e0 == 0) {  // the activations the expert GEMMs read, converted once
#pragma unroll
      for (int i = 0; i < MAXCH; ++i) {
        const int k0 = 512 * i + 8 * lane;
        if (k0 < a.H) {
          uint32_t h[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            h[j] = uint32_t(f32_to_f16_bits(xb[i].value(2 * j))) |
                   (uint32_t(f32_to_f16_bits(xb[i].value(2 * j + 1))) << 16);
          *reinterpret_cast<uint4 *>(a.x16 + k0) = (uint4){h[0], h[1], h[2], h[3]};
        }
      }
    }
    float ch[EE];
#pragma unroll
    for (int ee = 0; ee < EE; ++ee) ch[ee] = 0.f;
#pragma unroll
    for (int i = 0; i < MAXCH; ++i) {
      if (512 * i + 8 * lane < a.H) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float xv = xb[i].value(j);
#pragma unroll
          for (int ee = 0; ee < EE; ++ee) ch[ee] = __builtin_fmaf(xv, wb[i][ee].value(j), ch[ee]);
        }
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
#pragma unroll
      for (int ee = 0; ee < EE; ++ee) ch[ee] = ch[ee] + __shfl_xor(ch[ee], o);
#pragma unroll
    for (int ee = 0; ee < EE; ++ee) {
      const int e = e0 + ee;
      if (e < a.E) {
        float v = ch[ee];
        if (a.bias) v = v + a.bias[e];
        v = round_logit(v, a.logits_dtype);
        if (lane == 0) lg[e] = v;
        if (a.logits && lane == ee) store_logit(a.logits, a.store_dtype, e, v);
      }
    }
  }
  __syncthreads();
  if (wave != 0) return;
  one_token_grouping(lg, a, po);
}

// Expert group per wave: no larger than the experts need over 8 waves, and
// no larger than FIT, the largest group whose loaded rows stay in registers
// (16-bit gate rows: 8 at H <= 2048, 4 above; fp32 rows: 4 and 1).
template <int WDT, int MAXCH>
constexpr int route1_fit() {
  return WDT == MOEQ_F32 ? (MAXCH <= 4 ? 4 : 1) : (MAXCH <= 4 ? 8 : 4);
}

template <int XDT, int WDT, int MAXCH>
static void launch_route1_ch(const RouteArgs &a, const PermOut &po, hipStream_t s) {
  constexpr int FIT = route1_fit<WDT, MAXCH>();
  int ee = 1;
  while (ee < FIT && ee * kR1Waves < a.E) ee <<= 1;
  if (ee == 1) route1_kernel<XDT, WDT, 1, MAXCH><<<1, kR1Waves * 64, 0, s>>>(a, po);
  if constexpr (FIT >= 2) if (ee == 2) route1_kernel<XDT, WDT, 2, MAXCH><<<1, kR1Waves * 64, 0, s>>>(a, po);
  if constexpr (FIT >= 4) if (ee == 4) route1_kernel<XDT, WDT, 4, MAXCH><<<1, kR1Waves * 64, 0, s>>>(a, po);
  if constexpr (FIT >= 8) if (ee == 8) route1_kernel<XDT, WDT, 8, MAXCH><<<1, kR1Waves * 64, 0, s>>>(a, po);
}

template <int XDT, int WDT>
static void launch_route1_dt(const RouteArgs &a, const PermOut &po, hipStream_t s) {
  if (a.H <= 2048) launch_route1_ch<XDT, WDT, 4>(a, po, s);
  else launch_route1_ch<XDT, WDT, 8>(a, po, s);
}

bool launch_route1(const RouteArgs &a, const PermOut &po, hipStream_t s) {
  if (a.T != 1 || a.E > 256 || a.k > kMaxTopK || a.k > a.E || a.H % 8 || a.H > 4096) return false;
  const int x = a.x_dtype, w = a.wg_dtype;
  if (x == MOEQ_F16 && w == MOEQ_F16) launch_route1_dt<MOEQ_F16, MOEQ_F16>(a, po, s);
  else if (x == MOEQ_F16 && w == MOEQ_F32) launch_route1_dt<MOEQ_F16, MOEQ_F32>(a, po, s);
  else if (x == MOEQ_BF16 && w == MOEQ_BF16) launch_route1_dt<MOEQ_BF16, MOEQ_BF16>(a, po, s);
  else if (x == MOEQ_BF16 && w == MOEQ_F32) launch_route1_dt<MOEQ_BF16, MOEQ_F32>(a, po, s);
  else return false;
  return true;
}

// One token from logits already computed (logits_kernel, one logit per
// wave over the whole GPU): one wave reads the E rounded logits (stored in
// `dtype`, exact since they were rounded to it) and writes what route1_kernel
// writes.  For large gate matrices this beats route1_kernel, whose single
// work-group reads the whole matrix.
__global__ __launch_bounds__(64) void topk1_kernel(const void *logits, int dtype, RouteArgs a, PermOut po) {
  __shared__ float lg[256];
  for (int e = lane_id(); e < a.E; e += 64) lg[e] = load_as_f32(logits, dtype, e);
  __syncthreads();
  one_token_grouping(lg, a, po);
}

int launch_topk1(const void *logits, int dtype, const RouteArgs &a, const PermOut &po, hipStream_t s) {
  if (a.E > 256 || a.k > kMaxTopK) return fail(MOEQ_ERR_UNSUPPORTED, "topk1: E=%d k=%d", a.E, a.k);
  topk1_kernel<<<dim3(1), dim3(64), 0, s>>>(logits, dtype, a, po);
  return check_launch("route/topk1");
}

// Fused logits + top-k for batches above T * E = 16384; returns false (and
// launches nothing) for a dtype pair it does not cover.
bool launch_logits_topk(const RouteArgs &a, hipStream_t s) {
  if (a.T * a.E <= 16384 || a.E > 512 || a.k > kMaxTopK || a.H % 8 || a.H > 4096) return false;
  const int maxch = a.H <= 512 ? 1 : a.H <= 1024 ? 2 : a.H <= 2048 ? 4 : 8;
  const int x = a.x_dtype, w = a.wg_dtype;
  if (x == MOEQ_F16 && w == MOEQ_F16) launch_logits_topk_dt<MOEQ_F16, MOEQ_F16>(a, maxch, s);
  else if (x == MOEQ_F16 && w == MOEQ_F32) launch_logits_topk_dt<MOEQ_F16, MOEQ_F32>(a, maxch, s);
  else if (x == MOEQ_BF16 && w == MOEQ_BF16) launch_logits_topk_dt<MOEQ_BF16, MOEQ_BF16>(a, maxch, s);
  else if (x == MOEQ_BF16 && w == MOEQ_F32) launch_logits_topk_dt<MOEQ_BF16, MOEQ_F32>(a, maxch, s);
  else if (x == MOEQ_F32 && w == MOEQ_F32) launch_logits_topk_dt<MOEQ_F32, MOEQ_F32>(a, maxch, s);
  else return false;
  return true;
}

template <int TT, int EE>
static void launch_logits(const RouteArgs &a, int maxch, hipStream_t s) {
  const int n_et = int(cdiv(a.E, EE));
  const int64_t waves = cdiv(a.T, TT) * n_et;
  dim3 grid(unsigned(cdiv(waves, 4))), block(256);
  switch (maxch) {
    case 1: logits_kernel<TT, EE, 1><<<grid, block, 0, s>>>(a, n_et); break;
    case 2: logits_kernel<TT, EE, 2><<<grid, block, 0, s>>>(a, n_et); break;
    case 4: logits_kernel<TT, EE, 4><<<grid, block, 0, s>>>(a, n_et); break;
    default: logits_kernel<TT, EE, 8><<<grid, block, 0, s>>>(a, n_et); break;
  }
}

static int launch_topk(const void *logits, int dtype, int64_t T, int E, int k, int norm, int32_t *idx,
                       float *w, hipStream_t s) {
  dim3 grid(unsigned(cdiv(T, 4))), block(256);
  switch (ereg_for(E)) {
    case 1: topk_from_logits_kernel<1><<<grid, block, 0, s>>>(logits, dtype, T, E, k, norm, idx, w); break;
    case 2: topk_from_logits_kernel<2><<<grid, block, 0, s>>>(logits, dtype, T, E, k, norm, idx, w); break;
    case 4: topk_from_logits_kernel<4><<<grid, block, 0, s>>>(logits, dtype, T, E, k, norm, idx, w); break;
    default: topk_from_logits_kernel<8><<<grid, block, 0, s>>>(logits, dtype, T, E, k, norm, idx, w); break;
  }
  return check_launch("route/topk");
}


// Small batches take one logit per wave (up to 16384 waves) so enough waves
// read the router weights at once; larger ones share loads over 4 x 4 tiles.
// The summation order of a logit is the same for every tiling.
int launch_route_logits(const RouteArgs &a, hipStream_t s) {
  const int maxch = a.H <= 512 ? 1 : a.H <= 1024 ? 2 : a.H <= 2048 ? 4 : 8;
  if (a.T * a.E <= 16384)
    launch_logits<1, 1>(a, maxch, s);
  else
    launch_logits<4, 4>(a, maxch, s);
  return check_launch("route/logits");
}

static bool valid_dtype(int d) { return d == MOEQ_F16 || d == MOEQ_BF16 || d == MOEQ_F32; }

}  // namespace moeq

using namespace moeq;

extern "C" size_t moeq_route_workspace_size(int64_t T, int E) {
  if (T <= 0 || E <= 0) return 0;
  return align256(size_t(T) * size_t(E) * sizeof(float));
}

extern "C" int moeq_route(const void *x, int x_dtype, int64_t T, int H,
                          const void *gate_w, int gate_dtype, const float *logit_bias,
                          int E, int top_k, int norm_topk, void *logits_out,
                          int32_t *idx_out, float *w_out, void *ws, size_t ws_bytes,
                          void *stream) {
  if (!x || !gate_w || !idx_out || !w_out) return fail(MOEQ_ERR_INVALID, "route: null pointer");
  if (!valid_dtype(x_dtype) || !valid_dtype(gate_dtype))
    return fail(MOEQ_ERR_INVALID, "route: dtype x=%d gate=%d", x_dtype, gate_dtype);
  if (T <= 0) return fail(MOEQ_ERR_INVALID, "route: T=%lld", (long long)T);
  if (H <= 0 || H % 8) return fail(MOEQ_ERR_INVALID, "route: hidden=%d must be a positive multiple of 8", H);
  if (H > 4096) return fail(MOEQ_ERR_UNSUPPORTED, "route: hidden=%d > 4096", H);
  if (E <= 0 || E > 512) return fail(MOEQ_ERR_UNSUPPORTED, "route: n_experts=%d not in 1..512", E);
  if (top_k <= 0 || top_k > E || top_k > kMaxTopK)
    return fail(MOEQ_ERR_INVALID, "route: top_k=%d must be in 1..min(n_experts=%d, %d)", top_k, E, kMaxTopK);
  const int ldt = gate_dtype == MOEQ_F32 ? MOEQ_F32 : x_dtype;
  hipStream_t s = as_stream(stream);
  {
    // batches above 16384 logits: one fused launch, logits stored only if asked
    RouteArgs f{x, x_dtype, T, H, gate_w, gate_dtype, logit_bias, E, top_k, norm_topk ? 1 : 0,
                logits_out, ldt, ldt, idx_out, w_out};
    if (launch_logits_topk(f, s)) return check_launch("route/logits_topk");
  }
  void *lg = logits_out;
  int lg_dt = ldt;
  if (!lg) {
    if (!ws || ws_bytes < moeq_route_workspace_size(T, E))
      return fail(MOEQ_ERR_WORKSPACE, "route: logits_out is NULL and workspace %zu < %zu bytes", ws_bytes,
                  moeq_route_workspace_size(T, E));
    lg = ws;  // rounded logits kept as fp32 (exact)
    lg_dt = MOEQ_F32;
  }
  RouteArgs a{x, x_dtype, T, H, gate_w, gate_dtype, logit_bias, E, top_k, norm_topk ? 1 : 0,
              lg, ldt, lg_dt, idx_out, w_out};
  int rc = launch_route_logits(a, s);
  if (rc) return rc;
  // the selection reads the rounded logits (stored as ldt, or exactly as fp32)
  return launch_topk(lg, lg_dt, T, E, top_k, norm_topk ? 1 : 0, idx_out, w_out, s);
}

extern "C" int moeq_route_from_logits(const void *logits, int dtype, int64_t T,
                                      int E, int top_k, int norm_topk,
                                      int32_t *idx_out, float *w_out, void *stream) {
  if (!logits || !idx_out || !w_out) return fail(MOEQ_ERR_INVALID, "route_from_logits: null pointer");
  if (!valid_dtype(dtype)) return fail(MOEQ_ERR_INVALID, "route_from_logits: dtype=%d", dtype);
  if (T <= 0) return fail(MOEQ_ERR_INVALID, "route_from_logits: T=%lld", (long long)T);
  if (E <= 0 || E > 512) return fail(MOEQ_ERR_UNSUPPORTED, "route_from_logits: n_experts=%d not in 1..512", E);
  if (top_k <= 0 || top_k > E || top_k > kMaxTopK)
    return fail(MOEQ_ERR_INVALID, "route_from_logits: top_k=%d must be in 1..min(n_experts=%d, %d)", top_k, E, kMaxTopK);
  return launch_topk(logits, dtype, T, E, top_k, norm_topk ? 1 : 0, idx_out, w_out, as_stream(stream));
}
