/*
 * moeq.h -- C ABI of libmoeq.so, the MI355X (gfx950) real-quant MoE expert path.
 *
 * Every entry point:
 *   - takes plain device pointers, sizes and a hipStream_t (passed as void*),
 *   - returns MOEQ_OK (0) on success or a negative MOEQ_ERR_* code; nothing is
 *     launched when an argument check fails, and moeq_last_error() then names it,
 *   - never allocates device memory and never synchronizes the host: scratch
 *     memory is a caller-provided workspace whose size the *_workspace_size()
 *     query returns, so the calls can be captured into a HIP graph,
 *   - is reentrant across streams (no hidden global state besides the
 *     thread-local error string), except moeq_moe_forward_static, whose
 *     static per-GPU scratch array makes overlapping calls on one GPU race.
 *
 * Citations are path:line into lcj1111/RobustGEMQ and name the reference
 * interface each entry point replaces.
 */
#ifndef MOEQ_H_
#define MOEQ_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define MOEQ_OK 0
#define MOEQ_ERR_INVALID (-1)     /* bad argument (shape, pointer, enum)          */
#define MOEQ_ERR_UNSUPPORTED (-2) /* valid but not implemented for this shape     */
#define MOEQ_ERR_WORKSPACE (-3)   /* workspace missing or smaller than required   */
#define MOEQ_ERR_HIP (-4)         /* the HIP runtime reported a launch error      */

/* element types */
#define MOEQ_F16 0
#define MOEQ_BF16 1
#define MOEQ_F32 2

/* dequantization conventions (gemq/triton_kernels/utils.py:192-212 vs
 * gemq/quantizers/rtn.py:57-61) */
#define MOEQ_DQ_HQQ 0     /* w = fp16(fp16(q - z) * s)  (checkpoint / fake-quant weights) */
#define MOEQ_DQ_AFFINE 1  /* w = fp16(q * s + z')      (GemLite-packed zeros z' = -z*s)  */
#define MOEQ_DQ_HQQ_INT 2 /* as MOEQ_DQ_HQQ, one op less; every zero an integer 0..1023 */

/* Bits per code supported by the kernels: 1, 2, 3, 4. */

/* Quantized projection of all experts of one MoE layer, in the build layout
 * written by moeq_repack (codes) and moeq_prep_scales (scale/zero pairs).
 * Per expert e (bits b = nbits[e]) the code block holds K*N*b/32 words
 * starting at words + word_off[e]; the scale/zero block holds
 * (K/group_size)*N dwords starting at sz + sz_off[e].  Both are panel-major:
 * panel p = n / 16 holds its 16 columns' data over all of K, so a wave
 * streaming a panel reads one contiguous run.  Device arrays. */
typedef struct moeq_proj {
  const uint32_t *words;
  const int64_t *word_off; /* [n_experts] */
  const uint32_t *sz;      /* half2 pairs, see moeq_prep_scales       */
  const int64_t *sz_off;   /* [n_experts] */
  const int32_t *nbits;    /* [n_experts] */
  int32_t K, N, group_size, dq_mode;
} moeq_proj;

/* One MoE layer.  Experts [0, n_experts) are routed; experts
 * [n_experts, n_experts + n_shared) are always-on shared experts of the same
 * width `inter` (DeepSeek's fused shared MLP split into column blocks), added
 * with weight 1. */
typedef struct moeq_moe {
  int32_t hidden, inter, n_experts, top_k, n_shared;
  int32_t act_dtype;  /* MOEQ_F16 | MOEQ_BF16: x, logits (unless gate is F32)  */
  int32_t gate_dtype; /* MOEQ_F16 | MOEQ_BF16 | MOEQ_F32 (DeepSeek fp32 gate)   */
  int32_t norm_topk;  /* renormalize the top-k weights to sum to one           */
  const void *gate_w; /* [n_experts, hidden] in gate_dtype                     */
  moeq_proj w1, w3, w2; /* gate_proj, up_proj, down_proj                       */
  const float *logit_bias; /* [n_experts] fp32 added to the logits, or NULL     */
  /* Nonzero: a one-token forward (T == 1) routes as Mixtral's
   * forward_one_token does (gemq/inference/moe_block.py:280-283): softmax
   * probabilities rounded to act_dtype are ranked (equal values: lower expert
   * index first) and renormalised in act_dtype, w = rnd(p / rnd(sum p)).
   * Zero: every T ranks the logits with fp32 softmax weights (:245-249 and
   * the other families).  Ignored for T > 1. */
  int32_t one_token_act_softmax;
} moeq_moe;

const char *moeq_last_error(void);
int moeq_version(void);

/* ---------------------------------------------------------------- load time */

/* Pack uint8 codes [N, K] into int32 words [ceil(K/eps), N] (N contiguous),
 * eps = 32/nbits codes per word, LSB first, zero-padded tail (3-bit: 10 codes
 * per word, bits 30..31 zero).
 * Replaces pack_weights_over_cols_triton, gemq/triton_kernels/utils.py:74-113
 * (kernel :33-71), whose transposed result is the layout
 * QuantFused*MoEBlock.from_hf stacks (gemq/inference/moe_block.py:725-733). */
int moeq_pack_cols(const uint8_t *codes, int64_t N, int64_t K, int nbits,
                   int32_t *out, void *stream);

/* Rewrite one expert's reference-layout words [ceil(K/eps), N] (as above) into
 * the build layout (K*N*nbits/32 words).  K % 128 == 0, N % 16 == 0.
 * The 32 codes k = 128c + 32kb + i (i = 8t + 2d + h) of column n form the
 * nbits-word lane slice (c, n, kb), stored at word
 * ((n/16 * K/128 + c) * 64 + (n%16) * 4 + kb) * nbits; inside it the pair
 * h = 0, 1 of MFMA step t, pair d sits at one bit offset of the two 16-bit
 * halves of a word (4-bit: word t, bit 16h+4d; 2-bit: word t/2, bit
 * 16h+2(4(t%2)+d); 1-bit: word 0, bit 16h+4t+d; 3-bit: the low two bits as
 * the 2-bit plane in words 0-1, the high bit as the 1-bit plane in word 2).
 * Load-time counterpart of the stacking in from_hf,
 * gemq/inference/moe_block.py:725-757; the reference has no repack step. */
int moeq_repack(const int32_t *ref_words, int64_t K, int64_t N, int nbits,
                uint32_t *out, void *stream);

/* Fuse per-group fp16 scale s and zero z into half2 dwords:
 * MOEQ_DQ_HQQ -> (s, -z); MOEQ_DQ_AFFINE -> (s, z');
 * MOEQ_DQ_HQQ_INT -> (s, -(1024 + z)), exact for integer z in 0..1023 (the
 * caller checks that).  scales/zeros are `blocks` consecutive [groups, N]
 * arrays (one per expert, the reference's stacking); out has the same size,
 * each block panel-major: pair (g, n) at dword (n/16 * groups + g) * 16 + n%16
 * of its block.  N % 16 == 0.
 * Replaces the separate scales/zeros loads of dequantize(),
 * gemq/triton_kernels/utils.py:192-212. */
int moeq_prep_scales(const uint16_t *scales, const uint16_t *zeros, int64_t blocks,
                     int64_t groups, int64_t N, int dq_mode, uint32_t *out, void *stream);

/* ------------------------------------------------------------------ routing */

/* logits[T, E] = x[T, H] @ gate_w[E, H]^T with fp32 fused multiply-adds in a
 * fixed order (64 strided partial chains, then a xor-butterfly), plus
 * logit_bias[E] if not NULL (a routing prior for synthetic skewed workloads;
 * the reference has none), rounded to x_dtype unless gate_dtype is
 * MOEQ_F32; then p = softmax_fp32(logits),
 * top_k experts ranked by logit (ties: lower index first), optional
 * renormalisation.  logits_out may be NULL; the rounded logits are then kept
 * in ws (moeq_route_workspace_size bytes), which is unused otherwise.
 * Replaces the router of QuantFused*MoEBlock.forward_n_tokens /
 * forward_one_token: gemq/inference/moe_block.py:790-797 (OLMoE), :243-249
 * (Mixtral, always renormalized), :1020-1027 (Qwen3), :549-556 (DeepSeek,
 * fp32 gate), :828-833 (decode). */
size_t moeq_route_workspace_size(int64_t T, int E);
int moeq_route(const void *x, int x_dtype, int64_t T, int H,
               const void *gate_w, int gate_dtype, const float *logit_bias,
               int E, int top_k, int norm_topk, void *logits_out,
               int32_t *idx_out, float *w_out, void *ws, size_t ws_bytes,
               void *stream);

/* Same selection and weights from given logits [T, E] (dtype F16/BF16/F32).
 * Used for externally biased routing (e.g. a Zipf popularity prior). */
int moeq_route_from_logits(const void *logits, int dtype, int64_t T, int E,
                           int top_k, int norm_topk, int32_t *idx_out,
                           float *w_out, void *stream);

/* Stable token->expert grouping in the reference order: experts ascending,
 * then (top-k slot, token) ascending; shared experts append T rows each.
 * Outputs (device):
 *   counts[E + n_shared], offsets[E + n_shared + 1],
 *   row_token[T*top_k + n_shared*T]  token feeding each grouped row,
 *   row_pair[T*top_k]                t*top_k + slot of each routed row,
 *   inv_perm[T*top_k]                row of each (t, slot) pair,
 *   tiles[max_tiles*4]               (expert, row_start, row_count, 0): each
 *                                    expert's m rows split into
 *                                    ceil(m / moeq_tile_rows(bm)) tiles at
 *                                    16-row boundaries, the first ones of
 *                                    the class's largest block count, the
 *                                    rest of the next lower count (see
 *                                    moeq_tile_rows), in expert order,
 *   n_tiles[1].
 * max_tiles = moeq_max_tiles(T, top_k, E, n_shared, bm).
 * Replaces the one_hot / nonzero / torch.where grouping and its host syncs,
 * gemq/inference/moe_block.py:803-810 (also :256-262, :562-570, :1033-1040). */
int moeq_max_tiles(int64_t T, int top_k, int E, int n_shared, int bm);
/* Most rows one tile of tile class bm holds (the schedule's split size and
 * the grouped GEMM's row capacity): 16 -> 32, 32 -> 48, 64 -> 96,
 * 128 -> 160, 256 -> 256; 0 for any other bm.  No reference counterpart. */
int moeq_tile_rows(int bm);
size_t moeq_permute_workspace_size(int64_t T, int top_k, int E, int n_shared);
int moeq_permute(const int32_t *idx, int64_t T, int top_k, int E,
                 int n_shared, int bm, int32_t *counts, int32_t *offsets,
                 int32_t *row_token, int32_t *row_pair, int32_t *inv_perm,
                 int32_t *tiles, int32_t *n_tiles, void *ws, size_t ws_bytes,
                 void *stream);

/* ------------------------------------------------------------- expert GEMMs */

#define MOEQ_EPI_STORE 0    /* out = A @ deq(W_p0)                              */
#define MOEQ_EPI_SILU_MUL 1 /* out = silu(A @ deq(W_p0)) * (A @ deq(W_p1)), f16 */

typedef struct moeq_gemm {
  const void *a;            /* activations, rows addressed via row_src      */
  int32_t a_dtype;          /* MOEQ_F16 (any bm) | MOEQ_BF16 (bm == 16)      */
  int64_t lda;              /* elements                                      */
  const int32_t *row_src;   /* [rows] source row of each grouped row, NULL = identity */
  const int32_t *tiles;     /* from moeq_permute (or built by the caller)    */
  const int32_t *n_tiles;   /* device scalar                                 */
  int32_t max_tiles;        /* host bound on *n_tiles                        */
  int32_t bm;               /* tile class the schedule was built for: 16, 32, 64, 128 or 256;
                               every tile holds at most moeq_tile_rows(bm) rows */
  int32_t epilogue;         /* MOEQ_EPI_*                                    */
  void *out;                /* [rows, N] (split s at out + s*split_stride)   */
  int32_t out_dtype;        /* MOEQ_F16 | MOEQ_F32 (split-K needs F32)       */
  int64_t ldo;              /* elements                                      */
  int32_t splits;           /* >= 1, splits of K (single projection only)    */
  int64_t split_stride;     /* elements                                      */
} moeq_gemm;

/* One launch over every row tile of every expert:
 * out[r, :] = epilogue(A[row_src[r], :] @ deq(W[expert(r)])).
 * p1 must be NULL for MOEQ_EPI_STORE and match p0's layout for SILU_MUL.
 * Every A row the tiles address (row_src[r], or r) must lie wholly within
 * the first 2 GiB from a, i.e. (row + 1) * lda * element size <= 2^31
 * (every tile class addresses rows with 32-bit offsets; the caller checks
 * this, the library cannot see the rows row_src names); one expert's packed
 * words must be < 2 GiB.
 * Replaces the per-expert launches of dequant_group_gemm_triton
 * (gemq/triton_kernels/dequant_group_gemm.py:155-202, called once per hit
 * expert at gemq/inference/moe_block.py:766-777), dequant_gemm_triton
 * (dequant_gemm.py:150-193) and, at decode, fused_dequant_up_proj_triton /
 * fused_dequant_down_proj_triton (fused_dequant_bmm.py:122-173, :264-312)
 * and dequant_splitk_gemv_triton (dequant_gemv.py:118-156). */
int moeq_grouped_gemm(const moeq_gemm *g, const moeq_proj *p0,
                      const moeq_proj *p1, void *stream);

/* out[t, :] = sum_slot w[t, slot] * sum_s y_s[inv_perm[t*top_k+slot], :]
 *           + sum_{v < n_shared} sum_s y_s[T*top_k + v*T + t, :]
 * y is F16 or F32 ([rows, H], split s at y + s*split_stride); out is F16,
 * BF16 or F32.  Deterministic: fixed summation order, no atomics.
 * Replaces the weighted index_add_ / einsum combine,
 * gemq/inference/moe_block.py:811-812 (prefill), :849-850 (decode),
 * :575 and :620 (DeepSeek shared experts). */
int moeq_combine(const void *y, int y_dtype, int splits, int64_t split_stride,
                 int64_t ldy, const int32_t *inv_perm, const float *w,
                 int64_t T, int top_k, int n_shared, int H, void *out,
                 int out_dtype, void *stream);

/* out[i] = fp16(silu(x1[i]) * x3[i]) for i < n, computed in fp32 from fp16
 * x1 / x3 (the gate/up epilogue's arithmetic).  n % 8 == 0.
 * Replaces the fp32 SiLU*mul prologue of fused_dequant_down_proj_triton,
 * gemq/triton_kernels/fused_dequant_bmm.py:229-239 (and the eager
 * F.silu(x1) * x3 of moe_block.py:775); the product then feeds
 * moeq_grouped_gemm. */
int moeq_silu_mul(const uint16_t *x1, const uint16_t *x3, int64_t n,
                  uint16_t *out, void *stream);

/* ------------------------------------------------------------- whole layer */

/* Workspace for moeq_moe_forward with T tokens. */
size_t moeq_moe_workspace_size(const moeq_moe *m, int64_t T);

/* out[T, H] = MoE(x[T, H]); logits_out ([T, E], may be NULL) receives the
 * router logits in act_dtype (F32 for an F32 gate).  out_dtype is act_dtype
 * or MOEQ_F32.  Route, permute, grouped gate/up (SiLU*mul fused), grouped
 * down, combine: seven launches, no host synchronisation.
 * Replaces QuantFused*MoEBlock.forward (gemq/inference/moe_block.py:855-858)
 * and both branches it dispatches to: forward_n_tokens (:781-815; Mixtral
 * :234-267, Qwen3 :1011-1045, DeepSeek :540-578) and forward_one_token
 * (:817-853; DeepSeek :580-623). */
int moeq_moe_forward(const moeq_moe *m, const void *x, int64_t T, void *out,
                     int out_dtype, void *logits_out, void *ws,
                     size_t ws_bytes, void *stream);

/* Size of the static scratch array moeq_moe_forward_static uses on each GPU
 * (64 MiB: moeq_moe_workspace_size of up to about 1024 tokens of the
 * OLMoE / Qwen3 / DeepSeek-shaped layers, 800 of the Mixtral-shaped one). */
#define MOEQ_STATIC_SCRATCH_BYTES (64u << 20)

/* moeq_moe_forward without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Scratch memory is a file-scope device array of MOEQ_STATIC_SCRATCH_BYTES per
 * GPU, which the library holds until the process ends; the call allocates
 * nothing and returns MOEQ_ERR_WORKSPACE, launching nothing, when
 * moeq_moe_workspace_size(m, T) exceeds the array.  It runs on the current
 * device, which must be the stream's.  Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (other streams or threads) race
 * and must be serialised by the caller.  Same results as moeq_moe_forward. */
int moeq_moe_forward_static(const moeq_moe *m, const void *x, int64_t T, void *out,
                            int out_dtype, void *logits_out, void *stream);

/* ------------------------------------------------------------ introspection
 * No reference counterpart: launch-plan queries used by the Python host
 * layer, the tests and the benchmark. */

/* Column tile width of moeq_grouped_gemm for (bm, epilogue); 0 if invalid. */
int moeq_gemm_tile_n(int bm, int epilogue);

/* Plan moeq_moe_forward uses for T tokens: out4 = {bm, down-proj K splits,
 * max_tiles, dtype of the grouped down-projection output}. */
int moeq_moe_plan(const moeq_moe *m, int64_t T, int32_t *out4);

/* moeq_moe_forward that also records two HIP events (hipEvent_t, passed as
 * void *) on `stream`, just before and just after its gate/up grouped-GEMM
 * launch, so a benchmark can time that kernel inside the layer.  Benchmark
 * introspection; no reference counterpart. */
int moeq_moe_forward_timed(const moeq_moe *m, const void *x, int64_t T, void *out,
                           int out_dtype, void *logits_out, void *ws, size_t ws_bytes,
                           void *stream, void *ev_gate_up_begin, void *ev_gate_up_end);

/* Byte offsets, in the workspace of moeq_moe_forward for T tokens, of the
 * routing and permutation it leaves there: out9 = {idx, w, counts, offsets,
 * row_token, row_pair, inv_perm, tiles, n_tiles} (layouts as moeq_route and
 * moeq_permute write them).  Introspection for tests; no reference
 * counterpart. */
int moeq_moe_workspace_layout(const moeq_moe *m, int64_t T, int64_t *out9);

#ifdef __cplusplus
}
#endif

#endif /* MOEQ_H_ */
