/*
 * nt_moe.h -- C ABI of the MI355X (gfx950) mixture-of-experts layer (forward and backward).
 *
 * One shared library, libnt_moe.so, exports these entry points. Every entry point
 *   - returns an int status: NT_MOE_OK (0) or a negative NT_MOE_E* code;
 *   - records a message for the calling thread, read back with nt_moe_last_error();
 *   - never throws, never allocates device memory, never synchronises the stream;
 *   - takes caller-owned device buffers as plain pointers plus explicit sizes, and
 *     enqueues its kernels on the caller's hipStream_t (0 = the null stream).
 * Scratch memory is passed in as `workspace` and sized by the *_workspace_bytes queries.
 *
 * Element types: "bf16" buffers hold IEEE bfloat16 bit patterns (uint16_t); "e4m3" buffers
 * hold OCP FP8 E4M3FN bytes (max finite 448, the gfx950 hardware format); all indices are
 * int32 and all scales, weights and losses are fp32.
 *
 * Reference interfaces these replace (paths relative to the NextTransformer tree):
 *   router      -> NativeRouter.gating + TopKRouter routing
 *                  (nexttransformer/scaling/megatron_moe.py:86-102, :43-45),
 *                  RoutedFFN router/topk/softmax (nexttransformer/scaling/reference_blocks.py:37-38)
 *   route plan  -> mapping.T.nonzero / mapping.sum(0) / probs.T[mapping.T] / rows[ids]
 *                  (nexttransformer/scaling/megatron_moe.py:142-145)
 *   grouped ffn -> SequentialMLP over MasterLinear (megatron_moe.py:58-78, :145) and
 *                  FlexibleMLP (nexttransformer/models/lm.py:29-35)
 *   combine     -> zeros_like(rows).index_add(0, ids, output) + shared_experts
 *                  (megatron_moe.py:148-150); RoutedFFN index_add loop (reference_blocks.py:39-44)
 *   aux loss    -> TopKRouter aux/z loss with moe_aux_loss_coeff / moe_z_loss_coeff
 *                  (megatron_moe.py:44-45; nexttransformer/scaling/moe_recipe.py:40-41)
 */
#ifndef NT_MOE_H
#define NT_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NT_MOE_ABI_VERSION 1

#define NT_MOE_OK 0
#define NT_MOE_EINVAL (-22)  /* invalid argument: shape, pointer, enum, alignment */
#define NT_MOE_ENOSPC (-28)  /* workspace smaller than the matching *_workspace_bytes query */
#define NT_MOE_EDEVICE (-5)  /* HIP runtime error while launching */

/* score_fn values (TopKRouter moe_router_score_function). */
#define NT_MOE_SCORE_SOFTMAX 0 /* top-k on logits, softmax over the k selected */
#define NT_MOE_SCORE_SIGMOID 1 /* top-k on logits, sigmoid scores normalised over the k selected */

/* activation values of the expert FFN. */
#define NT_MOE_ACT_SWIGLU 0 /* fc1 rows [0,H) are the gate, [H,2H) the value: silu(g) * u */
#define NT_MOE_ACT_RELU2 1  /* fc1 has H rows: relu(g)^2 (megatron_moe.py:23-24) */

/* epilogue values of nt_moe_grouped_gemm_bf16. */
#define NT_MOE_EPI_SWIGLU 0 /* w has 2 n_out rows: c = silu(a.w[j]) * a.w[n_out + j] */
#define NT_MOE_EPI_RELU2 1  /* c = relu(a.w[j])^2 */
#define NT_MOE_EPI_NONE 2   /* c = a.w[j] */

/* Largest supported sizes. */
#define NT_MOE_MAX_EXPERTS 256
#define NT_MOE_MAX_TOPK 8
#define NT_MOE_MAX_SEGMENTS 512
/* Tokens per router / histogram block: aux partial buffers have ceil(T / 64) rows. */
#define NT_MOE_ROUTE_BLOCK 64

typedef struct ihipStream_t* nt_moe_stream_t; /* a hipStream_t */

int nt_moe_abi_version(void);
const char* nt_moe_last_error(void);

/*
 * Router: logits = x . Wr^T (+ bias) in fp32 with a fixed reduction order, then scoring and
 * top-k. Replaces NativeRouter.gating (megatron_moe.py:95-100) and TopKRouter's top-k /
 * softmax-over-selected (megatron_moe.py:43; reference_blocks.py:37-38).
 *
 * Fixed order (the bit-exact contract): for each (t, e), c_j = fma-chain over the features
 * k in [128 j, min(128 j + 128, d)) in ascending k, starting from 0.0f; logit = c_0 + c_1 + ...
 * added left to right; then logit += bias[e] when bias is given. x is widened exactly.
 * Top-k: descending logit; equal logits go to the lower expert index.
 *
 *   x           bf16 [T, ld_x], d used columns (d % 8 == 0, ld_x % 8 == 0)
 *   w_router_t  fp32 [d, E]  (the router weight transposed, E contiguous)
 *   logit_bias  fp32 [E] or NULL
 *   logits      fp32 [T, E] or NULL (written when given)
 *   topk_ids    int32 [T, k], topk_w fp32 [T, k]
 *   prob_partial fp32 [ceil(T/64), E]: per 64-token block, sum over its tokens of the
 *                full score s_te (softmax over all E, or sigmoid normalised over all E)
 *   z_partial   fp32 [ceil(T/64)]: per block, sum of logsumexp(logits_t)^2
 *   workspace   nt_moe_router_workspace_bytes(T, d, E, k) bytes; may be smaller (or NULL)
 *               for E <= 256, which then takes a single-kernel path (slower for small T);
 *               E > 256 needs it (or logits, with d <= 2048)
 */
size_t nt_moe_router_workspace_bytes(int64_t T, int32_t d, int32_t E, int32_t k);
int nt_moe_router_fwd(const uint16_t* x, int64_t ld_x, const float* w_router_t,
                      const float* logit_bias, int64_t T, int32_t d, int32_t E, int32_t k,
                      int32_t score_fn, float* logits, int32_t* topk_ids, float* topk_w,
                      float* prob_partial, float* z_partial, void* workspace,
                      size_t workspace_bytes, nt_moe_stream_t stream);

/*
 * Top-k and scoring from caller-supplied fp32 logits [T, E] (no gating GEMM): the same
 * selection, weights and partials as nt_moe_router_fwd. Lets routing be checked on logits
 * computed elsewhere (e.g. the reference's own F.linear, megatron_moe.py:99).
 */
int nt_moe_topk_from_logits(const float* logits, int64_t T, int32_t E, int32_t k,
                            int32_t score_fn, int32_t* topk_ids, float* topk_w,
                            float* prob_partial, float* z_partial, nt_moe_stream_t stream);

/*
 * Route plan: per-expert histogram of topk_ids with an LDS prefix scan.
 * Replaces counts = mapping.sum(0) (megatron_moe.py:143) and the offsets implied by the
 * expert-major order of mapping.T.nonzero() (megatron_moe.py:142).
 *   counts   int32 [E]    tokens routed to each expert
 *   offsets  int32 [E+1]  exclusive prefix of counts (offsets[E] = T*k)
 *   workspace nt_moe_route_workspace_bytes(T, k, E) bytes; pass the same buffer,
 *            unmodified, to nt_moe_permute.
 */
size_t nt_moe_route_workspace_bytes(int64_t T, int32_t k, int32_t E);
int nt_moe_histogram_scan(const int32_t* topk_ids, int64_t T, int32_t k, int32_t E,
                          int32_t* counts, int32_t* offsets, void* workspace,
                          size_t workspace_bytes, nt_moe_stream_t stream);

/*
 * Permute: the expert-major, token-ascending permutation (megatron_moe.py:142-145).
 * Destination row of (t, j) = offsets[e] + #{t' < t routed to e}, e = topk_ids[t, j].
 *   src_row       int32 [T*k]  token feeding each permuted row (ids of the reference)
 *   perm_w        fp32 [T*k] or NULL  routing weight of each permuted row (selected_probs)
 *   combine_dest  int32 [T, k] permuted rows of token t, in ascending expert order
 *   combine_w     fp32  [T, k] matching routing weights
 *   x_perm        bf16 [T*k, d] or NULL: the gathered rows rows[ids] (x read once per token)
 */
int nt_moe_permute(const uint16_t* x, int64_t ld_x, const int32_t* topk_ids,
                   const float* topk_w, int64_t T, int32_t d, int32_t k, int32_t E,
                   const void* workspace, size_t workspace_bytes, int32_t* src_row,
                   float* perm_w, int32_t* combine_dest, float* combine_w, uint16_t* x_perm,
                   nt_moe_stream_t stream);

/*
 * Route plan in one call: the outputs of nt_moe_histogram_scan followed by nt_moe_permute with
 * the same arguments (megatron_moe.py:142-145,149), the workspace sized by
 * nt_moe_route_workspace_bytes(T, k, E). With x_perm NULL and ceil(T/256) * E <= 16384 the
 * offset scan runs inside the permutation kernel (two launches instead of three); otherwise it
 * makes exactly those two calls.
 */
int nt_moe_route_plan(const uint16_t* x, int64_t ld_x, const int32_t* topk_ids,
                      const float* topk_w, int64_t T, int32_t d, int32_t k, int32_t E,
                      int32_t* counts, int32_t* offsets, void* workspace, size_t workspace_bytes,
                      int32_t* src_row, float* perm_w, int32_t* combine_dest, float* combine_w,
                      uint16_t* x_perm, nt_moe_stream_t stream);

/*
 * Router and route plan in one call: the outputs of nt_moe_router_fwd followed by those of
 * nt_moe_route_plan without x_perm, identical bits. When ceil(T/64) * E <= 16384 in two launches
 * instead of three: the router's top-k also writes each 64-token block's assignments per expert
 * and each assignment's rank within its block into the workspace, so the plan needs no
 * histogram launch; larger shapes make exactly the router and route-plan launches. Replaces
 * NativeRouter.gating + TopKRouter (megatron_moe.py:95-100, 43) followed by
 * mapping.T.nonzero() / mapping.sum(0) (megatron_moe.py:142-144).
 *   workspace  nt_moe_router_plan_workspace_bytes(T, d, E, k) bytes (never smaller)
 * Other arguments as in nt_moe_router_fwd and nt_moe_route_plan.
 */
size_t nt_moe_router_plan_workspace_bytes(int64_t T, int32_t d, int32_t E, int32_t k);
int nt_moe_router_plan(const uint16_t* x, int64_t ld_x, const float* w_router_t,
                       const float* logit_bias, int64_t T, int32_t d, int32_t E, int32_t k,
                       int32_t score_fn, float* logits, int32_t* topk_ids, float* topk_w,
                       float* prob_partial, float* z_partial, int32_t* counts, int32_t* offsets,
                       int32_t* src_row, float* perm_w, int32_t* combine_dest,
                       float* combine_w, void* workspace, size_t workspace_bytes,
                       nt_moe_stream_t stream);

/*
 * nt_moe_route_plan without a workspace argument: the same outputs, the same kernels, with
 * their scratch (ranks and per-block counts) in a static device array of the library instead.
 * No counterpart in the reference; it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): it calls no
 * hipMalloc, hipFree or other allocating routine. Limits: T * k <= NT_MOE_NOALLOC_MAX_ASSIGNMENTS
 * and ceil(T / 256) * E <= NT_MOE_NOALLOC_MAX_BLOCK_COUNTS (the array is 2 MiB per GPU, held
 * until the process ends); larger sizes fail with NT_MOE_EINVAL. The stream must belong to the
 * current device. Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (on different streams, or from different threads) race, so serialise them.
 */
#define NT_MOE_NOALLOC_MAX_ASSIGNMENTS (1 << 18)
#define NT_MOE_NOALLOC_MAX_BLOCK_COUNTS (1 << 18)
int nt_moe_route_plan_noalloc(const uint16_t* x, int64_t ld_x, const int32_t* topk_ids,
                              const float* topk_w, int64_t T, int32_t d, int32_t k, int32_t E,
                              int32_t* counts, int32_t* offsets, int32_t* src_row, float* perm_w,
                              int32_t* combine_dest, float* combine_w, uint16_t* x_perm,
                              nt_moe_stream_t stream);

/*
 * Grouped expert FFN over ragged segments, bf16 MFMA with fp32 accumulation:
 *   h[r] = act(a_r . W1_s^T)  (bf16 [rows, H]),   y[r] = h[r] . W2_s^T  (bf16 [rows, d])
 * for every row r of segment s, rows [seg_offsets[s], seg_offsets[s+1]).
 * Replaces SequentialMLP's per-expert loop (megatron_moe.py:145) over MasterLinear
 * fc1 -> activation -> fc2 (megatron_moe.py:58-78; lm.py:29-35).
 *   a            bf16 [a_rows, ld_a]: row r reads a[src_row[r]] when src_row is given
 *                (gather fused into the load; indices are clamped to [0, a_rows)), else a[r]
 *   seg_offsets  int32 [num_segments+1], device memory, non-decreasing, [0] = 0; values are
 *                clamped to [0, total_rows]
 *   w1           bf16 [num_segments, F, d], F = 2H (SWIGLU) or H (RELU2)
 *   w2           bf16 [num_segments, d, H]
 *   h            bf16 [total_rows, H] (intermediate, caller-owned)
 *   y            bf16 [total_rows, d]
 *   total_rows   upper bound of seg_offsets[num_segments] used to size the launch
 *   workspace    nt_moe_grouped_gemm_workspace_bytes() bytes of device memory, reserved for
 *                the tile scheduler: required, but the static per-XCD schedule of this
 *                version neither reads nor writes it
 * Requirements: d % 64 == 0, H % 64 == 0, 16-byte aligned buffers, a_rows * ld_a * 2 and one
 * segment's weights each within 4 GiB.
 */
size_t nt_moe_grouped_gemm_workspace_bytes(void);
int nt_moe_grouped_ffn_bf16(const uint16_t* a, int64_t ld_a, int64_t a_rows, const int32_t* src_row,
                            const int32_t* seg_offsets, int32_t num_segments,
                            int64_t total_rows, const uint16_t* w1, const uint16_t* w2,
                            int32_t d, int32_t H, int32_t activation, uint16_t* h,
                            uint16_t* y, void* workspace, size_t workspace_bytes,
                            nt_moe_stream_t stream);

/*
 * One grouped GEMM launch over ragged segments (the building block of nt_moe_grouped_ffn_bf16):
 *   c[r, j] = epilogue(a_r . w_s[j, :])  for r in segment s, j in [0, n_out)
 *   w  bf16 [num_segments, 2 n_out (SWIGLU) or n_out, K];  c bf16 [total_rows, n_out]
 * Requirements: K % 64 == 0, n_out % 4 == 0 (n_out % 64 == 0 for SWIGLU), 16-byte alignment;
 * workspace as for nt_moe_grouped_ffn_bf16. With K >= 128 and n_out % 8 == 0 the launch runs
 * 256 x 256 tiles with both operands staged through LDS, multiplying in the same K order as
 * nt_moe_grouped_gemm_bf16_packed (bit-identical results).
 */
int nt_moe_grouped_gemm_bf16(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                             const int32_t* src_row, const int32_t* seg_offsets,
                             int32_t num_segments, int64_t total_rows, const uint16_t* w,
                             int32_t K, int32_t n_out, int32_t epilogue, uint16_t* c,
                             void* workspace, size_t workspace_bytes, nt_moe_stream_t stream);

/*
 * nt_moe_grouped_gemm_bf16 with the SWIGLU or RELU2 epilogue that also stores the epilogue's
 * input, the fc1 pre-activations, to pre: bf16 [total_rows, 2 n_out] (SwiGLU: gate then value)
 * or [total_rows, n_out] (ReLU^2), rounded from the same fp32 accumulators: what autograd saves
 * from the fc1 product and activation for the backward (megatron_moe.py:23-24,58-78;
 * lm.py:29-35), read by nt_moe_act_bwd. Needs the 256 x 256 path: K >= 128, n_out % 8 == 0;
 * 16-byte aligned; total_rows * width * 2 < 2^31. No workspace.
 */
int nt_moe_grouped_gemm_bf16_keep(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                  const int32_t* src_row, const int32_t* seg_offsets,
                                  int32_t num_segments, int64_t total_rows, const uint16_t* w,
                                  int32_t K, int32_t n_out, int32_t epilogue, uint16_t* c,
                                  uint16_t* pre, nt_moe_stream_t stream);

/*
 * Weight preparation: the fp32 master weights w [num_matrices, rows, cols] to bf16, in one read:
 * out [num_matrices, rows, cols] (the cast MasterLinear applies before each product,
 * megatron_moe.py:74-75) and out_t [num_matrices, cols, rows] (its transpose, the dgrad
 * operand of the backward); either may be NULL. Rounding to nearest even. rows and cols
 * multiples of 64; 16-byte aligned buffers.
 */
int nt_moe_convert_expert_weights(const float* w, int64_t num_matrices, int32_t rows,
                                  int32_t cols, uint16_t* out, uint16_t* out_t,
                                  nt_moe_stream_t stream);

/*
 * The same single read of the fp32 masters, with two more optional outputs in the packed GEMM's
 * fragment order (the layout nt_moe_pack_expert_weights_bf16 writes): packed = w packed for
 * `epilogue` (for SWIGLU, rows = 2 n_out, gate and value rows paired), packed_t = w^T
 * [num_matrices, cols, rows] packed as a plain projection (EPI_NONE). Bit-identical to
 * nt_moe_convert_expert_weights followed by nt_moe_pack_expert_weights_bf16, without the second
 * pass over the bf16 copy that every weight update would otherwise pay. Any output may be NULL.
 * rows and cols multiples of 64; 16-byte aligned buffers. No counterpart in the reference beyond
 * the per-product cast it prepares (megatron_moe.py:74-75).
 */
int nt_moe_convert_expert_weights_packed(const float* w, int64_t num_matrices, int32_t rows,
                                         int32_t cols, uint16_t* out, uint16_t* out_t,
                                         uint16_t* packed, int32_t epilogue, uint16_t* packed_t,
                                         nt_moe_stream_t stream);

/*
 * The router's operands from its fp32 weight W [num_experts, d] (row stride ld_w), rebuilt after
 * every weight update in one pass (MasterLinear's per-product cast of the gate weight,
 * megatron_moe.py:58-78,99): w_router_t = W^T fp32 [dp, num_experts] (dp >= d; rows d .. dp - 1
 * zero), the layout nt_moe_router_fwd reads, and, when `first` is not NULL, the backward's
 * concatenated operand first bf16 [dp, Kc]: columns [0, Fs) = S^T for the shared expert's W1
 * S bf16 [Fs, dp] (row stride ld_s; Fs may be 0), hi = bf16(W^T) at [Fs, Fs + E),
 * lo = bf16(W^T - hi) at [Fs + Ep, Fs + Ep + E), hi at [Fs + 2 Ep, Fs + 2 Ep + E), every other
 * column zero (Ep >= E, Kc >= Fs + 3 Ep); rounding to nearest even. No counterpart in the
 * reference beyond the cast and the autograd of F.linear it prepares.
 */
int nt_moe_router_operands(const float* w, int64_t ld_w, int32_t num_experts, int32_t d,
                           int32_t dp, const uint16_t* shared_w1, int64_t ld_s, int32_t Fs,
                           float* w_router_t, uint16_t* first, int32_t Ep, int32_t Kc,
                           nt_moe_stream_t stream);

/*
 * Packed-weight variant of the grouped GEMM. nt_moe_pack_expert_weights_bf16 rearranges
 * w [num_segments, rows, K] once (same bytes, fragment order: 32-row x 64-K blocks in which
 * each lane's 16-byte operand chunk is contiguous with its neighbours', rows inside a block
 * ordered so that each lane's accumulators are 8 consecutive output columns); the packed GEMM then
 * streams each wave's weights straight into registers and stages only the token rows in LDS.
 * `epilogue` must be the one the packed weights will be used with (for SWIGLU the gate and value
 * rows of the same output columns are packed together). No counterpart in the reference beyond
 * the expert loop it replaces (megatron_moe.py:145).
 *   pack:  w bf16 [num_segments, rows, K] -> packed bf16 [num_segments, rows, K] (same size)
 *          rows % 32 == 0 (rows = 2 n_out for SWIGLU), K % 64 == 0
 *   gemm:  as nt_moe_grouped_gemm_bf16 with w = packed weights; K % 64 == 0 and K >= 256;
 *          n_out % 16 == 0 (SWIGLU) or % 32; total_rows * n_out * 2 < 2^31; a, w_packed and
 *          c 16-byte aligned.
 */
int nt_moe_pack_expert_weights_bf16(const uint16_t* w, int64_t num_segments, int32_t rows,
                                    int32_t K, int32_t epilogue, uint16_t* packed,
                                    nt_moe_stream_t stream);
int nt_moe_grouped_gemm_bf16_packed(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                    const int32_t* src_row, const int32_t* seg_offsets,
                                    int32_t num_segments, int64_t total_rows,
                                    const uint16_t* w_packed, int32_t K, int32_t n_out,
                                    int32_t epilogue, uint16_t* c, nt_moe_stream_t stream);

/*
 * nt_moe_grouped_gemm_bf16_packed with the SWIGLU or RELU2 epilogue that also stores the
 * epilogue's input, the fc1 pre-activations, to pre: bf16 [total_rows, 2 n_out] (SwiGLU: gate
 * then value) or [total_rows, n_out] (ReLU^2), rounded from the same fp32 accumulators: what
 * autograd saves from the fc1 product and activation for the backward (megatron_moe.py:23-24,
 * 58-78; lm.py:29-35), read by nt_moe_act_bwd; otherwise the backward recomputes them with an
 * EPI_NONE launch. 16-byte aligned; total_rows * width * 2 < 2^31.
 */
int nt_moe_grouped_gemm_bf16_packed_keep(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                         const int32_t* src_row, const int32_t* seg_offsets,
                                         int32_t num_segments, int64_t total_rows,
                                         const uint16_t* w_packed, int32_t K, int32_t n_out,
                                         int32_t epilogue, uint16_t* c, uint16_t* pre,
                                         nt_moe_stream_t stream);

/*
 * FP8 path (OCP E4M3FN, the format of gfx950's matrix cores). The reference has no fp8
 * experts -- its MasterLinear runs bf16/fp32 matmuls (megatron_moe.py:58-78) -- so these entry
 * points are the fp8 variant of the same expert computation (megatron_moe.py:145) for the
 * memory-bound small-batch regime, scored against the fp32 computation on dequantised values.
 *
 * Row-wise quantisation of activations: per row, s = amax(|row|) / 448 (1 for an all-zero
 * row), q = e4m3(v / s) rounded to nearest even.
 *   x      bf16 [rows, ld_x], d used columns (d % 8 == 0, ld_x % 8 == 0)
 *   q      e4m3 [rows, ld_q] (ld_q >= d, ld_q % 8 == 0);  scale fp32 [rows]
 */
int nt_moe_quantize_fp8_rowwise(const uint16_t* x, int64_t ld_x, int64_t rows, int32_t d,
                                uint8_t* q, int64_t ld_q, float* scale, nt_moe_stream_t stream);

/*
 * Block-wise quantisation of weights: every 128 x 128 block of each [rows, cols] matrix gets
 * s = amax(|block|) / 448 (1 for an all-zero block) and q = e4m3(v / s).
 *   w      fp32 [num_matrices, rows, cols] (rows % 128 == 0, cols % 128 == 0)
 *   q      e4m3 [num_matrices, rows, cols];  scale fp32 [num_matrices, rows/128, cols/128]
 */
int nt_moe_quantize_fp8_blockwise(const float* w, int64_t num_matrices, int32_t rows,
                                  int32_t cols, uint8_t* q, float* scale, nt_moe_stream_t stream);

/*
 * Grouped GEMM on e4m3 operands with fp32 scales, over ragged segments:
 *   c[r, j] = epilogue( a_scale[i] * sum_kb w_scale[s, row/128, kb] *
 *                       sum_{k in [128 kb, 128 kb + 128)} a[i, k] * w[s, row, k] )
 * with i = src_row[r] when given (gather fused into the load, clamped to [0, a_rows)), else r;
 * `row` is j for NONE/RELU2, and j (gate) and n_out + j (value) for SWIGLU.
 *   a        e4m3 [a_rows, ld_a] (ld_a % 32 == 0), a_scale fp32 [a_rows]
 *   w        e4m3 [num_segments, R, K], R = 2 n_out (SWIGLU) or n_out, R % 128 == 0
 *   w_scale  fp32 [num_segments, R/128, K/128]
 *   c        bf16 [total_rows, n_out]
 * Requirements: K % 128 == 0; n_out % 64 == 0 (SWIGLU) or n_out % 128 == 0; 32-byte aligned
 * a and w; 8-byte aligned c. The kernel streams each segment's weights once per 32 rows of the
 * segment: it is the right tool when segments are short (decode, small batches).
 */
int nt_moe_grouped_gemm_fp8(const uint8_t* a, int64_t ld_a, int64_t a_rows, const float* a_scale,
                            const int32_t* src_row, const int32_t* seg_offsets,
                            int32_t num_segments, int64_t total_rows, const uint8_t* w,
                            const float* w_scale, int32_t K, int32_t n_out, int32_t epilogue,
                            uint16_t* c, nt_moe_stream_t stream);

/*
 * Packed fp8 weights: nt_moe_pack_expert_weights_fp8 rearranges e4m3 w [num_segments, rows, K]
 * (same bytes; the block scales keep their [num_segments, rows/128, K/128] layout) so that each
 * wave of nt_moe_grouped_gemm_fp8_packed streams its 32 weight rows as consecutive 4 KB blocks,
 * one per 128-wide K block, instead of 32 strided 128-byte pieces. `epilogue` must match the
 * GEMM's (SWIGLU packs 16 gate rows with the 16 value rows of the same columns).
 *   pack: rows % 128 == 0 (rows = 2 n_out for SWIGLU), K % 128 == 0
 *   gemm: as nt_moe_grouped_gemm_fp8 with w = packed weights.
 */
int nt_moe_pack_expert_weights_fp8(const uint8_t* w, int64_t num_segments, int32_t rows,
                                   int32_t K, int32_t epilogue, uint8_t* packed,
                                   nt_moe_stream_t stream);
int nt_moe_grouped_gemm_fp8_packed(const uint8_t* a, int64_t ld_a, int64_t a_rows,
                                   const float* a_scale, const int32_t* src_row,
                                   const int32_t* seg_offsets, int32_t num_segments,
                                   int64_t total_rows, const uint8_t* w_packed,
                                   const float* w_scale, int32_t K, int32_t n_out,
                                   int32_t epilogue, uint16_t* c, nt_moe_stream_t stream);

/*
 * Deterministic weighted combine plus the load-balance and z auxiliary losses.
 *   out[t] = sum over j in ascending expert order of combine_w[t,j] * y[combine_dest[t,j]]
 *            (+ shared_y[t] when given), accumulated in fp32, rounded once to bf16.
 * Replaces zeros_like(rows).index_add(0, ids, output) + shared_experts(hidden)
 * (megatron_moe.py:148-150) and RoutedFFN's per-expert index_add (reference_blocks.py:39-44).
 * Aux (MCore "aux_loss" type, megatron_moe.py:44-45):
 *   lb = aux_coeff * E / (k * T^2) * sum_e (sum_t s_te) * counts[e]
 *   z  = z_coeff * mean_t logsumexp(logits_t)^2
 *   aux_out fp32 [3] = {lb + z, lb, z}
 */
int nt_moe_combine_aux(const uint16_t* y, const int32_t* combine_dest, const float* combine_w,
                       int64_t T, int32_t d, int32_t k, const uint16_t* shared_y,
                       int64_t ld_shared, uint16_t* out, int64_t ld_out,
                       const float* prob_partial, const float* z_partial,
                       const int32_t* counts, int32_t E, float aux_coeff, float z_coeff,
                       float* aux_out, nt_moe_stream_t stream);

/*
 * Backward of the layer (autograd through megatron_moe.py:137-150 and the MCore router and
 * aux losses, megatron_moe.py:43-45,95-100; the reference trains through it, e.g.
 * tests/test_megatron_moe.py:183-197). The grouped dgrad GEMMs use the forward entry points
 * with transposed weights; these three cover the rest. All reductions have a fixed shape.
 *
 * Combine transpose: for token t and its k assignments (combine_dest / combine_w from
 * nt_moe_permute, ascending expert order)
 *   grad_y[dest]   = w * grad_out[t]                 bf16 [T*k, d] (expert-major rows)
 *   grad_w[t, j]   = <grad_out[t], y[dest of slot j]> fp32 [T, k], top-k slot order of topk_ids
 * y is the forward's expert output (bf16 [T*k, d]); d % 8 == 0, ld_grad % 8 == 0.
 */
int nt_moe_combine_bwd(const uint16_t* grad_out, int64_t ld_grad, const uint16_t* y,
                       const int32_t* topk_ids, const int32_t* combine_dest,
                       const float* combine_w, int64_t T, int32_t d, int32_t k,
                       uint16_t* grad_y, float* grad_w, nt_moe_stream_t stream);

/*
 * Activation backward (megatron_moe.py:23-24, lm.py:29-35): grad_fc1 from grad_h [rows, H] and
 * the fc1 pre-activations [rows, F] (F = 2H for SwiGLU, gate then value; H for ReLU^2), bf16.
 * H % 8 == 0.
 */
int nt_moe_act_bwd(const uint16_t* fc1, const uint16_t* grad_h, int64_t rows, int32_t H,
                   int32_t activation, uint16_t* grad_fc1, nt_moe_stream_t stream);

/*
 * The backward's first-row operand (the shared expert's and the router's input gradients as
 * one GEMM over a concatenated K; autograd of megatron_moe.py:95-99's router GEMM and of the
 * shared expert, :150): out bf16 [T, Kc] rows
 *   [dfc1s (Fs) | g_hi (Ep) | g_hi (Ep) | g_lo (Ep) | 0 ...],   g = grad_logits fp32 [T, E]
 * g_hi = g rounded to bf16 (nearest even), g_lo = (g - g_hi) rounded to bf16, columns past E of
 * each Ep block zero. dfc1s bf16 [T, Fs] (the shared expert's fc1 gradient; Fs = 0: none).
 * E <= Ep; Fs, Ep, Kc multiples of 8; Kc >= Fs + 3 Ep. 16-byte aligned.
 */
int nt_moe_backward_first_operand(const float* grad_logits, int32_t E, const uint16_t* dfc1s,
                                  int32_t Fs, int64_t T, int32_t Ep, int32_t Kc, uint16_t* out,
                                  nt_moe_stream_t stream);

/*
 * The two expert weight gradients of the backward in one call, over the same segments
 * (autograd of the per-expert products of megatron_moe.py:145, as nt_moe_grouped_wgrad_bf16
 * computes each): product i is c_i[s] = a_i[rows of s]^T b_i[row_i(r)], e.g. dW1 (a0 = grad_fc1,
 * b0 = x gathered through b_src_row0) and dW2 (a1 = grad_y, b1 = h, b_src_row1 = NULL); no split
 * K; c_i fp32 [num_segments, N_i, M_i] when c_fp32, else bf16. Where both products' N and M are
 * multiples of 256 they run as one launch over both tile lists (one tail instead of two), else one
 * after the other. Results are bit-identical to two nt_moe_grouped_wgrad_splitk calls with
 * splits = 1. Arguments as nt_moe_grouped_wgrad_bf16's, for each product.
 */
int nt_moe_grouped_wgrad_pair(const uint16_t* a0, int64_t lda0, const uint16_t* b0, int64_t ldb0,
                              int64_t b_rows0, const int32_t* b_src_row0, int32_t N0, int32_t M0,
                              void* c0, const uint16_t* a1, int64_t lda1, const uint16_t* b1,
                              int64_t ldb1, int64_t b_rows1, const int32_t* b_src_row1,
                              int32_t N1, int32_t M1, void* c1, const int32_t* seg_offsets,
                              int32_t num_segments, int64_t total_rows, int32_t c_fp32,
                              nt_moe_stream_t stream);

/*
 * Router backward: grad_logits fp32 [T, E] from grad_w (the routing weights' gradient, top-k
 * slot order) through the k-selected normalisation of score_fn, plus the load-balance and
 * z-loss terms when grad_aux (device fp32 [3], the gradient of nt_moe_combine_aux's
 * {lb + z, lb, z}) is given. logits are the forward's (bias included); counts its counts.
 * Then grad Wr = grad_logits^T x and grad x += grad_logits Wr are plain GEMMs.
 */
/*
 * Grouped weight gradient (the expert weight gradients of the grouped FFN: autograd of the
 * per-expert MasterLinear products, megatron_moe.py:58-78,145), bf16 MFMA, fp32 accumulation:
 *   c[s, n, m] = sum over rows r of segment s of a[r, n] * b[row(r), m]   (bf16 [S, N, M])
 * row(r) = b_src_row[r] when given (e.g. the gathered token rows), else r. With a = grad_y,
 * b = h this is dW2; with a = grad_fc1, b = x and b_src_row = src_row, dW1. An empty segment's
 * matrix is zero. N and M multiples of 64; lda, ldb multiples of 8.
 */
int nt_moe_grouped_wgrad_bf16(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                              int64_t b_rows, const int32_t* b_src_row,
                              const int32_t* seg_offsets, int32_t num_segments,
                              int64_t total_rows, int32_t N, int32_t M, uint16_t* c,
                              nt_moe_stream_t stream);

/*
 * nt_moe_grouped_wgrad_bf16 with the reduction over each segment's rows split into `splits`
 * chunks (consecutive runs of whole 64-row slabs) that run as separate workgroups, for long
 * segments: the shared expert's weight gradient (one segment of all T rows,
 * megatron_moe.py:133,150) and the router's weight gradient (grad_logits^T x,
 * megatron_moe.py:95-99) would otherwise occupy only a few CUs. The chunks' fp32 sums go to
 * `partial` (fp32 [splits, num_segments, N, M], partial_bytes >= splits * num_segments * N * M
 * * 4; unused when splits == 1) and are added in ascending chunk order -- a fixed order -- into
 * c: fp32 [num_segments, N, M] when c_fp32, else bf16 (rounded once).
 */
int nt_moe_grouped_wgrad_splitk(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                                int64_t b_rows, const int32_t* b_src_row,
                                const int32_t* seg_offsets, int32_t num_segments,
                                int64_t total_rows, int32_t N, int32_t M, int32_t splits,
                                float* partial, size_t partial_bytes, int32_t c_fp32, void* c,
                                nt_moe_stream_t stream);

int nt_moe_router_bwd(const float* logits, const int32_t* topk_ids, const float* topk_w,
                      const float* grad_w, const int32_t* counts, int64_t T, int32_t E,
                      int32_t k, int32_t score_fn, const float* grad_aux, float aux_coeff,
                      float z_coeff, float* grad_logits, nt_moe_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NT_MOE_H */
