/*
 * C-ABI of the MI355X (gfx950) MoE expert-path kernels.
 *
 * Every entry point takes raw device pointers, element counts, dtype enums
 * and a hipStream_t (passed as void*), enqueues its kernels on that stream and
 * returns a status: TT_OK, or a negative code with a message available from
 * tt_last_error(). Entry points never allocate device memory: buffers (and
 * workspaces, sized by the *_workspace helpers) come from the caller, and no
 * entry point synchronises the host. Integer results (routing ids, row maps,
 * counts) are deterministic; floating-point reductions use a fixed order.
 *
 * Each declaration names the reference interface it replaces (paths relative
 * to the TorchTurbo checkout: src/torchturbo/...).
 */
#ifndef TORCHTURBO_MOE_H
#define TORCHTURBO_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtypes */
enum { TT_F32 = 0, TT_BF16 = 1, TT_F16 = 2, TT_F8E4M3 = 3, TT_F64 = 4 };
/* status codes */
enum { TT_OK = 0, TT_ERR_INVALID = -1, TT_ERR_UNSUPPORTED = -2, TT_ERR_HIP = -3 };
/* router score functions */
enum { TT_SCORE_SOFTMAX = 0, TT_SCORE_SIGMOID = 1, TT_SCORE_SQRTSOFTPLUS = 2 };

/* ABI version of this header; bumped on any signature change. */
int tt_abi_version(void);
/* Message of the last failing call on this host thread ("" if none). */
const char* tt_last_error(void);

/* ---- Router -------------------------------------------------------------
 * Replaces topk_softmax_with_capacity / group_limited_topk
 * (models/modules/moe/utils.py:30-80,127-230), called from
 * TopKRouter.routing (models/modules/moe/router.py:277-356).
 * logits [T, E] (f32/bf16/f16/f64) -> probs [T, E] (logits dtype, zeros
 * except the k selected), routing_map [T, E] (bytes 0/1), top_indices [T, k]
 * int64 in descending-score order (ties: lower expert id first). With f64
 * logits (moe_router_dtype "fp64", router.py:97-100) the top-k of the plain
 * softmax selects on the f64 logits, and the scores, softmax and
 * renormalisation run in fp32 and are widened, as utils.py:181-224 does
 * (softmax(..., dtype=float32), logits.float(), probs.type_as(logits)).
 * expert_bias [E] f32 or NULL (selection only). num_groups/group_topk = 0
 * disable group-limited selection. scaling_factor = 0 means none.
 * fixed_indices [T, k] int64 or NULL: hash routing (ids given).
 * Supports E <= 1024, k <= 64, k <= E. */
int tt_router_topk_fwd(const void* logits, int logits_dtype, int64_t num_tokens,
                       int32_t num_experts, int32_t topk, int32_t score_function,
                       int32_t pre_softmax, const float* expert_bias, int32_t num_groups,
                       int32_t group_topk, float scaling_factor, const int64_t* fixed_indices,
                       void* probs, uint8_t* routing_map, int64_t* top_indices, void* stream);

/* Backward of tt_router_topk_fwd: grad_probs [T, E] (logits dtype) ->
 * grad_logits [T, E] (logits dtype). Autograd of utils.py:175-228. */
int tt_router_topk_bwd(const void* logits, int logits_dtype, int64_t num_tokens,
                       int32_t num_experts, int32_t topk, int32_t score_function,
                       int32_t pre_softmax, float scaling_factor, const int64_t* top_indices,
                       const void* grad_probs, void* grad_logits, void* stream);

/* Gating linear fused with tt_router_topk_fwd. Replaces TopKRouter.gating
 * (models/modules/moe/router.py:25-58,84-101: linear(x.to(rdt), W.to(rdt)))
 * followed by the top-k above, for one MoE layer's router.
 * x [T, hidden] and weight [E, hidden] share in_dtype (bf16/f16); logits
 * [T, E] are written in logits_dtype (f32, or in_dtype) as fp32 sums of the
 * exact 16-bit products rounded once, then routed exactly as
 * tt_router_topk_fwd routes logits of that dtype (same outputs and
 * arguments). E in {32, 64, ..., 256}, hidden a multiple of 64, x and weight
 * 16-byte aligned. The backward is tt_router_topk_bwd plus the two plain
 * GEMMs of the linear. */
int tt_router_gate_fwd(const void* x, const void* weight, int in_dtype, int64_t num_tokens,
                       int64_t hidden, int32_t num_experts, int logits_dtype, int32_t topk,
                       int32_t score_function, int32_t pre_softmax, const float* expert_bias,
                       int32_t num_groups, int32_t group_topk, float scaling_factor,
                       const int64_t* fixed_indices, void* logits, void* probs,
                       uint8_t* routing_map, int64_t* top_indices, void* stream);

/* ---- Router loss statistics (aux load-balancing loss, z-loss) ------------
 * Replaces the [T, E] work of compute_routing_scores_for_aux_loss and
 * z_loss_func (models/modules/moe/moe_utils.py:15-70) as used by
 * TopKRouter._apply_aux_loss / apply_z_loss (router.py:164-270); the scalar
 * formulas on top of these sums stay with the caller. Over tokens t with
 * padding_mask[t] == 0 (padding_mask [T] bytes, or NULL = all valid):
 *   prob_sum [E] f32 = sum_t s_t[e], s_t the bias-free scores (softmax in
 *     fp32; sigmoid or sqrt(softplus) divided by their sum + 1e-20);
 *   tokens_per_expert [E] int64 = tokens whose top-k of s_t holds e (larger
 *     first, lower expert id on equal scores);
 *   z_sum [1] f32 = sum_t r(logsumexp(logits_t)^2), r = rounding to the
 *     logits dtype, logsumexp formed in that dtype step by step as
 *     torch.logsumexp does (max, x - max, exp, sum, log, + max); for f64
 *     logits in fp32 (the reference's fp64 logsumexp to fp32 precision).
 * prob_sum and tokens_per_expert are both NULL (aux off) or both set; z_sum
 * may be NULL (z off). Sums are reproducible (fixed grid, fixed order).
 * Workspace: tt_router_loss_workspace(T, E) bytes. E <= 1024. */
size_t tt_router_loss_workspace(int64_t num_tokens, int32_t num_experts);
int tt_router_loss_fwd(const void* logits, int logits_dtype, int64_t num_tokens,
                       int32_t num_experts, int32_t topk, int32_t score_function,
                       const uint8_t* padding_mask, float* prob_sum, int64_t* tokens_per_expert,
                       float* z_sum, void* workspace, size_t workspace_bytes, void* stream);

/* Backward: grad_logits [T, E] (logits dtype) = d/d logits of
 * sum_e grad_prob_sum[e] * prob_sum[e] + grad_z_sum[0] * z_sum; either grad
 * pointer may be NULL (that term is absent). Padding tokens get zeros. */
int tt_router_loss_bwd(const void* logits, int logits_dtype, int64_t num_tokens,
                       int32_t num_experts, int32_t score_function, const uint8_t* padding_mask,
                       const float* grad_prob_sum, const float* grad_z_sum, void* grad_logits,
                       void* stream);

/* ---- Routing index (counting sort by expert) ----------------------------
 * Replaces the index build of TorchMoEMaskPermutation
 * (ops/providers/native/moe_permutation.py:36-56: masked_select of token ids,
 * masked_scatter_ of packed rows, gather by expert_indices) and the counts of
 * MoEAlltoAllTokenDispatcher.preprocess (models/modules/moe/token_dispatcher.py:125-147).
 * expert_indices [T, k] int64 (k distinct ids in [0, E) per token) ->
 *   row_indices [T, k] int32: packed row of (t, slot j), rows ordered by
 *     expert then token (ops/moe.py:10-46);
 *   token_of_row [T*k] int32: source token of each packed row;
 *   packed_probs [T*k] (probs dtype) = probs_dense[t, e] of each row, if both
 *     pointers are non-NULL;
 *   tokens_per_expert [E] int64.
 * A slot whose id lies outside [0, E), or repeats an id of an earlier slot
 * of the same token, is rejected: it gets row_indices = -1 (which the
 * permute / unpermute kernels skip), no packed row and no count, so the
 * counts then sum to fewer than T*k rows. The call does not synchronise the
 * host; the number of rejected slots is written, as an int32, at byte offset
 * tt_route_index_rejected_offset(T, E) of the workspace, for the caller to
 * read once the stream has reached it. Only expert_indices is read: a
 * routing map that disagrees with it is the caller's error (the reference
 * requires the two to match, ops/dispatcher.py:559-562).
 * Workspace: tt_route_index_workspace(T, E) bytes. */
size_t tt_route_index_workspace(int64_t num_tokens, int32_t num_experts);
size_t tt_route_index_rejected_offset(int64_t num_tokens, int32_t num_experts);
int tt_route_index(const int64_t* expert_indices, int64_t num_tokens, int32_t topk,
                   int32_t num_experts, const void* probs_dense, int probs_dtype,
                   int32_t* row_indices, int32_t* token_of_row, void* packed_probs,
                   int64_t* tokens_per_expert, void* workspace, size_t workspace_bytes,
                   void* stream);

/* tt_route_index without a workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops). No
 * counterpart in the reference. The histograms live in a fixed 1 MiB device
 * array of the library (one per GPU, kept until the process ends), so the
 * call allocates nothing; it rejects problems whose
 * tt_route_index_workspace(T, E) exceeds 1 MiB (e.g. E = 128 up to about
 * 520k tokens) with TT_ERR_INVALID. Outputs are those of tt_route_index; the
 * rejected-slot count goes to *rejected (device int32) when non-NULL. All
 * calls on one GPU share the array: calls that overlap on a GPU (several
 * streams or host threads) race and must be serialised by the caller. */
int tt_route_index_noalloc(const int64_t* expert_indices, int64_t num_tokens, int32_t topk,
                           int32_t num_experts, const void* probs_dense, int probs_dtype,
                           int32_t* row_indices, int32_t* token_of_row, void* packed_probs,
                           int64_t* tokens_per_expert, int32_t* rejected, void* stream);

/* ---- Permute / unpermute -------------------------------------------------
 * Token rows -> packed rows: packed[row_indices[t, j]] = tokens[t].
 * Replaces the index_select of native moe_permutation.py:43 (and TE
 * moe_permute, ops/providers/cuda/moe_permutation.py:77-81); also the
 * backward of unweighted unpermutation. dtype f32/bf16/f16. */
int tt_permute_scatter(const void* tokens, int dtype, int64_t num_tokens, int64_t hidden,
                       int32_t topk, const int32_t* row_indices, void* packed, void* stream);

/* out[t] = sum_j packed[r_j] (* probs[t, expert_indices[t, j]]) over the
 * token's rows r_j in ascending row order, accumulated in fp32 and rounded
 * once to the packed dtype; the weight product is rounded to the promoted
 * dtype first. Replaces TorchMoEMaskUnpermutation
 * (ops/providers/native/moe_permutation.py:68-99) and, with probs == NULL,
 * the index_select backward of the permutation. probs [T, E] or NULL. */
int tt_unpermute_gather(const void* packed, int dtype, int64_t num_tokens, int64_t hidden,
                        int32_t topk, const int32_t* row_indices, const int64_t* expert_indices,
                        const void* probs, int probs_dtype, int32_t num_experts, void* out,
                        void* stream);

/* Backward of weighted tt_unpermute_gather: grad_packed[r_j] =
 * (grad_out[t] * w_j) cast to the packed dtype; grad_probs [T, E] (probs
 * dtype) = sum_h grad_out[t, h] * packed[r_j, h] at (t, expert_j), zero
 * elsewhere. Autograd of moe_permutation.py:90-98. */
int tt_unpermute_gather_bwd(const void* grad_out, const void* packed, int dtype,
                            int64_t num_tokens, int64_t hidden, int32_t topk,
                            const int32_t* row_indices, const int64_t* expert_indices,
                            const void* probs, int probs_dtype, int32_t num_experts,
                            void* grad_packed, void* grad_probs, void* stream);

/* Backward of the packed-probs gather: grad_probs_dense [T, E] =
 * grad_packed_probs[row_indices[t, j]] at (t, expert_indices[t, j]), zero
 * elsewhere (autograd of the masked_select at moe_permutation.py:44-46). */
int tt_packed_probs_bwd(const void* grad_packed_probs, int dtype, int64_t num_tokens,
                        int32_t topk, int32_t num_experts, const int32_t* row_indices,
                        const int64_t* expert_indices, void* grad_probs_dense, void* stream);

/* Chunk reorder: output = concat(input chunk sorted_idxs[0], chunk
 * sorted_idxs[1], ...) for row chunks of sizes split_sizes (device int64
 * [C]); also applied to probs [rows] when both pointers are non-NULL.
 * Replaces TorchMoESortChunks (ops/providers/native/moe_permutation.py:110-126)
 * and TE moe_sort_chunks_by_index (ops/providers/cuda/moe_permutation.py:159-197).
 * C <= 4096. */
int tt_sort_chunks(const void* input, int dtype, int64_t rows, int64_t hidden,
                   const int64_t* split_sizes, const int64_t* sorted_idxs, int32_t num_chunks,
                   const void* probs, int probs_dtype, void* output, void* out_probs,
                   void* stream);

/* ---- SwiGLU and probability weighting ------------------------------------
 * x [rows, 2F] = [gate | up] -> out [rows, F]:
 * a = round(round(silu(gate)) * up); with probs [rows] (non-NULL)
 * out = round(a * p) in the promoted dtype. Replaces native swiglu
 * (ops/providers/native/swiglu.py:10-12) and GroupedMLP.activation_func_with_probs
 * (models/modules/moe/experts.py:181-186). */
int tt_swiglu_fwd(const void* x, int dtype, int64_t rows, int64_t ffn, const void* probs,
                  int probs_dtype, void* out, void* stream);

/* Backward: grad_out [rows, F] -> grad_x [rows, 2F] (x dtype) and, if
 * grad_probs is non-NULL, grad_probs [rows] (probs dtype) = sum_f
 * grad_out * a. */
int tt_swiglu_bwd(const void* x, int dtype, int64_t rows, int64_t ffn, const void* probs,
                  int probs_dtype, const void* grad_out, void* grad_x, void* grad_probs,
                  void* stream);

/* Gated activation with an optional cap, fused with the probability
 * weighting: act = 0 (SiLU) or 1 (GELU, erf form); limit >= 0. limit == 0:
 * a = round(round(act(gate)) * up); limit > 0, in fp32 with one rounding:
 * a = round(act(min(gate, limit)) * clamp(up, -limit, limit)), or with
 * clamp_after != 0 a = round(min(act(gate), limit) * clamp(up, -limit, limit)).
 * Then out = round(a * p) as tt_swiglu_fwd. Replaces native gated_activation
 * (ops/providers/native/gated_activation.py:15-44) as GroupedMLP.glu calls it
 * (models/modules/moe/experts.py:71-84) and the probability product
 * (experts.py:181-186). */
int tt_gated_act_fwd(const void* x, int dtype, int64_t rows, int64_t ffn, int act, float limit,
                     int clamp_after, const void* probs, int probs_dtype, void* out,
                     void* stream);

/* Backward of tt_gated_act_fwd (autograd of the same expression; the caps
 * pass the gradient where their input lies inside the inclusive bounds). */
int tt_gated_act_bwd(const void* x, int dtype, int64_t rows, int64_t ffn, int act, float limit,
                     int clamp_after, const void* probs, int probs_dtype, const void* grad_out,
                     void* grad_x, void* grad_probs, void* stream);

/* ---- Grouped GEMM over expert segments ----------------------------------
 * Rows of x are grouped by expert: expert e owns counts[e] consecutive rows
 * (counts: device int64 [E]; sum(counts) == M). Replaces
 * TorchGroupedMatmul (ops/providers/native/grouped_matmul.py:16-56) and
 * grouped_gemm.ops.gmm (ops/providers/cuda/grouped_matmul.py:34-36).
 * dtype bf16/f16 (MFMA, fp32 accumulation) or f32.
 * Concurrency: every bf16 / f16 weight-gradient launch (tt_gmm_wgrad,
 * tt_gmm_wgrad_gather) keeps per-launch state in one of 64 slots of a
 * per-process device array, taken in turn by successive launches and written
 * on the launch stream before the GEMM kernel runs: the persistent kernel's
 * work queue (at most 512 rows per expert on average, M <= 512 * E, or at
 * least 512 output tiles of 256x256 per expert; tt_gmm_wgrad_persistent), or
 * the one-tile-per-block kernel's expert ranking. At most 64 weight-gradient
 * launches may be in flight at once across all streams of a device; launches
 * on one stream never overlap, so a single stream has no limit. A launch
 * captured into a graph keeps its slot in every replay, so replays of one
 * graph must not overlap each other.
 * fwd:   y[M, N] = x[M, K] @ W[e] with W [E, K, N]; trans_b: W [E, N, K], W[e]^T. */
int tt_gmm_fwd(const void* x, const void* w, int dtype, int64_t m, int64_t k, int64_t n,
               int32_t num_experts, int32_t trans_b, const int64_t* counts, void* y,
               void* stream);
/* dgrad: dx[M, K] = dy[M, N] @ W[e]^T (trans_b: dy @ W[e]). */
int tt_gmm_dgrad(const void* dy, const void* w, int dtype, int64_t m, int64_t k, int64_t n,
                 int32_t num_experts, int32_t trans_b, const int64_t* counts, void* dx,
                 void* stream);
/* wgrad: dW[e] = x_e^T @ dy_e ([E, K, N]); trans_b: dy_e^T @ x_e ([E, N, K]).
 * Experts with no rows get zeros. */
int tt_gmm_wgrad(const void* x, const void* dy, int dtype, int64_t m, int64_t k, int64_t n,
                 int32_t num_experts, int32_t trans_b, const int64_t* counts, void* dw,
                 void* stream);

/* fwd / dgrad with the activation rows gathered: packed row r is row
 * src_of_row[r] of x_src / dy_src ([src_rows, R], R = k for fwd, n for dgrad;
 * src_of_row: device int32 [m], e.g. token_of_row of tt_route_index). One
 * launch replaces a permutation followed by the GEMM (the index_select of
 * ops/providers/native/moe_permutation.py:43 feeding
 * ops/providers/native/grouped_matmul.py:16-56), with no packed copy of the
 * activations; the result equals tt_gmm_fwd / tt_gmm_dgrad on the gathered
 * rows bit for bit. bf16 / f16, R a multiple of 64 above 64, sources under
 * 2 GiB; other problems return TT_ERR_INVALID. A src_of_row entry outside
 * [0, src_rows) (negative included) reads a row of zeros. */
int tt_gmm_fwd_gather(const void* x_src, int64_t src_rows, const int32_t* src_of_row,
                      const void* w, int dtype, int64_t m, int64_t k, int64_t n,
                      int32_t num_experts, int32_t trans_b, const int64_t* counts, void* y,
                      void* stream);
int tt_gmm_dgrad_gather(const void* dy_src, int64_t src_rows, const int32_t* src_of_row,
                        const void* w, int dtype, int64_t m, int64_t k, int64_t n,
                        int32_t num_experts, int32_t trans_b, const int64_t* counts, void* dx,
                        void* stream);
/* wgrad with the rows of x or of dy gathered (exactly one of the two row maps
 * non-NULL; the other operand is packed [m, k] / [m, n]): x_src
 * [x_src_rows, k] or dy_src [dy_src_rows, n]. Equals tt_gmm_wgrad on the
 * gathered rows bit for bit. Long expert reductions only (m > 512 *
 * num_experts, the four-stage kernel), bf16 / f16, a source of fewer than
 * 2^24 rows of fewer than 2^23 elements and under 4 GiB (its row offsets
 * are 24-bit products); other problems return TT_ERR_INVALID. */
int tt_gmm_wgrad_gather(const void* x, int64_t x_src_rows, const int32_t* x_src_of_row,
                        const void* dy, int64_t dy_src_rows, const int32_t* dy_src_of_row,
                        int dtype, int64_t m, int64_t k, int64_t n, int32_t num_experts,
                        int32_t trans_b, const int64_t* counts, void* dw, void* stream);
/* Whether a gathering entry point takes a problem (1) or returns
 * TT_ERR_INVALID for its shape (0), without launching: op 0
 * tt_gmm_fwd_gather (x_src [src_rows, k]), 1 tt_gmm_dgrad_gather (dy_src
 * [src_rows, n]), 2 / 3 tt_gmm_wgrad_gather with the rows of x / of dy
 * gathered. No counterpart in the reference: the layer asks it before taking
 * the folded-permutation path, so shapes the gathering kernels do not cover
 * (e.g. more experts than their LDS schedule holds) keep the permutation. */
int tt_gmm_gather_supported(int32_t op, int dtype, int64_t src_rows, int64_t m, int64_t k,
                            int64_t n, int32_t num_experts);
/* Whether tt_gmm_wgrad runs this shape (bf16 / f16) on its persistent kernel
 * (1) rather than the one-tile-per-block kernel (0), without launching: short
 * reductions (m <= 512 * num_experts) or at least 512 output tiles of 256x256
 * per expert. No counterpart in the reference: it reports the launcher's
 * kernel choice, so that tests and tools can tell which kernel a shape
 * exercises. */
int tt_gmm_wgrad_persistent(int dtype, int64_t m, int64_t k, int64_t n, int32_t num_experts,
                            int32_t trans_b);

/* FP8 e4m3 weights with 128x128 block scales, HF [out, in] orientation:
 * qw [E, N, K] bytes, scale [E, ceil(N/128), ceil(K/128)] (bf16 or f32).
 * Weight element = bf16(f32(q) * f32(scale)), the rule of the reference's
 * offline dequantizer (scripts/dequant/bailing.py:57-102,
 * scripts/dequant/dequantize.py:62-78), applied while staging the operand.
 * fwd: y[M, N] = x[M, K] @ deq(qw[e])^T; dgrad: dx[M, K] = dy[M, N] @ deq(qw[e]).
 * x / dy / y / dx are bf16. */
int tt_gmm_fp8_fwd(const void* x, const uint8_t* qw, const void* scale, int scale_dtype,
                   int64_t m, int64_t k, int64_t n, int32_t num_experts,
                   const int64_t* counts, void* y, void* stream);
int tt_gmm_fp8_dgrad(const void* dy, const uint8_t* qw, const void* scale, int scale_dtype,
                     int64_t m, int64_t k, int64_t n, int32_t num_experts,
                     const int64_t* counts, void* dx, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TORCHTURBO_MOE_H */
