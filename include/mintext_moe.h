/*
 * mintext_moe.h -- C-ABI of the MI355X (gfx950) MoE hot path.
 *
 * Every entry point takes plain device pointers, element counts and a HIP stream
 * (passed as void*), enqueues its kernels asynchronously on that stream and returns
 * an MTX_* status code.  No entry point allocates device memory: scratch memory is
 * passed in by the caller as a `workspace` whose size is given by the matching
 * *_workspace_size() query.  All index arrays are int32, all scale arrays float32.
 * Matrices are row-major and dense.
 *
 * Reference interfaces replaced (bzantium/mintext, file:line):
 *   mtx_router_topk        <- MoERouter.__call__ / _group_topk_routing
 *                             (mintext/modules/moe.py:41-103); softmax mode has no
 *                             counterpart in the reference (Mixtral/Qwen3 router)
 *   mtx_router_topk_shared <- the same with MoEBlock's shared expert (moe.py:231-236,256-258)
 *                             folded in as an always-routed extra expert
 *   mtx_gate_router_topk   <- the gate Linear.__call__ (mintext/modules/linear.py:123-147) +
 *                             MoERouter (moe.py:41-103) in one kernel
 *   mtx_router_topk_bwd    <- jax.grad through MoERouter.__call__ (moe.py:52-67,101)
 *   mtx_expert_bias_update <- update_expert_biases (mintext/trainer.py:371-410), one layer
 *   mtx_route              <- route (mintext/kernels/moe_dispatch.py:47-81)
 *   mtx_gather_rows        <- _sort_with_vjp forward (moe_dispatch.py:21-24)
 *   mtx_scatter_rows       <- _sort_with_vjp backward (moe_dispatch.py:33-38)
 *   mtx_invert_permutation <- jnp.argsort(sort_indices) (moe_dispatch.py:102)
 *   mtx_unroute            <- unroute (moe_dispatch.py:84-111); with topk_w == NULL it is
 *                             the route VJP (sum over the K copies, moe_dispatch.py:33-38,67)
 *   mtx_unroute_add        <- unroute + `routed_out + shared_out` (mintext/modules/moe.py:256-258)
 *   mtx_unroute_bwd        <- VJP of unroute (_sort_bwd gather + einsum transpose,
 *                             moe_dispatch.py:33-38,102-111)
 *   mtx_gmm                <- grouped_matmul / _gmm_ragged_dot / _gmm_vjp_fwd
 *                             (mintext/kernels/grouped_matmul.py:58-76,128-148,242-277)
 *   mtx_gmm_swiglu         <- ragged_dot + split + silu*up
 *                             (grouped_matmul.py:143-147; mintext/modules/moe.py:189-196)
 *   mtx_gmm_dlhs           <- _gmm_vjp_bwd dlhs (grouped_matmul.py:162-176)
 *   mtx_tgmm               <- tgmm (grouped_matmul.py:197-235)
 *   mtx_swiglu             <- split + silu*up (mintext/modules/moe.py:195-196)
 *   mtx_swiglu_bwd         <- its autodiff VJP (taken by jax.grad through moe.py:195-196)
 *   mtx_quant_fp8_rows     <- no counterpart (per-tensor analogue: _fp8_matmul,
 *                             mintext/modules/linear.py:37-57); 1x128 activation groups
 *   mtx_route_quant_fp8    <- quantise (no counterpart) + route (moe_dispatch.py:47-81) fused
 *   mtx_quant_fp8_weights  <- no counterpart; 128x128 weight blocks
 *   mtx_gmm_fp8            <- no counterpart; blockwise-fp8 form of mtx_gmm
 *   mtx_gmm_fp8_swiglu     <- no counterpart; blockwise-fp8 form of mtx_gmm_swiglu
 *   mtx_gmm_gathered       <- route's row gather (moe_dispatch.py:67,76) fused into the
 *                             forward GEMMs of MoEExperts._forward_kernel (moe.py:161-196)
 *   mtx_gmm_fp8_swiglu_gathered <- the same for the blockwise-fp8 gate_up GEMM
 *   mtx_quant_fp8_weights_t, mtx_gmm_fp8_dlhs, mtx_quant_fp8_grouped_t, mtx_tgmm_fp8
 *                          <- no counterpart; fp8 forms of the dlhs and tgmm backward
 *                             (grouped_matmul.py:151-187, 197-235)
 *   mtx_transpose_batched  <- _import_expert_weights / _export_expert_weights
 *                             (mintext/checkpoint/conversion.py:80-166), on the device
 */
#ifndef MINTEXT_MOE_H
#define MINTEXT_MOE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------------------- */
#define MTX_OK               0
#define MTX_ERR_ARG         -1   /* invalid shape, dtype or argument combination      */
#define MTX_ERR_WORKSPACE   -2   /* workspace missing or smaller than required        */
#define MTX_ERR_UNSUPPORTED -3   /* valid request that this build does not implement  */
#define MTX_ERR_HIP         -4   /* a HIP runtime call failed (see mtx_last_hip_error) */

/* ---- dtype codes ------------------------------------------------------------------ */
#define MTX_F32      0
#define MTX_BF16     1
#define MTX_FP8E4M3  2   /* OCP float8_e4m3fn (max 448), as jnp.float8_e4m3fn      */

/* ---- router scoring modes ---------------------------------------------------------- */
#define MTX_SCORING_SOFTMAX       0  /* top-k on logits, softmax renormalised over top-k */
#define MTX_SCORING_SIGMOID_GROUP 1  /* sigmoid + bias, group-limited top-k (DeepSeek-V3) */

const char* mtx_status_string(int status);
int         mtx_last_hip_error(void);
/* Library version / capability word; bit 0 = gfx950 code object present. */
int         mtx_version(void);

/* ---- router top-k ------------------------------------------------------------------
 * logits [T,E] (F32 or BF16) -> topk_idx [T,K] int32 (descending by selection value,
 * ties to the lower expert index), topk_w [T,K] float32, scores [T,E] float32 (may be
 * NULL; sigmoid scores in SIGMOID_GROUP mode, softmax probabilities in SOFTMAX mode).
 * SOFTMAX: selection on the logits; w = exp(l-lmax)/sum_topk exp(l-lmax) when
 *   norm_topk_prob, else the full-softmax probability; then * routed_scaling_factor.
 * SIGMOID_GROUP: s = sigmoid(l); r = s + bias (bias may be NULL = zeros); group score =
 *   sum of the top-2 r in each of n_group groups; keep topk_group groups; top-K of r in
 *   the kept groups; w = s[idx]; if norm_topk_prob w /= (sum w + 1e-20); w *= scale.
 * Limits: 1 <= K <= min(E, 64), E <= 1024, E % n_group == 0.                          */
int mtx_router_topk(const void* logits, int logits_dtype, int64_t T, int64_t E, int64_t K,
                    int scoring, const float* bias, int64_t n_group, int64_t topk_group,
                    int norm_topk_prob, float routed_scaling_factor,
                    int32_t* topk_idx, float* topk_w, float* scores, void* stream);

/* As mtx_router_topk, with a shared expert folded in as an always-routed extra expert
 * (MoEBlock's shared expert, mintext/modules/moe.py:231-236,256-258, evaluated inside the
 * routed grouped GEMMs): topk_idx / topk_w are [T,K+1]; columns 0..K-1 as mtx_router_topk,
 * column K = shared_expert (>= E) with weight 1.0, so that the combine adds the shared output
 * last, after the routed sum, as routed_out + shared_out does.                          */
int mtx_router_topk_shared(const void* logits, int logits_dtype, int64_t T, int64_t E, int64_t K,
                           int scoring, const float* bias, int64_t n_group, int64_t topk_group,
                           int norm_topk_prob, float routed_scaling_factor, int64_t shared_expert,
                           int32_t* topk_idx, float* topk_w, float* scores, void* stream);

/* The router gate GEMM fused with mtx_router_topk: logits = x @ W_g (f32 accumulation, one
 * rounding to bf16, as the gate Linear.__call__, mintext/modules/linear.py:123-147, computes
 * them in the compute dtype) and the top-k on those logits, with no [T,E] round trip.
 * x [T,D] bf16, gate_weight_t [E,D] bf16 (the gate kernel [D,E] of moe.py:30-35 transposed
 * once: the nn.Linear layout), both 16-byte aligned; D % 64 == 0, E <= 256 (other shapes and
 * dtypes: MTX_ERR_UNSUPPORTED, use the gate GEMM + mtx_router_topk).  shared_expert: -1, or an
 * id >= E written as column K with weight 1 (as mtx_router_topk_shared; topk_* are then
 * [T,K+1]).  logits_out [T,E] bf16 and scores [T,E] f32 (the router's scores, as
 * mtx_router_topk writes them) may be NULL.  Selection, weights and scores are
 * mtx_router_topk's on the rounded logits, bit for bit.                                  */
int mtx_gate_router_topk(const void* x, int dtype, const void* gate_weight_t, int64_t T, int64_t D,
                         int64_t E, int64_t K, int scoring, const float* bias, int64_t n_group,
                         int64_t topk_group, int norm_topk_prob, float routed_scaling_factor,
                         int64_t shared_expert, int32_t* topk_idx, float* topk_w, void* logits_out,
                         float* scores, void* stream);

/* VJP of mtx_router_topk for fixed indices (what jax.grad takes through MoERouter.__call__,
 * mintext/modules/moe.py:52-67,101: take_along_axis of the scores, the norm and the scaling;
 * the top-k selection and the non-trainable bias carry no gradient).  logits [T,E] (F32/BF16)
 * as passed to the forward, topk_idx [T,idx_ld] its indices (idx_ld = K, or K+1 for the
 * _shared form, whose extra column has a constant weight), d_topk_w [T,K] f32 (may be NULL =
 * zeros), d_scores [T,E] f32 (the gradient of the scores output; may be NULL) -> d_logits
 * [T,E] (F32/BF16).  SOFTMAX with norm_topk_prob: unselected experts get zero gradient from
 * the weights (the renormalised weights depend on the selected logits only).             */
int mtx_router_topk_bwd(const void* logits, int logits_dtype, int64_t T, int64_t E, int64_t K,
                        int scoring, int norm_topk_prob, float routed_scaling_factor,
                        const int32_t* topk_idx, int64_t idx_ld, const float* d_topk_w,
                        const float* d_scores, void* d_logits, int d_logits_dtype, void* stream);

/* Loss-free load balancing for one MoE layer (update_expert_biases, mintext/trainer.py:371-410):
 * bias[e] += rate * sign(float(sum(counts))/E - counts[e]).  expert_counts [E] int32 is the
 * layer's bincount of topk_idx (trainer.py:297-308), i.e. the group_sizes mtx_route returns. */
int mtx_expert_bias_update(const int32_t* expert_counts, int64_t E, float rate, float* bias, void* stream);

/* ---- route (dispatch) ------------------------------------------------------------------
 * tokens [N,D] (F32/BF16/FP8E4M3), topk_idx [N,K] -> sorted_tokens [N*K,D] (same dtype),
 * sort_indices [N*K] (stable argsort of ravel(topk_idx): value = flat position n*K+k),
 * group_sizes [E], and optionally inverse [N*K] (inverse[sort_indices[j]] = j; may be NULL).
 * tokens / sorted_tokens may both be NULL to compute only the permutation.  N == 0 writes
 * only the E zero group sizes (the other buffers may then be NULL).
 * token_scales [N,D/128] f32 (may be NULL) are gathered alongside into sorted_scales.
 * Rows are moved in token order (each token row read once, written to its K positions);
 * with inverse == NULL the inverse permutation is kept in the workspace.
 * Expert ids outside [0,E) are sorted after every valid id and not counted.          */
int64_t mtx_route_workspace_size(int64_t N, int64_t K, int64_t E);
int mtx_route(const void* tokens, int dtype, const int32_t* topk_idx,
              int64_t N, int64_t D, int64_t K, int64_t E,
              void* sorted_tokens, int32_t* sort_indices, int32_t* group_sizes,
              int32_t* inverse, const float* token_scales, float* sorted_scales,
              void* workspace, int64_t workspace_bytes, void* stream);

/* out[j,:] = src[index[j] / div, :]  for j < rows (gather; rows with index outside
 * [0, src_rows*div) are zero-filled).  dtype F32/BF16/FP8E4M3.                         */
int mtx_gather_rows(const void* src, int dtype, int64_t src_rows, int64_t D,
                    const int32_t* index, int64_t rows, int64_t div, void* out, void* stream);

/* out[index[j],:] = src[j,:]  for j < rows (inverse of a permutation gather).          */
int mtx_scatter_rows(const void* src, int dtype, int64_t rows, int64_t D,
                     const int32_t* index, void* out, void* stream);

/* inverse[perm[j]] = j for j < M (entries of perm outside [0,M) are ignored).         */
int mtx_invert_permutation(const int32_t* perm, int64_t M, int32_t* inverse, void* stream);

/* ---- unroute (combine) -------------------------------------------------------------
 * sorted_output [N*K,D] (F32/BF16), inverse [N*K] (from mtx_route or
 * mtx_invert_permutation), topk_w [N,K] (F32/BF16, or NULL = all ones) -> out [N,D]
 * (out_dtype F32/BF16): out[n,:] = sum_k w[n,k] * sorted_output[inverse[n*K+k], :],
 * k ascending, f32 math.                                                              */
int mtx_unroute(const void* sorted_output, int y_dtype, const int32_t* inverse,
                const void* topk_w, int w_dtype, int64_t N, int64_t K, int64_t D,
                void* out, int out_dtype, void* stream);
/* mtx_unroute plus an [N,D] addend (F32/BF16), added in f32 after the k-sum:
 * out = unroute(...) + addend -- `output = routed_out + shared_out` of MoEBlock.__call__
 * (mintext/modules/moe.py:256-258) in the combine's pass (bit-identical to the two steps). */
int mtx_unroute_add(const void* sorted_output, int y_dtype, const int32_t* inverse,
                    const void* topk_w, int w_dtype, int64_t N, int64_t K, int64_t D,
                    const void* addend, int add_dtype, void* out, int out_dtype, void* stream);
/* VJP of mtx_unroute: d_sorted[inverse[n*K+k],:] = w[n,k] * dout[n,:]  (dtype y_dtype),
 * d_w[n,k] = sum_d dout[n,d] * sorted_output[inverse[n*K+k],d]  (dtype w_dtype; may be NULL). */
int mtx_unroute_bwd(const void* dout, int g_dtype, const void* sorted_output, int y_dtype,
                    const int32_t* inverse, const void* topk_w, int w_dtype, int64_t N, int64_t K,
                    int64_t D, void* d_sorted, void* d_w, void* stream);

/* ---- grouped GEMM ----------------------------------------------------------------------
 * Rows of x are grouped contiguously in group_sizes order (a device array that is never
 * read on the host).  Rows past sum(group_sizes) produce zeros.  F32 (exact fp32 FMA) or
 * BF16 (MFMA, f32 accumulate, one rounding).  Output dtype = input dtype.
 * The workspace holds the per-call tile lists and (64 MB) the f32 partial tiles of the
 * split tail: on the 256-row bf16 path, when an XCD's last round of output tiles is at most
 * half full, those tiles are split along the reduction into 2-4 pieces that run on the idle
 * CUs; the last piece to finish adds the pieces in piece order.  Results are deterministic;
 * a split tile's f32 sum is associated differently from a whole tile's, so outputs can differ
 * from the unsplit schedule by a bf16 rounding.  A workspace smaller than the size returned
 * here (but large enough for the tile lists) runs every tile whole.                      */
int64_t mtx_gmm_workspace_size(int64_t M, int64_t E);
/* out[r,:] = x[r,:] @ w[g(r)]       x [M,Kin], w [E,Kin,Kout] -> out [M,Kout]          */
int mtx_gmm(const void* x, const void* w, const int32_t* group_sizes, int dtype,
            int64_t M, int64_t Kin, int64_t Kout, int64_t E, void* out,
            void* workspace, int64_t workspace_bytes, void* stream);
/* h = x @ w[g] (w [E,Kin,2I], gate = first I columns); out = silu(gate) * up  [M,I]   */
int mtx_gmm_swiglu(const void* x, const void* w, const int32_t* group_sizes, int dtype,
                   int64_t M, int64_t Kin, int64_t I, int64_t E, void* out,
                   void* workspace, int64_t workspace_bytes, void* stream);
/* dx[r,:] = g[r,:] @ w[g(r)]^T      g [M,Kout], w [E,Kin,Kout] -> dx [M,Kin]           */
int mtx_gmm_dlhs(const void* g, const void* w, const int32_t* group_sizes, int dtype,
                 int64_t M, int64_t Kin, int64_t Kout, int64_t E, void* dx,
                 void* workspace, int64_t workspace_bytes, void* stream);
/* dw[e] = x[rows_e]^T @ g[rows_e]   x [M,K], g [M,N] -> dw [E,K,N]; empty group -> 0  */
int mtx_tgmm(const void* x, const void* g, const int32_t* group_sizes, int dtype,
             int64_t M, int64_t K, int64_t N, int64_t E, void* dw,
             void* workspace, int64_t workspace_bytes, void* stream);
/* The three GEMMs above with an explicit tile configuration (the `tiling` argument of the
 * Python API and the autotuner's search space; no counterpart in the C form of the reference,
 * which passes TPU tilings to XLA, grouped_matmul.py:58-76 / kernels/autotuner.py:177-310).
 * op: MTX_GMM_OP_FWD (out [M,Kout]), MTX_GMM_OP_SWIGLU (Kout = I, w [E,Kin,2I], out [M,I]),
 * MTX_GMM_OP_DLHS (x = g [M,Kout], out = dx [M,Kin]).  tile_m: 0 (shape heuristic), 128 or 256
 * rows per m-tile of the bf16 MFMA path; tile_group: 0 (heuristic) or 1..64 m-tiles per
 * scheduling group.  The f32 path and shapes outside the MFMA tiling ignore both.  Every
 * configuration computes the same f32 sums; they agree bit for bit unless the split tail
 * (mtx_gmm_workspace_size) splits different tiles, and then to a bf16 rounding.          */
#define MTX_GMM_OP_FWD    0
#define MTX_GMM_OP_SWIGLU 1
#define MTX_GMM_OP_DLHS   2
int mtx_gmm_tiled(int op, const void* x, const void* w, const int32_t* group_sizes, int dtype,
                  int64_t M, int64_t Kin, int64_t Kout, int64_t E, int64_t tile_m, int64_t tile_group,
                  void* out, void* workspace, int64_t workspace_bytes, void* stream);
/* mtx_gmm_tiled without a workspace: no counterpart in the reference.  For callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The tile lists live in a device array of the library (about 280 KB per
 * device, held until the process ends); every tile runs whole (no split tail), so the results
 * equal mtx_gmm_tiled's with a workspace of only the tile lists, bit for bit.  Limits:
 * M <= MTX_GMM_NOALLOC_MAX_ROWS and E <= MTX_GMM_NOALLOC_MAX_EXPERTS, else MTX_ERR_UNSUPPORTED.
 * Calls that overlap on one device (other streams or threads) race on the array: serialise them. */
#define MTX_GMM_NOALLOC_MAX_ROWS    1048576
#define MTX_GMM_NOALLOC_MAX_EXPERTS 1024
int mtx_gmm_tiled_noalloc(int op, const void* x, const void* w, const int32_t* group_sizes, int dtype,
                          int64_t M, int64_t Kin, int64_t Kout, int64_t E, int64_t tile_m,
                          int64_t tile_group, void* out, void* stream);
/* route (moe_dispatch.py:47-81, its row gather) fused into the A operand of the forward GEMMs
 * (MoEExperts._forward_kernel, mintext/modules/moe.py:161-196): x [x_rows,Kin] in token order
 * (BF16), row_index [M] = sort_indices of mtx_route (computed without tokens), index_div = K
 * (top-k): sorted row r is x[row_index[r] / index_div] (indices clamped into x).  op
 * MTX_GMM_OP_FWD or MTX_GMM_OP_SWIGLU, tile_m / tile_group as in mtx_gmm_tiled; results equal
 * mtx_gmm_tiled on the routed rows bit for bit.  Shapes outside the direct-to-LDS kernels
 * (Kin % 64, 16-byte alignment, Kout % 256 / I % 128) return MTX_ERR_UNSUPPORTED.         */
int mtx_gmm_gathered(int op, const void* x, int64_t x_rows, const int32_t* row_index,
                     int64_t index_div, const void* w, const int32_t* group_sizes, int dtype,
                     int64_t M, int64_t Kin, int64_t Kout, int64_t E, int64_t tile_m,
                     int64_t tile_group, void* out, void* workspace, int64_t workspace_bytes,
                     void* stream);
/* out[r,j] = silu(h[r,j]) * h[r,I+j]   h [M,2I] -> out [M,I] (F32/BF16)                */
int mtx_swiglu(const void* h, int dtype, int64_t M, int64_t I, void* out, void* stream);
/* VJP of mtx_swiglu: dh [M,2I] from h [M,2I] and dy [M,I]                              */
int mtx_swiglu_bwd(const void* h, const void* dy, int dtype, int64_t M, int64_t I, void* dh, void* stream);

/* ---- fp8 e4m3fn blockwise ----------------------------------------------------------------
 * Activations: 1x128 groups along the row, scale = amax/448 (1 when amax == 0),
 * q = RNE(x / scale).  Weights: 128x128 blocks over (Kout, Kin), stored k-contiguous
 * w_q [E,Kout,Kin] with w_scale [E,Kout/128,Kin/128] (the per-expert nn.Linear layout).
 * Kin, Kout (and I) must be multiples of 128.  The block scales passed to the GEMMs must be
 * finite and nonzero (the quantisers never produce 0).  mtx_quant_fp8_rows needs x and xq
 * 16-byte aligned (MTX_ERR_ARG otherwise).  Range: the GEMMs (and mtx_tgmm_fp8) carry each
 * accumulator in the units of the current 128-k block's scale product xs*ws, so a block whose
 * scale product is more than about 2^96 / (Kin/128) times smaller than an earlier block's of
 * the same output overflows the accumulator to inf (the true result may be finite).  Real
 * data stays far inside that; the power-of-two mode below has no such limit.              */
int mtx_quant_fp8_rows(const void* x, int dtype, int64_t M, int64_t D,
                       uint8_t* xq, float* x_scale, void* stream);
/* mtx_quant_fp8_rows followed by mtx_route of the codes and scales, in one row pass: tokens
 * [N,D] (F32/BF16, 16-byte aligned, D % 128 == 0) -> sorted_q [N*K,D] e4m3fn (16-byte aligned),
 * sorted_scales [N*K,D/128] f32, sort_indices, group_sizes, inverse (may be NULL) exactly as
 * the two calls produce them (route: mintext/kernels/moe_dispatch.py:47-81).  Workspace:
 * mtx_route_workspace_size.                                                              */
int mtx_route_quant_fp8(const void* tokens, int dtype, const int32_t* topk_idx, int64_t N,
                        int64_t D, int64_t K, int64_t E, uint8_t* sorted_q, float* sorted_scales,
                        int32_t* sort_indices, int32_t* group_sizes, int32_t* inverse,
                        void* workspace, int64_t workspace_bytes, void* stream);
/* w [E,Kin,Kout] (F32/BF16, reference layout) -> w_q [E,Kout,Kin], w_scale [E,Kout/128,Kin/128] */
int mtx_quant_fp8_weights(const void* w, int dtype, int64_t E, int64_t Kin, int64_t Kout,
                          uint8_t* w_q, float* w_scale, void* stream);
/* out [M,Kout] bf16 = sum_kb (xq*xs)(wq*ws) over 128-K blocks, f32 accumulate         */
int mtx_gmm_fp8(const uint8_t* xq, const float* x_scale, const uint8_t* w_q,
                const float* w_scale, const int32_t* group_sizes,
                int64_t M, int64_t Kin, int64_t Kout, int64_t E, void* out,
                void* workspace, int64_t workspace_bytes, void* stream);
/* SwiGLU of the fp8 gate_up GEMM (w_q [E,2I,Kin]) fused with 1x128 re-quantisation:
 * out_q [M,I] e4m3fn + out_scale [M,I/128]; out_bf16 [M,I] optional (may be NULL).    */
int mtx_gmm_fp8_swiglu(const uint8_t* xq, const float* x_scale, const uint8_t* w_q,
                       const float* w_scale, const int32_t* group_sizes,
                       int64_t M, int64_t Kin, int64_t I, int64_t E,
                       uint8_t* out_q, float* out_scale, void* out_bf16,
                       void* workspace, int64_t workspace_bytes, void* stream);
/* mtx_gmm_fp8_swiglu on gathered rows: xq [x_rows,Kin] + x_scale [x_rows,Kin/128] in token
 * order (mtx_quant_fp8_rows of the tokens), sorted row r = token row row_index[r] / index_div
 * (route fused into the A loads, as mtx_gmm_gathered).  Bit-identical to mtx_route_quant_fp8 +
 * mtx_gmm_fp8_swiglu; Kin < 256 returns MTX_ERR_UNSUPPORTED.                               */
int mtx_gmm_fp8_swiglu_gathered(const uint8_t* xq, const float* x_scale, int64_t x_rows,
                                const int32_t* row_index, int64_t index_div, const uint8_t* w_q,
                                const float* w_scale, const int32_t* group_sizes,
                                int64_t M, int64_t Kin, int64_t I, int64_t E,
                                uint8_t* out_q, float* out_scale, void* out_bf16,
                                void* workspace, int64_t workspace_bytes, void* stream);

/* ---- fp8 e4m3fn blockwise, power-of-two scales ("_p2"; no counterpart in the reference, whose
 * fp8 convention is per-tensor scaling, mintext/modules/linear.py:37-57) ----------------------
 * The same layouts and signatures as the entry points above, with every scale the power of two
 * 2^e, e = ceil(log2(amax/448)) clamped to [-126, 127] (1 when amax == 0): the codes are exact
 * quotients x * 2^-e.  The GEMMs hand the scales' exponents (the f32 exponent fields) to the
 * MFMA's E8M0 block-scale operands, so their scales must be powers of two in [2^-126, 2^127]
 * (quantised by the _p2 quantisers); the SwiGLU epilogue re-quantises in the same mode.  The
 * GEMMs need Kin >= 256 (MTX_ERR_UNSUPPORTED otherwise).                                    */
int mtx_quant_fp8_rows_p2(const void* x, int dtype, int64_t M, int64_t D,
                          uint8_t* xq, float* x_scale, void* stream);
int mtx_quant_fp8_weights_p2(const void* w, int dtype, int64_t E, int64_t Kin, int64_t Kout,
                             uint8_t* w_q, float* w_scale, void* stream);
int mtx_gmm_fp8_p2(const uint8_t* xq, const float* x_scale, const uint8_t* w_q,
                   const float* w_scale, const int32_t* group_sizes,
                   int64_t M, int64_t Kin, int64_t Kout, int64_t E, void* out,
                   void* workspace, int64_t workspace_bytes, void* stream);
int mtx_gmm_fp8_swiglu_p2(const uint8_t* xq, const float* x_scale, const uint8_t* w_q,
                          const float* w_scale, const int32_t* group_sizes,
                          int64_t M, int64_t Kin, int64_t I, int64_t E,
                          uint8_t* out_q, float* out_scale, void* out_bf16,
                          void* workspace, int64_t workspace_bytes, void* stream);
int mtx_gmm_fp8_swiglu_gathered_p2(const uint8_t* xq, const float* x_scale, int64_t x_rows,
                                   const int32_t* row_index, int64_t index_div, const uint8_t* w_q,
                                   const float* w_scale, const int32_t* group_sizes,
                                   int64_t M, int64_t Kin, int64_t I, int64_t E,
                                   uint8_t* out_q, float* out_scale, void* out_bf16,
                                   void* workspace, int64_t workspace_bytes, void* stream);

/* ---- fp8 e4m3fn blockwise backward (no reference counterpart; the bf16 forms are dlhs and tgmm,
 * mintext/kernels/grouped_matmul.py:151-187 and :197-235, with the forward's fp8 conventions) ----
 * dlhs: dX = dY @ W^T.  W's codes in its own layout, w_qt [E,Kin,Kout] with the same 128x128 block
 * scales as mtx_quant_fp8_weights transposed, w_scale_t [E,Kin/128,Kout/128]:                     */
int mtx_quant_fp8_weights_t(const void* w, int dtype, int64_t E, int64_t Kin, int64_t Kout,
                            uint8_t* w_qt, float* w_scale_t, void* stream);
/* dx [M,Kin] bf16 = sum_kb (gq*gs)(w_qt*ws_t)^T over 128-Kout blocks: gq [M,Kout] + g_scale
 * [M,Kout/128] from mtx_quant_fp8_rows of dY; Kin % 256 == 0 (else MTX_ERR_UNSUPPORTED).
 * Workspace: mtx_gmm_workspace_size(M,E).                                                         */
int mtx_gmm_fp8_dlhs(const uint8_t* gq, const float* g_scale, const uint8_t* w_qt, const float* w_scale_t,
                     const int32_t* group_sizes, int64_t M, int64_t Kin, int64_t Kout, int64_t E, void* dx,
                     void* workspace, int64_t workspace_bytes, void* stream);
/* tgmm: dW[e] = X_e^T G_e over the rows of group e.  Operands are quantised in expert-aligned
 * chunks of 128 rows (chunk c of group e = its rows 128c..128c+127, zero-padded), transposed:
 * xt [F, 128*C] e4m3fn with C = mtx_fp8_grouped_chunks(M,E) chunk slots, scales [F,C] (blocks = 0:
 * one per feature and chunk) or [F/128,C] (blocks = 1: one per 128x128 block).  F % 128 == 0.
 * Workspace: mtx_fp8_grouped_workspace_size(E).                                                   */
int64_t mtx_fp8_grouped_chunks(int64_t M, int64_t E);
int64_t mtx_fp8_grouped_workspace_size(int64_t E);
int mtx_quant_fp8_grouped_t(const void* x, int dtype, const int32_t* group_sizes, int64_t M, int64_t F,
                            int64_t E, int blocks, uint8_t* xt, float* xt_scale, void* workspace,
                            int64_t workspace_bytes, void* stream);
/* dw [E,F,N] bf16, f32 accumulation: xt/xt_scale of X (blocks = 0), gt/gt_scale of G (blocks = 1),
 * both from mtx_quant_fp8_grouped_t with the same group_sizes and M; an empty group gives zeros.
 * F % 256 == 0 and N % 256 == 0 (else MTX_ERR_UNSUPPORTED).                                       */
int mtx_tgmm_fp8(const uint8_t* xt, const float* xt_scale, const uint8_t* gt, const float* gt_scale,
                 const int32_t* group_sizes, int64_t M, int64_t F, int64_t N, int64_t E, void* dw,
                 void* workspace, int64_t workspace_bytes, void* stream);
/* The backward in the power-of-two mode (the _p2 forward's scales, same layouts and signatures):
 * quantisers with p2_scale instead of amax / 448, GEMMs whose scales go to the MFMA's E8M0
 * operands (so they must be powers of two in [2^-126, 2^127]: the outputs of these quantisers and
 * of mtx_quant_fp8_rows_p2).  The accumulators stay in true units over the whole reduction, so
 * neighbouring chunks of very different magnitude cannot overflow them.                          */
int mtx_quant_fp8_weights_t_p2(const void* w, int dtype, int64_t E, int64_t Kin, int64_t Kout,
                               uint8_t* w_qt, float* w_scale_t, void* stream);
int mtx_gmm_fp8_dlhs_p2(const uint8_t* gq, const float* g_scale, const uint8_t* w_qt, const float* w_scale_t,
                        const int32_t* group_sizes, int64_t M, int64_t Kin, int64_t Kout, int64_t E, void* dx,
                        void* workspace, int64_t workspace_bytes, void* stream);
int mtx_quant_fp8_grouped_t_p2(const void* x, int dtype, const int32_t* group_sizes, int64_t M, int64_t F,
                               int64_t E, int blocks, uint8_t* xt, float* xt_scale, void* workspace,
                               int64_t workspace_bytes, void* stream);
int mtx_tgmm_fp8_p2(const uint8_t* xt, const float* xt_scale, const uint8_t* gt, const float* gt_scale,
                    const int32_t* group_sizes, int64_t M, int64_t F, int64_t N, int64_t E, void* dw,
                    void* workspace, int64_t workspace_bytes, void* stream);

/* ---- expert weight layouts -------------------------------------------------------------
 * Batched transpose-copy (the per-expert HF <-> fused conversions of
 * mintext/checkpoint/conversion.py:80-166, done on the device at load time):
 * out[b*out_batch_stride + c*out_ld + r] = in[b*in_batch_stride + r*in_ld + c] for b < B,
 * r < R, c < C (strides in elements; F32 or BF16).  HF gate [E,I,D] and up [E,I,D] land in the
 * two halves of a fused gate_up [E,D,2I] with out_ld = 2I (up: out offset by I elements);
 * HF down [E,D,I] -> down [E,I,D]; the reverse calls export.  Input and output must not
 * overlap.  B <= 65535 and ceil(R/64) <= 65535.                                          */
int mtx_transpose_batched(const void* in, int dtype, int64_t B, int64_t R, int64_t C,
                          int64_t in_batch_stride, int64_t in_ld, void* out,
                          int64_t out_batch_stride, int64_t out_ld, void* stream);

/* ---- measurement ------------------------------------------------------------------------
 * No counterpart in the reference: the read+write streaming kernel that measures this device's
 * practical HBM ceiling for the dispatch and combine kernels (bench.py --study copy).
 * dst[i] = src[i] for nbytes bytes (nbytes % 16 == 0, both pointers 16-byte aligned, no
 * overlap).  variant: bit 0 = non-temporal loads and stores, bits 4..7 = 16-byte loads in
 * flight per lane (rounded up to 2, 4, 8 or 16; 0 = 8); grid = workgroups of 256 threads
 * (0 = 4 per CU).                                                                            */
int mtx_stream_copy(const void* src, void* dst, int64_t nbytes, int variant, int64_t grid, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* MINTEXT_MOE_H */
