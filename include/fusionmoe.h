/*
 * fusionmoe.h — C ABI of libfusionmoe.so, the gfx950 (MI355X) kernels behind
 * the DeepSeekMoE feed-forward block of FusionLLM.
 *
 * The reference (FusionLLM models/moe.py) has no FFI: its boundary is the
 * nn.Module API of DeepSeekMoE.  Each entry point below replaces one stretch
 * of that module's torch-op sequence; the citation on each names the lines.
 * The host side (fusionllm_amd/moe.py) binds these with ctypes and keeps the
 * reference's module interface (constructor, parameter names, forward,
 * update_gate_bias, get_load_balance_loss, _last_indices/_last_weights).
 *
 * Conventions shared by every entry point
 *   - Plain pointers and sizes only; every device pointer is borrowed.  The
 *     library never allocates or frees device memory: outputs and workspaces
 *     are caller-allocated (sizes from the *_workspace_bytes queries).
 *   - Every call is asynchronous on `stream` (a hipStream_t passed as void*;
 *     NULL is the legacy default stream).  No call synchronises the device.
 *   - Return value: FMOE_OK (0) or a nonzero status; fmoe_status_string()
 *     names it.  Nothing throws or aborts across the ABI.
 *   - Matrices are row-major and densely packed unless a leading dimension
 *     is passed.  bf16 is stored as 16-bit IEEE bfloat16 bit patterns.
 *   - "Rows" of the expert buffers: the routed slots in expert-major,
 *     token-ascending order (rows 0 .. rows_routed-1, rows_routed = T*k),
 *     followed by rows_shared rows for the shared expert (rows_shared = T,
 *     or 0 when the block has no shared expert).  Expert e owns rows
 *     offsets[e] .. offsets[e+1]-1; offsets[] lives in device memory and is
 *     produced by fmoe_dispatch, so no host synchronisation is needed.
 *   - Per-expert weights are passed as HOST arrays of device pointers, one
 *     entry per routed expert followed by one for the shared expert (when
 *     rows_shared > 0).  Each weight is the nn.Linear weight of the
 *     reference: w1, w3 are [inter, dim], w2 is [dim, inter].
 *   - dim and inter must be multiples of 64; n_experts <= FMOE_MAX_EXPERTS.
 *     The four row products (fmoe_gateup_fwd, fmoe_down_fwd, fmoe_down_bwd_dx,
 *     fmoe_gateup_bwd_dx) also need dim, inter < 2^22 and dim * inter < 2^31
 *     (their tile copies form 32-bit byte offsets), else FMOE_ERR_SHAPE.
 */
#ifndef FUSIONMOE_H
#define FUSIONMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FMOE_ABI_VERSION 13
#define FMOE_MAX_EXPERTS 64
#define FMOE_MAX_TOPK 8
#define FMOE_MAX_CAST 64

enum fmoe_status {
  FMOE_OK = 0,
  FMOE_ERR_INVALID_ARG = 1,   /* null pointer or negative size */
  FMOE_ERR_SHAPE = 2,         /* unsupported dimension (not a multiple of 64, k > E, ...) */
  FMOE_ERR_ALIGN = 3,         /* pointer not 16-byte aligned */
  FMOE_ERR_DTYPE = 4,         /* unknown dtype code */
  FMOE_ERR_LAUNCH = 5,        /* hipGetLastError after a launch */
  FMOE_ERR_WORKSPACE = 6,     /* workspace smaller than the size query returned */
  FMOE_ERR_TOO_MANY_EXPERTS = 7,
  FMOE_ERR_SCRATCH = 8        /* workload beyond the static scratch of an allocation-free entry point */
};

enum fmoe_dtype { FMOE_BF16 = 0, FMOE_F32 = 1 };

/* ABI version of the loaded library (FMOE_ABI_VERSION at build time). */
int fmoe_abi_version(void);

/* Static, human-readable text for a status code. */
const char* fmoe_status_string(int status);

/* ---------------------------------------------------------------------------
 * Routing.  Replaces DeepSeekMoE._route (models/moe.py:44-50):
 *   logits = gate(x) (moe.py:46), scores = sigmoid(logits) (:47),
 *   (v, idx) = topk(scores, k) (:48), w = v / (sum(v) + 1e-10) * route_scale (:49).
 * x [T, dim], gate_w [E, dim], gate_b [E] are bf16.  Logits are accumulated
 * in fp32 (products of bf16 operands are exact in fp32) in a fixed order, the
 * score is 1/(1+exp(-logit)), and top-k picks the k largest scores in
 * descending order, ties to the lowest expert index, NaN above every number.
 * Outputs: idx [T,k] int32, idx64 [T,k] int64 (may be NULL; it backs
 * DeepSeekMoE._last_indices, moe.py:83), weights [T,k] fp32 (moe.py:84),
 * topv [T,k] fp32 (the selected scores, kept for the backward pass).
 * ------------------------------------------------------------------------- */
int fmoe_router_fwd(const void* x, const void* gate_w, const void* gate_b,
                    int64_t T, int64_t dim, int n_experts, int k, float route_scale,
                    int32_t* idx, int64_t* idx64, float* weights, float* topv,
                    void* stream);

/* ---------------------------------------------------------------------------
 * Dispatch.  Replaces the permutation half of
 * DeepSeekMoE._dispatch_scatter_gather (models/moe.py:55-64) and the per-expert
 * row gathers x[token_ids] (moe.py:73,75):
 *   expert-count histogram -> exclusive scan -> stable counting-sort scatter
 *   -> gather of x rows into an expert-contiguous buffer.
 * Slot s = t*k + j is token t's j-th choice.  Outputs:
 *   counts [E] int32, offsets [E+1] int32 (exclusive scan of counts),
 *   perm [T*k] int32 (row -> slot, expert-major, slot-ascending; equals
 *   torch.argsort(idx.flatten(), stable=True)),
 *   pos_of_slot [T*k] int32 (slot -> row, the inverse of perm),
 *   x_perm [T*k, dim] bf16 (row r holds x[perm[r] / k]).
 * ------------------------------------------------------------------------- */
size_t fmoe_dispatch_workspace_bytes(int64_t T, int n_experts, int k);
int fmoe_dispatch(const int32_t* idx, const void* x, int64_t T, int64_t dim,
                  int n_experts, int k,
                  int32_t* counts, int32_t* offsets, int32_t* perm,
                  int32_t* pos_of_slot, void* x_perm,
                  void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free fmoe_dispatch.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP-graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * kernels and outputs as fmoe_dispatch, minus the workspace: the scratch is a
 * static 1 MiB array in device memory, one per GPU, held until the process
 * ends.  Workloads with fmoe_dispatch_workspace_bytes(T, E, k) > 1 MiB
 * (2 * ceil(T*k / 256) * E int32, e.g. T*k above 4.2 M slots at E = 8 or
 * 524288 slots at E = 64) return FMOE_ERR_SCRATCH.  The scratch needs no
 * clearing (every call rewrites what it reads).  Calls that overlap on one
 * GPU (on different streams) share the array and race: order them. */
int fmoe_dispatch_noalloc(const int32_t* idx, const void* x, int64_t T, int64_t dim,
                          int n_experts, int k,
                          int32_t* counts, int32_t* offsets, int32_t* perm,
                          int32_t* pos_of_slot, void* x_perm, void* stream);

/* Routing and dispatch of a tiny batch (T <= 16 tokens, decode) in one
 * launch: the outputs of fmoe_router_fwd followed by fmoe_dispatch on its idx,
 * bit for bit, without the round trip between two launches (moe.py:44-64 for
 * one decode step).  No workspace.  T > 16 returns FMOE_ERR_SHAPE (use the two
 * entry points); x_perm may be NULL (no gather). */
int fmoe_route_dispatch(const void* x, const void* gate_w, const void* gate_b,
                        int64_t T, int64_t dim, int n_experts, int k, float route_scale,
                        int32_t* idx, int64_t* idx64, float* weights, float* topv,
                        int32_t* counts, int32_t* offsets, int32_t* perm,
                        int32_t* pos_of_slot, void* x_perm, void* stream);

/* Routing and dispatch of any batch (replaces models/moe.py:44-64: _route,
 * then the flatten / argsort / unique_consecutive / cumsum of
 * _dispatch_scatter_gather and its per-expert gathers x[token_ids]), in three
 * launches instead of five: the router kernel of fmoe_router_fwd also counts
 * each workgroup's choices per expert (the dispatch histogram over blocks of
 * 32 tokens), one workgroup scans the counts, and the stable counting-sort
 * scatter copies each block's rows into x_perm itself.
 * The outputs are those of fmoe_router_fwd followed by fmoe_dispatch on its
 * idx, bit for bit.  counts_host (nullable): E int32 of pinned host memory
 * that also receives the expert counts (the host copy the module reads in
 * its backward, models/moe.py:66-72's skip of experts without tokens),
 * readable once the stream has passed this call.  dim <= 2048; x_perm may be
 * NULL (no gather); workspace: see the query (2 * ceil(T / 32) * E int32).
 * Meant for more than 128 tokens: up to 128, fmoe_router_fwd (one workgroup
 * per token) and fmoe_dispatch (one launch up to 256 slots) are faster. */
size_t fmoe_route_and_dispatch_workspace_bytes(int64_t T, int n_experts, int k);
int fmoe_route_and_dispatch(const void* x, const void* gate_w, const void* gate_b,
                            int64_t T, int64_t dim, int n_experts, int k, float route_scale,
                            int32_t* idx, int64_t* idx64, float* weights, float* topv,
                            int32_t* counts, int32_t* offsets, int32_t* perm,
                            int32_t* pos_of_slot, void* x_perm, int32_t* counts_host,
                            void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Grouped gate/up projection with the SwiGLU product fused in the epilogue.
 * Replaces w1(x), w3(x), F.silu and * of SwiGLUExpert.forward
 * (models/moe.py:21) for every active expert of the loop at moe.py:66-76 and
 * for the shared expert (moe.py:86), as one launch.
 *   a = x_e w1_e^T, b = x_e w3_e^T (bf16-rounded, as nn.Linear returns),
 *   h = bf16(bf16(silu(a)) * b).
 * x_routed: [rows_routed, dim] (x_perm from fmoe_dispatch), or, with gather
 * non-null, the token rows x [gather_tokens, dim]: routed row r then reads
 * x row gather[r] / gather_k (gather = perm from the dispatch; rows_routed
 * >= 8, rows_routed + rows_shared > 4096 (decode-sized launches take x_perm),
 * gather_tokens * dim * 2 < 2^31), so no gathered copy of x is needed
 * (the reference's x[token_ids], moe.py:75); x_shared: [T, dim].
 * Outputs over all rows: ab [rows, 2*inter] (a in columns 0..inter-1, b in
 * inter..2*inter-1; kept for the backward pass), h [rows, inter].
 * workspace: see fmoe_split_workspace_bytes.
 * ------------------------------------------------------------------------- */
int fmoe_gateup_fwd(const void* x_routed, const int32_t* gather, int gather_k,
                    int64_t gather_tokens, const void* x_shared,
                    const int32_t* offsets, int n_experts,
                    int64_t rows_routed, int64_t rows_shared,
                    int64_t dim, int64_t inter,
                    const void* const* w1, const void* const* w3,
                    void* ab, void* h, void* workspace, size_t workspace_bytes,
                    void* stream);

/* Workspace of the four row products (fmoe_gateup_fwd, fmoe_down_fwd,
 * fmoe_down_bwd_dx, fmoe_gateup_bwd_dx) for the current device: fp32
 * partials of the tiles of the last, partial round of the persistent grid,
 * which are split along K (up to 4 ranges), summed in range order
 * (deterministic) and then put through the product's epilogue, with the
 * same rounding points as a whole tile.  Passing no (or a smaller)
 * workspace runs those tiles whole.  Calls that share one workspace must
 * not overlap. */
size_t fmoe_split_workspace_bytes(void);

/* Grouped down projection w2(h) of SwiGLUExpert.forward (models/moe.py:21),
 * all experts plus the shared expert in one launch.  h: [rows, inter];
 * out: [rows, dim] bf16; workspace: see fmoe_split_workspace_bytes. */
int fmoe_down_fwd(const void* h, const int32_t* offsets, int n_experts,
                  int64_t rows_routed, int64_t rows_shared,
                  int64_t dim, int64_t inter, const void* const* w2,
                  void* out, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Weighted combine fused with the shared-expert add.  Replaces
 * y.index_add_(0, token_ids, (expert_out * w).to(fp32)) over the experts in
 * ascending order (models/moe.py:65-76), y.to(x.dtype) (:77) and
 * y_routed + y_shared (:87).  Per token, in fp32 and ascending expert order:
 *   acc = 0; acc = acc + (o_j * w_j)  (product rounded, then the add)
 * then y = out_dtype(acc) + shared (bf16 add for FMOE_BF16; for FMOE_F32 the
 * fp32 sum acc + shared, the autocast case where x is fp32).
 * With a residual (nullable, [T, dim] of out_dtype) the output is the FFN half
 * of FusionLLMBlock.forward, x + ffn(norm2(x)) (models/fusionllm.py:52):
 * y = residual + out_dtype(y_moe), added in out_dtype.
 * Deterministic: token-major gather, no atomics.
 * expert_out: [rows_routed + rows_shared, dim] bf16 (from fmoe_down_fwd).
 * ------------------------------------------------------------------------- */
int fmoe_combine_fwd(const void* expert_out, const int32_t* idx,
                     const float* weights, const int32_t* pos_of_slot,
                     int64_t T, int64_t dim, int k, int64_t rows_routed,
                     int has_shared, int out_dtype, const void* residual,
                     void* y, void* stream);

/* Backward of the combine (autograd of moe.py:76-77,87):
 *   d_expert_out[r] = bf16(dy[t] * w_slot)   for routed row r (slot perm[r]),
 *   d_weights[slot]  = sum_c dy[t,c] * o[r,c]  (fp32).
 * dy: [T, dim] of dy_dtype; d_expert_out: [rows_routed, dim] bf16;
 * d_weights: [T, k] fp32. */
int fmoe_combine_bwd(const void* dy, int dy_dtype, const void* expert_out,
                     const float* weights, const int32_t* perm,
                     int64_t T, int64_t dim, int k,
                     void* d_expert_out, float* d_weights, void* stream);

/* ---------------------------------------------------------------------------
 * Backward of SwiGLUExpert (autograd of models/moe.py:21), grouped like the
 * forward.  The dX products read the nn.Linear weights as they lie
 * (models/moe.py:16-18: w1, w3 [inter, dim], w2 [dim, inter]), one pointer
 * per group (G = routed experts + shared expert), 16-byte aligned.
 * ------------------------------------------------------------------------- */

/* dh = d_out w2 (bf16-rounded), then the SwiGLU backward in the epilogue:
 *   da = bf16(bf16(dh*b) * silu'(a)),  db = bf16(dh * bf16(silu(a))).
 * d_out_routed: [rows_routed, dim]; d_out_shared: [rows_shared, dim];
 * w2[g]: [dim, inter]; ab from fmoe_gateup_fwd; d_ab: [rows, 2*inter];
 * workspace: see fmoe_split_workspace_bytes.
 * Replaces the autograd of self.w2(...) in SwiGLUExpert.forward (models/moe.py:21). */
int fmoe_down_bwd_dx(const void* d_out_routed, const void* d_out_shared,
                     const int32_t* offsets, int n_experts,
                     int64_t rows_routed, int64_t rows_shared,
                     int64_t dim, int64_t inter, const void* const* w2,
                     const void* ab, void* d_ab, void* workspace, size_t workspace_bytes,
                     void* stream);

/* dx_rows = da w1 + db w3 for every row (one product over K = 2*inter);
 * w1[g], w3[g]: [inter, dim]; dx_rows: [rows, dim] bf16;
 * workspace: see fmoe_split_workspace_bytes.
 * Replaces the input-gradient half of the autograd of self.w1(x), self.w3(x)
 * (models/moe.py:21). */
int fmoe_gateup_bwd_dx(const void* d_ab, const int32_t* offsets, int n_experts,
                       int64_t rows_routed, int64_t rows_shared,
                       int64_t dim, int64_t inter, const void* const* w1,
                       const void* const* w3, void* dx_rows, void* workspace,
                       size_t workspace_bytes, void* stream);

/* Grouped weight gradient, the dW half of nn.Linear backward for every expert:
 *   G_e = A_e^T B_e,  A_e = rows of expert e of A ([*, m_out]),
 *                     B_e = the same rows of B ([*, n_out]).
 * Row i < m_split of G_e goes to out_lo[e] ([m_split, n_out]); rows >= m_split
 * go to out_hi[e] ([m_out - m_split, n_out]).  out dtype bf16 or f32; every
 * out_lo[e] / out_hi[e] 16-byte aligned (else FMOE_ERR_ALIGN); m_out <= lda < 2^24,
 * n_out <= ldb < 2^24 (else FMOE_ERR_SHAPE).
 * For w2: A = d_out, B = h, m_split = m_out = dim.  For w1/w3: A = d_ab,
 * B = x, m_split = inter (out_lo = dw1, out_hi = dw3).  With b_gather
 * non-null, b_routed is the token rows x [gather_tokens, n_out] and routed
 * row r of B is x row b_gather[r] / gather_k (gather_tokens * ldb * 2 < 2^31).
 * The reduction over rows is split into fixed chunks summed in chunk order,
 * so the result is deterministic.  Experts with no rows get a zero G_e
 * (the module still reports None for them, as the reference leaves their
 * .grad unset, moe.py:66-72; the graph-capturable operator returns the
 * zeros).  With rows_routed + rows_shared == 0 nothing is written. */
size_t fmoe_weight_grad_workspace_bytes(int64_t rows_routed, int64_t rows_shared,
                                        int n_experts, int64_t m_out, int64_t n_out);
int fmoe_weight_grad(const void* a_routed, const void* a_shared, int64_t lda,
                     const void* b_routed, const void* b_shared, int64_t ldb,
                     const int32_t* b_gather, int gather_k, int64_t gather_tokens,
                     const int32_t* offsets, int n_experts,
                     int64_t rows_routed, int64_t rows_shared,
                     int64_t m_out, int64_t n_out, int64_t m_split,
                     void* const* out_lo, void* const* out_hi, int out_dtype,
                     void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Router backward (autograd of models/moe.py:46-49): normalisation backward,
 * top-k scatter, sigmoid backward, then the gate Linear's weight and bias
 * gradients.  d_logits [T,k] fp32 holds dL/dlogit for each selected expert
 * (the other logits get zero gradient); d_gate_w [E, dim] and d_gate_b [E]
 * are written in grad_dtype.  The reductions over tokens run over the routed
 * rows in expert-contiguous order with a fixed chunking (deterministic); the
 * row r reads token row x[perm[r] / k] ([T, dim] bf16, 16-byte aligned).
 * ------------------------------------------------------------------------- */
size_t fmoe_router_bwd_workspace_bytes(int64_t T, int64_t dim, int n_experts, int k);
int fmoe_router_bwd(const float* d_weights, const float* topv,
                    const int32_t* perm, const int32_t* offsets,
                    const void* x, int64_t T, int64_t dim,
                    int n_experts, int k, float route_scale,
                    float* d_logits, void* d_gate_w, void* d_gate_b,
                    int grad_dtype, void* workspace, size_t workspace_bytes,
                    void* stream);

/* Input gradient of the block: the backward of every use of x in
 * DeepSeekMoE.forward (x[token_ids] at moe.py:75, the gate at :46, the shared
 * expert at :86), summed per token in fp32 in a fixed order:
 *   dx[t] = sum_j dx_rows[pos_of_slot[t*k+j]]  (ascending expert)
 *         + dx_rows[rows_routed + t] (shared, if has_shared)
 *         + sum_j d_logits[t,j] * gate_w[idx[t,j]]
 * written in out_dtype. */
int fmoe_dx_reduce(const void* dx_rows, const int32_t* pos_of_slot,
                   const int32_t* idx, const float* d_logits,
                   const void* gate_w, int64_t T, int64_t dim, int k,
                   int64_t rows_routed, int has_shared, int out_dtype,
                   void* dx, void* stream);

/* ---------------------------------------------------------------------------
 * RMSNorm around the block: FusionLLMBlock's FFN half x + ffn(norm2(x)) with
 * norm2 = nn.RMSNorm(dim, eps=1e-6) (models/fusionllm.py:48,52; torch's
 * F.rms_norm).  dim <= 4096.
 *
 * Forward: r[t] = 1 / sqrt(sum_c x[t,c]^2 / dim + eps) (fp32, correctly
 * rounded sqrt and divide; the sum in a fixed lane order), then
 * xn[t,c] = bf16((x[t,c] * r[t]) * norm_w[c]).  x: [T, dim] of x_dtype;
 * norm_w: [dim] of w_dtype, or NULL for a norm without weight; xn: [T, dim]
 * bf16, the MoE input; rstd: [T] fp32, kept for the backward.
 * ------------------------------------------------------------------------- */
int fmoe_rmsnorm_fwd(const void* x, int x_dtype, const void* norm_w, int w_dtype,
                     int64_t T, int64_t dim, float eps, void* xn, float* rstd,
                     void* stream);

/* Workspace of fmoe_dx_reduce_norm when d_norm_w is wanted: 4160 fp32 rows
 * of dim (4096 per-workgroup partial rows and 64 second-level rows). */
size_t fmoe_norm_bwd_workspace_bytes(int64_t dim);

/* Backward of x + moe(rmsnorm(x)): per token, d_xn as in fmoe_dx_reduce
 * (fp32, not rounded), then
 *   g = d_xn * norm_w,  xh = x * r,
 *   dx = r * (g - xh * (sum_c g*xh) / dim) + d_out      (written in x_dtype)
 * and d_norm_w[c] = sum_t d_xn[t,c] * xh[t,c] (w_dtype), reduced in a fixed
 * order.  d_out and dx have x_dtype; d_norm_w may be NULL (no weight
 * gradient; then the workspace may be NULL too). */
int fmoe_dx_reduce_norm(const void* dx_rows, const int32_t* pos_of_slot,
                        const int32_t* idx, const float* d_logits,
                        const void* gate_w, int64_t T, int64_t dim, int k,
                        int64_t rows_routed, int has_shared,
                        const void* x, const float* rstd, const void* norm_w,
                        int w_dtype, const void* d_out, int x_dtype, void* dx,
                        void* d_norm_w, void* workspace, size_t workspace_bytes,
                        void* stream);

/* ---------------------------------------------------------------------------
 * Fused NorMuon step (training/optimizer.py:11-58, NorMuon.step) for up to 32
 * tensors of one dtype and one step count: exp_avg, exp_avg_sq and the
 * parameter are updated in place, with the reference's operation order and
 * per-operation rounding to the tensor dtype (fp32 arithmetic).  Tensor i is
 * rows[i] x cols[i] (row-major, cols % 4 == 0, cols <= 4096); is_matrix[i]
 * (the parameter has ndim >= 2) enables the per-row RMS normalisation and the
 * cautious weight decay.  The scalars are the reference's Python values:
 * bias_corr1 = 1 - beta1**step, bias_corr2 = 1 - beta2**step.  Host arrays;
 * grads are read-only.  Deterministic (one wave per row, fixed-order row
 * sums).
 * ------------------------------------------------------------------------- */
int fmoe_normuon_step(void* const* params, const void* const* grads,
                      void* const* exp_avgs, void* const* exp_avg_sqs,
                      const int64_t* rows, const int64_t* cols,
                      const int* is_matrix, int n_tensors, int dtype,
                      double lr, double beta1, double beta2, double eps,
                      double weight_decay, int cautious, double bias_corr1,
                      double bias_corr2, void* stream);

/* ---------------------------------------------------------------------------
 * bf16 copies of up to FMOE_MAX_CAST fp32 tensors in one launch.  Under the
 * trainer's bf16 autocast (training/trainer.py:158) each nn.Linear of the
 * block casts its fp32 weight to bf16 (models/moe.py:16-18, the gate at
 * moe.py:36,46), one cast per weight; this replaces those casts (and the
 * input's) for the whole block.  dst[i] = bf16(src[i]) for n[i] elements,
 * round to nearest even as torch's .to(torch.bfloat16); src and dst 16-byte
 * aligned, contiguous.
 * ------------------------------------------------------------------------- */
int fmoe_cast_bf16(const void* const* src, void* const* dst, const int64_t* n,
                   int n_tensors, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FUSIONMOE_H */
