/*
 * moe_mi355x.h — C ABI of the MI355X (gfx950) Qwen3-MoE expert path.
 *
 * Every entry point takes raw device pointers, int64 sizes and a HIP stream
 * (passed as void*, it is a hipStream_t; NULL means the legacy default
 * stream).  All launches are asynchronous on that stream; no entry point
 * synchronises, allocates device memory or reads device memory on the host.
 * Outputs and workspaces are owned by the caller.
 *
 * Element types: "bf16" buffers hold IEEE bfloat16 as uint16; "f32" is IEEE
 * float; indices are int64 where the reference exposes torch.long tensors and
 * int32 for internal permutation maps.  Device pointers must be 16-byte
 * aligned and row strides (in elements) multiples of 8.  A buffer of zero
 * elements (no tokens or no routed rows, as on an EP rank that receives
 * none) may be NULL; the entry point then does nothing, except that weight
 * gradients are still written (zeros) or, when accumulating, left as they
 * are.
 *
 * Return value: MOE_OK (0) or a negative MOE_ERR_* status; moe_last_error()
 * gives a message for the last failure on the calling thread.
 *
 * Reference interfaces (paths relative to the reference checkout, "TF/" is the
 * transformers package the reference pins, installed here as 5.15.0):
 *   router     TF/models/qwen3_moe/modeling_qwen3_moe.py:249-267
 *   experts    TF/integrations/moe.py:377-478 (grouped_mm_experts_forward)
 *   aux loss   TF/models/qwen3_moe/modeling_qwen3_moe.py:514-593,
 *              parallel/parallel/engine/model_parallel/sequence_parallel.py:239-280
 *   dispatch   parallel/parallel/engine/model_parallel/token_dispatch.py:78-174
 *   FSDP grads parallel/parallel/engine/_dp_param_unit.py:268-277,395-417
 */
#ifndef MOE_MI355X_H
#define MOE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_OK 0
#define MOE_ERR_INVALID (-1)     /* bad argument: null pointer, negative size, misalignment */
#define MOE_ERR_UNSUPPORTED (-2) /* shape outside what the kernels handle */
#define MOE_ERR_LAUNCH (-3)      /* hipLaunchKernel / HIP runtime failure */
#define MOE_ERR_WORKSPACE (-4)   /* workspace smaller than *_workspace_bytes() */

/* Message for the last non-zero status returned on this thread. */
const char* moe_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int moe_abi_version(void);

/* ------------------------------------------------------------------ router */

/* logits[T,E] (f32) = x[T,H] (bf16) · wr[E,H]ᵀ (bf16), fp32 accumulation.
 * Replaces F.linear in Qwen3MoeTopKRouter.forward
 * (TF/models/qwen3_moe/modeling_qwen3_moe.py:260) computed as
 * x.float() @ wr.float().T. */
int moe_router_logits_fwd(const void* x, const void* wr, float* logits,
                          int64_t T, int64_t H, int64_t E, void* stream);

/* Fused router forward: logits = x · wrᵀ (+ logit_bias[E] when not NULL, f32),
 * then the top-k softmax of moe_router_topk_fwd.  For E <= 128 (a multiple
 * of 16) one kernel runs the GEMM, the reduction and the selection (no
 * workspace: the size query returns 0); otherwise the GEMM is split along H
 * into f32 partials held in the workspace and a second kernel reduces them
 * and selects.  With logits_bf16 (bf16 [T,E], may be NULL) the logits are
 * those of a bf16 linear, as the reference computes them under bf16 autocast
 * (parallel/parallel/engine/engine.py:141): rounded to bf16 before the
 * softmax, written there as bf16 and to `logits` as the same values in f32,
 * and the scores are rounded to bf16 (the reference's cast to the logits'
 * dtype, modeling_qwen3_moe.py:266).  Replaces Qwen3MoeTopKRouter.forward
 * (TF/models/qwen3_moe/modeling_qwen3_moe.py:258-267); the reference router
 * has no bias (the imbalanced benchmark configuration adds one). */
size_t moe_router_fwd_workspace_bytes(int64_t T, int64_t H, int64_t E);
int moe_router_fwd(const void* x, const void* wr, const float* logit_bias,
                   float* logits, void* logits_bf16, float* scores,
                   int64_t* indices, int64_t T, int64_t H, int64_t E, int64_t k,
                   int norm_topk_prob, void* workspace, size_t workspace_bytes,
                   void* stream);

/* Per token: p = softmax(logits) in fp32; indices = the k largest, sorted
 * descending (ties: lower expert index first); scores = p[indices],
 * divided by their sum when norm_topk_prob != 0.
 * Replaces softmax/topk/renorm of TF/models/qwen3_moe/modeling_qwen3_moe.py:261-265.
 * 1 <= k <= min(E, 16), E <= 1024. */
int moe_router_topk_fwd(const float* logits, float* scores, int64_t* indices,
                        int64_t T, int64_t E, int64_t k, int norm_topk_prob,
                        void* stream);

/* Backward of moe_router_topk_fwd: d_logits[T,E] from d_scores[T,k].
 * Writes (or, with accumulate != 0, adds into) f32 d_logits; also writes
 * a bf16 copy of the result to d_logits_bf16 when it is not NULL.
 * Autograd of TF/models/qwen3_moe/modeling_qwen3_moe.py:261-265. */
int moe_router_topk_bwd(const float* logits, const int64_t* indices,
                        const float* d_scores, int64_t T, int64_t E, int64_t k,
                        int norm_topk_prob, float* d_logits, int accumulate,
                        void* d_logits_bf16, void* stream);

/* moe_router_topk_bwd for a caller that only needs the bf16 d_logits (the
 * router GEMMs' input): d_logits_bf16 = bf16(g + d_add) with g the top-k /
 * softmax backward and d_add an optional f32 [T,E] gradient that reaches the
 * logits by another path (the aux loss's); d_add is only read, so the
 * caller's tensor need not be copied.  Same reference as moe_router_topk_bwd. */
int moe_router_topk_bwd_bf16(const float* logits, const int64_t* indices,
                             const float* d_scores, const float* d_add,
                             int64_t T, int64_t E, int64_t k,
                             int norm_topk_prob, void* d_logits_bf16,
                             void* stream);

/* Backward of the router top-k for bf16 router logits (the reference's
 * F.linear under bf16 autocast, parallel/parallel/engine/engine.py:141,
 * TF/models/qwen3_moe/modeling_qwen3_moe.py:260-265): logits[T,E] holds the
 * f32 values of the bf16 logits and d_logits (may be NULL) the values of
 * their incoming bf16 gradient [T,E] as f32.  With stats and d_aux (both or
 * neither; token_weight may be NULL) the aux loss's logits gradient of
 * moe_aux_loss_bwd over those logits is formed in the same pass (the aux loss
 * of load_balancing_loss_func, :514-593, on the bf16 logits).  As autograd
 * sums a bf16 tensor's gradients in bf16, each term is rounded to bf16 and
 * every sum again: d_logits_bf16 = bf16(bf16(g) + bf16(bf16(aux) + d_logits)),
 * g being the f32 softmax / top-k / renorm backward of d_scores rounded to
 * bf16 (the scores of bf16 logits are bf16, :266, and so is their gradient). */
int moe_router_bf16_logits_bwd(const float* logits, const int64_t* indices,
                               const float* d_scores, const float* d_logits,
                               const float* token_weight, const float* stats,
                               const float* d_aux, int64_t T, int64_t E,
                               int64_t k, int norm_topk_prob,
                               void* d_logits_bf16, void* stream);

/* moe_router_topk_bwd_bf16 with the aux loss's logits gradient (that of
 * moe_aux_loss_bwd for token_weight, stats and d_aux[1], which are what
 * moe_router_aux_fwd returned and the loss's incoming gradient) computed in
 * the same pass: d_logits_bf16 = bf16(g + (d_add + aux term)), bit for bit
 * moe_aux_loss_bwd's f32 output passed as d_add (added after the caller's
 * d_add, which may be NULL).  Autograd of modeling_qwen3_moe.py:261-265 and
 * of load_balancing_loss_func (:514-593) at the router logits. */
int moe_router_aux_bwd_bf16(const float* logits, const int64_t* indices,
                            const float* d_scores, const float* d_add,
                            const float* token_weight, const float* stats,
                            const float* d_aux, int64_t T, int64_t E,
                            int64_t k, int norm_topk_prob, void* d_logits_bf16,
                            void* stream);

/* Backward of the router GEMM (F.linear, modeling_qwen3_moe.py:260) from
 * bf16 d_logits[T,E]: dx[T,H] = d_logits · wr (bf16) and dwr[E,H] =
 * d_logitsᵀ · x (bf16, reduced in f32 over token chunks held in the
 * workspace, always in chunk order; for E <= 128 a multiple of 32 and H a
 * multiple of 32 one kernel forms dx and the chunks' partials together).
 * With dwr_accumulate, dwr holds an existing bf16 gradient and receives
 * bf16(dwr + bf16(d_logitsᵀ · x)), torch's accumulation of the fresh gradient
 * (parallel/parallel/engine/engine.py:165-178). */
size_t moe_router_logits_bwd_workspace_bytes(int64_t T, int64_t H, int64_t E);
int moe_router_logits_bwd(const void* d_logits_bf16, const void* x,
                          const void* wr, void* dx, void* dwr,
                          int dwr_accumulate, int64_t T, int64_t H, int64_t E,
                          void* workspace, size_t workspace_bytes,
                          void* stream);

/* ---------------------------------------------------------------- aux loss */

/* Switch load-balancing loss over logits[T,E] (f32):
 *   p = softmax(logits); sel = topk(p, k);
 *   W = sum_t w_t (w_t = token_weight[t], or 1 when token_weight is NULL);
 *   c_e = sum_t w_t * #{j : sel[t,j] == e};  P_e = sum_t w_t * p[t,e];
 *   aux = E * sum_e (c_e / W) * (P_e / W).
 * Writes aux[0] and stats[E+1] = (c_0..c_{E-1}, W) for the backward.
 * Replaces load_balancing_loss_func (TF/models/qwen3_moe/modeling_qwen3_moe.py:514-593)
 * and, on one rank, sequence_parallel_load_balancing_loss
 * (parallel/parallel/engine/model_parallel/sequence_parallel.py:239-280).
 * Deterministic (fixed-order reductions, no atomics). */
size_t moe_aux_loss_workspace_bytes(int64_t T, int64_t E);
int moe_aux_loss_fwd(const float* logits, const float* token_weight, int64_t T,
                     int64_t E, int64_t k, float* aux, float* stats,
                     void* workspace, size_t workspace_bytes, void* stream);

/* d_logits[t,e] (+)= p_te * (g_te - sum_e' p_te' g_te'),
 * g_te = d_aux[0] * E * w_t * c_e / W^2  (d_aux is a device scalar). */
int moe_aux_loss_bwd(const float* logits, const float* token_weight,
                     const float* stats, const float* d_aux, int64_t T,
                     int64_t E, float* d_logits, int accumulate, void* stream);

/* ------------------------------------- the step before: norm -> router -> aux */

/* RMSNorm of the MoE block's input (post_attention_layernorm), per row:
 *   r = rsqrt(mean(h^2) + eps) in fp32;  x = bf16(gamma * bf16(h * r));  rstd[t] = r.
 * h, gamma, x bf16 (16-byte aligned); H a multiple of 8, H <= 4096.
 * Replaces Qwen3MoeRMSNorm.forward (TF/models/qwen3_moe/modeling_qwen3_moe.py:294-299)
 * as applied before the MoE block (:345). */
int moe_rmsnorm_fwd(const void* h, const void* gamma, int64_t T, int64_t H,
                    float eps, void* x, float* rstd, void* stream);

/* Backward of moe_rmsnorm_fwd (autograd of :294-299): with g = bf16(dx + dx2)
 * (dx2 may be NULL; autograd adds the router's and the experts' gradients of
 * x in bf16), dhs = bf16(g * gamma):
 *   dh = bf16(r * dhs - (r^3 / H) * h * sum_j dhs_j h_j),
 *   dgamma = bf16(sum_t bf16(g * bf16(h * r)))  (fixed-order column sums). */
size_t moe_rmsnorm_bwd_workspace_bytes(int64_t T, int64_t H);
int moe_rmsnorm_bwd(const void* dx, const void* dx2, const void* h,
                    const void* gamma, const float* rstd, int64_t T, int64_t H,
                    void* dh, void* dgamma, void* workspace,
                    size_t workspace_bytes, void* stream);

/* moe_router_fwd plus the Switch aux loss of moe_aux_loss_fwd (same aux and
 * stats outputs, token_weight as there) from the router's own softmax and
 * top-k, where the reference recomputes both from the logits
 * (TF/models/qwen3_moe/modeling_qwen3_moe.py:550-552 inside load_balancing_loss_func
 * :514-593).  T >= 1. */
size_t moe_router_aux_fwd_workspace_bytes(int64_t T, int64_t H, int64_t E);
int moe_router_aux_fwd(const void* x, const void* wr, const float* logit_bias,
                       const float* token_weight, float* logits,
                       void* logits_bf16, float* scores, int64_t* indices,
                       int64_t T, int64_t H, int64_t E, int64_t k,
                       int norm_topk_prob, float* aux, float* stats,
                       void* workspace, size_t workspace_bytes, void* stream);

/* ----------------------------------------------------------------- permute */

/* Stable counting sort of S = T*k routed slots by bucket = ids[s] / divisor
 * (floor division).  Slots whose id is negative or whose bucket is >=
 * num_buckets are sentinels: they sort after every real bucket and are
 * excluded from counts.
 * Outputs (int32):
 *   perm[S]        sorted position -> slot index s = t*k + j
 *   pos_of_slot[S] slot index -> sorted position (inverse of perm)
 *   counts[nb]     slots per bucket (the send splits when bucket = owner rank)
 *   offsets[nb]    inclusive cumsum of counts (offsets[nb-1] = valid rows)
 * and, when permuted is not NULL, permuted[pos,:] = hidden[perm[pos]/k,:] for
 * valid rows and zero for sentinel rows (bf16 rows of width H).
 * Replaces torch.sort/gather/histc/cumsum of TF/integrations/moe.py:389-437
 * (divisor 1, buckets = local experts, sentinel = num_experts) and the
 * argsort/bincount/index_select of TokenDispatcher.dispatch,
 * parallel/parallel/engine/model_parallel/token_dispatch.py:86-123
 * (divisor = local expert count, buckets = EP ranks).
 * num_buckets <= 1024. */
size_t moe_permute_workspace_bytes(int64_t S, int64_t num_buckets);
int moe_permute_fwd(const void* hidden, int64_t T, int64_t H,
                    const int64_t* ids, int64_t k, int64_t divisor,
                    int64_t num_buckets, void* permuted, int32_t* perm,
                    int32_t* pos_of_slot, int32_t* counts, int32_t* offsets,
                    void* workspace, size_t workspace_bytes, void* stream);

/* moe_permute_fwd without a workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  It has no counterpart in the
 * reference.  The histogram lives in a fixed 1 MiB device array per GPU
 * (held until the process ends), so S = T*k routes over num_buckets buckets
 * must satisfy moe_permute_workspace_bytes(S, num_buckets) <= 1 MiB (about a
 * million routes at 128 buckets); larger sizes return MOE_ERR_UNSUPPORTED
 * before any launch.  Calls no hipMalloc or other allocating routine.  Every
 * call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (different streams, threads or graph replays in flight together) race.
 * Make the first call on each device outside graph capture: it looks up the
 * array's device address (hipGetSymbolAddress), which may load the library's
 * code onto that device.  Later calls may be captured and replayed.
 * Outputs and semantics are those of moe_permute_fwd, bit for bit. */
int moe_permute_fwd_noalloc(const void* hidden, int64_t T, int64_t H,
                            const int64_t* ids, int64_t k, int64_t divisor,
                            int64_t num_buckets, void* permuted, int32_t* perm,
                            int32_t* pos_of_slot, int32_t* counts,
                            int32_t* offsets, void* stream);

/* Per sorted position: local_ids[pos] = ids[perm[pos]] - bucket*divisor,
 * routed_scores[pos] = scores[perm[pos]] and source_tokens[pos] =
 * perm[pos] / k, the token of the slot (any output may be NULL).  Replaces
 * send_experts/send_scores of token_dispatch.py:124-125 and the sorted
 * source_tokens of :106-118. */
int moe_dispatch_meta(const int64_t* ids, const float* scores,
                      const int32_t* perm, int64_t S, int64_t divisor,
                      int64_t k, int64_t* local_ids, float* routed_scores,
                      int64_t* source_tokens, void* stream);

/* Backward of the row gather: d_hidden[t,:] = sum_j d_permuted[pos_of_slot[t*k+j],:]
 * over valid positions (pos < offsets[nb-1]), fp32 accumulation, plus
 * d_add[t,:] when d_add is not NULL; bf16 in and out.
 * Autograd of hidden_states[perm // k] (TF/integrations/moe.py:394) and of
 * hidden_states.index_select (token_dispatch.py:123). */
int moe_permute_bwd(const void* d_permuted, const int32_t* pos_of_slot,
                    const int32_t* offsets, int64_t num_buckets, int64_t T,
                    int64_t H, int64_t k, const void* d_add, void* d_hidden,
                    void* stream);

/* ----------------------------------------------------------------- combine */

/* out[t,:] = sum_j s[t*k+j] * y[pos_of_slot[t*k+j],:] over valid positions,
 * fp32 accumulation, bf16 out; s = 1 when scores is NULL.
 * Replaces the weight/mask/inverse-permute/sum of TF/integrations/moe.py:461-478
 * and, with scores NULL, the index_add of TokenDispatcher.combine
 * (token_dispatch.py:169-174). */
int moe_combine_fwd(const void* y, const int32_t* pos_of_slot,
                    const int32_t* offsets, int64_t num_buckets,
                    const float* scores, int64_t T, int64_t H, int64_t k,
                    void* out, void* stream);

/* Backward of moe_combine_fwd: d_y[pos,:] = s * d_out[t,:] (bf16) for valid
 * positions, zero for sentinel rows; d_scores[t*k+j] = <y[pos,:], d_out[t,:]>
 * (fp32, 0 for sentinels) when d_scores is not NULL. */
int moe_combine_bwd(const void* d_out, const void* y,
                    const int32_t* pos_of_slot, const int32_t* offsets,
                    int64_t num_buckets, const float* scores, int64_t T,
                    int64_t H, int64_t k, void* d_y, float* d_scores,
                    void* stream);

/* moe_combine_bwd followed, token by token in the same launch, by the
 * router's top-k backward on the routing weights' gradient it forms (the
 * gradient of the router's scores in the one-op block, where nothing else
 * uses them): d_logits_bf16[T,E] is what moe_router_topk_bwd_bf16
 * (stats and d_aux NULL, bf16_terms 0), moe_router_aux_bwd_bf16 (bf16_terms
 * 0) or moe_router_bf16_logits_bwd (bf16_terms 1) gives on that d_scores,
 * bit for bit, with d_logits the incoming logits gradient (may be NULL);
 * d_scores (may be NULL) receives the weights' gradient as moe_combine_bwd
 * writes it.  logits fp32 [T,E], indices [T,k] int64 as the router wrote
 * them.  Fuses the autograd of TF/integrations/moe.py:461-478 with that of
 * TF/models/qwen3_moe/modeling_qwen3_moe.py:258-267 (and :514-593 with
 * stats/d_aux). */
int moe_combine_router_bwd(const void* d_out, const void* y,
                           const int32_t* pos_of_slot, const int32_t* offsets,
                           int64_t num_buckets, const float* scores, int64_t T,
                           int64_t H, int64_t k, void* d_y, float* d_scores,
                           const float* logits, const int64_t* indices,
                           const float* d_logits, const float* token_weight,
                           const float* stats, const float* d_aux, int64_t E,
                           int norm_topk_prob, int bf16_terms,
                           void* d_logits_bf16, void* stream);

/* ------------------------------------------------------------ grouped GEMM */
/* Groups partition the rows of the activation operand: group g owns rows
 * [offs[g-1], offs[g]) (offs[-1] = 0; offs is the inclusive int32 cumsum,
 * the F.grouped_mm `offs` convention of TF/integrations/moe.py:403).  Rows at
 * or beyond offs[G-1] are not touched.  offs may be NULL for a single group
 * of M rows (G must then be 1).  No host synchronisation: tiles are mapped to
 * groups on the device. */

/* act[M,I] = silu(gate) * up, pre[M,2I] = (gate | up), where
 * (gate | up)[r,:] = xp[r,:] · w_gate_up[g]ᵀ, w_gate_up [G,2I,H] (first I rows
 * are the gate).  Replaces F.grouped_mm up (TF/integrations/moe.py:440-442)
 * plus _default_apply_gate (:509-521).  pre may be NULL. */
int moe_grouped_gemm_swiglu_fwd(const void* xp, const void* w_gate_up,
                                const int32_t* offs, int64_t G, int64_t M,
                                int64_t H, int64_t I, void* act, void* pre,
                                void* stream);

/* c[M,N] = a[M,K] · w[g]ᵀ with w [G,N,K].  Replaces F.grouped_mm down
 * (TF/integrations/moe.py:456-459). */
int moe_grouped_gemm_fwd(const void* a, const void* w, const int32_t* offs,
                         int64_t G, int64_t M, int64_t N, int64_t K, void* c,
                         void* stream);

/* da[M,K] = dc[M,N] · w[g] with w [G,N,K] (input gradient of
 * moe_grouped_gemm_fwd; autograd formula restated at TF/integrations/moe.py:236). */
int moe_grouped_gemm_dgrad(const void* dc, const void* w, const int32_t* offs,
                           int64_t G, int64_t M, int64_t N, int64_t K,
                           void* da, void* stream);

/* d_act[M,I] = dy[M,H] · w_down[g] (w_down [G,H,I]) fused with the SwiGLU
 * backward against the saved pre[M,2I]: writes d_pre[M,2I] = (d_gate | d_up)
 * for the rows of the groups; rows at or beyond offs[G-1] are neither read
 * nor written. */
int moe_grouped_gemm_dgrad_swiglu_bwd(const void* dy, const void* w_down,
                                      const void* pre, const int32_t* offs,
                                      int64_t G, int64_t M, int64_t H,
                                      int64_t I, void* d_pre, void* stream);

/* dw[g] [N,K] (+)= dc[rows of g, N]ᵀ · a[rows of g, K] (weight gradient of
 * moe_grouped_gemm_fwd; TF/integrations/moe.py:237).  Empty groups get zeros
 * (accumulate == 0) or are left untouched (accumulate != 0).
 * dw_is_f32 selects an f32 instead of a bf16 dw buffer. */
int moe_grouped_gemm_wgrad(const void* dc, const void* a, const int32_t* offs,
                           int64_t G, int64_t M, int64_t N, int64_t K,
                           void* dw, int dw_is_f32, int accumulate,
                           void* stream);

/* moe_grouped_gemm_wgrad with group g's [N,K] block written into an FSDP
 * unit's rank-major gradient bucket instead of a dense [G,N,K] tensor: at
 * element (g / bucket_rows) * bucket_stride + (g % bucket_rows) * N * K from
 * `bucket`.  This replaces the copy of a parameter's full gradient into the
 * reduce-scatter input in DPParamUnit.start_gradient_reduction
 * (parallel/parallel/engine/_dp_param_unit.py:395-417): `bucket` points at the
 * parameter's bucket_offset in rank 0's chunk, bucket_rows is its padded
 * rows per rank, ceil(G / world_size) (:200), and bucket_stride the unit's
 * bucket_numel (:268-277).  Padding rows are not written (the reference
 * zero-fills the bucket); bucket_stride must keep rank chunks 16-byte aligned. */
int moe_grouped_gemm_wgrad_bucket(const void* dc, const void* a,
                                  const int32_t* offs, int64_t G, int64_t M,
                                  int64_t N, int64_t K, void* bucket,
                                  int64_t bucket_rows, int64_t bucket_stride,
                                  int dw_is_f32, int accumulate, void* stream);

/* ------------------------------------------------------ the fp32 expert path */

/* The reference's grouped experts accept fp32 modules and then compute in
 * fp32 (TF/integrations/moe.py:377-478).  These entry points run that path
 * with fp32 operands and arithmetic; the row permutation is moe_permute_fwd
 * over each row's bytes (H fp32 = 2H bf16-sized units).  They serve small
 * fp32 layers (the C1 configuration), not the tuned bf16 step.
 *
 * Grouped GEMM: C(i, j) = sum_r A(i, r) B(r, j) (+ C(i, j) with accumulate),
 * A(i, r) = A[i sAi + r sAr], B(r, j) = B[r sBr + j sBj], C(i, j) =
 * C[i sCi + j sCj], on v_mfma_f32_32x32x2_f32.
 *   mode 0 (projections, input gradients): output rows i in [0, M) are
 *     grouped by the inclusive offsets offs[G] (rows of group g use B + g sBg;
 *     rows from offs[G-1] on are left untouched), r in [0, K);
 *   mode 1 (weight gradients): reduction rows r in [0, K) are grouped by offs;
 *     group g writes C + g sCg over i in [0, M), j in [0, N) (zeros, or
 *     nothing added, for an empty group).
 * F.grouped_mm of TF/integrations/moe.py:440-459 and its autograd. */
int moe_f32_grouped_gemm(const float* A, const float* B, const int32_t* offs,
                         int64_t G, int mode, int64_t M, int64_t N, int64_t K,
                         int64_t sAi, int64_t sAr, int64_t sBr, int64_t sBj,
                         int64_t sBg, float* C, int64_t sCi, int64_t sCj,
                         int64_t sCg, int accumulate, void* stream);

/* act[S,I] = silu(pre[:, :I]) * pre[:, I:] and its backward (d_pre[S,2I]
 * from d_act[S,I] and pre), over the rows below offsets[num_buckets-1]
 * (TF/integrations/moe.py:447-450). */
int moe_f32_swiglu_fwd(const float* pre, float* act, const int32_t* offsets,
                       int64_t num_buckets, int64_t S, int64_t I, void* stream);
int moe_f32_swiglu_bwd(const float* d_act, const float* pre, float* d_pre,
                       const int32_t* offsets, int64_t num_buckets, int64_t S,
                       int64_t I, void* stream);

/* moe_combine_fwd / moe_combine_bwd / moe_permute_bwd for fp32 rows (same
 * slot semantics: slots at or past offsets[num_buckets-1] contribute
 * nothing, and receive zero gradient rows and zero score gradients).  The
 * permute backward adds d_add[T,H] (may be NULL) after each token's sum. */
int moe_f32_combine_fwd(const float* y, const int32_t* pos_of_slot,
                        const int32_t* offsets, int64_t num_buckets,
                        const float* scores, int64_t T, int64_t H, int64_t k,
                        float* out, void* stream);
int moe_f32_combine_bwd(const float* d_out, const float* y,
                        const int32_t* pos_of_slot, const int32_t* offsets,
                        int64_t num_buckets, const float* scores, int64_t T,
                        int64_t H, int64_t k, float* d_y, float* d_scores,
                        void* stream);
int moe_f32_permute_bwd(const float* d_xp, const int32_t* pos_of_slot,
                        const int32_t* offsets, int64_t num_buckets, int64_t T,
                        int64_t H, int64_t k, const float* d_add, float* d_x,
                        void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_MI355X_H */
