/*
 * sgsa.h -- C ABI of libsgsa_hip.so, the MI355X (gfx950) SGSA layer-forward
 * library.  Plain pointers and sizes only; every entry point is asynchronous
 * on the caller's HIP stream (passed as void*, NULL = default stream), never
 * allocates device memory and never synchronises.  Device buffers are owned
 * by the caller.
 *
 * Layouts (the reference's, modelings/sgsa_ops/naive.py:24-29):
 *   q, k, v, sparse_k, sparse_v, k_hat, v_hat, write_key, out : [B,T,H,D], D contiguous
 *   beta, gamma, alpha, budget                                : [B,T,H] fp32
 *   initial_state, final_state                                : [B,H,D,D] fp32 (key-major)
 *   indices, scores, weights                                  : [B,H,Tq,top_k]
 *   top2 : [B,H,Tq,2]   counts : [B,H,Tq]   diag : [SGSA_NDIAG,B,H,Tq]
 * dtype: SGSA_F32 or SGSA_BF16 for q/k/v-like tensors; everything else is
 * fp32 (int32 for indices/counts).  D <= 128.
 *
 * Return value: SGSA_OK (0) or an sgsa_status; sgsa_last_error() gives the
 * message of the last failure on the calling thread.  Unsupported input is an
 * error, never a silent fallback.
 */
#ifndef SGSA_H_
#define SGSA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SGSA_ABI_VERSION 1
#define SGSA_NDIAG 10

enum sgsa_status {
  SGSA_OK = 0,
  SGSA_ERR_INVALID_ARG = 1,
  SGSA_ERR_UNSUPPORTED = 2,
  SGSA_ERR_HIP = 3,
  SGSA_ERR_WORKSPACE = 4
};

enum sgsa_dtype { SGSA_F32 = 0, SGSA_BF16 = 1 };

/* Order of the diagnostics planes written by sgsa_sparse_gather
 * (modelings/modeling_sgsa.py:385-404). */
enum sgsa_diag {
  SGSA_DIAG_SCORE_MARGIN = 0,
  SGSA_DIAG_CONCENTRATION = 1,
  SGSA_DIAG_MAX_CONFIDENCE = 2,
  SGSA_DIAG_NOVELTY = 3,
  SGSA_DIAG_WRITE_CONFLICT = 4,
  SGSA_DIAG_ENTROPY = 5,
  SGSA_DIAG_AVG_DISTANCE = 6,
  SGSA_DIAG_LOCAL_RATIO = 7,
  SGSA_DIAG_SINK_RATIO = 8,
  SGSA_DIAG_REMOTE_RATIO = 9
};

int sgsa_abi_version(void);
const char* sgsa_status_string(int status);
const char* sgsa_last_error(void);

/* ---- chunked gated-delta-rule core ------------------------------------------
 * Replaces chunk_sgsa_fwd (modelings/sgsa_ops/chunk_fwd.py:12-131), reached
 * through chunk_sgsa / ChunkSGSAFunction.forward (modelings/sgsa_ops/chunk.py:
 * 104-148, :17-56).  sparse_k, sparse_v, alpha: all three NULL = no sparse
 * write (chunk.py:123).  initial_state NULL = zeros; final_state NULL = not
 * requested.  chunk_size is accepted for signature compatibility; the kernels
 * always use 64-token chunks (the result does not depend on it beyond
 * rounding).  Needs sgsa_chunk_fwd_workspace_size() bytes of workspace. */
int sgsa_chunk_fwd_workspace_size(int B, int T, int H, int D, int has_sparse, size_t* bytes);
int sgsa_chunk_fwd(int dtype, int B, int T, int H, int D, int chunk_size,
                   const void* q, const void* k, const void* v,
                   const float* beta, const float* gamma,
                   const void* sparse_k, const void* sparse_v, const float* alpha,
                   const float* initial_state,
                   void* out, float* final_state,
                   void* workspace, size_t workspace_bytes, void* stream);

/* Backward of sgsa_chunk_fwd: the gradients of <o, d_out> + <final_state,
 * d_final_state> w.r.t. every input, for the function sgsa_chunk_fwd computes.
 * Replaces chunk_sgsa_bwd (modelings/sgsa_ops/chunk_bwd.py:12-77), which
 * recomputes the forward under torch autograd, and the backward the reference
 * plans in modelings/sgsa_bwd_derivation.md:699-832.  Runs the fp32 chunk form
 * for bf16 or fp32 inputs: the forward's per-chunk intermediates, a reverse
 * scan of the state gradient over chunks, then every chunk's gradients in
 * parallel.  d_out and dq, dk, dv, dsparse_k, dsparse_v are [B,T,H,D] in the
 * input dtype; dbeta, dgamma, dalpha [B,T,H] fp32; d_final_state and
 * d_initial_state [B,H,D,D] fp32 (either may be NULL).  The sparse write's
 * inputs and gradients are given together or not at all.  Needs
 * sgsa_chunk_bwd_workspace_size() bytes (about 0.8 MB per 64-token chunk and
 * head with the sparse write). */
int sgsa_chunk_bwd_workspace_size(int B, int T, int H, int D, int has_sparse, size_t* bytes);
int sgsa_chunk_bwd(int dtype, int B, int T, int H, int D,
                   const void* q, const void* k, const void* v,
                   const float* beta, const float* gamma,
                   const void* sparse_k, const void* sparse_v, const float* alpha,
                   const float* initial_state, const void* d_out, const float* d_final_state,
                   void* dq, void* dk, void* dv, float* dbeta, float* dgamma,
                   void* dsparse_k, void* dsparse_v, float* dalpha, float* d_initial_state,
                   void* workspace, size_t workspace_bytes, void* stream);

/* ---- score GEMM + exact token top-k ----------------------------------------
 * Replaces the dense scores and the per-row top-k loop of
 * SparseRetriever.forward / _masked_topk (modelings/modeling_sgsa.py:420-428,
 * :144-165) and of TopKSparseKVReuseAttention.forward
 * (modelings/hybrid_dense_delta_topk.py:343-349).  score = (q.k)/scale for
 * scale_mode 0 (retriever: scale = sqrt(D)), (q.k)*scale for scale_mode 1
 * (hybrid: scale = 1/sqrt(D)).  Query row r sits at key position r+q_offset;
 * causal keeps keys <= that position.  Each row gets
 * counts = min(top_k, valid keys) selected slots, ties broken by lowest key
 * index; slots >= counts hold index 0 and score -FLT_MAX (:151-153).
 * sorted = 0: the selected slots in a deterministic order made of two runs
 * that each ascend in key index; split (may be NULL) receives the length of
 * the first run [B,H,Tq];
 * sorted = 1: (score desc, index asc) as torch.topk(sorted=True) with the
 * lowest-index tie rule.  top2 (may be NULL) receives the two largest valid
 * scores (-FLT_MAX if absent).  Needs sgsa_score_topk_workspace_size() bytes
 * of workspace (per-row candidate lists). */
int sgsa_score_topk_workspace_size(int B, int Tq, int H, size_t* bytes);
/* Workspace that also enables the few-row form of sgsa_score_topk: bf16,
 * D % 32 == 0, at most 8 query rows per (b, h), B*H*Tq <= 2048 and Tk <= 32768
 * (decode).  Each row's keys are scored by many workgroups into a [rows, Tk]
 * buffer, then selected by an exact radix select in LDS; same results and
 * contract, the unsorted order being one ascending run.  Equals
 * sgsa_score_topk_workspace_size() where the form does not apply.  The
 * workspace must be 256-byte aligned for the form to be used. */
int sgsa_score_topk_fast_workspace_size(int dtype, int B, int Tq, int Tk, int H, int D, size_t* bytes);
int sgsa_score_topk(int dtype, int B, int Tq, int Tk, int H, int D, int top_k,
                    int causal, int q_offset, float scale, int scale_mode,
                    const void* q, const void* k,
                    int32_t* indices, float* scores, float* top2, int32_t* counts,
                    int32_t* split, int sorted, void* workspace, size_t workspace_bytes, void* stream);

/* Scratch held by sgsa_score_topk_noalloc on each GPU it runs on (32 MiB), from
 * its first call on that GPU until the process ends. */
#define SGSA_NOALLOC_SCRATCH_BYTES (32u << 20)
/* sgsa_score_topk without a workspace argument and without any device
 * allocation.  No counterpart in the reference: it is for callers that cannot
 * allocate -- code under HIP graph capture, tight decode/serving loops,
 * harnesses that forbid hipMalloc.  Its workspace is a fixed per-GPU device
 * array of SGSA_NOALLOC_SCRATCH_BYTES; it behaves as sgsa_score_topk given
 * sgsa_score_topk_fast_workspace_size() bytes (same launches, same results)
 * and returns SGSA_ERR_WORKSPACE when that size exceeds the array (a decode
 * step of B*H*Tq = 128 rows over 32768 keys needs 17 MB).  Every call on one
 * GPU shares the array: calls that overlap in time on one GPU (two streams,
 * two host threads) race and must be serialised by the caller.  Nothing in
 * the array needs to start at zero. */
int sgsa_score_topk_noalloc(int dtype, int B, int Tq, int Tk, int H, int D, int top_k,
                            int causal, int q_offset, float scale, int scale_mode,
                            const void* q, const void* k,
                            int32_t* indices, float* scores, float* top2, int32_t* counts,
                            int32_t* split, int sorted, void* stream);

/* Masked form of sgsa_score_topk: the padding masks of SparseRetriever.forward
 * (modelings/modeling_sgsa.py:421-428: valid = causal & key_valid &
 * query_valid) and of TopKSparseKVReuseAttention.forward
 * (modelings/hybrid_dense_delta_topk.py:343-349 with _merge_masks :153-175:
 * future keys and padded keys masked, no query mask).  key_mask [B,Tk] and
 * query_mask [B,Tq] are bytes, nonzero = valid; either may be NULL (all
 * valid).  Row (b,h,r) has nv valid keys.  kq_rule 0 (retriever, :159-160): the
 * row takes kq = min(top_k, max(1, max over the batch of nv)) slots; kq_rule 1
 * (hybrid, :348): kq = top_k.  The first counts = min(kq, nv) slots hold the
 * selected valid keys (ties to the lowest key index; sorted as
 * sgsa_score_topk, or in an unspecified order with sorted = 0); slots
 * [counts, kq) hold the row's lowest-index invalid keys with score -FLT_MAX
 * (the reference fills invalid scores with finfo.min, which tie); slots >= kq
 * hold index 0 and -FLT_MAX (:151-153).  slot_valid [B,H,Tq,top_k] (may be
 * NULL) receives 1 for the selected slots and 0 elsewhere; fill [B,H,Tq] (may
 * be NULL) receives kq.  kv_layout: k is [B,Tk,H,D] (0) or [B,H,Tk,D] (1, the
 * hybrid's dense-layer KV).  counts is required; top2 as sgsa_score_topk.
 * Needs sgsa_score_topk_masked_workspace_size() bytes (with has_key_mask or
 * kv_layout 1 it includes a copy of the keys in valid-first order). */
int sgsa_score_topk_masked_workspace_size(int dtype, int B, int Tq, int Tk, int H, int D, int has_key_mask,
                                          int kv_layout, size_t* bytes);
int sgsa_score_topk_masked(int dtype, int B, int Tq, int Tk, int H, int D, int top_k,
                           int causal, int q_offset, float scale, int scale_mode, int kq_rule, int kv_layout,
                           const void* q, const void* k, const uint8_t* key_mask, const uint8_t* query_mask,
                           int32_t* indices, float* scores, uint8_t* slot_valid, float* top2,
                           int32_t* counts, int32_t* fill, int sorted,
                           void* workspace, size_t workspace_bytes, void* stream);

/* Known-answer hook: writes the exact fp32 scores sgsa_score_topk selects on,
 * for query rows [row0, row0+rows), to out [B,H,rows,Tk]; keys outside the
 * causal range get -FLT_MAX. */
int sgsa_score_dump(int dtype, int B, int Tq, int Tk, int H, int D,
                    int causal, int q_offset, float scale, int scale_mode,
                    const void* q, const void* k, int row0, int rows, float* out, void* stream);

/* ---- sparse gather + weights + diagnostics + write gate ---------------------
 * Replaces the softmax/gather of SparseRetriever._token_only
 * (modelings/modeling_sgsa.py:126-134), its _diagnostics (:361-405), the write
 * key and alpha gate of SGSAStateLayer (:546-552, :497-504), and the V-only
 * gather of TopKSparseKVReuseAttention (hybrid_dense_delta_topk.py:350-356;
 * pass k = NULL, k_hat = NULL).  Consumes sgsa_score_topk's output (either
 * order).  top2 may be NULL: the row maximum is then tracked with an
 * online-softmax rescale.  self_key [B,Tq,H,D]: key of each query token (the retriever's
 * self_key = k, :459); needed for diag and for the gate.  budget NULL = no
 * gate (write_key/alpha untouched); else alpha = alpha_max * concentration *
 * novelty * sigmoid(budget), clipped (:497-504), write_mode 0 direct / 1
 * residual.  weights, diag, k_hat, write_key, alpha may be NULL.  workspace:
 * >= 256 bytes when diag is requested, else may be NULL.  Given
 * sgsa_sparse_gather_workspace_size() bytes, calls with few rows and many
 * slots (decode: at most 2048 rows, more than 128 slots) split each row's
 * slots over several waves and merge the partial sums in a fixed order. */
int sgsa_sparse_gather_workspace_size(int B, int Tq, int H, int D, int top_k, size_t* bytes);
int sgsa_sparse_gather(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, int q_offset,
                       const void* k, const void* v, const void* self_key,
                       const int32_t* indices, const float* scores, const float* top2,
                       const int32_t* counts,
                       const float* budget, int write_mode, float alpha_max, float tau_c,
                       int local_window, int sink_size,
                       void* k_hat, void* v_hat, void* write_key, float* alpha,
                       float* weights, float* diag,
                       void* workspace, size_t workspace_bytes, void* stream);

/* sgsa_sparse_gather over the output of sgsa_score_topk_masked: counts is
 * its fill (kq slots per row); slot_valid (may be NULL) zeroes the weight of
 * the invalid slots before the renormalisation (the retriever's
 * softmax * valid / sum, modelings/modeling_sgsa.py:126-128).  With
 * slot_valid = NULL every filled slot takes its softmax weight, as the
 * hybrid's probabilities do (hybrid_dense_delta_topk.py:350): the -FLT_MAX
 * fills weigh 0 unless a row has no valid key, which then averages its kq
 * filled keys.  kv_layout: k and v are [B,Tk,H,D] (0) or [B,H,Tk,D] (1);
 * self_key stays [B,Tq,H,D].  row_stats (may be NULL): as sgsa_layer_fwd_stats. */
int sgsa_sparse_gather_masked(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, int q_offset,
                              int kv_layout, const void* k, const void* v, const void* self_key,
                              const int32_t* indices, const float* scores, const uint8_t* slot_valid,
                              const float* top2, const int32_t* counts, const float* budget, int write_mode,
                              float alpha_max, float tau_c, int local_window, int sink_size, void* k_hat,
                              void* v_hat, void* write_key, float* alpha, float* weights, float* diag,
                              float* row_stats, void* workspace, size_t workspace_bytes, void* stream);

/* Scores at given keys: for every query row and slot i < counts[row],
 * scores[row,i] = (q_row . k[indices[row,i]]) * scale' with fp32 accumulation,
 * where scale' is sgsa_score_topk's (1/scale, or scale for scale_mode 1).
 * Layouts as sgsa_score_topk: q [B,Tq,H,D], k [B,Tk,H,D], indices and scores
 * [B,H,Tq,top_k], counts [B,H,Tq]; indices outside [0,Tk) score 0.  No
 * reference counterpart: it serves top-k reuse, where a candidate set selected
 * once is re-scored by later queries instead of selected again
 * (modelings/idea.md:395-401; config 4 reuses each SGSA layer's top-k over 4
 * decode steps).  Feed the scores to sgsa_sparse_gather with top2 = NULL. */
int sgsa_score_at(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, float scale, int scale_mode,
                  const void* q, const void* k, const int32_t* indices, const int32_t* counts,
                  float* scores, void* stream);

/* Tiled form of sgsa_sparse_gather for the layer path (bf16, D = 128,
 * top_k % 4 == 0, causal, Tq = Tk = T): streams K/V through LDS in 64-key tiles and applies the exact
 * top-k weights with MFMA.  Needs the unsorted output of sgsa_score_topk with
 * top2 and split; computes k_hat, v_hat, the write key and alpha (no
 * weights / diagnostics outputs).  Same references as sgsa_sparse_gather. */
/* ---- block retrieval modes --------------------------------------------------
 * SparseRetriever.forward with retrieval_mode "block_only" (mode 0) or
 * "block_token" (mode 1) on its torch path (modelings/modeling_sgsa.py:444-463;
 * block selection :167-195, candidates :302-359, diagnostics :361-405).
 * Scores (q.k)/sqrt(D); key block b = keys [b*block_size, (b+1)*block_size);
 * block score = max causal score of the block (-FLT_MAX if none); each row
 * keeps eb = min(top_blocks, nb) blocks (nb = ceil(T/block_size)), score
 * desc, ties to the lowest index, padded with 0 (:188-195).  Candidates = the
 * causal keys of the kept blocks; eb * min(block_size, T) <= 2048.
 * Outputs: block_indices [B,H,T,eb]; block_scores [B,H,T,nb] (may be NULL;
 * a copy of the workspace's block-major scores); k_hat, v_hat [B,T,H,D]; diag
 * [SGSA_NDIAG,B,H,T] (may be NULL; block_only leaves planes 6-9 meaningless,
 * as the reference has no token indices there).
 *   mode 1: indices [B,H,T,kk], kk = min(top_k, T): the masked top-k of the
 *     candidates (:322-330), weights [B,H,T,kk] (may be NULL);
 *   mode 0: indices unused (NULL), weights [B,H,T,T] dense (may be NULL),
 *     margin = kept block index 0 - index 1 (:455-463).
 * Workspace: sgsa_block_retrieve_workspace_size() bytes. */
int sgsa_block_retrieve_workspace_size(int B, int T, int H, int top_k, int block_size, int top_blocks, int mode,
                                       size_t* bytes);
int sgsa_block_retrieve(int dtype, int B, int T, int H, int D, int top_k, int block_size, int top_blocks,
                        int mode, int causal, float tau_c, int local_window, int sink_size,
                        const void* q, const void* k, const void* v,
                        int32_t* indices, int32_t* block_indices, float* block_scores, float* weights,
                        void* k_hat, void* v_hat, float* diag, void* workspace, size_t workspace_bytes,
                        void* stream);
/* The same with SparseRetriever.forward's attention_mask (modelings/
 * modeling_sgsa.py:421-428): attention_mask [B,T] uint8, nonzero = real token.
 * A row sees the causal keys that are real tokens; a padded row sees none.
 * Block scores take the max over the keys a row sees (-FLT_MAX if none); a
 * block is valid when it holds one (:188-189); each row keeps k_q = min(eb,
 * max(1, most valid blocks of any (b, h) at that position)) blocks (:159-160),
 * its valid ones by score, then its invalid ones (-FLT_MAX) by ascending
 * index; slots past k_q hold 0.  Candidates = the keys the row sees in its
 * kept blocks (:313-320); block_token's k_q and fills follow the same rule over
 * the candidates, block_only's rows with no candidate get zero weights, k_hat
 * and v_hat.  Same workspace size as sgsa_block_retrieve. */
int sgsa_block_retrieve_masked(int dtype, int B, int T, int H, int D, int top_k, int block_size, int top_blocks,
                               int mode, int causal, float tau_c, int local_window, int sink_size,
                               const void* q, const void* k, const void* v, const uint8_t* attention_mask,
                               int32_t* indices, int32_t* block_indices, float* block_scores, float* weights,
                               void* k_hat, void* v_hat, float* diag, void* workspace, size_t workspace_bytes,
                               void* stream);

/* ---- block retrieval inside the SGSA block (the layer's retrieval half) --------
 * Replaces the retrieval + gate of SGSABlock.forward in the block modes
 * (modelings/modeling_sgsa.py:669-684 with SparseRetriever.forward :444-463 and
 * SGSAStateLayer :543-552, _compute_alpha :497-504; retrieval_mode
 * "block_token" is the reference config's default, :61): the block retrieval of
 * sgsa_block_retrieve(_masked) on (q_ret, k, v), causal, then the write key
 * (write_mode 0 direct: k_hat; 1 residual: k_hat - (k_hat.k / max(|k|^2, 1e-6)) k)
 * and alpha = alpha_max * concentration * clamp(novelty, 0, 1) * sigmoid(budget),
 * clipped by 1 / max(alpha |v_hat| |write key|, 1).  block_only's concentration
 * reads the kept block indices' difference as the reference's does (:455-463).
 * attention_mask [B,T] uint8 or NULL.  budget [B,T,H] fp32 logits.  Outputs:
 * write_key, v_hat [B,T,H,D] in dtype, alpha [B,T,H] fp32, row_stats [2,B,H,T]
 * (largest weight; |write key| / |k_hat| clamped to [0, 10] in residual mode,
 * else 0) or NULL.  Index lists stay in the workspace:
 * sgsa_block_layer_retrieve_workspace_size() bytes. */
int sgsa_block_layer_retrieve_workspace_size(int B, int T, int H, int top_k, int block_size, int top_blocks,
                                             int mode, size_t* bytes);
int sgsa_block_layer_retrieve(int dtype, int B, int T, int H, int D, int top_k, int block_size, int top_blocks,
                              int mode, float tau_c, const void* q_ret, const void* k, const void* v,
                              const uint8_t* attention_mask, const float* budget, int write_mode, float alpha_max,
                              void* write_key, void* v_hat, float* alpha, float* row_stats, void* workspace,
                              size_t workspace_bytes, void* stream);

/* ---- RMSNorm of the model shells -------------------------------------------
 * y = x * rsqrt(mean(x^2) + eps) * weight over the last dimension, in fp32,
 * stored in x's dtype: the RMSNorm of the SGSA and hybrid stacks
 * (modelings/hybrid_dense_delta_topk.py:94-103; the fla RMSNorm the SGSA model
 * imports, modeling_sgsa.py:40, evaluated in fp32).  x, y [rows, C] contiguous
 * in dtype; weight [C] in dtype (weight_f32 = 0) or fp32 (weight_f32 = 1). */
int sgsa_rms_norm(int dtype, int weight_f32, long rows, int C, const void* x, const void* weight, float eps, void* y,
                  void* stream);

/* The residual add before a block's second norm (SGSABlock.forward,
 * modelings/modeling_sgsa.py:684-686; hybrid_dense_delta_topk.py:240-244)
 * in one launch: sum = a + b (rounded to dtype), y = sgsa_rms_norm(sum).
 * a, b, sum, y [rows, C] contiguous in dtype; sum may not alias a or b. */
int sgsa_add_rms_norm(int dtype, int weight_f32, long rows, int C, const void* a, const void* b, void* sum,
                      const void* weight, float eps, void* y, void* stream);

/* nn.Linear on a few rows, for the decode step's projections (the model
 * shells' q/k/v, output, MLP and LM-head linears at B <= 16 tokens):
 * y = x weight^T (+ bias), bf16 in and out, fp32 accumulation.  x [M, K]
 * (row stride x_row_stride elements, a multiple of 8), weight [N, K]
 * contiguous, bias [N] or NULL, y [M, N] (row stride y_row_stride);
 * M <= 16, K a multiple of 32, x and weight 16-byte aligned. */
int sgsa_linear_rows(int dtype, int M, int N, int K, const void* x, long x_row_stride, const void* weight,
                     const void* bias, void* y, long y_row_stride, void* stream);

/* sgsa_linear_rows' weight in its tiled layout, for callers that keep a
 * weight across many calls (the decode loop; no counterpart in the
 * reference, whose linears are nn.Linear): tiled[ceil(N / 16)][K / 32][64][8]
 * with tiled[t][s][l] = weight[16t + l % 16][32s + 8 (l / 16) .. + 7] (zero
 * for rows past N), 16 ceil(N / 16) K elements, so that one step of the
 * product reads 1 KB in one piece.  weight [N, K] contiguous, bf16, K a
 * multiple of 32, both 16-byte aligned. */
int sgsa_linear_rows_tile(int dtype, int N, int K, const void* weight, void* tiled, void* stream);

/* sgsa_linear_rows on a weight in sgsa_linear_rows_tile's layout: the same
 * arguments and the same results bit for bit, 20-25% faster at the decode
 * shapes. */
int sgsa_linear_rows_tiled(int dtype, int M, int N, int K, const void* x, long x_row_stride, const void* tiled,
                           const void* bias, void* y, long y_row_stride, void* stream);

/* The gated MLP's activation (down(silu(gate(x)) * up(x)), modeling_sgsa.py's
 * and the hybrid's MLP) on a fused gate | up projection: row r of gate_up
 * (row_stride elements) holds gate's I values then up's.  y [rows, I]
 * contiguous = silu(gate) rounded to dtype, times up, rounded to dtype. */
int sgsa_silu_mul(int dtype, long rows, int I, const void* gate_up, long row_stride, void* y, void* stream);

/* Rotary embedding of a dense attention layer's q and k (rotate-half form,
 * modelings/hybrid_dense_delta_topk.py:140-150), in x's dtype with a rounding
 * after each product and the sum (torch's elementwise semantics).  Row (b, t)
 * of the projection output starts at qk + (b*T + t) * row_stride: q's Hq heads
 * of D, then k's Hk heads.  cos_table / sin_table [table_len, D] fp32, rows
 * pos0 .. pos0+T-1 used.  q_out [B,Hq,T,D], k_out [B,Hk,T,D] contiguous. */
int sgsa_rope_qk(int dtype, int B, int T, int Hq, int Hk, int D, int pos0, int table_len, const void* qk,
                 long row_stride, const float* cos_table, const float* sin_table, void* q_out, void* k_out,
                 void* stream);

/* The SGSA layer's gates from its gate projections' logits (SGSAStateLayer,
 * modelings/modeling_sgsa.py:543-544 and the budget logits): beta = max(sigmoid(b), 1e-4),
 * gamma = sigmoid(g), budget = u, as fp32 [rows, H].  Row r's logits start at
 * logits + r * row_stride (elements of dtype): b's H values, then g's, then u's.
 * row_stride >= 3H. */
int sgsa_layer_gates(int dtype, long rows, int H, const void* logits, long row_stride, float* beta, float* gamma,
                     float* budget, void* stream);

/* The hybrid decoder's dense causal GQA attention for a block of query rows
 * (prefill; modelings/hybrid_dense_delta_topk.py:178-192): query row t sits at
 * position pos0 + t and attends to cache rows [0, pos0 + t].  The reference's
 * rounding points in bf16: the score product and its 1/sqrt(D) scaling rounded
 * to bf16, the softmax in fp32, the probabilities rounded to bf16 after
 * normalisation, fp32 accumulation with V.  bf16 only.  q, out [B, H, Tq, D];
 * k_cache, v_cache [B, Hkv, cache_len, D] contiguous with rows
 * [0, pos0 + Tq) filled; D = 128, H a multiple of Hkv.  workspace: B*H*Tq*8
 * bytes (each row's softmax maximum and sum). */
int sgsa_dense_attention(int dtype, int B, int H, int Hkv, int D, int Tq, int pos0, const void* q,
                         const void* k_cache, const void* v_cache, long cache_len, void* out, void* workspace,
                         size_t workspace_bytes, void* stream);

/* The hybrid decoder's dense GQA attention for one decode token per sequence
 * (modelings/hybrid_dense_delta_topk.py:178-192 at q_len = 1, the query at
 * position kend - 1): o = softmax(q K^T / sqrt(D)) V over cache rows
 * [0, kend), with the reference's rounding points in bf16 (score product and
 * its scaling rounded to bf16, softmax in fp32, probabilities rounded to bf16,
 * fp32 accumulation with V).  q, out [B, H, 1, D]; k_cache, v_cache
 * [B, Hkv, cache_len, D], all contiguous in dtype; D = 128, H / Hkv in
 * {1, 2, 4, 8}.  Workspace from sgsa_decode_attention_workspace_size. */
int sgsa_decode_attention_workspace_size(int dtype, int B, int H, int kend, size_t* bytes);
int sgsa_decode_attention(int dtype, int B, int H, int Hkv, int D, const void* q, const void* k_cache,
                          const void* v_cache, long cache_len, int kend, void* out, void* workspace,
                          size_t workspace_bytes, void* stream);

/* One SGSA decode step's projections, split for the decode kernels: the
 * strided views and casts of SGSABlock's projections and gates
 * (modelings/modeling_sgsa.py:480-482, :543-544) and the KV-cache append of
 * one token, in one launch.  Row b of proj (row_stride elements of dtype)
 * holds q, k, v, q_ret (H*D each) then the gate logits b, g, u (H each).
 * Writes q, k, v, q_ret contiguous [B, H*D] in dtype and beta, gamma, budget
 * fp32 [B, H] as sgsa_layer_gates does; with k_cache / v_cache
 * ([B, cache_len, H, D] contiguous, dtype; both or neither) also k and v into
 * cache row pos (0 <= pos < cache_len).  row_stride >= 4*H*D + 3*H. */
int sgsa_decode_split(int dtype, int B, int H, int D, const void* proj, long row_stride, void* q, void* k, void* v,
                      void* q_ret, float* beta, float* gamma, float* budget, void* k_cache, void* v_cache,
                      long cache_len, long pos, void* stream);

int sgsa_sparse_gather_tiled(int B, int T, int H, int D, int top_k, const void* k, const void* v,
                             const int32_t* indices, const float* scores, const float* top2,
                             const int32_t* counts, const int32_t* split, const float* budget,
                             int write_mode, float alpha_max, float tau_c, void* k_hat, void* v_hat,
                             void* write_key, float* alpha, void* stream);

/* ---- recurrent form (decode step) -----------------------------------------------
 * fused_recurrent_sgsa (modelings/sgsa_ops/recurrent.py:138-175, Triton kernel
 * recurrent_fwd_triton.py:25-145) with the semantics of naive_recurrent_sgsa
 * (naive.py:34-57): token by token, decay first, both writes read the decayed
 * state, o_t = S^T q_t.  q, k, v, sparse_k, sparse_v [B,T,H,D] (dtype);
 * beta, gamma, alpha [B,T,H] fp32; sparse_k / sparse_v / alpha all NULL or all
 * given; initial_state / final_state [B,H,D,D] fp32 or NULL; out [B,T,H,D]
 * in dtype.  T = 1 is one decode step.  No workspace. */
int sgsa_recurrent_fwd(int dtype, int B, int T, int H, int D,
                       const void* q, const void* k, const void* v,
                       const float* beta, const float* gamma,
                       const void* sparse_k, const void* sparse_v, const float* alpha,
                       const float* initial_state, void* out, float* final_state, void* stream);

/* ---- layer-path building blocks: tile lists ----------------------------------
 * The fused layer (sgsa_layer_fwd, bf16 with D = 128) does not materialise
 * per-row index/score lists: K1 writes, for every 64-row block, every 16-row
 * wave of it and every 64-key tile, the selected (score, row, key) entries of
 * that tile, which is the order the tiled gather consumes them in.  These
 * entries run the two halves separately (causal, Tq = Tk = T, scores
 * q.k / sqrt(D) as in the retriever, modelings/modeling_sgsa.py:420-428,
 * :144-165, :126-134).  Layout: region r = ((b*H + h) * ceil(T/64) + block)
 * * 4 + wave holds 16 * (min(top_k,T) + 512) 8-byte entries {float score,
 * uint32 row_in_wave << 8 | key_in_tile} (the score of a candidate that lost
 * the threshold tie-break is -inf) and ceil(T/64) + 1 int32 tile offsets. */
int sgsa_topk_lists_size(int B, int T, int H, int top_k, size_t* list_bytes, size_t* offset_bytes);
/* bf16 q, k [B,T,H,D]; top2 [B,H,T,2], counts [B,H,T]; workspace as sgsa_score_topk. */
int sgsa_score_topk_lists(int B, int T, int H, int D, int top_k, const void* q, const void* k,
                          void* lists, int32_t* offsets, float* top2, int32_t* counts,
                          void* workspace, size_t workspace_bytes, void* stream);
/* The tiled gather (D = 128) on those lists: k_hat or write key, v_hat, alpha
 * (same outputs and references as sgsa_sparse_gather_tiled). */
int sgsa_sparse_gather_lists(int B, int T, int H, int D, int top_k, const void* k, const void* v,
                             const void* lists, const int32_t* offsets, const float* top2,
                             const int32_t* counts, const float* budget, int write_mode,
                             float alpha_max, float tau_c, void* k_hat, void* v_hat,
                             void* write_key, float* alpha, void* stream);

/* ---- layer-path building blocks: row thresholds ------------------------------
 * What sgsa_layer_fwd runs for bf16 with D = 128.  K1 leaves, per row, only the
 * exact cut of its top-k: thr[b,h,t] = {float th, int32 cut}; key j (causal,
 * j <= t) is selected iff score_j > th, or score_j == th and j <= cut (the
 * lowest indices win ties at the threshold; cut = INT32_MAX when there is no
 * tie to break).  The gather recomputes the scores of every causal key with
 * the same products -- bit-identical fp32 -- and applies the cut, so both
 * halves select exactly the rows of modelings/modeling_sgsa.py:144-165
 * (lowest-index ties) and weigh them as :126-134.  Causal, Tq = Tk = T,
 * scores q.k / sqrt(D) (:420-428).  bf16 q, k, v [B,T,H,D]; thr [B,H,T] of
 * 8 bytes; top2 [B,H,T,2] fp32; counts [B,H,T] int32; workspace as
 * sgsa_score_topk. */
int sgsa_score_topk_thresholds(int B, int T, int H, int D, int top_k, const void* q, const void* k,
                               void* thr, float* top2, int32_t* counts, void* workspace,
                               size_t workspace_bytes, void* stream);
/* k_hat or write key, v_hat, alpha from those thresholds (D = 128; same outputs
 * and references as sgsa_sparse_gather_tiled). */
int sgsa_sparse_gather_thresholds(int B, int T, int H, int D, int top_k, const void* q, const void* k,
                                  const void* v, const void* thr, const float* top2,
                                  const int32_t* counts, const float* budget, int write_mode,
                                  float alpha_max, float tau_c, void* k_hat, void* v_hat,
                                  void* write_key, float* alpha, void* stream);

/* Known-answer hook of sgsa_sparse_gather_thresholds: the same kernel with
 * the same selection, writing instead of the gathered rows each row's
 * selection summary selection[b,h,t] = {count, sum of the selected key
 * indices, xor of (index * 2654435761) mod 2^32} as int32 [B,H,T,3], to be
 * compared exactly with the index lists of sgsa_score_topk. */
int sgsa_gather_thresholds_selection(int B, int T, int H, int D, int top_k, const void* q, const void* k,
                                     const void* v, const void* thr, const float* top2,
                                     const int32_t* counts, int32_t* selection, void* stream);

/* ---- whole SGSA layer forward ------------------------------------------------
 * The attention half of SGSABlock.forward (modelings/modeling_sgsa.py:669-684)
 * with the projections as inputs: token top-k retrieval on (q_ret, k, v)
 * (causal, scale sqrt(D)), write key + alpha gate from budget logits, then
 * chunk_sgsa(q, k, v, beta, gamma, write_key, v_hat, alpha, initial_state)
 * (:584-596).  out [B,T,H,D] dtype; final_state [B,H,D,D] fp32 or NULL. */
int sgsa_layer_fwd_workspace_size(int dtype, int B, int T, int H, int D, int top_k, size_t* bytes);
int sgsa_layer_fwd(int dtype, int B, int T, int H, int D, int top_k, int chunk_size,
                   const void* q, const void* k, const void* v, const void* q_ret,
                   const float* beta, const float* gamma, const float* budget,
                   const float* initial_state, int write_mode, float alpha_max, float tau_c,
                   void* out, float* final_state,
                   void* workspace, size_t workspace_bytes, void* stream);

/* The retrieval half of sgsa_layer_fwd on its own: the token top-k over
 * (q_ret, k, v), the write key (write_mode 0: k_hat; 1: k_hat minus its
 * projection on k) and the alpha gate -- the sparse_k / sparse_v / alpha that
 * SGSABlock.forward hands to chunk_sgsa (modelings/modeling_sgsa.py:669-684,
 * :546-552).  Same kernels and workspace (sgsa_layer_fwd_workspace_size) as
 * sgsa_layer_fwd.  write_key / v_hat [B,T,H,D] dtype, alpha [B,T,H] fp32. */
int sgsa_layer_retrieve(int dtype, int B, int T, int H, int D, int top_k,
                        const void* q_ret, const void* k, const void* v, const float* budget,
                        int write_mode, float alpha_max, float tau_c,
                        void* write_key, void* v_hat, float* alpha,
                        void* workspace, size_t workspace_bytes, void* stream);

/* The retrieval half of the layer with SparseRetriever.forward's attention_mask
 * (modelings/modeling_sgsa.py:421-428; SGSABlock.forward passes it to the retriever,
 * :668-675) on the threshold form: bf16, D = 128, T <= 65536.  attention_mask [B,T]
 * uint8, nonzero = real token.  A query row sees the real tokens at or before it and
 * takes k_q = min(top_k, max(1, most real tokens any batch row sees at that position))
 * slots (:159-160); slots past its own real tokens hold nothing (weight 0), and a
 * padded query row retrieves nothing (write key, v_hat and alpha 0).  The keys and
 * values are copied in valid-first order into the workspace, then K1 cuts each row
 * and K2 recomputes and weighs the scores as in sgsa_layer_retrieve.  Outputs as
 * sgsa_layer_retrieve_stats.  Workspace: sgsa_layer_retrieve_masked_workspace_size()
 * bytes (it returns SGSA_ERR_UNSUPPORTED outside bf16 / D = 128 / T <= 65536). */
int sgsa_layer_retrieve_masked_workspace_size(int dtype, int B, int T, int H, int D, int top_k, size_t* bytes);
int sgsa_layer_retrieve_masked(int dtype, int B, int T, int H, int D, int top_k, const void* q_ret, const void* k,
                               const void* v, const uint8_t* attention_mask, const float* budget, int write_mode,
                               float alpha_max, float tau_c, void* write_key, void* v_hat, float* alpha,
                               float* row_stats, void* workspace, size_t workspace_bytes, void* stream);

/* sgsa_layer_fwd / sgsa_layer_retrieve with the per-row figures behind
 * SGSABlock.forward's metrics (modelings/modeling_sgsa.py:697-708):
 * alpha_out [B,T,H] fp32 (may be NULL) receives alpha ("alpha_mean");
 * row_stats [2,B,H,T] fp32 (may be NULL) receives in plane 0 each row's
 * largest retrieval weight (_diagnostics' max_confidence, :374,
 * "retrieval_confidence_mean") and in plane 1 |write key| / max(|k_hat|, 1e-6)
 * clamped to [0, 10] for write_mode 1 ("k_hat_perp_ratio_mean", :614), 0 for
 * write_mode 0.  The means are left to the caller. */
int sgsa_layer_fwd_stats(int dtype, int B, int T, int H, int D, int top_k, int chunk_size,
                         const void* q, const void* k, const void* v, const void* q_ret,
                         const float* beta, const float* gamma, const float* budget,
                         const float* initial_state, int write_mode, float alpha_max, float tau_c,
                         void* out, float* final_state, float* alpha_out, float* row_stats,
                         void* workspace, size_t workspace_bytes, void* stream);
int sgsa_layer_retrieve_stats(int dtype, int B, int T, int H, int D, int top_k,
                              const void* q_ret, const void* k, const void* v, const float* budget,
                              int write_mode, float alpha_max, float tau_c,
                              void* write_key, void* v_hat, float* alpha, float* row_stats,
                              void* workspace, size_t workspace_bytes, void* stream);

/* ---- hybrid decoder: one decode step of the whole layer stack -----------------
 * HybridForCausalLM.decode_step's layer loop (the reference's hybrid stack,
 * modelings/hybrid_dense_delta_topk.py:394-437, one greedy decode token per
 * sequence, :510-532) in one host call, so that a step costs one call rather
 * than several hundred Python dispatches.  Each layer runs the same launches,
 * in the same order, as sgsa_amd.hybrid's per-layer decode:
 *   SGSA layer (kind 0; SGSABlock, modeling_sgsa.py:660-709, with the
 *   recurrent backend and top-k reuse): RMSNorm, the fused projection
 *   q|k|v|q_ret|beta|gamma|budget (sgsa_linear_rows), sgsa_decode_split (the
 *   k, v cache row at pos), the selection (sgsa_score_topk over cache rows
 *   [0, pos], written to cand_idx / cand_cnt) when select != 0, else the
 *   re-score of the kept candidates (sgsa_score_at), sgsa_sparse_gather (the
 *   write key, v_hat, alpha), sgsa_recurrent_fwd (state updated in place),
 *   then the shell;
 *   dense layer (kind 1; :195-244): RMSNorm, the fused q|k|v projection, RoPE
 *   of q and k at position pos with k and v written to cache row pos
 *   (sgsa_rope_qk's arithmetic), sgsa_decode_attention over cache rows
 *   [0, pos], then the shell;
 *   shell: o projection, the residual add and second RMSNorm
 *   (sgsa_add_rms_norm), the gated MLP (the gate/up projection with
 *   sgsa_silu_mul's silu(gate) * up in its epilogue, the down projection with
 *   the residual add in its epilogue).
 * h [B, C] bf16 is the residual stream, updated in place.  All tensors bf16
 * except state (fp32), the rope tables (fp32 [rope_len, D]) and the norm
 * weights (bf16, or fp32 with norm_w_f32 = 1).  Weights are [out, in] in
 * sgsa_linear_rows_tile's layout: w_in [4HD + 3H, C] (SGSA) or
 * [(H + 2Hkv) D, C] (dense), w_o [C, HD], w_gu [2I, C] with gate and up rows
 * interleaved in groups of 8 (rows 16b .. 16b + 7 = gate rows 8b .. 8b + 7,
 * rows 16b + 8 .. 16b + 15 = up rows 8b .. 8b + 7), w_down [C, I]; biases
 * [out] or NULL (w_gu and w_down take none).  Caches: SGSA k/v [B, cache_len,
 * H, D], dense k/v [B, Hkv, cache_len, D], contiguous; cand_idx [B, H, top_k]
 * int32, cand_cnt [B, H] int32.  Limits: B <= 16, D = 128, C, HD and I
 * multiples of 32, H / Hkv in {1, 2, 4, 8}, top_k <= pos + 1 <= cache_len
 * (the candidate rows hold top_k slots), rope_len > pos; select must be set
 * on a layer stack's first step (there are no candidates to re-score).
 * Workspace: sgsa_decode_stack_workspace_size() bytes, 256-byte aligned. */
typedef struct SgsaDecodeConfig {
  int B, C, H, Hkv, D, I;
  int top_k, write_mode;      /* write_mode 0 direct, 1 residual */
  float alpha_max, tau_c, eps;
  int norm_w_f32;
  long cache_len;
  const float* rope_cos;      /* dense layers: [rope_len, D] */
  const float* rope_sin;
  int rope_len;
} SgsaDecodeConfig;

typedef struct SgsaDecodeLayer {
  int kind;                   /* 0 SGSA, 1 dense */
  const void* input_norm;
  const void* post_norm;
  const void* w_in;
  const void* b_in;
  const void* w_o;
  const void* b_o;
  const void* w_gu;
  const void* w_down;
  void* k_cache;
  void* v_cache;
  float* state;               /* SGSA */
  int32_t* cand_idx;          /* SGSA */
  int32_t* cand_cnt;          /* SGSA */
} SgsaDecodeLayer;

int sgsa_decode_stack_workspace_size(const SgsaDecodeConfig* cfg, size_t* bytes);
int sgsa_decode_stack(const SgsaDecodeConfig* cfg, int n_layers, const SgsaDecodeLayer* layers, void* h, int pos,
                      int select, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SGSA_H_ */
