// Internal host-side interface between the C ABI (api.cpp) and the kernel
// translation units.  Not installed; the public interface is include/sgsa.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace sgsa {

enum DType { DT_F32 = 0, DT_BF16 = 1 };

struct ChunkArgs {
  int dtype;
  int B, T, H, D;
  const void* q;
  const void* k;
  const void* v;
  const float* beta;
  const float* gamma;
  const void* sparse_k;   // nullptr together with sparse_v/alpha: no sparse write
  const void* sparse_v;
  const float* alpha;
  const float* initial_state;   // [B,H,D,D] fp32 or nullptr
  void* out;                    // [B,T,H,D] dtype
  float* final_state;           // [B,H,D,D] fp32 or nullptr
  void* workspace;
};

size_t chunk_workspace_bytes(int B, int T, int H, int has_sparse);   // covers both paths
size_t chunk_bf16_workspace_bytes(int B, int T, int H, int has_sparse);
hipError_t launch_chunk_fwd(const ChunkArgs& a, hipStream_t st);
hipError_t launch_chunk_bf16(const ChunkArgs& a, hipStream_t st);
// The fp32 chunk path's per-chunk intermediates for the backward (chunk.hip): per
// (b*H + h, chunk) W, U [M][128], the log-decay prefix [64] and A [M][M]
// (M = 128 with the sparse write, else 64).
hipError_t launch_chunk_intra(const ChunkArgs& a, float* W, float* U, float* lgd, float* A, hipStream_t st);
// The same operands for bf16 inputs from the forward's K3 (chunk_inv_bf16 in its backward form).
hipError_t launch_chunk_intra_bf16(const ChunkArgs& a, float* W, float* U, float* lgd, float* A, hipStream_t st);

// Backward of chunk_sgsa (chunk_bwd.hip).
struct ChunkBwdArgs {
  ChunkArgs f;                  // the forward's inputs (out / final_state unused)
  const void* d_out;            // [B,T,H,D] in the input dtype
  const float* d_final_state;   // [B,H,D,D] fp32 or nullptr
  void *dq, *dk, *dv, *dsk, *dsv;   // [B,T,H,D] in the input dtype (dsk / dsv with the sparse write)
  float *dbeta, *dgamma, *dalpha;   // [B,T,H] fp32 (dalpha with the sparse write)
  float* d_initial_state;       // [B,H,D,D] fp32 or nullptr
  void* workspace;
};
size_t chunk_bwd_workspace_bytes(int B, int T, int H, int has_sparse);
hipError_t launch_chunk_bwd(const ChunkBwdArgs& a, hipStream_t st);

struct RecurrentArgs {
  int dtype;
  int B, T, H, D;
  const void* q;              // [B,T,H,D]
  const void* k;
  const void* v;
  const float* beta;          // [B,T,H]
  const float* gamma;
  const void* sparse_k;       // [B,T,H,D] or nullptr (no sparse write)
  const void* sparse_v;
  const float* alpha;         // [B,T,H]
  const float* initial_state; // [B,H,D,D] fp32 or nullptr
  void* out;                  // [B,T,H,D] in the input dtype
  float* final_state;         // [B,H,D,D] fp32 or nullptr
};
hipError_t launch_recurrent(const RecurrentArgs& a, hipStream_t st);

struct TopkArgs {
  int dtype;
  int B, Tq, Tk, H, D;
  int top_k;          // slots per row actually written (topk_dim)
  int causal;
  int q_offset;       // query row r sits at key position r + q_offset
  float scale;        // score = acc / scale (scale_mode 0) or acc * scale (scale_mode 1)
  int scale_mode;
  const void* q;      // [B,Tq,H,D]
  const void* k;      // [B,Tk,H,D]
  // Masked select (row kernel, non-list): the valid keys of row (b, r) are keys
  // [0, row_nv[b*Tq + r]) -- a prefix, after the key compaction of mask.hip --
  // and the row selects min(row_kq[r], row_nv) of them.  nullptr: the causal /
  // full key range and top_k for every row.
  const int32_t* row_nv;     // [B,Tq] or nullptr
  const int32_t* row_kq;     // [Tq] or nullptr (only with row_nv)
  int32_t* indices;   // [B,H,Tq,top_k]
  float* scores;      // [B,H,Tq,top_k]
  float* top2;        // [B,H,Tq,2] or nullptr
  int32_t* counts;    // [B,H,Tq] valid selected slots, or nullptr
  int32_t* split;     // [B,H,Tq] length of the leading ascending-index run, or nullptr
  float* dump;        // score-dump mode: [B,H,dump_rows,Tk]; nullptr = select mode
  int dump_row0, dump_rows;
  uint2* tl_list;     // layer path (bf16): per-wave tile lists, topk_list_bytes(); nullptr otherwise
  int32_t* tl_off;    // per-wave tile start offsets, topk_list_off_bytes()
  int tl_ntmax;       // set by the launcher: key tiles per row block
  uint2* thr;         // threshold mode (bf16, D = 128, top-2 required): [B,H,Tq] {fp32 th, cut}; no lists
  void* workspace;    // topk_workspace_bytes(): candidate lists + per-head key norms
  uint2* scratch;     // set by the launcher
  int* flags;         // set by the launcher
  const float* kmax;  // set by the launcher
};

// Padding masks for the select (mask.hip).
struct MaskArgs {
  int dtype;
  int B, Tq, Tk, H, D;
  int causal, q_offset;
  int top_k;                  // slots per row of the outputs
  int kq_rule;                // 0: kq = min(top_k, max(1, max_b nv)) per row; 1: kq = top_k
  int kv_hm;                  // key layout: 0 [B,Tk,H,D], 1 [B,H,Tk,D]
  int compacted;              // 1: keys copied to kc in valid-first order (needed with a key mask or kv_hm)
  const uint8_t* key_mask;    // [B,Tk] (nonzero = valid) or nullptr
  const uint8_t* query_mask;  // [B,Tq] or nullptr
  const void* k;
  // workspace (mask_carve)
  int32_t* pc;                // [B,Tk+1] valid keys below j
  int32_t* perm;              // [B,Tk] valid keys' indices, ascending
  int32_t* inv;               // [B,Tk] masked keys' indices, ascending
  int32_t* nv;                // [B,Tq] valid keys per row
  int32_t* kq;                // [Tq] slots per row
  void* kc;                   // [B,Tk,H,D] compacted keys (compacted only)
};
size_t mask_workspace_bytes(int dtype, int B, int Tq, int Tk, int H, int D, int compact);
void mask_carve(MaskArgs& m, void* ws);
hipError_t launch_mask_prepare(const MaskArgs& m, hipStream_t st);
// Another [B,Tk,H,D] (or kv_hm [B,H,Tk,D]) tensor in the valid-first key order of m (after launch_mask_prepare).
hipError_t launch_mask_compact(const MaskArgs& m, const void* src, void* dst, hipStream_t st);
hipError_t launch_mask_finish(const MaskArgs& m, int32_t* indices, float* scores, uint8_t* slot_valid,
                              const int32_t* counts, int32_t* fill, hipStream_t st);

constexpr int TOPK_CAP = 512;   // collected threshold-bin candidates per row

// Few-row form of the select (topk_rows.hip): bf16, D % 32 == 0, at most
// TR_MAX_TQ query rows per (b, h), TR_MAX_ROWS rows and TR_MAXK keys.  Extra
// workspace (a [rows, Tk] fp32 score buffer) or 0 when the form does not apply.
constexpr int DP_ROWS = 128;
constexpr int TR_MAXK = 32768;
constexpr int TR_MAX_TQ = 8;
constexpr long TR_MAX_ROWS = 2048;
size_t topk_rows_bytes(const TopkArgs& a);
hipError_t launch_score_topk_rows(const TopkArgs& a, float* sbuf, hipStream_t st);
size_t topk_workspace_bytes(int B, int Tq, int H);
// Tile-list layout shared by the layer-path K1 and K2: one region per
// (batch*head, 64-row block, wave) of 16 * (top_k + TOPK_CAP) entries and of
// ceil(Tk / 64) + 1 tile offsets.
size_t topk_list_bytes(int B, int Tq, int H, int top_k);
size_t topk_list_off_bytes(int B, int Tq, int Tk, int H);

hipError_t launch_score_topk(const TopkArgs& a, hipStream_t st);
// The multiplier K1 applies to q.k accumulators (score = acc * multiplier).
inline float score_multiplier(float scale, int scale_mode) {
  return scale_mode == 0 ? (float)(1.0 / (double)scale) : scale;
}
hipError_t launch_sort_rows(int32_t* indices, float* scores, long rows, int top_k, const int32_t* counts,
                            hipStream_t st);

struct GatherArgs {
  int dtype;
  int B, Tq, Tk, H, D;
  int top_k;                 // slots per row (topk_dim)
  int q_offset;              // query row r sits at key position r + q_offset
  const void* k;             // [B,Tk,H,D]  (nullptr: V-only gather)
  const void* v;             // [B,Tk,H,D]
  int kv_hm;                 // 1: k and v are [B,H,Tk,D] (row kernels only)
  const void* self_key;      // [B,Tq,H,D] key of the query token (diagnostics / residual key), or nullptr
  const int32_t* indices;    // [B,H,Tq,top_k]
  const float* scores;       // [B,H,Tq,top_k]
  const float* top2;         // [B,H,Tq,2] row max / second max, or nullptr (online max)
  const int32_t* counts;     // [B,H,Tq] valid slots (prefix) per row
  const uint8_t* slot_valid; // [B,H,Tq,top_k] or nullptr (all slots < counts valid)
  int use_valid;             // 1: weights are multiplied by validity and renormalised (retriever)
  float tau_c, eps;
  int local_window, sink_size;
  const float* budget;       // [B,Tq,H] budget logits -> alpha gate, or nullptr
  int write_mode;            // 0 direct, 1 residual
  float alpha_max;
  void* k_hat;               // [B,Tq,H,D] dtype or nullptr
  void* v_hat;               // [B,Tq,H,D] dtype
  void* write_key;           // [B,Tq,H,D] dtype or nullptr
  float* alpha;              // [B,Tq,H] or nullptr
  float* weights;            // [B,H,Tq,top_k] or nullptr
  float* diag;               // [NDIAG,B,H,Tq] or nullptr
  float* stats;              // [2,B,H,Tq] or nullptr: largest weight; |write key| / |k_hat| (residual mode, else 0)
  int32_t* sel_dbg;          // threshold gather only: [B,H,Tq,3] selection summary instead of the outputs
  int32_t* max_index;        // GATHER_MAXIDX_SLOTS ints of scratch (256 bytes, diagnostics); required with diag
  const float* margin_in;    // [B,H,Tq] score margin to report instead of top-2 (block_only), or nullptr
  const int32_t* row_nv;     // threshold gather: [B,Tq] valid-key prefix per row (keys compacted valid-first
                             // under a padding mask), or nullptr for the causal range
  float ent_pad;             // zero-weight entries of the row beyond the slots (entropy terms of eps)
  int nsplit;                // > 0: split-row form, nsplit partials of split_len slots per row
  int split_len;
  float* part;               // [B,H,Tq,nsplit,4+2D] partials (split-row form)
  const void* rq;            // split-row form, bf16, D = 128, [B,Tk,H,D] keys: [B,Tq,H,D] queries whose slot
                             // scores (q . k) * rq_ms the partial kernel computes from the key rows it gathers
                             // (scores is then not read), or nullptr
  float rq_ms;
  int pieces_only;           // split-row form: launch the partial kernel only (the caller merges)
};

// Split-row gather: used for at most GATHER_SPLIT_ROWS rows with more than
// GATHER_SPLIT_LEN slots; partial buffer bytes for a call.
constexpr long GATHER_SPLIT_ROWS = 2048;
constexpr int GATHER_SPLIT_LEN = 128;
inline int gather_nsplit(long rows, int top_k) {
  if (rows > GATHER_SPLIT_ROWS || top_k <= GATHER_SPLIT_LEN) return 0;
  return (top_k + GATHER_SPLIT_LEN - 1) / GATHER_SPLIT_LEN;
}
inline size_t gather_part_bytes(long rows, int top_k, int D) {
  return (size_t)rows * gather_nsplit(rows, top_k) * (4 + 2 * D) * sizeof(float);
}

constexpr int NDIAG = 10;
constexpr int GATHER_MAXIDX_SLOTS = 64;   // words the diagnostics' largest-index atomics are spread over

// Block retrieval (block.hip).
constexpr int BLK_MAX_D = 128;   // head dim limit
constexpr int BLK_MAXC = 2048;   // candidate keys per row: top_blocks * block_size

struct BlockArgs {
  int dtype;
  int B, T, H, D;
  int bs, nb, eb;            // block size, blocks, kept blocks min(top_blocks, nb)
  int mode;                  // 0 block_only, 1 block_token
  int kk;                    // block_token slots min(top_k, T)
  int ks;                    // block_only slots eb * bs
  int causal;
  int fill_invalid;          // write -FLT_MAX to blocks with no causal key (block scores are an output)
  const void* q;             // [B,T,H,D]
  const void* k;             // [B,T,H,D]
  float* block_scores;       // [B,H,nb,T] (block-major)
  int32_t* block_indices;    // [B,H,T,eb]
  int32_t* ncand;            // [B,H,T] candidate keys of each row
  float* bmargin;            // [B,H,T] block_only margin, or nullptr
  int32_t* slot_idx;         // [B,H,T,kk or ks]
  float* slot_sc;            // [B,H,T,kk or ks]
  uint8_t* slot_valid;       // [B,H,T,kk] (block_token)
  float* top2;               // [B,H,T,2]
  int32_t* counts;           // [B,H,T] slots handed to the gather
  // padding mask (nullptr: none): mask [B,T] nonzero = real token, for keys and queries alike
  const uint8_t* mask;
  int nmw;                   // 32-bit words per batch of mbits, ceil(T/32)
  int32_t* mpc;              // [B,T+1] valid keys before each position
  int32_t* mperm;            // [B,T] valid keys in ascending order
  int32_t* mnvb;             // [B,T] blocks holding a valid key the row sees (0 for a padded query)
  int32_t* mkqb;             // [T] kept blocks per position: min(eb, max(1, max over b of mnvb))
  uint32_t* mbits;           // [B,nmw] the mask as bits
};

hipError_t launch_block_select(const BlockArgs& a, hipStream_t st);

// RMSNorm of the model shells (norm.hip): x, y [rows, C] in dtype; weight [C] in dtype or fp32.
hipError_t launch_rms_norm(int dtype, int w_f32, long rows, int C, const void* x, const void* w, float eps, void* y,
                           hipStream_t st);
hipError_t launch_add_rms_norm(int dtype, int w_f32, long rows, int C, const void* a, const void* b, void* sum,
                               const void* w, float eps, void* y, hipStream_t st);
hipError_t launch_silu_mul(int dtype, const void* src, long stride, long rows, int I, void* y, hipStream_t st);
// y = x W^T (+ bias) on <= 16 bf16 rows (small_gemm.hip); with res, y = that rounded to bf16 plus res
// [M, N] (row stride rs), rounded again: a residual add after the product.  W row-major [N, K], or with
// tiled in launch_tile_rows' layout.
hipError_t launch_small_gemm(const void* x, long xs, const void* W, const void* bias, int M, int N, int K, void* y,
                             long ys, hipStream_t st, const void* res = nullptr, long rs = 0, bool tiled = false);
// W [N, K] row-major -> out [ceil(N / 16)][K / 32][64][8] (K a multiple of 32, rows past N zero): tile t,
// step s, lane l holds W[16t + l % 16][32s + 8 (l / 16) .. + 7], one wave step's operand in 1 KB.
hipError_t launch_tile_rows(const void* W, int N, int K, void* out, hipStream_t st);
// The SGSA decode projection's outputs (launch_small_gemm_split): bf16 q, k, v, q_ret [M, HD], the k and
// v rows of cache row pos ([M, cache_len, HD]) and the fp32 gates [M, H], as launch_decode_split writes them.
struct SgSplit {
  uint16_t *q, *k, *v, *qr;
  float *beta, *gamma, *budget;
  uint16_t *kc, *vc;
  long cache_len, pos, HD;
  int H;
};
// (W tiled, as for the swiglu form below)
hipError_t launch_small_gemm_split(const void* x, long xs, const void* W, const void* bias, int M, int N, int K,
                                   const SgSplit& sp, hipStream_t st);
// y [M, N / 2] = silu(gate) * up from a projection whose W rows interleave gate and up in groups of 8
// (W tiled: launch_tile_rows of the interleaved rows).
hipError_t launch_small_gemm_swiglu(const void* x, long xs, const void* W, int M, int N, int K, void* y, long ys,
                                    hipStream_t st);
// RoPE of a dense layer's q and k from the fused projection rows (norm.hip); k (and, with vo, the
// unrotated v heads after it) to rows koff .. of a [B, Hk, klen, D] buffer (klen < 0: T).
hipError_t launch_rope_qk(int dtype, const void* src, long stride, int B, int T, int Hq, int Hk, int D, int pos0,
                          const float* cosv, const float* sinv, void* qo, void* ko, hipStream_t st, long klen = -1,
                          long koff = 0, void* vo = nullptr);
// The SGSA layer's gates from the logit groups of a projection row (norm.hip).
hipError_t launch_gates(int dtype, const void* src, long stride, long rows, int H, float* beta, float* gamma,
                        float* budget, hipStream_t st);
hipError_t launch_decode_split(int dtype, const void* src, long stride, int B, int H, int D, void* q, void* k, void* v,
                               void* qr, float* beta, float* gamma, float* budget, void* kc, void* vc, long cache_len,
                               long pos, hipStream_t st);
size_t decode_attn_workspace_bytes(int dtype, int B, int H, int kend);
hipError_t launch_decode_attn(int dtype, int B, int H, int Hkv, const void* q, const void* kc, const void* vc,
                              long Tmax, int kend, void* out, void* ws, hipStream_t st);
hipError_t launch_block_scores_transpose(const float* src, int B, int H, int T, int nb, float* dst, hipStream_t st);
hipError_t launch_block_dense_weights(int B, int H, int T, int ks, const int32_t* idx, const float* w,
                                      const int32_t* counts, float* dense, hipStream_t st);
// The split-row gather's merge of each row, then K6 at T = 1 on its outputs, in one launch
// (bf16, D = 128, r.sparse_k / sparse_v / alpha = g.write_key or k_hat / v_hat / alpha).
hipError_t launch_merge_recurrent(const GatherArgs& g, const RecurrentArgs& r, hipStream_t st);
hipError_t launch_sparse_gather(const GatherArgs& a, hipStream_t st);
// Scores of given keys (top-k reuse across decode steps): scores[r, i] =
// (q_r . k[indices[r, i]]) * mscale for i < counts[r].
hipError_t launch_rescore(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, const void* q, const void* k,
                          const int32_t* indices, const int32_t* counts, float mscale, float* scores,
                          hipStream_t st);
// LDS-staged variant for the fused layer path: bf16, D = 128, rows whose
// slots [0, split) ascend in key index; no weights/diag outputs.
hipError_t launch_sparse_gather_staged(const GatherArgs& a, const int32_t* split, hipStream_t st);
// Layer path: the same kernel fed by the tile lists of the list-mode K1.
hipError_t launch_sparse_gather_lists(const GatherArgs& a, const uint2* tl_list, const int32_t* tl_off,
                                      hipStream_t st);
// Layer path, threshold form: the selection recomputed from q and each row's
// cut (score threshold, tie index) left by the threshold-mode K1.
hipError_t launch_sparse_gather_thr(const GatherArgs& a, const void* q, const uint2* thr, float mscale,
                                    hipStream_t st);
hipError_t launch_dense_attn(const void* q, const void* k, const void* v, int B, int H, int Hkv, int Tq, int pos0,
                             long L, float2* stats, void* out, hipStream_t st);

}  // namespace sgsa
