// sgsa_decode_stack: one decode step of the hybrid decoder's whole layer stack
// in one host call (include/sgsa.h states the contract).  The per-layer
// launches are the ones sgsa_amd.hybrid issues from Python for the same step
// -- the same kernels, arguments and order, so the results are the same bit
// for bit -- minus the Python dispatch around each of them: a step of the
// 24-layer stack is about 300 launches, whose host cost through torch and
// ctypes exceeded the GPU time of the kernels.  Four launches are folded into
// neighbours, with the same arithmetic: the SGSA projection's split (and its
// KV-cache row) into the projection's epilogue, the dense layer's KV-cache
// append into its RoPE launch, silu(gate) * up into the gate/up projection's
// epilogue (over gate and up rows interleaved in groups of 8), and the block's
// final residual add into the down projection's epilogue.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/sgsa.h"
#include "kernels.h"

namespace sgsa {
int abi_set_error(int status, const char* msg);
// sgsa_sparse_gather (no mask) then, with rec, sgsa_recurrent_fwd on its outputs (api.hip).
// With q, the slot scores are (q . k) * scale at the slots' keys, computed inside the
// split-row gather where its form allows (written to scores first otherwise); where the
// split form applies, the update runs in the launch that merges the split rows.  The results
// equal sgsa_score_at + sgsa_sparse_gather + sgsa_recurrent_fwd bit for bit.
int sparse_gather_stack(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, int q_offset, float scale,
                        int scale_mode, const void* q, const void* k, const void* v, const void* self_key,
                        const int32_t* indices, float* scores, const float* top2, const int32_t* counts,
                        const float* budget, int write_mode, float alpha_max, float tau_c, int local_window,
                        int sink_size, void* k_hat, void* v_hat, void* write_key, float* alpha, void* workspace,
                        size_t workspace_bytes, const RecurrentArgs* rec, void* stream);
}

namespace {

int fail(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return sgsa::abi_set_error(status, buf);
}

int hip_fail(hipError_t e, const char* where) {
  if (e == hipSuccess) return SGSA_OK;
  return fail(SGSA_ERR_HIP, "sgsa_decode_stack: %s: %s", where, hipGetErrorString(e));
}

size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

// Byte offsets of the step's intermediates in the workspace.
struct StackWs {
  size_t n, y, q, k, v, qr, beta, gamma, budget, tws, sc, top2, gws, wk, vh, alpha, o, aws, a, h2, n2, act, total;
  size_t tws_bytes, gws_bytes, aws_bytes;
};

int check_config(const SgsaDecodeConfig* c) {
  if (c == nullptr) return fail(SGSA_ERR_INVALID_ARG, "cfg must not be NULL");
  if (c->B < 1 || c->B > 16) return fail(SGSA_ERR_UNSUPPORTED, "sgsa_decode_stack: B=%d must be in [1, 16]", c->B);
  if (c->D != 128) return fail(SGSA_ERR_UNSUPPORTED, "sgsa_decode_stack: D=%d must be 128", c->D);
  if (c->H <= 0 || c->Hkv <= 0 || c->H % c->Hkv != 0) return fail(SGSA_ERR_INVALID_ARG, "H=%d Hkv=%d", c->H, c->Hkv);
  const int G = c->H / c->Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return fail(SGSA_ERR_UNSUPPORTED, "H / Hkv = %d not in {1, 2, 4, 8}", G);
  if (c->C <= 0 || c->C % 32 != 0 || c->I <= 0 || c->I % 32 != 0)
    return fail(SGSA_ERR_UNSUPPORTED, "C=%d and I=%d must be positive multiples of 32", c->C, c->I);
  if (c->top_k < 1) return fail(SGSA_ERR_INVALID_ARG, "top_k=%d", c->top_k);
  if (c->write_mode != 0 && c->write_mode != 1) return fail(SGSA_ERR_INVALID_ARG, "write_mode=%d", c->write_mode);
  if (c->cache_len < 1 || c->cache_len > 0x7fffffffL) return fail(SGSA_ERR_INVALID_ARG, "cache_len=%ld", c->cache_len);
  if (!(c->eps >= 0.f)) return fail(SGSA_ERR_INVALID_ARG, "eps must be >= 0");
  return SGSA_OK;
}

int stack_ws(const SgsaDecodeConfig& c, StackWs& w) {
  const size_t B = c.B, C = c.C, H = c.H, D = c.D, HD = H * D, I = c.I;
  const size_t n_sgsa = 4 * HD + 3 * H, n_dense = (H + 2 * (size_t)c.Hkv) * D;
  const size_t nin = n_sgsa > n_dense ? n_sgsa : n_dense;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = al256(off + bytes);
    return o;
  };
  w.n = take(B * C * 2);
  w.y = take(B * nin * 2);
  w.q = take(B * HD * 2);
  w.k = take(B * HD * 2);
  w.v = take(B * HD * 2);
  w.qr = take(B * HD * 2);
  w.beta = take(B * H * 4);
  w.gamma = take(B * H * 4);
  w.budget = take(B * H * 4);
  if (int s = sgsa_score_topk_fast_workspace_size(SGSA_BF16, c.B, 1, (int)c.cache_len, c.H, c.D, &w.tws_bytes)) return s;
  w.tws = take(w.tws_bytes);
  w.sc = take(B * H * (size_t)c.top_k * 4);
  w.top2 = take(B * H * 2 * 4);
  if (int s = sgsa_sparse_gather_workspace_size(c.B, 1, c.H, c.D, c.top_k, &w.gws_bytes)) return s;
  w.gws = take(w.gws_bytes);
  w.wk = take(B * HD * 2);
  w.vh = take(B * HD * 2);
  w.alpha = take(B * H * 4);
  w.o = take(B * HD * 2);
  if (int s = sgsa_decode_attention_workspace_size(SGSA_BF16, c.B, c.H, (int)c.cache_len, &w.aws_bytes)) return s;
  w.aws = take(w.aws_bytes);
  w.a = take(B * C * 2);
  w.h2 = take(B * C * 2);
  w.n2 = take(B * C * 2);
  w.act = take(B * I * 2);
  w.total = off;
  return SGSA_OK;
}

}  // namespace

extern "C" {

int sgsa_decode_stack_workspace_size(const SgsaDecodeConfig* cfg, size_t* bytes) {
  if (bytes == nullptr) return fail(SGSA_ERR_INVALID_ARG, "bytes must not be NULL");
  if (int s = check_config(cfg)) return s;
  StackWs w;
  if (int s = stack_ws(*cfg, w)) return s;
  *bytes = w.total;
  return SGSA_OK;
}

int sgsa_decode_stack(const SgsaDecodeConfig* cfg, int n_layers, const SgsaDecodeLayer* layers, void* h, int pos,
                      int select, void* workspace, size_t workspace_bytes, void* stream) {
  if (int s = check_config(cfg)) return s;
  const SgsaDecodeConfig& c = *cfg;
  if (n_layers < 0 || (n_layers > 0 && layers == nullptr)) return fail(SGSA_ERR_INVALID_ARG, "n_layers=%d", n_layers);
  if (pos < 0 || pos >= c.cache_len) return fail(SGSA_ERR_INVALID_ARG, "pos=%d must be in [0, cache_len=%ld)", pos, c.cache_len);
  if (pos + 1 < c.top_k)
    return fail(SGSA_ERR_UNSUPPORTED, "sgsa_decode_stack: pos + 1 = %d < top_k = %d (the candidate rows hold top_k slots)",
                pos + 1, c.top_k);
  if (h == nullptr) return fail(SGSA_ERR_INVALID_ARG, "h must not be NULL");
  StackWs w;
  if (int s = stack_ws(c, w)) return s;
  if (workspace == nullptr || (uintptr_t)workspace % 256 != 0 || workspace_bytes < w.total)
    return fail(SGSA_ERR_WORKSPACE, "sgsa_decode_stack: workspace of %zu bytes (256-byte aligned), need %zu",
                workspace_bytes, w.total);
  bool dense = false;
  for (int i = 0; i < n_layers; ++i) {
    const SgsaDecodeLayer& L = layers[i];
    if (L.kind != 0 && L.kind != 1) return fail(SGSA_ERR_INVALID_ARG, "layer %d: kind=%d", i, L.kind);
    if (!L.input_norm || !L.post_norm || !L.w_in || !L.w_o || !L.w_gu || !L.w_down || !L.k_cache || !L.v_cache)
      return fail(SGSA_ERR_INVALID_ARG, "layer %d: a weight or cache pointer is NULL", i);
    if (L.kind == 0 && (!L.state || !L.cand_idx || !L.cand_cnt))
      return fail(SGSA_ERR_INVALID_ARG, "layer %d: state, cand_idx and cand_cnt must be given", i);
    if (((uintptr_t)L.w_in | (uintptr_t)L.w_o | (uintptr_t)L.w_gu | (uintptr_t)L.w_down) % 16 != 0)
      return fail(SGSA_ERR_INVALID_ARG, "layer %d: weights must be 16-byte aligned", i);
    dense |= L.kind == 1;
  }
  if (dense && (c.rope_cos == nullptr || c.rope_sin == nullptr || c.rope_len <= pos))
    return fail(SGSA_ERR_INVALID_ARG, "dense layers need rope tables of more than pos=%d rows (rope_len=%d)", pos,
                c.rope_len);

  const hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const int B = c.B, C = c.C, H = c.H, Hkv = c.Hkv, D = c.D, I = c.I, HD = H * D;
  const int n_sgsa = 4 * HD + 3 * H, n_dense = (H + 2 * Hkv) * D;
  void* n = ws + w.n;
  void* y = ws + w.y;
  void* q = ws + w.q;
  void* k = ws + w.k;
  void* v = ws + w.v;
  void* qr = ws + w.qr;
  float* beta = (float*)(ws + w.beta);
  float* gamma = (float*)(ws + w.gamma);
  float* budget = (float*)(ws + w.budget);
  float* sc = (float*)(ws + w.sc);
  float* top2 = (float*)(ws + w.top2);
  void* wk = ws + w.wk;
  void* vh = ws + w.vh;
  float* alpha = (float*)(ws + w.alpha);
  void* o = ws + w.o;
  void* a = ws + w.a;
  void* h2 = ws + w.h2;
  void* n2 = ws + w.n2;
  void* act = ws + w.act;
  const float scale = sqrtf((float)D);

  for (int li = 0; li < n_layers; ++li) {
    const SgsaDecodeLayer& L = layers[li];
    if (hipError_t e = sgsa::launch_rms_norm(sgsa::DT_BF16, c.norm_w_f32, B, C, h, L.input_norm, c.eps, n, st))
      return hip_fail(e, "input norm");
    if (L.kind == 0) {
      // the projection, routed by its epilogue as sgsa_decode_split routes it
      sgsa::SgSplit sp{(uint16_t*)q, (uint16_t*)k, (uint16_t*)v, (uint16_t*)qr, beta, gamma, budget,
                       (uint16_t*)L.k_cache, (uint16_t*)L.v_cache, c.cache_len, pos, HD, H};
      if (hipError_t e = sgsa::launch_small_gemm_split(n, C, L.w_in, L.b_in, B, n_sgsa, C, sp, st))
        return hip_fail(e, "input projection");
      if (select) {
        if (int s = sgsa_score_topk(SGSA_BF16, B, 1, (int)c.cache_len, H, D, c.top_k, 1, pos, scale, 0, qr, L.k_cache,
                                    L.cand_idx, sc, top2, L.cand_cnt, nullptr, 0, ws + w.tws, w.tws_bytes, stream))
          return s;
      }
      // the gather (the kept candidates re-scored against this step's query inside it on
      // steps that keep them), then K6 on its outputs, the state updated in place
      sgsa::RecurrentArgs r{};
      r.dtype = sgsa::DT_BF16; r.B = B; r.T = 1; r.H = H; r.D = D;
      r.q = q; r.k = k; r.v = v; r.beta = beta; r.gamma = gamma;
      r.sparse_k = wk; r.sparse_v = vh; r.alpha = alpha;
      r.initial_state = L.state; r.out = o; r.final_state = L.state;
      if (int s = sgsa::sparse_gather_stack(SGSA_BF16, B, 1, (int)c.cache_len, H, D, c.top_k, pos, scale, 0,
                                            select ? nullptr : qr, L.k_cache, L.v_cache, k, L.cand_idx, sc,
                                            select ? top2 : nullptr, L.cand_cnt, budget, c.write_mode, c.alpha_max,
                                            c.tau_c, 64, 8, c.write_mode == 0 ? wk : nullptr, vh,
                                            c.write_mode == 1 ? wk : nullptr, alpha, ws + w.gws, w.gws_bytes, &r,
                                            stream))
        return s;
    } else {
      if (hipError_t e = sgsa::launch_small_gemm(n, C, L.w_in, L.b_in, B, n_dense, C, y, n_dense, st, nullptr, 0, true))
        return hip_fail(e, "input projection");
      if (hipError_t e = sgsa::launch_rope_qk(sgsa::DT_BF16, y, n_dense, B, 1, H, Hkv, D, pos, c.rope_cos, c.rope_sin, q,
                                              L.k_cache, st, c.cache_len, pos, L.v_cache))
        return hip_fail(e, "rope");
      if (int s = sgsa_decode_attention(SGSA_BF16, B, H, Hkv, D, q, L.k_cache, L.v_cache, c.cache_len, pos + 1, o,
                                        ws + w.aws, w.aws_bytes, stream))
        return s;
    }
    // the shell: h2 = h + o_proj(o), n2 = norm(h2), h = h2 + down(silu(gate(n2)) * up(n2))
    if (hipError_t e = sgsa::launch_small_gemm(o, HD, L.w_o, L.b_o, B, C, HD, a, C, st, nullptr, 0, true)) return hip_fail(e, "o projection");
    if (hipError_t e = sgsa::launch_add_rms_norm(sgsa::DT_BF16, c.norm_w_f32, B, C, h, a, h2, L.post_norm, c.eps, n2, st))
      return hip_fail(e, "post norm");
    if (hipError_t e = sgsa::launch_small_gemm_swiglu(n2, C, L.w_gu, B, 2 * I, C, act, I, st))
      return hip_fail(e, "gate/up projection");
    if (hipError_t e = sgsa::launch_small_gemm(act, I, L.w_down, nullptr, B, C, I, h, C, st, h2, C, true))
      return hip_fail(e, "down projection");
  }
  return SGSA_OK;
}

}  // extern "C"
