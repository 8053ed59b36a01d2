// C ABI of libsgsa_hip.so (declared in include/sgsa.h): argument validation,
// workspace carving and kernel dispatch.  Validation runs on the host before
// any HIP call, so the error paths are testable without a GPU.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <mutex>
#include <string>

#include "../../include/sgsa.h"
#include "kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}

int hip_status(hipError_t e, const char* where) {
  if (e == hipSuccess) return SGSA_OK;
  return fail(SGSA_ERR_HIP, "%s: %s", where, hipGetErrorString(e));
}

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) & ~(kAlign - 1); }

size_t dtype_size(int dtype) { return dtype == SGSA_F32 ? 4 : 2; }

int check_dtype(int dtype) {
  if (dtype != SGSA_F32 && dtype != SGSA_BF16) return fail(SGSA_ERR_INVALID_ARG, "dtype %d is not SGSA_F32 or SGSA_BF16", dtype);
  return SGSA_OK;
}

int check_dims(int B, int T, int H, int D) {
  if (B <= 0 || T <= 0 || H <= 0 || D <= 0) return fail(SGSA_ERR_INVALID_ARG, "shape B=%d T=%d H=%d D=%d must be positive", B, T, H, D);
  if (D > 128) return fail(SGSA_ERR_UNSUPPORTED, "head dim D=%d > 128 is not supported", D);
  if ((long)B * T * H * D > (1L << 40)) return fail(SGSA_ERR_UNSUPPORTED, "tensor too large");
  if ((long)B * T > 0x7fffffffL) return fail(SGSA_ERR_UNSUPPORTED, "B*T too large for 32-bit token indexing");
  return SGSA_OK;
}

#define REQUIRE(ptr) \
  do { if ((ptr) == nullptr) return fail(SGSA_ERR_INVALID_ARG, "%s must not be NULL", #ptr); } while (0)

struct LayerWs {
  size_t idx, sc, cnt, top2, split, wk, vh, al, misc, topk, chunk, total;
  bool thr;   // bf16, D = 128: K1 leaves per-row thresholds (idx region) for the threshold K2
};

LayerWs layer_ws(int dtype, int B, int T, int H, int D, int top_k) {
  LayerWs w{};
  const size_t rows = (size_t)B * H * T;
  const size_t kk = (size_t)(top_k < T ? top_k : T);
  size_t off = 0;
  // (the threshold gather addresses one head's keys with 32-bit byte offsets)
  w.thr = dtype == SGSA_BF16 && D == 128 && (long)T * H * D * 2 <= 0x7fffffffL;
  if (w.thr) {
    w.idx = off; off = align_up(off + rows * 8);
    w.sc = off;
  } else {
    w.idx = off; off = align_up(off + rows * kk * 4);
    w.sc = off; off = align_up(off + rows * kk * 4);
  }
  w.cnt = off; off = align_up(off + rows * 4);
  w.top2 = off; off = align_up(off + rows * 2 * 4);
  w.split = off; off = align_up(off + rows * 4);
  w.wk = off; off = align_up(off + (size_t)B * T * H * D * dtype_size(dtype));
  w.vh = off; off = align_up(off + (size_t)B * T * H * D * dtype_size(dtype));
  w.al = off; off = align_up(off + (size_t)B * T * H * 4);
  w.misc = off; off = align_up(off + 256);
  w.topk = off; off = align_up(off + sgsa::topk_workspace_bytes(B, T, H));
  w.chunk = off; off = align_up(off + sgsa::chunk_workspace_bytes(B, T, H, 1));
  w.total = off + kAlign;
  return w;
}

}  // namespace

extern "C" {

int sgsa_abi_version(void) { return SGSA_ABI_VERSION; }

const char* sgsa_status_string(int status) {
  switch (status) {
    case SGSA_OK: return "ok";
    case SGSA_ERR_INVALID_ARG: return "invalid argument";
    case SGSA_ERR_UNSUPPORTED: return "unsupported shape or option";
    case SGSA_ERR_HIP: return "HIP runtime error";
    case SGSA_ERR_WORKSPACE: return "workspace too small";
    default: return "unknown status";
  }
}

const char* sgsa_last_error(void) { return g_last_error.c_str(); }

}  // extern "C"

namespace sgsa {
// The last-error hook for entry points defined in other translation units.
int abi_set_error(int status, const char* msg) {
  g_last_error = msg;
  return status;
}
}  // namespace sgsa

extern "C" {

int sgsa_chunk_fwd_workspace_size(int B, int T, int H, int D, int has_sparse, size_t* bytes) {
  REQUIRE(bytes);
  if (int s = check_dims(B, T, H, D)) return s;
  *bytes = sgsa::chunk_workspace_bytes(B, T, H, has_sparse ? 1 : 0);
  return SGSA_OK;
}

int sgsa_chunk_fwd(int dtype, int B, int T, int H, int D, int chunk_size, const void* q, const void* k,
                   const void* v, const float* beta, const float* gamma, const void* sparse_k,
                   const void* sparse_v, const float* alpha, const float* initial_state, void* out,
                   float* final_state, void* workspace, size_t workspace_bytes, void* stream) {
  if (int s = check_dtype(dtype)) return s;
  if (int s = check_dims(B, T, H, D)) return s;
  if (chunk_size <= 0) return fail(SGSA_ERR_INVALID_ARG, "chunk_size=%d must be positive", chunk_size);
  REQUIRE(q); REQUIRE(k); REQUIRE(v); REQUIRE(beta); REQUIRE(gamma); REQUIRE(out); REQUIRE(workspace);
  const int nsp = (sparse_k != nullptr) + (sparse_v != nullptr) + (alpha != nullptr);
  if (nsp != 0 && nsp != 3) return fail(SGSA_ERR_INVALID_ARG, "sparse_k, sparse_v and alpha must be given together");
  const size_t need = sgsa::chunk_workspace_bytes(B, T, H, nsp == 3);
  if (workspace_bytes < need) return fail(SGSA_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, need);
  sgsa::ChunkArgs a{};
  a.dtype = dtype; a.B = B; a.T = T; a.H = H; a.D = D;
  a.q = q; a.k = k; a.v = v; a.beta = beta; a.gamma = gamma;
  a.sparse_k = nsp == 3 ? sparse_k : nullptr;
  a.sparse_v = nsp == 3 ? sparse_v : nullptr;
  a.alpha = nsp == 3 ? alpha : nullptr;
  a.initial_state = initial_state; a.out = out; a.final_state = final_state; a.workspace = workspace;
  return hip_status(sgsa::launch_chunk_fwd(a, (hipStream_t)stream), "sgsa_chunk_fwd");
}

int sgsa_chunk_bwd_workspace_size(int B, int T, int H, int D, int has_sparse, size_t* bytes) {
  if (int s = check_dims(B, T, H, D)) return s;
  REQUIRE(bytes);
  *bytes = sgsa::chunk_bwd_workspace_bytes(B, T, H, has_sparse != 0);
  return SGSA_OK;
}

int sgsa_chunk_bwd(int dtype, int B, int T, int H, int D, const void* q, const void* k, const void* v,
                   const float* beta, const float* gamma, const void* sparse_k, const void* sparse_v,
                   const float* alpha, const float* initial_state, const void* d_out, const float* d_final_state,
                   void* dq, void* dk, void* dv, float* dbeta, float* dgamma, void* dsparse_k, void* dsparse_v,
                   float* dalpha, float* d_initial_state, void* workspace, size_t workspace_bytes, void* stream) {
  if (int s = check_dtype(dtype)) return s;
  if (int s = check_dims(B, T, H, D)) return s;
  REQUIRE(q); REQUIRE(k); REQUIRE(v); REQUIRE(beta); REQUIRE(gamma); REQUIRE(d_out);
  REQUIRE(dq); REQUIRE(dk); REQUIRE(dv); REQUIRE(dbeta); REQUIRE(dgamma); REQUIRE(workspace);
  const int nsp = (sparse_k != nullptr) + (sparse_v != nullptr) + (alpha != nullptr);
  if (nsp != 0 && nsp != 3) return fail(SGSA_ERR_INVALID_ARG, "sparse_k, sparse_v and alpha must be given together");
  if (nsp == 3 && (dsparse_k == nullptr || dsparse_v == nullptr || dalpha == nullptr))
    return fail(SGSA_ERR_INVALID_ARG, "the sparse write needs dsparse_k, dsparse_v and dalpha outputs");
  if ((long)T * H > 0x7fffffffL) return fail(SGSA_ERR_UNSUPPORTED, "T*H too large");
  const size_t need = sgsa::chunk_bwd_workspace_bytes(B, T, H, nsp == 3);
  if (workspace_bytes < need) return fail(SGSA_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, need);
  sgsa::ChunkBwdArgs a{};
  a.f.dtype = dtype; a.f.B = B; a.f.T = T; a.f.H = H; a.f.D = D;
  a.f.q = q; a.f.k = k; a.f.v = v; a.f.beta = beta; a.f.gamma = gamma;
  a.f.sparse_k = nsp == 3 ? sparse_k : nullptr;
  a.f.sparse_v = nsp == 3 ? sparse_v : nullptr;
  a.f.alpha = nsp == 3 ? alpha : nullptr;
  a.f.initial_state = initial_state;
  a.d_out = d_out; a.d_final_state = d_final_state;
  a.dq = dq; a.dk = dk; a.dv = dv; a.dbeta = dbeta; a.dgamma = dgamma;
  a.dsk = nsp == 3 ? dsparse_k : nullptr;
  a.dsv = nsp == 3 ? dsparse_v : nullptr;
  a.dalpha = nsp == 3 ? dalpha : nullptr;
  a.d_initial_state = d_initial_state;
  a.workspace = workspace;
  return hip_status(sgsa::launch_chunk_bwd(a, (hipStream_t)stream), "sgsa_chunk_bwd");
}

static int validate_topk(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, int scale_mode, float scale) {
  if (int s = check_dtype(dtype)) return s;
  if (int s = check_dims(B, Tq, H, D)) return s;
  if (int s = check_dims(B, Tk, H, D)) return s;
  if (top_k <= 0) return fail(SGSA_ERR_INVALID_ARG, "top_k=%d must be positive", top_k);
  if (top_k > Tk) return fail(SGSA_ERR_INVALID_ARG, "top_k=%d exceeds the key length %d (pass min(top_k, Tk))", top_k, Tk);
  if (scale_mode != 0 && scale_mode != 1) return fail(SGSA_ERR_INVALID_ARG, "scale_mode must be 0 (divide) or 1 (multiply)");
  if (!(scale > 0.f) || !isfinite(scale)) return fail(SGSA_ERR_INVALID_ARG, "scale must be positive and finite");
  return SGSA_OK;
}

int sgsa_recurrent_fwd(int dtype, int B, int T, int H, int D, const void* q, const void* k, const void* v,
                       const float* beta, const float* gamma, const void* sparse_k, const void* sparse_v,
                       const float* alpha, const float* initial_state, void* out, float* final_state, void* stream) {
  if (int s = check_dtype(dtype)) return s;
  if (int s = check_dims(B, T, H, D)) return s;
  REQUIRE(q); REQUIRE(k); REQUIRE(v); REQUIRE(beta); REQUIRE(gamma); REQUIRE(out);
  const int ns = (sparse_k != nullptr) + (sparse_v != nullptr) + (alpha != nullptr);
  if (ns != 0 && ns != 3) return fail(SGSA_ERR_INVALID_ARG, "sparse_k, sparse_v and alpha must be given together");
  sgsa::RecurrentArgs a{};
  a.dtype = dtype; a.B = B; a.T = T; a.H = H; a.D = D;
  a.q = q; a.k = k; a.v = v; a.beta = beta; a.gamma = gamma;
  a.sparse_k = sparse_k; a.sparse_v = sparse_v; a.alpha = alpha;
  a.initial_state = initial_state; a.out = out; a.final_state = final_state;
  return hip_status(sgsa::launch_recurrent(a, (hipStream_t)stream), "sgsa_recurrent_fwd");
}

int sgsa_score_topk_workspace_size(int B, int Tq, int H, size_t* bytes) {
  REQUIRE(bytes);
  if (int s = check_dims(B, Tq, H, 1)) return s;
  *bytes = sgsa::topk_workspace_bytes(B, Tq, H);
  return SGSA_OK;
}

}  // extern "C"

namespace {

// Argument checks of sgsa_score_topk other than the workspace.
int score_topk_check(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, int q_offset, float scale,
                     int scale_mode, const void* q, const void* k, const int32_t* indices, const float* scores,
                     const int32_t* counts, const int32_t* split, int sorted) {
  if (int s = validate_topk(dtype, B, Tq, Tk, H, D, top_k, scale_mode, scale)) return s;
  REQUIRE(q); REQUIRE(k); REQUIRE(indices); REQUIRE(scores);
  if (sorted && counts == nullptr) return fail(SGSA_ERR_INVALID_ARG, "sorted output needs counts");
  if (sorted && split != nullptr) return fail(SGSA_ERR_INVALID_ARG, "split describes the unsorted order; pass NULL with sorted=1");
  if (q_offset < 0) return fail(SGSA_ERR_INVALID_ARG, "q_offset must be >= 0");
  if (top_k > 4096 && sorted) return fail(SGSA_ERR_UNSUPPORTED, "sorted output supports top_k <= 4096");
  return SGSA_OK;
}

// The launches of sgsa_score_topk on a checked workspace: the few-row form when the
// workspace holds its score buffer (and is 256-byte aligned), the row kernel otherwise.
int score_topk_launch(const sgsa::TopkArgs& a0, int sorted, void* workspace, size_t workspace_bytes,
                      hipStream_t st) {
  sgsa::TopkArgs a = a0;
  a.workspace = workspace;
  const size_t base_ws = (sgsa::topk_workspace_bytes(a.B, a.Tq, a.H) + 255) & ~(size_t)255;
  const size_t rows_ws = sgsa::topk_rows_bytes(a);
  if (rows_ws > 0 && workspace_bytes >= base_ws + rows_ws && ((uintptr_t)workspace & 255u) == 0) {
    float* sbuf = reinterpret_cast<float*>(static_cast<char*>(workspace) + base_ws);
    if (int s = hip_status(sgsa::launch_score_topk_rows(a, sbuf, st), "sgsa_score_topk (few rows)")) return s;
  } else if (int s = hip_status(sgsa::launch_score_topk(a, st), "sgsa_score_topk")) {
    return s;
  }
  if (sorted)
    return hip_status(sgsa::launch_sort_rows(a.indices, a.scores, (long)a.B * a.H * a.Tq, a.top_k, a.counts, st),
                      "sgsa_score_topk(sort)");
  return SGSA_OK;
}

sgsa::TopkArgs score_topk_args(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, int causal, int q_offset,
                               float scale, int scale_mode, const void* q, const void* k, int32_t* indices,
                               float* scores, float* top2, int32_t* counts, int32_t* split) {
  sgsa::TopkArgs a{};
  a.dtype = dtype; a.B = B; a.Tq = Tq; a.Tk = Tk; a.H = H; a.D = D; a.top_k = top_k;
  a.causal = causal ? 1 : 0; a.q_offset = q_offset; a.scale = scale; a.scale_mode = scale_mode;
  a.q = q; a.k = k; a.indices = indices; a.scores = scores; a.top2 = top2; a.counts = counts; a.split = split;
  return a;
}

// ---- scratch of the allocation-free entry point ------------------------------
// One array per GPU, held until the process ends.  Host code never passes the
// array's name to a kernel or a copy (in host code it is a stand-in, not a device
// address): it uses the per-device address hipGetSymbolAddress returns.
static __device__ __align__(256) unsigned char scratch[SGSA_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of the scratch array, looked up once per device
// with that device current.
int scratch_address(void** out) {
  int dev = -1;
  if (int s = hip_status(hipGetDevice(&dev), "sgsa_score_topk_noalloc (hipGetDevice)")) return s;
  if (dev < 0 || dev >= kMaxDevices) return fail(SGSA_ERR_UNSUPPORTED, "device ordinal %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (int s = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "sgsa_score_topk_noalloc (hipGetSymbolAddress)"))
      return s;
    if (p == nullptr || ((uintptr_t)p & 255u) != 0)
      return fail(SGSA_ERR_HIP, "sgsa_score_topk_noalloc: scratch address %p is not 256-byte aligned", p);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SGSA_OK;
}

}  // namespace

extern "C" {

int sgsa_score_topk(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, int causal, int q_offset,
                    float scale, int scale_mode, const void* q, const void* k, int32_t* indices, float* scores,
                    float* top2, int32_t* counts, int32_t* split, int sorted, void* workspace,
                    size_t workspace_bytes, void* stream) {
  if (int s = score_topk_check(dtype, B, Tq, Tk, H, D, top_k, q_offset, scale, scale_mode, q, k, indices, scores,
                               counts, split, sorted))
    return s;
  REQUIRE(workspace);
  const size_t need_ws = sgsa::topk_workspace_bytes(B, Tq, H);
  if (workspace_bytes < need_ws) return fail(SGSA_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, need_ws);
  const sgsa::TopkArgs a = score_topk_args(dtype, B, Tq, Tk, H, D, top_k, causal, q_offset, scale, scale_mode, q, k,
                                           indices, scores, top2, counts, split);
  return score_topk_launch(a, sorted, workspace, workspace_bytes, (hipStream_t)stream);
}

int sgsa_score_topk_noalloc(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, int causal, int q_offset,
                            float scale, int scale_mode, const void* q, const void* k, int32_t* indices,
                            float* scores, float* top2, int32_t* counts, int32_t* split, int sorted, void* stream) {
  if (int s = score_topk_check(dtype, B, Tq, Tk, H, D, top_k, q_offset, scale, scale_mode, q, k, indices, scores,
                               counts, split, sorted))
    return s;
  const sgsa::TopkArgs a = score_topk_args(dtype, B, Tq, Tk, H, D, top_k, causal, q_offset, scale, scale_mode, q, k,
                                           indices, scores, top2, counts, split);
  // the workspace sgsa_score_topk_fast_workspace_size asks for: the few-row form where it applies
  const size_t base_ws = (sgsa::topk_workspace_bytes(B, Tq, H) + 255) & ~(size_t)255;
  const size_t need = base_ws + sgsa::topk_rows_bytes(a);
  if (need > (size_t)SGSA_NOALLOC_SCRATCH_BYTES)
    return fail(SGSA_ERR_WORKSPACE,
                "sgsa_score_topk_noalloc: B=%d Tq=%d Tk=%d H=%d needs %zu bytes of scratch; its fixed scratch holds "
                "%zu (SGSA_NOALLOC_SCRATCH_BYTES); use sgsa_score_topk with a workspace", B, Tq, Tk, H, need,
                (size_t)SGSA_NOALLOC_SCRATCH_BYTES);
  void* ptr = nullptr;
  if (int s = scratch_address(&ptr)) return s;
  return score_topk_launch(a, sorted, ptr, need, (hipStream_t)stream);
}

int sgsa_score_topk_fast_workspace_size(int dtype, int B, int Tq, int Tk, int H, int D, size_t* bytes) {
  if (int s = check_dtype(dtype)) return s;
  if (int s = check_dims(B, Tq, H, D)) return s;
  if (int s = check_dims(B, Tk, H, D)) return s;
  REQUIRE(bytes);
  sgsa::TopkArgs a{};
  a.dtype = dtype; a.B = B; a.Tq = Tq; a.Tk = Tk; a.H = H; a.D = D;
  static const uint4 probe{};   // aligned stand-ins: the form also needs 16-byte aligned q and k
  a.q = &probe; a.k = &probe;
  const size_t need_ws = (sgsa::topk_workspace_bytes(B, Tq, H) + 255) & ~(size_t)255;
  *bytes = need_ws + sgsa::topk_rows_bytes(a);
  return SGSA_OK;
}

int sgsa_score_topk_masked_workspace_size(int dtype, int B, int Tq, int Tk, int H, int D, int has_key_mask,
                                          int kv_layout, size_t* bytes) {
  if (int s = check_dtype(dtype)) return s;
  if (int s = check_dims(B, Tq, H, D)) return s;
  if (int s = check_dims(B, Tk, H, D)) return s;
  REQUIRE(bytes);
  const int compact = (has_key_mask != 0 || kv_layout == 1) ? 1 : 0;
  *bytes = align_up(sgsa::mask_workspace_bytes(dtype, B, Tq, Tk, H, D, compact)) +
           align_up(sgsa::topk_workspace_bytes(B, Tq, H)) + kAlign;
  return SGSA_OK;
}

int sgsa_score_topk_masked(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, int causal, int q_offset,
                           float scale, int scale_mode, int kq_rule, int kv_layout, const void* q, const void* k,
                           const uint8_t* key_mask, const uint8_t* query_mask, int32_t* indices, float* scores,
                           uint8_t* slot_valid, float* top2, int32_t* counts, int32_t* fill, int sorted,
                           void* workspace, size_t workspace_bytes, void* stream) {
  if (int s = score_topk_check(dtype, B, Tq, Tk, H, D, top_k, q_offset, scale, scale_mode, q, k, indices, scores,
                               counts, nullptr, sorted))
    return s;
  REQUIRE(counts); REQUIRE(workspace);
  if (kq_rule != 0 && kq_rule != 1) return fail(SGSA_ERR_INVALID_ARG, "kq_rule must be 0 (retriever) or 1 (fixed top_k)");
  if (kv_layout != 0 && kv_layout != 1) return fail(SGSA_ERR_INVALID_ARG, "kv_layout must be 0 ([B,Tk,H,D]) or 1 ([B,H,Tk,D])");
  if ((long)B * (Tk + 1) > 0x7fffffffL) return fail(SGSA_ERR_UNSUPPORTED, "B*(Tk+1) too large for 32-bit key counts");
  size_t need = 0;
  if (int s = sgsa_score_topk_masked_workspace_size(dtype, B, Tq, Tk, H, D, key_mask != nullptr, kv_layout, &need))
    return s;
  if (workspace_bytes < need) return fail(SGSA_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, need);
  const hipStream_t st = (hipStream_t)stream;
  char* base = reinterpret_cast<char*>(((uintptr_t)workspace + kAlign - 1) & ~(uintptr_t)(kAlign - 1));
  sgsa::MaskArgs m{};
  m.dtype = dtype; m.B = B; m.Tq = Tq; m.Tk = Tk; m.H = H; m.D = D;
  m.causal = causal ? 1 : 0; m.q_offset = q_offset; m.top_k = top_k; m.kq_rule = kq_rule; m.kv_hm = kv_layout;
  m.compacted = (key_mask != nullptr || kv_layout == 1) ? 1 : 0;
  m.key_mask = key_mask; m.query_mask = query_mask; m.k = k;
  sgsa::mask_carve(m, base);
  if (int s = hip_status(sgsa::launch_mask_prepare(m, st), "sgsa_score_topk_masked (mask)")) return s;
  sgsa::TopkArgs a = score_topk_args(dtype, B, Tq, Tk, H, D, top_k, causal, q_offset, scale, scale_mode, q,
                                     m.compacted ? m.kc : k, indices, scores, top2, counts, nullptr);
  a.row_nv = m.nv;
  a.row_kq = m.kq;
  a.workspace = base + align_up(sgsa::mask_workspace_bytes(dtype, B, Tq, Tk, H, D, m.compacted));
  if (int s = hip_status(sgsa::launch_score_topk(a, st), "sgsa_score_topk_masked")) return s;
  if (sorted) {   // (score desc, index asc): the compaction keeps the index order
    if (int s = hip_status(sgsa::launch_sort_rows(indices, scores, (long)B * H * Tq, top_k, counts, st),
                           "sgsa_score_topk_masked (sort)"))
      return s;
  }
  return hip_status(sgsa::launch_mask_finish(m, indices, scores, slot_valid, counts, fill, st),
                    "sgsa_score_topk_masked (finish)");
}

int sgsa_topk_lists_size(int B, int T, int H, int top_k, size_t* list_bytes, size_t* offset_bytes) {
  REQUIRE(list_bytes); REQUIRE(offset_bytes);
  if (int s = check_dims(B, T, H, 1)) return s;
  if (top_k <= 0) return fail(SGSA_ERR_INVALID_ARG, "top_k=%d must be positive", top_k);
  const int kk = top_k < T ? top_k : T;
  *list_bytes = sgsa::topk_list_bytes(B, T, H, kk);
  *offset_bytes = sgsa::topk_list_off_bytes(B, T, T, H);
  return SGSA_OK;
}

int sgsa_score_topk_lists(int B, int T, int H, int D, int top_k, const void* q, const void* k, void* lists,
                          int32_t* offsets, float* top2, int32_t* counts, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (int s = check_dims(B, T, H, D)) return s;
  if (top_k <= 0) return fail(SGSA_ERR_INVALID_ARG, "top_k=%d must be positive", top_k);
  REQUIRE(q); REQUIRE(k); REQUIRE(lists); REQUIRE(offsets); REQUIRE(top2); REQUIRE(counts); REQUIRE(workspace);
  const size_t need_ws = sgsa::topk_workspace_bytes(B, T, H);
  if (workspace_bytes < need_ws) return fail(SGSA_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, need_ws);
  sgsa::TopkArgs a{};
  a.dtype = SGSA_BF16; a.B = B; a.Tq = T; a.Tk = T; a.H = H; a.D = D; a.top_k = top_k < T ? top_k : T;
  a.causal = 1; a.q_offset = 0; a.scale = (float)sqrt((double)D); a.scale_mode = 0;
  a.q = q; a.k = k; a.top2 = top2; a.counts = counts;
  a.tl_list = reinterpret_cast<uint2*>(lists); a.tl_off = offsets;
  a.workspace = workspace;
  return hip_status(sgsa::launch_score_topk(a, (hipStream_t)stream), "sgsa_score_topk_lists");
}

int sgsa_sparse_gather_lists(int B, int T, int H, int D, int top_k, const void* k, const void* v, const void* lists,
                             const int32_t* offsets, const float* top2, const int32_t* counts, const float* budget,
                             int write_mode, float alpha_max, float tau_c, void* k_hat, void* v_hat,
                             void* write_key, float* alpha, void* stream) {
  if (int s = check_dims(B, T, H, D)) return s;
  if (D != 128) return fail(SGSA_ERR_UNSUPPORTED, "the tiled gather needs D == 128 (got %d)", D);
  if (top_k <= 0) return fail(SGSA_ERR_INVALID_ARG, "top_k=%d must be positive", top_k);
  REQUIRE(k); REQUIRE(v); REQUIRE(lists); REQUIRE(offsets); REQUIRE(top2); REQUIRE(counts); REQUIRE(v_hat);
  if (write_mode != 0 && write_mode != 1) return fail(SGSA_ERR_INVALID_ARG, "write_mode must be 0 (direct) or 1 (residual)");
  if (budget != nullptr && alpha == nullptr) return fail(SGSA_ERR_INVALID_ARG, "the write gate needs an alpha output");
  if (write_mode == 1 && budget != nullptr && write_key == nullptr)
    return fail(SGSA_ERR_INVALID_ARG, "residual write mode needs a write_key output");
  sgsa::GatherArgs g{};
  g.dtype = SGSA_BF16; g.B = B; g.Tq = T; g.Tk = T; g.H = H; g.D = D; g.top_k = top_k < T ? top_k : T;
  g.q_offset = 0; g.k = k; g.v = v; g.self_key = k; g.top2 = top2; g.counts = counts;
  g.use_valid = 1; g.tau_c = tau_c; g.eps = 1e-6f; g.budget = budget; g.write_mode = write_mode;
  g.alpha_max = alpha_max; g.k_hat = k_hat; g.v_hat = v_hat; g.write_key = write_key; g.alpha = alpha;
  return hip_status(sgsa::launch_sparse_gather_lists(g, reinterpret_cast<const uint2*>(lists), offsets,
                                                     (hipStream_t)stream),
                    "sgsa_sparse_gather_lists");
}

int sgsa_score_topk_thresholds(int B, int T, int H, int D, int top_k, const void* q, const void* k, void* thr,
                               float* top2, int32_t* counts, void* workspace, size_t workspace_bytes,
                               void* stream) {
  if (int s = check_dims(B, T, H, D)) return s;
  if (D != 128) return fail(SGSA_ERR_UNSUPPORTED, "the threshold form needs D == 128 (got %d)", D);
  if (top_k <= 0) return fail(SGSA_ERR_INVALID_ARG, "top_k=%d must be positive", top_k);
  REQUIRE(q); REQUIRE(k); REQUIRE(thr); REQUIRE(top2); REQUIRE(counts); REQUIRE(workspace);
  const size_t need_ws = sgsa::topk_workspace_bytes(B, T, H);
  if (workspace_bytes < need_ws) return fail(SGSA_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, need_ws);
  sgsa::TopkArgs a{};
  a.dtype = SGSA_BF16; a.B = B; a.Tq = T; a.Tk = T; a.H = H; a.D = D; a.top_k = top_k < T ? top_k : T;
  a.causal = 1; a.q_offset = 0; a.scale = (float)sqrt((double)D); a.scale_mode = 0;
  a.q = q; a.k = k; a.top2 = top2; a.counts = counts; a.thr = reinterpret_cast<uint2*>(thr);
  a.workspace = workspace;
  return hip_status(sgsa::launch_score_topk(a, (hipStream_t)stream), "sgsa_score_topk_thresholds");
}

int sgsa_sparse_gather_thresholds(int B, int T, int H, int D, int top_k, const void* q, const void* k,
                                  const void* v, const void* thr, const float* top2, const int32_t* counts,
                                  const float* budget, int write_mode, float alpha_max, float tau_c, void* k_hat,
                                  void* v_hat, void* write_key, float* alpha, void* stream) {
  if (int s = check_dims(B, T, H, D)) return s;
  if (D != 128) return fail(SGSA_ERR_UNSUPPORTED, "the threshold form needs D == 128 (got %d)", D);
  if (top_k <= 0) return fail(SGSA_ERR_INVALID_ARG, "top_k=%d must be positive", top_k);
  if ((long)T * H * D * 2 > 0x7fffffffL) return fail(SGSA_ERR_UNSUPPORTED, "one head's keys exceed 2 GiB of offsets");
  REQUIRE(q); REQUIRE(k); REQUIRE(v); REQUIRE(thr); REQUIRE(top2); REQUIRE(counts); REQUIRE(v_hat);
  if (write_mode != 0 && write_mode != 1) return fail(SGSA_ERR_INVALID_ARG, "write_mode must be 0 (direct) or 1 (residual)");
  if (budget != nullptr && alpha == nullptr) return fail(SGSA_ERR_INVALID_ARG, "the write gate needs an alpha output");
  if (write_mode == 1 && budget != nullptr && write_key == nullptr)
    return fail(SGSA_ERR_INVALID_ARG, "residual write mode needs a write_key output");
  sgsa::GatherArgs g{};
  g.dtype = SGSA_BF16; g.B = B; g.Tq = T; g.Tk = T; g.H = H; g.D = D; g.top_k = top_k < T ? top_k : T;
  g.q_offset = 0; g.k = k; g.v = v; g.self_key = k; g.top2 = top2; g.counts = counts;
  g.use_valid = 1; g.tau_c = tau_c; g.eps = 1e-6f; g.budget = budget; g.write_mode = write_mode;
  g.alpha_max = alpha_max; g.k_hat = k_hat; g.v_hat = v_hat; g.write_key = write_key; g.alpha = alpha;
  const float ms = sgsa::score_multiplier((float)sqrt((double)D), 0);
  return hip_status(sgsa::launch_sparse_gather_thr(g, q, reinterpret_cast<const uint2*>(thr), ms, (hipStream_t)stream),
                    "sgsa_sparse_gather_thresholds");
}

int sgsa_gather_thresholds_selection(int B, int T, int H, int D, int top_k, const void* q, const void* k,
                                     const void* v, const void* thr, const float* top2, const int32_t* counts,
                                     int32_t* selection, void* stream) {
  if (int s = check_dims(B, T, H, D)) return s;
  if (D != 128) return fail(SGSA_ERR_UNSUPPORTED, "the threshold form needs D == 128 (got %d)", D);
  if (top_k <= 0) return fail(SGSA_ERR_INVALID_ARG, "top_k=%d must be positive", top_k);
  if ((long)T * H * D * 2 > 0x7fffffffL) return fail(SGSA_ERR_UNSUPPORTED, "one head's keys exceed 2 GiB of offsets");
  REQUIRE(q); REQUIRE(k); REQUIRE(v); REQUIRE(thr); REQUIRE(top2); REQUIRE(counts); REQUIRE(selection);
  sgsa::GatherArgs g{};
  g.dtype = SGSA_BF16; g.B = B; g.Tq = T; g.Tk = T; g.H = H; g.D = D; g.top_k = top_k < T ? top_k : T;
  g.q_offset = 0; g.k = k; g.v = v; g.self_key = k; g.top2 = top2; g.counts = counts;
  g.use_valid = 1; g.eps = 1e-6f; g.sel_dbg = selection;
  const float ms = sgsa::score_multiplier((float)sqrt((double)D), 0);
  return hip_status(sgsa::launch_sparse_gather_thr(g, q, reinterpret_cast<const uint2*>(thr), ms, (hipStream_t)stream),
                    "sgsa_gather_thresholds_selection");
}

int sgsa_score_dump(int dtype, int B, int Tq, int Tk, int H, int D, int causal, int q_offset, float scale,
                    int scale_mode, const void* q, const void* k, int row0, int rows, float* out, void* stream) {
  if (int s = validate_topk(dtype, B, Tq, Tk, H, D, 1, scale_mode, scale)) return s;
  REQUIRE(q); REQUIRE(k); REQUIRE(out);
  if (row0 < 0 || rows <= 0 || row0 + rows > Tq) return fail(SGSA_ERR_INVALID_ARG, "row range [%d,%d) outside [0,%d)", row0, row0 + rows, Tq);
  sgsa::TopkArgs a{};
  a.dtype = dtype; a.B = B; a.Tq = Tq; a.Tk = Tk; a.H = H; a.D = D; a.top_k = 1;
  a.causal = causal ? 1 : 0; a.q_offset = q_offset; a.scale = scale; a.scale_mode = scale_mode;
  a.q = q; a.k = k; a.dump = out; a.dump_row0 = row0; a.dump_rows = rows;
  return hip_status(sgsa::launch_score_topk(a, (hipStream_t)stream), "sgsa_score_dump");
}

int sgsa_sparse_gather(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, int q_offset, const void* k,
                       const void* v, const void* self_key, const int32_t* indices, const float* scores,
                       const float* top2, const int32_t* counts, const float* budget, int write_mode,
                       float alpha_max, float tau_c, int local_window, int sink_size, void* k_hat, void* v_hat,
                       void* write_key, float* alpha, float* weights, float* diag, void* workspace,
                       size_t workspace_bytes, void* stream) {
  return sgsa_sparse_gather_masked(dtype, B, Tq, Tk, H, D, top_k, q_offset, 0, k, v, self_key, indices, scores,
                                   nullptr, top2, counts, budget, write_mode, alpha_max, tau_c, local_window,
                                   sink_size, k_hat, v_hat, write_key, alpha, weights, diag, nullptr, workspace,
                                   workspace_bytes, stream);
}

// sgsa_sparse_gather_masked; with rq, the slot scores are (rq . k) * rq_ms at the slots' keys,
// computed inside the split-row gather where its form allows (bf16, D = 128, [B,Tk,H,D], no slot
// mask), else by launch_rescore into scores first: the same values either way.
static int sparse_gather_impl(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, int q_offset,
                              int kv_layout, const void* k, const void* v, const void* self_key,
                              const int32_t* indices, const float* scores, const uint8_t* slot_valid,
                              const float* top2, const int32_t* counts, const float* budget, int write_mode,
                              float alpha_max, float tau_c, int local_window, int sink_size, void* k_hat,
                              void* v_hat, void* write_key, float* alpha, float* weights, float* diag,
                              float* row_stats, void* workspace, size_t workspace_bytes, void* stream,
                              const void* rq, float rq_ms, const sgsa::RecurrentArgs* rec = nullptr) {
  if (kv_layout != 0 && kv_layout != 1) return fail(SGSA_ERR_INVALID_ARG, "kv_layout must be 0 ([B,Tk,H,D]) or 1 ([B,H,Tk,D])");
  if (int s = check_dtype(dtype)) return s;
  if (int s = check_dims(B, Tq, H, D)) return s;
  if (int s = check_dims(B, Tk, H, D)) return s;
  if (top_k <= 0) return fail(SGSA_ERR_INVALID_ARG, "top_k=%d must be positive", top_k);
  REQUIRE(v); REQUIRE(indices); REQUIRE(scores); REQUIRE(counts); REQUIRE(v_hat);
  if (write_mode != 0 && write_mode != 1) return fail(SGSA_ERR_INVALID_ARG, "write_mode must be 0 (direct) or 1 (residual)");
  if ((diag != nullptr || budget != nullptr) && self_key == nullptr)
    return fail(SGSA_ERR_INVALID_ARG, "self_key is required for diagnostics and for the write gate");
  if ((diag != nullptr || budget != nullptr) && k == nullptr)
    return fail(SGSA_ERR_INVALID_ARG, "diagnostics and the write gate need k (the K gather)");
  if (k_hat != nullptr && k == nullptr) return fail(SGSA_ERR_INVALID_ARG, "k_hat requested without k");
  if (budget != nullptr && (alpha == nullptr)) return fail(SGSA_ERR_INVALID_ARG, "the write gate needs an alpha output");
  if (write_mode == 1 && budget != nullptr && write_key == nullptr)
    return fail(SGSA_ERR_INVALID_ARG, "residual write mode needs a write_key output");
  if (diag != nullptr && (workspace == nullptr || workspace_bytes < 256))
    return fail(SGSA_ERR_WORKSPACE, "diagnostics need a workspace of at least 256 bytes");
  sgsa::GatherArgs a{};
  a.dtype = dtype; a.B = B; a.Tq = Tq; a.Tk = Tk; a.H = H; a.D = D; a.top_k = top_k; a.q_offset = q_offset;
  a.k = k; a.v = v; a.kv_hm = kv_layout; a.self_key = self_key; a.indices = indices; a.scores = scores; a.top2 = top2; a.counts = counts;
  a.slot_valid = slot_valid;
  a.use_valid = 1; a.tau_c = tau_c; a.eps = 1e-6f; a.local_window = local_window; a.sink_size = sink_size;
  a.budget = budget; a.write_mode = write_mode; a.alpha_max = alpha_max;
  a.k_hat = k_hat; a.v_hat = v_hat; a.write_key = write_key; a.alpha = alpha; a.weights = weights; a.diag = diag;
  a.stats = row_stats;
  a.max_index = diag ? (int32_t*)workspace : nullptr;
  const long rows = (long)B * H * Tq;
  const size_t pb = sgsa::gather_part_bytes(rows, top_k, D);
  if (pb > 0 && workspace != nullptr && workspace_bytes >= 256 + pb) {
    a.nsplit = sgsa::gather_nsplit(rows, top_k);
    a.split_len = sgsa::GATHER_SPLIT_LEN;
    a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + 256);
  }
  if (rq != nullptr) {
    auto aligned = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
    if (dtype == SGSA_BF16 && D == 128 && kv_layout == 0 && slot_valid == nullptr && a.nsplit > 0 && k != nullptr &&
        aligned(k) && aligned(v) && aligned(rq) && (self_key == nullptr || aligned(self_key))) {
      a.rq = rq;
      a.rq_ms = rq_ms;
    } else if (int s = hip_status(sgsa::launch_rescore(dtype, B, Tq, Tk, H, D, top_k, rq, k, indices, counts, rq_ms,
                                                       const_cast<float*>(scores), (hipStream_t)stream),
                                  "sgsa_sparse_gather (scores)")) {
      return s;
    }
  }
  if (rec == nullptr) return hip_status(sgsa::launch_sparse_gather(a, (hipStream_t)stream), "sgsa_sparse_gather");
  // K6 at T = 1 on the outputs: in the launch that merges the split rows where that form
  // applies, else after the gather
  auto aligned16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  if (a.nsplit > 0 && dtype == SGSA_BF16 && D == 128 && Tq == 1 && rec->T == 1 && diag == nullptr &&
      weights == nullptr && aligned16(v) && (k == nullptr || aligned16(k)) &&
      (self_key == nullptr || aligned16(self_key))) {
    a.pieces_only = 1;
    if (int s = hip_status(sgsa::launch_sparse_gather(a, (hipStream_t)stream), "sgsa_sparse_gather")) return s;
    return hip_status(sgsa::launch_merge_recurrent(a, *rec, (hipStream_t)stream), "sgsa_sparse_gather (merge, K6)");
  }
  if (int s = hip_status(sgsa::launch_sparse_gather(a, (hipStream_t)stream), "sgsa_sparse_gather")) return s;
  return hip_status(sgsa::launch_recurrent(*rec, (hipStream_t)stream), "sgsa_recurrent_fwd");
}

int sgsa_sparse_gather_masked(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, int q_offset,
                              int kv_layout, const void* k, const void* v, const void* self_key,
                              const int32_t* indices, const float* scores, const uint8_t* slot_valid,
                              const float* top2, const int32_t* counts, const float* budget, int write_mode,
                              float alpha_max, float tau_c, int local_window, int sink_size, void* k_hat,
                              void* v_hat, void* write_key, float* alpha, float* weights, float* diag,
                              float* row_stats, void* workspace, size_t workspace_bytes, void* stream) {
  return sparse_gather_impl(dtype, B, Tq, Tk, H, D, top_k, q_offset, kv_layout, k, v, self_key, indices, scores,
                            slot_valid, top2, counts, budget, write_mode, alpha_max, tau_c, local_window, sink_size,
                            k_hat, v_hat, write_key, alpha, weights, diag, row_stats, workspace, workspace_bytes,
                            stream, nullptr, 0.f);
}

}  // extern "C"

namespace sgsa {
int sparse_gather_stack(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, int q_offset, float scale,
                        int scale_mode, const void* q, const void* k, const void* v, const void* self_key,
                        const int32_t* indices, float* scores, const float* top2, const int32_t* counts,
                        const float* budget, int write_mode, float alpha_max, float tau_c, int local_window,
                        int sink_size, void* k_hat, void* v_hat, void* write_key, float* alpha, void* workspace,
                        size_t workspace_bytes, const RecurrentArgs* rec, void* stream) {
  if (scale_mode != 0 && scale_mode != 1) return fail(SGSA_ERR_INVALID_ARG, "scale_mode must be 0 or 1");
  if (rec != nullptr && (rec->B != B || rec->T != Tq || rec->H != H || rec->D != D || rec->dtype != dtype))
    return fail(SGSA_ERR_INVALID_ARG, "the recurrent update's shape differs from the gather's");
  return sparse_gather_impl(dtype, B, Tq, Tk, H, D, top_k, q_offset, 0, k, v, self_key, indices, scores, nullptr,
                            top2, counts, budget, write_mode, alpha_max, tau_c, local_window, sink_size, k_hat,
                            v_hat, write_key, alpha, nullptr, nullptr, nullptr, workspace, workspace_bytes, stream, q,
                            q != nullptr ? score_multiplier(scale, scale_mode) : 0.f, rec);
}
}  // namespace sgsa

extern "C" {

int sgsa_sparse_gather_workspace_size(int B, int Tq, int H, int D, int top_k, size_t* bytes) {
  if (int s = check_dims(B, Tq, H, D)) return s;
  if (top_k <= 0) return fail(SGSA_ERR_INVALID_ARG, "top_k=%d must be positive", top_k);
  REQUIRE(bytes);
  *bytes = 256 + sgsa::gather_part_bytes((long)B * H * Tq, top_k, D);
  return SGSA_OK;
}

int sgsa_score_at(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, float scale, int scale_mode,
                  const void* q, const void* k, const int32_t* indices, const int32_t* counts, float* scores,
                  void* stream) {
  if (int s = check_dtype(dtype)) return s;
  if (int s = check_dims(B, Tq, H, D)) return s;
  if (int s = check_dims(B, Tk, H, D)) return s;
  if (top_k <= 0) return fail(SGSA_ERR_INVALID_ARG, "top_k=%d must be positive", top_k);
  if (scale_mode != 0 && scale_mode != 1) return fail(SGSA_ERR_INVALID_ARG, "scale_mode must be 0 or 1");
  REQUIRE(q); REQUIRE(k); REQUIRE(indices); REQUIRE(counts); REQUIRE(scores);
  return hip_status(sgsa::launch_rescore(dtype, B, Tq, Tk, H, D, top_k, q, k, indices, counts,
                                         sgsa::score_multiplier(scale, scale_mode), scores, (hipStream_t)stream),
                    "sgsa_score_at");
}

// ---- block retrieval -----------------------------------------------------------
namespace {
struct BlockWs {
  size_t bscores, ncand, bmargin, top2, counts, valid, slot_sc, slot_idx, slot_w, maxidx;
  size_t mpc, mperm, mnvb, mkqb, mbits;   // padding-mask layout (always reserved)
  size_t own_idx, own_bidx;               // the layer form's token and block index lists
  size_t total;
};

// The write gate of SGSAStateLayer (modeling_sgsa.py:497-504, :543-552) folded into the block
// retrieval's gather, for the layer form (sgsa_block_layer_retrieve); all NULL for the retriever.
struct BlockGate {
  const float* budget = nullptr;   // [B,T,H] budget logits
  int write_mode = 0;              // 0 direct, 1 residual
  float alpha_max = 0.f;
  void* write_key = nullptr;       // [B,T,H,D] dtype
  float* alpha = nullptr;          // [B,T,H]
  float* stats = nullptr;          // [2,B,H,T] largest weight, |write key| / |k_hat|, or NULL
};

int block_dims(int B, int T, int H, int top_k, int block_size, int top_blocks, int mode, int& nb, int& eb, int& kk,
               int& ks) {
  if (mode != 0 && mode != 1) return fail(SGSA_ERR_INVALID_ARG, "mode must be 0 (block_only) or 1 (block_token)");
  if (B <= 0 || T <= 0 || H <= 0) return fail(SGSA_ERR_INVALID_ARG, "B=%d T=%d H=%d must be positive", B, T, H);
  if (block_size <= 0 || top_blocks <= 0)
    return fail(SGSA_ERR_INVALID_ARG, "block_size=%d and top_blocks=%d must be positive", block_size, top_blocks);
  if (mode == 1 && top_k <= 0) return fail(SGSA_ERR_INVALID_ARG, "top_k=%d must be positive", top_k);
  nb = (T - 1) / block_size + 1;
  eb = top_blocks < nb ? top_blocks : nb;
  const int bsz = block_size < T ? block_size : T;
  if ((long)eb * bsz > sgsa::BLK_MAXC)
    return fail(SGSA_ERR_UNSUPPORTED, "top_blocks * block_size = %ld candidate keys per row exceeds %d",
                (long)eb * bsz, sgsa::BLK_MAXC);
  kk = mode == 1 ? (top_k < T ? top_k : T) : 0;
  ks = eb * bsz;
  return SGSA_OK;
}

BlockWs block_ws(int B, int T, int H, int nb, int kk, int ks, int mode, bool want_weights, int eb = 0,
                 bool own_lists = false) {
  const size_t rows = (size_t)B * H * T;
  const size_t w = mode == 1 ? (size_t)kk : (size_t)ks;
  BlockWs L{};
  size_t o = 0;
  auto take = [&](size_t bytes) { size_t at = o; o = align_up(o + bytes); return at; };
  L.bscores = take(rows * nb * 4);
  L.ncand = take(rows * 4);
  L.bmargin = take(rows * 4);
  L.top2 = take(rows * 8);
  L.counts = take(rows * 4);
  L.valid = take(rows * kk);
  L.slot_sc = take(rows * w * 4);
  L.slot_idx = mode == 0 ? take(rows * w * 4) : 0;
  L.slot_w = (mode == 0 && want_weights) ? take(rows * w * 4) : 0;
  L.maxidx = take(256);
  L.mpc = take((size_t)B * (T + 1) * 4);
  L.mperm = take((size_t)B * T * 4);
  L.mnvb = take((size_t)B * T * 4);
  L.mkqb = take((size_t)T * 4);
  L.mbits = take((size_t)B * ((T + 31) / 32) * 4);
  L.own_idx = (own_lists && mode == 1) ? take(rows * kk * 4) : 0;
  L.own_bidx = own_lists ? take(rows * eb * 4) : 0;
  L.total = o;
  return L;
}

int block_retrieve_impl(int dtype, int B, int T, int H, int D, int top_k, int block_size, int top_blocks, int mode,
                        int causal, float tau_c, int local_window, int sink_size, const void* q, const void* k,
                        const void* v, const uint8_t* mask, int32_t* indices, int32_t* block_indices,
                        float* block_scores, float* weights, void* k_hat, void* v_hat, float* diag, void* workspace,
                        size_t workspace_bytes, void* stream, const BlockGate* gate = nullptr);
}  // namespace

int sgsa_block_retrieve_workspace_size(int B, int T, int H, int top_k, int block_size, int top_blocks, int mode,
                                       size_t* bytes) {
  int nb, eb, kk, ks;
  if (int s = block_dims(B, T, H, top_k, block_size, top_blocks, mode, nb, eb, kk, ks)) return s;
  REQUIRE(bytes);
  *bytes = block_ws(B, T, H, nb, kk, ks, mode, true).total;
  return SGSA_OK;
}

int sgsa_block_retrieve(int dtype, int B, int T, int H, int D, int top_k, int block_size, int top_blocks, int mode,
                        int causal, float tau_c, int local_window, int sink_size, const void* q, const void* k,
                        const void* v, int32_t* indices, int32_t* block_indices, float* block_scores, float* weights,
                        void* k_hat, void* v_hat, float* diag, void* workspace, size_t workspace_bytes,
                        void* stream) {
  return block_retrieve_impl(dtype, B, T, H, D, top_k, block_size, top_blocks, mode, causal, tau_c, local_window,
                             sink_size, q, k, v, nullptr, indices, block_indices, block_scores, weights, k_hat, v_hat,
                             diag, workspace, workspace_bytes, stream);
}

int sgsa_block_retrieve_masked(int dtype, int B, int T, int H, int D, int top_k, int block_size, int top_blocks,
                               int mode, int causal, float tau_c, int local_window, int sink_size, const void* q,
                               const void* k, const void* v, const uint8_t* attention_mask, int32_t* indices,
                               int32_t* block_indices, float* block_scores, float* weights, void* k_hat, void* v_hat,
                               float* diag, void* workspace, size_t workspace_bytes, void* stream) {
  REQUIRE(attention_mask);
  return block_retrieve_impl(dtype, B, T, H, D, top_k, block_size, top_blocks, mode, causal, tau_c, local_window,
                             sink_size, q, k, v, attention_mask, indices, block_indices, block_scores, weights, k_hat,
                             v_hat, diag, workspace, workspace_bytes, stream);
}

int sgsa_block_layer_retrieve_workspace_size(int B, int T, int H, int top_k, int block_size, int top_blocks,
                                             int mode, size_t* bytes) {
  int nb, eb, kk, ks;
  if (int s = block_dims(B, T, H, top_k, block_size, top_blocks, mode, nb, eb, kk, ks)) return s;
  REQUIRE(bytes);
  *bytes = block_ws(B, T, H, nb, kk, ks, mode, false, eb, true).total;
  return SGSA_OK;
}

int sgsa_block_layer_retrieve(int dtype, int B, int T, int H, int D, int top_k, int block_size, int top_blocks,
                              int mode, float tau_c, const void* q_ret, const void* k, const void* v,
                              const uint8_t* attention_mask, const float* budget, int write_mode, float alpha_max,
                              void* write_key, void* v_hat, float* alpha, float* row_stats, void* workspace,
                              size_t workspace_bytes, void* stream) {
  BlockGate gate;
  gate.budget = budget; gate.write_mode = write_mode; gate.alpha_max = alpha_max;
  gate.write_key = write_key; gate.alpha = alpha; gate.stats = row_stats;
  return block_retrieve_impl(dtype, B, T, H, D, top_k, block_size, top_blocks, mode, 1, tau_c, 64, 8, q_ret, k, v,
                             attention_mask, nullptr, nullptr, nullptr, nullptr, nullptr, v_hat, nullptr, workspace,
                             workspace_bytes, stream, &gate);
}

}  // extern "C"

namespace {
int block_retrieve_impl(int dtype, int B, int T, int H, int D, int top_k, int block_size, int top_blocks, int mode,
                        int causal, float tau_c, int local_window, int sink_size, const void* q, const void* k,
                        const void* v, const uint8_t* mask, int32_t* indices, int32_t* block_indices,
                        float* block_scores, float* weights, void* k_hat, void* v_hat, float* diag, void* workspace,
                        size_t workspace_bytes, void* stream, const BlockGate* gate) {
  if (int s = check_dtype(dtype)) return s;
  if (int s = check_dims(B, T, H, D)) return s;
  int nb, eb, kk, ks;
  if (int s = block_dims(B, T, H, top_k, block_size, top_blocks, mode, nb, eb, kk, ks)) return s;
  REQUIRE(q); REQUIRE(k); REQUIRE(v); REQUIRE(v_hat); REQUIRE(workspace);
  if (gate == nullptr) {
    REQUIRE(block_indices); REQUIRE(k_hat);
    if (mode == 1 && indices == nullptr) return fail(SGSA_ERR_INVALID_ARG, "block_token needs the indices output");
  } else {
    if (gate->budget == nullptr || gate->write_key == nullptr || gate->alpha == nullptr)
      return fail(SGSA_ERR_INVALID_ARG, "budget logits, write_key and alpha must not be NULL");
    if (gate->write_mode != 0 && gate->write_mode != 1)
      return fail(SGSA_ERR_INVALID_ARG, "write_mode must be 0 (direct) or 1 (residual)");
  }
  if ((long)T * H * D * 4 > 0x7fffffffL) return fail(SGSA_ERR_UNSUPPORTED, "one head's keys exceed 2 GiB of offsets");
  const BlockWs L = block_ws(B, T, H, nb, kk, ks, mode, weights != nullptr, eb, gate != nullptr);
  if (workspace_bytes < L.total) return fail(SGSA_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, L.total);
  char* base = static_cast<char*>(workspace);
  if (gate != nullptr) {
    block_indices = reinterpret_cast<int32_t*>(base + L.own_bidx);
    if (mode == 1) indices = reinterpret_cast<int32_t*>(base + L.own_idx);
  }
  sgsa::BlockArgs a{};
  a.dtype = dtype; a.B = B; a.T = T; a.H = H; a.D = D;
  a.bs = block_size; a.nb = nb; a.eb = eb; a.mode = mode; a.kk = kk; a.ks = ks; a.causal = causal ? 1 : 0;
  a.q = q; a.k = k; a.fill_invalid = block_scores != nullptr;
  a.block_scores = reinterpret_cast<float*>(base + L.bscores);
  a.block_indices = block_indices;
  a.ncand = reinterpret_cast<int32_t*>(base + L.ncand);
  a.bmargin = mode == 0 ? reinterpret_cast<float*>(base + L.bmargin) : nullptr;
  a.slot_idx = mode == 1 ? indices : reinterpret_cast<int32_t*>(base + L.slot_idx);
  a.slot_sc = reinterpret_cast<float*>(base + L.slot_sc);
  a.slot_valid = mode == 1 ? reinterpret_cast<uint8_t*>(base + L.valid) : nullptr;
  a.top2 = reinterpret_cast<float*>(base + L.top2);
  a.counts = reinterpret_cast<int32_t*>(base + L.counts);
  a.mask = mask;
  a.nmw = (T + 31) / 32;
  a.mpc = reinterpret_cast<int32_t*>(base + L.mpc);
  a.mperm = reinterpret_cast<int32_t*>(base + L.mperm);
  a.mnvb = reinterpret_cast<int32_t*>(base + L.mnvb);
  a.mkqb = reinterpret_cast<int32_t*>(base + L.mkqb);
  a.mbits = reinterpret_cast<uint32_t*>(base + L.mbits);
  hipStream_t st = (hipStream_t)stream;
  if (int s = hip_status(sgsa::launch_block_select(a, st), "sgsa_block_retrieve (select)")) return s;
  if (block_scores != nullptr)
    if (int s = hip_status(sgsa::launch_block_scores_transpose(a.block_scores, B, H, T, nb, block_scores, st),
                           "sgsa_block_retrieve (block scores)"))
      return s;

  sgsa::GatherArgs g{};
  g.dtype = dtype; g.B = B; g.Tq = T; g.Tk = T; g.H = H; g.D = D; g.top_k = mode == 1 ? kk : ks; g.q_offset = 0;
  g.k = k; g.v = v; g.self_key = k; g.indices = a.slot_idx; g.scores = a.slot_sc; g.top2 = a.top2;
  g.counts = a.counts; g.slot_valid = a.slot_valid; g.use_valid = 1; g.tau_c = tau_c; g.eps = 1e-6f;
  g.local_window = local_window; g.sink_size = sink_size; g.k_hat = k_hat; g.v_hat = v_hat;
  g.weights = mode == 1 ? weights : (weights ? reinterpret_cast<float*>(base + L.slot_w) : nullptr);
  g.diag = diag; g.max_index = reinterpret_cast<int32_t*>(base + L.maxidx);
  g.margin_in = a.bmargin;
  g.ent_pad = mode == 0 ? (float)(T - ks) : 0.f;
  if (gate != nullptr) {
    g.budget = gate->budget; g.write_mode = gate->write_mode; g.alpha_max = gate->alpha_max;
    g.write_key = gate->write_key; g.alpha = gate->alpha; g.stats = gate->stats;
  }
  if (int s = hip_status(sgsa::launch_sparse_gather(g, st), "sgsa_block_retrieve (gather)")) return s;
  if (mode == 0 && weights != nullptr)
    return hip_status(sgsa::launch_block_dense_weights(B, H, T, ks, a.slot_idx, g.weights, a.counts, weights, st),
                      "sgsa_block_retrieve (weights)");
  return SGSA_OK;
}
}  // namespace

extern "C" {

int sgsa_rms_norm(int dtype, int weight_f32, long rows, int C, const void* x, const void* weight, float eps, void* y,
                  void* stream) {
  if (int s = check_dtype(dtype)) return s;
  if (rows < 0 || C <= 0) return fail(SGSA_ERR_INVALID_ARG, "rows=%ld C=%d", rows, C);
  if (rows > 0x7fffffffL) return fail(SGSA_ERR_UNSUPPORTED, "rows=%ld exceeds the grid", rows);
  if (dtype == SGSA_F32 && !weight_f32) return fail(SGSA_ERR_INVALID_ARG, "fp32 input needs an fp32 weight");
  if (!(eps >= 0.f)) return fail(SGSA_ERR_INVALID_ARG, "eps must be >= 0");
  if (rows == 0) return SGSA_OK;
  REQUIRE(x); REQUIRE(weight); REQUIRE(y);
  return hip_status(sgsa::launch_rms_norm(dtype, weight_f32 ? 1 : 0, rows, C, x, weight, eps, y, (hipStream_t)stream),
                    "sgsa_rms_norm");
}

int sgsa_rope_qk(int dtype, int B, int T, int Hq, int Hk, int D, int pos0, int table_len, const void* qk,
                 long row_stride, const float* cos_table, const float* sin_table, void* q_out, void* k_out,
                 void* stream) {
  if (int s = check_dtype(dtype)) return s;
  if (B <= 0 || T < 0 || Hq <= 0 || Hk <= 0 || D <= 0 || D % 2 != 0)
    return fail(SGSA_ERR_INVALID_ARG, "B=%d T=%d Hq=%d Hk=%d D=%d (D even)", B, T, Hq, Hk, D);
  if (pos0 < 0 || (long)pos0 + T > table_len) return fail(SGSA_ERR_INVALID_ARG, "positions [%d, %d) outside the %d-row tables", pos0, pos0 + T, table_len);
  if (row_stride < (long)(Hq + Hk) * D) return fail(SGSA_ERR_INVALID_ARG, "row_stride=%ld < (Hq+Hk)*D", row_stride);
  if ((long)B * T * (Hq + Hk) * D > 0x7fffffffL * 256L) return fail(SGSA_ERR_UNSUPPORTED, "too many elements");
  if (T == 0) return SGSA_OK;
  REQUIRE(qk); REQUIRE(cos_table); REQUIRE(sin_table); REQUIRE(q_out); REQUIRE(k_out);
  return hip_status(sgsa::launch_rope_qk(dtype, qk, row_stride, B, T, Hq, Hk, D, pos0, cos_table, sin_table, q_out,
                                         k_out, (hipStream_t)stream),
                    "sgsa_rope_qk");
}

int sgsa_add_rms_norm(int dtype, int weight_f32, long rows, int C, const void* a, const void* b, void* sum,
                      const void* weight, float eps, void* y, void* stream) {
  if (int s = check_dtype(dtype)) return s;
  if (rows < 0 || C <= 0) return fail(SGSA_ERR_INVALID_ARG, "rows=%ld C=%d", rows, C);
  if (rows > 0x7fffffffL) return fail(SGSA_ERR_UNSUPPORTED, "rows=%ld exceeds the grid", rows);
  if (dtype == SGSA_F32 && !weight_f32) return fail(SGSA_ERR_INVALID_ARG, "fp32 input needs an fp32 weight");
  if (!(eps >= 0.f)) return fail(SGSA_ERR_INVALID_ARG, "eps must be >= 0");
  if (rows == 0) return SGSA_OK;
  REQUIRE(a); REQUIRE(b); REQUIRE(sum); REQUIRE(weight); REQUIRE(y);
  return hip_status(sgsa::launch_add_rms_norm(dtype, weight_f32 ? 1 : 0, rows, C, a, b, sum, weight, eps, y,
                                              (hipStream_t)stream),
                    "sgsa_add_rms_norm");
}

int sgsa_linear_rows(int dtype, int M, int N, int K, const void* x, long x_row_stride, const void* weight,
                     const void* bias, void* y, long y_row_stride, void* stream) {
  if (int s = check_dtype(dtype)) return s;
  if (dtype != SGSA_BF16) return fail(SGSA_ERR_UNSUPPORTED, "sgsa_linear_rows takes bf16");
  if (M < 0 || M > 16 || N <= 0 || K <= 0) return fail(SGSA_ERR_INVALID_ARG, "M=%d (<= 16) N=%d K=%d", M, N, K);
  if (K % 32 != 0) return fail(SGSA_ERR_UNSUPPORTED, "K=%d must be a multiple of 32", K);
  if (x_row_stride < K || x_row_stride % 8 != 0 || y_row_stride < N)
    return fail(SGSA_ERR_INVALID_ARG, "x_row_stride=%ld (>= K, multiple of 8) y_row_stride=%ld (>= N)", x_row_stride,
                y_row_stride);
  if (M == 0) return SGSA_OK;
  REQUIRE(x); REQUIRE(weight); REQUIRE(y);
  if (((uintptr_t)x | (uintptr_t)weight) % 16 != 0) return fail(SGSA_ERR_INVALID_ARG, "x and weight must be 16-byte aligned");
  return hip_status(sgsa::launch_small_gemm(x, x_row_stride, weight, bias, M, N, K, y, y_row_stride, (hipStream_t)stream),
                    "sgsa_linear_rows");
}

int sgsa_linear_rows_tile(int dtype, int N, int K, const void* weight, void* tiled, void* stream) {
  if (int s = check_dtype(dtype)) return s;
  if (dtype != SGSA_BF16) return fail(SGSA_ERR_UNSUPPORTED, "sgsa_linear_rows_tile takes bf16");
  if (N <= 0 || K <= 0) return fail(SGSA_ERR_INVALID_ARG, "N=%d K=%d must be positive", N, K);
  if (K % 32 != 0) return fail(SGSA_ERR_UNSUPPORTED, "K=%d must be a multiple of 32", K);
  if ((long)((N + 15) / 16) * (K / 32) * 64 > 0x7fffffffL * 256L) return fail(SGSA_ERR_UNSUPPORTED, "N * K exceeds the grid");
  REQUIRE(weight); REQUIRE(tiled);
  if (((uintptr_t)weight | (uintptr_t)tiled) % 16 != 0)
    return fail(SGSA_ERR_INVALID_ARG, "weight and tiled must be 16-byte aligned");
  return hip_status(sgsa::launch_tile_rows(weight, N, K, tiled, (hipStream_t)stream), "sgsa_linear_rows_tile");
}

int sgsa_linear_rows_tiled(int dtype, int M, int N, int K, const void* x, long x_row_stride, const void* tiled,
                           const void* bias, void* y, long y_row_stride, void* stream) {
  if (int s = check_dtype(dtype)) return s;
  if (dtype != SGSA_BF16) return fail(SGSA_ERR_UNSUPPORTED, "sgsa_linear_rows_tiled takes bf16");
  if (M < 0 || M > 16 || N <= 0 || K <= 0) return fail(SGSA_ERR_INVALID_ARG, "M=%d (<= 16) N=%d K=%d", M, N, K);
  if (K % 32 != 0) return fail(SGSA_ERR_UNSUPPORTED, "K=%d must be a multiple of 32", K);
  if (x_row_stride < K || x_row_stride % 8 != 0 || y_row_stride < N)
    return fail(SGSA_ERR_INVALID_ARG, "x_row_stride=%ld (>= K, multiple of 8) y_row_stride=%ld (>= N)", x_row_stride,
                y_row_stride);
  if (M == 0) return SGSA_OK;
  REQUIRE(x); REQUIRE(tiled); REQUIRE(y);
  if (((uintptr_t)x | (uintptr_t)tiled) % 16 != 0) return fail(SGSA_ERR_INVALID_ARG, "x and tiled must be 16-byte aligned");
  return hip_status(sgsa::launch_small_gemm(x, x_row_stride, tiled, bias, M, N, K, y, y_row_stride, (hipStream_t)stream,
                                            nullptr, 0, true),
                    "sgsa_linear_rows_tiled");
}

int sgsa_silu_mul(int dtype, long rows, int I, const void* gate_up, long row_stride, void* y, void* stream) {
  if (int s = check_dtype(dtype)) return s;
  if (rows < 0 || I <= 0 || row_stride < 2L * I) return fail(SGSA_ERR_INVALID_ARG, "rows=%ld I=%d row_stride=%ld", rows, I, row_stride);
  if (rows * I > 0x7fffffffL * 256L) return fail(SGSA_ERR_UNSUPPORTED, "rows * I exceeds the grid");
  if (rows == 0) return SGSA_OK;
  REQUIRE(gate_up); REQUIRE(y);
  return hip_status(sgsa::launch_silu_mul(dtype, gate_up, row_stride, rows, I, y, (hipStream_t)stream), "sgsa_silu_mul");
}

int sgsa_layer_gates(int dtype, long rows, int H, const void* logits, long row_stride, float* beta, float* gamma,
                     float* budget, void* stream) {
  if (int s = check_dtype(dtype)) return s;
  if (rows < 0 || H <= 0 || row_stride < 3L * H) return fail(SGSA_ERR_INVALID_ARG, "rows=%ld H=%d row_stride=%ld", rows, H, row_stride);
  if (rows * H > 0x7fffffffL * 256L) return fail(SGSA_ERR_UNSUPPORTED, "rows * H exceeds the grid");
  if (rows == 0) return SGSA_OK;
  REQUIRE(logits); REQUIRE(beta); REQUIRE(gamma); REQUIRE(budget);
  return hip_status(sgsa::launch_gates(dtype, logits, row_stride, rows, H, beta, gamma, budget, (hipStream_t)stream),
                    "sgsa_layer_gates");
}

int sgsa_dense_attention(int dtype, int B, int H, int Hkv, int D, int Tq, int pos0, const void* q,
                         const void* k_cache, const void* v_cache, long cache_len, void* out, void* workspace,
                         size_t workspace_bytes, void* stream) {
  if (int s = check_dtype(dtype)) return s;
  if (dtype != SGSA_BF16) return fail(SGSA_ERR_UNSUPPORTED, "sgsa_dense_attention takes bf16");
  if (B < 0 || Tq < 0 || pos0 < 0 || H <= 0 || Hkv <= 0 || H % Hkv != 0)
    return fail(SGSA_ERR_INVALID_ARG, "B=%d H=%d Hkv=%d Tq=%d pos0=%d", B, H, Hkv, Tq, pos0);
  if (D != 128) return fail(SGSA_ERR_UNSUPPORTED, "sgsa_dense_attention needs D == 128 (got %d)", D);
  if ((long)pos0 + Tq > cache_len) return fail(SGSA_ERR_INVALID_ARG, "pos0 + Tq = %ld exceeds cache_len %ld", (long)pos0 + Tq, cache_len);
  if (((long)pos0 + Tq) * 256L >= 0x7fffffffL) return fail(SGSA_ERR_UNSUPPORTED, "too many cached keys for 32-bit offsets");
  const long nqb2 = (Tq + 127) / 128;
  if ((long)B * H * nqb2 > 0x7fffffffL) return fail(SGSA_ERR_UNSUPPORTED, "grid too large");
  if (B == 0 || Tq == 0) return SGSA_OK;
  REQUIRE(q); REQUIRE(k_cache); REQUIRE(v_cache); REQUIRE(out); REQUIRE(workspace);
  const size_t need = (size_t)B * H * Tq * 8;
  if (workspace_bytes < need) return fail(SGSA_ERR_WORKSPACE, "workspace of %zu bytes, need %zu", workspace_bytes, need);
  return hip_status(sgsa::launch_dense_attn(q, k_cache, v_cache, B, H, Hkv, Tq, pos0, cache_len, (float2*)workspace, out,
                                            (hipStream_t)stream),
                    "sgsa_dense_attention");
}

int sgsa_decode_attention_workspace_size(int dtype, int B, int H, int kend, size_t* bytes) {
  REQUIRE(bytes);
  if (int s = check_dtype(dtype)) return s;
  if (B < 0 || H <= 0 || kend < 0) return fail(SGSA_ERR_INVALID_ARG, "B=%d H=%d kend=%d", B, H, kend);
  *bytes = sgsa::decode_attn_workspace_bytes(dtype, B, H, kend);
  return SGSA_OK;
}

int sgsa_decode_attention(int dtype, int B, int H, int Hkv, int D, const void* q, const void* k_cache,
                          const void* v_cache, long cache_len, int kend, void* out, void* workspace,
                          size_t workspace_bytes, void* stream) {
  if (int s = check_dtype(dtype)) return s;
  if (B < 0 || H <= 0 || Hkv <= 0 || H % Hkv != 0) return fail(SGSA_ERR_INVALID_ARG, "B=%d H=%d Hkv=%d", B, H, Hkv);
  const int G = H / Hkv;
  if (D != 128 || (G != 1 && G != 2 && G != 4 && G != 8))
    return fail(SGSA_ERR_UNSUPPORTED, "decode attention needs D == 128 and H / Hkv in {1, 2, 4, 8} (D=%d, G=%d)", D, G);
  if (kend < 1 || kend > cache_len) return fail(SGSA_ERR_INVALID_ARG, "kend=%d must be in [1, cache_len=%ld]", kend, cache_len);
  if ((long)B * Hkv > 65535) return fail(SGSA_ERR_UNSUPPORTED, "B * Hkv exceeds the grid");
  if (B == 0) return SGSA_OK;
  REQUIRE(q); REQUIRE(k_cache); REQUIRE(v_cache); REQUIRE(out); REQUIRE(workspace);
  if (workspace_bytes < sgsa::decode_attn_workspace_bytes(dtype, B, H, kend))
    return fail(SGSA_ERR_WORKSPACE, "workspace of %zu bytes, need %zu", workspace_bytes,
                sgsa::decode_attn_workspace_bytes(dtype, B, H, kend));
  return hip_status(sgsa::launch_decode_attn(dtype, B, H, Hkv, q, k_cache, v_cache, cache_len, kend, out, workspace,
                                             (hipStream_t)stream),
                    "sgsa_decode_attention");
}

int sgsa_decode_split(int dtype, int B, int H, int D, const void* proj, long row_stride, void* q, void* k, void* v,
                      void* q_ret, float* beta, float* gamma, float* budget, void* k_cache, void* v_cache,
                      long cache_len, long pos, void* stream) {
  if (int s = check_dtype(dtype)) return s;
  if (B < 0 || H <= 0 || D <= 0) return fail(SGSA_ERR_INVALID_ARG, "B=%d H=%d D=%d", B, H, D);
  if (row_stride < 4L * H * D + 3L * H)
    return fail(SGSA_ERR_INVALID_ARG, "row_stride=%ld < 4*H*D + 3*H", row_stride);
  if ((k_cache == nullptr) != (v_cache == nullptr))
    return fail(SGSA_ERR_INVALID_ARG, "k_cache and v_cache must both be given or both be NULL");
  if (k_cache != nullptr && (pos < 0 || pos >= cache_len))
    return fail(SGSA_ERR_INVALID_ARG, "pos=%ld outside the cache [0, %ld)", pos, cache_len);
  if (4L * B * H * D + (long)B * H > 0x7fffffffL * 256L) return fail(SGSA_ERR_UNSUPPORTED, "too many elements");
  if (B == 0) return SGSA_OK;
  REQUIRE(proj); REQUIRE(q); REQUIRE(k); REQUIRE(v); REQUIRE(q_ret); REQUIRE(beta); REQUIRE(gamma); REQUIRE(budget);
  return hip_status(sgsa::launch_decode_split(dtype, proj, row_stride, B, H, D, q, k, v, q_ret, beta, gamma, budget,
                                              k_cache, v_cache, cache_len, pos, (hipStream_t)stream),
                    "sgsa_decode_split");
}

int sgsa_sparse_gather_tiled(int B, int T, int H, int D, int top_k, const void* k, const void* v,
                             const int32_t* indices, const float* scores, const float* top2,
                             const int32_t* counts, const int32_t* split, const float* budget, int write_mode,
                             float alpha_max, float tau_c, void* k_hat, void* v_hat, void* write_key,
                             float* alpha, void* stream) {
  if (int s = check_dims(B, T, H, D)) return s;
  if (D != 128) return fail(SGSA_ERR_UNSUPPORTED, "the tiled gather needs D == 128 (got %d)", D);
  if (top_k <= 0 || top_k > T) return fail(SGSA_ERR_INVALID_ARG, "top_k=%d must be in [1, T]", top_k);
  if (top_k % 4 != 0) return fail(SGSA_ERR_UNSUPPORTED, "the tiled gather needs top_k %% 4 == 0 (got %d)", top_k);
  REQUIRE(k); REQUIRE(v); REQUIRE(indices); REQUIRE(scores); REQUIRE(top2); REQUIRE(counts); REQUIRE(split);
  REQUIRE(v_hat);
  if (write_mode != 0 && write_mode != 1) return fail(SGSA_ERR_INVALID_ARG, "write_mode must be 0 (direct) or 1 (residual)");
  if (budget != nullptr && alpha == nullptr) return fail(SGSA_ERR_INVALID_ARG, "the write gate needs an alpha output");
  if (write_mode == 1 && budget != nullptr && write_key == nullptr)
    return fail(SGSA_ERR_INVALID_ARG, "residual write mode needs a write_key output");
  sgsa::GatherArgs g{};
  g.dtype = SGSA_BF16; g.B = B; g.Tq = T; g.Tk = T; g.H = H; g.D = D; g.top_k = top_k; g.q_offset = 0;
  g.k = k; g.v = v; g.self_key = k; g.indices = indices; g.scores = scores; g.top2 = top2; g.counts = counts;
  g.use_valid = 1; g.tau_c = tau_c; g.eps = 1e-6f; g.budget = budget; g.write_mode = write_mode;
  g.alpha_max = alpha_max; g.k_hat = k_hat; g.v_hat = v_hat; g.write_key = write_key; g.alpha = alpha;
  return hip_status(sgsa::launch_sparse_gather_staged(g, split, (hipStream_t)stream), "sgsa_sparse_gather_tiled");
}

int sgsa_layer_fwd_workspace_size(int dtype, int B, int T, int H, int D, int top_k, size_t* bytes) {
  REQUIRE(bytes);
  if (int s = check_dtype(dtype)) return s;
  if (int s = check_dims(B, T, H, D)) return s;
  if (top_k <= 0) return fail(SGSA_ERR_INVALID_ARG, "top_k=%d must be positive", top_k);
  *bytes = layer_ws(dtype, B, T, H, D, top_k).total;
  return SGSA_OK;
}

}  // extern "C"

namespace {

// A padding mask for the threshold form: the keys and values in valid-first order and each
// row's valid prefix and slot count (mask.hip); nullptr members for an unmasked layer.
struct LayerMask {
  const int32_t* row_nv = nullptr;
  const int32_t* row_kq = nullptr;
  const void* kc = nullptr;
  const void* vc = nullptr;
};

// K1 + K2 of the layer path into (wk, vh, al); the workspace is laid out by layer_ws.
int layer_retrieve_impl(const LayerWs& L, char* base, int dtype, int B, int T, int H, int D, int top_k,
                        const void* q_ret, const void* k, const void* v, const float* budget, int write_mode,
                        float alpha_max, float tau_c, void* wk, void* vh, float* al, float* stats,
                        hipStream_t st, const char* who, const LayerMask& mk = LayerMask{}) {
  const int kk = top_k < T ? top_k : T;
  int32_t* cnt = (int32_t*)(base + L.cnt);
  float* t2 = (float*)(base + L.top2);

  sgsa::TopkArgs ta{};
  ta.dtype = dtype; ta.B = B; ta.Tq = T; ta.Tk = T; ta.H = H; ta.D = D; ta.top_k = kk; ta.causal = 1;
  ta.q_offset = 0; ta.scale = (float)sqrt((double)D); ta.scale_mode = 0;
  ta.q = q_ret; ta.k = mk.kc != nullptr ? mk.kc : k; ta.counts = cnt;
  ta.row_nv = mk.row_nv; ta.row_kq = mk.row_kq;
  if (L.thr) {
    ta.thr = reinterpret_cast<uint2*>(base + L.idx);
    ta.top2 = t2;
  } else {
    ta.indices = (int32_t*)(base + L.idx); ta.scores = (float*)(base + L.sc);
  }
  ta.workspace = base + L.topk;
  if (int s = hip_status(sgsa::launch_score_topk(ta, st), who)) return s;

  sgsa::GatherArgs ga{};
  ga.dtype = dtype; ga.B = B; ga.Tq = T; ga.Tk = T; ga.H = H; ga.D = D; ga.top_k = kk; ga.q_offset = 0;
  ga.k = mk.kc != nullptr ? mk.kc : k; ga.v = mk.vc != nullptr ? mk.vc : v; ga.self_key = k; ga.counts = cnt;
  ga.row_nv = mk.row_nv;
  ga.use_valid = 1; ga.tau_c = tau_c; ga.eps = 1e-6f; ga.local_window = 64; ga.sink_size = 8;
  ga.budget = budget; ga.write_mode = write_mode; ga.alpha_max = alpha_max;
  ga.k_hat = write_mode == 0 ? wk : nullptr; ga.v_hat = vh; ga.write_key = write_mode == 1 ? wk : nullptr;
  ga.alpha = al;
  ga.stats = stats;
  if (L.thr) {
    ga.top2 = t2;
    return hip_status(sgsa::launch_sparse_gather_thr(ga, q_ret, ta.thr, sgsa::score_multiplier(ta.scale, ta.scale_mode),
                                                     st), who);
  }
  ga.indices = ta.indices; ga.scores = ta.scores; ga.top2 = nullptr;
  return hip_status(sgsa::launch_sparse_gather(ga, st), who);
}

int layer_check(int dtype, int B, int T, int H, int D, int top_k, int write_mode) {
  if (int s = check_dtype(dtype)) return s;
  if (int s = check_dims(B, T, H, D)) return s;
  if (top_k <= 0) return fail(SGSA_ERR_INVALID_ARG, "top_k=%d must be positive", top_k);
  if (write_mode != 0 && write_mode != 1) return fail(SGSA_ERR_INVALID_ARG, "write_mode must be 0 (direct) or 1 (residual)");
  return SGSA_OK;
}

}  // namespace

extern "C" {

int sgsa_layer_retrieve(int dtype, int B, int T, int H, int D, int top_k, const void* q_ret, const void* k,
                        const void* v, const float* budget, int write_mode, float alpha_max, float tau_c,
                        void* write_key, void* v_hat, float* alpha, void* workspace, size_t workspace_bytes,
                        void* stream) {
  return sgsa_layer_retrieve_stats(dtype, B, T, H, D, top_k, q_ret, k, v, budget, write_mode, alpha_max, tau_c,
                                   write_key, v_hat, alpha, nullptr, workspace, workspace_bytes, stream);
}

int sgsa_layer_retrieve_stats(int dtype, int B, int T, int H, int D, int top_k, const void* q_ret, const void* k,
                              const void* v, const float* budget, int write_mode, float alpha_max, float tau_c,
                              void* write_key, void* v_hat, float* alpha, float* row_stats, void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (int s = layer_check(dtype, B, T, H, D, top_k, write_mode)) return s;
  REQUIRE(q_ret); REQUIRE(k); REQUIRE(v); REQUIRE(budget); REQUIRE(write_key); REQUIRE(v_hat); REQUIRE(alpha);
  REQUIRE(workspace);
  const LayerWs L = layer_ws(dtype, B, T, H, D, top_k);
  if (workspace_bytes < L.total) return fail(SGSA_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, L.total);
  char* base = (char*)(((uintptr_t)workspace + kAlign - 1) & ~(uintptr_t)(kAlign - 1));
  return layer_retrieve_impl(L, base, dtype, B, T, H, D, top_k, q_ret, k, v, budget, write_mode, alpha_max, tau_c,
                             write_key, v_hat, alpha, row_stats, (hipStream_t)stream, "sgsa_layer_retrieve");
}

int sgsa_layer_retrieve_masked_workspace_size(int dtype, int B, int T, int H, int D, int top_k, size_t* bytes) {
  REQUIRE(bytes);
  if (int s = layer_check(dtype, B, T, H, D, top_k, 0)) return s;
  const LayerWs L = layer_ws(dtype, B, T, H, D, top_k);
  if (!L.thr || T > 65536)
    return fail(SGSA_ERR_UNSUPPORTED, "the masked threshold form needs bf16, D == 128 and T <= 65536");
  *bytes = align_up(sgsa::mask_workspace_bytes(dtype, B, T, T, H, D, 1)) +
           align_up((size_t)B * T * H * D * dtype_size(dtype)) + L.total + kAlign;
  return SGSA_OK;
}

int sgsa_layer_retrieve_masked(int dtype, int B, int T, int H, int D, int top_k, const void* q_ret, const void* k,
                               const void* v, const uint8_t* attention_mask, const float* budget, int write_mode,
                               float alpha_max, float tau_c, void* write_key, void* v_hat, float* alpha,
                               float* row_stats, void* workspace, size_t workspace_bytes, void* stream) {
  size_t need = 0;
  if (int s = sgsa_layer_retrieve_masked_workspace_size(dtype, B, T, H, D, top_k, &need)) return s;
  if (write_mode != 0 && write_mode != 1) return fail(SGSA_ERR_INVALID_ARG, "write_mode must be 0 (direct) or 1 (residual)");
  REQUIRE(q_ret); REQUIRE(k); REQUIRE(v); REQUIRE(attention_mask); REQUIRE(budget); REQUIRE(write_key);
  REQUIRE(v_hat); REQUIRE(alpha); REQUIRE(workspace);
  if (workspace_bytes < need) return fail(SGSA_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, need);
  const hipStream_t st = (hipStream_t)stream;
  char* base = (char*)(((uintptr_t)workspace + kAlign - 1) & ~(uintptr_t)(kAlign - 1));
  const int kk = top_k < T ? top_k : T;
  sgsa::MaskArgs m{};
  m.dtype = dtype; m.B = B; m.Tq = T; m.Tk = T; m.H = H; m.D = D;
  m.causal = 1; m.q_offset = 0; m.top_k = kk; m.kq_rule = 0; m.kv_hm = 0; m.compacted = 1;
  m.key_mask = attention_mask; m.query_mask = attention_mask; m.k = k;
  sgsa::mask_carve(m, base);
  char* vc = base + align_up(sgsa::mask_workspace_bytes(dtype, B, T, T, H, D, 1));
  char* lbase = vc + align_up((size_t)B * T * H * D * dtype_size(dtype));
  if (int s = hip_status(sgsa::launch_mask_prepare(m, st), "sgsa_layer_retrieve_masked (mask)")) return s;
  if (int s = hip_status(sgsa::launch_mask_compact(m, v, vc, st), "sgsa_layer_retrieve_masked (values)")) return s;
  LayerMask mk;
  mk.row_nv = m.nv; mk.row_kq = m.kq; mk.kc = m.kc; mk.vc = vc;
  const LayerWs L = layer_ws(dtype, B, T, H, D, top_k);
  return layer_retrieve_impl(L, lbase, dtype, B, T, H, D, top_k, q_ret, k, v, budget, write_mode, alpha_max, tau_c,
                             write_key, v_hat, alpha, row_stats, st, "sgsa_layer_retrieve_masked", mk);
}

int sgsa_layer_fwd(int dtype, int B, int T, int H, int D, int top_k, int chunk_size, const void* q, const void* k,
                   const void* v, const void* q_ret, const float* beta, const float* gamma, const float* budget,
                   const float* initial_state, int write_mode, float alpha_max, float tau_c, void* out,
                   float* final_state, void* workspace, size_t workspace_bytes, void* stream) {
  return sgsa_layer_fwd_stats(dtype, B, T, H, D, top_k, chunk_size, q, k, v, q_ret, beta, gamma, budget,
                              initial_state, write_mode, alpha_max, tau_c, out, final_state, nullptr, nullptr,
                              workspace, workspace_bytes, stream);
}

int sgsa_layer_fwd_stats(int dtype, int B, int T, int H, int D, int top_k, int chunk_size, const void* q,
                         const void* k, const void* v, const void* q_ret, const float* beta, const float* gamma,
                         const float* budget, const float* initial_state, int write_mode, float alpha_max,
                         float tau_c, void* out, float* final_state, float* alpha_out, float* row_stats,
                         void* workspace, size_t workspace_bytes, void* stream) {
  if (int s = layer_check(dtype, B, T, H, D, top_k, write_mode)) return s;
  if (chunk_size <= 0) return fail(SGSA_ERR_INVALID_ARG, "chunk_size=%d must be positive", chunk_size);
  REQUIRE(q); REQUIRE(k); REQUIRE(v); REQUIRE(q_ret); REQUIRE(beta); REQUIRE(gamma); REQUIRE(budget);
  REQUIRE(out); REQUIRE(workspace);
  const LayerWs L = layer_ws(dtype, B, T, H, D, top_k);
  if (workspace_bytes < L.total) return fail(SGSA_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, L.total);
  char* base = (char*)(((uintptr_t)workspace + kAlign - 1) & ~(uintptr_t)(kAlign - 1));
  void* wk = base + L.wk;
  void* vh = base + L.vh;
  float* al = alpha_out ? alpha_out : (float*)(base + L.al);
  hipStream_t st = (hipStream_t)stream;
  if (int s = layer_retrieve_impl(L, base, dtype, B, T, H, D, top_k, q_ret, k, v, budget, write_mode, alpha_max,
                                  tau_c, wk, vh, al, row_stats, st, "sgsa_layer_fwd(retrieve)"))
    return s;

  sgsa::ChunkArgs ca{};
  ca.dtype = dtype; ca.B = B; ca.T = T; ca.H = H; ca.D = D;
  ca.q = q; ca.k = k; ca.v = v; ca.beta = beta; ca.gamma = gamma;
  ca.sparse_k = wk; ca.sparse_v = vh; ca.alpha = al; ca.initial_state = initial_state;
  ca.out = out; ca.final_state = final_state; ca.workspace = base + L.chunk;
  return hip_status(sgsa::launch_chunk_fwd(ca, st), "sgsa_layer_fwd(chunk)");
}

}  // extern "C"
