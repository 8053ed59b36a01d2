// Padding masks for the token top-k select (gfx950).
//
// The reference builds a dense [B,H,Q,K] valid mask (causal & key_valid &
// query_valid, modelings/modeling_sgsa.py:421-428; future | ~key_valid for the
// hybrid's KV reuse, modelings/hybrid_dense_delta_topk.py:153-175), fills the
// invalid scores with finfo.min and takes a fixed number of slots per row
// (:144-165; hybrid :346-349).  Here the mask never exists as a matrix:
//
//   1. mask_scan_kernel: per batch, the exclusive prefix count pc[j] of valid
//      keys below j, the valid keys' original indices in order (perm) and the
//      masked keys' indices in order (inv);
//   2. mask_rows_kernel: per query row, its valid key count nv (with causality
//      the valid keys of a row are keys <= its position that are not masked,
//      i.e. the first pc[pos + 1] keys of the compacted order) and its slot
//      count kq (SparseRetriever: min(top_k, max(1, max over the batch of nv)),
//      :159-160; hybrid: top_k for every row);
//   3. mask_compact_kernel: the keys copied into valid-first order, so that
//      every row's valid keys are a prefix and the row kernel of topk.hip runs
//      unchanged on them with per-row bounds (TopkArgs::row_nv / row_kq);
//   4. mask_finish_kernel: selected slots mapped back to original key indices,
//      and the slots between a row's valid count and its kq filled the way the
//      reference's masked top-k fills them: the row's lowest-index invalid keys
//      (finfo.min scores tie, and ties go to the lowest index), score -FLT_MAX,
//      valid 0; slots past kq get index 0 (:151-153).
#include <float.h>

#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace sgsa {

namespace {

// One block per batch: a 1024-wide scan repeated over the keys.
__global__ __launch_bounds__(1024) void mask_scan_kernel(const uint8_t* __restrict__ key_mask, int Tk,
                                                         int32_t* __restrict__ pc, int32_t* __restrict__ perm,
                                                         int32_t* __restrict__ inv) {
  __shared__ int wsum[16];
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint8_t* km = key_mask ? key_mask + (long)b * Tk : nullptr;
  int32_t* pcb = pc + (long)b * (Tk + 1);
  int32_t* pb = perm + (long)b * Tk;
  int32_t* ib = inv + (long)b * Tk;
  int carry = 0;
  for (int base = 0; base < Tk; base += 1024) {
    const int j = base + tid;
    const bool v = j < Tk && (km == nullptr || km[j] != 0);
    const uint64_t bal = ballot64(v);
    if (lane == 0) wsum[w] = __popcll(bal);
    __syncthreads();
    int off = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int s = wsum[i];
      off += i < w ? s : 0;
      tot += s;
    }
    const int ex = carry + off + (int)lane_rank(bal);
    if (j < Tk) {
      pcb[j] = ex;
      if (v) pb[ex] = j;
      else ib[j - ex] = j;
    }
    carry += tot;
    __syncthreads();   // wsum is rewritten by the next step
  }
  if (tid == 0) pcb[Tk] = carry;
}

__global__ __launch_bounds__(256) void mask_rows_kernel(const uint8_t* __restrict__ query_mask,
                                                        const int32_t* __restrict__ pc, int B, int Tq, int Tk,
                                                        int causal, int q_offset, int top_k, int kq_rule,
                                                        int32_t* __restrict__ nv, int32_t* __restrict__ kq) {
  const int q = blockIdx.x * 256 + threadIdx.x;
  if (q >= Tq) return;
  const int lim = causal ? min(Tk, q + q_offset + 1) : Tk;   // q_offset >= 0: lim >= 1
  int mx = 0;
  for (int b = 0; b < B; ++b) {
    const bool qv = query_mask == nullptr || query_mask[(long)b * Tq + q] != 0;
    const int n = qv ? pc[(long)b * (Tk + 1) + lim] : 0;
    nv[(long)b * Tq + q] = n;
    mx = max(mx, n);
  }
  kq[q] = kq_rule == 0 ? min(top_k, max(1, mx)) : top_k;
}

// kc[b, jc, h, :] = k[b, perm[b, jc], h, :] for jc < (valid keys of b), zeros
// after; U is the copy unit (16-byte vectors when rows allow, else elements).
// Source layout [B,Tk,H,D] (kv_hm = 0) or [B,H,Tk,D] (kv_hm = 1).
template <typename U>
__global__ __launch_bounds__(256) void mask_compact_kernel(const U* __restrict__ k, U* __restrict__ kc,
                                                           const int32_t* __restrict__ perm,
                                                           const int32_t* __restrict__ pc, int B, int Tk, int H,
                                                           int upr, int kv_hm) {
  const long n = (long)B * Tk * H * upr;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    const int cu = (int)(i % upr);
    const long r = i / upr;   // (b * Tk + jc) * H + h
    const int h = (int)(r % H);
    const long bt = r / H;
    const int jc = (int)(bt % Tk), b = (int)(bt / Tk);
    U val{};
    if (jc < pc[(long)b * (Tk + 1) + Tk]) {
      const long j = perm[(long)b * Tk + jc];
      const long src = kv_hm ? (((long)b * H + h) * Tk + j) * upr : (((long)b * Tk + j) * H + h) * upr;
      val = k[src + cu];
    }
    kc[i] = val;
  }
}

// One wave per row (b, h, q) of the [B,H,Tq,top_k] outputs.
__global__ __launch_bounds__(256) void mask_finish_kernel(MaskArgs m, int32_t* __restrict__ indices,
                                                          float* __restrict__ scores, uint8_t* __restrict__ slot_valid,
                                                          const int32_t* __restrict__ counts,
                                                          int32_t* __restrict__ fill) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const long rows = (long)m.B * m.H * m.Tq;
  if (row >= rows) return;
  const int Tq = m.Tq, Tk = m.Tk, topk = m.top_k;
  const int q = (int)(row % Tq), b = (int)(row / Tq) / m.H;
  const int c = counts[row], kqr = m.kq[q];
  const bool qv = m.query_mask == nullptr || m.query_mask[(long)b * Tq + q] != 0;
  const int lim = m.causal ? min(Tk, q + m.q_offset + 1) : Tk;
  const int nm = lim - m.pc[(long)b * (Tk + 1) + lim];   // masked keys below lim
  const int32_t* pb = m.perm + (long)b * Tk;
  const int32_t* ib = m.inv + (long)b * Tk;
  int32_t* ip = indices + row * topk;
  float* sp = scores + row * topk;
  uint8_t* vp = slot_valid ? slot_valid + row * topk : nullptr;
  for (int s = lane; s < topk; s += 64) {
    int j = 0;
    bool ok = false;
    if (s < c) {
      j = ip[s];
      if (m.compacted) j = pb[j];
      ok = true;
    } else if (s < kqr) {
      // the (s - c)-th lowest-index invalid key of the row: every key when the
      // query itself is masked; else the masked keys below lim, then (causal)
      // the keys from lim on.  s - c < Tk - nv keeps both inside [0, Tk).
      const int t = s - c;
      j = !qv ? t : (t < nm ? ib[t] : lim + (t - nm));
    }
    ip[s] = j;
    if (!ok) sp[s] = -FLT_MAX;
    if (vp) vp[s] = ok ? 1 : 0;
  }
  if (fill && lane == 0) fill[row] = kqr;
}

}  // namespace

size_t mask_workspace_bytes(int dtype, int B, int Tq, int Tk, int H, int D, int compact) {
  auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
  size_t n = al((size_t)B * (Tk + 1) * 4) + 2 * al((size_t)B * Tk * 4) + al((size_t)B * Tq * 4) + al((size_t)Tq * 4);
  if (compact) n += al((size_t)B * Tk * H * D * (dtype == DT_F32 ? 4 : 2));
  return n;
}

void mask_carve(MaskArgs& m, void* ws) {
  auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
  char* p = static_cast<char*>(ws);
  m.pc = reinterpret_cast<int32_t*>(p); p += al((size_t)m.B * (m.Tk + 1) * 4);
  m.perm = reinterpret_cast<int32_t*>(p); p += al((size_t)m.B * m.Tk * 4);
  m.inv = reinterpret_cast<int32_t*>(p); p += al((size_t)m.B * m.Tk * 4);
  m.nv = reinterpret_cast<int32_t*>(p); p += al((size_t)m.B * m.Tq * 4);
  m.kq = reinterpret_cast<int32_t*>(p); p += al((size_t)m.Tq * 4);
  m.kc = m.compacted ? p : nullptr;
}

hipError_t launch_mask_compact(const MaskArgs& m, const void* src, void* dst, hipStream_t st) {
  const size_t es = m.dtype == DT_F32 ? 4 : 2;
  const size_t row_bytes = (size_t)m.D * es;
  const bool vec = row_bytes % 16 == 0 && ((uintptr_t)src & 15u) == 0 && ((uintptr_t)dst & 15u) == 0;
  const int upr = (int)(vec ? row_bytes / 16 : (size_t)m.D);
  const long n = (long)m.B * m.Tk * m.H * upr;
  const unsigned grid = (unsigned)std::min<long>((n + 255) / 256, 65536L);
  if (vec)
    mask_compact_kernel<uint4><<<grid, 256, 0, st>>>((const uint4*)src, (uint4*)dst, m.perm, m.pc, m.B, m.Tk, m.H,
                                                     upr, m.kv_hm);
  else if (es == 4)
    mask_compact_kernel<float><<<grid, 256, 0, st>>>((const float*)src, (float*)dst, m.perm, m.pc, m.B, m.Tk, m.H,
                                                     upr, m.kv_hm);
  else
    mask_compact_kernel<uint16_t><<<grid, 256, 0, st>>>((const uint16_t*)src, (uint16_t*)dst, m.perm, m.pc, m.B,
                                                        m.Tk, m.H, upr, m.kv_hm);
  return hipGetLastError();
}

hipError_t launch_mask_prepare(const MaskArgs& m, hipStream_t st) {
  mask_scan_kernel<<<dim3((unsigned)m.B), 1024, 0, st>>>(m.key_mask, m.Tk, m.pc, m.perm, m.inv);
  mask_rows_kernel<<<dim3((unsigned)((m.Tq + 255) / 256)), 256, 0, st>>>(
      m.query_mask, m.pc, m.B, m.Tq, m.Tk, m.causal, m.q_offset, m.top_k, m.kq_rule, m.nv, m.kq);
  if (!m.compacted) return hipGetLastError();
  return launch_mask_compact(m, m.k, m.kc, st);
}

hipError_t launch_mask_finish(const MaskArgs& m, int32_t* indices, float* scores, uint8_t* slot_valid,
                              const int32_t* counts, int32_t* fill, hipStream_t st) {
  const long rows = (long)m.B * m.H * m.Tq;
  mask_finish_kernel<<<dim3((unsigned)((rows + 3) / 4)), 256, 0, st>>>(m, indices, scores, slot_valid, counts, fill);
  return hipGetLastError();
}

}  // namespace sgsa
