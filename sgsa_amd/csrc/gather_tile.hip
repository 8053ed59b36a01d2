// K2t: top-k weighted K/V sum by streaming K/V tiles through LDS (bf16, D = 128).
//
// Same result as K2 (gather.hip) for the fused layer path -- k_hat, v_hat, the
// write key and the alpha gate (modelings/modeling_sgsa.py:126-134, :369-381,
// :497-504, :546-551) -- computed the MI355X way: instead of fetching each of
// the ~2048 selected K and V rows of every query row from HBM/L2 with 16-byte
// gathers, a block of 64 query rows walks the causal key range once in tiles
// of 64 keys.  Each tile of K and V is read from HBM with coalesced 16-byte
// loads (prefetched one tile ahead into registers) and stored transposed in
// LDS; the exact top-k weights of the tile form a sparse 64x64 block P built
// from the rows' slot lists; then k_hat += P K and v_hat += P V run on
// v_mfma_f32_16x16x32_bf16 (P rounded to bf16, weights in (0,1]).
//
// Slot lists come from K1: per row, slots [0, split) ascend in key index and
// slots [split, count) ascend in key index, so each row keeps two cursors that
// advance monotonically with the tile index.  The four lanes of a row hold a
// 32-slot window of each run in registers (16-byte loads, issued right after
// the tile that consumed the previous window, so their latency overlaps the
// MFMA work and the next K/V tile); a row that exhausts a window inside one
// tile reloads it and goes round again.  Weights are exp(s - m) with the row
// maximum m from K1 (top2); the softmax denominator is summed in fp32 from the
// unrounded weights.  Requires top_k % 4 == 0 (16-byte aligned windows).
#include "common.h"
#include "kernels.h"

#include <float.h>

namespace sgsa {

namespace {

constexpr int QB = 64;
constexpr int KT = 64;
constexpr int DP = 128;
constexpr int PT = KT + 8;   // pitch (bf16) of the transposed K/V tiles and of P

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ bf16x8 as_bf8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

// One ascending run of a row's slot list.  Lane quarter lg holds positions
// base + 16h + 4lg + e (h = 0, 1; e = 0..3) of the window.
struct SlotRun {
  int c, end, base;
  int4 ix[2];
  float4 sc[2];
};

// (Re)load the 32-slot window at the cursor.  Always issues the same four
// loads (addresses clamped into the row) so the wait counts stay static;
// positions at or past `end` are masked when consumed.
__device__ __forceinline__ void slot_window(SlotRun& r, const int* __restrict__ idxp,
                                            const float* __restrict__ scp, int lg, int topk) {
  r.base = r.c & ~3;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int p = min(r.base + 16 * hh + 4 * lg, topk - 4);
    r.ix[hh] = *reinterpret_cast<const int4*>(idxp + p);
    r.sc[hh] = *reinterpret_cast<const float4*>(scp + p);
  }
}

// Scatter the window's slots with key in [t0, t1) into this wave's P rows.
// Returns the lane's consumed count; `stop` is set when a held slot lies at or
// beyond t1 (the row is done with this tile).
__device__ __forceinline__ int slot_consume(const SlotRun& r, int t0, int t1, int lg, float m, uint16_t* prow,
                                            float& esum, bool& stop) {
  int n = 0;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int js[4] = {r.ix[hh].x, r.ix[hh].y, r.ix[hh].z, r.ix[hh].w};
    const float ss[4] = {r.sc[hh].x, r.sc[hh].y, r.sc[hh].z, r.sc[hh].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int pos = r.base + 16 * hh + 4 * lg + e;
      if (pos >= r.c && pos < r.end) {
        const int j = js[e];
        if (j < t1) {
          ++n;
          if (j >= t0) {
            const float wv = __expf(ss[e] - m);
            esum += wv;
            prow[j - t0] = f32_to_bf16(wv);
          }
        } else {
          stop = true;
        }
      }
    }
  }
  return n;
}

}  // namespace

__global__ __launch_bounds__(256) void gather_tile_kernel(GatherArgs a, const int32_t* __restrict__ split,
                                                          int nqb) {
  __shared__ __align__(16) uint16_t Kt[DP * PT];
  __shared__ __align__(16) uint16_t Vt[DP * PT];
  __shared__ __align__(16) uint16_t P[4][16 * PT];
  __shared__ float rowE[4][16];

  const int BH = a.B * a.H;
  const int bid = blockIdx.x;
  const int bh = bid % BH;
  const int qb = nqb - 1 - bid / BH;    // heaviest query blocks first
  const int b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int Tq = a.Tq, Tk = a.Tk, H = a.H, topk = a.top_k;
  const int r0 = qb * QB;
  const uint16_t* K = reinterpret_cast<const uint16_t*>(a.k);
  const uint16_t* V = reinterpret_cast<const uint16_t*>(a.v);

  // ---- slot-list ownership: lane -> (row = r0 + 16w + lr, quarter lg) -------
  const int prow = r0 + 16 * w + lr;
  const bool plive = prow < Tq;
  const long pbase = ((long)bh * Tq + (plive ? prow : 0)) * topk;
  int end1 = 0, end2 = 0;
  float m = 0.f;
  if (plive) {
    const long rg = (long)bh * Tq + prow;
    end2 = a.counts[rg];
    end1 = min(split[rg], end2);
    m = a.top2[2 * rg];
  }
  float esum = 0.f;

  int kend = Tk;
  {
    const int last = min(Tq, r0 + QB) - 1 + a.q_offset;
    kend = min(Tk, last + 1);
  }
  const int ntile = (kend + KT - 1) / KT;

  // ---- K/V tile staging (transposed), register prefetch one tile ahead -----
  // thread t: key pair kp = t % 32 (keys 2kp, 2kp+1), 8-dim chunks c = t/32 and c+8
  const int kp = tid & 31, cq = tid >> 5;
  // Loads are unconditional (key index clamped into [0, Tk)) so every thread
  // issues the same number of memory operations per tile; keys past Tk are
  // zeroed at commit.
  uint4 pk[2][2], pv[2][2];   // [chunk half][key of the pair]
  uint32_t pmask[2];          // all-ones for keys < Tk
  auto issue = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = kt * KT + 2 * kp + u;
      pmask[u] = j < Tk ? 0xffffffffu : 0u;
      const int jc = min(j, Tk - 1);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const long off = ((long)(b * Tk + jc) * H + h) * DP + 8 * (cq + 8 * hh);
        pk[hh][u] = *reinterpret_cast<const uint4*>(K + off);
        pv[hh][u] = *reinterpret_cast<const uint4*>(V + off);
      }
    }
  };
  auto commit = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint32_t mk = pmask[u];
        pk[hh][u] = make_uint4(pk[hh][u].x & mk, pk[hh][u].y & mk, pk[hh][u].z & mk, pk[hh][u].w & mk);
        pv[hh][u] = make_uint4(pv[hh][u].x & mk, pv[hh][u].y & mk, pv[hh][u].z & mk, pv[hh][u].w & mk);
      }
    }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int c = cq + 8 * hh;
      const uint32_t k0[4] = {pk[hh][0].x, pk[hh][0].y, pk[hh][0].z, pk[hh][0].w};
      const uint32_t k1[4] = {pk[hh][1].x, pk[hh][1].y, pk[hh][1].z, pk[hh][1].w};
      const uint32_t v0[4] = {pv[hh][0].x, pv[hh][0].y, pv[hh][0].z, pv[hh][0].w};
      const uint32_t v1[4] = {pv[hh][1].x, pv[hh][1].y, pv[hh][1].z, pv[hh][1].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // dims 8c+2i (low halves) and 8c+2i+1 (high halves) of keys 2kp, 2kp+1
        const uint32_t klo = (k0[i] & 0xffffu) | (k1[i] << 16);
        const uint32_t khi = (k0[i] >> 16) | (k1[i] & 0xffff0000u);
        const uint32_t vlo = (v0[i] & 0xffffu) | (v1[i] << 16);
        const uint32_t vhi = (v0[i] >> 16) | (v1[i] & 0xffff0000u);
        *reinterpret_cast<uint32_t*>(&Kt[(8 * c + 2 * i) * PT + 2 * kp]) = klo;
        *reinterpret_cast<uint32_t*>(&Kt[(8 * c + 2 * i + 1) * PT + 2 * kp]) = khi;
        *reinterpret_cast<uint32_t*>(&Vt[(8 * c + 2 * i) * PT + 2 * kp]) = vlo;
        *reinterpret_cast<uint32_t*>(&Vt[(8 * c + 2 * i + 1) * PT + 2 * kp]) = vhi;
      }
    }
  };

  f4 ok_[DP / 16], ov_[DP / 16];
#pragma unroll
  for (int n = 0; n < DP / 16; ++n) { ok_[n] = f4_zero(); ov_[n] = f4_zero(); }
  uint16_t* Pw = P[w];
  uint16_t* prw = Pw + lr * PT;
  const int* idxp = a.indices + pbase;
  const float* scp = a.scores + pbase;
  SlotRun run1, run2;
  run1.c = 0; run1.end = end1;
  run2.c = end1; run2.end = end2;
  issue(0);   // same order as in the loop: K/V tile, then the slot windows
  slot_window(run1, idxp, scp, lg, topk);
  slot_window(run2, idxp, scp, lg, topk);

  for (int kt = 0; kt < ntile; ++kt) {
    const int t0 = kt * KT, t1 = t0 + KT;
    __syncthreads();           // previous tile's K/V and P reads are done
    commit();
    // clear this wave's P rows (16 x PT bf16 = 144 uint4)
    for (int e = lane; e < 16 * PT / 8; e += 64) reinterpret_cast<uint4*>(Pw)[e] = make_uint4(0, 0, 0, 0);
    issue(min(kt + 1, ntile - 1));   // unconditional: keeps the wait counts static
    wave_lds_sync();
    // scatter this tile's weights from both runs and reload each window behind
    // it; the first pass uses windows loaded during the previous tile
    auto scatter_pass = [&]() __attribute__((always_inline)) -> bool {
      bool stop1 = false, stop2 = false;
      int n1 = slot_consume(run1, t0, t1, lg, m, prw, esum, stop1);
      int n2 = slot_consume(run2, t0, t1, lg, m, prw, esum, stop2);
      n1 += __shfl_xor(n1, 16, 64);
      n1 += __shfl_xor(n1, 32, 64);
      n2 += __shfl_xor(n2, 16, 64);
      n2 += __shfl_xor(n2, 32, 64);
      const uint64_t s1 = __ballot(stop1), s2 = __ballot(stop2);
      stop1 = ((s1 >> lr) | (s1 >> (lr + 16)) | (s1 >> (lr + 32)) | (s1 >> (lr + 48))) & 1;
      stop2 = ((s2 >> lr) | (s2 >> (lr + 16)) | (s2 >> (lr + 32)) | (s2 >> (lr + 48))) & 1;
      run1.c += n1;
      run2.c += n2;
      slot_window(run1, idxp, scp, lg, topk);
      slot_window(run2, idxp, scp, lg, topk);
      // a row that consumed its whole window without meeting t1 may have more keys in this tile
      return (!stop1 && run1.c < run1.end) || (!stop2 && run2.c < run2.end);
    };
    if (__ballot(scatter_pass())) {
      while (__ballot(scatter_pass())) {
      }
    }
    __syncthreads();           // K/V tile committed by all threads; P rows written
    // k_hat += P K, v_hat += P V  (P: 16 rows x 64 keys, K/V: 64 keys x 128 dims)
#pragma unroll
    for (int s = 0; s < KT / 32; ++s) {
      const uint4 pa = *reinterpret_cast<const uint4*>(&Pw[lr * PT + 32 * s + 8 * lg]);
#pragma unroll
      for (int n = 0; n < DP / 16; ++n) {
        const uint4 kb = *reinterpret_cast<const uint4*>(&Kt[(16 * n + lr) * PT + 32 * s + 8 * lg]);
        const uint4 vb = *reinterpret_cast<const uint4*>(&Vt[(16 * n + lr) * PT + 32 * s + 8 * lg]);
        ok_[n] = mma_bf16(as_bf8(pa), as_bf8(kb), ok_[n]);
        ov_[n] = mma_bf16(as_bf8(pa), as_bf8(vb), ov_[n]);
      }
    }
  }

  // ---- epilogue: normalise, gate, write key, stores ------------------------
  esum += __shfl_xor(esum, 16, 64);
  esum += __shfl_xor(esum, 32, 64);
  if (lg == 0) rowE[w][lr] = esum;
  wave_lds_sync();
  const float eps = a.eps;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int rl = 4 * lg + e;
    const int row = r0 + 16 * w + rl;
    const bool live = row < Tq;
    const long rg = (long)bh * Tq + (live ? row : 0);
    const float E = rowE[w][rl];
    const float inv = E > 0.f ? 1.f / E : 0.f;
    const long qoff = ((long)(b * Tq + (live ? row : 0)) * H + h) * DP;
    float kh[DP / 16], vh[DP / 16], ks[DP / 16];
    float pdot = 0.f, pkk = 0.f, phh = 0.f, pvv = 0.f;
#pragma unroll
    for (int n = 0; n < DP / 16; ++n) {
      kh[n] = ok_[n][e] * inv;
      vh[n] = ov_[n][e] * inv;
      ks[n] = live ? bf16_to_f32(reinterpret_cast<const uint16_t*>(a.self_key)[qoff + 16 * n + lr]) : 0.f;
      pdot += kh[n] * ks[n];
      pkk += ks[n] * ks[n];
      phh += kh[n] * kh[n];
      pvv += vh[n] * vh[n];
    }
    const float dot = group_sum(pdot, 16), kk2 = group_sum(pkk, 16), hh2 = group_sum(phh, 16),
                vv2 = group_sum(pvv, 16);
    const int kq = live ? a.counts[rg] : 0;
    float margin = 0.f;
    if (topk >= 2 && live) margin = a.top2[2 * rg] - a.top2[2 * rg + 1];
    if (kq == 0) margin = 0.f;
    const float conc = 1.f / (1.f + expf(-(margin / fmaxf(a.tau_c, eps))));
    const float self_norm = fmaxf(sqrtf(kk2), eps);
    const float kh_norm = fmaxf(sqrtf(hh2), eps);
    const float proj = dot / (self_norm * self_norm + eps);
    float pperp = 0.f;
#pragma unroll
    for (int n = 0; n < DP / 16; ++n) {
      const float d = kh[n] - proj * ks[n];
      pperp += d * d;
    }
    const float novelty = fminf(fmaxf(sqrtf(group_sum(pperp, 16)) / (kh_norm + eps), 0.f), 1.f);
    float wk[DP / 16];
#pragma unroll
    for (int n = 0; n < DP / 16; ++n) wk[n] = kh[n];
    float alpha_v = 0.f;
    if (a.budget != nullptr) {
      float wn2 = hh2;
      if (a.write_mode == 1) {
        const float c = dot / fmaxf(kk2, eps);
        float pw = 0.f;
#pragma unroll
        for (int n = 0; n < DP / 16; ++n) {
          wk[n] = kh[n] - c * ks[n];
          pw += wk[n] * wk[n];
        }
        wn2 = group_sum(pw, 16);
      }
      const float bud = live ? a.budget[(long)(b * Tq + row) * H + h] : 0.f;
      const float al = a.alpha_max * conc * novelty * (1.f / (1.f + expf(-bud)));
      const float prox = al * sqrtf(vv2) * sqrtf(wn2);
      alpha_v = al * fminf(1.f / fmaxf(prox, 1.f), 1.f);
    }
    if (!live) continue;
#pragma unroll
    for (int n = 0; n < DP / 16; ++n) {
      const long o = qoff + 16 * n + lr;
      if (a.k_hat) reinterpret_cast<uint16_t*>(a.k_hat)[o] = f32_to_bf16(kh[n]);
      if (a.write_key) reinterpret_cast<uint16_t*>(a.write_key)[o] = f32_to_bf16(wk[n]);
      reinterpret_cast<uint16_t*>(a.v_hat)[o] = f32_to_bf16(vh[n]);
    }
    if (a.alpha && lr == 0) a.alpha[(long)(b * Tq + row) * H + h] = alpha_v;
  }
}

hipError_t launch_sparse_gather_staged(const GatherArgs& a, const int32_t* split, hipStream_t st) {
  const int nqb = (a.Tq + QB - 1) / QB;
  gather_tile_kernel<<<dim3((unsigned)(a.B * a.H * nqb)), 256, 0, st>>>(a, split, nqb);
  return hipGetLastError();
}

}  // namespace sgsa
