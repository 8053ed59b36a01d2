// K2t: top-k weighted K/V sum by streaming K/V tiles through LDS (bf16, D = 128).
//
// Same result as K2 (gather.hip) -- k_hat, v_hat, the write key and the alpha
// gate (modelings/modeling_sgsa.py:126-134, :369-381, :497-504, :546-551) --
// computed the MI355X way: instead of fetching each of the ~2048 selected K
// and V rows of every query row from HBM/L2 with 16-byte gathers, a block of
// query rows walks the causal key range once in tiles of 64 keys.  Each tile
// of K and V is read with coalesced 16-byte loads (prefetched one tile ahead
// into registers) and stored transposed in LDS; the exact top-k weights of the
// tile form a sparse block P; then k_hat += P K and v_hat += P V run on
// v_mfma_f32_16x16x32_bf16 (P rounded to bf16, weights in (0,1]).
//
// Two kernels, by where the selection comes from:
//  * gather_list_kernel (layer path): K1 wrote, per 16-row wave and per key
//    tile, the selected (score, row, key) entries.  A block owns 128 rows,
//    each wave 32 (two MFMA row tiles sharing every K/V operand read from
//    LDS); each tile's entries are read with coalesced loads issued one tile
//    ahead and scattered into P without branches.  The softmax denominator
//    is P times a ones vector on the same MFMA, i.e. the sum of the bf16
//    weights that the numerators use.
//  * gather_tile_kernel (sgsa_sparse_gather_tiled): per-row slot lists of
//    K1's row output, 64-row blocks, 16 rows per wave.  Per row, slots
//    [0, split) and [split, count) each ascend in key index, so each row keeps
//    two cursors that advance monotonically with the tile index.  The four
//    lanes of a row hold a 32-slot window of each run in registers (16-byte
//    loads, reloaded behind the consumed part); a row that exhausts a window
//    inside one tile reloads it and goes round again.  Weights are exp(s - m)
//    with the row maximum m from K1 (top2), the denominator summed in fp32
//    from the unrounded weights.  Requires top_k % 4 == 0.
#include "common.h"
#include "kernels.h"

#include <float.h>

#include <type_traits>

namespace sgsa {

namespace {

constexpr int QB = 64;     // rows per block, slot-list kernel
constexpr int QL = 128;    // rows per block, tile-list kernel
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

// Scatter half HH of the window (positions base + 16HH + 4lg + e) with key in
// [t0, t1) into this wave's P row, without branches: lanes with nothing to
// write store into a padding column (`junk`, never read by the MFMA).
// Returns the lane's consumed count; `stop` is set when a held slot lies at or
// beyond t1 (the row is done with this tile).
template <int HH>
__device__ __forceinline__ int slot_half(const SlotRun& r, int t0, int t1, int lg, float m, uint16_t* prow, int junk,
                                         float& esum, int& stop) {
  const int js[4] = {r.ix[HH].x, r.ix[HH].y, r.ix[HH].z, r.ix[HH].w};
  const float ss[4] = {r.sc[HH].x, r.sc[HH].y, r.sc[HH].z, r.sc[HH].w};
  const int p0 = r.base + 16 * HH + 4 * lg - r.c;
  const unsigned span = (unsigned)(r.end - r.c);
  int n = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int inr = (unsigned)(p0 + e) < span;
    const int j = js[e];
    const int below = j < t1;
    const int take = inr & below;
    stop |= inr & (below ^ 1);
    n += take;
    const bool hit = take && j >= t0;
    const float wv = __expf(ss[e] - m);
    esum += hit ? wv : 0.f;
    prow[hit ? j - t0 : junk] = f32_to_bf16(wv);
  }
  return n;
}


// Transposed K/V tile staging for 256 threads: thread t loads keys 2kp, 2kp+1
// (kp = t % 32), 8-dim chunks cq = t / 32 and cq + 8, of one 64-key tile.  The
// loads are unconditional (key index clamped into [0, Tk)) so every thread
// issues the same number of memory operations per tile; keys past Tk are
// zeroed at commit.
struct KVStage {
  uint4 pk[2][2], pv[2][2];   // [chunk half][key of the pair]
  uint32_t pmask[2];          // all-ones for keys < Tk

  __device__ __forceinline__ void issue(const uint16_t* __restrict__ K, const uint16_t* __restrict__ V, int b, int h,
                                        int H, int Tk, int kt, int kp, int cq) {
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
  }

  __device__ __forceinline__ void commit(uint16_t* Kt, uint16_t* Vt, int kp, int cq) {
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
        *reinterpret_cast<uint32_t*>(&Kt[(8 * c + 2 * i) * PT + 2 * kp]) = __builtin_amdgcn_perm(k1[i], k0[i], 0x05040100u);
        *reinterpret_cast<uint32_t*>(&Kt[(8 * c + 2 * i + 1) * PT + 2 * kp]) = __builtin_amdgcn_perm(k1[i], k0[i], 0x07060302u);
        *reinterpret_cast<uint32_t*>(&Vt[(8 * c + 2 * i) * PT + 2 * kp]) = __builtin_amdgcn_perm(v1[i], v0[i], 0x05040100u);
        *reinterpret_cast<uint32_t*>(&Vt[(8 * c + 2 * i + 1) * PT + 2 * kp]) = __builtin_amdgcn_perm(v1[i], v0[i], 0x07060302u);
      }
    }
  }
};

// Normalise one 16-row MFMA tile of k_hat / v_hat sums (row 4lg + e of the
// tile in register e, column 16n + lr) by the row denominators E[e], then the
// gate: concentration from the top-2 margin, novelty of k_hat against the
// token's own key, the (residual) write key and alpha
// (modelings/modeling_sgsa.py:126-134, :369-381, :497-504, :546-551).
__device__ __forceinline__ void tile_epilogue(const GatherArgs& a, const f4 (&ok)[DP / 16], const f4 (&ov)[DP / 16],
                                              const float (&E)[4], int row0, int bh, int b, int h, int lr, int lg) {
  const int Tq = a.Tq, H = a.H;
  const float eps = a.eps;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int row = row0 + 4 * lg + e;
    const bool live = row < Tq;
    const long rg = (long)bh * Tq + (live ? row : 0);
    const float inv = E[e] > 0.f ? 1.f / E[e] : 0.f;
    const long qoff = ((long)(b * Tq + (live ? row : 0)) * H + h) * DP;
    float kh[DP / 16], vh[DP / 16], ks[DP / 16];
    float pdot = 0.f, pkk = 0.f, phh = 0.f, pvv = 0.f;
#pragma unroll
    for (int n = 0; n < DP / 16; ++n) {
      kh[n] = ok[n][e] * inv;
      vh[n] = ov[n][e] * inv;
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
    if (a.top_k >= 2 && live) margin = a.top2[2 * rg] - a.top2[2 * rg + 1];
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
    float alpha_v = 0.f, perp_ratio = 0.f;
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
        perp_ratio = fminf(fmaxf(sqrtf(wn2) / kh_norm, 0.f), 10.f);
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
    if (a.stats && lr == 0) {
      a.stats[rg] = kq > 0 ? inv : 0.f;   // the largest weight, exp(0) / E
      a.stats[(long)a.B * H * Tq + rg] = perp_ratio;
    }
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// Slot-list form (sgsa_sparse_gather_tiled)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gather_tile_kernel(GatherArgs a, const int32_t* __restrict__ split, int nqb) {
  __shared__ __align__(16) uint16_t Kt[DP * PT];
  __shared__ __align__(16) uint16_t Vt[DP * PT];
  __shared__ __align__(16) uint16_t P[4][16 * PT];
  __shared__ float rowE[4][16];

  const int BH = a.B * a.H;
  const int bid = blockIdx.x;
  const int bh = bid % BH;
  const int qb = nqb - 1 - bid / BH;    // heaviest query blocks first
  const int b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
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

  const int kend = min(Tk, min(Tq, r0 + QB) + a.q_offset);
  const int ntile = (kend + KT - 1) / KT;
  const int kp = tid & 31, cq = tid >> 5;
  KVStage kv;

  f4 ok_[DP / 16], ov_[DP / 16];
#pragma unroll
  for (int n = 0; n < DP / 16; ++n) { ok_[n] = f4_zero(); ov_[n] = f4_zero(); }
  uint16_t* Pw = P[w];
  uint16_t* prw = Pw + lr * PT;
  const int junk = KT + lg;   // padding column of the P row
  const int* idxp = a.indices + pbase;
  const float* scp = a.scores + pbase;
  SlotRun run1, run2;
  run1.c = 0; run1.end = end1;
  run2.c = end1; run2.end = end2;
  kv.issue(K, V, b, h, H, Tk, 0, kp, cq);
  slot_window(run1, idxp, scp, lg, topk);
  slot_window(run2, idxp, scp, lg, topk);
  // Nothing outstanding on entry: the loop head then only waits for the K/V
  // tile, not for the slot windows reloaded after it.
  __builtin_amdgcn_s_waitcnt(0);

  for (int kt = 0; kt < ntile; ++kt) {
    const int t0 = kt * KT, t1 = t0 + KT;
    __syncthreads();           // previous tile's K/V and P reads are done
    kv.commit(Kt, Vt, kp, cq);
    // clear this wave's P rows (16 x PT bf16 = 144 uint4)
    for (int e = lane; e < 16 * PT / 8; e += 64) reinterpret_cast<uint4*>(Pw)[e] = make_uint4(0, 0, 0, 0);
    kv.issue(K, V, b, h, H, Tk, min(kt + 1, ntile - 1), kp, cq);   // unconditional: static wait counts
    wave_lds_sync();
    // scatter this tile's weights from both runs and reload each window behind
    // it; the first pass uses windows loaded during the previous tile
    auto scatter_pass = [&]() __attribute__((always_inline)) -> bool {
      int stop1 = 0, stop2 = 0;
      int n1 = slot_half<0>(run1, t0, t1, lg, m, prw, junk, esum, stop1);
      int n2 = slot_half<0>(run2, t0, t1, lg, m, prw, junk, esum, stop2);
      // the second half matters only to rows that neither stopped nor ran out in the first
      const uint64_t h1 = ballot64(stop1), h2 = ballot64(stop2);
      const bool s1 = ((h1 >> lr) | (h1 >> (lr + 16)) | (h1 >> (lr + 32)) | (h1 >> (lr + 48))) & 1;
      const bool s2 = ((h2 >> lr) | (h2 >> (lr + 16)) | (h2 >> (lr + 32)) | (h2 >> (lr + 48))) & 1;
      if (ballot64((!s1 && run1.end > run1.base + 16) || (!s2 && run2.end > run2.base + 16))) {
        n1 += slot_half<1>(run1, t0, t1, lg, m, prw, junk, esum, stop1);
        n2 += slot_half<1>(run2, t0, t1, lg, m, prw, junk, esum, stop2);
      }
      n1 += __shfl_xor(n1, 16, 64);
      n1 += __shfl_xor(n1, 32, 64);
      n2 += __shfl_xor(n2, 16, 64);
      n2 += __shfl_xor(n2, 32, 64);
      const uint64_t g1 = ballot64(stop1), g2 = ballot64(stop2);
      const bool f1 = ((g1 >> lr) | (g1 >> (lr + 16)) | (g1 >> (lr + 32)) | (g1 >> (lr + 48))) & 1;
      const bool f2 = ((g2 >> lr) | (g2 >> (lr + 16)) | (g2 >> (lr + 32)) | (g2 >> (lr + 48))) & 1;
      run1.c += n1;
      run2.c += n2;
      slot_window(run1, idxp, scp, lg, topk);
      slot_window(run2, idxp, scp, lg, topk);
      // a row that consumed its whole window without meeting t1 may have more keys in this tile
      return (!f1 && run1.c < run1.end) || (!f2 && run2.c < run2.end);
    };
    if (ballot64(scatter_pass())) {
      while (ballot64(scatter_pass())) {
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

  esum += __shfl_xor(esum, 16, 64);
  esum += __shfl_xor(esum, 32, 64);
  if (lg == 0) rowE[w][lr] = esum;
  wave_lds_sync();
  float E[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) E[e] = rowE[w][4 * lg + e];
  tile_epilogue(a, ok_, ov_, E, r0 + 16 * w, bh, b, h, lr, lg);
}

// ---------------------------------------------------------------------------
// Tile-list form (layer path)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, 2) void gather_list_kernel(GatherArgs a, const uint2* __restrict__ tl,
                                                          const int32_t* __restrict__ toff, int nqb2, int nqb,
                                                          int ntmax) {
  __shared__ __align__(16) uint16_t Kt[DP * PT];
  __shared__ __align__(16) uint16_t Vt[DP * PT];
  __shared__ __align__(16) uint16_t P[4][32 * PT];
  __shared__ float mrow[4][32];

  const int BH = a.B * a.H;
  const int bid = blockIdx.x;
  const int bh = bid % BH;
  const int qb2 = nqb2 - 1 - bid / BH;   // heaviest row blocks first
  const int b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const int lr = lane & 15, lg = lane >> 4;
  const int Tq = a.Tq, Tk = a.Tk, H = a.H, topk = a.top_k;
  const int r0 = qb2 * QL;
  const int wr0 = r0 + 32 * w;   // first row of this wave
  const uint16_t* K = reinterpret_cast<const uint16_t*>(a.k);
  const uint16_t* V = reinterpret_cast<const uint16_t*>(a.v);

  const int kend = min(Tk, min(Tq, r0 + QL) + a.q_offset);
  const int ntile = (kend + KT - 1) / KT;
  const int kp = tid & 31, cq = tid >> 5;
  KVStage kv;

  // The wave's rows are the two 16-row waves 2(w&1), 2(w&1)+1 of K1's 64-row
  // block qb64; their lists end at that block's own last tile nt64.
  const int qb64 = 2 * qb2 + (w >> 1);
  const bool rvalid = qb64 < nqb;
  const int nt64 = rvalid ? (min(Tk, min(Tq, 64 * qb64 + 64) + a.q_offset) + KT - 1) / KT : 0;
  const int tlcap = 16 * (topk + TOPK_CAP);
  const long reg0 = ((long)bh * nqb + (rvalid ? qb64 : 0)) * 4 + 2 * (w & 1);
  const uint2* tlr[2] = {tl + reg0 * tlcap, tl + (reg0 + 1) * tlcap};
  const int32_t* tor[2] = {toff + reg0 * (ntmax + 1), toff + (reg0 + 1) * (ntmax + 1)};

  if (lane < 32) {
    const int row = wr0 + lane;
    mrow[w][lane] = row < Tq ? a.top2[2 * ((long)bh * Tq + row)] : 0.f;
  }

  // tile offsets, 64 at a time in one register per list, picked with readlane
  int ofb[2] = {-(1 << 20), -(1 << 20)}, ofr[2] = {0, 0};
  auto off_at = [&](int mt, int i) __attribute__((always_inline)) -> int {
    if (!rvalid) return 0;
    i = min(i, nt64);
    if (i < ofb[mt] || i >= ofb[mt] + 64) {   // wave-uniform
      ofb[mt] = i;
      ofr[mt] = tor[mt][min(i + lane, nt64)];
    }
    return __builtin_amdgcn_readlane(ofr[mt], i - ofb[mt]);
  };
  constexpr int NPE = 2;               // entries prefetched per lane and list: the first 128 of a tile
  uint2 pe[2][NPE];                    // [list][i]; reloaded for the next tile right after the scatter
  int c0[2] = {0, 0}, c1[2] = {0, 0};  // entry ranges of this tile
  auto entries = [&](uint2 (&d)[NPE], int mt, int e0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NPE; ++i) d[i] = tlr[mt][min(max(e0 + 64 * i + lane, 0), tlcap - 1)];
  };
  uint16_t* Pw = P[w];
  // scatter one entry of list mt without branches on the LDS address: invalid
  // lanes store into a padding column that the MFMA never reads
  auto scat = [&](uint2 en, int mt, bool valid) __attribute__((always_inline)) {
    const int rr = 16 * mt + ((en.y >> 8) & 15), kk = en.y & 63;
    const float wv = __expf(__uint_as_float(en.x) - mrow[w][rr]);
    Pw[valid ? rr * PT + kk : (16 * mt + lr) * PT + KT + lg] = f32_to_bf16(wv);
  };

  f4 ok_[2][DP / 16], ov_[2][DP / 16], es[2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    es[mt] = f4_zero();
#pragma unroll
    for (int n = 0; n < DP / 16; ++n) { ok_[mt][n] = f4_zero(); ov_[mt][n] = f4_zero(); }
  }
  const uint4 ones4 = make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);   // bf16 1.0 x 8

  wave_lds_sync();   // mrow
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    c0[mt] = off_at(mt, 0);
    c1[mt] = off_at(mt, 1);
    entries(pe[mt], mt, c0[mt]);
  }
  kv.issue(K, V, b, h, H, Tk, 0, kp, cq);
  __builtin_amdgcn_s_waitcnt(0);   // nothing outstanding on entry: static wait counts in the loop

  for (int kt = 0; kt < ntile; ++kt) {
    __syncthreads();           // previous tile's K/V and P reads are done
    kv.commit(Kt, Vt, kp, cq);
    // clear this wave's P rows (32 x PT bf16 = 288 uint4)
    for (int e = lane; e < 32 * PT / 8; e += 64) reinterpret_cast<uint4*>(Pw)[e] = make_uint4(0, 0, 0, 0);
    kv.issue(K, V, b, h, H, Tk, min(kt + 1, ntile - 1), kp, cq);   // unconditional: static wait counts
    wave_lds_sync();
    // the prefetched entries of both lists, without branches (independent LDS reads batch)
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int i = 0; i < NPE; ++i) scat(pe[mt][i], mt, c0[mt] + 64 * i + lane < c1[mt]);
    }
    // dense tiles: the rest, four loads in flight at a time
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      for (int e0 = c0[mt] + 64 * NPE; e0 < c1[mt]; e0 += 256) {
        uint2 en[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) en[i] = tlr[mt][min(max(e0 + 64 * i + lane, 0), tlcap - 1)];
#pragma unroll
        for (int i = 0; i < 4; ++i) scat(en[i], mt, e0 + 64 * i + lane < c1[mt]);
      }
    }
    // the next tile's first entries go straight into the registers just consumed
    // (no copies, so no wait on loads still in flight)
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      c0[mt] = off_at(mt, kt + 1);
      c1[mt] = off_at(mt, kt + 2);
      entries(pe[mt], mt, c0[mt]);
    }
    __syncthreads();           // K/V tile committed by all threads; P rows written
    // k_hat += P K, v_hat += P V, E += P 1  (two 16-row tiles share each K/V operand)
    // Operand reads are software-pipelined by hand: the K/V fragments of step
    // n+1 are in flight while step n multiplies (the accumulators leave too few
    // registers for the compiler to hoist them on its own).
#pragma unroll
    for (int s = 0; s < KT / 32; ++s) {
      const int cofs = 32 * s + 8 * lg;
      const uint4 pa0 = *reinterpret_cast<const uint4*>(&Pw[lr * PT + cofs]);
      const uint4 pa1 = *reinterpret_cast<const uint4*>(&Pw[(16 + lr) * PT + cofs]);
      uint4 kb[2], vb[2];
      kb[0] = *reinterpret_cast<const uint4*>(&Kt[lr * PT + cofs]);
      vb[0] = *reinterpret_cast<const uint4*>(&Vt[lr * PT + cofs]);
#pragma unroll
      for (int n = 0; n < DP / 16; ++n) {
        if (n + 1 < DP / 16) {
          kb[(n + 1) & 1] = *reinterpret_cast<const uint4*>(&Kt[(16 * (n + 1) + lr) * PT + cofs]);
          vb[(n + 1) & 1] = *reinterpret_cast<const uint4*>(&Vt[(16 * (n + 1) + lr) * PT + cofs]);
        }
        ok_[0][n] = mma_bf16(as_bf8(pa0), as_bf8(kb[n & 1]), ok_[0][n]);
        ok_[1][n] = mma_bf16(as_bf8(pa1), as_bf8(kb[n & 1]), ok_[1][n]);
        ov_[0][n] = mma_bf16(as_bf8(pa0), as_bf8(vb[n & 1]), ov_[0][n]);
        ov_[1][n] = mma_bf16(as_bf8(pa1), as_bf8(vb[n & 1]), ov_[1][n]);
      }
      es[0] = mma_bf16(as_bf8(pa0), as_bf8(ones4), es[0]);
      es[1] = mma_bf16(as_bf8(pa1), as_bf8(ones4), es[1]);
    }
  }

#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const float E[4] = {es[mt][0], es[mt][1], es[mt][2], es[mt][3]};
    tile_epilogue(a, ok_[mt], ov_[mt], E, wr0 + 16 * mt, bh, b, h, lr, lg);
  }
}

// ---------------------------------------------------------------------------
// Threshold form (layer path): the selection is recomputed, not read.
//
// K1 in threshold mode leaves per row only the exact top-k cut (th, cut): key j
// with score s is selected iff j is causal for the row and s > th, or s == th
// and j <= cut (ties at the threshold go to the lowest indices).  This kernel
// recomputes each tile's scores with K1's products -- A operand K rows, B
// operand q, the same 32 dims per instruction -- so its accumulators are K1's
// bit for bit.  The cut is applied to them exactly: per row, the smallest
// accumulator whose fp32 score (acc * mscale) reaches th, or exceeds it, is
// found once by bisection, and a score is then selected by one compare.  The
// weights exp(s - max) never leave registers: exp2(acc * mscale*log2e -
// max*log2e) (one fused multiply-add), and the score accumulator C[key][row]
// is the A operand of P K once MFMA row 4a + b of half h of a 32-key chunk
// holds key 8a + 4h + b.
//
// K and V tiles go global -> LDS with direct buffer loads (no VGPR staging),
// double-buffered.  LDS row r of a tile holds key tile_row_key(r) (the order
// above) with a pitch of 288 bytes, and its 16-byte chunk c at slot
// c ^ ((r >> 3) & 1): the score operand reads (16 rows, one chunk) and the
// transposing reads (4 rows x four 8-byte pieces per 16 lanes) then hit
// distinct banks, and the slot of chunk c + 2n is the slot of c plus 2n.  The
// B operands of P K and P V come from ds_read_b64_tr_b16: within 16 lanes,
// lane i gets element i % 4 of the 8 bytes that lane 4e + i / 4 addresses,
// e = 0..3, so lanes addressing keys 8g + e, dims 16n + 4(i/4).. receive dim
// 16n + i of four consecutive keys -- the MFMA's B layout.
// ---------------------------------------------------------------------------
constexpr int RP = DP + 16;            // LDS pitch (bf16) of a K/V tile row: 16 data chunks + 2 pad
constexpr int TILE_SLOTS = KT * RP / 8;   // 16-byte slots of one tile: 1152 = 18 loads of 64 lanes

__device__ __forceinline__ int tile_row_key(int r) {
  return (r & 32) + 8 * ((r >> 2) & 3) + 4 * ((r >> 4) & 1) + (r & 3);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two floats to two bf16 (round to nearest even) in one v_cvt_pk_bf16_f32; lo in bits 0-15.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2_t));
}

// Smallest accumulator value c whose score c * mscale (one rounded fp32
// product, monotone in c for mscale > 0) is >= t, by bisection over the
// order-preserving keys.  t = -inf gives -inf, t = +inf gives +inf.
__device__ __forceinline__ float acc_bound(float t, float mscale) {
#pragma clang fp contract(off)
  if (!(t > -INFINITY)) return -INFINITY;
  if (!(t < INFINITY)) return INFINITY;
  uint32_t lo = 0x007fffffu, hi = 0xff800000u;   // keys of -inf (fails) and +inf (passes)
  while (hi - lo > 1u) {
    const uint32_t mid = lo + ((hi - lo) >> 1);
    if (key_to_f32(mid) * mscale >= t) hi = mid;
    else lo = mid;
  }
  return key_to_f32(hi);
}

__device__ __forceinline__ s16x4 lds_read_tr(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
}

// DBG: a known-answer variant that writes, instead of the gathered rows, each
// row's selection summary {count, sum of key indices, xor of (index * 2654435761)}
// to a.sel_dbg [B,H,Tq,3] -- the selection applied exactly as the gather applies it.
template <bool DBG>
__global__ __launch_bounds__(256, 2) void gather_thr_kernel(GatherArgs a, const uint16_t* __restrict__ qg,
                                                         const uint2* __restrict__ thr, float mscale, int nqb2) {
  __shared__ __align__(16) uint16_t K0[KT * RP], V0[KT * RP], K1[KT * RP], V1[KT * RP];

  const int BH = a.B * a.H;
  const int bid = blockIdx.x;
  const int bh = bid % BH;
  const int qb2 = nqb2 - 1 - bid / BH;   // heaviest row blocks first
  const int b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const int lr = lane & 15, lg = lane >> 4;
  const int Tq = a.Tq, Tk = a.Tk, H = a.H;
  const int r0 = qb2 * QL;
  const int wr0 = r0 + 32 * w;   // first row of this wave
  const uint16_t* K = reinterpret_cast<const uint16_t*>(a.k);
  const uint16_t* V = reinterpret_cast<const uint16_t*>(a.v);

  const int kend = min(Tk, min(Tq, r0 + QL) + a.q_offset);
  const int ntile = (kend + KT - 1) / KT;

  // Direct loads.  One buffer resource per head covers its keys [0, Tk): a key
  // past Tk reads as zeros (never selected).  Wave w issues the tile's loads
  // w, w + 4, ... (18 per tensor); lane l of load i fills slot 64 i + l, i.e.
  // row (64 i + l) / 18, slot (64 i + l) % 18 (slots 16, 17 are padding and
  // re-read chunk 0).  The byte offsets within a tile do not change from tile
  // to tile; the tile start goes into the scalar offset.
  const long hbase = ((long)b * Tk * H + h) * DP;
  const int rbytes = H * DP * 2;   // bytes between consecutive keys of a head
  const int nrec = (Tk - 1) * rbytes + DP * 2;
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(K + hbase), 0, nrec, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(V + hbase), 0, nrec, 0x00020000);
  int doff[5];
#pragma unroll
  for (int t = 0; t < 5; ++t) {
    const int slot = 64 * (w + 4 * t) + lane;
    const int r = slot / 18, p = slot % 18;
    const int c = p < 16 ? p ^ ((r >> 3) & 1) : 0;
    doff[t] = tile_row_key(min(r, KT - 1)) * rbytes + 16 * c;
  }
  // (the tile start goes into the per-lane offset, which the range check covers)
  auto dma = [&](int kt, uint16_t* Kd, uint16_t* Vd) __attribute__((always_inline)) {
    const int toff = kt * KT * rbytes;
#pragma unroll
    for (int t = 0; t < 5; ++t) {
      const int i = w + 4 * t;
      if (i < TILE_SLOTS / 64) {   // wave-uniform
        __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (__attribute__((address_space(3))) void*)(Kd + 512 * i), 16,
                                                 doff[t] + toff, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (__attribute__((address_space(3))) void*)(Vd + 512 * i), 16,
                                                 doff[t] + toff, 0, 0, 0);
      }
    }
  };
  // A tile that reaches past Tk: its rows there are never selected (weight 0),
  // but 0 * NaN is NaN, so whatever the out-of-range loads leave in LDS must be
  // finite.  Zero the buffers once (block-uniform), before any load lands.
  if (Tk % KT != 0) {
    uint4* z[4] = {reinterpret_cast<uint4*>(K0), reinterpret_cast<uint4*>(V0), reinterpret_cast<uint4*>(K1),
                   reinterpret_cast<uint4*>(V1)};
#pragma unroll
    for (int u = 0; u < 4; ++u)
      for (int i = tid; i < KT * RP / 8; i += 256) z[u][i] = make_uint4(0, 0, 0, 0);
    __syncthreads();
  }

  // The lane's rows wr0 + 16 mt + lr: q (B operand of the score product), the
  // cut, the row maximum and the causal end.  Dead rows select nothing.
  // Selection and weights work on the raw accumulator c (score = c * mscale):
  // ce[mt] / cg[mt] are the smallest c with score >= th / score > th, and the
  // weight exp(score - max) is evaluated as exp2(c * mscale*log2e - max*log2e).
  bf16x8 qf[2][4];
  float ce[2], cg[2], mxl[2];
  int cut[2], nv[2];
  const float msl = mscale * 1.44269504f;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const int row = wr0 + 16 * mt + lr;
    const bool live = row < Tq;
    const uint16_t* qp = qg + ((long)(b * Tq + (live ? row : 0)) * H + h) * DP + 8 * lg;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u16x8 raw = *reinterpret_cast<const u16x8*>(qp + 32 * s);
      if (!live) raw = (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
      qf[mt][s] = __builtin_bit_cast(bf16x8, raw);
    }
    float th = INFINITY, mx = 0.f;
    cut[mt] = -1; nv[mt] = 0;
    if (live) {
      const long rg = (long)bh * Tq + row;
      const uint2 t = thr[rg];
      th = __uint_as_float(t.x);
      cut[mt] = (int)t.y;
      mx = a.top2[2 * rg];
      nv[mt] = a.row_nv != nullptr ? a.row_nv[(long)b * Tq + row] : max(0, min(Tk, row + a.q_offset + 1));
    }
    ce[mt] = acc_bound(th, mscale);
    cg[mt] = acc_bound(next_up(th), mscale);
    mxl[mt] = mx * 1.44269504f;
  }
  // every key below wmin is valid for every row of the wave (the causal range; with a
  // padding mask the least of the rows' valid prefixes)
  int wmin = wr0 + 31 < Tq ? max(0, min(Tk, wr0 + a.q_offset + 1)) : 0;
  if (a.row_nv != nullptr) {
    int m = min(nv[0], nv[1]);
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) m = min(m, __shfl_xor(m, o, 64));
    wmin = wr0 + 31 < Tq ? __builtin_amdgcn_readfirstlane(m) : 0;
  }

  f4 ok_[2][DP / 16], ov_[2][DP / 16], es[2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    es[mt] = f4_zero();
#pragma unroll
    for (int n = 0; n < DP / 16; ++n) { ok_[mt][n] = f4_zero(); ov_[mt][n] = f4_zero(); }
  }
  const uint4 ones4 = make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);   // bf16 1.0 x 8
  uint32_t dcnt[2] = {0u, 0u}, dsum[2] = {0u, 0u}, dxor[2] = {0u, 0u};   // DBG only

  // score operand: row 32 sp + 16 hf + lr, chunk 4 s + lg -> slot 4 s + (lg ^ (lr >> 3))
  const int s_off = lr * RP + 8 * (lg ^ (lr >> 3));
  // transposing reads: row 32 sp + 16 jb + 4 lg + lr / 4, dims 16 n + 4 (lr % 4) ..
  // -> chunk 2n + (lr % 4) / 2 at slot 2n + ((lr % 4) / 2 ^ lg / 2), byte 8 (lr % 2) in it
  const int t_off = (4 * lg + (lr >> 2)) * RP + 8 * (((lr & 3) >> 1) ^ (lg >> 1)) + 4 * (lr & 1);

  // One 32-key chunk sp of the tile in (Kc, Vc) starting at key t0: scores,
  // weights, then k_hat += P K, v_hat += P V, E += P 1.  fast: every key is
  // causal for every row and no row's tie cut falls inside the tile, so
  // acc >= the[mt] decides; only the weights depend on it.
  auto chunk = [&](bool fast, const uint16_t* Kc, const uint16_t* Vc, int sp, int t0, const float (&the)[2])
      __attribute__((always_inline)) {
    // scores of both halves (16 keys each) first, then the weights of each: a half's
    // weights read accumulators that finished while the other half's products ran.
    // A operand rows 32 sp + 16 hf + lr of the tile; the weights of keys 8 lg + 4 hf + i
    uint32_t pw[2][4];
    f4 sc[2][2] = {{f4_zero(), f4_zero()}, {f4_zero(), f4_zero()}};
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint4 kf = *reinterpret_cast<const uint4*>(&Kc[(32 * sp + 16 * hf) * RP + s_off + 32 * s]);
        sc[hf][0] = mma_bf16(as_bf8(kf), qf[0][s], sc[hf][0]);
        sc[hf][1] = mma_bf16(as_bf8(kf), qf[1][s], sc[hf][1]);
      }
    }
    auto half = [&](int hf) __attribute__((always_inline)) {
      auto weights = [&](auto fast_t) __attribute__((always_inline)) {
        constexpr bool FAST = decltype(fast_t)::value;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          float p[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float c = sc[hf][mt][i];
            bool sel;
            if constexpr (FAST) {
              sel = c >= the[mt];
            } else {
              const int j = t0 + 32 * sp + 8 * lg + 4 * hf + i;
              sel = (j < nv[mt]) & ((c >= cg[mt]) | ((c >= ce[mt]) & (j <= cut[mt])));   // no short circuit: no branches
            }
            const float e = __builtin_amdgcn_exp2f(fmaf(c, msl, -mxl[mt]));
            p[i] = sel ? e : 0.f;
            if constexpr (DBG) {
              const uint32_t j = (uint32_t)(t0 + 32 * sp + 8 * lg + 4 * hf + i);
              dcnt[mt] += sel ? 1u : 0u;
              dsum[mt] += sel ? j : 0u;
              dxor[mt] ^= sel ? j * 2654435761u : 0u;
            }
          }
          pw[mt][2 * hf] = pack_bf16x2(p[0], p[1]);
          pw[mt][2 * hf + 1] = pack_bf16x2(p[2], p[3]);
        }
      };
      if (fast) weights(std::true_type{});
      else weights(std::false_type{});
    };
    half(0);
    half(1);
    const uint4 pa[2] = {make_uint4(pw[0][0], pw[0][1], pw[0][2], pw[0][3]),
                         make_uint4(pw[1][0], pw[1][1], pw[1][2], pw[1][3])};
    __builtin_amdgcn_sched_barrier(0);
    // B operands one dim block ahead of the products (software pipeline kept
    // by scheduling barriers: the accumulators leave no room for more)
    const uint16_t* kt_ = Kc + 32 * sp * RP + t_off;
    const uint16_t* vt_ = Vc + 32 * sp * RP + t_off;
    auto operands = [&](int n, bf16x8& kb, bf16x8& vb) __attribute__((always_inline)) {
      const s16x4 k0 = lds_read_tr(kt_ + 16 * n), k1 = lds_read_tr(kt_ + 16 * RP + 16 * n);
      const s16x4 v0 = lds_read_tr(vt_ + 16 * n), v1 = lds_read_tr(vt_ + 16 * RP + 16 * n);
      kb = __builtin_bit_cast(bf16x8, __builtin_shufflevector(k0, k1, 0, 1, 2, 3, 4, 5, 6, 7));
      vb = __builtin_bit_cast(bf16x8, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    bf16x8 kb[2], vb[2];
    operands(0, kb[0], vb[0]);
#pragma unroll
    for (int n = 0; n < DP / 16; ++n) {
      if (n + 1 < DP / 16) operands(n + 1, kb[(n + 1) & 1], vb[(n + 1) & 1]);
      ok_[0][n] = mma_bf16(as_bf8(pa[0]), kb[n & 1], ok_[0][n]);
      ok_[1][n] = mma_bf16(as_bf8(pa[1]), kb[n & 1], ok_[1][n]);
      ov_[0][n] = mma_bf16(as_bf8(pa[0]), vb[n & 1], ov_[0][n]);
      ov_[1][n] = mma_bf16(as_bf8(pa[1]), vb[n & 1], ov_[1][n]);
      __builtin_amdgcn_sched_barrier(0);
    }
    es[0] = mma_bf16(as_bf8(pa[0]), as_bf8(ones4), es[0]);
    es[1] = mma_bf16(as_bf8(pa[1]), as_bf8(ones4), es[1]);
  };

  auto tile = [&](int kt, const uint16_t* Kc, const uint16_t* Vc) __attribute__((always_inline)) {
    const int t0 = kt * KT;
    float the[2];
    bool mixed = false;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const bool le = t0 + KT - 1 <= cut[mt], gt = t0 > cut[mt];
      mixed |= !(le || gt);
      the[mt] = le ? ce[mt] : cg[mt];
    }
    const bool fast = t0 + KT <= wmin && !ballot64(mixed);
#pragma unroll
    for (int sp = 0; sp < KT / 32; ++sp) chunk(fast, Kc, Vc, sp, t0, the);
  };

  // Double buffering (two static buffers, so the compiler sees that the loads
  // in flight never alias the tile being read): the loads of tile kt + 1 run
  // while tile kt is multiplied.
  dma(0, K0, V0);
  for (int kt = 0; kt < ntile; kt += 2) {
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's loads of tile kt are done
    __syncthreads();                      // ... every wave's; buffer 1 is free
    if (kt + 1 < ntile) dma(kt + 1, K1, V1);
    tile(kt, K0, V0);
    if (kt + 1 < ntile) {
      __builtin_amdgcn_s_waitcnt(0x0f70);
      __syncthreads();
      if (kt + 2 < ntile) dma(kt + 2, K0, V0);
      tile(kt + 1, K1, V1);
    }
  }

  if constexpr (DBG) {
    // lanes lr, lr + 16, lr + 32, lr + 48 hold row lr's keys
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int o = 16; o < 64; o <<= 1) {
        dcnt[mt] += __shfl_xor(dcnt[mt], o, 64);
        dsum[mt] += __shfl_xor(dsum[mt], o, 64);
        dxor[mt] ^= __shfl_xor(dxor[mt], o, 64);
      }
      const int row = wr0 + 16 * mt + lr;
      if (lg == 0 && row < Tq) {
        int32_t* d = a.sel_dbg + ((long)bh * Tq + row) * 3;
        d[0] = (int32_t)dcnt[mt];
        d[1] = (int32_t)dsum[mt];
        d[2] = (int32_t)dxor[mt];
      }
    }
    return;
  }
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const float E[4] = {es[mt][0], es[mt][1], es[mt][2], es[mt][3]};
    tile_epilogue(a, ok_[mt], ov_[mt], E, wr0 + 16 * mt, bh, b, h, lr, lg);
  }
}

// ---------------------------------------------------------------------------
// Dense causal GQA attention for prefill (the hybrid decoder's dense layers,
// modelings/hybrid_dense_delta_topk.py:178-192) with the reference's rounding
// points: s = bf16(bf16(q.k) * 1/sqrt(d)), p = bf16(exp(s - max) / sum) with
// the softmax in fp32 over every causal key, o = bf16(sum p v) in fp32.
// Because p is rounded after normalisation, the row maximum and sum come
// first: PASS 1 walks the causal keys for them (scores only, K tiles only);
// PASS 2 walks them again, forms p and accumulates p V.  The K/V tiles, the
// score operand layout and the transposing reads are those of
// gather_thr_kernel: 128 query rows per block, 32 per wave.
//   q, out [B, H, Tq, D]; k, v [B, Hkv, L, D] (a cache of L rows, keys
//   [0, pos0 + Tq) valid); query row t sits at key position pos0 + t.
// e^x as 2^(x log2 e) on v_exp_f32 (relative error below 1e-5 for the |x| < 100 a softmax
// meets, far inside the bf16 rounding of the probabilities); e^-inf = 0.
__device__ __forceinline__ float dexp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

struct DenseAttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int B, H, Hkv, Tq, pos0;
  long L;
  float scale;
  float2* stats;   // [B, H, Tq]: (max, sum of exp(s - max))
  uint16_t* out;
};

template <int PASS>
__global__ __launch_bounds__(256, 2) void dense_attn_kernel(DenseAttnArgs a, int nqb2) {
  __shared__ __align__(16) uint16_t K0[KT * RP], V0[PASS == 2 ? KT * RP : 8], K1[KT * RP], V1[PASS == 2 ? KT * RP : 8];

  const int BH = a.B * a.H;
  const int bid = blockIdx.x;
  const int bh = bid % BH;
  const int qb2 = nqb2 - 1 - bid / BH;   // heaviest row blocks first
  const int b = bh / a.H, h = bh % a.H, kh = h / (a.H / a.Hkv);
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int Tq = a.Tq;
  const int Tk = a.pos0 + Tq;   // valid keys
  const int r0 = qb2 * QL;
  const int wr0 = r0 + 32 * w;
  const int kend = min(Tk, min(Tq, r0 + QL) + a.pos0);
  const int ntile = (kend + KT - 1) / KT;

  const long hbase = ((long)(b * a.Hkv + kh) * a.L) * DP;
  const int rbytes = DP * 2;
  const int nrec = Tk * rbytes;
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.k + hbase), 0, nrec, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.v + hbase), 0, nrec, 0x00020000);
  int doff[5];
#pragma unroll
  for (int t = 0; t < 5; ++t) {
    const int slot = 64 * (w + 4 * t) + lane;
    const int r = slot / 18, p = slot % 18;
    const int c = p < 16 ? p ^ ((r >> 3) & 1) : 0;
    doff[t] = tile_row_key(min(r, KT - 1)) * rbytes + 16 * c;
  }
  auto dma = [&](int kt, uint16_t* Kd, uint16_t* Vd) __attribute__((always_inline)) {
    const int toff = kt * KT * rbytes;
#pragma unroll
    for (int t = 0; t < 5; ++t) {
      const int i = w + 4 * t;
      if (i < TILE_SLOTS / 64) {   // wave-uniform
        __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (__attribute__((address_space(3))) void*)(Kd + 512 * i), 16,
                                                 doff[t] + toff, 0, 0, 0);
        if constexpr (PASS == 2)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (__attribute__((address_space(3))) void*)(Vd + 512 * i), 16,
                                                   doff[t] + toff, 0, 0, 0);
      }
    }
  };
  // a tile reaching past the valid keys: those LDS rows must hold finite values (their weights are 0)
  if (Tk % KT != 0) {
    uint4* z[2] = {reinterpret_cast<uint4*>(K0), reinterpret_cast<uint4*>(K1)};
#pragma unroll
    for (int u = 0; u < 2; ++u)
      for (int i = tid; i < KT * RP / 8; i += 256) z[u][i] = make_uint4(0, 0, 0, 0);
    if constexpr (PASS == 2) {
      uint4* zv[2] = {reinterpret_cast<uint4*>(V0), reinterpret_cast<uint4*>(V1)};
#pragma unroll
      for (int u = 0; u < 2; ++u)
        for (int i = tid; i < KT * RP / 8; i += 256) zv[u][i] = make_uint4(0, 0, 0, 0);
    }
    __syncthreads();
  }

  // the lane's rows wr0 + 16 mt + lr: q (B operand of the score product) and the causal end
  bf16x8 qf[2][4];
  int nv[2];
  float mrow[2], ilrow[2];   // PASS 2: the row's maximum and 1 / sum
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const int row = wr0 + 16 * mt + lr;
    const bool live = row < Tq;
    const uint16_t* qp = a.q + (((long)b * a.H + h) * Tq + (live ? row : 0)) * DP + 8 * lg;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u16x8 raw = *reinterpret_cast<const u16x8*>(qp + 32 * s);
      if (!live) raw = (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
      qf[mt][s] = __builtin_bit_cast(bf16x8, raw);
    }
    nv[mt] = live ? min(Tk, row + a.pos0 + 1) : 0;
    mrow[mt] = 0.f;
    ilrow[mt] = 0.f;
    if constexpr (PASS == 2) {
      if (live) {
        const float2 st = a.stats[((long)b * a.H + h) * Tq + row];
        mrow[mt] = st.x;
        ilrow[mt] = 1.0f / st.y;
      }
    }
  }
  const int wmin = wr0 + 31 < Tq ? min(Tk, wr0 + a.pos0 + 1) : 0;   // keys below are causal for every row of the wave

  float ml[2] = {-INFINITY, -INFINITY}, ll[2] = {0.f, 0.f};   // PASS 1: the lane's running max and sum
  f4 ov_[2][PASS == 2 ? DP / 16 : 1];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int n = 0; n < (PASS == 2 ? DP / 16 : 1); ++n) ov_[mt][n] = f4_zero();

  const int s_off = lr * RP + 8 * (lg ^ (lr >> 3));
  const int t_off = (4 * lg + (lr >> 2)) * RP + 8 * (((lr & 3) >> 1) ^ (lg >> 1)) + 4 * (lr & 1);
  const float scale = a.scale;

  auto chunk = [&](bool full, const uint16_t* Kc, const uint16_t* Vc, int sp, int t0) __attribute__((always_inline)) {
    uint32_t pw[2][4];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      f4 sc[2] = {f4_zero(), f4_zero()};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint4 kf = *reinterpret_cast<const uint4*>(&Kc[(32 * sp + 16 * hf) * RP + s_off + 32 * s]);
        sc[0] = mma_bf16(as_bf8(kf), qf[0][s], sc[0]);
        sc[1] = mma_bf16(as_bf8(kf), qf[1][s], sc[1]);
      }
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        float sv[4];
        bool ok[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = t0 + 32 * sp + 8 * lg + 4 * hf + i;
          ok[i] = full || j < nv[mt];
          // the product rounded to bf16, scaled, rounded again (the reference's bf16 matmul and scaling)
          sv[i] = bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16(sc[mt][i])) * scale));
        }
        if constexpr (PASS == 1) {
          float tm = -INFINITY;
#pragma unroll
          for (int i = 0; i < 4; ++i) tm = fmaxf(tm, ok[i] ? sv[i] : -INFINITY);
          const float mn = fmaxf(ml[mt], tm);
          if (mn > -INFINITY) {
            float acc = ll[mt] * dexp(ml[mt] - mn);   // ml = -inf: exp(-inf) = 0
#pragma unroll
            for (int i = 0; i < 4; ++i) acc += ok[i] ? dexp(sv[i] - mn) : 0.f;
            ll[mt] = acc;
            ml[mt] = mn;
          }
        } else {
          float p[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) p[i] = ok[i] ? dexp(sv[i] - mrow[mt]) * ilrow[mt] : 0.f;
          pw[mt][2 * hf] = pack_bf16x2(p[0], p[1]);
          pw[mt][2 * hf + 1] = pack_bf16x2(p[2], p[3]);
        }
      }
    }
    if constexpr (PASS == 2) {
      const uint4 pa[2] = {make_uint4(pw[0][0], pw[0][1], pw[0][2], pw[0][3]),
                           make_uint4(pw[1][0], pw[1][1], pw[1][2], pw[1][3])};
      __builtin_amdgcn_sched_barrier(0);
      const uint16_t* vt_ = Vc + 32 * sp * RP + t_off;
      auto operands = [&](int n, bf16x8& vb) __attribute__((always_inline)) {
        const s16x4 v0 = lds_read_tr(vt_ + 16 * n), v1 = lds_read_tr(vt_ + 16 * RP + 16 * n);
        vb = __builtin_bit_cast(bf16x8, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
      };
      bf16x8 vb[2];
      operands(0, vb[0]);
#pragma unroll
      for (int n = 0; n < DP / 16; ++n) {
        if (n + 1 < DP / 16) operands(n + 1, vb[(n + 1) & 1]);
        ov_[0][n] = mma_bf16(as_bf8(pa[0]), vb[n & 1], ov_[0][n]);
        ov_[1][n] = mma_bf16(as_bf8(pa[1]), vb[n & 1], ov_[1][n]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  auto tile = [&](int kt, const uint16_t* Kc, const uint16_t* Vc) __attribute__((always_inline)) {
    const int t0 = kt * KT;
    const bool full = t0 + KT <= wmin;
#pragma unroll
    for (int sp = 0; sp < KT / 32; ++sp) chunk(full, Kc, Vc, sp, t0);
  };

  dma(0, K0, V0);
  for (int kt = 0; kt < ntile; kt += 2) {
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's loads of tile kt are done
    __syncthreads();                      // ... every wave's; buffer 1 is free
    if (kt + 1 < ntile) dma(kt + 1, K1, V1);
    tile(kt, K0, V0);
    if (kt + 1 < ntile) {
      __builtin_amdgcn_s_waitcnt(0x0f70);
      __syncthreads();
      if (kt + 2 < ntile) dma(kt + 2, K0, V0);
      tile(kt + 1, K1, V1);
    }
  }

  if constexpr (PASS == 1) {
    // lanes lr, lr + 16, lr + 32, lr + 48 hold row lr's keys
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      float m = ml[mt], l = ll[mt];
#pragma unroll
      for (int o = 16; o < 64; o <<= 1) {
        const float m2 = __shfl_xor(m, o, 64), l2 = __shfl_xor(l, o, 64);
        const float mn = fmaxf(m, m2);
        l = (m > -INFINITY ? l * dexp(m - mn) : 0.f) + (m2 > -INFINITY ? l2 * dexp(m2 - mn) : 0.f);
        m = mn;
      }
      const int row = wr0 + 16 * mt + lr;
      if (lg == 0 && row < Tq) a.stats[((long)b * a.H + h) * Tq + row] = make_float2(m, l);
    }
  } else {
    // accumulator element e of lane (lr, lg): row 16 mt + 4 lg + e of the wave, dim 16 n + lr
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = wr0 + 16 * mt + 4 * lg + e;
        if (row < Tq) {
          uint16_t* op = a.out + (((long)b * a.H + h) * Tq + row) * DP + lr;
#pragma unroll
          for (int n = 0; n < DP / 16; ++n) op[16 * n] = f32_to_bf16(ov_[mt][n][e]);
        }
      }
  }
}

hipError_t launch_dense_attn(const void* q, const void* k, const void* v, int B, int H, int Hkv, int Tq, int pos0,
                             long L, float2* stats, void* out, hipStream_t st) {
  DenseAttnArgs a{};
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v;
  a.B = B; a.H = H; a.Hkv = Hkv; a.Tq = Tq; a.pos0 = pos0; a.L = L;
  a.scale = (float)(1.0 / 11.313708498984761);   // 1 / sqrt(128), as the fp32 of the double
  a.stats = stats; a.out = (uint16_t*)out;
  const int nqb2 = (Tq + QL - 1) / QL;
  const dim3 grid((unsigned)(B * H * nqb2));
  dense_attn_kernel<1><<<grid, 256, 0, st>>>(a, nqb2);
  dense_attn_kernel<2><<<grid, 256, 0, st>>>(a, nqb2);
  return hipGetLastError();
}

hipError_t launch_sparse_gather_staged(const GatherArgs& a, const int32_t* split, hipStream_t st) {
  const int nqb = (a.Tq + QB - 1) / QB;
  gather_tile_kernel<<<dim3((unsigned)(a.B * a.H * nqb)), 256, 0, st>>>(a, split, nqb);
  return hipGetLastError();
}

hipError_t launch_sparse_gather_lists(const GatherArgs& a, const uint2* tl_list, const int32_t* tl_off,
                                      hipStream_t st) {
  const int nqb = (a.Tq + QB - 1) / QB;
  const int nqb2 = (a.Tq + QL - 1) / QL;
  const int ntmax = (a.Tk + KT - 1) / KT;
  gather_list_kernel<<<dim3((unsigned)(a.B * a.H * nqb2)), 256, 0, st>>>(a, tl_list, tl_off, nqb2, nqb, ntmax);
  return hipGetLastError();
}

hipError_t launch_sparse_gather_thr(const GatherArgs& a, const void* q, const uint2* thr, float mscale,
                                    hipStream_t st) {
  const int nqb2 = (a.Tq + QL - 1) / QL;
  if (a.sel_dbg)
    gather_thr_kernel<true><<<dim3((unsigned)(a.B * a.H * nqb2)), 256, 0, st>>>(
        a, reinterpret_cast<const uint16_t*>(q), thr, mscale, nqb2);
  else
    gather_thr_kernel<false><<<dim3((unsigned)(a.B * a.H * nqb2)), 256, 0, st>>>(
        a, reinterpret_cast<const uint16_t*>(q), thr, mscale, nqb2);
  return hipGetLastError();
}

}  // namespace sgsa
