// K1: causal score GEMM + exact token top-k on gfx950.
//
// Replaces the dense score matmul and the per-row torch.topk loop of the
// retriever (modelings/modeling_sgsa.py:420-428, :144-165) and of the hybrid
// KV-reuse attention (modelings/hybrid_dense_delta_topk.py:343-349), without
// ever materialising the [T,T] score matrix.
//
// Work unit: one (batch, head) and a block of 64 query rows; wave w owns rows
// [16w, 16w+16) so all per-row state (histograms, counters) is wave-private.
// Score tiles of 64 keys are recomputed with MFMA in every pass (K tile staged
// in LDS, q fragments held in registers), fp32 accumulation, then
// score = acc * (1/scale) (retriever, reciprocal rounded once on the host) or
// acc * scale (hybrid).
//
// Selection is an exact radix select over order-preserving uint32 keys of the
// fp32 scores (-0.0 folded onto +0.0): up to four 8-bit digit passes build a
// per-row 256-bin histogram of the still-tied candidates, each pass fixing one
// digit of the k-th key; a row leaves early once its threshold bin holds
// exactly the number still needed.  A final pass emits, in ascending key
// index order, every candidate above the threshold prefix plus the first
// `need` candidates equal to it (ordered ballot ranks), so ties are broken by
// lowest index.  Output rows are therefore in ascending index order; the
// optional sort kernel reorders them to (score desc, index asc).
#include "common.h"
#include "kernels.h"

#include <float.h>

#include <type_traits>

namespace sgsa {

namespace {

constexpr int QB = 64;        // query rows per block
constexpr int KT = 64;        // keys per tile
constexpr int DP = 128;       // padded head dim
constexpr int NBIN = 256;

template <typename X> struct KTile;
template <> struct KTile<bf16_t> {
  static constexpr int PITCH = DP + 8;   // ushorts; 272 B rows keep 16 B alignment
  typedef uint16_t T;
};
template <> struct KTile<float> {
  static constexpr int PITCH = DP + 4;
  typedef float T;
};

// Stage a 64-key x DP tile of K (rows j0.., zero beyond Tk / D) into LDS.
template <typename X>
__device__ __forceinline__ void load_k_tile(typename KTile<X>::T* ks, const X* __restrict__ k, int b, int h,
                                            int j0, int Tk, int H, int D) {
  constexpr int P = KTile<X>::PITCH;
  for (int e = threadIdx.x; e < KT * DP; e += blockDim.x) {
    const int r = e / DP, d = e % DP, j = j0 + r;
    typename KTile<X>::T x = 0;
    if (j < Tk && d < D) {
      const long off = ((long)(b * Tk + j) * H + h) * D + d;
      if constexpr (sizeof(X) == 2) x = reinterpret_cast<const uint16_t*>(k)[off];
      else x = reinterpret_cast<const float*>(k)[off];
    }
    ks[r * P + d] = x;
  }
}

struct RowInfo {
  uint32_t pfx, msk;
  int need, done;
};

}  // namespace

template <typename X, bool DUMP, bool C16>
__global__ __launch_bounds__(256) void score_topk_kernel(TopkArgs a, int nqb, float mscale) {
  constexpr int P = KTile<X>::PITCH;
  constexpr bool BF = sizeof(X) == 2;
  constexpr int NQF = BF ? DP / 32 : DP / 4;          // q fragments per lane
  constexpr int EPV = 16 / (int)sizeof(X);             // elements per 16 B vector
  constexpr int VPR = DP / EPV;                        // vectors per K row
  constexpr int NPF = KT * VPR / 256;                  // prefetch vectors per thread
  constexpr int HW = DUMP ? 1 : (C16 ? NBIN / 2 : NBIN);   // histogram words per row
  __shared__ __align__(16) typename KTile<X>::T ks[KT * P];
  __shared__ uint32_t hist[4][16][HW];
  __shared__ RowInfo rinfo[4][16];

  const int BH = a.B * a.H;
  const int bid = blockIdx.x;
  const int bh = bid % BH;   // with B*H a multiple of 8, a head always lands on the same XCD
  int qb = nqb - 1 - bid / BH;   // heaviest (latest) query blocks first
  if (DUMP) qb = (a.dump_row0 / QB) + bid / BH;
  const int b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int r0 = qb * QB;
  const int Tq = a.Tq, Tk = a.Tk, H = a.H, D = a.D;
  const X* kbase = reinterpret_cast<const X*>(a.k);

  // q fragments (A operand rows r0+16w+lr)
  typedef typename std::conditional<BF, bf16x8, float>::type QF;
  QF qf[NQF];
  {
    const int qr = r0 + 16 * w + lr;
    const X* qp = reinterpret_cast<const X*>(a.q) + ((long)(b * Tq + (qr < Tq ? qr : 0)) * H + h) * D;
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
      if constexpr (BF) {
        u16x8 raw;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int d = 32 * s + 8 * lg + j;
          raw[j] = (qr < Tq && d < D) ? reinterpret_cast<const uint16_t*>(qp)[d] : (uint16_t)0;
        }
        qf[s] = __builtin_bit_cast(bf16x8, raw);
      } else {
        const int d = 4 * s + lg;
        qf[s] = (qr < Tq && d < D) ? reinterpret_cast<const float*>(qp)[d] : 0.f;
      }
    }
  }

  // rows this lane holds in the accumulator: 4*lg + e
  int nvalid[4];
  bool live[4];
  int minvalid = 0x7fffffff;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int qr = r0 + 16 * w + 4 * lg + e;
    live[e] = qr < Tq;
    int nv = Tk;
    if (a.causal) nv = min(Tk, qr + a.q_offset + 1);
    if (nv < 0) nv = 0;
    nvalid[e] = live[e] ? nv : 0;
    if (live[e]) minvalid = min(minvalid, nvalid[e]);
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) minvalid = min(minvalid, __shfl_xor(minvalid, o, 64));
  int kend = Tk;
  if (a.causal && !DUMP) {
    const int last = min(Tq, r0 + QB) - 1 + a.q_offset;
    kend = min(Tk, last + 1);
  }
  const int ntile = DUMP ? (Tk + KT - 1) / KT : (kend + KT - 1) / KT;
  const bool vec = (D == DP);

  uint4 pf[NPF];
  auto issue = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NPF; ++i) {
      const int e = tid + 256 * i, r = e / VPR, cv = e % VPR, j = kt * KT + r;
      pf[i] = make_uint4(0, 0, 0, 0);
      if (j < Tk) pf[i] = *reinterpret_cast<const uint4*>(kbase + ((long)(b * Tk + j) * H + h) * DP + cv * EPV);
    }
  };
  auto commit = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NPF; ++i) {
      const int e = tid + 256 * i, r = e / VPR, cv = e % VPR;
      *reinterpret_cast<uint4*>(ks + r * P + cv * EPV) = pf[i];
    }
  };
  // Runs fn(kt, acc) for every key tile with the score tile in acc; K tiles are
  // prefetched one tile ahead into registers.
  auto sweep = [&](auto&& fn) __attribute__((always_inline)) {
    if (vec) issue(0);
    for (int kt = 0; kt < ntile; ++kt) {
      __syncthreads();
      if (vec) commit();
      else load_k_tile<X>(ks, kbase, b, h, kt * KT, Tk, H, D);
      __syncthreads();
      if (vec && kt + 1 < ntile) issue(kt + 1);
      f4 acc[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        f4 c = f4_zero();
#pragma unroll
        for (int s = 0; s < NQF; ++s) {
          if constexpr (BF) {
            const uint4 raw = *reinterpret_cast<const uint4*>(&ks[(16 * nt + lr) * P + 32 * s + 8 * lg]);
            c = mma_bf16(qf[s], __builtin_bit_cast(bf16x8, raw), c);
          } else {
            c = mma_f32(qf[s], ks[(16 * nt + lr) * P + 4 * s + lg], c);
          }
        }
        acc[nt] = c * mscale + 0.0f;   // fold -0.0 onto +0.0
      }
      fn(kt, acc);
    }
  };

  if constexpr (DUMP) {
    sweep([&](int kt, f4* acc) __attribute__((always_inline)) {
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int j = kt * KT + 16 * nt + lr;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int qr = r0 + 16 * w + 4 * lg + e;
          if (!live[e] || j >= Tk || qr < a.dump_row0 || qr >= a.dump_row0 + a.dump_rows) continue;
          a.dump[((long)bh * a.dump_rows + (qr - a.dump_row0)) * Tk + j] = j < nvalid[e] ? acc[nt][e] : -FLT_MAX;
        }
      }
    });
    return;
  }

  // ---- radix select -------------------------------------------------------
  const int topk = a.top_k;
  if (lane < 16) {
    const int qr = r0 + 16 * w + lane;
    int nv = 0;
    if (qr < Tq) nv = a.causal ? max(0, min(Tk, qr + a.q_offset + 1)) : Tk;
    RowInfo ri;
    ri.pfx = 0; ri.msk = 0; ri.need = min(topk, nv);
    ri.done = (nv <= topk) ? 1 : 0;
    rinfo[w][lane] = ri;
  }
  for (int i = lane; i < 16 * HW; i += 64) (&hist[w][0][0])[i] = 0;
  __syncthreads();

  uint32_t pfx[4], msk[4];
  int need[4], done[4];
  auto reload = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const RowInfo ri = rinfo[w][4 * lg + e];
      pfx[e] = ri.pfx; msk[e] = ri.msk; need[e] = ri.need; done[e] = ri.done;
    }
  };
  reload();

  for (int sh = 24; sh >= 0; sh -= 8) {
    int mine = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) mine |= !done[e];
    const bool wave_busy = __ballot(mine) != 0;
    if (!__syncthreads_or(mine)) break;
    sweep([&](int kt, f4* acc) __attribute__((always_inline)) {
      if (!wave_busy) return;
      const bool full = (kt + 1) * KT <= minvalid;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int j = kt * KT + 16 * nt + lr;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t key = f32_order_key(acc[nt][e]);
          const bool ok = !done[e] && (full || j < nvalid[e]) && (key & msk[e]) == pfx[e];
          if (ok) {
            const uint32_t bin = (key >> sh) & 255u;
            if constexpr (C16) atomicAdd(&hist[w][4 * lg + e][bin >> 1], 1u << ((bin & 1u) << 4));
            else atomicAdd(&hist[w][4 * lg + e][bin], 1u);
          }
        }
      }
    });
    __syncthreads();
    // resolve one digit per unfinished row of this wave
    for (int rr = 0; rr < 16; ++rr) {
      RowInfo ri = rinfo[w][rr];
      if (ri.done) continue;
      // lane l covers bins 255-4l .. 252-4l (descending)
      uint32_t c[4];
      if constexpr (C16) {
        const uint32_t w0 = hist[w][rr][127 - 2 * lane], w1 = hist[w][rr][126 - 2 * lane];
        c[0] = w0 >> 16; c[1] = w0 & 0xffffu; c[2] = w1 >> 16; c[3] = w1 & 0xffffu;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) c[q] = hist[w][rr][255 - 4 * lane - q];
      }
      const uint32_t loc = c[0] + c[1] + c[2] + c[3];
      uint32_t inc = loc;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t n = __shfl_up(inc, o, 64);
        if (lane >= o) inc += n;
      }
      const uint32_t exc = inc - loc;
      const bool hit = exc < (uint32_t)ri.need && (uint32_t)ri.need <= inc;
      const uint64_t bal = __ballot(hit);
      const int src = __ffsll((unsigned long long)bal) - 1;
      int bin = 0;
      uint32_t above = 0, cnt = 0;
      if (hit) {
        uint32_t cum = exc;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (cnt == 0 && cum + c[q] >= (uint32_t)ri.need) {
            bin = 255 - 4 * lane - q;
            above = cum;
            cnt = c[q];
          }
          if (cnt == 0) cum += c[q];
        }
      }
      bin = __shfl(bin, src, 64);
      above = __shfl(above, src, 64);
      cnt = __shfl(cnt, src, 64);
      if (lane == 0) {
        ri.pfx |= (uint32_t)bin << sh;
        ri.msk |= 0xffu << sh;
        ri.need -= (int)above;
        ri.done = (cnt == (uint32_t)ri.need || sh == 0) ? 1 : 0;
        rinfo[w][rr] = ri;
      }
      if constexpr (C16) {
        hist[w][rr][127 - 2 * lane] = 0;
        hist[w][rr][126 - 2 * lane] = 0;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) hist[w][rr][255 - 4 * lane - q] = 0;
      }
    }
    __syncthreads();
    reload();
  }

  // ---- emit pass ------------------------------------------------------------
  int outc[4], eqc[4];
  float m1[4], m2[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) { outc[e] = 0; eqc[e] = 0; m1[e] = -FLT_MAX; m2[e] = -FLT_MAX; }
  const uint32_t lower = (1u << lr) - 1u;
  long rowbase[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) rowbase[e] = ((long)bh * Tq + (r0 + 16 * w + 4 * lg + e)) * topk;
  sweep([&](int kt, f4* acc) __attribute__((always_inline)) {
    const bool full = (kt + 1) * KT <= minvalid;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int j = kt * KT + 16 * nt + lr;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok = full || j < nvalid[e];
        const float s = acc[nt][e];
        const uint32_t key = f32_order_key(s);
        const uint32_t km = key & msk[e];
        const bool eq = ok && km == pfx[e];
        const uint32_t eqb = (uint32_t)(__ballot(eq) >> (16 * lg)) & 0xffffu;
        const bool sel = ok && (km > pfx[e] || (eq && eqc[e] + __popc(eqb & lower) < need[e]));
        const uint32_t sb = (uint32_t)(__ballot(sel) >> (16 * lg)) & 0xffffu;
        const int slot = outc[e] + __popc(sb & lower);
        if (sel && slot < topk) {
          a.indices[rowbase[e] + slot] = j;
          a.scores[rowbase[e] + slot] = s;
        }
        const float so = ok ? s : -FLT_MAX;   // running top-2 with multiplicity
        m2[e] = fmaxf(m2[e], fminf(m1[e], so));
        m1[e] = fmaxf(m1[e], so);
        outc[e] += __popc(sb);
        eqc[e] += __popc(eqb);
      }
    }
  });
  // merge top-2 over the 16 lanes holding each row, then pad and write counts
#pragma unroll
  for (int e = 0; e < 4; ++e) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const float b1 = __shfl_xor(m1[e], o, 64), b2 = __shfl_xor(m2[e], o, 64);
      const float hi = fmaxf(m1[e], b1), lo = fmaxf(fminf(m1[e], b1), fmaxf(m2[e], b2));
      m1[e] = hi; m2[e] = lo;
    }
    if (!live[e]) continue;
    const long row = rowbase[e] / topk;
    for (int p = outc[e] + lr; p < topk; p += 16) {
      a.indices[rowbase[e] + p] = 0;
      a.scores[rowbase[e] + p] = -FLT_MAX;
    }
    if (lr == 0) {
      if (a.counts) a.counts[row] = outc[e];
      if (a.top2) { a.top2[2 * row] = m1[e]; a.top2[2 * row + 1] = m2[e]; }
    }
  }
}

// ---------------------------------------------------------------------------
// Row sort: (score desc, index asc) over the first counts[row] slots.  One
// block of 256 threads per row; bitonic sort of 64-bit composite keys in LDS.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void sort_rows_kernel(int32_t* __restrict__ indices, float* __restrict__ scores,
                                                        int top_k, const int32_t* __restrict__ counts, int npow2) {
  extern __shared__ unsigned long long sk[];
  const long row = blockIdx.x;
  const int n = counts ? counts[row] : top_k;
  int32_t* ip = indices + row * top_k;
  float* sp = scores + row * top_k;
  for (int i = threadIdx.x; i < npow2; i += blockDim.x) {
    unsigned long long key = 0ull;   // padding sorts last
    if (i < n) {
      const uint32_t ok = f32_order_key(sp[i]);
      key = ((unsigned long long)ok << 32) | (uint32_t)(0xffffffffu - (uint32_t)ip[i]);
    }
    sk[i] = key;
  }
  __syncthreads();
  for (int size = 2; size <= npow2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < npow2; i += blockDim.x) {
        const int jx = i ^ stride;
        if (jx > i) {
          const bool desc = (i & size) == 0;
          const unsigned long long x = sk[i], y = sk[jx];
          if ((x < y) == desc) { sk[i] = y; sk[jx] = x; }
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const unsigned long long key = sk[i];
    const uint32_t ok = (uint32_t)(key >> 32);
    const uint32_t u = (ok & 0x80000000u) ? (ok & 0x7fffffffu) : ~ok;
    ip[i] = (int32_t)(0xffffffffu - (uint32_t)(key & 0xffffffffu));
    sp[i] = __uint_as_float(u);
  }
}

hipError_t launch_score_topk(const TopkArgs& a, hipStream_t st) {
  const int nqb = (a.Tq + QB - 1) / QB;
  const int BH = a.B * a.H;
  // score = acc / scale is evaluated as acc * (1/scale) with the reciprocal
  // rounded once on the host; scale_mode 1 multiplies by scale directly.
  const float ms = a.scale_mode == 0 ? (float)(1.0 / (double)a.scale) : a.scale;
  if (a.dump) {
    const int qb0 = a.dump_row0 / QB;
    const int qb1 = (a.dump_row0 + a.dump_rows + QB - 1) / QB;
    const dim3 grid((unsigned)(BH * (qb1 - qb0)));
    if (a.dtype == DT_F32) score_topk_kernel<float, true, true><<<grid, 256, 0, st>>>(a, nqb, ms);
    else score_topk_kernel<bf16_t, true, true><<<grid, 256, 0, st>>>(a, nqb, ms);
    return hipGetLastError();
  }
  const dim3 grid((unsigned)(BH * nqb));
  const bool c16 = a.Tk <= 65535;   // 16-bit histogram counters cannot overflow
  if (a.dtype == DT_F32) {
    if (c16) score_topk_kernel<float, false, true><<<grid, 256, 0, st>>>(a, nqb, ms);
    else score_topk_kernel<float, false, false><<<grid, 256, 0, st>>>(a, nqb, ms);
  } else {
    if (c16) score_topk_kernel<bf16_t, false, true><<<grid, 256, 0, st>>>(a, nqb, ms);
    else score_topk_kernel<bf16_t, false, false><<<grid, 256, 0, st>>>(a, nqb, ms);
  }
  return hipGetLastError();
}

hipError_t launch_sort_rows(int32_t* indices, float* scores, long rows, int top_k, const int32_t* counts,
                            hipStream_t st) {
  int np = 1;
  while (np < top_k) np <<= 1;
  sort_rows_kernel<<<dim3((unsigned)rows), 256, sizeof(unsigned long long) * np, st>>>(indices, scores, top_k,
                                                                                     counts, np);
  return hipGetLastError();
}

}  // namespace sgsa
