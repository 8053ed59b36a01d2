// K2: sparse top-k gather with softmax weights, retrieval diagnostics and
// the SGSA write gate, fused into one pass per query row.
//
// Replaces, per query row:
//   weights = softmax(fp32 scores) * valid / max(sum, eps)
//                                        modelings/modeling_sgsa.py:126-128
//   k_hat, v_hat = sum_i w_i K[idx_i], sum_i w_i V[idx_i]        :130-134
//   margin, concentration, max_confidence, novelty, write_conflict,
//   entropy, distance ratios                                     :361-405
//   write key (direct | residual) and alpha gate     :546-552, :497-504
//   V-only variant for the hybrid KV reuse  hybrid_dense_delta_topk.py:350-356
// without the reference's [B,H,T,k,D] expand+gather temporary.
//
// One wave per query row.  The row's slot list (int32 index + fp32 score,
// ascending key index from K1) is read 64 slots at a time, one slot per lane;
// weights are exp(s - m) with m the row maximum, taken from K1 or kept as a
// running maximum with an online-softmax rescale of the partial sums.  The wave is
// then split into groups of LPR lanes, each lane owning 16 B of a key row, and
// walks the 64 slots with every group fetching a different K and V row, so a
// wave keeps 2 x 16 rows of 16 B loads in flight per unrolled step.
#include "common.h"
#include "kernels.h"
#include "recurrent_body.h"

#include <float.h>

namespace sgsa {

namespace {

template <typename X, bool VEC> struct GatherShape {
  static constexpr int NE = VEC ? 16 / (int)sizeof(X) : 2;   // elements per lane
};

template <typename X, bool VEC>
__device__ __forceinline__ void load_row(const X* __restrict__ base, long rowoff, int sub, int D, int lpr,
                                         float (&x)[GatherShape<X, VEC>::NE]) {
  constexpr int NE = GatherShape<X, VEC>::NE;
  if constexpr (VEC) {
    const int d0 = sub * NE;
    if (d0 < D) {
      const uint4 raw = *reinterpret_cast<const uint4*>(base + rowoff + d0);
      if constexpr (sizeof(X) == 2) {
        const uint32_t u[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[2 * i] = __uint_as_float(u[i] << 16);
          x[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
        }
      } else {
        x[0] = __uint_as_float(raw.x); x[1] = __uint_as_float(raw.y);
        x[2] = __uint_as_float(raw.z); x[3] = __uint_as_float(raw.w);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NE; ++i) x[i] = 0.f;
    }
  } else {
#pragma unroll
    for (int m = 0; m < NE; ++m) {
      const int d = sub + lpr * m;
      x[m] = d < D ? ld(base, rowoff + d) : 0.f;
    }
  }
}

// The elements of one 16-byte piece of a row, as load_row<X, true> reads them.
template <typename X>
__device__ __forceinline__ void unpack_row(const uint4 raw, float (&x)[16 / (int)sizeof(X)]) {
  if constexpr (sizeof(X) == 2) {
    const uint32_t u[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(u[i] << 16);
      x[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    }
  } else {
    x[0] = __uint_as_float(raw.x); x[1] = __uint_as_float(raw.y);
    x[2] = __uint_as_float(raw.z); x[3] = __uint_as_float(raw.w);
  }
}

template <typename X, bool VEC>
__device__ __forceinline__ int elem_d(int sub, int m, int lpr) {
  return VEC ? sub * GatherShape<X, VEC>::NE + m : sub + lpr * m;
}

}  // namespace

// Element offset of key / value row j of (b, h): [B,Tk,H,D] or, with kv_hm, [B,H,Tk,D].
__device__ __forceinline__ long kv_row_offset(const GatherArgs& a, int b, int h, int j) {
  return a.kv_hm ? (((long)b * a.H + h) * a.Tk + j) * a.D : (((long)b * a.Tk + j) * a.H + h) * a.D;
}

// Adds slots [base, base + nstep) of a row (their key indices in lane j, weights
// in wgt, lane order) into ak / av: the lane group grp takes slots it, it + 1, ..
// of each step of rpi = 64 / lpr.
template <typename X, bool VEC>
__device__ __forceinline__ void gather_step(const GatherArgs& a, int j, float wgt, int nstep, const X* K, const X* V,
                                            int b, int h, int grp, int sub, int lpr,
                                            float (&ak)[GatherShape<X, VEC>::NE],
                                            float (&av)[GatherShape<X, VEC>::NE]) {
  constexpr int NE = GatherShape<X, VEC>::NE;
  const int D = a.D;
  const int rpi = 64 / lpr;
  if constexpr (VEC) {
    // U slots per lane group at a time: every load issued before any is used
    // (no branch around them, so the compiler keeps them all in flight).
    // Slots past the step read slot 0's row (index 0 past kq) with weight 0;
    // lanes past D read dims from 0 and weigh them 0.
    constexpr int U = 4;
    const int d0 = sub * NE < D ? sub * NE : 0;
    const float lw = sub * NE < D ? 1.f : 0.f;
    for (int it0 = 0; it0 * rpi < nstep; it0 += U) {
      uint4 rk[U], rv[U];
      float wv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int src = (it0 + u) * rpi + grp;
        const int jj = __shfl(j, src & 63, 64);
        const float ww = __shfl(wgt, src & 63, 64);
        wv[u] = src < nstep ? ww * lw : 0.f;
        const long off = kv_row_offset(a, b, h, src < nstep ? jj : 0) + d0;
        rv[u] = *reinterpret_cast<const uint4*>(V + off);
        if (K) rk[u] = *reinterpret_cast<const uint4*>(K + off);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float xv[NE];
        unpack_row<X>(rv[u], xv);
#pragma unroll
        for (int i = 0; i < NE; ++i) av[i] += wv[u] * xv[i];
        if (K) {
          float xk[NE];
          unpack_row<X>(rk[u], xk);
#pragma unroll
          for (int i = 0; i < NE; ++i) ak[i] += wv[u] * xk[i];
        }
      }
    }
  } else {
#pragma unroll 4
    for (int it = 0; it * rpi < nstep; ++it) {
      const int src = it * rpi + grp;
      const int jj = __shfl(j, src, 64);
      const float ww = __shfl(wgt, src, 64);
      if (src < nstep && ww != 0.f) {
        const long off = kv_row_offset(a, b, h, jj);
        float xv[NE];
        load_row<X, VEC>(V, off, sub, D, lpr, xv);
        if (K) {
          float xk[NE];
          load_row<X, VEC>(K, off, sub, D, lpr, xk);
#pragma unroll
          for (int i = 0; i < NE; ++i) ak[i] += ww * xk[i];
        }
#pragma unroll
        for (int i = 0; i < NE; ++i) av[i] += ww * xv[i];
      }
    }
  }
}

// Accumulates slots [s0, s1) of one row into (ak, av, esum) with weights
// exp(score - mrun).  Online mode (no top2) raises mrun as larger scores
// arrive, rescaling what was accumulated, and keeps the running top-2.
template <typename X, bool VEC>
__device__ __forceinline__ void gather_slots(const GatherArgs& a, int s0, int s1, const int32_t* idxp,
                                             const float* scp, const uint8_t* vp, const X* K, const X* V, int b,
                                             int h, int grp, int sub, int lpr, bool fixed_max, float& mrun,
                                             float& t1, float& t2, float& esum,
                                             float (&ak)[GatherShape<X, VEC>::NE],
                                             float (&av)[GatherShape<X, VEC>::NE]) {
  constexpr int NE = GatherShape<X, VEC>::NE;
  const int lane = threadIdx.x & 63;
  for (int base = s0; base < s1; base += 64) {
    const int slot = base + lane;
    int j = 0;
    float sc = -INFINITY;
    if (slot < s1) {
      j = idxp[slot];
      const bool ok = vp ? (vp[slot] != 0) : true;
      if (ok) sc = scp[slot];
    }
    if (!fixed_max) {
      // online-softmax merge: rescale what was accumulated under the old max
      const float bm = wave_max(sc);
      if (bm > mrun) {
        const float f = (mrun == -INFINITY) ? 0.f : __expf(mrun - bm);
        esum *= f;
#pragma unroll
        for (int i = 0; i < NE; ++i) { ak[i] *= f; av[i] *= f; }
        mrun = bm;
      }
      const float so = sc == -INFINITY ? -FLT_MAX : sc;
      t2 = fmaxf(t2, fminf(t1, so));
      t1 = fmaxf(t1, so);
    }
    const float wgt = sc == -INFINITY ? 0.f : __expf(sc - mrun);
    esum += wgt;
    const int nstep = min(64, s1 - base);
    gather_step<X, VEC>(a, j, wgt, nstep, K, V, b, h, grp, sub, lpr, ak, av);
  }
}

// gather_slots for bf16 rows of D = 128 ([B,Tk,H,D], 16 lanes per row) whose slot scores
// are computed here, from the query's 8 elements of the lane (qv) and the key rows the
// gather loads anyway: each 64-slot block loads its 64 key and value rows (lane group g:
// slots 4u + g, u = 0..15) before using any, scores them as rescore_kernel does (the same
// fused multiply-adds, lane swaps and multiplier, 0 for an index outside [0, Tk)), hands
// slot l's score to lane l, and then weighs and sums as gather_slots and gather_step do,
// in the same order: the results equal rescore_kernel followed by gather_slots bit for
// bit, with one read of the key rows instead of two.
__device__ __forceinline__ void gather_slots_rescored(const GatherArgs& a, int s0, int s1, const int32_t* idxp,
                                                      const float (&qv)[8], float ms, const uint16_t* K,
                                                      const uint16_t* V, int b, int h, int grp, int sub,
                                                      bool fixed_max, float& mrun, float& t1, float& t2,
                                                      float& esum, float (&ak)[8], float (&av)[8]) {
  const int lane = threadIdx.x & 63;
  const int Tk = a.Tk;
  // the (b, h) rows from one base; a row's offset from it fits 32 bits (j H D + D < 2^31 elements)
  const long hb = kv_row_offset(a, b, h, 0);
  const uint16_t* Kb = K + hb;
  const uint16_t* Vb = V + hb;
  const uint32_t rstride = (uint32_t)a.H * 128u;
  for (int base = s0; base < s1; base += 64) {
    const int slot = base + lane;
    const int jl = slot < s1 ? idxp[slot] : 0;
    const int nstep = min(64, s1 - base);
    uint4 rk[16], rv[16];
    uint32_t okm = 0;   // bit u: slot 4u + grp is in the block and its index in [0, Tk)
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int src = 4 * u + grp;
      const int jj = __shfl(jl, src, 64);
      const bool ok = src < nstep && jj >= 0 && jj < Tk;
      okm |= ok ? 1u << u : 0u;
      const uint32_t off = (ok ? (uint32_t)jj : 0u) * rstride + 8u * (uint32_t)sub;
      rk[u] = *reinterpret_cast<const uint4*>(Kb + off);
      rv[u] = *reinterpret_cast<const uint4*>(Vb + off);
    }
    // the scores: all 16 lanes of group g hold slot 4u + g's in sco[u]; lane 16g + u then
    // offers sco[u], which lane 4u + g takes
    float mine = 0.f;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const uint32_t wv[4] = {rk[u].x, rk[u].y, rk[u].z, rk[u].w};
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc = fmaf(qv[2 * e], __uint_as_float(wv[e] << 16), acc);
        acc = fmaf(qv[2 * e + 1], __uint_as_float(wv[e] & 0xffff0000u), acc);
      }
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) acc += __shfl_xor(acc, o, 64);
      const float sco = (okm >> u) & 1u ? acc * ms : 0.f;
      mine = sub == u ? sco : mine;
    }
    // the key rows stay packed until the sums: the unpacked copies of the scoring loop are
    // not kept for them (128 more registers live), they are unpacked again
#pragma unroll
    for (int u = 0; u < 16; ++u) asm volatile("" : "+v"(rk[u].x), "+v"(rk[u].y), "+v"(rk[u].z), "+v"(rk[u].w));
    const float got = __shfl(mine, 16 * (lane & 3) + (lane >> 2), 64);
    const float sc = slot < s1 ? got : -INFINITY;
    if (!fixed_max) {
      const float bm = wave_max(sc);
      if (bm > mrun) {
        const float f = (mrun == -INFINITY) ? 0.f : __expf(mrun - bm);
        esum *= f;
#pragma unroll
        for (int i = 0; i < 8; ++i) { ak[i] *= f; av[i] *= f; }
        mrun = bm;
      }
      const float so = sc == -INFINITY ? -FLT_MAX : sc;
      t2 = fmaxf(t2, fminf(t1, so));
      t1 = fmaxf(t1, so);
    }
    const float wgt = sc == -INFINITY ? 0.f : __expf(sc - mrun);
    esum += wgt;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int src = 4 * u + grp;
      const float ww = __shfl(wgt, src, 64);
      const float wv = src < nstep ? ww : 0.f;
      float xv[8], xk[8];
      unpack_row<bf16_t>(rv[u], xv);
#pragma unroll
      for (int i = 0; i < 8; ++i) av[i] += wv * xv[i];
      unpack_row<bf16_t>(rk[u], xk);
#pragma unroll
      for (int i = 0; i < 8; ++i) ak[i] += wv * xk[i];
    }
  }
}

// One wave's row (over B*H*Tq) of the gather: its slots (or, SPLIT, its partials), then the
// epilogue.  Wave-local: no LDS and no block barrier.
// PA: the split partials are 16-byte aligned (the launcher checks a.part), so their row pieces
// load 16 bytes at a time.
template <typename X, bool VEC, bool SPLIT, bool PA = false>
__device__ __forceinline__ void gather_row(const GatherArgs& a, long row, int lpr) {
  constexpr int NE = GatherShape<X, VEC>::NE;
  const int lane = threadIdx.x & 63;
  const long nrows = (long)a.B * a.H * a.Tq;
  if (row >= nrows) return;
  const int Tq = a.Tq, H = a.H, D = a.D, topk = a.top_k;
  const int bh = (int)(row / Tq), qr = (int)(row % Tq);
  const int b = bh / H, h = bh % H;
  const int pos = qr + a.q_offset;
  const int grp = lane / lpr, sub = lane % lpr;

  const int kq = a.counts[row];
  const bool fixed_max = a.top2 != nullptr;
  float mrun = fixed_max ? a.top2[2 * row] : -INFINITY;   // running max of the row's valid scores
  float t1 = -FLT_MAX, t2 = -FLT_MAX;                      // running top-2 (online mode)
  const int32_t* idxp = a.indices + row * topk;
  const float* scp = a.scores + row * topk;
  const uint8_t* vp = a.slot_valid ? a.slot_valid + row * topk : nullptr;
  const X* K = reinterpret_cast<const X*>(a.k);
  const X* V = reinterpret_cast<const X*>(a.v);

  float ak[NE], av[NE];
#pragma unroll
  for (int i = 0; i < NE; ++i) { ak[i] = 0.f; av[i] = 0.f; }
  float esum = 0.f;
  // the epilogue's own inputs, loaded first (they do not depend on the slots)
  const long qoff = ((long)(b * Tq + qr) * H + h) * D;
  float kt[NE];
  if (a.self_key != nullptr && (a.diag != nullptr || a.budget != nullptr)) {
    load_row<X, VEC>(reinterpret_cast<const X*>(a.self_key), qoff, sub, D, lpr, kt);
  } else {
#pragma unroll
    for (int i = 0; i < NE; ++i) kt[i] = 0.f;
  }
  const float bud = a.budget != nullptr ? a.budget[(long)(b * Tq + qr) * H + h] : 0.f;

  if constexpr (!SPLIT) {
    for (int base = 0; base < kq; base += 64) {
      const int slot = base + lane;
      int j = 0;
      float sc = -INFINITY;
      if (slot < kq) {
        j = idxp[slot];
        const bool ok = vp ? (vp[slot] != 0) : true;
        if (ok) sc = scp[slot];
      }
      if (!fixed_max) {
        // online-softmax merge: rescale what was accumulated under the old max
        const float bm = wave_max(sc);
        if (bm > mrun) {
          const float f = (mrun == -INFINITY) ? 0.f : __expf(mrun - bm);
          esum *= f;
  #pragma unroll
          for (int i = 0; i < NE; ++i) { ak[i] *= f; av[i] *= f; }
          mrun = bm;
        }
        const float so = sc == -INFINITY ? -FLT_MAX : sc;
        t2 = fmaxf(t2, fminf(t1, so));
        t1 = fmaxf(t1, so);
      }
      const float wgt = sc == -INFINITY ? 0.f : __expf(sc - mrun);
      esum += wgt;
      const int nstep = min(64, kq - base);
      gather_step<X, VEC>(a, j, wgt, nstep, K, V, b, h, grp, sub, lpr, ak, av);
    }
  } else {
    // merge the row's partials (gather_part_kernel): lane c takes partials c, c + 64, .. for the
    // sums and top-2 pairs; lane group g adds partials g, g + 64 / lpr, .. to the row vectors
    // (the groups are summed below).  Every load after the maximum is independent of the others.
    const long pst = 4 + 2 * (long)D;
    const int ns = a.nsplit;
    const float* P = a.part + row * (long)ns * pst;
    constexpr int SPG = 4;
    const int ng = 64 / lpr;
    if (ns <= ng * SPG) {
      // every load first: lane c < ns the header of partial c; lane group g the row-vector
      // pieces of partials g, g + ng, .. (at most SPG); then the same sums in the same
      // order as the loops below
      // 16-byte loads where the partials allow them (PA; VEC: a lane's NE elements are
      // consecutive, D and the partial stride multiples of 4); the same values either way
      constexpr bool f4 = PA && VEC && NE % 4 == 0;
      float hm = -INFINITY, hs = 0.f, h1 = -FLT_MAX, h2 = -FLT_MAX;
      if (lane < ns) {
        const float* pc = P + lane * pst;
        if constexpr (f4) {
          const float4 hv = *reinterpret_cast<const float4*>(pc);
          hm = hv.x; hs = hv.y; h1 = hv.z; h2 = hv.w;
        } else {
          hm = pc[0]; hs = pc[1]; h1 = pc[2]; h2 = pc[3];
        }
      }
      float pk[SPG][NE], pvv[SPG][NE];
      if constexpr (f4) {
        const int d0 = elem_d<X, VEC>(sub, 0, lpr);   // the lane's NE elements d0 .. d0 + NE - 1
        const bool in = d0 < D;
#pragma unroll
        for (int u = 0; u < SPG; ++u) {
          const int c = min(grp + ng * u, ns - 1);
          const float* pc = P + c * pst + 4 + (in ? d0 : 0);
#pragma unroll
          for (int i4 = 0; i4 < NE / 4; ++i4) {
            const uint4 kv = *reinterpret_cast<const uint4*>(pc + 4 * i4);
            const uint4 vv = *reinterpret_cast<const uint4*>(pc + D + 4 * i4);
            pk[u][4 * i4] = __uint_as_float(kv.x); pk[u][4 * i4 + 1] = __uint_as_float(kv.y);
            pk[u][4 * i4 + 2] = __uint_as_float(kv.z); pk[u][4 * i4 + 3] = __uint_as_float(kv.w);
            pvv[u][4 * i4] = __uint_as_float(vv.x); pvv[u][4 * i4 + 1] = __uint_as_float(vv.y);
            pvv[u][4 * i4 + 2] = __uint_as_float(vv.z); pvv[u][4 * i4 + 3] = __uint_as_float(vv.w);
          }
        }
      } else {
#pragma unroll
        for (int u = 0; u < SPG; ++u) {
          const int c = min(grp + ng * u, ns - 1);
          const float* pc = P + c * pst;
#pragma unroll
          for (int i = 0; i < NE; ++i) {
            const int d = min(elem_d<X, VEC>(sub, i, lpr), D - 1);
            pk[u][i] = pc[4 + d];
            pvv[u][i] = pc[4 + D + d];
          }
        }
      }
      if (!fixed_max) mrun = wave_max(hm);
      if (lane < ns) {
        const float f = hm == -INFINITY ? 0.f : __expf(hm - mrun);
        esum += hs * f;
        const float hi = fmaxf(t1, h1), lo = fmaxf(fminf(t1, h1), fmaxf(t2, h2));
        t1 = hi;
        t2 = lo;
      }
#pragma unroll
      for (int u = 0; u < SPG; ++u) {
        const int c = grp + ng * u;
        const float pm = __shfl(hm, min(c, 63), 64);
        if (c < ns) {
          const float f = pm == -INFINITY ? 0.f : __expf(pm - mrun);
#pragma unroll
          for (int i = 0; i < NE; ++i) {
            if (elem_d<X, VEC>(sub, i, lpr) < D) {
              ak[i] += pk[u][i] * f;
              av[i] += pvv[u][i] * f;
            }
          }
        }
      }
    } else {
    if (!fixed_max) {
      float mc = -INFINITY;
      for (int c = lane; c < ns; c += 64) mc = fmaxf(mc, P[c * pst]);
      mrun = wave_max(mc);
    }
    for (int c = lane; c < ns; c += 64) {
      const float* pc = P + c * pst;
      const float f = pc[0] == -INFINITY ? 0.f : __expf(pc[0] - mrun);
      esum += pc[1] * f;
      const float u1 = pc[2], u2 = pc[3];
      const float hi = fmaxf(t1, u1), lo = fmaxf(fminf(t1, u1), fmaxf(t2, u2));
      t1 = hi;
      t2 = lo;
    }
    for (int c = grp; c < ns; c += 64 / lpr) {
      const float* pc = P + c * pst;
      const float f = pc[0] == -INFINITY ? 0.f : __expf(pc[0] - mrun);
#pragma unroll
      for (int i = 0; i < NE; ++i) {
        const int d = elem_d<X, VEC>(sub, i, lpr);
        if (d < D) {
          ak[i] += pc[4 + d] * f;
          av[i] += pc[4 + D + d] * f;
        }
      }
    }
    }
  }
  // combine the groups (lanes with equal `sub`)
  for (int o = lpr; o < 64; o <<= 1) {
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      ak[i] += __shfl_xor(ak[i], o, 64);
      av[i] += __shfl_xor(av[i], o, 64);
    }
  }
  float s0 = mrun, s1;
  if (fixed_max) {
    s1 = a.top2[2 * row + 1];
  } else {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float b1 = __shfl_xor(t1, o, 64), b2 = __shfl_xor(t2, o, 64);
      const float hi = fmaxf(t1, b1), lo = fmaxf(fminf(t1, b1), fmaxf(t2, b2));
      t1 = hi; t2 = lo;
    }
    s0 = kq > 0 ? t1 : -FLT_MAX;
    s1 = t2;
  }
  const float E = wave_sum(esum);
  const float inv = E > 0.f ? 1.f / E : 0.f;
#pragma unroll
  for (int i = 0; i < NE; ++i) { ak[i] *= inv; av[i] *= inv; }

  // ---- per-row scalars (group 0 lanes hold the row vectors) ----
  float pdot = 0.f, pkk = 0.f, phh = 0.f, pvv = 0.f;
  if (grp == 0) {
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      pdot += ak[i] * kt[i];
      pkk += kt[i] * kt[i];
      phh += ak[i] * ak[i];
      pvv += av[i] * av[i];
    }
  }
  const float dot = wave_sum(pdot), kk2 = wave_sum(pkk), hh2 = wave_sum(phh), vv2 = wave_sum(pvv);
  const float eps = a.eps;

  float margin = 0.f;
  if (a.margin_in) margin = a.margin_in[row];
  else if (topk >= 2) margin = s0 - s1;
  const float conc = 1.f / (1.f + expf(-(margin / fmaxf(a.tau_c, eps))));
  const float self_norm = fmaxf(sqrtf(kk2), eps);
  const float kh_norm = fmaxf(sqrtf(hh2), eps);
  const float proj = dot / (self_norm * self_norm + eps);
  float pperp = 0.f;
  if (grp == 0) {
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const float dlt = ak[i] - proj * kt[i];
      pperp += dlt * dlt;
    }
  }
  const float perp = sqrtf(wave_sum(pperp));
  const float novelty = fminf(fmaxf(perp / (kh_norm + eps), 0.f), 1.f);

  // ---- write gate ----
  float wk[NE];
#pragma unroll
  for (int i = 0; i < NE; ++i) wk[i] = ak[i];
  float alpha_v = 0.f, perp_ratio = 0.f;
  if (a.budget != nullptr) {
    float wnorm2 = hh2;
    if (a.write_mode == 1) {
      const float c = dot / fmaxf(kk2, eps);
      float pw = 0.f;
#pragma unroll
      for (int i = 0; i < NE; ++i) {
        wk[i] = ak[i] - c * kt[i];
        pw += grp == 0 ? wk[i] * wk[i] : 0.f;
      }
      wnorm2 = wave_sum(pw);
      perp_ratio = fminf(fmaxf(sqrtf(wnorm2) / kh_norm, 0.f), 10.f);
    }
    float al = a.alpha_max * conc * novelty * (1.f / (1.f + expf(-bud)));
    const float prox = al * sqrtf(vv2) * sqrtf(wnorm2);
    const float clip = fminf(1.f / fmaxf(prox, 1.f), 1.f);
    alpha_v = al * clip;
  }
  if (a.stats != nullptr && lane == 0) {
    a.stats[row] = kq > 0 ? inv : 0.f;   // the largest weight, exp(0) / E
    a.stats[nrows + row] = perp_ratio;
  }

  // ---- stores of the row vectors ----
  if (grp == 0) {
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int d = elem_d<X, VEC>(sub, i, lpr);
      if (d >= D) continue;
      if (a.k_hat) st(reinterpret_cast<X*>(a.k_hat), qoff + d, ak[i]);
      st(reinterpret_cast<X*>(a.v_hat), qoff + d, av[i]);
      if (a.write_key) st(reinterpret_cast<X*>(a.write_key), qoff + d, wk[i]);
    }
  }
  if (a.alpha && lane == 0) a.alpha[(long)(b * Tq + qr) * H + h] = alpha_v;

  // ---- second pass over the slot list: weights, entropy, distance stats ----
  if (a.diag != nullptr || a.weights != nullptr) {
    float ent = 0.f, dsum = 0.f, nloc = 0.f, nsink = 0.f, nrem = 0.f;
    int imax = 0;
    for (int base = 0; base < topk; base += 64) {
      const int slot = base + lane;
      if (slot >= topk) break;
      int j = 0;
      float wv = 0.f;
      if (slot < kq) {
        j = idxp[slot];
        const bool ok = vp ? (vp[slot] != 0) : true;
        wv = ok ? __expf(scp[slot] - mrun) * inv : 0.f;
      }
      if (a.weights) a.weights[row * topk + slot] = wv;
      const float wc = fmaxf(wv, eps);
      ent += wc * logf(wc);
      const int dist = max(pos - j, 0);
      dsum += (float)dist;
      nloc += dist <= a.local_window ? 1.f : 0.f;
      nsink += j < a.sink_size ? 1.f : 0.f;
      nrem += (dist > a.local_window && j >= a.sink_size) ? 1.f : 0.f;
      imax = max(imax, j);
    }
    if (a.diag != nullptr) {
      ent = wave_sum(ent) + a.ent_pad * (eps * logf(eps));
      dsum = wave_sum(dsum);
      nloc = wave_sum(nloc);
      nsink = wave_sum(nsink);
      nrem = wave_sum(nrem);
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) imax = max(imax, __shfl_xor(imax, o, 64));
      if (lane == 0) {
        const long plane = (long)a.B * a.H * a.Tq;
        const float inv_k = 1.f / (float)topk;
        float* dg = a.diag;
        dg[0 * plane + row] = margin;
        dg[1 * plane + row] = conc;
        dg[2 * plane + row] = kq > 0 ? inv : 0.f;
        dg[3 * plane + row] = novelty;
        dg[4 * plane + row] = fminf(fmaxf(dot / (self_norm * kh_norm + eps), -1.f), 1.f);
        dg[5 * plane + row] = -ent;
        dg[6 * plane + row] = dsum * inv_k;    // divided by (max index + 1) in finish_diag
        dg[7 * plane + row] = nloc * inv_k;
        dg[8 * plane + row] = nsink * inv_k;
        dg[9 * plane + row] = nrem * inv_k;
        atomicMax(a.max_index + (row & (GATHER_MAXIDX_SLOTS - 1)), imax);   // spread: one word takes 1/64 of the rows
      }
    }
  }
}

template <typename X, bool VEC, bool SPLIT, bool PA = false>
__global__ __launch_bounds__(256) void sparse_gather_kernel(GatherArgs a, int lpr) {
  gather_row<X, VEC, SPLIT, PA>(a, (long)blockIdx.x * 4 + (threadIdx.x >> 6), lpr);
}

// avg_distance /= max(max_index + 1, 1)  (modelings/modeling_sgsa.py:395, :401); the largest index is the
// max over the GATHER_MAXIDX_SLOTS words the rows spread their atomics over.
__global__ __launch_bounds__(256) void finish_diag_kernel(float* __restrict__ avgd, long n,
                                                          const int32_t* __restrict__ max_index) {
  __shared__ int mx;
  if (threadIdx.x < 64) {
    int m = max_index[threadIdx.x & (GATHER_MAXIDX_SLOTS - 1)];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = max(m, __shfl_xor(m, o, 64));
    if (threadIdx.x == 0) mx = m;
  }
  __syncthreads();
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) avgd[i] = avgd[i] / (float)max(mx + 1, 1);
}

__global__ void zero_int_kernel(int32_t* p) {
  if (threadIdx.x < GATHER_MAXIDX_SLOTS) p[threadIdx.x] = 0;
}

// Split-row form of the gather for rows with many slots and few rows (decode):
// wave (row, c) accumulates slots [c*split_len, (c+1)*split_len) of the row
// and writes its partial {max, sum, top-1, top-2, ak[D], av[D]}
// (unnormalised, relative to that max); sparse_gather_kernel merges a row's
// partials in a fixed order, then runs its epilogue unchanged.  RS: the slot scores are
// computed from a.rq and the gathered key rows (gather_slots_rescored; bf16, D = 128).
template <typename X, bool VEC, bool RS>
__global__ __launch_bounds__(256) void gather_part_kernel(GatherArgs a, int lpr) {
  constexpr int NE = GatherShape<X, VEC>::NE;
  const int lane = threadIdx.x & 63;
  const long wid = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const long nrows = (long)a.B * a.H * a.Tq;
  if (wid >= nrows * a.nsplit) return;
  const long row = wid / a.nsplit;
  const int c = (int)(wid % a.nsplit);
  const int Tq = a.Tq, H = a.H, D = a.D, topk = a.top_k;
  const int bh = (int)(row / Tq);
  const int b = bh / H, h = bh % H;
  const int grp = lane / lpr, sub = lane % lpr;
  const int kq = a.counts[row];
  const bool fixed_max = a.top2 != nullptr;
  float mrun = fixed_max ? a.top2[2 * row] : -INFINITY;
  float t1 = -FLT_MAX, t2 = -FLT_MAX;
  float ak[NE], av[NE];
#pragma unroll
  for (int i = 0; i < NE; ++i) { ak[i] = 0.f; av[i] = 0.f; }
  float esum = 0.f;
  const int s0 = c * a.split_len, s1 = min(kq, s0 + a.split_len);
  if constexpr (RS) {
    static_assert(VEC && sizeof(X) == 2 && NE == 8, "the rescored partials take bf16 rows of 16-byte pieces");
    const long qoff = ((long)(b * Tq + (int)(row % Tq)) * H + h) * D;
    float qv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[e] = ld(reinterpret_cast<const X*>(a.rq), qoff + 8 * sub + e);
    gather_slots_rescored(a, s0, s1, a.indices + row * topk, qv, a.rq_ms, reinterpret_cast<const uint16_t*>(a.k),
                          reinterpret_cast<const uint16_t*>(a.v), b, h, grp, sub, fixed_max, mrun, t1, t2, esum, ak,
                          av);
  } else {
    gather_slots<X, VEC>(a, s0, s1, a.indices + row * topk, a.scores + row * topk,
                         a.slot_valid ? a.slot_valid + row * topk : nullptr, reinterpret_cast<const X*>(a.k),
                         reinterpret_cast<const X*>(a.v), b, h, grp, sub, lpr, fixed_max, mrun, t1, t2, esum, ak,
                         av);
  }
  for (int o = lpr; o < 64; o <<= 1) {
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      ak[i] += __shfl_xor(ak[i], o, 64);
      av[i] += __shfl_xor(av[i], o, 64);
    }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float b1 = __shfl_xor(t1, o, 64), b2 = __shfl_xor(t2, o, 64);
    const float hi = fmaxf(t1, b1), lo = fmaxf(fminf(t1, b1), fmaxf(t2, b2));
    t1 = hi; t2 = lo;
  }
  const float E = wave_sum(esum);
  float* P = a.part + wid * (4 + 2 * D);
  if (lane == 0) {
    P[0] = mrun;
    P[1] = E;
    P[2] = t1;
    P[3] = t2;
  }
  if (grp == 0) {
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int d = elem_d<X, VEC>(sub, i, lpr);
      if (d < D) {
        P[4 + d] = ak[i];
        P[4 + D + d] = av[i];
      }
    }
  }
}

// Decode step (T = 1): wave 0 of each block merges its row's partials and writes the write
// key, v_hat and alpha (gather_row: the merge kernel's arithmetic; the CS column blocks of a
// row write the same values), then the block runs K6's update of its state columns on them
// (recurrent_body), as sparse_gather_kernel followed by recurrent_kernel compute them.
template <int CS, bool PA>
__global__ __launch_bounds__(256) void merge_recurrent_kernel(GatherArgs g, RecurrentArgs r) {
  if (threadIdx.x < 64) gather_row<bf16_t, true, true, PA>(g, (long)blockIdx.x, 16);
  __syncthreads();
  recurrent_body<bf16_t, true, CS>(r);
}

hipError_t launch_merge_recurrent(const GatherArgs& g, const RecurrentArgs& r, hipStream_t st) {
  if (g.dtype != DT_BF16 || g.D != 128 || g.Tq != 1 || g.nsplit <= 0 || r.T != 1 || r.dtype != DT_BF16 ||
      r.D != 128 || r.B != g.B || r.H != g.H || r.sparse_k == nullptr || g.diag != nullptr || g.weights != nullptr)
    return hipErrorInvalidValue;
  const bool pa = ((uintptr_t)g.part & 15u) == 0;
  const dim3 grid4((unsigned)(r.B * r.H), 4), grid1((unsigned)(r.B * r.H), 1);
  if (r.B * r.H < 256) {
    if (pa) merge_recurrent_kernel<4, true><<<grid4, 256, 0, st>>>(g, r);
    else merge_recurrent_kernel<4, false><<<grid4, 256, 0, st>>>(g, r);
  } else {
    if (pa) merge_recurrent_kernel<1, true><<<grid1, 256, 0, st>>>(g, r);
    else merge_recurrent_kernel<1, false><<<grid1, 256, 0, st>>>(g, r);
  }
  return hipGetLastError();
}

hipError_t launch_sparse_gather(const GatherArgs& a, hipStream_t st) {
  const long nrows = (long)a.B * a.H * a.Tq;
  const dim3 grid((unsigned)((nrows + 3) / 4));
  if (a.diag) zero_int_kernel<<<1, 64, 0, st>>>(a.max_index);
  const int epv = 16 / (a.dtype == DT_F32 ? 4 : 2);
  bool vec = (a.D % epv) == 0;
  auto aligned = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  vec = vec && aligned(a.v) && (a.k == nullptr || aligned(a.k)) && (a.self_key == nullptr || aligned(a.self_key));
  if (a.nsplit > 0) {
    const dim3 pgrid((unsigned)((nrows * a.nsplit + 3) / 4));
    if (a.rq != nullptr) {
      // the caller checked the form: bf16, D = 128, [B,Tk,H,D] keys, no slot mask, aligned rows
      if (a.dtype != DT_BF16 || a.D != 128 || a.kv_hm != 0 || a.slot_valid != nullptr || !vec || a.k == nullptr)
        return hipErrorInvalidValue;
      gather_part_kernel<bf16_t, true, true><<<pgrid, 256, 0, st>>>(a, 16);
    } else if (vec) {
      int lpr = 1;
      while (lpr * epv < a.D) lpr <<= 1;
      if (a.dtype == DT_F32) gather_part_kernel<float, true, false><<<pgrid, 256, 0, st>>>(a, lpr);
      else gather_part_kernel<bf16_t, true, false><<<pgrid, 256, 0, st>>>(a, lpr);
    } else {
      if (a.dtype == DT_F32) gather_part_kernel<float, false, false><<<pgrid, 256, 0, st>>>(a, 64);
      else gather_part_kernel<bf16_t, false, false><<<pgrid, 256, 0, st>>>(a, 64);
    }
  }
  const bool sp = a.nsplit > 0;
  if (sp && a.pieces_only) return hipGetLastError();
  if (vec) {
    int lpr = 1;
    while (lpr * epv < a.D) lpr <<= 1;
    const bool pa = sp && ((uintptr_t)a.part & 15u) == 0;
    if (a.dtype == DT_F32) {
      if (pa) sparse_gather_kernel<float, true, true, true><<<grid, 256, 0, st>>>(a, lpr);
      else if (sp) sparse_gather_kernel<float, true, true><<<grid, 256, 0, st>>>(a, lpr);
      else sparse_gather_kernel<float, true, false><<<grid, 256, 0, st>>>(a, lpr);
    } else {
      if (pa) sparse_gather_kernel<bf16_t, true, true, true><<<grid, 256, 0, st>>>(a, lpr);
      else if (sp) sparse_gather_kernel<bf16_t, true, true><<<grid, 256, 0, st>>>(a, lpr);
      else sparse_gather_kernel<bf16_t, true, false><<<grid, 256, 0, st>>>(a, lpr);
    }
  } else {
    if (a.dtype == DT_F32) {
      if (sp) sparse_gather_kernel<float, false, true><<<grid, 256, 0, st>>>(a, 64);
      else sparse_gather_kernel<float, false, false><<<grid, 256, 0, st>>>(a, 64);
    } else {
      if (sp) sparse_gather_kernel<bf16_t, false, true><<<grid, 256, 0, st>>>(a, 64);
      else sparse_gather_kernel<bf16_t, false, false><<<grid, 256, 0, st>>>(a, 64);
    }
  }
  if (a.diag) {
    const long plane = nrows;
    finish_diag_kernel<<<dim3((unsigned)((plane + 255) / 256)), 256, 0, st>>>(a.diag + 6 * plane, plane,
                                                                            a.max_index);
  }
  return hipGetLastError();
}

// Scores at given keys, for top-k reuse across decode steps: for every row r
// and slot i < counts[r], scores[r, i] = (q_r . k_{indices[r, i]}) * mscale in
// fp32.  A block takes 256 slots of one row (decode has few rows, so the slots
// are what fills the GPU); each 16-lane group of a wave takes one key per step,
// and with D <= 128 and D % 8 == 0 each lane reads 8 consecutive elements (16
// bytes of bf16) of the query and the key.  Partial dot products are summed over
// the group with lane swaps.  Indices outside [0, Tk) score 0.
constexpr int RS_SLOTS = 256;   // slots per block

template <typename X, bool VEC>
__global__ __launch_bounds__(256) void rescore_kernel(int B, int Tq, int Tk, int H, int D, int top_k,
                                                     const X* __restrict__ q, const X* __restrict__ k,
                                                     const int32_t* __restrict__ indices,
                                                     const int32_t* __restrict__ counts, float mscale,
                                                     float* __restrict__ scores) {
  const int nchunk = (top_k + RS_SLOTS - 1) / RS_SLOTS;
  const long row = blockIdx.x / nchunk;
  const int base = (blockIdx.x % nchunk) * RS_SLOTS + (threadIdx.x >> 6) * 64;   // the wave's 64 slots
  const int lane = threadIdx.x & 63, grp = lane >> 4, l16 = lane & 15;
  const int qr = (int)(row % Tq);
  const long bh = row / Tq;
  const int h = (int)(bh % H), b = (int)(bh / H);
  const int kq = min(counts[row], top_k);
  if (base >= kq) return;   // wave-uniform
  const long qoff = ((long)(b * Tq + qr) * H + h) * D;
  // element e of the lane: dim VEC ? 8 l16 + e : l16 + 16 e
  auto dim = [&](int e) { return VEC ? 8 * l16 + e : l16 + 16 * e; };
  float qv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) qv[e] = dim(e) < D ? ld(q, qoff + dim(e)) : 0.f;
  const int32_t* ip = indices + row * top_k;
  float* sp = scores + row * top_k;
  const int nend = min(kq, base + 64);
  if constexpr (VEC && sizeof(X) == 2) {
    if (D == 128) {
      // the wave's 64 indices in one load (lane l: slot base + l), then the 16-byte pieces of all
      // 64 keys (lane group g: keys base + 4u + g) loaded before the first is used: two memory
      // round trips per wave
      const int jl = base + lane < nend ? ip[base + lane] : -1;
      uint4 kv[16];
      bool ok[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int i = base + 4 * u + grp;
        const int j = __shfl(jl, 4 * u + grp, 64);
        ok[u] = i < nend && j >= 0 && j < Tk;
        const long koff = ((long)(b * Tk + (ok[u] ? j : 0)) * H + h) * 128 + 8 * l16;
        kv[u] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(k) + koff);
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const uint32_t wv[4] = {kv[u].x, kv[u].y, kv[u].z, kv[u].w};
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc = fmaf(qv[2 * e], __uint_as_float(wv[e] << 16), acc);
          acc = fmaf(qv[2 * e + 1], __uint_as_float(wv[e] & 0xffff0000u), acc);
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) acc += __shfl_xor(acc, o, 64);
        const int i = base + 4 * u + grp;
        if (i < nend && l16 == 0) sp[i] = ok[u] ? acc * mscale : 0.f;
      }
      return;
    }
  }
#pragma unroll 4
  for (int i0 = base; i0 < nend; i0 += 4) {
    const int i = i0 + grp;
    float acc = 0.f;
    if (i < nend) {
      const int j = ip[i];
      if (j >= 0 && j < Tk) {
        const long koff = ((long)(b * Tk + j) * H + h) * D;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (dim(e) < D) acc = fmaf(qv[e], ld(k, koff + dim(e)), acc);
      }
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) acc += __shfl_xor(acc, o, 64);
    if (i < nend && l16 == 0) sp[i] = acc * mscale;
  }
}

hipError_t launch_rescore(int dtype, int B, int Tq, int Tk, int H, int D, int top_k, const void* q, const void* k,
                          const int32_t* indices, const int32_t* counts, float mscale, float* scores,
                          hipStream_t st) {
  const long nrows = (long)B * H * Tq;
  const long nchunk = (top_k + RS_SLOTS - 1) / RS_SLOTS;
  const dim3 grid((unsigned)(nrows * nchunk));
  const bool vec = D % 8 == 0;   // 8 consecutive elements per lane cover D <= 128
#define SGSA_RESCORE(XT, V)                                                                          \
  rescore_kernel<XT, V><<<grid, 256, 0, st>>>(B, Tq, Tk, H, D, top_k, (const XT*)q, (const XT*)k, indices, \
                                              counts, mscale, scores)
  if (dtype == DT_F32) { if (vec) SGSA_RESCORE(float, true); else SGSA_RESCORE(float, false); }
  else { if (vec) SGSA_RESCORE(bf16_t, true); else SGSA_RESCORE(bf16_t, false); }
#undef SGSA_RESCORE
  return hipGetLastError();
}

}  // namespace sgsa
