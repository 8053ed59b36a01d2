// Block retrieval modes of the retriever on its torch path
// (modelings/modeling_sgsa.py:167-195 block selection, :302-359 candidates,
// :444-463 dispatch).  Three kernels, then the row gather of gather.hip:
//
//   block_max_kernel     block scores: per query row and key block of
//                        block_size keys, the max causal score (-FLT_MAX when
//                        the block has no causal key), [B,H,T,nb] fp32;
//   block_select_kernel  per row, the top `top_blocks` blocks (score desc,
//                        lowest index on ties) and the row's candidate count;
//   block_cand_kernel    per row, the causal keys of the kept blocks with
//                        their scores: block_token sorts them in LDS and emits
//                        the masked top-k slots; block_only emits them all.
//
// Scores here are acc * (1/sqrt(D)) with acc an fp32 fma chain over d = 0..D-1
// in ascending order, in both the block sweep and the candidate scorer, so a
// candidate's score is bit-identical to the value its block max was taken on.
#include <float.h>

#include "common.h"
#include "kernels.h"

namespace sgsa {

__device__ __forceinline__ float block_score(float acc, float mscale) {
#pragma clang fp contract(off)
  return acc * mscale + 0.0f;
}

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---- block maxima ----------------------------------------------------------
// One workgroup per (64 query rows, b, h).  The q tile stays in LDS as fp32;
// keys come in tiles of 64 keys x 32 dims.  Thread (ty, tx) owns rows ty+16i
// and keys tx+16j (i, j < 4).  After a key tile, its 64x64 scores go to LDS and
// each (row, block) pair the tile touches is folded into the block score with
// a max.  The workgroup owns its rows, and the barrier between key tiles
// orders the read-modify-writes of a block that spans two tiles.
constexpr int BM_DC = 32;   // dims per key chunk

template <typename X>
__global__ __launch_bounds__(256) void block_max_kernel(BlockArgs a, float mscale) {
  __shared__ float qs[64 * (BLK_MAX_D + 1)];
  __shared__ float ks[64 * (BM_DC + 1)];
  __shared__ float ss[64 * 65];
  const int D = a.D, DP = D + 1, T = a.T, H = a.H, bs = a.bs, nb = a.nb;
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  const int r0 = blockIdx.x * 64;
  const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
  const X* Q = reinterpret_cast<const X*>(a.q);
  const X* K = reinterpret_cast<const X*>(a.k);

  for (int e = tid; e < 64 * D; e += 256) {
    const int r = e / D, d = e % D, t = r0 + r;
    qs[r * DP + d] = t < T ? ld(Q, ((long)(b * T + t) * H + h) * D + d) : 0.f;
  }
  float* bsc = a.block_scores + (long)bh * T * nb;
  for (long e = tid; e < 64L * nb; e += 256) {
    const int t = r0 + (int)(e / nb);
    if (t < T) bsc[(long)t * nb + e % nb] = -FLT_MAX;
  }

  const int kend = a.causal ? min(T, r0 + 64) : T;
  for (int k0 = 0; k0 < kend; k0 += 64) {
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
    for (int d0 = 0; d0 < D; d0 += BM_DC) {
      const int dc = min(BM_DC, D - d0);
      __syncthreads();
      for (int e = tid; e < 64 * dc; e += 256) {
        const int r = e / dc, d = e % dc, key = k0 + r;
        ks[r * (BM_DC + 1) + d] = key < T ? ld(K, ((long)(b * T + key) * H + h) * D + d0 + d) : 0.f;
      }
      __syncthreads();
      for (int d = 0; d < dc; ++d) {
        float qa[4], kb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) qa[i] = qs[(ty + 16 * i) * DP + d0 + d];
#pragma unroll
        for (int j = 0; j < 4; ++j) kb[j] = ks[(tx + 16 * j) * (BM_DC + 1) + d];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(qa[i], kb[j], acc[i][j]);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = ty + 16 * i, c = tx + 16 * j, t = r0 + r, key = k0 + c;
        const bool ok = t < T && key < T && (!a.causal || key <= t);
        ss[r * 65 + c] = ok ? block_score(acc[i][j], mscale) : -FLT_MAX;
      }
    __syncthreads();
    const int kt_end = min(k0 + 64, T);
    const int bA = k0 / bs, nbt = (kt_end - 1) / bs - bA + 1;
    for (int it = tid; it < 64 * nbt; it += 256) {
      const int r = it / nbt, bb = bA + it % nbt, t = r0 + r;
      if (t >= T) continue;
      const int lo = max(bb * bs, k0), hi = min(bb * bs + bs, kt_end);
      float m = -FLT_MAX;
      for (int key = lo; key < hi; ++key) m = fmaxf(m, ss[r * 65 + key - k0]);
      float* p = bsc + (long)t * nb + bb;
      *p = fmaxf(*p, m);
    }
  }
}

// ---- top blocks per row ----------------------------------------------------
// One wave per row.  Blocks 0..lim/bs hold a key <= lim (lim = t causal, else
// T-1); they are the valid blocks of :188-189, the same count for every (b, h)
// of a row, so the masked top-k keeps kqb = min(eb, that count) of them
// (:159-160) and pads the rest with index 0 (:151-152).  Each round takes the
// best block after the previous one in (score desc, index asc) order.
__global__ __launch_bounds__(256) void block_select_kernel(BlockArgs a) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const long nrows = (long)a.B * a.H * a.T;
  if (row >= nrows) return;
  const int lane = threadIdx.x & 63;
  const int t = (int)(row % a.T), bs = a.bs, eb = a.eb;
  const int lim = a.causal ? t : a.T - 1;
  const int nvb = lim / bs + 1;
  const int kqb = min(eb, nvb);
  const float* bsc = a.block_scores + row * a.nb;
  int32_t* bi = a.block_indices + row * eb;
  float ls = INFINITY;
  int lj = -1, ncand = 0, first = 0, second = 0;
  for (int s = 0; s < kqb; ++s) {
    float bv = -INFINITY;
    int bj = 0x7fffffff;
    for (int j = lane; j < nvb; j += 64) {
      const float v = bsc[j];
      const bool after = v < ls || (v == ls && j > lj);
      if (after && v > bv) { bv = v; bj = j; }   // j ascends per lane: ties keep the lower index
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oj = __shfl_xor(bj, o, 64);
      if (ov > bv || (ov == bv && oj < bj)) { bv = ov; bj = oj; }
    }
    if (bj == 0x7fffffff) bj = 0;   // only NaN scores left: keep block 0 so every key stays in range
    ls = bv;
    lj = bj;
    if (lane == 0) bi[s] = bj;
    ncand += min(bj * bs + bs, lim + 1) - bj * bs;
    if (s == 0) first = bj;
    if (s == 1) second = bj;
  }
  for (int s = kqb + lane; s < eb; s += 64) bi[s] = 0;
  if (lane == 0) {
    a.ncand[row] = ncand;
    if (a.bmargin) a.bmargin[row] = eb >= 2 ? (float)first - (float)second : 0.f;
  }
}

// q . k over d = 0..D-1 as one fp32 fma chain (16-byte loads when VEC).
template <typename X, bool VEC> struct KeyDot;
template <bool VEC> struct KeyDot<float, VEC> {
  __device__ __forceinline__ static float run(const float* qrow, const float* kp, int D) {
    float acc = 0.f;
    if (VEC) {
      for (int d0 = 0; d0 < D; d0 += 4) {
        const float4 v = *reinterpret_cast<const float4*>(kp + d0);
        acc = fmaf(qrow[d0], v.x, acc);
        acc = fmaf(qrow[d0 + 1], v.y, acc);
        acc = fmaf(qrow[d0 + 2], v.z, acc);
        acc = fmaf(qrow[d0 + 3], v.w, acc);
      }
    } else {
      for (int d = 0; d < D; ++d) acc = fmaf(qrow[d], kp[d], acc);
    }
    return acc;
  }
};
template <bool VEC> struct KeyDot<bf16_t, VEC> {
  __device__ __forceinline__ static float run(const float* qrow, const bf16_t* kp, int D) {
    float acc = 0.f;
    if (VEC) {
      for (int d0 = 0; d0 < D; d0 += 8) {
        const uint4 v = *reinterpret_cast<const uint4*>(kp + d0);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc = fmaf(qrow[d0 + 2 * e], __uint_as_float(w[e] << 16), acc);
          acc = fmaf(qrow[d0 + 2 * e + 1], __uint_as_float(w[e] & 0xffff0000u), acc);
        }
      }
    } else {
      for (int d = 0; d < D; ++d) acc = fmaf(qrow[d], bf16_to_f32(kp[d].bits), acc);
    }
    return acc;
  }
};

// ---- candidates of the kept blocks -----------------------------------------
// One wave (workgroup) per row.  Candidate c maps to a kept slot by binary
// search over the slots' prefix counts; its key is scored by the lane.
// block_token (:322-344): sort keys (~order(score) << 32 | key) ascending in
// LDS (bitonic), i.e. score desc, key asc; the row keeps kq = min(kk, max over
// (b, h) of the position's candidate count) slots (:159-160); slots past the
// row's own candidates but below kq take the lowest-index keys outside the
// candidate set with score -FLT_MAX and are invalid (what the masked top-k over
// -FLT_MAX ties returns under the lowest-index rule); slots >= kq hold index 0.
// block_only (:346-359): every candidate becomes a slot, in generation order.
template <typename X, bool VEC, bool TOKEN>
__global__ __launch_bounds__(64) void block_cand_kernel(BlockArgs a, float mscale) {
  __shared__ float qrow[BLK_MAX_D];
  __shared__ int pre[BLK_MAXC + 1];
  __shared__ uint64_t keys[TOKEN ? BLK_MAXC : 1];
  const long row = blockIdx.x;
  const int lane = threadIdx.x;
  const int T = a.T, H = a.H, D = a.D, bs = a.bs, eb = a.eb;
  const int t = (int)(row % T);
  const long bh = row / T;
  const int b = (int)(bh / H), h = (int)(bh % H);
  const int lim = a.causal ? t : T - 1;
  const int nvb = lim / bs + 1;
  const int kqb = min(eb, nvb);
  const int32_t* bi = a.block_indices + row * eb;
  const X* Q = reinterpret_cast<const X*>(a.q);
  const X* K = reinterpret_cast<const X*>(a.k);

  for (int d = lane; d < D; d += 64) qrow[d] = ld(Q, ((long)(b * T + t) * H + h) * D + d);
  int run = 0;
  for (int s0 = 0; s0 < kqb; s0 += 64) {
    const int s = s0 + lane;
    int c = 0;
    if (s < kqb) {
      const int bj = bi[s];
      c = min(bj * bs + bs, lim + 1) - bj * bs;
    }
    const int inc = (int)wave_incl_scan((uint32_t)c);
    if (s < kqb) pre[s] = run + inc - c;
    run += __shfl(inc, 63, 64);
  }
  const int ncand = run;
  wave_sync_lds();

  float m1 = -FLT_MAX;
  for (int c = lane; c < ncand; c += 64) {
    int lo = 0, hi = kqb - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (pre[mid] <= c) lo = mid;
      else hi = mid - 1;
    }
    const int key = bi[lo] * bs + (c - pre[lo]);
    const float s = block_score(KeyDot<X, VEC>::run(qrow, K + ((long)(b * T + key) * H + h) * D, D), mscale);
    if (TOKEN) {
      keys[c] = ((uint64_t)(~f32_order_key(s)) << 32) | (uint32_t)key;
    } else {
      a.slot_idx[row * a.ks + c] = key;
      a.slot_sc[row * a.ks + c] = s;
      m1 = fmaxf(m1, s);
    }
  }

  if (!TOKEN) {
    m1 = wave_max(m1);
    if (lane == 0) {
      a.counts[row] = ncand;
      a.top2[2 * row] = m1;
      a.top2[2 * row + 1] = -FLT_MAX;
    }
    return;
  }

  int npad = 1;
  while (npad < ncand) npad <<= 1;
  for (int c = ncand + lane; c < npad; c += 64) keys[c] = ~0ull;
  wave_sync_lds();
  for (int span = 2; span <= npad; span <<= 1) {
    for (int j = span >> 1; j > 0; j >>= 1) {
      for (int i = lane; i < npad; i += 64) {
        const int p = i ^ j;
        if (p > i) {
          const uint64_t x = keys[i], y = keys[p];
          if ((x > y) == ((i & span) == 0)) {
            keys[i] = y;
            keys[p] = x;
          }
        }
      }
      wave_sync_lds();
    }
  }

  int mc = 1;
  for (int e = lane; e < a.B * a.H; e += 64) mc = max(mc, a.ncand[(long)e * T + t]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mc = max(mc, __shfl_xor(mc, o, 64));
  const int kk = a.kk, kq = min(kk, mc), nv = min(ncand, kq);
  int32_t* oi = a.slot_idx + row * kk;
  float* os = a.slot_sc + row * kk;
  uint8_t* ov = a.slot_valid + row * kk;
  for (int i = lane; i < kk; i += 64) {
    if (i < nv) {
      const uint64_t x = keys[i];
      oi[i] = (int)(uint32_t)x;
      os[i] = key_to_f32(~(uint32_t)(x >> 32));
      ov[i] = 1;
    } else if (i >= kq) {
      oi[i] = 0;
      os[i] = -FLT_MAX;
      ov[i] = 0;
    }
  }
  if (nv < kq) {
    const int need = kq - nv;
    const bool all_kept = kqb == nvb;
    int found = 0;
    for (int j0 = 0; found < need && j0 < T; j0 += 64) {
      const int j = j0 + lane;
      bool member = false;
      if (j < T && j <= lim) {
        if (all_kept) {
          member = true;
        } else {
          const int bj = j / bs;
          for (int s = 0; s < kqb; ++s) member |= bi[s] == bj;
        }
      }
      const bool outside = j < T && !member;
      const uint64_t m = ballot64(outside);
      const int r = found + (int)lane_rank(m);
      if (outside && r < need) {
        oi[nv + r] = j;
        os[nv + r] = -FLT_MAX;
        ov[nv + r] = 0;
      }
      found += popc64(m);
    }
  }
  if (lane == 0) {
    a.counts[row] = kq;
    a.top2[2 * row] = nv >= 1 ? key_to_f32(~(uint32_t)(keys[0] >> 32)) : -FLT_MAX;
    a.top2[2 * row + 1] = nv >= 2 ? key_to_f32(~(uint32_t)(keys[1] >> 32)) : -FLT_MAX;
  }
}

// block_only weights as the reference returns them, dense [B,H,T,T]: zero the
// row, then place each slot's weight at its key (keys of a row are distinct).
__global__ __launch_bounds__(256) void block_dense_weights_kernel(int T, int ks, const int32_t* __restrict__ idx,
                                                                  const float* __restrict__ w,
                                                                  const int32_t* __restrict__ counts,
                                                                  float* __restrict__ dense) {
  const long row = blockIdx.x;
  float* out = dense + row * T;
  for (int j = threadIdx.x; j < T; j += 256) out[j] = 0.f;
  __syncthreads();
  const int n = counts[row];
  for (int s = threadIdx.x; s < n; s += 256) out[idx[row * ks + s]] = w[row * ks + s];
}

template <typename X>
static void launch_cand(const BlockArgs& a, float ms, bool vec, hipStream_t st) {
  const dim3 grid((unsigned)((long)a.B * a.H * a.T));
  if (a.mode == 1) {
    if (vec) block_cand_kernel<X, true, true><<<grid, 64, 0, st>>>(a, ms);
    else block_cand_kernel<X, false, true><<<grid, 64, 0, st>>>(a, ms);
  } else {
    if (vec) block_cand_kernel<X, true, false><<<grid, 64, 0, st>>>(a, ms);
    else block_cand_kernel<X, false, false><<<grid, 64, 0, st>>>(a, ms);
  }
}

hipError_t launch_block_select(const BlockArgs& a, hipStream_t st) {
  const float ms = score_multiplier((float)sqrt((double)a.D), 0);
  const dim3 g1((unsigned)((a.T + 63) / 64), (unsigned)(a.B * a.H));
  if (a.dtype == DT_F32) block_max_kernel<float><<<g1, 256, 0, st>>>(a, ms);
  else block_max_kernel<bf16_t><<<g1, 256, 0, st>>>(a, ms);
  const long rows = (long)a.B * a.H * a.T;
  block_select_kernel<<<dim3((unsigned)((rows + 3) / 4)), 256, 0, st>>>(a);
  const int epv = a.dtype == DT_F32 ? 4 : 8;
  const bool vec = a.D % epv == 0 && ((uintptr_t)a.k & 15u) == 0;
  if (a.dtype == DT_F32) launch_cand<float>(a, ms, vec, st);
  else launch_cand<bf16_t>(a, ms, vec, st);
  return hipGetLastError();
}

hipError_t launch_block_dense_weights(int B, int H, int T, int ks, const int32_t* idx, const float* w,
                                      const int32_t* counts, float* dense, hipStream_t st) {
  block_dense_weights_kernel<<<dim3((unsigned)((long)B * H * T)), 256, 0, st>>>(T, ks, idx, w, counts, dense);
  return hipGetLastError();
}

}  // namespace sgsa
