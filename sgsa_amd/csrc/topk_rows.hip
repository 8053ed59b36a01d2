// Few-row form of K1 (decode: one query row per (b, h) over a long KV cache).
// The row kernel sweeps a row block's keys inside one workgroup, so a call
// with B*H*Tq ~ 128 rows occupies only 128 workgroups.  Here the keys of a row
// are spread over many workgroups:
//
//   rows_score_kernel   grid (key chunks of 512, rows): each wave loads its 128
//                       keys first, then scores them 16 at a time on
//                       v_mfma_f32_16x16x32_bf16 with the row
//                       kernel's operand roles (A = query, B = keys, d at
//                       k-position 32s + 8lg + j, steps s in order) and its
//                       score_of(), so the scores are bit-identical to the row
//                       kernel's; written to a [rows, Tk] fp32 buffer;
//   rows_select_kernel  one workgroup per row: the row's valid scores as
//                       order keys in LDS (<= 32768), an exact radix select
//                       (4 rounds of 8 bits) for the kq-th largest key, then
//                       the selected keys emitted in ascending key index, ties
//                       at the cut to the lowest indices.
//
// Output contract as the row kernel (sgsa_score_topk): counts = kq = min(top_k,
// valid keys); slots >= kq hold index 0 and -FLT_MAX; top2 the two largest
// valid scores; the unsorted order is one ascending run (split = kq).
#include <float.h>

#include "common.h"
#include "kernels.h"

namespace sgsa {

constexpr int TR_THREADS = 1024;
constexpr int TR_KG = 8;   // 16-key groups per wave of rows_score_kernel (all loads issued first)

// NKS = D / 32 as a template argument keeps the k-steps' loads and MFMAs free of branches.
template <int NKS>
__global__ __launch_bounds__(256) void rows_score_kernel(TopkArgs a, float mscale, float* __restrict__ sbuf) {
  const long row = blockIdx.y;
  const int Tq = a.Tq, Tk = a.Tk, H = a.H, D = NKS * 32;
  const int qr = (int)(row % Tq);
  const long bh = row / Tq;
  const int b = (int)(bh / H), h = (int)(bh % H);
  const int nv = a.causal ? min(Tk, qr + a.q_offset + 1) : Tk;
  const int lane = threadIdx.x & 63, lg = lane >> 4, lc = lane & 15;
  const int k0 = blockIdx.x * (64 * TR_KG) + 16 * TR_KG * (threadIdx.x >> 6);
  if (k0 >= nv) return;
  const uint16_t* qp = reinterpret_cast<const uint16_t*>(a.q) + ((long)(b * Tq + qr) * H + h) * D;
  const uint16_t* kb = reinterpret_cast<const uint16_t*>(a.k) + ((long)b * Tk * H + h) * D;
  const long kstride = (long)H * D;
  bf16x8 qf[NKS];
#pragma unroll
  for (int s = 0; s < NKS; ++s) qf[s] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8*>(qp + 32 * s + 8 * lg));
  u16x8 kr[TR_KG][NKS];
#pragma unroll
  for (int g = 0; g < TR_KG; ++g) {
    const int key = min(k0 + 16 * g + lc, nv - 1);
#pragma unroll
    for (int s = 0; s < NKS; ++s) kr[g][s] = *reinterpret_cast<const u16x8*>(kb + key * kstride + 32 * s + 8 * lg);
  }
  float* out = sbuf + row * (long)Tk;
#pragma unroll
  for (int g = 0; g < TR_KG; ++g) {
    f4 c = f4_zero();
#pragma unroll
    for (int s = 0; s < NKS; ++s) c = mma_bf16(qf[s], __builtin_bit_cast(bf16x8, kr[g][s]), c);
    const float sv = score_of(c, mscale)[0];
    const int key = k0 + 16 * g + lc;
    if (lg == 0 && key < nv) out[key] = sv;
  }
}

// Exclusive scan of x over the 512 threads; *total receives the block sum.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t x, uint32_t* wsum, uint32_t* total) {
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t inc = wave_incl_scan(x);
  if (lane == 63) wsum[wv] = inc;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < TR_THREADS / 64; ++w) {
    const uint32_t v = wsum[w];
    before += w < wv ? v : 0u;
    all += v;
  }
  __syncthreads();
  *total = all;
  return before + inc - x;
}

__global__ __launch_bounds__(TR_THREADS) void rows_select_kernel(TopkArgs a, const float* __restrict__ sbuf) {
  __shared__ uint32_t key[TR_MAXK];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t wsum[TR_THREADS / 64];
  __shared__ uint32_t pick[2];
  __shared__ float tops[TR_THREADS / 64][2];
  const long row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int Tq = a.Tq, Tk = a.Tk, top_k = a.top_k;
  const int qr = (int)(row % Tq);
  const int nv = a.causal ? min(Tk, qr + a.q_offset + 1) : Tk;
  const int kq = min(top_k, nv);
  const float* sr = sbuf + row * (long)Tk;

  float t1 = -FLT_MAX, t2 = -FLT_MAX;
  // eight scores per thread loaded before they are used (one load at a time leaves the pass latency-bound)
  for (int j0 = 0; j0 < nv; j0 += 8 * TR_THREADS) {
    float sv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = j0 + u * TR_THREADS + tid;
      sv[u] = j < nv ? sr[j] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = j0 + u * TR_THREADS + tid;
      if (j < nv) {
        const float s = sv[u];
        key[j] = f32_order_key(s);
        t2 = fmaxf(t2, fminf(t1, s));
        t1 = fmaxf(t1, s);
      }
    }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float b1 = __shfl_xor(t1, o, 64), b2 = __shfl_xor(t2, o, 64);
    const float hi = fmaxf(t1, b1), lo = fmaxf(fminf(t1, b1), fmaxf(t2, b2));
    t1 = hi; t2 = lo;
  }
  if (lane == 0) { tops[wv][0] = t1; tops[wv][1] = t2; }
  __syncthreads();

  // radix select of the kq-th largest order key
  const bool all = kq >= nv;
  uint32_t prefix = 0, pmask = 0;
  uint32_t need = (uint32_t)kq;   // keys still to take among those matching the prefix
  if (!all) {
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int i = tid; i < 256; i += TR_THREADS) hist[i] = 0;
      __syncthreads();
      for (int j = tid; j < nv; j += TR_THREADS) {
        const uint32_t kv = key[j];
        if ((kv & pmask) == prefix) atomicAdd(&hist[(kv >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (wv == 0) {
        uint32_t c[4], tot = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) { c[e] = hist[255 - 4 * lane - e]; tot += c[e]; }
        uint32_t above = wave_incl_scan(tot) - tot;   // keys in higher bins than this lane's
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (above < need && above + c[e] >= need) { pick[0] = 255u - 4u * lane - e; pick[1] = above; }
          above += c[e];
        }
      }
      __syncthreads();
      prefix |= pick[0] << shift;
      pmask |= 255u << shift;
      need -= pick[1];
      __syncthreads();
    }
  }
  const uint32_t thr = prefix;

  int32_t* oi = a.indices + row * top_k;
  float* os = a.scores + row * top_k;
  // emission in ascending key index: thread t owns keys [t CH, t CH + CH) (CH odd, so the
  // strided LDS reads hit distinct banks; CH <= 65 since nv <= 32768), marks them in
  // 64-bit masks, and two block scans give the ties' ranks and the output positions
  const int CH = ((nv + TR_THREADS - 1) / TR_THREADS) | 1;
  const int c0 = tid * CH;
  uint64_t gtm = 0, eqm = 0, hi_gt = 0, hi_eq = 0;   // bits of keys c0 + i (i < 64), then i = 64
  for (int i = 0; i < CH; ++i) {
    const int j = c0 + i;
    if (j < nv) {
      const uint32_t kv = key[j];
      const bool g = all || kv > thr, e = !all && kv == thr;
      if (i < 64) {
        gtm |= (uint64_t)g << i;
        eqm |= (uint64_t)e << i;
      } else {
        hi_gt = g;
        hi_eq = e;
      }
    }
  }
  uint32_t ntot;
  const uint32_t neq = (uint32_t)(__popcll(eqm) + hi_eq);
  const uint32_t eqbase = block_excl_scan(neq, wsum, &ntot);
  // ties at the cut go to the lowest indices: this chunk takes the first `take` of its equal keys
  uint32_t take = eqbase < need ? min(neq, need - eqbase) : 0u;
  uint64_t selm = gtm, hi_sel = hi_gt;
  for (uint64_t m = eqm; take > 0 && m != 0; --take) {
    const uint64_t lowbit = m & (~m + 1);
    selm |= lowbit;
    m ^= lowbit;
  }
  if (take > 0 && hi_eq) hi_sel = 1;
  const uint32_t nsel = (uint32_t)(__popcll(selm) + hi_sel);
  uint32_t pos = block_excl_scan(nsel, wsum, &ntot);
  for (uint64_t m = selm; m != 0; m &= m - 1) {
    const int i = __ffsll((long long)m) - 1;
    oi[pos] = c0 + i;
    os[pos] = key_to_f32(key[c0 + i]);
    ++pos;
  }
  if (hi_sel) {
    oi[pos] = c0 + 64;
    os[pos] = key_to_f32(key[c0 + 64]);
  }
  for (int i = kq + tid; i < top_k; i += TR_THREADS) {
    oi[i] = 0;
    os[i] = -FLT_MAX;
  }
  if (tid == 0) {
    if (a.counts) a.counts[row] = kq;
    if (a.split) a.split[row] = kq;
    if (a.top2) {
      float u1 = -FLT_MAX, u2 = -FLT_MAX;
      for (int w = 0; w < TR_THREADS / 64; ++w) {
        const float b1 = tops[w][0], b2 = tops[w][1];
        const float hi = fmaxf(u1, b1), lo = fmaxf(fminf(u1, b1), fmaxf(u2, b2));
        u1 = hi; u2 = lo;
      }
      a.top2[2 * row] = u1;
      a.top2[2 * row + 1] = u2;
    }
  }
}

size_t topk_rows_bytes(const TopkArgs& a) {
  const long rows = (long)a.B * a.H * a.Tq;
  auto aligned = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  if (a.dtype != DT_BF16 || a.D % 32 != 0 || a.D > DP_ROWS || a.Tq > TR_MAX_TQ || rows > TR_MAX_ROWS ||
      a.Tk > TR_MAXK || a.q == nullptr || a.k == nullptr || !aligned(a.q) || !aligned(a.k))
    return 0;
  return ((size_t)rows * a.Tk * sizeof(float) + 255) & ~(size_t)255;
}

hipError_t launch_score_topk_rows(const TopkArgs& a, float* sbuf, hipStream_t st) {
  const float ms = score_multiplier(a.scale, a.scale_mode);
  const long rows = (long)a.B * a.H * a.Tq;
  const dim3 grid((unsigned)((a.Tk + 64 * TR_KG - 1) / (64 * TR_KG)), (unsigned)rows);
  switch (a.D / 32) {   // D is a multiple of 32, at most DP_ROWS (topk_rows_bytes)
    case 1: rows_score_kernel<1><<<grid, 256, 0, st>>>(a, ms, sbuf); break;
    case 2: rows_score_kernel<2><<<grid, 256, 0, st>>>(a, ms, sbuf); break;
    case 3: rows_score_kernel<3><<<grid, 256, 0, st>>>(a, ms, sbuf); break;
    case 4: rows_score_kernel<4><<<grid, 256, 0, st>>>(a, ms, sbuf); break;
    default: return hipErrorInvalidValue;
  }
  rows_select_kernel<<<dim3((unsigned)rows), TR_THREADS, 0, st>>>(a, sbuf);
  return hipGetLastError();
}

}  // namespace sgsa
