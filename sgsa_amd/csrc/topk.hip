// K1: causal score GEMM + exact token top-k on gfx950.
//
// Replaces the dense score matmul and the per-row torch.topk loop of the
// retriever (modelings/modeling_sgsa.py:420-428, :144-165) and of the hybrid
// KV-reuse attention (modelings/hybrid_dense_delta_topk.py:343-349), without
// ever materialising the [T,T] score matrix.
//
// Work unit: one (batch, head) and a block of 64 query rows; wave w owns rows
// [16w, 16w+16), so every per-row counter and histogram is wave-private.  Score
// tiles of 64 keys are recomputed with MFMA in each pass (K tiles prefetched
// one ahead into registers, staged in LDS; q fragments stay in registers),
// fp32 accumulation, score = acc * (1/scale) with the reciprocal rounded once
// on the host (retriever) or acc * scale (hybrid).
//
// Exact selection in two sweeps for typical rows:
//   pass A  a 256-bin histogram per row of bin(s) = clamp(int(s*iw + 128), 0, 255),
//           iw = 128 / (|q_row| * max_j |k_j| * scale): a monotone map of the
//           score (any iw keeps the selection exact; the Cauchy-Schwarz bound
//           only makes the bins informative).  The threshold bin b*, the count
//           above it and the number `need` still to take from it follow.
//   pass B  emits every candidate with bin > b* in ascending key index and
//           appends the candidates of bin b* (in index order) to a per-row
//           scratch list of at most TOPK_CAP entries.
//   resolve an exact radix select over the order-preserving uint32 keys of the
//           collected scores (-0.0 folded onto +0.0) finds the need-th largest;
//           the winners -- keys above it, then equal keys in index order -- are
//           appended.  Ties are therefore broken by lowest index.
// Rows whose b* holds exactly `need` candidates skip the scratch.  A block
// with a row whose b* holds more than TOPK_CAP candidates (coarse bins, mass
// ties) is flagged and redone by a second launch of the kernel that selects
// with up to four 8-bit radix digit passes over the keys, then emits.  The output
// order of a row is deterministic (emitted part in index order, then the
// resolved part in index order); the sort kernel reorders rows to
// (score desc, index asc) when requested.
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
constexpr int KNCH = 32;      // partial key-norm maxima per (batch, head)

enum RowMode { SELECT_ALL = 0, BIN_ALL = 1, COLLECT = 2, RADIX = 3 };

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
  float iw;          // bin scale
  float bc;          // bin offset (score_bin_bits); set by score_thr128_kernel only
  int bstar;         // threshold bin
  int need;          // still to take at the current resolution
  int mode;          // RowMode
  uint32_t pfx, msk; // RADIX key prefix inside b*
  int done;          // RADIX resolution finished
  float th0, th1;    // pass B: select s >= th1; collect th0 <= s < th1
};

// bin(s) = round(s * iw + bc - 2^23) clamped to [0, 255], read from the mantissa
// of fma(s, iw, bc) (no float-to-int conversion); bc = 2^23 + 128 centres the
// bins on 0.  Monotone non-decreasing in s for iw > 0, which is all the exact
// select needs; NaN lands in bin 0.
constexpr float BIN_C0 = 8388736.0f;
__device__ __forceinline__ uint32_t score_bin_bits(float s, float iw, float bc = BIN_C0) {
  return __float_as_uint(__builtin_amdgcn_fmed3f(fmaf(s, iw, bc), 8388608.0f, 8388863.0f));
}
__device__ __forceinline__ int score_bin(float s, float iw, float bc = BIN_C0) {
  return (int)(score_bin_bits(s, iw, bc) & 255u);
}


// The float threshold t of a key bound: for finite scores s, s >= t <=> key(s) >= k.
// (Keys below key(-FLT_MAX) or above key(FLT_MAX) decode to -inf/+inf or NaN;
// no finite score has them.)
__device__ __forceinline__ float threshold_of_key(uint32_t k) {
  return key_to_f32(min(max(k, 0x00800000u), 0xff7fffffu));
}

// Smallest float s with score_bin(s, iw) >= bt (1 <= bt <= 255), by bisection over
// the order-preserving keys between -inf and +inf (score_bin is monotone in s).
__device__ __forceinline__ float bin_lower_edge(int bt, float iw, float bc = BIN_C0) {
  uint32_t lo = 0x007fffffu, hi = 0xff800000u;   // keys of -inf and +inf
  while (hi - lo > 1u) {
    const uint32_t mid = lo + ((hi - lo) >> 1);
    if (score_bin(key_to_f32(mid), iw, bc) >= bt) hi = mid;
    else lo = mid;
  }
  return key_to_f32(hi);
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Over 256 counts laid out as lane l <-> bins 255-4l .. 252-4l (descending),
// finds the bin holding the `need`-th largest element.  Wave-uniform results.
__device__ __forceinline__ void find_bin(const uint32_t (&c)[4], int lane, uint32_t need, int& bin, uint32_t& above,
                                         uint32_t& cnt) {
  const uint32_t loc = c[0] + c[1] + c[2] + c[3];
  const uint32_t inc = wave_incl_scan(loc);
  const uint32_t exc = inc - loc;
  const bool hit = exc < need && need <= inc;
  const uint64_t bal = ballot64(hit);
  const int src = bal ? (int)__builtin_ctzll(bal) : 0;   // wave-uniform
  int b = 0;
  uint32_t ab = 0, ct = 0;
  if (hit) {
    uint32_t cum = exc;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (ct == 0 && cum + c[q] >= need) {
        b = 255 - 4 * lane - q;
        ab = cum;
        ct = c[q];
      }
      if (ct == 0) cum += c[q];
    }
  }
  bin = __builtin_amdgcn_readlane(b, src);
  above = (uint32_t)__builtin_amdgcn_readlane((int)ab, src);
  cnt = (uint32_t)__builtin_amdgcn_readlane((int)ct, src);
}


// Inclusive prefix sum within each aligned group of 16 lanes (row_shr 1/2/4/8,
// lanes past the row edge read 0).
__device__ __forceinline__ uint32_t row16_incl_scan(uint32_t x) {
  int v = (int)x;
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);
  return (uint32_t)v;
}
// Sum over the aligned group of 16 lanes, in every lane of the group.
__device__ __forceinline__ uint32_t row16_sum(uint32_t x, int lane) {
  return (uint32_t)__shfl((int)row16_incl_scan(x), lane | 15, 64);
}

// find_bin for four independent histograms, one per group of 16 lanes: lane
// 16s + u holds bins 255-16u .. 240-16u (descending) of group s, and need is the
// group's.  Results are uniform within each group.
__device__ __forceinline__ void find_bin16(const uint32_t (&c)[16], int lane, uint32_t need, int& bin,
                                           uint32_t& above, uint32_t& cnt) {
  const int u = lane & 15;
  uint32_t loc = 0;
#pragma unroll
  for (int q = 0; q < 16; ++q) loc += c[q];
  const uint32_t inc = row16_incl_scan(loc);
  const uint32_t exc = inc - loc;
  const bool hit = exc < need && need <= inc;
  const uint32_t rowbits = (uint32_t)(ballot64(hit) >> (lane & 48)) & 0xffffu;
  const int src = (lane & 48) + (rowbits ? (int)__builtin_ctz(rowbits) : 0);
  int b = 0;
  uint32_t ab = 0, ct = 0;
  if (hit) {
    uint32_t cum = exc;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      if (ct == 0 && cum + c[q] >= need) {
        b = 255 - 16 * u - q;
        ab = cum;
        ct = c[q];
      }
      if (ct == 0) cum += c[q];
    }
  }
  bin = __shfl(b, src, 64);
  above = (uint32_t)__shfl((int)ab, src, 64);
  cnt = (uint32_t)__shfl((int)ct, src, 64);
}

}  // namespace

// Max |k_j| per (b,h): the denominator of the pass-A bin scale.  grid (B*H), 256 threads.
// Squared key-norm maxima of one (batch, head): block (bh, c) covers rows
// j = c (mod KNCH), 16 lanes per row; kmax2[bh * KNCH + c] = max_j |k_j|^2.
template <typename X>
__global__ __launch_bounds__(256) void key_norm_max_kernel(const X* __restrict__ k, int Tk, int H, int D,
                                                           float* __restrict__ kmax2) {
  __shared__ float red[4];
  const int bh = blockIdx.x / KNCH, c = blockIdx.x % KNCH, b = bh / H, h = bh % H;
  const int sub = threadIdx.x & 15, rw = threadIdx.x >> 4;
  constexpr int EPV = 16 / (int)sizeof(X);   // elements per 16-byte load
  float m = 0.f;
  const bool vec = D % EPV == 0 && ((uintptr_t)k & 15u) == 0;
  for (int j0 = c; j0 < Tk; j0 += KNCH * 16) {   // trip count uniform over the block
    const int j = j0 + KNCH * rw;
    float s = 0.f;
    if (j < Tk) {
      const X* row = k + ((long)(b * Tk + j) * H + h) * D;
      if (vec) {   // 16 lanes read a row in 16-byte pieces
        for (int d = EPV * sub; d < D; d += 16 * EPV) {
          const uint4 u = *reinterpret_cast<const uint4*>(row + d);
          if constexpr (sizeof(X) == 2) {
            const uint32_t wv[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float lo = __uint_as_float(wv[q] << 16), hi = __uint_as_float(wv[q] & 0xffff0000u);
              s = fmaf(lo, lo, s);
              s = fmaf(hi, hi, s);
            }
          } else {
            const float xs[4] = {__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w)};
#pragma unroll
            for (int q = 0; q < 4; ++q) s = fmaf(xs[q], xs[q], s);
          }
        }
      } else {
        for (int d = sub; d < D; d += 16) {
          const float x = ld(row, d);
          s = fmaf(x, x, s);
        }
      }
    }
    m = fmaxf(m, group_sum(s, 16));
  }
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) kmax2[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// FB = false: the two-pass select; a block with a row whose threshold bin holds
// more than TOPK_CAP candidates sets flags[block] and returns without output.
// FB = true: re-runs exactly the flagged blocks with 8-bit radix digit passes
// over the order-preserving keys (up to 4 passes + emit).
// THR (with FB and LIST): no tile lists; each row's cut goes to thr instead
// (the fallback of the threshold-mode tiles kernel).
template <typename X, bool DUMP, bool C16, bool TOP2, bool FB, bool LIST, bool THR = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(LIST && !FB ? 3 : 1))) void score_topk_kernel(TopkArgs a, int nqb, float mscale) {
  static_assert(!THR || (FB && LIST), "threshold output only from the list-mode fallback");
  constexpr bool TL = LIST && !THR;   // writes tile lists
  constexpr int P = KTile<X>::PITCH;
  constexpr bool BF = sizeof(X) == 2;
  constexpr int NQF = BF ? DP / 32 : DP / 4;          // q fragments per lane
  constexpr int EPV = 16 / (int)sizeof(X);             // elements per 16 B vector
  constexpr int VPR = DP / EPV;                        // vectors per K row
  constexpr int NPF = KT * VPR / 256;                  // prefetch vectors per thread
  constexpr int HW = DUMP ? 1 : (C16 ? NBIN / 2 : NBIN);   // histogram words per row
  constexpr int HWA = HW < 16 ? 16 : HW;               // >= 256 words per wave for the resolve
  constexpr int CAPL = TOPK_CAP / 64;                  // collected entries per lane in the resolve
  __shared__ __align__(16) typename KTile<X>::T ks[KT * P];
  __shared__ uint32_t hist[4][16][HWA];
  __shared__ RowInfo rinfo[4][16];
  __shared__ int rowcnt[4][16][2];   // emitted count, collected count
  __shared__ int run1[4][16];        // length of the leading ascending run
  __shared__ float qnorm[4][16];

  const int BH = a.B * a.H;
  const int bid = blockIdx.x;
  if constexpr (FB) {
    if (a.flags[bid] == 0) return;   // block-uniform: only the flagged blocks are redone
  }
  const int bh = bid % BH;   // with B*H a multiple of 8, a head always lands on the same XCD
  int qb = nqb - 1 - bid / BH;   // heaviest (latest) query blocks first
  if (DUMP) qb = (a.dump_row0 / QB) + bid / BH;
  const int b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const int lr = lane & 15, lg = lane >> 4;
  const int r0 = qb * QB;
  const int Tq = a.Tq, Tk = a.Tk, H = a.H, D = a.D;
  const X* kbase = reinterpret_cast<const X*>(a.k);

  // q fragments (A operand rows r0+16w+lr) and their norms
  typedef typename std::conditional<BF, bf16x8, float>::type QF;
  QF qf[NQF];
  {
    float qn2 = 0.f;
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
          const float x = bf16_to_f32(raw[j]);
          qn2 = fmaf(x, x, qn2);
        }
        qf[s] = __builtin_bit_cast(bf16x8, raw);
      } else {
        const int d = 4 * s + lg;
        qf[s] = (qr < Tq && d < D) ? reinterpret_cast<const float*>(qp)[d] : 0.f;
        qn2 = fmaf(qf[s], qf[s], qn2);
      }
    }
    qn2 += __shfl_xor(qn2, 16, 64);
    qn2 += __shfl_xor(qn2, 32, 64);
    if (!DUMP && lg == 0) qnorm[w][lr] = sqrtf(qn2);
  }

  // rows this lane holds in the accumulator: 4*lg + e
  // valid keys of query row qr (< Tq): a prefix of the keys
  const bool masked = !DUMP && (!LIST || THR) && a.row_nv != nullptr;   // not in tile-list mode
  auto row_valid = [&](int qr) __attribute__((always_inline)) {
    if (masked) return a.row_nv[(long)b * Tq + qr];
    return a.causal ? max(0, min(Tk, qr + a.q_offset + 1)) : Tk;
  };
  int nvalid[4];
  bool live[4];
  int minvalid = 0x7fffffff;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int qr = r0 + 16 * w + 4 * lg + e;
    live[e] = qr < Tq;
    nvalid[e] = live[e] ? row_valid(qr) : 0;
    if (live[e]) minvalid = min(minvalid, nvalid[e]);
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) minvalid = min(minvalid, __shfl_xor(minvalid, o, 64));
  int kend = Tk;
  if (masked) {   // the block's largest valid prefix (QB = 64 rows, one per lane)
    kend = r0 + lane < Tq ? row_valid(r0 + lane) : 0;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) kend = max(kend, __shfl_xor(kend, o, 64));
  } else if (a.causal && !DUMP) {
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
  // Runs fn(kt, acc) for every key tile with the score tile in acc.
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
        acc[nt] = score_of(c, mscale);
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

  const int topk = a.top_k;
  __syncthreads();   // qnorm visible
  float kmx2 = lane < KNCH ? a.kmax[(long)bh * KNCH + lane] : 0.f;
  const float kmx = sqrtf(wave_max(kmx2));
  if (lane < 16) {
    const int qr = r0 + 16 * w + lane;
    const int nv = qr < Tq ? row_valid(qr) : 0;
    const int kr = (masked && a.row_kq != nullptr && qr < Tq) ? min(topk, a.row_kq[qr]) : topk;   // row's slots
    RowInfo ri;
    const float bound = qnorm[w][lane] * kmx * fabsf(mscale) * 1.001f;
    ri.iw = (bound > 0.f && bound < FLT_MAX) ? 128.0f / bound : 0.f;
    ri.bstar = -1;
    ri.need = min(kr, nv);
    ri.mode = (nv <= kr) ? SELECT_ALL : (FB ? RADIX : BIN_ALL);
    ri.pfx = 0; ri.msk = 0; ri.done = (FB && nv > kr) ? 0 : 1; ri.th0 = -INFINITY; ri.th1 = -INFINITY;
    rinfo[w][lane] = ri;
  }
  for (int i = lane; i < 16 * HWA; i += 64) (&hist[w][0][0])[i] = 0;
  __syncthreads();

  float iw[4];
  int mode[4], bstar[4], need[4], rdone[4];
  uint32_t pfx[4], msk[4];
  auto reload = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const RowInfo ri = rinfo[w][4 * lg + e];
      iw[e] = ri.iw; mode[e] = ri.mode; bstar[e] = ri.bstar; need[e] = ri.need;
      pfx[e] = ri.pfx; msk[e] = ri.msk; rdone[e] = ri.done;
    }
  };
  reload();

  auto read_counts = [&](int rr, uint32_t (&c)[4]) __attribute__((always_inline)) {
    if constexpr (C16) {
      const uint32_t w0 = hist[w][rr][127 - 2 * lane], w1 = hist[w][rr][126 - 2 * lane];
      c[0] = w0 >> 16; c[1] = w0 & 0xffffu; c[2] = w1 >> 16; c[3] = w1 & 0xffffu;
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) c[q] = hist[w][rr][255 - 4 * lane - q];
    }
  };
  auto clear_counts = [&](int rr) __attribute__((always_inline)) {
    if constexpr (C16) {
      hist[w][rr][127 - 2 * lane] = 0;
      hist[w][rr][126 - 2 * lane] = 0;
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) hist[w][rr][255 - 4 * lane - q] = 0;
    }
  };
  // bits: score_bin_bits (bin in the low 8 bits)
  auto bump = [&](int row, uint32_t bits) __attribute__((always_inline)) {
    // C16: word bin >> 1, half bin & 1; the increment's shift 16 (bin & 1) equals
    // (bits << 4) mod 32, and the shift instruction reads only those 5 bits
    if constexpr (C16) atomicAdd(&hist[w][row][__builtin_amdgcn_ubfe(bits, 1, 7)], 1u << ((bits << 4) & 31u));
    else atomicAdd(&hist[w][row][bits & 0xffu], 1u);
  };

  // ---- pass A: score-bin histogram -------------------------------------------
  if constexpr (!FB) {
    int mine = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) mine |= (mode[e] != SELECT_ALL);
    const bool wave_busy = ballot64(mine) != 0;
    if (__syncthreads_or(mine)) {
      bool hrow[4];   // rows of this lane that build a histogram
#pragma unroll
      for (int e = 0; e < 4; ++e) hrow[e] = live[e] && mode[e] != SELECT_ALL;
      sweep([&](int kt, f4* acc) __attribute__((always_inline)) {
        if (!wave_busy) return;
        if ((kt + 1) * KT <= minvalid) {   // every key of the tile is valid for every live row
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (hrow[e]) bump(4 * lg + e, score_bin_bits(acc[nt][e], iw[e]));
            }
          }
        } else {
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) {
            const int j = kt * KT + 16 * nt + lr;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (hrow[e] && j < nvalid[e]) bump(4 * lg + e, score_bin_bits(acc[nt][e], iw[e]));
            }
          }
        }
      });
      __syncthreads();
      for (int rr = 0; rr < 16; ++rr) {
        RowInfo ri = rinfo[w][rr];
        if (ri.mode == SELECT_ALL) continue;
        uint32_t c[4];
        read_counts(rr, c);
        int bin;
        uint32_t above, cnt;
        find_bin(c, lane, (uint32_t)ri.need, bin, above, cnt);
        if (lane == 0) {
          ri.bstar = bin;
          ri.need -= (int)above;
          if (cnt == (uint32_t)ri.need) ri.mode = BIN_ALL;
          else if (cnt <= (uint32_t)TOPK_CAP) ri.mode = COLLECT;
          else ri.mode = RADIX;
          rinfo[w][rr] = ri;
        }
        clear_counts(rr);
      }
      __syncthreads();
      reload();
    }
    int overflow = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) overflow |= (mode[e] == RADIX);
    overflow = __syncthreads_or(overflow);
    if (tid == 0) a.flags[bid] = overflow;
    if (overflow) return;   // block-uniform; the fallback launch redoes this block
  }

  // ---- fallback: radix digits over the keys ---------------------------------
  if constexpr (FB) for (int sh = 24; sh >= 0; sh -= 8) {
    int mine = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) mine |= (mode[e] == RADIX && !rdone[e]);
    const bool wave_busy = ballot64(mine) != 0;
    if (!__syncthreads_or(mine)) break;
    sweep([&](int kt, f4* acc) __attribute__((always_inline)) {
      if (!wave_busy) return;
      const bool full = (kt + 1) * KT <= minvalid;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int j = kt * KT + 16 * nt + lr;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float s = acc[nt][e];
          const uint32_t key = f32_order_key(s);
          if (live[e] && mode[e] == RADIX && !rdone[e] && (full || j < nvalid[e]) && (key & msk[e]) == pfx[e])
            bump(4 * lg + e, (key >> sh) & 255u);
        }
      }
    });
    __syncthreads();
    for (int rr = 0; rr < 16; ++rr) {
      RowInfo ri = rinfo[w][rr];
      if (ri.mode != RADIX || ri.done) continue;
      uint32_t c[4];
      read_counts(rr, c);
      int bin;
      uint32_t above, cnt;
      find_bin(c, lane, (uint32_t)ri.need, bin, above, cnt);
      if (lane == 0) {
        ri.pfx |= (uint32_t)bin << sh;
        ri.msk |= 0xffu << sh;
        ri.need -= (int)above;
        ri.done = (cnt == (uint32_t)ri.need || sh == 0) ? 1 : 0;
        rinfo[w][rr] = ri;
      }
      clear_counts(rr);
    }
    __syncthreads();
    reload();
  }

  // ---- thresholds for pass B -------------------------------------------------
  if (lane < 16) {
    RowInfo ri = rinfo[w][lane];
    float t0 = -INFINITY, t1 = -INFINITY;
    if (FB && ri.mode == RADIX) {
      t0 = INFINITY; t1 = INFINITY;   // every candidate goes through the key path
    } else if (!FB && ri.mode != SELECT_ALL) {
      const float lo_b = ri.bstar > 0 ? bin_lower_edge(ri.bstar, ri.iw) : -INFINITY;
      const float hi_b = ri.bstar < NBIN - 1 ? bin_lower_edge(ri.bstar + 1, ri.iw) : INFINITY;
      if (ri.mode == BIN_ALL) { t0 = lo_b; t1 = lo_b; }
      else { t0 = lo_b; t1 = hi_b; }   // COLLECT
    }
    ri.th0 = t0; ri.th1 = t1;
    rinfo[w][lane] = ri;
  }
  __syncthreads();

  // ---- pass B: emit above b*, collect b* -------------------------------------
  float th0[4], th1[4];
  int outc[4], colc[4];
  float m1[4], m2[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    th0[e] = rinfo[w][4 * lg + e].th0;
    th1[e] = rinfo[w][4 * lg + e].th1;
    outc[e] = 0; colc[e] = 0; m1[e] = -FLT_MAX; m2[e] = -FLT_MAX;
  }
  const int grow0 = bh * Tq + r0 + 16 * w + 4 * lg;   // global row of e = 0
  const uint32_t lower = (1u << lr) - 1u;
  uint2* scratch = a.scratch;
  // LIST: the wave's tile list (layer path) -- entries (score, row << 8 | key in
  // tile) grouped by key tile in ascending tile order, toff[kt] = first entry of
  // tile kt, toff[ntile] = end.  Threshold-bin candidates get an entry as well;
  // the resolve overwrites the score of those not selected with -inf.
  const int tlcap = 16 * (topk + TOPK_CAP);
  const long lreg = ((long)bh * nqb + qb) * 4 + w;
  uint2* tl = TL ? a.tl_list + lreg * tlcap : nullptr;
  int32_t* toff = TL ? a.tl_off + lreg * (a.tl_ntmax + 1) : nullptr;
  int woff = 0;
  int cutj[4] = {-1, -1, -1, -1};   // THR: key index of the last threshold tie selected (lane-local)
  auto emit = [&](int e, int kk, int j, float s, bool sel, bool col) __attribute__((always_inline)) {
    const uint32_t sm = (uint32_t)(ballot64(sel) >> (16 * lg)) & 0xffffu;
    const uint32_t cm = (uint32_t)(ballot64(col) >> (16 * lg)) & 0xffffu;
    const long row = (long)(grow0 + e);
    if (sel) {
      const int slot = outc[e] + __popc(sm & lower);
      if (!LIST && slot < topk) {
        a.indices[row * topk + slot] = j;
        a.scores[row * topk + slot] = s;
      }
    }
    if (col) {
      const int slot = colc[e] + __popc(cm & lower);
      if (slot < TOPK_CAP) scratch[row * TOPK_CAP + slot] = make_uint2(__float_as_uint(s), (uint32_t)j);
    }
    outc[e] += __popc(sm);
    colc[e] += __popc(cm);
  };
  auto top2_update = [&](int e, bool ok, float s) __attribute__((always_inline)) {
    if constexpr (TOP2) {
      const float so = ok ? s : -FLT_MAX;   // running top-2 with multiplicity
      m2[e] = fmaxf(m2[e], fminf(m1[e], so));
      m1[e] = fmaxf(m1[e], so);
    }
  };
  // LIST entries: {score, row_in_wave << 8 | key_in_tile}.  Every candidate
  // (s >= th0: selected or in the threshold bin) gets the next entry of the
  // wave's list in lane order; the position is a ballot + mbcnt against the
  // wave-uniform running offset.
  const uint32_t rk0 = ((uint32_t)(4 * lg) << 8) | (uint32_t)lr;
  float th0e[4];                                       // th0 with dead rows folded in (+inf)
#pragma unroll
  for (int e = 0; e < 4; ++e) th0e[e] = live[e] ? th0[e] : INFINITY;
  // direct emission (radix fallback launch: no threshold bin)
  auto emit_list = [&](int e, int nt, float s, bool cand) __attribute__((always_inline)) {
    const uint64_t cb = ballot64(cand);
    const uint32_t pos = min((uint32_t)woff + lane_rank(cb), (uint32_t)tlcap - 1u);
    if (cand) tl[pos] = make_uint2(__float_as_uint(s), rk0 + (uint32_t)((e << 8) + 16 * nt));
    woff = __builtin_amdgcn_readfirstlane(woff + __popcll(cb));
  };
  // running top-2 (m1 >= m2): med3 gives the new second before m1 moves
  auto top2_fast = [&](int e, float x) __attribute__((always_inline)) {
    m2[e] = __builtin_amdgcn_fmed3f(m1[e], m2[e], x);
    m1[e] = fmaxf(m1[e], x);
  };
  if constexpr (!FB && LIST) {
    // A tile's candidates are first gathered in LDS -- the wave's histogram area,
    // idle between pass A and the resolve, holds a whole tile (16 rows x 64 keys)
    // -- and then written to the wave's list with full-wave stores.  Bit 31 of
    // a buffered entry marks a threshold-bin candidate; the flush also gives it
    // a slot in its row's scratch list (an LDS counter per row), so the slot
    // order within a row is arbitrary and the resolve breaks ties by position.
    static_assert(16 * HWA >= 2 * 16 * KT, "a tile's candidates must fit the histogram area");
    uint2* ebuf = reinterpret_cast<uint2*>(&hist[w][0][0]);
    const long srow0 = (long)bh * Tq + r0 + 16 * w;   // global row of the wave's row 0
    if (lane < 16) rowcnt[w][lane][1] = 0;
    int tcnt = 0;
    auto emit_buf = [&](int e, int nt, float s, bool cand) __attribute__((always_inline)) {
      const uint64_t cb = ballot64(cand);
      if (cand)
        ebuf[(uint32_t)tcnt + lane_rank(cb)] =
            make_uint2(__float_as_uint(s), rk0 + (uint32_t)((e << 8) + 16 * nt) + (s < th1[e] ? 0x80000000u : 0u));
      tcnt = __builtin_amdgcn_readfirstlane(tcnt + __popcll(cb));
    };
    sweep([&](int kt, f4* acc) __attribute__((always_inline)) {
      // A row holds at most top_k + TOPK_CAP candidates of which at most TOPK_CAP
      // in its threshold bin, so neither list can fill up; the bounds below only
      // keep one tile's writes inside the regions whatever the inputs.
      woff = min(woff, tlcap - 16 * KT);
      if (lane == 0) toff[kt] = woff;
      tcnt = 0;
      if ((kt + 1) * KT <= minvalid) {
        // full tile: every key is valid for every live row
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float s = acc[nt][e];
            emit_buf(e, nt, s, s >= th0e[e]);
            top2_fast(e, s);
          }
        }
      } else {
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          const int j = kt * KT + 16 * nt + lr;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const bool ok = live[e] && j < nvalid[e];
            const float s = acc[nt][e];
            emit_buf(e, nt, s, s >= th0e[e] && j < nvalid[e]);
            top2_fast(e, ok ? s : -FLT_MAX);
          }
        }
      }
      // flush, two chunks of 64 per step (LDS accesses of one wave complete in order)
      auto flush_one = [&](bool ok, uint2 ent, int c) __attribute__((always_inline)) {
        const bool col = ok && (ent.y >> 31) != 0u;
        ent.y &= 0x7fffffffu;
        const uint32_t pos = (uint32_t)(woff + c + lane);
        if (ok) tl[pos] = ent;
        if (col) {
          const int r = (int)(ent.y >> 8);   // row in wave
          const int slot = (int)atomicAdd((uint32_t*)&rowcnt[w][r][1], 1u);
          if (slot < TOPK_CAP) scratch[(srow0 + r) * TOPK_CAP + slot] = make_uint2(ent.x, pos);
        }
      };
      for (int c0 = 0; c0 < tcnt; c0 += 128) {
        const bool ok0 = c0 + lane < tcnt, ok1 = c0 + 64 + lane < tcnt;
        const uint2 e0 = ok0 ? ebuf[c0 + lane] : make_uint2(0u, 0u);
        const uint2 e1 = ok1 ? ebuf[c0 + 64 + lane] : make_uint2(0u, 0u);
        flush_one(ok0, e0, c0);
        flush_one(ok1, e1, c0 + 64);
      }
      woff = __builtin_amdgcn_readfirstlane(woff + tcnt);
    });
  } else if constexpr (!FB) {
    sweep([&](int kt, f4* acc) __attribute__((always_inline)) {
      const bool full = (kt + 1) * KT <= minvalid;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int j = kt * KT + 16 * nt + lr;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool ok = live[e] && (full || j < nvalid[e]);
          const float s = acc[nt][e];
          const bool sel = ok && s >= th1[e];
          const bool col = ok && s >= th0[e] && s < th1[e];
          emit(e, 16 * nt + lr, j, s, sel, col);
          top2_update(e, ok, s);
        }
      }
    });
  } else {
    int eqc[4] = {0, 0, 0, 0};
    sweep([&](int kt, f4* acc) __attribute__((always_inline)) {
      if constexpr (TL) {
        if (lane == 0) toff[kt] = woff;
      }
      const bool full = (kt + 1) * KT <= minvalid;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int j = kt * KT + 16 * nt + lr;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool ok = live[e] && (full || j < nvalid[e]);
          const float s = acc[nt][e];
          bool sel = ok && s >= th1[e];
          const bool col = ok && s >= th0[e] && s < th1[e];
          const uint32_t km = f32_order_key(s) & msk[e];
          const bool inb = ok && mode[e] == RADIX;
          const bool eq = inb && km == pfx[e];
          const uint32_t eqm = (uint32_t)(ballot64(eq) >> (16 * lg)) & 0xffffu;
          sel = sel || (inb && (km > pfx[e] || (eq && eqc[e] + __popc(eqm & lower) < need[e])));
          if constexpr (THR) {
            if (eq && eqc[e] + (int)__popc(eqm & lower) == need[e] - 1) cutj[e] = j;   // last tie selected
          }
          eqc[e] += __popc(eqm);
          if constexpr (TL) emit_list(e, nt, s, sel);
          else if constexpr (!THR) emit(e, 16 * nt + lr, j, s, sel, col);
          top2_update(e, ok, s);
        }
      }
    });
  }
  if constexpr (TL) {
    if (lane == 0) toff[ntile] = woff;
  }
  if (lr == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      rowcnt[w][4 * lg + e][0] = outc[e];
      if (!LIST || FB) rowcnt[w][4 * lg + e][1] = colc[e];
      run1[w][4 * lg + e] = outc[e];
    }
  }
  __syncthreads();

  // ---- resolve collected rows: exact threshold among <= TOPK_CAP scores -----
  uint32_t* h256 = &hist[w][0][0];   // 256 words of this wave's histogram area
  if constexpr (!FB) for (int rr = 0; rr < 16; ++rr) {
    const RowInfo ri = rinfo[w][rr];
    if (ri.mode != COLLECT) continue;
    const long row = (long)bh * Tq + (r0 + 16 * w + rr);
    const int n = min(rowcnt[w][rr][1], TOPK_CAP);
    int base = rowcnt[w][rr][0];
    uint32_t key[CAPL];
    int idx[CAPL];
#pragma unroll
    for (int m = 0; m < CAPL; ++m) {
      const int p = 64 * m + lane;
      key[m] = 0; idx[m] = 0;
      if (p < n) {
        const uint2 v = scratch[row * TOPK_CAP + p];
        key[m] = f32_order_key(__uint_as_float(v.x));
        idx[m] = (int)v.y;
      }
    }
    // every collected key lies in [key(th0), key(th1) - 1]: the bytes those two
    // share are the same for all of them and need no pass
    const uint32_t klo = f32_order_key(ri.th0), dif = klo ^ (f32_order_key(ri.th1) - 1u);
    uint32_t rm = 0;
    int sh = 24;
    while (sh > 0 && (dif >> sh) == 0u) { rm |= 0xffu << sh; sh -= 8; }
    uint32_t rp = klo & rm;
    uint32_t rneed = (uint32_t)ri.need;
    for (; sh >= 0; sh -= 8) {
#pragma unroll
      for (int q = 0; q < 4; ++q) h256[4 * lane + q] = 0;
      wave_lds_sync();
#pragma unroll
      for (int m = 0; m < CAPL; ++m) {
        if (64 * m + lane < n && (key[m] & rm) == rp) atomicAdd(&h256[(key[m] >> sh) & 255u], 1u);
      }
      wave_lds_sync();
      uint32_t c[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) c[q] = h256[255 - 4 * lane - q];
      int bin;
      uint32_t above, cnt;
      find_bin(c, lane, rneed, bin, above, cnt);
      rp |= (uint32_t)bin << sh;
      rm |= 0xffu << sh;
      rneed -= above;
      wave_lds_sync();
      if (cnt == rneed) break;
    }
    // Keys equal to the threshold key: the rneed with the smallest idx win (idx
    // is the key index, or in LIST mode the entry position, which grows with the
    // key index within a row).  Only when more are equal than needed does a radix
    // select over ~idx find the cut; the slot order of the scratch list is free.
    uint32_t neq = 0;
#pragma unroll
    for (int m = 0; m < CAPL; ++m) neq += (uint32_t)__popcll(ballot64(64 * m + lane < n && (key[m] & rm) == rp));
    uint32_t ip = 0, im = 0;
    if (neq > rneed) {
      uint32_t need2 = rneed;
      for (int sh = 24; sh >= 0; sh -= 8) {
#pragma unroll
        for (int q = 0; q < 4; ++q) h256[4 * lane + q] = 0;
        wave_lds_sync();
#pragma unroll
        for (int m = 0; m < CAPL; ++m) {
          const uint32_t ik = ~(uint32_t)idx[m];
          if (64 * m + lane < n && (key[m] & rm) == rp && (ik & im) == ip) atomicAdd(&h256[(ik >> sh) & 255u], 1u);
        }
        wave_lds_sync();
        uint32_t c[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) c[q] = h256[255 - 4 * lane - q];
        int bin;
        uint32_t above, cnt;
        find_bin(c, lane, need2, bin, above, cnt);
        ip |= (uint32_t)bin << sh;
        im |= 0xffu << sh;
        need2 -= above;
        wave_lds_sync();
        if (cnt == need2) break;
      }
    }
    const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
    for (int m = 0; m < CAPL; ++m) {
      const bool valid = 64 * m + lane < n;
      const uint32_t km = key[m] & rm;
      const bool eq = valid && km == rp;
      const bool sel = valid && (km > rp || (eq && (neq <= rneed || ((~(uint32_t)idx[m]) & im) >= ip)));
      const uint64_t sb = ballot64(sel);
      if constexpr (LIST) {
        if (valid && !sel && idx[m] >= 0 && idx[m] < tlcap) tl[idx[m]].x = 0xff800000u;   // -inf: weight 0
      } else if (sel) {
        const int slot = base + __popcll(sb & below);
        if (slot < topk) {
          a.indices[row * topk + slot] = idx[m];
          a.scores[row * topk + slot] = key_to_f32(key[m]);
        }
      }
      base += __popcll(sb);
    }
    if (lane == 0) rowcnt[w][rr][0] = base;
  }
  __syncthreads();

  // ---- merge top-2, pad, counts --------------------------------------------
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const long rowg = (long)(grow0 + e);
    if constexpr (TOP2) {
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const float b1 = __shfl_xor(m1[e], o, 64), b2 = __shfl_xor(m2[e], o, 64);
        const float hi = fmaxf(m1[e], b1), lo = fmaxf(fminf(m1[e], b1), fmaxf(m2[e], b2));
        m1[e] = hi; m2[e] = lo;
      }
    }
    if constexpr (THR) {
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) cutj[e] = max(cutj[e], __shfl_xor(cutj[e], o, 64));
    }
    if (!live[e]) continue;
    if constexpr (THR) {
      if (lr == 0) {
        float th = -INFINITY;
        int cut = 0x7fffffff;
        if (mode[e] == RADIX) {
          th = threshold_of_key(pfx[e]);
          if (msk[e] == 0xffffffffu) cut = cutj[e];
        }
        a.thr[rowg] = make_uint2(__float_as_uint(th), (uint32_t)cut);
      }
    }
    // LIST: every row selects exactly min(its slots, valid keys)
    const int qre = r0 + 16 * w + 4 * lg + e;
    const int kre = (masked && a.row_kq != nullptr) ? min(topk, a.row_kq[qre]) : topk;
    const int oc = LIST ? min(kre, nvalid[e]) : min(rowcnt[w][4 * lg + e][0], topk);
    if (!LIST) for (int p = oc + lr; p < topk; p += 16) {
      a.indices[rowg * topk + p] = 0;
      a.scores[rowg * topk + p] = -FLT_MAX;
    }
    if (lr == 0) {
      if (a.counts) a.counts[rowg] = oc;
      if (a.split) a.split[rowg] = min(run1[w][4 * lg + e], oc);
      if constexpr (TOP2) { a.top2[2 * rowg] = m1[e]; a.top2[2 * rowg + 1] = m2[e]; }
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
    ip[i] = (int32_t)(0xffffffffu - (uint32_t)(key & 0xffffffffu));
    sp[i] = key_to_f32((uint32_t)(key >> 32));
  }
}

// ---------------------------------------------------------------------------
// K1, tile-list form (layer path: bf16, D = 128, top-2 required).
//
// The same selection as score_topk_kernel<..., LIST = true>, with pass A laid
// out so that no K tile goes through LDS.  The K tiles are re-read from L2 for
// every 64-row block; staging them (global -> VGPR -> LDS -> VGPR, two barriers
// a tile) for 16 rows per wave cost more than the histogram arithmetic.  In
// pass A wave w owns keys [16w, 16w+16) of every 64-key tile for all 64 rows of
// the block: its 16 keys are the MFMA A operand, loaded straight into registers
// one tile ahead, and the block's q rows are the B operand, resident in
// registers.  The product C[key][row] puts 4 keys of 4 rows (16g + lr) in each
// lane and all four waves bump the same 64 row histograms.  Each product sums
// the same 32 dims per instruction as score_topk_kernel, so the fp32 scores
// are identical.  MFMA row rho of the A operand holds key rho/4 + 4 (rho%4).
//
// Pass B keeps score_topk_kernel's layout (wave w: rows 16w.., K tile in LDS):
// every score of a row is then in one wave, which keeps the emission buffer,
// its flush to the tile list and the top-2 wave-private.
// A block with a row whose threshold bin overflows is flagged for the radix
// fallback launch of score_topk_kernel<..., FB = true, LIST = true>, which
// writes the same lists.
// ---------------------------------------------------------------------------
//
// THR (threshold mode, the layer path): no lists.  Pass B runs pass A's
// register sweep again and only collects the threshold-bin candidates (from
// every wave into per-row LDS counters and the scratch lists); the resolve
// then leaves each row's exact cut in thr: {fp32 threshold th, key index cut},
// key j selected iff s > th, or s == th and j <= cut.
// ---------------------------------------------------------------------------
template <bool C16, bool THR>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void score_topk_tiles_kernel(
    TopkArgs a, int nqb, float mscale) {
  constexpr int HW = C16 ? NBIN / 2 : NBIN;   // histogram words per row
  constexpr int CAPL = TOPK_CAP / 64;
  constexpr int PB = DP + 8;                  // LDS pitch of a K row (272 B keeps 16 B alignment)
  __shared__ __align__(16) uint32_t hist[64][HW];   // rows of the block; pass B: emission buffers
  __shared__ RowInfo rinfo[4][16];
  __shared__ int colcnt[4][16];                     // threshold-bin candidates collected per row
  __shared__ float qnorm[4][16];
  __shared__ __align__(16) uint16_t ks[KT * PB];    // pass B: the K tile

  const int BH = a.B * a.H;
  const int bid = blockIdx.x;
  const int bh = bid % BH;
  const int qb = nqb - 1 - bid / BH;   // heaviest (latest) query blocks first
  const int b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int r0 = qb * QB;
  const int Tq = a.Tq, Tk = a.Tk, H = a.H;
  const uint16_t* kb = reinterpret_cast<const uint16_t*>(a.k);
  const int topk = a.top_k;

  // B operand: q^T of the block's rows; lane holds row r0 + 16g + lr, dims 32s + 8lg + [0, 8)
  bf16x8 qf[4][4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int qr = r0 + 16 * g + lr;
    const uint16_t* qp = reinterpret_cast<const uint16_t*>(a.q) + ((long)(b * Tq + (qr < Tq ? qr : 0)) * H + h) * DP;
    float qn2 = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u16x8 raw;
      if (qr < Tq) raw = *reinterpret_cast<const u16x8*>(qp + 32 * s + 8 * lg);
      else raw = (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float x = bf16_to_f32(raw[j]);
        qn2 = fmaf(x, x, qn2);
      }
      qf[g][s] = __builtin_bit_cast(bf16x8, raw);
    }
    qn2 += __shfl_xor(qn2, 16, 64);
    qn2 += __shfl_xor(qn2, 32, 64);
    if (g == w && lg == 0) qnorm[w][lr] = sqrtf(qn2);
  }

  // the lane's rows r0 + 16g + lr
  int nvalid[4];
  bool live[4];
  int minvalid = 0x7fffffff;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int qr = r0 + 16 * g + lr;
    live[g] = qr < Tq;
    int nv = Tk;
    if (a.causal) nv = min(Tk, qr + a.q_offset + 1);
    if (nv < 0) nv = 0;
    nvalid[g] = live[g] ? nv : 0;
    if (live[g]) minvalid = min(minvalid, nvalid[g]);
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) minvalid = min(minvalid, __shfl_xor(minvalid, o, 64));
  int kend = Tk;
  if (a.causal) kend = min(Tk, min(Tq, r0 + QB) - 1 + a.q_offset + 1);
  const int ntile = (kend + KT - 1) / KT;

  // A operand: the wave's 16 keys of a tile; MFMA row lr holds key lr/4 + 4 (lr%4)
  const int krow = (lr >> 2) + 4 * (lr & 3);
  bf16x8 kf[4];
  auto kload = [&](int kt) __attribute__((always_inline)) {
    const int j = kt * KT + 16 * w + krow;
    const bool okj = j < Tk;
    const uint16_t* p = kb + ((long)(b * Tk + (okj ? j : 0)) * H + h) * DP + 8 * lg;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u16x8 raw = *reinterpret_cast<const u16x8*>(p + 32 * s);
      if (!okj) raw = (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
      kf[s] = __builtin_bit_cast(bf16x8, raw);
    }
  };
  // fn(kt, acc): acc[g][i] = score of row r0 + 16g + lr against key kt*64 + 16w + lg + 4i
  auto sweep = [&](auto&& fn) __attribute__((always_inline)) {
    kload(0);
    for (int kt = 0; kt < ntile; ++kt) {
      f4 acc[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f4 c = f4_zero();
#pragma unroll
        for (int s = 0; s < 4; ++s) c = mma_bf16(kf[s], qf[g][s], c);
        acc[g] = score_of(c, mscale);
      }
      if (kt + 1 < ntile) kload(kt + 1);
      fn(kt, acc);
    }
  };

  // row set-up (wave w: rows r0 + 16w + lane)
  __syncthreads();   // qnorm visible
  float kmx2 = lane < KNCH ? a.kmax[(long)bh * KNCH + lane] : 0.f;
  const float kmx = sqrtf(wave_max(kmx2));
  if (lane < 16) {
    const int qr = r0 + 16 * w + lane;
    int nv = 0;
    if (qr < Tq) nv = a.causal ? max(0, min(Tk, qr + a.q_offset + 1)) : Tk;
    RowInfo ri;
    const float bound = qnorm[w][lane] * kmx * fabsf(mscale) * 1.001f;
    ri.iw = (bound > 0.f && bound < FLT_MAX) ? 128.0f / bound : 0.f;
    ri.bstar = -1;
    ri.need = min(topk, nv);
    ri.mode = (nv <= topk) ? SELECT_ALL : BIN_ALL;
    ri.pfx = 0; ri.msk = 0; ri.done = 1; ri.th0 = -INFINITY; ri.th1 = -INFINITY;
    rinfo[w][lane] = ri;
    colcnt[w][lane] = 0;
  }
  for (int i = tid; i < 64 * HW; i += 256) (&hist[0][0])[i] = 0;
  __syncthreads();

  float iw[4];
  int mode[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) { iw[g] = rinfo[g][lr].iw; mode[g] = rinfo[g][lr].mode; }

  // ---- pass A: block-shared row histograms ------------------------------------
  {
    int mine = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) mine |= (live[g] && mode[g] != SELECT_ALL);
    if (__syncthreads_or(mine)) {
      bool hrow[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) hrow[g] = live[g] && mode[g] != SELECT_ALL;
      auto bump = [&](int row, uint32_t bits) __attribute__((always_inline)) {
        // C16: word bin >> 1, half bin & 1; the shift 16 (bin & 1) is (bits << 4) mod 32
        if constexpr (C16) atomicAdd(&hist[row][__builtin_amdgcn_ubfe(bits, 1, 7)], 1u << ((bits << 4) & 31u));
        else atomicAdd(&hist[row][bits & 0xffu], 1u);
      };
      sweep([&](int kt, f4* acc) __attribute__((always_inline)) {
        if ((kt + 1) * KT <= minvalid) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (hrow[g]) bump(16 * g + lr, score_bin_bits(acc[g][i], iw[g]));
          }
        } else {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int j = kt * KT + 16 * w + lg + 4 * i;
              if (hrow[g] && j < nvalid[g]) bump(16 * g + lr, score_bin_bits(acc[g][i], iw[g]));
            }
          }
        }
      });
      __syncthreads();
      for (int rr = 0; rr < 16; ++rr) {
        RowInfo ri = rinfo[w][rr];
        if (ri.mode == SELECT_ALL) continue;
        const uint32_t* hr = hist[16 * w + rr];
        uint32_t c[4];
        if constexpr (C16) {
          const uint32_t w0 = hr[127 - 2 * lane], w1 = hr[126 - 2 * lane];
          c[0] = w0 >> 16; c[1] = w0 & 0xffffu; c[2] = w1 >> 16; c[3] = w1 & 0xffffu;
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) c[q] = hr[255 - 4 * lane - q];
        }
        int bin;
        uint32_t above, cnt;
        find_bin(c, lane, (uint32_t)ri.need, bin, above, cnt);
        if (lane == 0) {
          ri.bstar = bin;
          ri.need -= (int)above;
          if (cnt == (uint32_t)ri.need) ri.mode = BIN_ALL;
          else if (cnt <= (uint32_t)TOPK_CAP) ri.mode = COLLECT;
          else ri.mode = RADIX;
          rinfo[w][rr] = ri;
        }
      }
    }
    __syncthreads();
    int overflow = 0;
    if (lane < 16) overflow = rinfo[w][lane].mode == RADIX;
    overflow = __syncthreads_or(overflow);
    if (tid == 0) a.flags[bid] = overflow;
    if (overflow) return;   // block-uniform; the fallback launch redoes this block
  }

  // ---- thresholds for pass B ---------------------------------------------------
  if (lane < 16) {
    RowInfo ri = rinfo[w][lane];
    float t0 = -INFINITY, t1 = -INFINITY;
    if (ri.mode != SELECT_ALL) {
      const float lo_b = ri.bstar > 0 ? bin_lower_edge(ri.bstar, ri.iw) : -INFINITY;
      const float hi_b = ri.bstar < NBIN - 1 ? bin_lower_edge(ri.bstar + 1, ri.iw) : INFINITY;
      if (ri.mode == BIN_ALL) { t0 = lo_b; t1 = lo_b; }
      else { t0 = lo_b; t1 = hi_b; }   // COLLECT
    }
    ri.th0 = t0; ri.th1 = t1;
    rinfo[w][lane] = ri;
  }
  __syncthreads();

  if constexpr (THR) {
    // ---- pass B (threshold mode): threshold-bin candidates, top-2 --------------
    // Lane (w, lg, lr) sees row r0 + 16g + lr against keys kt*64 + 16w + lg + 4i.
    float tb0[4], tb1[4], m1[4], m2[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const RowInfo ri = rinfo[g][lr];
      tb0[g] = (live[g] && ri.mode == COLLECT) ? ri.th0 : INFINITY;   // only COLLECT rows have a bin to resolve
      tb1[g] = ri.th1;
      m1[g] = -FLT_MAX; m2[g] = -FLT_MAX;
    }
    uint2* scratch = a.scratch;
    const long srowb = (long)bh * Tq + r0;   // global row of the block's row 0
    auto collect = [&](int g, int j, float sc) __attribute__((always_inline)) {
      const int slot = (int)atomicAdd((uint32_t*)&colcnt[g][lr], 1u);
      if (slot < TOPK_CAP) scratch[(srowb + 16 * g + lr) * TOPK_CAP + slot] = make_uint2(__float_as_uint(sc), (uint32_t)j);
    };
    sweep([&](int kt, f4* acc) __attribute__((always_inline)) {
      const bool full = (kt + 1) * KT <= minvalid;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = kt * KT + 16 * w + lg + 4 * i;
          const float sc = acc[g][i];
          const bool ok = full || j < nvalid[g];   // nvalid is 0 for dead rows
          m2[g] = __builtin_amdgcn_fmed3f(m1[g], m2[g], ok ? sc : -FLT_MAX);
          m1[g] = fmaxf(m1[g], ok ? sc : -FLT_MAX);
          if (ok & (sc >= tb0[g]) & (sc < tb1[g])) collect(g, j, sc);
        }
      }
    });
    // top-2 over the row's lanes of this wave (lg), then over the waves (LDS)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
      for (int o = 16; o < 64; o <<= 1) {
        const float b1 = __shfl_xor(m1[g], o, 64), b2 = __shfl_xor(m2[g], o, 64);
        const float hi = fmaxf(m1[g], b1), lo = fmaxf(fminf(m1[g], b1), fmaxf(m2[g], b2));
        m1[g] = hi; m2[g] = lo;
      }
    }
    __syncthreads();   // candidates and counters of every wave are in place; hist is free
    float2* t2s = reinterpret_cast<float2*>(&hist[0][0]);   // [wave][64 rows]
    if (lg == 0) {
#pragma unroll
      for (int g = 0; g < 4; ++g) t2s[64 * w + 16 * g + lr] = make_float2(m1[g], m2[g]);
    }
    __syncthreads();
    float2 t2 = make_float2(-FLT_MAX, -FLT_MAX);
    if (lane < 16) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float2 o = t2s[64 * v + 16 * w + lane];
        const float hi = fmaxf(t2.x, o.x), lo = fmaxf(fminf(t2.x, o.x), fmaxf(t2.y, o.y));
        t2.x = hi; t2.y = lo;
      }
    }
    __syncthreads();   // hist is the resolve's histogram area from here on

    // ---- resolve: the exact cut of every COLLECT row of the wave --------------
    uint32_t* h256 = &hist[16 * w][0];
    float thv = -INFINITY;   // lane rr < 16: row 16w + rr
    int cutv = 0x7fffffff;
    for (int rr = 0; rr < 16; ++rr) {
      const RowInfo ri = rinfo[w][rr];
      if (ri.mode == BIN_ALL && lane == rr) thv = ri.th0;   // everything from the bin's lower edge up
      if (ri.mode != COLLECT) continue;
      const long row = srowb + 16 * w + rr;
      const int n = min(colcnt[w][rr], TOPK_CAP);
      uint32_t key[CAPL];
      int idx[CAPL];
#pragma unroll
      for (int m = 0; m < CAPL; ++m) {
        const int p = 64 * m + lane;
        key[m] = 0; idx[m] = 0;
        if (p < n) {
          const uint2 v = scratch[row * TOPK_CAP + p];
          key[m] = f32_order_key(__uint_as_float(v.x));
          idx[m] = (int)v.y;
        }
      }
      const uint32_t klo = f32_order_key(ri.th0), dif = klo ^ (f32_order_key(ri.th1) - 1u);
      uint32_t rm = 0;
      int sh = 24;
      while (sh > 0 && (dif >> sh) == 0u) { rm |= 0xffu << sh; sh -= 8; }
      uint32_t rp = klo & rm;
      uint32_t rneed = (uint32_t)ri.need;
      for (; sh >= 0; sh -= 8) {
#pragma unroll
        for (int q = 0; q < 4; ++q) h256[4 * lane + q] = 0;
        wave_lds_sync();
#pragma unroll
        for (int m = 0; m < CAPL; ++m) {
          if (64 * m + lane < n && (key[m] & rm) == rp) atomicAdd(&h256[(key[m] >> sh) & 255u], 1u);
        }
        wave_lds_sync();
        uint32_t c[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) c[q] = h256[255 - 4 * lane - q];
        int bin;
        uint32_t above, cnt;
        find_bin(c, lane, rneed, bin, above, cnt);
        rp |= (uint32_t)bin << sh;
        rm |= 0xffu << sh;
        rneed -= above;
        wave_lds_sync();
        if (cnt == rneed) break;
      }
      // Keys at the threshold key rp: the rneed with the smallest key index win;
      // a radix select over ~index finds the last of them when more are equal.
      uint32_t neq = 0;
#pragma unroll
      for (int m = 0; m < CAPL; ++m) neq += (uint32_t)__popcll(ballot64(64 * m + lane < n && (key[m] & rm) == rp));
      uint32_t ip = 0;
      if (neq > rneed) {
        uint32_t im = 0, need2 = rneed;
        for (int sh2 = 24; sh2 >= 0; sh2 -= 8) {
#pragma unroll
          for (int q = 0; q < 4; ++q) h256[4 * lane + q] = 0;
          wave_lds_sync();
#pragma unroll
          for (int m = 0; m < CAPL; ++m) {
            const uint32_t ik = ~(uint32_t)idx[m];
            if (64 * m + lane < n && (key[m] & rm) == rp && (ik & im) == ip) atomicAdd(&h256[(ik >> sh2) & 255u], 1u);
          }
          wave_lds_sync();
          uint32_t c[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) c[q] = h256[255 - 4 * lane - q];
          int bin;
          uint32_t above, cnt;
          find_bin(c, lane, need2, bin, above, cnt);
          ip |= (uint32_t)bin << sh2;
          im |= 0xffu << sh2;
          need2 -= above;
          wave_lds_sync();
          if (cnt == need2) break;
        }
      }
      // selected: key > rp (rp's low bits are zero when the loop stopped early), or
      // key == rp and ~index >= ip, i.e. index <= ~ip
      if (lane == rr) {
        thv = threshold_of_key(rp);
        cutv = neq > rneed ? (int)~ip : 0x7fffffff;
      }
    }
    if (lane < 16) {
      const int qr = r0 + 16 * w + lane;
      if (qr < Tq) {
        const long rowg = srowb + 16 * w + lane;
        const int nv = a.causal ? max(0, min(Tk, qr + a.q_offset + 1)) : Tk;
        a.thr[rowg] = make_uint2(__float_as_uint(thv), (uint32_t)cutv);
        if (a.counts) a.counts[rowg] = min(topk, nv);
        if (a.split) a.split[rowg] = 0;
        a.top2[2 * rowg] = t2.x;
        a.top2[2 * rowg + 1] = t2.y;
      }
    }
    return;
  } else {

  // ---- pass B: wave w takes rows r0 + 16w + 4lg + e against the K tile in LDS --
  // (every score of a row is then in one wave, which keeps the emission, the
  // flush and the top-2 wave-private).  A operand: the wave's row group of qf.
  bf16x8 qa[4] = {qf[0][0], qf[0][1], qf[0][2], qf[0][3]};
#pragma unroll
  for (int g = 1; g < 4; ++g) {
#pragma unroll
    for (int s = 0; s < 4; ++s) qa[s] = g == w ? qf[g][s] : qa[s];
  }
  float th0e[4], th1[4], m1[4], m2[4];
  int nv4[4];
  bool live4[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int rr = 4 * lg + e, qr = r0 + 16 * w + rr;
    live4[e] = qr < Tq;
    int nv = Tk;
    if (a.causal) nv = min(Tk, qr + a.q_offset + 1);
    if (nv < 0) nv = 0;
    nv4[e] = live4[e] ? nv : 0;
    th0e[e] = live4[e] ? rinfo[w][rr].th0 : INFINITY;   // dead rows take nothing
    th1[e] = rinfo[w][rr].th1;
    m1[e] = -FLT_MAX; m2[e] = -FLT_MAX;
  }
  uint4 pf[4];   // the next tile: 64 keys x 16 vectors of 16 B over 256 threads
  auto issue = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + 256 * i, r = e >> 4, cv = e & 15, j = kt * KT + r;
      pf[i] = make_uint4(0, 0, 0, 0);
      if (j < Tk) pf[i] = *reinterpret_cast<const uint4*>(kb + ((long)(b * Tk + j) * H + h) * DP + cv * 8);
    }
  };
  auto sweepB = [&](auto&& fn) __attribute__((always_inline)) {
    issue(0);
    for (int kt = 0; kt < ntile; ++kt) {
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = tid + 256 * i;
        *reinterpret_cast<uint4*>(ks + (e >> 4) * PB + (e & 15) * 8) = pf[i];
      }
      __syncthreads();
      if (kt + 1 < ntile) issue(kt + 1);
      f4 acc[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        f4 c = f4_zero();
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const uint4 raw = *reinterpret_cast<const uint4*>(&ks[(16 * nt + lr) * PB + 32 * s + 8 * lg]);
          c = mma_bf16(qa[s], __builtin_bit_cast(bf16x8, raw), c);
        }
        acc[nt] = score_of(c, mscale);
      }
      fn(kt, acc);
    }
  };
  const int tlcap = 16 * (topk + TOPK_CAP);
  const long lreg = ((long)bh * nqb + qb) * 4 + w;
  uint2* tl = a.tl_list + lreg * tlcap;
  int32_t* toff = a.tl_off + lreg * (a.tl_ntmax + 1);
  const long srow0 = (long)bh * Tq + r0 + 16 * w;    // global row of the wave's row 0
  uint2* scratch = a.scratch;
  // A tile's candidates are gathered in LDS -- the wave's 16 histogram rows hold
  // 16 rows x 64 keys -- and written with full-wave stores.  Bit 31 of a
  // buffered entry marks a threshold-bin candidate; the flush also gives it a
  // slot in its row's scratch list (an LDS counter per row), so the slot order
  // within a row is arbitrary and the resolve breaks ties by list position.
  static_assert(16 * HW >= 2 * 16 * KT, "a tile's candidates must fit the wave's histogram rows");
  uint2* ebuf = reinterpret_cast<uint2*>(&hist[16 * w][0]);
  const uint32_t rk0 = ((uint32_t)(4 * lg) << 8) | (uint32_t)lr;
  int woff = 0, tcnt = 0;
  auto emit_buf = [&](int e, int nt, float sc, bool cand) __attribute__((always_inline)) {
    const uint64_t cb = ballot64(cand);
    if (cand)
      ebuf[(uint32_t)tcnt + lane_rank(cb)] =
          make_uint2(__float_as_uint(sc), rk0 + (uint32_t)((e << 8) + 16 * nt) + (sc < th1[e] ? 0x80000000u : 0u));
    tcnt = __builtin_amdgcn_readfirstlane(tcnt + __popcll(cb));
  };
  auto top2_fast = [&](int e, float x) __attribute__((always_inline)) {
    m2[e] = __builtin_amdgcn_fmed3f(m1[e], m2[e], x);
    m1[e] = fmaxf(m1[e], x);
  };
  sweepB([&](int kt, f4* acc) __attribute__((always_inline)) {
    // A row holds at most top_k + TOPK_CAP candidates, so the list cannot fill
    // up; the bound only keeps one tile's writes inside the region whatever the inputs.
    woff = min(woff, tlcap - 16 * KT);
    if (lane == 0) toff[kt] = woff;
    tcnt = 0;
    if ((kt + 1) * KT <= minvalid) {
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float sc = acc[nt][e];
          emit_buf(e, nt, sc, sc >= th0e[e]);
          top2_fast(e, sc);
        }
      }
    } else {
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int j = kt * KT + 16 * nt + lr;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float sc = acc[nt][e];
          emit_buf(e, nt, sc, sc >= th0e[e] && j < nv4[e]);
          top2_fast(e, live4[e] && j < nv4[e] ? sc : -FLT_MAX);
        }
      }
    }
    // flush, two chunks of 64 per step (LDS accesses of one wave complete in order)
    auto flush_one = [&](bool ok, uint2 ent, int c) __attribute__((always_inline)) {
      const bool col = ok && (ent.y >> 31) != 0u;
      ent.y &= 0x7fffffffu;
      const uint32_t pos = (uint32_t)(woff + c + lane);
      if (ok) tl[pos] = ent;
      if (col) {
        const int r = (int)(ent.y >> 8);   // row in wave
        const int slot = (int)atomicAdd((uint32_t*)&colcnt[w][r], 1u);
        if (slot < TOPK_CAP) scratch[(srow0 + r) * TOPK_CAP + slot] = make_uint2(ent.x, pos);
      }
    };
    for (int c0 = 0; c0 < tcnt; c0 += 128) {
      const bool ok0 = c0 + lane < tcnt, ok1 = c0 + 64 + lane < tcnt;
      const uint2 e0 = ok0 ? ebuf[c0 + lane] : make_uint2(0u, 0u);
      const uint2 e1 = ok1 ? ebuf[c0 + 64 + lane] : make_uint2(0u, 0u);
      flush_one(ok0, e0, c0);
      flush_one(ok1, e1, c0 + 64);
    }
    woff = __builtin_amdgcn_readfirstlane(woff + tcnt);
  });
  if (lane == 0) toff[ntile] = woff;

  // ---- resolve the collected rows of the wave ----------------------------------
  uint32_t* h256 = &hist[16 * w][0];   // 256 words of the wave's histogram rows
  for (int rr = 0; rr < 16; ++rr) {
    const RowInfo ri = rinfo[w][rr];
    if (ri.mode != COLLECT) continue;
    const long row = srow0 + rr;
    const int n = min(colcnt[w][rr], TOPK_CAP);
    uint32_t key[CAPL];
    int idx[CAPL];
#pragma unroll
    for (int m = 0; m < CAPL; ++m) {
      const int p = 64 * m + lane;
      key[m] = 0; idx[m] = 0;
      if (p < n) {
        const uint2 v = scratch[row * TOPK_CAP + p];
        key[m] = f32_order_key(__uint_as_float(v.x));
        idx[m] = (int)v.y;
      }
    }
    // every collected key lies in [key(th0), key(th1) - 1]: the bytes those two
    // share are the same for all of them and need no pass
    const uint32_t klo = f32_order_key(ri.th0), dif = klo ^ (f32_order_key(ri.th1) - 1u);
    uint32_t rm = 0;
    int sh = 24;
    while (sh > 0 && (dif >> sh) == 0u) { rm |= 0xffu << sh; sh -= 8; }
    uint32_t rp = klo & rm;
    uint32_t rneed = (uint32_t)ri.need;
    for (; sh >= 0; sh -= 8) {
#pragma unroll
      for (int q = 0; q < 4; ++q) h256[4 * lane + q] = 0;
      wave_lds_sync();
#pragma unroll
      for (int m = 0; m < CAPL; ++m) {
        if (64 * m + lane < n && (key[m] & rm) == rp) atomicAdd(&h256[(key[m] >> sh) & 255u], 1u);
      }
      wave_lds_sync();
      uint32_t c[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) c[q] = h256[255 - 4 * lane - q];
      int bin;
      uint32_t above, cnt;
      find_bin(c, lane, rneed, bin, above, cnt);
      rp |= (uint32_t)bin << sh;
      rm |= 0xffu << sh;
      rneed -= above;
      wave_lds_sync();
      if (cnt == rneed) break;
    }
    // equal keys at the threshold: the rneed with the smallest list position
    // (positions grow with the key index within a row)
    uint32_t neq = 0;
#pragma unroll
    for (int m = 0; m < CAPL; ++m) neq += (uint32_t)__popcll(ballot64(64 * m + lane < n && (key[m] & rm) == rp));
    uint32_t ip = 0, im = 0;
    if (neq > rneed) {
      uint32_t need2 = rneed;
      for (int sh = 24; sh >= 0; sh -= 8) {
#pragma unroll
        for (int q = 0; q < 4; ++q) h256[4 * lane + q] = 0;
        wave_lds_sync();
#pragma unroll
        for (int m = 0; m < CAPL; ++m) {
          const uint32_t ik = ~(uint32_t)idx[m];
          if (64 * m + lane < n && (key[m] & rm) == rp && (ik & im) == ip) atomicAdd(&h256[(ik >> sh) & 255u], 1u);
        }
        wave_lds_sync();
        uint32_t c[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) c[q] = h256[255 - 4 * lane - q];
        int bin;
        uint32_t above, cnt;
        find_bin(c, lane, need2, bin, above, cnt);
        ip |= (uint32_t)bin << sh;
        im |= 0xffu << sh;
        need2 -= above;
        wave_lds_sync();
        if (cnt == need2) break;
      }
    }
#pragma unroll
    for (int m = 0; m < CAPL; ++m) {
      const bool valid = 64 * m + lane < n;
      const uint32_t km = key[m] & rm;
      const bool eq = valid && km == rp;
      const bool sel = valid && (km > rp || (eq && (neq <= rneed || ((~(uint32_t)idx[m]) & im) >= ip)));
      if (valid && !sel && idx[m] >= 0 && idx[m] < tlcap) tl[idx[m]].x = 0xff800000u;   // -inf: weight 0
    }
  }

  // ---- top-2 over the row's 16 lanes, counts -----------------------------------
#pragma unroll
  for (int e = 0; e < 4; ++e) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const float b1 = __shfl_xor(m1[e], o, 64), b2 = __shfl_xor(m2[e], o, 64);
      const float hi = fmaxf(m1[e], b1), lo = fmaxf(fminf(m1[e], b1), fmaxf(m2[e], b2));
      m1[e] = hi; m2[e] = lo;
    }
    if (lr == 0 && live4[e]) {
      const long rowg = srow0 + 4 * lg + e;
      if (a.counts) a.counts[rowg] = min(topk, nv4[e]);
      if (a.split) a.split[rowg] = 0;
      a.top2[2 * rowg] = m1[e];
      a.top2[2 * rowg + 1] = m2[e];
    }
  }
  }   // !THR
}

// The largest float below x (x not -inf or NaN): s < x  <=>  s <= next_down(x)
// for every score s that is not NaN.
__device__ __forceinline__ float next_down(float x) {
  const uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) == 0u) return __uint_as_float(0x80000001u);   // below +-0: -min denormal
  return __uint_as_float((int32_t)u > 0 ? u - 1u : u + 1u);
}

// The score of one raw accumulator, as score_of computes it.
__device__ __forceinline__ float score1(float acc, float mscale) {
#pragma clang fp contract(off)
  return acc * mscale + 0.0f;
}

// For mscale > 0, score1 is non-decreasing in the accumulator, and several
// accumulators can round to one score.  acc_lo_of(a): the smallest x with
// score1(x) == score1(a); acc_hi_of(a): the largest.  Bisection over the
// order-preserving keys between -inf and +inf; a is not NaN.
__device__ __forceinline__ float acc_lo_of(float a, float mscale) {
  const float S = score1(a, mscale);
  if (S == -INFINITY) return -INFINITY;
  uint32_t lo = 0x007fffffu, hi = f32_order_key(a);   // score1(key -inf) < S <= score1(key hi)
  while (hi - lo > 1u) {
    const uint32_t mid = lo + ((hi - lo) >> 1);
    if (score1(key_to_f32(mid), mscale) >= S) hi = mid;
    else lo = mid;
  }
  return key_to_f32(hi);
}
__device__ __forceinline__ float acc_hi_of(float a, float mscale) {
  const float S = score1(a, mscale);
  if (S == INFINITY) return INFINITY;
  uint32_t lo = f32_order_key(a), hi = 0xff800000u;   // score1(key lo) <= S < score1(key +inf)
  while (hi - lo > 1u) {
    const uint32_t mid = lo + ((hi - lo) >> 1);
    if (score1(key_to_f32(mid), mscale) <= S) lo = mid;
    else hi = mid;
  }
  return key_to_f32(lo);
}

// ---------------------------------------------------------------------------
// K1, threshold form at 128 query rows per block (the layer path: bf16,
// D = 128, counts that fit 16 bits).
//
// The selection of score_topk_tiles_kernel<true, THR = true> with twice the
// rows per K tile.  Wave w owns keys [16w, 16w+16) of every 64-key tile for all
// 128 rows of the block: its 16 keys are the MFMA A operand, loaded straight
// into registers one tile ahead, and the block's q rows are the B operand,
// resident in registers as 8 groups of 16 rows.  Both sweeps are bound by the
// K bytes delivered into the CU, which this halves per score; the histogram
// adds per score stay the same.  The operands of every product are those of the
// 64-row kernel (A row rho holds key rho/4 + 4 (rho%4) of the wave's 16, the
// same 32 dims per instruction), so the fp32 scores are identical.  Lane
// (w, lg, lr) holds rows 16g + lr (g = 0..7) against keys kt*64 + 16w + lg + 4i.
// Wave w does the per-row work (b*, thresholds, resolve, output) for row
// groups w and w + 4.  A block with a row whose threshold bin overflows flags
// both of its 64-row halves for the radix fallback launch of
// score_topk_kernel<..., FB, LIST, THR>, which writes the same outputs.
// ---------------------------------------------------------------------------
// MASKED: rows carry a valid prefix and slot count (a.row_nv / a.row_kq, keys
// compacted valid-first); the unmasked instantiation computes the causal range.
template <bool MASKED>
__global__ __launch_bounds__(256, 2) void score_thr128_kernel(TopkArgs a, int nqb, float mscale) {
  constexpr int QR = 128;
  constexpr int NG = QR / 16;
  constexpr int CAPL = TOPK_CAP / 64;
  // Row histograms, 16-bit counters: rows 16g + r and 16(g + 4) + r (g < 4)
  // share the words of pair 16g + r, bin b in word b, the first row in the low
  // half.  64 KB; between the sweeps the same memory holds other per-block data.
  __shared__ __align__(16) uint32_t hist[QR / 2][NBIN];
  __shared__ RowInfo rinfo[NG][16];
  __shared__ int colcnt[NG][16];
  __shared__ float qnorm[NG][16];
  __shared__ float ra0[NG][16];   // lower edge a0 of b* (accumulator domain)
  __shared__ int rcntb[NG][16];   // keys in b*
  __shared__ int force_fb;        // a row's 16-bit bin counter could overflow: radix fallback
  __shared__ float2 smap[NG][16]; // the sample histogram's map (iws, bcs) per row
  __shared__ int rnv[MASKED ? NG : 1][16];   // MASKED: valid keys per row (0 past Tq)

  const int BH = a.B * a.H;
  const int nqr = (a.Tq + QR - 1) / QR;
  const int bid = blockIdx.x;
  const int bh = bid % BH;
  const int qb = nqr - 1 - bid / BH;   // heaviest (latest) row blocks first
  const int b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int r0 = qb * QR;
  const int Tq = a.Tq, Tk = a.Tk, H = a.H;
  const uint16_t* kb = reinterpret_cast<const uint16_t*>(a.k);
  const int topk = a.top_k;
  // valid keys of query row qr < Tq: the causal (or full) range, or with a padding mask
  // (row_nv, keys compacted valid-first) the row's valid prefix; and its slots
  auto nv_row = [&](int qr) __attribute__((always_inline)) {
    if constexpr (MASKED) return a.row_nv[(long)b * Tq + qr];
    return a.causal ? max(0, min(Tk, qr + a.q_offset + 1)) : Tk;
  };
  auto kq_row = [&](int qr) __attribute__((always_inline)) {
    if constexpr (MASKED) return a.row_kq != nullptr ? min(topk, a.row_kq[qr]) : topk;
    return topk;
  };
  // valid keys of row r0 + 16g + lr (0 for rows past Tq); the masked rows' counts
  // come from LDS in the sweeps (rnv, written below and visible after the row set-up)
  auto nv_direct = [&](int g) __attribute__((always_inline)) {
    const int qr = r0 + 16 * g + lr;
    return qr < Tq ? nv_row(qr) : 0;
  };
  auto nv_of = [&](int g) __attribute__((always_inline)) {
    if constexpr (MASKED) return rnv[g][lr];
    return nv_direct(g);
  };
  if constexpr (MASKED) {
    if (tid < QR) {
      const int qr = r0 + tid;
      rnv[tid >> 4][tid & 15] = qr < Tq ? nv_row(qr) : 0;
    }
  }

  // B operand: q^T of the block's rows; lane holds row r0 + 16g + lr, dims 32s + 8lg + [0, 8).
  // All loads first, the norms after.  Rows past Tq load row 0 of the head: their
  // scores, bins and norms are never used (no output, no histogram or candidate
  // that anyone reads, no sample range: nv = 0).
  bf16x8 qf[NG][4];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const int qr = r0 + 16 * g + lr;
    const uint16_t* qp = reinterpret_cast<const uint16_t*>(a.q) + ((long)(b * Tq + (qr < Tq ? qr : 0)) * H + h) * DP;
#pragma unroll
    for (int s = 0; s < 4; ++s) qf[g][s] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8*>(qp + 32 * s + 8 * lg));
  }
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    float qn2 = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u16x8 raw = __builtin_bit_cast(u16x8, qf[g][s]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float x = bf16_to_f32(raw[j]);
        qn2 = fmaf(x, x, qn2);
      }
    }
    qn2 += __shfl_xor(qn2, 16, 64);
    qn2 += __shfl_xor(qn2, 32, 64);
    if ((g & 3) == w && lg == 0) qnorm[g][lr] = sqrtf(qn2);
  }

  // keys below minvalid are valid for every live row of the block
  int minvalid = 0x7fffffff;
#pragma unroll
  for (int g = 0; g < NG; ++g)
    if (r0 + 16 * g + lr < Tq) minvalid = min(minvalid, nv_direct(g));
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) minvalid = min(minvalid, __shfl_xor(minvalid, o, 64));
  minvalid = __builtin_amdgcn_readfirstlane(minvalid);   // block-uniform: tile tests branch on the scalar unit
  int kend = Tk;
  if (a.causal) kend = min(Tk, min(Tq, r0 + QR) - 1 + a.q_offset + 1);
  const int ntile = kend > 0 ? (kend + KT - 1) / KT : 0;

  // A operand: the wave's 16 keys of a tile; MFMA row lr holds key lr/4 + 4 (lr%4).
  // Keys past Tk load key 0 instead: their scores are finite and never used (a
  // tile with such keys is past minvalid, where every use checks j < nv <= Tk),
  // and no select on the loaded data keeps the compiler from waiting for the
  // prefetch right after issuing it.
  const int krow = (lr >> 2) + 4 * (lr & 3);
  bf16x8 kf[1][4];   // the next tile's fragments, loaded while the current one is processed
  auto kload = [&](bf16x8 (&dst)[4], int kt) __attribute__((always_inline)) {
    const int j = kt * KT + 16 * w + krow;
    const uint16_t* p = kb + ((long)(b * Tk + (j < Tk ? j : 0)) * H + h) * DP + 8 * lg;
#pragma unroll
    for (int s = 0; s < 4; ++s) dst[s] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8*>(p + 32 * s));
  };
  // fn(kt, g0, acc): acc[gg][i] = the raw accumulator of row r0 + 16 (g0 + gg) + lr
  // against key kt*64 + 16w + lg + 4i, for the row groups g0 = 0 and then g0 = 4
  // of tile kt; its score is score1(acc, mscale), non-decreasing in acc (mscale >
  // 0), so both sweeps bin and test accumulators.  Half the groups at a time keeps
  // 16 accumulator VGPRs live instead of 32.
  // fn's last argument is std::true_type in tiles whose keys are valid for every
  // row of the wave (kt < minvalid / 64: no per-key tests), std::false_type
  // otherwise; the test is made once per tile, so a full tile is straight-line code.
  auto tile = [&](bf16x8 (&kfc)[4], int kt, auto&& fn) __attribute__((always_inline)) {
    auto body = [&](auto full) __attribute__((always_inline)) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        f4 acc[NG / 2];
#pragma unroll
        for (int gg = 0; gg < NG / 2; ++gg) {
          f4 c = f4_zero();
#pragma unroll
          for (int s = 0; s < 4; ++s) c = mma_bf16(kfc[s], qf[NG / 2 * hh + gg][s], c);
          acc[gg] = c;
        }
        // unconditional (the last tile reloads tile ntile - 1): with a conditional
        // load the compiler waits for every load in flight at the top of a tile
        if (hh == 1) kload(kfc, min(kt + 1, ntile - 1));
        fn(kt, NG / 2 * hh, acc, full);
      }
    };
    if ((kt + 1) * KT <= minvalid) body(std::true_type{});
    else body(std::false_type{});
  };
  auto sweep = [&](auto&& fn) __attribute__((always_inline)) {
    if (ntile > 0) kload(kf[0], 0);
    for (int kt = 0; kt < ntile; ++kt) tile(kf[0], kt, fn);
  };

  // row set-up (wave w: rows of groups w and w + 4; lane < 32 -> group w + 4 (lane / 16), row lane % 16)
  __syncthreads();   // qnorm visible
  float kmx2 = lane < KNCH ? a.kmax[(long)bh * KNCH + lane] : 0.f;
  const float kmx = sqrtf(wave_max(kmx2));
  if (lane < 32) {
    const int g = w + 4 * (lane >> 4), rr = lane & 15;
    const int qr = r0 + 16 * g + rr;
    const int nv = qr < Tq ? nv_row(qr) : 0;
    const int kr = qr < Tq ? kq_row(qr) : topk;
    RowInfo ri;
    const float bound = qnorm[g][rr] * kmx * 1.001f;   // of |acc|
    ri.iw = (bound > 0.f && bound < FLT_MAX) ? 128.0f / bound : 0.f;
    ri.bc = BIN_C0;
    ri.bstar = -1;
    ri.need = min(kr, nv);
    ri.mode = (nv <= kr) ? SELECT_ALL : BIN_ALL;
    ri.pfx = 0; ri.msk = 0; ri.done = 1; ri.th0 = -INFINITY; ri.th1 = -INFINITY;
    rinfo[g][rr] = ri;
    colcnt[g][rr] = 0;
  }
  if (tid == 0) force_fb = 0;
  __syncthreads();

  // ---- the bins' range from a sample -------------------------------------------
  // The bins are a monotone map of the accumulator (so of the score); any monotone
  // map keeps the selection exact, and a row the map misjudges (a bin with more
  // than TOPK_CAP keys) goes to the radix fallback like any other.  The bound above
  // spans the Cauchy-Schwarz range, several times what the scores fill, so the
  // threshold bin would hold several times the keys it needs to.  Instead each
  // row's accumulators over 8 tiles spread across its sweep (about 512 keys) fit
  // the bins in two steps:
  //  1. min l and max h: bins over [l, h] widened by a quarter of h - l on each
  //     side, used where finer than the bound's;
  //  2. where the sample is outlying (its span above 9 standard deviations, as a
  //     heavy tail of keys makes it), a 256-bin histogram of the same sample over
  //     [l, h] gives approximate order statistics: the bins then span [x16 - (u - x16) / 4, u], where x16 is the
  //     16th smallest sampled accumulator and u = 2 x(r/2) - x(2r), x(i) the i-th
  //     largest and r = n k / nv the expected rank of the row's cut among the n
  //     sampled keys (bin edges taken on the safe side).  A few far-out keys (a
  //     heavy tail) then no longer stretch the bins: the keys above u share the top
  //     bin, the rare ones below the lower end the bottom bin, and the cut lies
  //     below u except with a small probability.
  // 16-bit counters: a row's bin count stays below 65536 while it has at most 65535
  // keys, and also with 65536 keys once two of them are known to fall in different
  // bins -- the sample's lowest and highest accumulators, checked under the final
  // map.  A row of 65536 keys without such a pair sends its block to the radix
  // fallback, whose counters are 32-bit.
  {
    constexpr int NS = 8;
    float lo[NG], hi[NG], sm[NG], sq[NG];   // min, max, sum and sum of squares of the sampled accumulators
    int cn[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) { lo[g] = FLT_MAX; hi[g] = -FLT_MAX; sm[g] = 0.f; sq[g] = 0.f; cn[g] = 0; }
    const int ns = min(ntile, NS);
    auto sample_kt = [&](int t) __attribute__((always_inline)) { return (int)(((long)min(t, ns - 1) * ntile) / ns); };
    {
      // sample tile t's fragments in ks[t & 1], the next one's loaded meanwhile
      bf16x8 ks[2][4];
      if (ns > 0) kload(ks[0], sample_kt(0));
#pragma unroll
      for (int t = 0; t < NS; ++t) {
        if (t >= ns) break;   // uniform
        const int kt = sample_kt(t);
        kload(ks[(t + 1) & 1], sample_kt(t + 1));
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          f4 c = f4_zero();
#pragma unroll
          for (int s = 0; s < 4; ++s) c = mma_bf16(ks[t & 1][s], qf[g][s], c);
          const int nv = nv_of(g);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const bool ok = kt * KT + 16 * w + lg + 4 * i < nv;
            const float x = ok ? c[i] : 0.f;
            lo[g] = fminf(lo[g], ok ? c[i] : FLT_MAX);
            hi[g] = fmaxf(hi[g], ok ? c[i] : -FLT_MAX);
            sm[g] += x;
            sq[g] = fmaf(x, x, sq[g]);
            cn[g] += ok ? 1 : 0;
          }
        }
      }
    }
    // the fitted bins' sample pass: fn(g, kt, c) for the accumulators c of row group g
    // against sample tile kt.  A rolled loop, one tile at a time: it runs only in
    // blocks with an outlying sample, and unrolled copies would crowd the registers
    // of the sweeps.
    auto sample = [&](auto&& fn) __attribute__((always_inline)) {
#pragma unroll 1
      for (int t = 0; t < ns; ++t) {
        const int kt = sample_kt(t);
        bf16x8 ks[4];
        kload(ks, kt);
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          f4 c = f4_zero();
#pragma unroll
          for (int s = 0; s < 4; ++s) c = mma_bf16(ks[s], qf[g][s], c);
          fn(g, kt, c);
        }
      }
    };
#pragma unroll
    for (int g = 0; g < NG; ++g) {
#pragma unroll
      for (int o = 16; o < 64; o <<= 1) {
        lo[g] = fminf(lo[g], __shfl_xor(lo[g], o, 64));
        hi[g] = fmaxf(hi[g], __shfl_xor(hi[g], o, 64));
        sm[g] += __shfl_xor(sm[g], o, 64);
        sq[g] += __shfl_xor(sq[g], o, 64);
        cn[g] += __shfl_xor(cn[g], o, 64);
      }
    }
    float4* rg = reinterpret_cast<float4*>(&hist[0][0]);   // [wave][128 rows][2]
    if (lg == 0) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        rg[2 * (QR * w + 16 * g + lr)] = make_float4(lo[g], hi[g], (float)cn[g], 0.f);
        rg[2 * (QR * w + 16 * g + lr) + 1] = make_float4(sm[g], sq[g], 0.f, 0.f);
      }
    }
    __syncthreads();
    // step 1, and the sample histogram's map (iws, bcs: bin 0 at l, bin 255 at h)
    if (lane < 32) {
      const int g = w + 4 * (lane >> 4), r = lane & 15;
      float l = FLT_MAX, h = -FLT_MAX, n = 0.f, s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float4 o = rg[2 * (QR * v + 16 * g + r)], p = rg[2 * (QR * v + 16 * g + r) + 1];
        l = fminf(l, o.x); h = fmaxf(h, o.y); n += o.z; s1 += p.x; s2 += p.y;
      }
      RowInfo ri = rinfo[g][r];
      const float sp = h - l;
      float iws = 0.f, bcs = 0.f;
      if (l < h && sp < FLT_MAX) {
        const float l2 = l - 0.25f * sp, iw2 = 255.0f / (1.5f * sp);
        const float bc2 = 8388608.0f - l2 * iw2;
        if (iw2 > ri.iw && iw2 < FLT_MAX && fabsf(bc2) < 1.0e30f) { ri.iw = iw2; ri.bc = bc2; }
        // an outlying sample (a span above 9 standard deviations: about 6.5 for 512
        // normal scores) gets the fitted bins of step 2
        const float mean = s1 / fmaxf(n, 1.f);
        const float var = fmaxf(s2 / fmaxf(n, 1.f) - mean * mean, 0.f);
        if (ri.mode != SELECT_ALL && n >= 64.f && sp * sp > 81.f * var) {
          iws = 255.0f / sp;
          bcs = 8388608.0f - l * iws;
          if (!(iws < FLT_MAX && fabsf(bcs) < 1.0e30f)) iws = 0.f;
        }
      }
      ri.th0 = h;   // l and h for the overflow check below (th0 and colcnt are reset there)
      rinfo[g][r] = ri;
      smap[g][r] = make_float2(iws, bcs);
      rcntb[g][r] = (int)n;
      colcnt[g][r] = __float_as_int(l);
    }
    __syncthreads();   // the range sums are read before hist is cleared
    for (int i = tid; i < QR / 2 * NBIN; i += 256) (&hist[0][0])[i] = 0;
    __syncthreads();
    // step 2: the sample's 256-bin histograms (rows with keys to select and a sample span)
    {
      const uint32_t hb = (uint32_t)lr * (NBIN * 4u) - 0x2c000000u;
      float iws[NG], bcs[NG];
      uint32_t smask = 0;
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const float2 m = smap[g][lr];
        iws[g] = m.x; bcs[g] = m.y;
        if (m.x > 0.f && rinfo[g][lr].mode != SELECT_ALL) smask |= 1u << g;
      }
      if (__syncthreads_or(smask != 0u)) {
        sample([&](int g, int kt, f4 c) __attribute__((always_inline)) {
          const int nv = nv_of(g);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (((smask >> g) & 1u) && kt * KT + 16 * w + lg + 4 * i < nv) {
              const uint32_t bits = score_bin_bits(c[i], iws[g], bcs[g]);
              atomicAdd(reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(&hist[0][0]) +
                                                    (hb + (bits << 2) + (uint32_t)(g & 3) * (16u * NBIN * 4u))),
                        g < 4 ? 1u : 0x10000u);
            }
          }
        });
        __syncthreads();
        // step 3: wave w fits the bins of its rows (groups w and w + 4) in turn
        for (int rr = 0; rr < 32; ++rr) {
          const int g = w + 4 * (rr >> 4), r = rr & 15;
          RowInfo ri = rinfo[g][r];
          const float2 m = smap[g][r];
          const int n = rcntb[g][r];
          if (!(m.x > 0.f)) continue;   // wave-uniform: no fit for this row
          const int nv = nv_row(r0 + 16 * g + r);
          const uint32_t* hr = hist[16 * (g & 3) + r];
          const uint32_t sh = 16u * (uint32_t)(g >> 2);
          uint32_t c[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) c[q] = (hr[255 - 4 * lane - q] >> sh) & 0xffffu;
          const float rexp = (float)n * (float)ri.need / (float)max(nv, 1);
          const int rA = min(n, max(1, (int)(0.5f * rexp)));
          const int rB = min(n, max(rA + 1, (int)(2.0f * rexp)));
          const int rL = max(1, n - 15);
          int bA, bB, bL;
          uint32_t ab, ct;
          find_bin(c, lane, (uint32_t)rA, bA, ab, ct);
          find_bin(c, lane, (uint32_t)rB, bB, ab, ct);
          find_bin(c, lane, (uint32_t)rL, bL, ab, ct);
          if (lane == 0) {
            const float l = __int_as_float(colcnt[g][r]);
            const float inv = 1.0f / m.x;
            const float a_hi = l + ((float)bA + 0.5f) * inv;   // >= x(rA)
            const float b_lo = l + ((float)bB - 0.5f) * inv;   // <= x(rB)
            const float x16 = l + ((float)bL - 0.5f) * inv;    // <= the 16th smallest
            const float up = a_hi + (a_hi - b_lo);
            const float low = x16 - 0.25f * (up - x16);
            if (up > low) {
              const float iw3 = 255.0f / (up - low);
              const float bc3 = 8388608.0f - low * iw3;
              if (iw3 > ri.iw && iw3 < FLT_MAX && fabsf(bc3) < 1.0e30f) {
                ri.iw = iw3;
                ri.bc = bc3;
                rinfo[g][r].iw = iw3;
                rinfo[g][r].bc = bc3;
              }
            }
          }
        }
      }
    }
    __syncthreads();
    // rows of 65536 keys: the sample's lowest and highest accumulators in different bins
    if (lane < 32) {
      const int g = w + 4 * (lane >> 4), r = lane & 15;
      const RowInfo ri = rinfo[g][r];
      const float l = __int_as_float(colcnt[g][r]), h = ri.th0;
      if (ri.mode != SELECT_ALL && nv_of(g) > 65535 &&
          !(l < h && score_bin_bits(l, ri.iw, ri.bc) != score_bin_bits(h, ri.iw, ri.bc)))
        force_fb = 1;
      rinfo[g][r].th0 = -INFINITY;
      colcnt[g][r] = 0;
    }
    __syncthreads();   // the sample's words are read before hist is cleared
  }
  for (int i = tid; i < QR / 2 * NBIN; i += 256) (&hist[0][0])[i] = 0;
  __syncthreads();

  // ---- pass A: block-shared row histograms and each row's top-2 ---------------
  float m1[NG], m2[NG];   // top-2 of row 16g + lr over this lane's keys, then over the row
#pragma unroll
  for (int g = 0; g < NG; ++g) { m1[g] = -FLT_MAX; m2[g] = -FLT_MAX; }
  {
    float iw[NG], bc[NG];
    uint32_t hmask = 0;   // bit g: row 16g + lr is live and needs a histogram
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const RowInfo ri = rinfo[g][lr];
      iw[g] = ri.iw;
      bc[g] = ri.bc;
      if (r0 + 16 * g + lr < Tq && ri.mode != SELECT_ALL) hmask |= 1u << g;
    }
    const bool any_hist = __syncthreads_or(hmask != 0u);
    // bits = 2^23 + bin as a float's bits (0x4b000000 + bin), so (bits << 2) mod 2^32
    // is 0x2c000000 + 4 bin: the byte offset of bin b of pair 16(g & 3) + lr is
    // hb + (bits << 2) + 16384 (g & 3), and the increment is a constant per g.
    const uint32_t hb = (uint32_t)lr * (NBIN * 4u) - 0x2c000000u;
    auto bump = [&](int g, uint32_t bits) __attribute__((always_inline)) {
      uint32_t* p = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(&hist[0][0]) +
                                                (hb + (bits << 2) + (uint32_t)(g & 3) * (16u * NBIN * 4u)));
      atomicAdd(p, g < 4 ? 1u : 0x10000u);
    };
    // The running max is med3(m1, x, FLT_MAX), one instruction (fmaxf, or med3
    // against +inf, which the compiler turns into fmaxf, canonicalises both
    // operands first: two more per score).  It equals max(m1, x) for every finite
    // accumulator; a q.k product that overflows to +inf is kept as FLT_MAX.
    auto top2 = [&](int g, float x) __attribute__((always_inline)) {
      m2[g] = __builtin_amdgcn_fmed3f(m1[g], m2[g], x);
      m1[g] = __builtin_amdgcn_fmed3f(m1[g], x, FLT_MAX);
    };
    // Every block has a live row: the sweep gives the top-2 even where no row
    // needs a histogram.  In full tiles every row's histogram takes the adds
    // (rows that need none -- past Tq, or taking all their keys -- own rows
    // nobody reads), so the adds need no branch, not even in blocks where no
    // row needs a histogram: a branch per score would split the tile into basic
    // blocks the compiler cannot interleave with the next MFMAs.
    sweep([&](int kt, int g0, f4* acc, auto full) __attribute__((always_inline)) {
      if constexpr (decltype(full)::value) {
#pragma unroll
        for (int gg = 0; gg < NG / 2; ++gg) {
          const int g = g0 + gg;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            top2(g, acc[gg][i]);
            bump(g, score_bin_bits(acc[gg][i], iw[g], bc[g]));
          }
        }
      } else {
#pragma unroll
        for (int gg = 0; gg < NG / 2; ++gg) {
          const int g = g0 + gg;
          const int nv = nv_of(g);   // 0 for rows past Tq
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int j = kt * KT + 16 * w + lg + 4 * i;
            top2(g, j < nv ? acc[gg][i] : -FLT_MAX);
            if (((hmask >> g) & 1u) && j < nv) bump(g, score_bin_bits(acc[gg][i], iw[g], bc[g]));
          }
        }
      }
    });
    // top-2 over the row's lanes of this wave (lg)
#pragma unroll
    for (int g = 0; g < NG; ++g) {
#pragma unroll
      for (int o = 16; o < 64; o <<= 1) {
        const float b1 = __shfl_xor(m1[g], o, 64), b2 = __shfl_xor(m2[g], o, 64);
        const float hi = fmaxf(m1[g], b1), lo = fmaxf(fminf(m1[g], b1), fmaxf(m2[g], b2));
        m1[g] = hi; m2[g] = lo;
      }
    }
    __syncthreads();
    if (any_hist) {
      for (int rr = 0; rr < 32; ++rr) {
        const int g = w + 4 * (rr >> 4), r = rr & 15;
        RowInfo ri = rinfo[g][r];
        if (ri.mode == SELECT_ALL) continue;
        const uint32_t* hr = hist[16 * (g & 3) + r];
        const uint32_t sh = 16u * (uint32_t)(g >> 2);
        uint32_t c[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) c[q] = (hr[255 - 4 * lane - q] >> sh) & 0xffffu;
        int bin;
        uint32_t above, cnt;
        find_bin(c, lane, (uint32_t)ri.need, bin, above, cnt);
        if (lane == 0) {
          ri.bstar = bin;
          rcntb[g][r] = (int)cnt;
          ri.need -= (int)above;
          if (cnt == (uint32_t)ri.need) ri.mode = BIN_ALL;
          else if (cnt <= (uint32_t)TOPK_CAP) ri.mode = COLLECT;
          else ri.mode = RADIX;
          rinfo[g][r] = ri;
        }
      }
    }
    __syncthreads();
    int overflow = force_fb;
    if (lane < 32) overflow |= rinfo[w + 4 * (lane >> 4)][lane & 15].mode == RADIX;
    overflow = __syncthreads_or(overflow);
    if (tid < 2) {   // both 64-row halves, as the fallback launch indexes its blocks
      const int q64 = 2 * qb + tid;
      if (q64 < nqb) a.flags[(long)(nqb - 1 - q64) * BH + bh] = overflow;
    }
    if (overflow) return;   // block-uniform; the fallback launch redoes both halves
  }

  // top-2 over the waves, through LDS (the histograms are no longer needed)
  float2* t2s = reinterpret_cast<float2*>(&hist[0][0]);   // [wave][128 rows]
  if (lg == 0) {
#pragma unroll
    for (int g = 0; g < NG; ++g) t2s[QR * w + 16 * g + lr] = make_float2(m1[g], m2[g]);
  }
  __syncthreads();
  float2 t2 = make_float2(-FLT_MAX, -FLT_MAX);   // lane < 32: row 16 (w + 4 (lane / 16)) + lane % 16 (accumulators)
  if (lane < 32) {
    const int row = 16 * (w + 4 * (lane >> 4)) + (lane & 15);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float2 o = t2s[QR * v + row];
      const float hi = fmaxf(t2.x, o.x), lo = fmaxf(fminf(t2.x, o.x), fmaxf(t2.y, o.y));
      t2.x = hi; t2.y = lo;
    }
  }

  // ---- thresholds for pass B ---------------------------------------------------
  // b* spans accumulators [a0, a1).  Accumulators that round to one score can
  // straddle a0 or a1; the selection is by score with ties to the lowest index,
  // so a tie at the cut may involve keys on both sides of a bin edge.  The
  // collection window [th0, th1] therefore reaches out to every accumulator
  // whose score equals that of a0 or of the largest accumulator below a1.  Keys
  // above th1 are all selected, keys below th0 none; the resolve takes
  // need - cntb + (collected keys at or above a0) of the collected ones, which
  // counts the keys above b* that the window takes in.  A BIN_ALL row takes
  // everything from a0 up unless a tie straddles a0: then it collects just the
  // accumulators of a0's score.
  int any_collect = 0;
  if (lane < 32) {
    const int g = w + 4 * (lane >> 4), r = lane & 15;
    RowInfo ri = rinfo[g][r];
    float t0 = -INFINITY, t1 = -INFINITY;
    if (ri.mode != SELECT_ALL) {
      const float lo_b = ri.bstar > 0 ? bin_lower_edge(ri.bstar, ri.iw, ri.bc) : -INFINITY;
      const float lo_w = acc_lo_of(lo_b, mscale);
      ra0[g][r] = lo_b;
      if (ri.mode == BIN_ALL) {
        if (lo_w == lo_b) { t0 = lo_b; t1 = lo_b; }   // no tie below a0: s >= score1(a0) selects
        else { ri.mode = COLLECT; t0 = lo_w; t1 = acc_hi_of(lo_b, mscale); }
      } else {   // COLLECT
        t0 = lo_w;
        t1 = ri.bstar < NBIN - 1 ? acc_hi_of(next_down(bin_lower_edge(ri.bstar + 1, ri.iw, ri.bc)), mscale)
                                 : INFINITY;
      }
    }
    ri.th0 = t0; ri.th1 = t1;
    rinfo[g][r] = ri;
    any_collect = ri.mode == COLLECT;
  }
  // ---- pass B: threshold-bin candidates (blocks with a row to collect) -----------
  uint2* scratch = a.scratch;
  const long srowb = (long)bh * Tq + r0;   // global row of the block's row 0
  bool full_col = false;   // pass B: a candidate found no room in its lane's staging column
  if (__syncthreads_or(any_collect)) {
    // candidate of row 16g + lr: th0 <= acc <= th1, i.e. med3(acc, th0, th1) == acc;
    // rows that collect nothing take +inf, +inf, which no finite accumulator matches
    float tlo[NG], thi[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const RowInfo ri = rinfo[g][lr];
      const bool col = r0 + 16 * g + lr < Tq && ri.mode == COLLECT;
      tlo[g] = col ? ri.th0 : INFINITY;
      thi[g] = col ? ri.th1 : INFINITY;
    }
    // Candidates are staged in LDS, each lane in a column of its own (entry r of
    // lane l at 64 r + l, 32 entries: the histogram area is free, 32 of its
    // rows per wave), and flushed -- each takes a slot in its row's scratch list
    // through an LDS atomic and is stored, four entries per lane at a time --
    // after a tile that leaves some lane of the wave holding 16 or more, and
    // after the sweep.  (Flushing every tile put the stores ahead of the next
    // tile's K loads in the memory counter the loads are waited on.)  A tile
    // starts with at most 15 entries per lane; a lane that reaches 32 (17 or more
    // of its 32 scores of one tile in the window) sends the block to the radix
    // fallback, like an overflowing bin.  Entry: {accumulator
    // bits, g << 16 | key}: the row is 16g + lr of the lane that staged and flushes
    // it; keys fit 16 bits (Tk <= 65536 on this path).
    uint2* ebuf = reinterpret_cast<uint2*>(&hist[0][0] + 4096 * w);
    uint32_t* rowcnt = reinterpret_cast<uint32_t*>(&colcnt[0][0]);   // row 16g + lr at 16g + lr
    uint32_t kc = 0;   // this lane's staged entries
    auto flush = [&]() __attribute__((always_inline)) {
      wave_lds_sync();   // this wave's buffer writes before its reads
      for (uint32_t r0e = 0; ballot64(r0e < kc) != 0ull; r0e += 4) {
        uint2 e[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (r0e + u < kc) e[u] = ebuf[64 * (r0e + u) + lane];
        uint32_t slot[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (r0e + u < kc) slot[u] = atomicAdd(rowcnt + 16 * (e[u].y >> 16) + lr, 1u);
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (r0e + u < kc && slot[u] < (uint32_t)TOPK_CAP && r0 + 16 * (int)(e[u].y >> 16) + lr < Tq)
            scratch[(srowb + 16 * (e[u].y >> 16) + lr) * TOPK_CAP + slot[u]] = make_uint2(e[u].x, e[u].y & 0xffffu);
      }
      wave_lds_sync();   // reads done before the buffer is written again
      kc = 0;
    };
    sweep([&](int kt, int g0, f4* acc, auto full) __attribute__((always_inline)) {
      // Where any lane of the wave has a candidate, every lane writes its entry
      // at its next position, min(kc, 31), and only candidates keep theirs
      // (advance kc): the others are overwritten or lie past kc.  kc >= 32 after
      // the tile means an entry was lost (position 31 written again).
      auto stage = [&](bool cand, int g, float sc, int j) __attribute__((always_inline)) {
        if (ballot64(cand) != 0ull) {
          ebuf[64 * min(kc, 31u) + lane] = make_uint2(__float_as_uint(sc), ((uint32_t)g << 16) | (uint32_t)j);
          kc += cand ? 1u : 0u;
        }
      };
      if constexpr (decltype(full)::value) {
#pragma unroll
        for (int gg = 0; gg < NG / 2; ++gg) {
          const int g = g0 + gg;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float sc = acc[gg][i];
            stage(__builtin_amdgcn_fmed3f(sc, tlo[g], thi[g]) == sc, g, sc, kt * KT + 16 * w + lg + 4 * i);
          }
        }
      } else {
#pragma unroll
        for (int gg = 0; gg < NG / 2; ++gg) {
          const int g = g0 + gg;
          const int nv = nv_of(g);   // 0 for rows past Tq
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int j = kt * KT + 16 * w + lg + 4 * i;
            const float sc = acc[gg][i];
            stage((__builtin_amdgcn_fmed3f(sc, tlo[g], thi[g]) == sc) & (j < nv), g, sc, j);
          }
        }
      }
      if (g0 == 0) return;   // the rest once per tile, after its second half
      // Positions 0..30 only ever hold candidates; position 31 may hold a later
      // non-candidate entry once the column is full, so a full lane (block flagged
      // for the fallback) flushes 31.
      full_col |= kc >= 32u;
      kc = min(kc, 31u);
      if (ballot64(kc >= 16u) != 0ull) flush();
    });
    if (ballot64(kc != 0u) != 0ull) flush();
  }
  if (__syncthreads_or(full_col)) {   // block-uniform: the fallback launch redoes both halves
    if (tid < 2) {
      const int q64 = 2 * qb + tid;
      if (q64 < nqb) a.flags[(long)(nqb - 1 - q64) * BH + bh] = 1;
    }
    return;
  }
  // A window wider than b* (ties across its edges) can exceed the scratch list.
  int over = 0;
  if (lane < 32) {
    const int g = w + 4 * (lane >> 4), r = lane & 15;
    over = rinfo[g][r].mode == COLLECT && colcnt[g][r] > TOPK_CAP;
  }
  // (also the barrier after which candidates and counters of every wave are in
  // place and hist is the resolve's area)
  if (__syncthreads_or(over)) {
    if (tid < 2) {
      const int q64 = 2 * qb + tid;
      if (q64 < nqb) a.flags[(long)(nqb - 1 - q64) * BH + bh] = 1;
    }
    return;
  }

  // ---- resolve: the exact cut of every COLLECT row of the wave --------------
  uint32_t* h256 = &hist[0][0] + 4096 * w;   // 256 words of the wave's own staging area
  float thv = -INFINITY;   // lane rr < 32: row (group w + 4 (rr / 16), rr % 16)
  int cutv = 0x7fffffff;
  // The wave's COLLECT rows (bit rr), resolved in turn; each row's candidates
  // are loaded while the row before it is resolved.  All CAPL loads of a row are
  // issued (slots past its count re-read slot 0, which every COLLECT row has), so
  // the number of loads in flight is the same on every path.
  uint32_t cmask = 0;
  if (lane < 32) {
    const RowInfo ri = rinfo[w + 4 * (lane >> 4)][lane & 15];
    if (ri.mode == BIN_ALL) thv = score1(ri.th0, mscale);   // everything from a0's score up
    cmask = ri.mode == COLLECT;
  }
  cmask = (uint32_t)ballot64(cmask != 0u);
  // Four rows at a time first: lanes 16s..16s+15 take the s-th of the four
  // lowest rows left, lane u its candidates 16m + u (m < CAPQ), and each group
  // runs the byte radix below on a 256-bin histogram of its own (words 256s.. of
  // the wave's area).  Rows with more than 16 CAPQ candidates, and rows whose
  // cut key is shared by more candidates than it takes (the index tie-break),
  // stay in cmask for the one-row resolve.
  {
    constexpr int CAPQ = 16;
    const int qs = lane >> 4, qu = lane & 15;
    uint32_t big = 0;
    if (lane < 32 && ((cmask >> lane) & 1u)) big = colcnt[w + 4 * (lane >> 4)][lane & 15] > 16 * CAPQ;
    const uint32_t bigm = (uint32_t)ballot64(big != 0u);
    uint32_t todo = cmask & ~bigm;
    cmask &= bigm;
    // A quad is four rows packed in bytes (row id, 0xff for none), wave-uniform;
    // lanes of an empty group take group 0's row.
    auto quad_rows = [&](uint32_t m) __attribute__((always_inline)) {
      uint32_t rq = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        rq |= (m != 0u ? (uint32_t)__builtin_ctz(m) : 0xffu) << (8 * q);
        m &= m - 1u;
      }
      return rq;
    };
    auto load_quad = [&](uint32_t rq, uint2 (&buf)[CAPQ]) __attribute__((always_inline)) {
      const uint32_t rsel = (rq >> (8 * qs)) & 0xffu;
      const int rr = (int)(rsel != 0xffu ? rsel : rq & 0xffu);
      const int g = w + 4 * (rr >> 4), r = rr & 15;
      const long row = srowb + 16 * g + r;
      const int n = min(colcnt[g][r], TOPK_CAP);
#pragma unroll
      for (int m = 0; m < CAPQ; ++m) {
        const int p = 16 * m + qu;
        buf[m] = scratch[row * TOPK_CAP + (p < n ? p : 0)];
      }
    };
    uint32_t* hq = h256 + 256 * qs;
    auto resolve_quad = [&](uint32_t rq, const uint2 (&cb)[CAPQ]) __attribute__((always_inline)) {
      const uint32_t rsel = (rq >> (8 * qs)) & 0xffu;
      const bool live = rsel != 0xffu;
      const int rr = (int)(live ? rsel : rq & 0xffu);
      const int g = w + 4 * (rr >> 4), r = rr & 15;
      const RowInfo ri = rinfo[g][r];
      const int n = live ? min(colcnt[g][r], TOPK_CAP) : 0;
      const float a0 = ra0[g][r];
      uint32_t key[CAPQ];
      uint32_t nin = 0;   // collected keys at or above a0
#pragma unroll
      for (int m = 0; m < CAPQ; ++m) {
        const bool ok = 16 * m + qu < n;
        const float x = __uint_as_float(cb[m].x);
        key[m] = ok ? f32_order_key(score1(x, mscale)) : 0u;
        nin += (ok && x >= a0) ? 1u : 0u;
      }
      nin = row16_sum(nin, lane);
      uint32_t rneed = (uint32_t)(ri.need - rcntb[g][r]) + nin;
      float thq = -INFINITY;
      bool done = !live, radix = false;
      if (live && rneed == 0u) {   // none of the window's keys: s > score1(th1)
        thq = next_up(score1(ri.th1, mscale));
        done = true;
      }
      radix = !done;
      // bytes that key(score1(th0)) and key(score1(th1)) share need no pass
      const uint32_t klo = f32_order_key(score1(ri.th0, mscale));
      const uint32_t dif = klo ^ f32_order_key(score1(ri.th1, mscale));
      uint32_t rm = 0;
      int sh = 24;
      while (sh > 0 && (dif >> sh) == 0u) { rm |= 0xffu << sh; sh -= 8; }
      uint32_t rp = klo & rm;
      while (ballot64(!done) != 0ull) {
#pragma unroll
        for (int q = 0; q < 4; ++q) reinterpret_cast<uint4*>(hq)[4 * qu + q] = make_uint4(0u, 0u, 0u, 0u);
        wave_lds_sync();
#pragma unroll
        for (int m = 0; m < CAPQ; ++m) {
          if (!done && 16 * m + qu < n && (key[m] & rm) == rp) atomicAdd(&hq[(key[m] >> sh) & 255u], 1u);
        }
        wave_lds_sync();
        uint32_t c[16];
        {
          const uint4* hr = reinterpret_cast<const uint4*>(hq + 240 - 16 * qu);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint4 v4 = hr[q];
            c[15 - 4 * q] = v4.x; c[14 - 4 * q] = v4.y; c[13 - 4 * q] = v4.z; c[12 - 4 * q] = v4.w;
          }
        }
        int bin;
        uint32_t above, cnt;
        find_bin16(c, lane, rneed, bin, above, cnt);
        wave_lds_sync();   // counts read before the next pass clears them
        if (!done) {
          rp |= (uint32_t)bin << sh;
          rm |= 0xffu << sh;
          rneed -= above;
          if (cnt == rneed) done = true;
          else if ((sh -= 8) < 0) done = true;
        }
      }
      uint32_t neq = 0;
#pragma unroll
      for (int m = 0; m < CAPQ; ++m) neq += (16 * m + qu < n && (key[m] & rm) == rp) ? 1u : 0u;
      neq = row16_sum(neq, lane);
      const bool tie = radix && neq > rneed;   // index tie-break: the one-row resolve
      if (radix) thq = threshold_of_key(rp);
      // results to lane rr (rows < 32 of this wave)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t rq_q = (rq >> (8 * q)) & 0xffu;
        if (rq_q == 0xffu) continue;   // uniform
        const float tq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(thq), 16 * q));
        const bool tie_q = __builtin_amdgcn_readlane((int)tie, 16 * q) != 0;
        if (tie_q) cmask |= 1u << rq_q;
        else if (lane == (int)rq_q) { thv = tq; cutv = 0x7fffffff; }
      }
    };
    // two buffers in turn, the next quad's candidates loaded while one is resolved
    auto drop4 = [](uint32_t m) __attribute__((always_inline)) {
#pragma unroll
      for (int q = 0; q < 4; ++q) m &= m - 1u;
      return m;
    };
    uint2 qA[CAPQ], qB[CAPQ];
    if (todo != 0u) load_quad(quad_rows(todo), qA);
    while (todo != 0u) {
      const uint32_t ra = quad_rows(todo);
      todo = drop4(todo);
      const uint32_t rb = todo != 0u ? quad_rows(todo) : ra;
      load_quad(rb, qB);
      resolve_quad(ra, qA);
      if (todo == 0u) break;
      todo = drop4(todo);
      load_quad(todo != 0u ? quad_rows(todo) : rb, qA);
      resolve_quad(rb, qB);
    }
  }
  auto load_row = [&](int rr, uint2 (&buf)[CAPL]) __attribute__((always_inline)) {
    const int g = w + 4 * (rr >> 4), r = rr & 15;
    const long row = srowb + 16 * g + r;
    const int n = min(colcnt[g][r], TOPK_CAP);
#pragma unroll
    for (int m = 0; m < CAPL; ++m) {
      const int p = 64 * m + lane;
      buf[m] = scratch[row * TOPK_CAP + (p < n ? p : 0)];
    }
  };
  uint2 cbA[CAPL], cbB[CAPL];
  auto resolve_row = [&](int rr, const uint2 (&cb)[CAPL]) __attribute__((always_inline)) {
    const int g = w + 4 * (rr >> 4), r = rr & 15;
    const RowInfo ri = rinfo[g][r];
    const int n = min(colcnt[g][r], TOPK_CAP);
    uint32_t key[CAPL];
    int idx[CAPL];
    uint32_t nin = 0;   // collected keys at or above a0
#pragma unroll
    for (int m = 0; m < CAPL; ++m) {
      const int p = 64 * m + lane;
      key[m] = 0; idx[m] = 0;
      float x = -INFINITY;
      if (p < n) {
        x = __uint_as_float(cb[m].x);
        key[m] = f32_order_key(score1(x, mscale));
        idx[m] = (int)cb[m].y;
      }
      nin += (uint32_t)__popcll(ballot64(p < n && x >= ra0[g][r]));
    }
    uint32_t rneed = (uint32_t)(ri.need - rcntb[g][r]) + nin;
    if (rneed == 0u) {   // none of the window's keys (all tied at a0's score): s > score1(th1)
      if (lane == rr) thv = next_up(score1(ri.th1, mscale));
      return;
    }
    // every collected key lies in [key(score1(th0)), key(score1(th1))]: the bytes
    // those two share are the same for all of them and need no pass
    const uint32_t klo = f32_order_key(score1(ri.th0, mscale));
    const uint32_t dif = klo ^ f32_order_key(score1(ri.th1, mscale));
    uint32_t rm = 0;
    int sh = 24;
    while (sh > 0 && (dif >> sh) == 0u) { rm |= 0xffu << sh; sh -= 8; }
    uint32_t rp = klo & rm;
    for (; sh >= 0; sh -= 8) {
#pragma unroll
      for (int q = 0; q < 4; ++q) h256[4 * lane + q] = 0;
      wave_lds_sync();
#pragma unroll
      for (int m = 0; m < CAPL; ++m) {
        if (64 * m + lane < n && (key[m] & rm) == rp) atomicAdd(&h256[(key[m] >> sh) & 255u], 1u);
      }
      wave_lds_sync();
      uint32_t c[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) c[q] = h256[255 - 4 * lane - q];
      int bin;
      uint32_t above, cnt;
      find_bin(c, lane, rneed, bin, above, cnt);
      rp |= (uint32_t)bin << sh;
      rm |= 0xffu << sh;
      rneed -= above;
      wave_lds_sync();
      if (cnt == rneed) break;
    }
    // Keys at the threshold key rp: the rneed with the smallest key index win;
    // a radix select over ~index finds the last of them when more are equal.
    uint32_t neq = 0;
#pragma unroll
    for (int m = 0; m < CAPL; ++m) neq += (uint32_t)__popcll(ballot64(64 * m + lane < n && (key[m] & rm) == rp));
    uint32_t ip = 0;
    if (neq > rneed) {
      uint32_t im = 0, need2 = rneed;
      for (int sh2 = 24; sh2 >= 0; sh2 -= 8) {
#pragma unroll
        for (int q = 0; q < 4; ++q) h256[4 * lane + q] = 0;
        wave_lds_sync();
#pragma unroll
        for (int m = 0; m < CAPL; ++m) {
          const uint32_t ik = ~(uint32_t)idx[m];
          if (64 * m + lane < n && (key[m] & rm) == rp && (ik & im) == ip) atomicAdd(&h256[(ik >> sh2) & 255u], 1u);
        }
        wave_lds_sync();
        uint32_t c[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) c[q] = h256[255 - 4 * lane - q];
        int bin;
        uint32_t above, cnt;
        find_bin(c, lane, need2, bin, above, cnt);
        ip |= (uint32_t)bin << sh2;
        im |= 0xffu << sh2;
        need2 -= above;
        wave_lds_sync();
        if (cnt == need2) break;
      }
    }
    // selected: key > rp (rp's low bits are zero when the loop stopped early), or
    // key == rp and ~index >= ip, i.e. index <= ~ip
    if (lane == rr) {
      thv = threshold_of_key(rp);
      cutv = neq > rneed ? (int)~ip : 0x7fffffff;
    }
  };
  // Two buffers in turn.  The prefetch is unconditional (with no next row it
  // reloads the current one): a conditional load would make the compiler wait for
  // both buffers before using the first.
  if (cmask != 0u) load_row(__builtin_ctz(cmask), cbA);
  while (cmask != 0u) {
    const int ra = __builtin_ctz(cmask);
    cmask &= cmask - 1u;
    load_row(cmask != 0u ? __builtin_ctz(cmask) : ra, cbB);
    resolve_row(ra, cbA);
    if (cmask == 0u) break;
    const int rb = __builtin_ctz(cmask);
    cmask &= cmask - 1u;
    load_row(cmask != 0u ? __builtin_ctz(cmask) : rb, cbA);
    resolve_row(rb, cbB);
  }
  if (lane < 32) {
    const int g = w + 4 * (lane >> 4), r = lane & 15;
    const int qr = r0 + 16 * g + r;
    if (qr < Tq) {
      const long rowg = srowb + 16 * g + r;
      a.thr[rowg] = make_uint2(__float_as_uint(thv), (uint32_t)cutv);
      if (a.counts) a.counts[rowg] = min(kq_row(qr), nv_row(qr));
      if (a.split) a.split[rowg] = 0;
      // scores of the top-2 accumulators (score1 is monotone); -FLT_MAX marks "none"
      a.top2[2 * rowg] = t2.x == -FLT_MAX ? -FLT_MAX : score1(t2.x, mscale);
      a.top2[2 * rowg + 1] = t2.y == -FLT_MAX ? -FLT_MAX : score1(t2.y, mscale);
    }
  }
}

size_t topk_workspace_bytes(int B, int Tq, int H) {
  const size_t nqb = (Tq + QB - 1) / QB;
  return (size_t)B * H * Tq * TOPK_CAP * sizeof(uint2) + (((size_t)B * H * nqb * sizeof(int) + 255) & ~(size_t)255) +
         (size_t)B * H * KNCH * sizeof(float) + 512;
}

size_t topk_list_bytes(int B, int Tq, int H, int top_k) {
  const size_t nqb = (Tq + QB - 1) / QB;
  return (size_t)B * H * nqb * 4 * 16 * (size_t)(top_k + TOPK_CAP) * sizeof(uint2);
}

size_t topk_list_off_bytes(int B, int Tq, int Tk, int H) {
  const size_t nqb = (Tq + QB - 1) / QB;
  return (size_t)B * H * nqb * 4 * (size_t)((Tk + KT - 1) / KT + 1) * sizeof(int32_t);
}

hipError_t launch_score_topk(const TopkArgs& a0, hipStream_t st) {
  TopkArgs a = a0;
  const int nqb = (a.Tq + QB - 1) / QB;
  const int BH = a.B * a.H;
  // score = acc / scale is evaluated as acc * (1/scale) with the reciprocal
  // rounded once on the host; scale_mode 1 multiplies by scale directly.
  const float ms = score_multiplier(a.scale, a.scale_mode);
  if (a.dump) {
    const int qb0 = a.dump_row0 / QB;
    const int qb1 = (a.dump_row0 + a.dump_rows + QB - 1) / QB;
    const dim3 grid((unsigned)(BH * (qb1 - qb0)));
    if (a.dtype == DT_F32) score_topk_kernel<float, true, true, false, false, false><<<grid, 256, 0, st>>>(a, nqb, ms);
    else score_topk_kernel<bf16_t, true, true, false, false, false><<<grid, 256, 0, st>>>(a, nqb, ms);
    return hipGetLastError();
  }
  // workspace: [scratch lists | block flags | kmax]
  char* ws = (char*)(((uintptr_t)a.workspace + 255) & ~(uintptr_t)255);
  a.scratch = (uint2*)ws;
  ws += (size_t)BH * a.Tq * TOPK_CAP * sizeof(uint2);
  a.flags = (int*)ws;
  ws += ((size_t)BH * nqb * sizeof(int) + 255) & ~(size_t)255;
  float* kmax = (float*)ws;
  a.kmax = kmax;
  const dim3 kgrid((unsigned)(BH * KNCH));
  if (a.dtype == DT_F32) key_norm_max_kernel<float><<<kgrid, 256, 0, st>>>((const float*)a.k, a.Tk, a.H, a.D, kmax);
  else key_norm_max_kernel<bf16_t><<<kgrid, 256, 0, st>>>((const bf16_t*)a.k, a.Tk, a.H, a.D, kmax);
  const dim3 grid((unsigned)(BH * nqb));
  const bool c16 = a.Tk <= 65535;   // 16-bit histogram counters cannot overflow
  const bool t2 = a.top2 != nullptr;
  if (a.thr != nullptr) {   // layer path, threshold mode (bf16, D = 128, top-2 required)
    if (a.dtype != DT_BF16 || !t2 || a.D != DP) return hipErrorInvalidValue;
    // score_thr128_kernel bins accumulators (needs mscale > 0) and holds key indices in 16
    // bits; at Tk = 65536 it sends rows whose counters could overflow to the fallback,
    // which then counts in 32 bits
    if (a.Tk <= 65536 && ms > 0.f && ms < FLT_MAX) {
      const dim3 grid128((unsigned)(BH * ((a.Tq + 127) / 128)));
      if (a.row_nv != nullptr) score_thr128_kernel<true><<<grid128, 256, 0, st>>>(a, nqb, ms);
      else score_thr128_kernel<false><<<grid128, 256, 0, st>>>(a, nqb, ms);
      if (c16) score_topk_kernel<bf16_t, false, true, true, true, true, true><<<grid, 256, 0, st>>>(a, nqb, ms);
      else score_topk_kernel<bf16_t, false, false, true, true, true, true><<<grid, 256, 0, st>>>(a, nqb, ms);
    } else {
      score_topk_tiles_kernel<false, true><<<grid, 256, 0, st>>>(a, nqb, ms);
      score_topk_kernel<bf16_t, false, false, true, true, true, true><<<grid, 256, 0, st>>>(a, nqb, ms);
    }
    return hipGetLastError();
  }
  if (a.tl_list != nullptr) {   // layer path: tile lists (bf16, top-2 required)
    a.tl_ntmax = (a.Tk + KT - 1) / KT;
    if (a.dtype != DT_BF16 || !t2) return hipErrorInvalidValue;
    const bool regs = a.D == DP;   // K fragments straight into registers (D = 128)
    if (c16) {
      if (regs) score_topk_tiles_kernel<true, false><<<grid, 256, 0, st>>>(a, nqb, ms);
      else score_topk_kernel<bf16_t, false, true, true, false, true><<<grid, 256, 0, st>>>(a, nqb, ms);
      score_topk_kernel<bf16_t, false, true, true, true, true><<<grid, 256, 0, st>>>(a, nqb, ms);
    } else {
      if (regs) score_topk_tiles_kernel<false, false><<<grid, 256, 0, st>>>(a, nqb, ms);
      else score_topk_kernel<bf16_t, false, false, true, false, true><<<grid, 256, 0, st>>>(a, nqb, ms);
      score_topk_kernel<bf16_t, false, false, true, true, true><<<grid, 256, 0, st>>>(a, nqb, ms);
    }
    return hipGetLastError();
  }
#define SGSA_TOPK_LAUNCH(XT, C, T2)                                                   \
  do {                                                                                \
    score_topk_kernel<XT, false, C, T2, false, false><<<grid, 256, 0, st>>>(a, nqb, ms);     \
    score_topk_kernel<XT, false, C, T2, true, false><<<grid, 256, 0, st>>>(a, nqb, ms);      \
  } while (0)
  if (a.dtype == DT_F32) {
    if (c16) { if (t2) SGSA_TOPK_LAUNCH(float, true, true); else SGSA_TOPK_LAUNCH(float, true, false); }
    else { if (t2) SGSA_TOPK_LAUNCH(float, false, true); else SGSA_TOPK_LAUNCH(float, false, false); }
  } else {
    if (c16) { if (t2) SGSA_TOPK_LAUNCH(bf16_t, true, true); else SGSA_TOPK_LAUNCH(bf16_t, true, false); }
    else { if (t2) SGSA_TOPK_LAUNCH(bf16_t, false, true); else SGSA_TOPK_LAUNCH(bf16_t, false, false); }
  }
#undef SGSA_TOPK_LAUNCH
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
