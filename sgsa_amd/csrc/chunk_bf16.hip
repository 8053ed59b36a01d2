// Chunked SGSA forward, bf16-input path (v_mfma_f32_16x16x32_bf16).
//
// Same algorithm and notation as chunk.hip (the fp32 path); the difference is
// how each contraction maps onto bf16 MFMA without losing the fp32 state:
//   * products of two bf16 inputs (kappa kappa^T, q kappa^T) are exact in the
//     fp32 accumulator and use one MFMA;
//   * an fp32 operand X (A = (I+T)^-1, the state S, the residuals R, the
//     readout weights P) is split X = hi + lo into two bf16 planes, and
//     X.Y = hi.Y + lo.Y (both operands fp32: hi.hi + hi.lo + lo.hi), which
//     keeps ~16 mantissa bits;
//   * the transition T and its blocked inverse stay in fp32 (v_mfma 16x16x4 f32).
// Workspace planes are stored in the operand layouts the consumers read with
// 16-byte loads (row-major W, transposed kappa / S / R).
//
// K3 chunk_intra_bf16  grid (NT, B*H)      Gram, T, (I+T)^-1, W = A D_tau kappa, U = A nu, kappa^T
// K4 chunk_seg_bf16    grid (B*H, G, 2|1)  state pass over G segments of chunks: per-segment affine
//    chunk_seg_scan_bf16 grid (B*H)        maps, a scan over segments, then each segment replays its
//                                          chunks from its start state (operands of chunk c+1 are
//                                          prefetched into registers while chunk c is processed)
// K5 chunk_out_bf16    grid (NT, B*H)      o = D Q S + P R
#include "common.h"
#include "kernels.h"

namespace sgsa {

namespace {

constexpr int L = 64;
constexpr int DP = 128;
constexpr int PB = DP + 8;     // bf16 LDS pitch (272 B rows)
constexpr int PF = DP + 4;     // fp32 LDS pitch

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroup barrier that orders LDS only: each wave waits for its own LDS
// operations, not for global loads and stores still in flight (__syncthreads
// waits for those too, which would stall register prefetches at the barrier).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ bf16x8 as_bf8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

__device__ __forceinline__ uint4 zero4() { return make_uint4(0, 0, 0, 0); }

// 8 consecutive bf16 of an input row starting at d0 (zero outside [0,D) or !valid).
__device__ __forceinline__ uint4 load8(const bf16_t* row, int d0, int D, bool valid) {
  if (!valid || d0 >= D) return zero4();
  if ((D & 7) == 0) return *reinterpret_cast<const uint4*>(row + d0);
  u16x8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = (d0 + j < D) ? row[d0 + j].bits : (uint16_t)0;
  return __builtin_bit_cast(uint4, r);
}

__device__ __forceinline__ void split8(const float (&x)[8], uint4& hi, uint4& lo) {
  u16x8 h, l;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint16_t b = f32_to_bf16(x[j]);
    h[j] = b;
    l[j] = f32_to_bf16(x[j] - bf16_to_f32(b));
  }
  hi = __builtin_bit_cast(uint4, h);
  lo = __builtin_bit_cast(uint4, l);
}

__device__ __forceinline__ void split1(float x, uint16_t& hi, uint16_t& lo) {
  hi = f32_to_bf16(x);
  lo = f32_to_bf16(x - bf16_to_f32(hi));
}

// sample i of a chunk -> (token offset, which input)
template <bool SP> __device__ __forceinline__ int samp_t(int i) { return SP ? (i >> 1) : i; }
template <bool SP> __device__ __forceinline__ int samp_r(int i) { return SP ? (i & 1) : 0; }

}  // namespace

struct Bf16Ws {
  uint16_t* Whi;   // [BH,NT,M,DP]
  uint16_t* Wlo;
  float* U;        // [BH,NT,M,DP]
  uint16_t* KT;    // [BH,NT,DP,M]   kappa^T
  uint16_t* STh;   // [BH,NT,DP,DP]  chunk-start state, transposed [col][row]
  uint16_t* STl;
  uint16_t* RTh;   // [BH,NT,DP,M]   residuals, transposed [col][sample]
  uint16_t* RTl;
  float* logd;     // [BH,NT,L]
};

// ---------------------------------------------------------------------------
// K3
// ---------------------------------------------------------------------------
template <bool SP>
__global__ __launch_bounds__(256) void chunk_intra_bf16(
    const bf16_t* __restrict__ k, const bf16_t* __restrict__ v, const bf16_t* __restrict__ sk,
    const bf16_t* __restrict__ sv, const float* __restrict__ beta, const float* __restrict__ alpha,
    const float* __restrict__ gamma, int T, int H, int D, int NT, Bf16Ws ws) {
  constexpr int M = SP ? 2 * L : L;
  constexpr int NB = M / 16;
  constexpr int PM = M + 8;
  constexpr int KAPN = (M * PB > DP * PM) ? M * PB : DP * PM;
  __shared__ __align__(16) uint16_t kap[KAPN];        // kappa rows; later nu^T [DP][PM]
  __shared__ __align__(16) uint16_t kapT[DP * PM];    // kappa^T
  __shared__ __align__(16) float Tm[M][M + 4];
  __shared__ float inv[NB][16][17];
  __shared__ float scr[4][16][17];
  __shared__ float lam[M];
  __shared__ float dtau[M];
  __shared__ float logd[L];

  const int c = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const int lr = lane & 15, lg = lane >> 4;
  const int t0 = c * L;
  const long cidx = (long)bh * NT + c;

  if (tid < L) {
    const int t = t0 + tid;
    float x = 0.f;
    if (t < T) x = logf(fmaxf(gamma[(long)(b * T + t) * H + h], 1e-6f));
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float n = __shfl_up(x, o, 64);
      if (lane >= o) x += n;
    }
    logd[tid] = x;
    ws.logd[cidx * L + tid] = x;
  }
  if (tid < M) {
    const int t = t0 + samp_t<SP>(tid);
    float lm = 0.f;
    if (t < T) lm = samp_r<SP>(tid) ? alpha[(long)(b * T + t) * H + h] : beta[(long)(b * T + t) * H + h];
    lam[tid] = lm;
  }
  // kappa rows and kappa^T (16-byte chunks of 8 dims)
  for (int e = tid; e < M * (DP / 8); e += 256) {
    const int i = e / (DP / 8), cv = e % (DP / 8);
    const int t = t0 + samp_t<SP>(i);
    const bf16_t* src = samp_r<SP>(i) ? sk : k;
    const uint4 x = load8(src + ((long)(b * T + (t < T ? t : 0)) * H + h) * D, 8 * cv, D, t < T);
    *reinterpret_cast<uint4*>(&kap[i * PB + 8 * cv]) = x;
    const u16x8 xs = __builtin_bit_cast(u16x8, x);
#pragma unroll
    for (int j = 0; j < 8; ++j) kapT[(8 * cv + j) * PM + i] = xs[j];
  }
  __syncthreads();
  if (tid < M) dtau[tid] = expf(logd[samp_t<SP>(tid)]);

  // Gram on the lower block triangle -> transition T (fp32)
  constexpr int NTILE = NB * (NB + 1) / 2;
  for (int ti = w; ti < NTILE; ti += 4) {
    int I = 0;
    while ((I + 1) * (I + 2) / 2 <= ti) ++I;
    const int J = ti - I * (I + 1) / 2;
    f4 acc = f4_zero();
#pragma unroll
    for (int s = 0; s < DP / 32; ++s) {
      const uint4 a = *reinterpret_cast<const uint4*>(&kap[(16 * I + lr) * PB + 32 * s + 8 * lg]);
      const uint4 bb = *reinterpret_cast<const uint4*>(&kap[(16 * J + lr) * PB + 32 * s + 8 * lg]);
      acc = mma_bf16(as_bf8(a), as_bf8(bb), acc);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * I + 4 * lg + e, j = 16 * J + lr;
      const int tI = samp_t<SP>(i), tJ = samp_t<SP>(j);
      Tm[i][j] = (tJ < tI) ? lam[j] * expf(logd[tI] - logd[tJ]) * acc[e] : 0.f;
    }
  }
  __syncthreads();

  // kappa^T -> workspace (consumed by K4 as the A operand of kappa^T R')
  {
    uint16_t* dst = ws.KT + cidx * DP * M;
    for (int e = tid; e < DP * (M / 8); e += 256) {
      const int d = e / (M / 8), cv = e % (M / 8);
      *reinterpret_cast<uint4*>(dst + d * M + 8 * cv) = *reinterpret_cast<const uint4*>(&kapT[d * PM + 8 * cv]);
    }
  }
  // nu^T into the kappa buffer (kappa rows are no longer needed)
  for (int e = tid; e < M * (DP / 8); e += 256) {
    const int i = e / (DP / 8), cv = e % (DP / 8);
    const int t = t0 + samp_t<SP>(i);
    const bf16_t* src = samp_r<SP>(i) ? sv : v;
    const uint4 x = load8(src + ((long)(b * T + (t < T ? t : 0)) * H + h) * D, 8 * cv, D, t < T);
    const u16x8 xs = __builtin_bit_cast(u16x8, x);
#pragma unroll
    for (int j = 0; j < 8; ++j) kap[(8 * cv + j) * PM + i] = xs[j];
  }

  // diagonal 16x16 inverses
  for (int Ib = w; Ib < NB; Ib += 4) {
    if (lane < 16) {
      for (int i = 0; i < 16; ++i) {
        float x = (i == lane) ? 1.f : 0.f;
        for (int j = 0; j < i; ++j) x -= Tm[16 * Ib + i][16 * Ib + j] * inv[Ib][j][lane];
        inv[Ib][i][lane] = x;
      }
    }
  }
  __syncthreads();

  // off-diagonal blocks of A = (I+T)^-1 (fp32), written over T
  for (int I = 1; I < NB; ++I) {
    f4 res0 = f4_zero(), res1 = f4_zero();
#pragma unroll
    for (int slot = 0; slot < 2; ++slot) {
      const int J = w + 4 * slot;
      if (J >= I) continue;
      f4 tmp = f4_zero();
      for (int K = J; K < I; ++K) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const float a = Tm[16 * I + lr][16 * K + 4 * s + lg];
          const float bb = (K == J) ? inv[J][4 * s + lg][lr] : Tm[16 * K + 4 * s + lg][16 * J + lr];
          tmp = mma_f32(a, bb, tmp);
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) scr[w][4 * lg + e][lr] = tmp[e];
      wave_lds_sync();
      f4 r = f4_zero();
#pragma unroll
      for (int s = 0; s < 4; ++s) r = mma_f32(inv[I][lr][4 * s + lg], scr[w][4 * s + lg][lr], r);
      wave_lds_sync();
      if (slot == 0) res0 = -r; else res1 = -r;
    }
    __syncthreads();
#pragma unroll
    for (int slot = 0; slot < 2; ++slot) {
      const int J = w + 4 * slot;
      if (J >= I) continue;
      const f4 r = slot == 0 ? res0 : res1;
#pragma unroll
      for (int e = 0; e < 4; ++e) Tm[16 * I + 4 * lg + e][16 * J + lr] = r[e];
    }
    __syncthreads();
  }
  // complete A in Tm: diagonal blocks from inv, zeros above
  for (int e = tid; e < M * M; e += 256) {
    const int i = e / M, j = e % M, I = i >> 4, J = j >> 4;
    if (J == I) Tm[i][j] = inv[I][i & 15][j & 15];
    else if (J > I) Tm[i][j] = 0.f;
  }
  __syncthreads();

  // W = (A diag(D_tau)) kappa, U = A nu.  Wave w owns the row blocks I = w and
  // NB-1-w (equal k-step counts per wave) across all 8 column tiles, so the
  // hi/lo split of each A fragment is done once and feeds 8 column tiles.
  uint16_t* Wh = ws.Whi + cidx * M * DP;
  uint16_t* Wl = ws.Wlo + cidx * M * DP;
  float* Uc = ws.U + cidx * M * DP;
  for (int ii = 0; ii < NB / 4; ++ii) {
    const int I = ii == 0 ? w : NB - 1 - w;
    if (I >= NB) continue;
    const int nks = (16 * (I + 1) + 31) / 32;   // A is zero right of column 16 (I + 1)
    f4 aw[DP / 16], au[DP / 16];
#pragma unroll
    for (int n = 0; n < DP / 16; ++n) { aw[n] = f4_zero(); au[n] = f4_zero(); }
    for (int s = 0; s < nks; ++s) {
      const int k0 = 32 * s + 8 * lg;
      float xa[8], xw[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        xa[j] = Tm[16 * I + lr][k0 + j];
        xw[j] = xa[j] * dtau[k0 + j];
      }
      uint4 ahi, alo, whi, wlo;
      split8(xa, ahi, alo);
      split8(xw, whi, wlo);
      // transposed products (kappa^T / nu^T as the A operand): lane (lr, lg) ends
      // up with columns 16n + 4lg .. +3 of row 16I + lr, stored as one 8-byte
      // (W planes) or 16-byte (U) vector; same products and order as W, U
#pragma unroll
      for (int n = 0; n < DP / 16; ++n) {
        const uint4 bk = *reinterpret_cast<const uint4*>(&kapT[(16 * n + lr) * PM + k0]);
        const uint4 bv = *reinterpret_cast<const uint4*>(&kap[(16 * n + lr) * PM + k0]);
        aw[n] = mma_bf16(as_bf8(bk), as_bf8(whi), aw[n]);
        aw[n] = mma_bf16(as_bf8(bk), as_bf8(wlo), aw[n]);
        au[n] = mma_bf16(as_bf8(bv), as_bf8(ahi), au[n]);
        au[n] = mma_bf16(as_bf8(bv), as_bf8(alo), au[n]);
      }
    }
#pragma unroll
    for (int n = 0; n < DP / 16; ++n) {
      const long off = (long)(16 * I + lr) * DP + 16 * n + 4 * lg;
      uint16_t hi[4], lo[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) split1(aw[n][e], hi[e], lo[e]);
      *reinterpret_cast<uint2*>(Wh + off) =
          make_uint2((uint32_t)hi[0] | ((uint32_t)hi[1] << 16), (uint32_t)hi[2] | ((uint32_t)hi[3] << 16));
      *reinterpret_cast<uint2*>(Wl + off) =
          make_uint2((uint32_t)lo[0] | ((uint32_t)lo[1] << 16), (uint32_t)lo[2] | ((uint32_t)lo[3] << 16));
      *reinterpret_cast<float4*>(Uc + off) = make_float4(au[n][0], au[n][1], au[n][2], au[n][3]);
    }
  }
}

// ---------------------------------------------------------------------------
// K4: the inter-chunk state pass, segment-parallel.
//
// One chunk maps its start state S to D_L S + kappa^T (lambda' (U - W S)),
// which is affine in S, so a segment of consecutive chunks maps its start
// state to its end state as S_end = Phi S_start + P: Phi is the segment's
// chunk maps applied to the identity with U = 0, P the same maps applied to 0
// with U.  Three launches replace the one sequential pass over all chunks:
//   1. chunk_seg_bf16<SEG_MAPS>: one block per (b*h, segment, P or Phi) runs
//      the segment's chunks; all segments at once;
//   2. chunk_seg_scan_bf16: per b*h, S_start(0) = h0 and
//      S_start(g+1) = Phi_g S_start(g) + P_g;
//   3. chunk_seg_bf16<SEG_FULL>: each segment reruns its chunks from its start
//      state and writes the chunk-start states and residuals K5 reads.
// A block owns all 128 state columns: each chunk's W, kappa^T and U cross into
// the CU once and feed the products of all four waves.  Wave w owns state rows
// 32w .. 32w + 31 and residual (sample) rows (M/64) w * 16 .. + M/64 * 16.
// Products keep the fp32 state exact to about 2^-16: W, S and R' are split
// into bf16 hi + lo (the lo * lo term is dropped).
// ---------------------------------------------------------------------------
enum SegMode { SEG_MAPS = 0, SEG_FULL = 1 };

__device__ __forceinline__ uint4 neg_bf16x8(uint4 u) {
  return make_uint4(u.x ^ 0x80008000u, u.y ^ 0x80008000u, u.z ^ 0x80008000u, u.w ^ 0x80008000u);
}

// Number of segments of the state pass: enough (b*h, segment) blocks to fill
// the GPU, at least 8 chunks per segment, at most 16 segments.
inline int seg_count(int BH, int NT) {
  int g = (256 + BH - 1) / BH;
  g = g < 16 ? g : 16;
  const int gmax = (NT + 7) / 8;
  g = g < gmax ? g : gmax;
  return g < 1 ? 1 : g;
}

// MODE SEG_MAPS: blockIdx.z 0 builds P (start 0, with U), 1 builds Phi (start
// I, U = 0); the end state goes to sout[(z * BH + bh) * G + g] ([DP][DP] fp32).
// MODE SEG_FULL: the start state is sinit[bh * G + g] with leading dimension
// sld (rows and columns >= sld read as 0); chunk-start states and residuals go
// to the workspace, and the last segment's end state to ht ([DP][DP]-padded
// rows/cols < D, leading dimension D).
template <bool SP, int MODE>
__global__ __launch_bounds__(256, 1) void chunk_seg_bf16(const float* __restrict__ beta, const float* __restrict__ alpha,
                                                       int T, int H, int D, int NT, int CPS, Bf16Ws ws,
                                                       const float* __restrict__ sinit, int sld,
                                                       float* __restrict__ sout, float* __restrict__ ht) {
  constexpr int M = SP ? 2 * L : L;
  constexpr int RT = M / 64;      // residual row tiles per wave
  constexpr int KS = DP / 32;     // k-steps over the key dim
  constexpr int KSM = M / 32;     // k-steps over samples
  constexpr int PM = M + 8;
  constexpr int NC = DP / 16;     // column tiles
  __shared__ __align__(16) uint16_t Sh[DP * PB];   // S transposed [col][row], hi
  __shared__ __align__(16) uint16_t Sl[DP * PB];
  __shared__ __align__(16) uint16_t Rh[DP * PM];   // R' transposed [col][sample], hi
  __shared__ __align__(16) uint16_t Rl[DP * PM];
  __shared__ float lam[M];
  __shared__ float logd[L];

  const int bh = blockIdx.x, g = blockIdx.y, G = gridDim.y, BH = gridDim.x;
  const bool phi = MODE == SEG_MAPS && blockIdx.z == 1;   // block-uniform
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const int lr = lane & 15, lg = lane >> 4;
  const int cb = g * CPS, ce = min(NT, cb + CPS);

  // state rows 32w + 16u + 4lg + e, columns 16n + lr
  f4 S[2][NC];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int n = 0; n < NC; ++n) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 32 * w + 16 * u + 4 * lg + e, col = 16 * n + lr;
        float x = 0.f;
        if (MODE == SEG_MAPS) x = (phi && row == col) ? 1.f : 0.f;
        else if (sinit != nullptr && row < sld && col < sld) x = sinit[((long)(bh * G + g) * sld + row) * sld + col];
        S[u][n][e] = x;
      }
    }
  }

  // Per-chunk operand fragments, one set each: W and U are reloaded for the
  // next chunk as soon as the residual products have used them, kappa^T as
  // soon as the state update has, so each load has the rest of a chunk to land.
  uint4 wh[RT][KS], wl[RT][KS], kt[2][KSM];
  f4 uu[RT][NC];
  float nlogd = 0.f, nlam = 0.f;   // this thread's log-decay / write-strength entries of the next chunk
  const bool use_u = !phi;
  auto load_wu = [&](int c) __attribute__((always_inline)) {
    const long cidx = (long)bh * NT + c;
    const uint16_t* Wh = ws.Whi + cidx * M * DP;
    const uint16_t* Wl = ws.Wlo + cidx * M * DP;
    const float* Uc = ws.U + cidx * M * DP;
#pragma unroll
    for (int u = 0; u < RT; ++u) {
      const int I = RT * w + u;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        wh[u][s] = neg_bf16x8(*reinterpret_cast<const uint4*>(Wh + (16 * I + lr) * DP + 32 * s + 8 * lg));
        wl[u][s] = neg_bf16x8(*reinterpret_cast<const uint4*>(Wl + (16 * I + lr) * DP + 32 * s + 8 * lg));
      }
#pragma unroll
      for (int n = 0; n < NC; ++n) {
#pragma unroll
        for (int e = 0; e < 4; ++e) uu[u][n][e] = use_u ? Uc[(16 * I + 4 * lg + e) * DP + 16 * n + lr] : 0.f;
      }
    }
  };
  auto load_kt = [&](int c) __attribute__((always_inline)) {
    const uint16_t* KTc = ws.KT + ((long)bh * NT + c) * DP * M;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int s = 0; s < KSM; ++s)
        kt[u][s] = *reinterpret_cast<const uint4*>(KTc + (32 * w + 16 * u + lr) * M + 32 * s + 8 * lg);
    }
  };
  auto load_gates = [&](int c) __attribute__((always_inline)) {
    if (tid < L) nlogd = ws.logd[((long)bh * NT + c) * L + tid];
    if (tid < M) {
      const int t = c * L + samp_t<SP>(tid);
      nlam = 0.f;
      if (t < T) nlam = samp_r<SP>(tid) ? alpha[(long)(b * T + t) * H + h] : beta[(long)(b * T + t) * H + h];
    }
  };

  if (cb < ce) {
    load_wu(cb);
    load_kt(cb);
    load_gates(cb);
  }
  for (int c = cb; c < ce; ++c) {
    const long cidx = (long)bh * NT + c;
    // logd / lam of this chunk into LDS (the previous chunk's readers passed a barrier)
    if (tid < L) logd[tid] = nlogd;
    if (tid < M) lam[tid] = nlam;
    if (c + 1 < ce) load_gates(c + 1);
    // chunk-start state: LDS operand copy, and the workspace copy K5 reads (both [col][row], hi/lo)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int row0 = 32 * w + 16 * u + 4 * lg;
#pragma unroll
      for (int n = 0; n < NC; ++n) {
        uint16_t hh[4], ll[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) split1(S[u][n][e], hh[e], ll[e]);
        const ushort4 hv = make_ushort4(hh[0], hh[1], hh[2], hh[3]);
        const ushort4 lv = make_ushort4(ll[0], ll[1], ll[2], ll[3]);
        const int col = 16 * n + lr;
        *reinterpret_cast<ushort4*>(&Sh[col * PB + row0]) = hv;
        *reinterpret_cast<ushort4*>(&Sl[col * PB + row0]) = lv;
        if constexpr (MODE == SEG_FULL) {
          *reinterpret_cast<ushort4*>(&ws.STh[cidx * DP * DP + (long)col * DP + row0]) = hv;
          *reinterpret_cast<ushort4*>(&ws.STl[cidx * DP * DP + (long)col * DP + row0]) = lv;
        }
      }
    }
    lds_barrier();

    // R = U - W S (the W fragments are negated: acc = U + (-W) S; Wl.Sl dropped),
    // one 16-column tile at a time (a scheduling barrier keeps the compiler from
    // hoisting every tile's LDS operands at once)
    const float logdL = logd[L - 1];
#pragma unroll
    for (int u = 0; u < RT; ++u) {
      const int I = RT * w + u;
      const int i0 = 16 * I + 4 * lg;
      float fac[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) fac[e] = lam[i0 + e] * expf(logdL - logd[samp_t<SP>(i0 + e)]);
#pragma unroll
      for (int n = 0; n < NC; ++n) {
        f4 r = uu[u][n];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const uint4 bh_ = *reinterpret_cast<const uint4*>(&Sh[(16 * n + lr) * PB + 32 * s + 8 * lg]);
          const uint4 bl_ = *reinterpret_cast<const uint4*>(&Sl[(16 * n + lr) * PB + 32 * s + 8 * lg]);
          r = mma_bf16(as_bf8(wh[u][s]), as_bf8(bh_), r);
          r = mma_bf16(as_bf8(wh[u][s]), as_bf8(bl_), r);
          r = mma_bf16(as_bf8(wl[u][s]), as_bf8(bh_), r);
        }
        const int col = 16 * n + lr;
        uint16_t hh[4], ll[4], h2[4], l2[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          split1(r[e], hh[e], ll[e]);
          split1(r[e] * fac[e], h2[e], l2[e]);
        }
        if constexpr (MODE == SEG_FULL) {
          *reinterpret_cast<ushort4*>(&ws.RTh[cidx * DP * M + (long)col * M + i0]) = make_ushort4(hh[0], hh[1], hh[2], hh[3]);
          *reinterpret_cast<ushort4*>(&ws.RTl[cidx * DP * M + (long)col * M + i0]) = make_ushort4(ll[0], ll[1], ll[2], ll[3]);
        }
        *reinterpret_cast<ushort4*>(&Rh[col * PM + i0]) = make_ushort4(h2[0], h2[1], h2[2], h2[3]);
        *reinterpret_cast<ushort4*>(&Rl[col * PM + i0]) = make_ushort4(l2[0], l2[1], l2[2], l2[3]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (c + 1 < ce) load_wu(c + 1);
    lds_barrier();

    // S <- D_L S + kappa^T R'
    const float DL = expf(logdL);
#pragma unroll
    for (int n = 0; n < NC; ++n) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        f4 acc = S[u][n] * DL;
#pragma unroll
        for (int s = 0; s < KSM; ++s) {
          const uint4 rh = *reinterpret_cast<const uint4*>(&Rh[(16 * n + lr) * PM + 32 * s + 8 * lg]);
          const uint4 rl = *reinterpret_cast<const uint4*>(&Rl[(16 * n + lr) * PM + 32 * s + 8 * lg]);
          acc = mma_bf16(as_bf8(kt[u][s]), as_bf8(rh), acc);
          acc = mma_bf16(as_bf8(kt[u][s]), as_bf8(rl), acc);
        }
        S[u][n] = acc;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (c + 1 < ce) load_kt(c + 1);
  }

#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int n = 0; n < NC; ++n) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 32 * w + 16 * u + 4 * lg + e, col = 16 * n + lr;
        if constexpr (MODE == SEG_MAPS) {
          sout[((long)((blockIdx.z * BH + bh) * G + g) * DP + row) * DP + col] = S[u][n][e];
        } else {
          if (ht != nullptr && g == G - 1 && row < D && col < D) ht[((long)bh * D + row) * D + col] = S[u][n][e];
        }
      }
    }
  }
}

// The segment start states: sinit[bh*G + g] for g < G, from h0 ([B*H][D][D] or
// NULL) and the maps of chunk_seg_bf16<SEG_MAPS> (maps[0]: P, maps[1]: Phi).
// S <- Phi S + P runs in fp32 with Phi and S split into bf16 hi + lo.
__global__ __launch_bounds__(256, 1) void chunk_seg_scan_bf16(int G, int D, const float* __restrict__ h0,
                                                            const float* __restrict__ maps, float* __restrict__ sinit) {
  constexpr int NC = DP / 16;
  constexpr int KS = DP / 32;
  __shared__ __align__(16) uint16_t Sh[DP * PB];   // S transposed [col][row], hi
  __shared__ __align__(16) uint16_t Sl[DP * PB];
  const int bh = blockIdx.x, BH = gridDim.x;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const float* P = maps;
  const float* Phi = maps + (long)BH * G * DP * DP;
  f4 S[2][NC];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int n = 0; n < NC; ++n) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 32 * w + 16 * u + 4 * lg + e, col = 16 * n + lr;
        S[u][n][e] = (h0 != nullptr && row < D && col < D) ? h0[((long)bh * D + row) * D + col] : 0.f;
      }
    }
  }
  for (int g = 0; g < G; ++g) {
    float* dst = sinit + (long)(bh * G + g) * DP * DP;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int n = 0; n < NC; ++n) {
        const int row0 = 32 * w + 16 * u + 4 * lg, col = 16 * n + lr;
        uint16_t hh[4], ll[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          dst[(long)(row0 + e) * DP + col] = S[u][n][e];
          split1(S[u][n][e], hh[e], ll[e]);
        }
        *reinterpret_cast<ushort4*>(&Sh[col * PB + row0]) = make_ushort4(hh[0], hh[1], hh[2], hh[3]);
        *reinterpret_cast<ushort4*>(&Sl[col * PB + row0]) = make_ushort4(ll[0], ll[1], ll[2], ll[3]);
      }
    }
    if (g + 1 == G) break;
    __syncthreads();
    const float* Pg = P + (long)(bh * G + g) * DP * DP;
    const float* Fg = Phi + (long)(bh * G + g) * DP * DP;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int rowA = 32 * w + 16 * u + lr;   // A operand row (Phi)
      uint4 ah[KS], al[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        float x[8];
        const float4 x0 = *reinterpret_cast<const float4*>(Fg + (long)rowA * DP + 32 * s + 8 * lg);
        const float4 x1 = *reinterpret_cast<const float4*>(Fg + (long)rowA * DP + 32 * s + 8 * lg + 4);
        x[0] = x0.x; x[1] = x0.y; x[2] = x0.z; x[3] = x0.w; x[4] = x1.x; x[5] = x1.y; x[6] = x1.z; x[7] = x1.w;
        split8(x, ah[s], al[s]);
      }
#pragma unroll
      for (int n = 0; n < NC; ++n) {
        f4 acc;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = Pg[(long)(32 * w + 16 * u + 4 * lg + e) * DP + 16 * n + lr];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const uint4 bh_ = *reinterpret_cast<const uint4*>(&Sh[(16 * n + lr) * PB + 32 * s + 8 * lg]);
          const uint4 bl_ = *reinterpret_cast<const uint4*>(&Sl[(16 * n + lr) * PB + 32 * s + 8 * lg]);
          acc = mma_bf16(as_bf8(ah[s]), as_bf8(bh_), acc);
          acc = mma_bf16(as_bf8(ah[s]), as_bf8(bl_), acc);
          acc = mma_bf16(as_bf8(al[s]), as_bf8(bh_), acc);
        }
        S[u][n] = acc;
      }
    }
    __syncthreads();   // Sh/Sl are rewritten next
  }
}

// ---------------------------------------------------------------------------
// K5
// ---------------------------------------------------------------------------
template <bool SP>
__global__ __launch_bounds__(256) void chunk_out_bf16(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ sk,
    const float* __restrict__ beta, const float* __restrict__ alpha, int T, int H, int D, int NT, Bf16Ws ws,
    bf16_t* __restrict__ out) {
  constexpr int M = SP ? 2 * L : L;
  constexpr int PM = M + 8;
  constexpr int KS = DP / 32;
  constexpr int KSM = M / 32;
  __shared__ __align__(16) uint16_t Ph[4][16 * PM];
  __shared__ __align__(16) uint16_t Pl[4][16 * PM];
  __shared__ float lam[M];
  __shared__ float logd[L];

  const int c = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const int lr = lane & 15, lg = lane >> 4;
  const int t0 = c * L;
  const long cidx = (long)bh * NT + c;

  if (tid < L) logd[tid] = ws.logd[cidx * L + tid];
  if (tid < M) {
    const int t = t0 + samp_t<SP>(tid);
    float lm = 0.f;
    if (t < T) lm = samp_r<SP>(tid) ? alpha[(long)(b * T + t) * H + h] : beta[(long)(b * T + t) * H + h];
    lam[tid] = lm;
  }
  // q fragments: rows t0 + 16w + lr
  uint4 qf[KS];
  {
    const int t = t0 + 16 * w + lr;
    const bf16_t* qr = q + ((long)(b * T + (t < T ? t : 0)) * H + h) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = load8(qr, 32 * s + 8 * lg, D, t < T);
  }
  __syncthreads();

  const uint16_t* STh = ws.STh + cidx * DP * DP;
  const uint16_t* STl = ws.STl + cidx * DP * DP;
  const uint16_t* RTh = ws.RTh + cidx * DP * M;
  const uint16_t* RTl = ws.RTl + cidx * DP * M;

  // P = mask(q kappa^T) * lam_i * D_t / D_tau_i, staged hi/lo in this wave's LDS rows
#pragma unroll
  for (int m = 0; m < M / 16; ++m) {
    const int i = 16 * m + lr;
    const int t = t0 + samp_t<SP>(i);
    const bf16_t* kr = (samp_r<SP>(i) ? sk : k) + ((long)(b * T + (t < T ? t : 0)) * H + h) * D;
    f4 acc = f4_zero();
#pragma unroll
    for (int s = 0; s < KS; ++s) acc = mma_bf16(as_bf8(qf[s]), as_bf8(load8(kr, 32 * s + 8 * lg, D, t < T)), acc);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int tt = 16 * w + 4 * lg + e;
      const int ti = samp_t<SP>(i);
      const float p = (ti <= tt) ? lam[i] * expf(logd[tt] - logd[ti]) * acc[e] : 0.f;
      uint16_t hi, lo;
      split1(p, hi, lo);
      Ph[w][(4 * lg + e) * PM + i] = hi;
      Pl[w][(4 * lg + e) * PM + i] = lo;
    }
  }
  wave_lds_sync();

  float dt[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) dt[e] = expf(logd[16 * w + 4 * lg + e]);
#pragma unroll
  for (int n = 0; n < DP / 16; ++n) {
    const int cc = 16 * n + lr;
    f4 o1 = f4_zero();
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint4 bh_ = *reinterpret_cast<const uint4*>(STh + (long)cc * DP + 32 * s + 8 * lg);
      const uint4 bl_ = *reinterpret_cast<const uint4*>(STl + (long)cc * DP + 32 * s + 8 * lg);
      o1 = mma_bf16(as_bf8(qf[s]), as_bf8(bh_), o1);
      o1 = mma_bf16(as_bf8(qf[s]), as_bf8(bl_), o1);
    }
    f4 o2 = f4_zero();
#pragma unroll
    for (int s = 0; s < KSM; ++s) {
      const uint4 ph = *reinterpret_cast<const uint4*>(&Ph[w][lr * PM + 32 * s + 8 * lg]);
      const uint4 pl = *reinterpret_cast<const uint4*>(&Pl[w][lr * PM + 32 * s + 8 * lg]);
      const uint4 rh = *reinterpret_cast<const uint4*>(RTh + (long)cc * M + 32 * s + 8 * lg);
      const uint4 rl = *reinterpret_cast<const uint4*>(RTl + (long)cc * M + 32 * s + 8 * lg);
      o2 = mma_bf16(as_bf8(ph), as_bf8(rh), o2);
      o2 = mma_bf16(as_bf8(ph), as_bf8(rl), o2);
      o2 = mma_bf16(as_bf8(pl), as_bf8(rh), o2);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = t0 + 16 * w + 4 * lg + e;
      if (t < T && cc < D) out[((long)(b * T + t) * H + h) * D + cc].bits = f32_to_bf16(dt[e] * o1[e] + o2[e]);
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

size_t chunk_bf16_workspace_bytes(int B, int T, int H, int has_sparse) {
  const size_t NT = (T + L - 1) / L;
  const size_t M = has_sparse ? 2 * L : L;
  const size_t n = (size_t)B * H * NT;
  size_t total = 0;
  total += 2 * n * M * DP * 2;     // Whi, Wlo
  total += n * M * DP * 4;         // U
  total += n * DP * M * 2;         // KT
  total += 2 * n * DP * DP * 2;    // STh, STl
  total += 2 * n * DP * M * 2;     // RTh, RTl
  total += n * L * 4;              // logd
  const size_t G = seg_count(B * H, (int)NT);
  if (G > 1) total += 3 * (size_t)B * H * G * DP * DP * 4;   // segment maps P, Phi and start states
  return total + 256 * 12;
}

template <bool SP>
static hipError_t launch_bf16_t(const ChunkArgs& a, hipStream_t st) {
  const int NT = (a.T + L - 1) / L;
  const int M = SP ? 2 * L : L;
  const size_t n = (size_t)a.B * a.H * NT;
  auto align = [](char* p) { return (char*)(((uintptr_t)p + 255) & ~(uintptr_t)255); };
  char* p = align((char*)a.workspace);
  Bf16Ws ws;
  ws.Whi = (uint16_t*)p; p = align(p + n * M * DP * 2);
  ws.Wlo = (uint16_t*)p; p = align(p + n * M * DP * 2);
  ws.U = (float*)p;      p = align(p + n * M * DP * 4);
  ws.KT = (uint16_t*)p;  p = align(p + n * DP * M * 2);
  ws.STh = (uint16_t*)p; p = align(p + n * DP * DP * 2);
  ws.STl = (uint16_t*)p; p = align(p + n * DP * DP * 2);
  ws.RTh = (uint16_t*)p; p = align(p + n * DP * M * 2);
  ws.RTl = (uint16_t*)p; p = align(p + n * DP * M * 2);
  ws.logd = (float*)p;    p = align(p + n * L * 4);
  const int BH = a.B * a.H;
  const int G = seg_count(BH, NT);
  const int CPS = (NT + G - 1) / G;
  float* maps = (float*)p;   // [2][BH][G][DP][DP]: P, Phi
  float* sinit = maps + 2 * (size_t)BH * G * DP * DP;
  const bf16_t* q = (const bf16_t*)a.q;
  const bf16_t* k = (const bf16_t*)a.k;
  const bf16_t* v = (const bf16_t*)a.v;
  const bf16_t* sk = (const bf16_t*)a.sparse_k;
  const bf16_t* sv = (const bf16_t*)a.sparse_v;
  chunk_intra_bf16<SP><<<dim3(NT, BH), 256, 0, st>>>(k, v, sk, sv, a.beta, a.alpha, a.gamma, a.T, a.H, a.D, NT, ws);
  if (G == 1) {
    chunk_seg_bf16<SP, SEG_FULL><<<dim3(BH, 1, 1), 256, 0, st>>>(a.beta, a.alpha, a.T, a.H, a.D, NT, NT, ws,
                                                               a.initial_state, a.D, nullptr, a.final_state);
  } else {
    chunk_seg_bf16<SP, SEG_MAPS><<<dim3(BH, G, 2), 256, 0, st>>>(a.beta, a.alpha, a.T, a.H, a.D, NT, CPS, ws, nullptr,
                                                               0, maps, nullptr);
    chunk_seg_scan_bf16<<<dim3(BH), 256, 0, st>>>(G, a.D, a.initial_state, maps, sinit);
    chunk_seg_bf16<SP, SEG_FULL><<<dim3(BH, G, 1), 256, 0, st>>>(a.beta, a.alpha, a.T, a.H, a.D, NT, CPS, ws, sinit,
                                                               DP, nullptr, a.final_state);
  }
  chunk_out_bf16<SP><<<dim3(NT, BH), 256, 0, st>>>(q, k, sk, a.beta, a.alpha, a.T, a.H, a.D, NT, ws,
                                                   (bf16_t*)a.out);
  return hipGetLastError();
}

hipError_t launch_chunk_bf16(const ChunkArgs& a, hipStream_t st) {
  return a.sparse_k != nullptr ? launch_bf16_t<true>(a, st) : launch_bf16_t<false>(a, st);
}

}  // namespace sgsa
