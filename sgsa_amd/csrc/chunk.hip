// Chunked SGSA forward on gfx950: the replacement for the per-chunk Python
// loop of modelings/sgsa_ops/chunk_fwd.py:39-129 and its Triton pieces
// (chunk_fwd_triton.py:19-260).
//
// Per (batch, head) the sequence is cut into chunks of L=64 tokens.  Each
// token carries two virtual write samples (local: k,v,beta; sparse: k~,v^,alpha)
// interleaved as sample i = 2t + r (chunk_fwd.py:53-56), so a chunk has M=128
// samples (M=64 without the sparse write).  With D_t the inclusive chunk-local
// product of gamma (kept as a log-cumsum), and S the state at the chunk start:
//
//   T_ij = 1[tau_j < tau_i] lam_j exp(logD_tau_i - logD_tau_j) (kappa_i . kappa_j)
//   A    = (I + T)^-1                       W = A diag(D_tau) kappa     U = A nu
//   R    = U - W S                          (residuals, all samples)
//   o_t  = D_t S^T q_t + sum_{tau_i <= t} lam_i (D_t / D_tau_i) (q_t . kappa_i) R_i
//   S'   = D_L S + sum_i kappa_i lam_i (D_L / D_tau_i) R_i^T
//
// Three kernels:
//   chunk_intra  (K3)  parallel over all chunks: Gram, transition, blocked
//                      inverse, W and U.
//   chunk_state  (K4)  sequential over chunks per (b,h, 16-column slice of S):
//                      the fp32 state recurrence; stores R and the chunk-start
//                      states.
//   chunk_out    (K5)  parallel over all chunks: the readout.
// This file is the fp32-input path: all contractions use v_mfma_f32_16x16x4_f32
// with fp32 operands.  bf16 inputs take chunk_bf16.hip.  The head dimension is padded to DP=128 in LDS and
// in the workspace; padded rows/columns are zero and never stored.
#include "common.h"
#include "kernels.h"

namespace sgsa {

namespace {

constexpr int L = 64;
constexpr int DP = 128;
constexpr int PIT = DP + 4;  // LDS row pitch (floats)

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Loads the M x DP sample matrix of one chunk (rows interleaved local/sparse)
// into LDS as fp32, zero outside [0,T) x [0,D).
template <typename X, bool SP>
__device__ __forceinline__ void load_samples(float (*dst)[PIT], const X* __restrict__ a, const X* __restrict__ sa,
                                             int b, int h, int t0, int T, int H, int D) {
  constexpr int M = SP ? 2 * L : L;
  for (int e = threadIdx.x; e < M * DP; e += blockDim.x) {
    const int i = e / DP, d = e % DP;
    const int tl = SP ? (i >> 1) : i;
    const int r = SP ? (i & 1) : 0;
    const int t = t0 + tl;
    float x = 0.f;
    if (t < T && d < D) x = ld(r ? sa : a, ((long)(b * T + t) * H + h) * D + d);
    dst[i][d] = x;
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// K3: intra-chunk transform.  grid (NT, B*H), 256 threads.
// ---------------------------------------------------------------------------
template <typename X, bool SP>
__global__ __launch_bounds__(256) void chunk_intra_kernel(
    const X* __restrict__ k, const X* __restrict__ v, const X* __restrict__ sk, const X* __restrict__ sv,
    const float* __restrict__ beta, const float* __restrict__ alpha, const float* __restrict__ gamma,
    int T, int H, int D, int NT, float* __restrict__ Wout, float* __restrict__ Uout,
    float* __restrict__ logd_out, float* __restrict__ Aout = nullptr) {
  constexpr int M = SP ? 2 * L : L;
  constexpr int NB = M / 16;
  __shared__ float kap[M][PIT];
  __shared__ float Tm[M][PIT];
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
    logd_out[((long)bh * NT + c) * L + tid] = x;
  }
  if (tid < M) {
    const int tl = SP ? (tid >> 1) : tid;
    const int r = SP ? (tid & 1) : 0;
    const int t = t0 + tl;
    float lm = 0.f;
    if (t < T) lm = r ? alpha[(long)(b * T + t) * H + h] : beta[(long)(b * T + t) * H + h];
    lam[tid] = lm;
  }
  load_samples<X, SP>(kap, k, sk, b, h, t0, T, H, D);
  __syncthreads();
  if (tid < M) dtau[tid] = expf(logd[SP ? (tid >> 1) : tid]);

  // Gram + transition on the lower block triangle (diagonal blocks included).
  constexpr int NTILE = NB * (NB + 1) / 2;
  for (int ti = w; ti < NTILE; ti += 4) {
    int I = 0;
    while ((I + 1) * (I + 2) / 2 <= ti) ++I;
    const int J = ti - I * (I + 1) / 2;
    f4 acc = f4_zero();
#pragma unroll 8
    for (int s = 0; s < DP / 4; ++s) {
      const float a = kap[16 * I + lr][4 * s + lg];
      const float bb = kap[16 * J + lr][4 * s + lg];
      acc = mma_f32(a, bb, acc);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * I + 4 * lg + e, j = 16 * J + lr;
      const int tI = SP ? (i >> 1) : i, tJ = SP ? (j >> 1) : j;
      float val = 0.f;
      if (tJ < tI) val = lam[j] * expf(logd[tI] - logd[tJ]) * acc[e];
      Tm[i][j] = val;
    }
  }
  __syncthreads();

  // Inverse of each 16x16 unit-lower diagonal block by forward substitution.
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

  // Off-diagonal blocks: A_IJ = -inv_I * sum_{K=J}^{I-1} T_IK A_KJ, written over T_IJ.
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

  // A itself (the backward's operand): [M][M] row-major, zero above the diagonal.
  if (Aout != nullptr) {
    float* Ac = Aout + ((long)bh * NT + c) * M * M;
    for (int e = tid; e < M * M; e += 256) {
      const int i = e / M, j = e % M, I = i >> 4, J = j >> 4;
      float x = 0.f;
      if (I == J) x = inv[I][i & 15][j & 15];
      else if (J < I) x = Tm[i][j];
      Ac[e] = x;
    }
  }

  // W = A diag(D_tau) kappa, then U = A nu.  Wave w owns output column tiles 2w, 2w+1.
  float* Wc = Wout + ((long)bh * NT + c) * M * DP;
  float* Uc = Uout + ((long)bh * NT + c) * M * DP;
  for (int pass = 0; pass < 2; ++pass) {
    if (pass == 1) {
      __syncthreads();
      load_samples<X, SP>(kap, v, sv, b, h, t0, T, H, D);
      __syncthreads();
    }
    float* dst = pass == 0 ? Wc : Uc;
    for (int I = 0; I < NB; ++I) {
#pragma unroll
      for (int nn = 0; nn < 2; ++nn) {
        const int n = 2 * w + nn;
        f4 acc = f4_zero();
        for (int J = 0; J <= I; ++J) {
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const float a = (J == I) ? inv[I][lr][4 * s + lg] : Tm[16 * I + lr][16 * J + 4 * s + lg];
            const int kk = 16 * J + 4 * s + lg;
            float bb = kap[kk][16 * n + lr];
            if (pass == 0) bb *= dtau[kk];
            acc = mma_f32(a, bb, acc);
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[(long)(16 * I + 4 * lg + e) * DP + 16 * n + lr] = acc[e];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// K4: inter-chunk state recurrence.  grid (DP/16, B*H), 256 threads.
// Block (cs, bh) owns columns [16cs, 16cs+16) of the state of head bh.
// ---------------------------------------------------------------------------
template <typename X, bool SP>
__global__ __launch_bounds__(256) void chunk_state_kernel(
    const X* __restrict__ k, const X* __restrict__ sk, const float* __restrict__ beta,
    const float* __restrict__ alpha, const float* __restrict__ Wg, const float* __restrict__ Ug,
    const float* __restrict__ logd_g, const float* __restrict__ h0, int T, int H, int D, int NT,
    float* __restrict__ Hs, float* __restrict__ Rg, float* __restrict__ ht) {
  constexpr int M = SP ? 2 * L : L;
  constexpr int RT = M / 64;   // residual row tiles per wave
  __shared__ float Ssh[DP][17];
  __shared__ float Rsh[M][17];
  __shared__ float lam[M];
  __shared__ float logd[L];

  const int cs = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const int lr = lane & 15, lg = lane >> 4;
  const int col = 16 * cs + lr;

  // wave w owns state rows [32w, 32w+32): tiles 2w, 2w+1
  f4 S[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 16 * (2 * w + u) + 4 * lg + e;
      float x = 0.f;
      if (h0 != nullptr && row < D && col < D) x = h0[((long)bh * D + row) * D + col];
      S[u][e] = x;
    }
  }

  for (int c = 0; c < NT; ++c) {
    const int t0 = c * L;
    if (tid < L) logd[tid] = logd_g[((long)bh * NT + c) * L + tid];
    if (tid < M) {
      const int tl = SP ? (tid >> 1) : tid;
      const int r = SP ? (tid & 1) : 0;
      const int t = t0 + tl;
      float lm = 0.f;
      if (t < T) lm = r ? alpha[(long)(b * T + t) * H + h] : beta[(long)(b * T + t) * H + h];
      lam[tid] = lm;
    }
    float* Hc = Hs + ((long)bh * NT + c) * DP * DP;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * (2 * w + u) + 4 * lg + e;
        Ssh[row][lr] = S[u][e];
        Hc[(long)row * DP + col] = S[u][e];
      }
    }
    __syncthreads();

    // R = U - W S for this wave's residual row tiles.
    const float* Wc = Wg + ((long)bh * NT + c) * M * DP;
    const float* Uc = Ug + ((long)bh * NT + c) * M * DP;
    float* Rc = Rg + ((long)bh * NT + c) * M * DP;
    const float logdL = logd[L - 1];
#pragma unroll
    for (int u = 0; u < RT; ++u) {
      const int I = RT * w + u;
      f4 acc;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = Uc[(long)(16 * I + 4 * lg + e) * DP + col];
#pragma unroll 8
      for (int s = 0; s < DP / 4; ++s) {
        const float a = -Wc[(long)(16 * I + lr) * DP + 4 * s + lg];
        acc = mma_f32(a, Ssh[4 * s + lg][lr], acc);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 16 * I + 4 * lg + e;
        Rc[(long)i * DP + col] = acc[e];
        const int ti = SP ? (i >> 1) : i;
        Rsh[i][lr] = acc[e] * lam[i] * expf(logdL - logd[ti]);
      }
    }
    __syncthreads();

    // S <- D_L S + kappa^T R'
    const float DL = expf(logdL);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int row = 16 * (2 * w + u) + lr;   // state row (key dim) for the A operand
      f4 acc = S[u] * DL;
#pragma unroll 4
      for (int s = 0; s < M / 4; ++s) {
        const int i = 4 * s + lg;
        const int tl = SP ? (i >> 1) : i;
        const int r = SP ? (i & 1) : 0;
        const int t = t0 + tl;
        float a = 0.f;
        if (t < T && row < D) a = ld(r ? sk : k, ((long)(b * T + t) * H + h) * D + row);
        acc = mma_f32(a, Rsh[i][lr], acc);
      }
      S[u] = acc;
    }
    __syncthreads();
  }

  if (ht != nullptr) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * (2 * w + u) + 4 * lg + e;
        if (row < D && col < D) ht[((long)bh * D + row) * D + col] = S[u][e];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// K5: chunk readout.  grid (NT, B*H), 256 threads; wave w owns tokens [16w, 16w+16).
// ---------------------------------------------------------------------------
template <typename X, bool SP>
__global__ __launch_bounds__(256) void chunk_out_kernel(
    const X* __restrict__ q, const X* __restrict__ k, const X* __restrict__ sk,
    const float* __restrict__ beta, const float* __restrict__ alpha, const float* __restrict__ logd_g,
    const float* __restrict__ Hs, const float* __restrict__ Rg, int T, int H, int D, int NT,
    X* __restrict__ out) {
  constexpr int M = SP ? 2 * L : L;
  __shared__ float qs[L][PIT];
  __shared__ float kap[M][PIT];
  __shared__ float ps[4][16][M + 4];
  __shared__ float lam[M];
  __shared__ float logd[L];

  const int c = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const int lr = lane & 15, lg = lane >> 4;
  const int t0 = c * L;

  if (tid < L) logd[tid] = logd_g[((long)bh * NT + c) * L + tid];
  if (tid < M) {
    const int tl = SP ? (tid >> 1) : tid;
    const int r = SP ? (tid & 1) : 0;
    const int t = t0 + tl;
    float lm = 0.f;
    if (t < T) lm = r ? alpha[(long)(b * T + t) * H + h] : beta[(long)(b * T + t) * H + h];
    lam[tid] = lm;
  }
  for (int e = tid; e < L * DP; e += 256) {
    const int i = e / DP, d = e % DP, t = t0 + i;
    qs[i][d] = (t < T && d < D) ? ld(q, ((long)(b * T + t) * H + h) * D + d) : 0.f;
  }
  load_samples<X, SP>(kap, k, sk, b, h, t0, T, H, D);
  __syncthreads();

  const float* Sc = Hs + ((long)bh * NT + c) * DP * DP;
  const float* Rc = Rg + ((long)bh * NT + c) * M * DP;
  const int trow = 16 * w + lr;   // token row of this lane's A operand

  // O = diag(D) Q S
  f4 O[DP / 16];
#pragma unroll
  for (int n = 0; n < DP / 16; ++n) {
    f4 acc = f4_zero();
#pragma unroll 8
    for (int s = 0; s < DP / 4; ++s) acc = mma_f32(qs[trow][4 * s + lg], Sc[(4 * s + lg) * DP + 16 * n + lr], acc);
    O[n] = acc;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float dt = expf(logd[16 * w + 4 * lg + e]);
#pragma unroll
    for (int n = 0; n < DP / 16; ++n) O[n][e] *= dt;
  }

  // P = mask(Q kappa^T) scaled, staged in this wave's LDS rows.
#pragma unroll
  for (int m = 0; m < M / 16; ++m) {
    f4 acc = f4_zero();
#pragma unroll 8
    for (int s = 0; s < DP / 4; ++s) acc = mma_f32(qs[trow][4 * s + lg], kap[16 * m + lr][4 * s + lg], acc);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * w + 4 * lg + e, i = 16 * m + lr;
      const int ti = SP ? (i >> 1) : i;
      ps[w][4 * lg + e][i] = (ti <= t) ? lam[i] * expf(logd[t] - logd[ti]) * acc[e] : 0.f;
    }
  }
  wave_lds_sync();

  // O += P R
#pragma unroll
  for (int n = 0; n < DP / 16; ++n) {
    f4 acc = O[n];
#pragma unroll 8
    for (int s = 0; s < M / 4; ++s) acc = mma_f32(ps[w][lr][4 * s + lg], Rc[(4 * s + lg) * DP + 16 * n + lr], acc);
    O[n] = acc;
  }

#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int t = t0 + 16 * w + 4 * lg + e;
    if (t >= T) continue;
#pragma unroll
    for (int n = 0; n < DP / 16; ++n) {
      const int d = 16 * n + lr;
      if (d < D) st(out, ((long)(b * T + t) * H + h) * D + d, O[n][e]);
    }
  }
}

// ---------------------------------------------------------------------------
// Host launcher
// ---------------------------------------------------------------------------

size_t chunk_workspace_bytes(int B, int T, int H, int has_sparse) {
  const long NT = (T + L - 1) / L;
  const long M = has_sparse ? 2 * L : L;
  const long BH = (long)B * H;
  const long wu = BH * NT * M * DP;         // W, U, R each
  const long hs = BH * NT * DP * DP;        // chunk-start states
  const long lgd = BH * NT * L;
  const size_t f32 = sizeof(float) * (3 * wu + hs + lgd) + 256 * 5;
  const size_t b16 = chunk_bf16_workspace_bytes(B, T, H, has_sparse);
  return f32 > b16 ? f32 : b16;
}

template <typename X, bool SP>
static hipError_t launch_chunk_t(const ChunkArgs& a, hipStream_t st) {
  const int NT = (a.T + L - 1) / L;
  const int M = SP ? 2 * L : L;
  const int BH = a.B * a.H;
  auto align = [](char* p) { return (char*)(((uintptr_t)p + 255) & ~(uintptr_t)255); };
  char* p = align((char*)a.workspace);
  float* W = (float*)p;  p = align(p + sizeof(float) * (size_t)BH * NT * M * DP);
  float* U = (float*)p;  p = align(p + sizeof(float) * (size_t)BH * NT * M * DP);
  float* R = (float*)p;  p = align(p + sizeof(float) * (size_t)BH * NT * M * DP);
  float* Hs = (float*)p; p = align(p + sizeof(float) * (size_t)BH * NT * DP * DP);
  float* lgd = (float*)p;
  const X* q = (const X*)a.q;
  const X* k = (const X*)a.k;
  const X* v = (const X*)a.v;
  const X* sk = (const X*)a.sparse_k;
  const X* sv = (const X*)a.sparse_v;
  chunk_intra_kernel<X, SP><<<dim3(NT, BH), 256, 0, st>>>(k, v, sk, sv, a.beta, a.alpha, a.gamma, a.T, a.H, a.D,
                                                          NT, W, U, lgd);
  chunk_state_kernel<X, SP><<<dim3(DP / 16, BH), 256, 0, st>>>(k, sk, a.beta, a.alpha, W, U, lgd,
                                                               a.initial_state, a.T, a.H, a.D, NT, Hs, R,
                                                               a.final_state);
  chunk_out_kernel<X, SP><<<dim3(NT, BH), 256, 0, st>>>(q, k, sk, a.beta, a.alpha, lgd, Hs, R, a.T, a.H, a.D, NT,
                                                        (X*)a.out);
  return hipGetLastError();
}

// The forward's per-chunk intermediates for the backward (chunk_bwd.hip): W, U,
// the log-decay prefix and A, for bf16 or fp32 inputs alike (loaded into fp32).
template <typename X, bool SP>
static hipError_t launch_intra_t(const ChunkArgs& a, float* W, float* U, float* lgd, float* A, hipStream_t st) {
  const int NT = (a.T + L - 1) / L;
  const int BH = a.B * a.H;
  chunk_intra_kernel<X, SP><<<dim3(NT, BH), 256, 0, st>>>((const X*)a.k, (const X*)a.v, (const X*)a.sparse_k,
                                                          (const X*)a.sparse_v, a.beta, a.alpha, a.gamma, a.T, a.H,
                                                          a.D, NT, W, U, lgd, A);
  return hipGetLastError();
}

hipError_t launch_chunk_intra(const ChunkArgs& a, float* W, float* U, float* lgd, float* A, hipStream_t st) {
  const bool sp = a.sparse_k != nullptr;
  if (a.dtype == DT_BF16) return launch_chunk_intra_bf16(a, W, U, lgd, A, st);
  return sp ? launch_intra_t<float, true>(a, W, U, lgd, A, st) : launch_intra_t<float, false>(a, W, U, lgd, A, st);
}

hipError_t launch_chunk_fwd(const ChunkArgs& a, hipStream_t st) {
  if (a.dtype == DT_BF16) return launch_chunk_bf16(a, st);
  const bool sp = a.sparse_k != nullptr;
  return sp ? launch_chunk_t<float, true>(a, st) : launch_chunk_t<float, false>(a, st);
}

}  // namespace sgsa
