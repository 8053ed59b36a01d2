// Backward of the chunked SGSA forward on gfx950 (chunk_sgsa's gradient).
//
// The reference differentiates chunk_sgsa by recomputing the forward in torch
// under autograd (modelings/sgsa_ops/chunk_bwd.py:12-77; the plan of a kernel
// backward is modelings/sgsa_bwd_derivation.md:699-832).  Here the gradient of
// the chunk form is written out and run as three stages, all on MFMA in fp32:
//
//   1. the forward's intermediates (chunk.hip, launch_chunk_recompute): per
//      chunk the WY inverse A = (I+T)^-1, W = A diag(D_tau) kappa, U = A nu,
//      R = U - W S, the chunk-start state S and the log-decay prefix l;
//   2. chunk_bwd_scan_kernel, sequential over chunks from the last, per
//      16-column slice of the state: the state gradient G at every chunk end,
//      and dR = P^T dO + diag(c) kappa G;
//   3. chunk_bwd_grad_kernel, parallel over chunks: every input gradient of a
//      chunk from (S, G, dR) and its inputs.
//
// Per chunk (tokens t, samples i at token tau_i, M = 2L samples with the
// sparse write, lambda = beta / alpha per sample):
//
//   P_ti = 1[tau_i <= t] exp(l_t - l_tau_i) lambda_i (q_t . kappa_i)
//   c_i  = lambda_i exp(l_L - l_tau_i),   l_L the chunk's last prefix
//   o    = diag(e^l) Q S + P R            S' = e^l_L S + kappa^T diag(c) R
//
// and with dO the output gradient of the chunk and G = dS':
//
//   dR = P^T dO + diag(c) kappa G
//   dS = Q^T diag(e^l) dO + e^l_L G - W^T dR                 (the scan's step)
//   dP = dO R^T;  Y = dP * 1[tau<=t] exp(l_t - l_tau) lambda
//   dq = diag(e^l) dO S^T + Y kappa
//   dW = -dR S^T;  Z = A^T dW;  dnu = A^T dR
//   dA = dR nu^T + dW (diag(e^l_tau) kappa)^T;  dT = -A^T dA A^T
//   X  = dT * 1[tau_j < tau_i] exp(l_tau_i - l_tau_j)
//   dkappa = Y^T Q + diag(c) R G^T + diag(e^l_tau) Z + X diag(lambda) kappa + diag(lambda) X^T kappa
//   dlambda_j = sum_t dP_tj exp(.) (q_t . kappa_j) + sum_i X_ij (kappa_i . kappa_j) + dc_j exp(l_L - l_tau_j)
//   dl: from P (dP_ti P_ti to l_t, minus to l_tau_i), from diag(e^l) Q S
//       (e^l_t q_t^T S dO_t), from c (dc_i c_i to l_L, minus to l_tau_i), from
//       e^l_L S (e^l_L <G, S>), from W (e^l_tau_i kappa_i . Z_i) and from T
//       (X_ij lambda_j (kappa_i . kappa_j) to l_tau_i, minus to l_tau_j);
//   dgamma_p = [gamma_p >= 1e-6] / gamma_p * sum_{t >= p in the chunk} dl_t
//
// with dc_i = (kappa G)_i . R_i, and d(initial_state) the scan's dS of chunk 0.
// The intermediates of stage 3 go through a per-chunk workspace (L2 traffic).
#include <float.h>

#include "common.h"
#include "kernels.h"

namespace sgsa {

namespace {

constexpr int L = 64;
constexpr int DP = 128;

// Reads of one (b, h) row block of the [B,T,H,D] inputs, zero outside [0,T) x [0,D).
template <typename X>
struct Rows {
  const X* p;
  int b, h, T, H, D;
  __device__ __forceinline__ float operator()(int t, int d) const {
    return (t < T && d < D) ? ld(p, ((long)(b * T + t) * H + h) * D + d) : 0.f;
  }
};

// One 16 x 16 output tile: acc += sum_k fa(row, k) fb(k, col) over k in [0, K),
// with the MFMA operand roles (lane l: A[l%16][l/16], B[l/16][l%16]).
template <typename FA, typename FB>
__device__ __forceinline__ f4 mm(f4 acc, int K, FA&& fa, FB&& fb) {
  const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
#pragma unroll 4
  for (int k0 = 0; k0 < K; k0 += 4) acc = mma_f32(fa(lr, k0 + lg), fb(k0 + lg, lr), acc);
  return acc;
}

// Stage 2.  grid (DP/16, B*H), 256 threads; block (cs, bh) owns state columns
// [16 cs, 16 cs + 16); wave w owns state rows [32 w, 32 w + 32).
template <typename X, bool SP>
__global__ __launch_bounds__(256) void chunk_bwd_scan_kernel(ChunkBwdArgs a, const float* __restrict__ Wg,
                                                             const float* __restrict__ lgd, float* __restrict__ Gend,
                                                             float* __restrict__ dRg, int NT) {
  constexpr int M = SP ? 2 * L : L;
  __shared__ float Pm[L][M + 1];
  __shared__ float Gs[DP][17];
  __shared__ float dRs[M][17];
  __shared__ float lam[M], cf[M], logd[L], el[L];

  const int cs = blockIdx.x, bh = blockIdx.y;
  const int B = a.f.B, T = a.f.T, H = a.f.H, D = a.f.D;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int col = 16 * cs + lr;
  (void)B;
  const Rows<X> q{(const X*)a.f.q, b, h, T, H, D}, dO{(const X*)a.d_out, b, h, T, H, D};
  const Rows<X> kk{(const X*)a.f.k, b, h, T, H, D}, ks{(const X*)a.f.sparse_k, b, h, T, H, D};

  f4 G[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 16 * (2 * w + u) + 4 * lg + e;
      float x = 0.f;
      if (a.d_final_state != nullptr && row < D && col < D) x = a.d_final_state[((long)bh * D + row) * D + col];
      G[u][e] = x;
    }
  }

  for (int c = NT - 1; c >= 0; --c) {
    const int t0 = c * L;
    auto kap = [&](int i, int d) __attribute__((always_inline)) {
      const int tl = SP ? (i >> 1) : i;
      return (SP && (i & 1)) ? ks(t0 + tl, d) : kk(t0 + tl, d);
    };
    if (tid < L) {
      const float x = lgd[((long)bh * NT + c) * L + tid];
      logd[tid] = x;
      el[tid] = expf(x);
    }
    __syncthreads();
    if (tid < M) {
      const int tl = SP ? (tid >> 1) : tid;
      const int r = SP ? (tid & 1) : 0;
      const int t = t0 + tl;
      float lm = 0.f;
      if (t < T) lm = r ? a.f.alpha[(long)(b * T + t) * H + h] : a.f.beta[(long)(b * T + t) * H + h];
      lam[tid] = lm;
      cf[tid] = lm * expf(logd[L - 1] - logd[tl]);
    }
    float* Gc = Gend + ((long)bh * NT + c) * DP * DP;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * (2 * w + u) + 4 * lg + e;
        Gs[row][lr] = G[u][e];
        Gc[(long)row * DP + col] = G[u][e];
      }
    }
    __syncthreads();

    // P [L][M]
    for (int tile = w; tile < (L / 16) * (M / 16); tile += 4) {
      const int I = tile / (M / 16), J = tile % (M / 16);
      f4 acc = mm(f4_zero(), DP, [&](int r, int k) { return q(t0 + 16 * I + r, k); },
                  [&](int k, int cc) { return kap(16 * J + cc, k); });
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = 16 * I + 4 * lg + e, i = 16 * J + lr;
        const int ti = SP ? (i >> 1) : i;
        Pm[t][i] = ti <= t ? expf(logd[t] - logd[ti]) * lam[i] * acc[e] : 0.f;
      }
    }
    __syncthreads();

    // dR[:, slice] = P^T dO[:, slice] + diag(c) kappa G[:, slice]
    float* dRc = dRg + ((long)bh * NT + c) * M * DP;
    for (int I = w; I < M / 16; I += 4) {
      f4 acc = mm(f4_zero(), L, [&](int r, int k) { return Pm[k][16 * I + r]; },
                  [&](int k, int cc) { return dO(t0 + k, 16 * cs + cc); });
      f4 acc2 = mm(f4_zero(), DP, [&](int r, int k) { return kap(16 * I + r, k); },
                   [&](int k, int cc) { return Gs[k][cc]; });
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 16 * I + 4 * lg + e;
        const float x = acc[e] + cf[i] * acc2[e];
        dRs[i][lr] = x;
        dRc[(long)i * DP + col] = x;
      }
    }
    __syncthreads();

    // G <- e^l_L G + Q^T diag(e^l) dO - W^T dR
    const float* Wc = Wg + ((long)bh * NT + c) * M * DP;
    const float eL = el[L - 1];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int R0 = 16 * (2 * w + u);
      f4 acc = mm(G[u] * eL, L, [&](int r, int k) { return q(t0 + k, R0 + r) * el[k]; },
                  [&](int k, int cc) { return dO(t0 + k, 16 * cs + cc); });
      f4 acc2 = mm(f4_zero(), M, [&](int r, int k) { return Wc[(long)k * DP + R0 + r]; },
                   [&](int k, int cc) { return dRs[k][cc]; });
      G[u] = acc - acc2;
    }
    __syncthreads();
  }

  if (a.d_initial_state != nullptr) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * (2 * w + u) + 4 * lg + e;
        if (row < D && col < D) a.d_initial_state[((long)bh * D + row) * D + col] = G[u][e];
      }
    }
  }
}

// Stage 3.  grid (NT, B*H), 256 threads: every gradient of one chunk.
template <typename X, bool SP>
__global__ __launch_bounds__(256) void chunk_bwd_grad_kernel(ChunkBwdArgs a, const float* __restrict__ Rg,
                                                             const float* __restrict__ Hs,
                                                             const float* __restrict__ lgd,
                                                             const float* __restrict__ Ag,
                                                             const float* __restrict__ Gend,
                                                             const float* __restrict__ dRg, float* __restrict__ scr,
                                                             int NT) {
  constexpr int M = SP ? 2 * L : L;
  __shared__ float lam[M], cf[M], etau[M], dlam[M], dcv[M];
  __shared__ float logd[L], el[L], dl[L];
  __shared__ float red[4];

  const int c = blockIdx.x, bh = blockIdx.y;
  const int T = a.f.T, H = a.f.H, D = a.f.D;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lg = lane >> 4;
  const int t0 = c * L;
  const Rows<X> q{(const X*)a.f.q, b, h, T, H, D}, dO{(const X*)a.d_out, b, h, T, H, D};
  const Rows<X> kk{(const X*)a.f.k, b, h, T, H, D}, ks{(const X*)a.f.sparse_k, b, h, T, H, D};
  const Rows<X> vv{(const X*)a.f.v, b, h, T, H, D}, vs{(const X*)a.f.sparse_v, b, h, T, H, D};
  auto kap = [&](int i, int d) __attribute__((always_inline)) {
    const int tl = SP ? (i >> 1) : i;
    return (SP && (i & 1)) ? ks(t0 + tl, d) : kk(t0 + tl, d);
  };
  auto nu = [&](int i, int d) __attribute__((always_inline)) {
    const int tl = SP ? (i >> 1) : i;
    return (SP && (i & 1)) ? vs(t0 + tl, d) : vv(t0 + tl, d);
  };
  auto tau = [](int i) { return SP ? (i >> 1) : i; };

  const long cb = (long)bh * NT + c;
  const float* S = Hs + cb * DP * DP;      // [DP][DP] chunk-start state
  const float* G = Gend + cb * DP * DP;    // [DP][DP] state gradient at the chunk end
  const float* R = Rg + cb * M * DP;       // [M][DP]
  const float* dR = dRg + cb * M * DP;     // [M][DP]
  const float* A = Ag + cb * M * M;        // [M][M]
  // per-chunk workspace: Y [L][M], dW [M][DP], Z [M][DP], dA [M][M], Tm [M][M], Xm [M][M]
  float* Y = scr + cb * (size_t)(L * M + 2 * M * DP + 3 * M * M);
  float* dW = Y + L * M;
  float* Z = dW + M * DP;
  float* dA = Z + M * DP;
  float* Tm = dA + M * M;
  float* Xm = Tm + M * M;

  if (tid < L) {
    const float x = lgd[cb * L + tid];
    logd[tid] = x;
    el[tid] = expf(x);
    dl[tid] = 0.f;
  }
  __syncthreads();
  if (tid < M) {
    const int tl = tau(tid);
    const int r = SP ? (tid & 1) : 0;
    const int t = t0 + tl;
    float lm = 0.f;
    if (t < T) lm = r ? a.f.alpha[(long)(b * T + t) * H + h] : a.f.beta[(long)(b * T + t) * H + h];
    lam[tid] = lm;
    cf[tid] = lm * expf(logd[L - 1] - logd[tl]);
    etau[tid] = el[tl];
    dlam[tid] = 0.f;
    dcv[tid] = 0.f;
  }
  __syncthreads();

  // P1: Y, and the P-terms of dlambda and dl
  for (int tile = w; tile < (L / 16) * (M / 16); tile += 4) {
    const int I = tile / (M / 16), J = tile % (M / 16);
    const f4 qk = mm(f4_zero(), DP, [&](int r, int k) { return q(t0 + 16 * I + r, k); },
                     [&](int k, int cc) { return kap(16 * J + cc, k); });
    const f4 dp = mm(f4_zero(), DP, [&](int r, int k) { return dO(t0 + 16 * I + r, k); },
                     [&](int k, int cc) { return R[(long)(16 * J + cc) * DP + k]; });
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * I + 4 * lg + e, i = 16 * J + (lane & 15);
      const int ti = tau(i);
      const float E = ti <= t ? expf(logd[t] - logd[ti]) : 0.f;
      Y[t * M + i] = dp[e] * E * lam[i];
      atomicAdd(&dlam[i], dp[e] * E * qk[e]);
      const float v = dp[e] * E * lam[i] * qk[e];
      atomicAdd(&dl[t], v);
      atomicAdd(&dl[ti], -v);
    }
  }
  // P2: dW = -dR S^T, and dnu = A^T dR (the v / v-hat gradients)
  X* dvo = (X*)a.dv;
  X* dsvo = (X*)a.dsv;
  for (int tile = w; tile < (M / 16) * (DP / 16); tile += 4) {
    const int I = tile / (DP / 16), J = tile % (DP / 16);
    const f4 x = mm(f4_zero(), DP, [&](int r, int k) { return dR[(long)(16 * I + r) * DP + k]; },
                    [&](int k, int cc) { return S[(long)(16 * J + cc) * DP + k]; });
    const f4 y = mm(f4_zero(), M, [&](int r, int k) { return A[(long)k * M + 16 * I + r]; },
                    [&](int k, int cc) { return dR[(long)k * DP + 16 * J + cc]; });
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * I + 4 * lg + e, d = 16 * J + (lane & 15);
      dW[(long)i * DP + d] = -x[e];
      const int t = t0 + tau(i);
      if (t < T && d < D) {
        X* o = (SP && (i & 1)) ? dsvo : dvo;
        st(o, ((long)(b * T + t) * H + h) * D + d, y[e]);
      }
    }
  }
  __syncthreads();
  // P3: Z = A^T dW; dl_tau += e^l_tau kappa . Z
  for (int tile = w; tile < (M / 16) * (DP / 16); tile += 4) {
    const int I = tile / (DP / 16), J = tile % (DP / 16);
    const f4 z = mm(f4_zero(), M, [&](int r, int k) { return A[(long)k * M + 16 * I + r]; },
                    [&](int k, int cc) { return dW[(long)k * DP + 16 * J + cc]; });
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * I + 4 * lg + e, d = 16 * J + (lane & 15);
      Z[(long)i * DP + d] = z[e];
      atomicAdd(&dl[tau(i)], etau[i] * kap(i, d) * z[e]);
    }
  }
  // P4: dA = dR nu^T + dW (diag(e^l_tau) kappa)^T
  for (int tile = w; tile < (M / 16) * (M / 16); tile += 4) {
    const int I = tile / (M / 16), J = tile % (M / 16);
    f4 x = mm(f4_zero(), DP, [&](int r, int k) { return dR[(long)(16 * I + r) * DP + k]; },
              [&](int k, int cc) { return nu(16 * J + cc, k); });
    x = mm(x, DP, [&](int r, int k) { return dW[(long)(16 * I + r) * DP + k]; },
           [&](int k, int cc) { return etau[16 * J + cc] * kap(16 * J + cc, k); });
#pragma unroll
    for (int e = 0; e < 4; ++e) dA[(long)(16 * I + 4 * lg + e) * M + 16 * J + (lane & 15)] = x[e];
  }
  __syncthreads();
  // P5: Tm = dA A^T
  for (int tile = w; tile < (M / 16) * (M / 16); tile += 4) {
    const int I = tile / (M / 16), J = tile % (M / 16);
    const f4 x = mm(f4_zero(), M, [&](int r, int k) { return dA[(long)(16 * I + r) * M + k]; },
                    [&](int k, int cc) { return A[(long)(16 * J + cc) * M + k]; });
#pragma unroll
    for (int e = 0; e < 4; ++e) Tm[(long)(16 * I + 4 * lg + e) * M + 16 * J + (lane & 15)] = x[e];
  }
  __syncthreads();
  // P6: dT = -A^T Tm; X = dT on the strictly lower token blocks, times the decay
  // ratio; the T-terms of dlambda and dl
  for (int tile = w; tile < (M / 16) * (M / 16); tile += 4) {
    const int I = tile / (M / 16), J = tile % (M / 16);
    const f4 dt = mm(f4_zero(), M, [&](int r, int k) { return A[(long)k * M + 16 * I + r]; },
                     [&](int k, int cc) { return Tm[(long)k * M + 16 * J + cc]; });
    const f4 gk = mm(f4_zero(), DP, [&](int r, int k) { return kap(16 * I + r, k); },
                     [&](int k, int cc) { return kap(16 * J + cc, k); });
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * I + 4 * lg + e, j = 16 * J + (lane & 15);
      const int ti = tau(i), tj = tau(j);
      const float x = tj < ti ? -dt[e] * expf(logd[ti] - logd[tj]) : 0.f;
      Xm[(long)i * M + j] = x;
      const float xg = x * gk[e];
      atomicAdd(&dlam[j], xg);
      atomicAdd(&dl[ti], xg * lam[j]);
      atomicAdd(&dl[tj], -xg * lam[j]);
    }
  }
  __syncthreads();
  // P7: dkappa (the k / k-tilde gradients) and dc = (kappa G) . R
  X* dko = (X*)a.dk;
  X* dsko = (X*)a.dsk;
  for (int tile = w; tile < (M / 16) * (DP / 16); tile += 4) {
    const int I = tile / (DP / 16), J = tile % (DP / 16);
    f4 x = mm(f4_zero(), L, [&](int r, int k) { return Y[(long)k * M + 16 * I + r]; },
              [&](int k, int cc) { return q(t0 + k, 16 * J + cc); });
    const f4 rg = mm(f4_zero(), DP, [&](int r, int k) { return R[(long)(16 * I + r) * DP + k]; },
                     [&](int k, int cc) { return G[(long)(16 * J + cc) * DP + k]; });
    x = mm(x, M, [&](int r, int k) { return Xm[(long)(16 * I + r) * M + k] * lam[k]; },
           [&](int k, int cc) { return kap(k, 16 * J + cc); });
    const f4 xt = mm(f4_zero(), M, [&](int r, int k) { return Xm[(long)k * M + 16 * I + r]; },
                     [&](int k, int cc) { return kap(k, 16 * J + cc); });
    const f4 kg = mm(f4_zero(), DP, [&](int r, int k) { return kap(16 * I + r, k); },
                     [&](int k, int cc) { return G[(long)k * DP + 16 * J + cc]; });
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * I + 4 * lg + e, d = 16 * J + (lane & 15);
      const float g = x[e] + cf[i] * rg[e] + etau[i] * Z[(long)i * DP + d] + lam[i] * xt[e];
      const int t = t0 + tau(i);
      if (t < T && d < D) {
        X* o = (SP && (i & 1)) ? dsko : dko;
        st(o, ((long)(b * T + t) * H + h) * D + d, g);
      }
      atomicAdd(&dcv[i], kg[e] * R[(long)i * DP + d]);
    }
  }
  // P8: dq = diag(e^l) dO S^T + Y kappa; dl_t += e^l_t q_t . (S dO_t)
  X* dqo = (X*)a.dq;
  for (int tile = w; tile < (L / 16) * (DP / 16); tile += 4) {
    const int I = tile / (DP / 16), J = tile % (DP / 16);
    const f4 ds = mm(f4_zero(), DP, [&](int r, int k) { return dO(t0 + 16 * I + r, k); },
                     [&](int k, int cc) { return S[(long)(16 * J + cc) * DP + k]; });
    const f4 yk = mm(f4_zero(), M, [&](int r, int k) { return Y[(long)(16 * I + r) * M + k]; },
                     [&](int k, int cc) { return kap(k, 16 * J + cc); });
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int tl = 16 * I + 4 * lg + e, d = 16 * J + (lane & 15);
      const int t = t0 + tl;
      if (t < T && d < D) st(dqo, ((long)(b * T + t) * H + h) * D + d, el[tl] * ds[e] + yk[e]);
      atomicAdd(&dl[tl], el[tl] * q(t, d) * ds[e]);
    }
  }
  // P9: <G, S>
  float gs = 0.f;
  for (int e = tid; e < DP * DP; e += 256) gs += G[e] * S[e];
  gs = wave_sum(gs);
  if (lane == 0) red[w] = gs;
  __syncthreads();
  if (tid == 0) dl[L - 1] += el[L - 1] * (red[0] + red[1] + red[2] + red[3]);
  __syncthreads();
  if (tid < M) {   // the c-terms
    const int ti = tau(tid);
    const float dc = dcv[tid];
    atomicAdd(&dl[L - 1], dc * cf[tid]);
    atomicAdd(&dl[ti], -dc * cf[tid]);
    dlam[tid] += dc * expf(logd[L - 1] - logd[ti]);
  }
  __syncthreads();
  // P10: dgamma from the suffix sums of dl; dbeta / dalpha from dlambda
  if (tid < L) {
    float sfx = 0.f;
    for (int t = L - 1; t >= tid; --t) sfx += dl[t];
    const int t = t0 + tid;
    if (t < T) {
      const long o = (long)(b * T + t) * H + h;
      const float g = a.f.gamma[o];
      a.dgamma[o] = g >= 1e-6f ? sfx / g : 0.f;
    }
  }
  if (tid < M) {
    const int t = t0 + tau(tid);
    if (t < T) {
      const long o = (long)(b * T + t) * H + h;
      if (SP && (tid & 1)) a.dalpha[o] = dlam[tid];
      else a.dbeta[o] = dlam[tid];
    }
  }
}

struct BwdWs {
  float *W, *U, *R, *Hs, *lgd, *A, *Gend, *dR, *scr;
};

BwdWs bwd_ws(void* base, int B, int T, int H, int sp) {
  const size_t NT = (T + L - 1) / L, M = sp ? 2 * L : L, BH = (size_t)B * H;
  auto al = [](char* p) { return (char*)(((uintptr_t)p + 255) & ~(uintptr_t)255); };
  char* p = al((char*)base);
  BwdWs w;
  w.W = (float*)p; p = al(p + 4 * BH * NT * M * DP);
  w.U = (float*)p; p = al(p + 4 * BH * NT * M * DP);
  w.R = (float*)p; p = al(p + 4 * BH * NT * M * DP);
  w.Hs = (float*)p; p = al(p + 4 * BH * NT * DP * DP);
  w.lgd = (float*)p; p = al(p + 4 * BH * NT * L);
  w.A = (float*)p; p = al(p + 4 * BH * NT * M * M);
  w.Gend = (float*)p; p = al(p + 4 * BH * NT * DP * DP);
  w.dR = (float*)p; p = al(p + 4 * BH * NT * M * DP);
  w.scr = (float*)p;
  return w;
}

template <typename X, bool SP>
hipError_t launch_bwd_t(const ChunkBwdArgs& a, const BwdWs& w, hipStream_t st) {
  const int NT = (a.f.T + L - 1) / L;
  const int BH = a.f.B * a.f.H;
  chunk_bwd_scan_kernel<X, SP><<<dim3(DP / 16, BH), 256, 0, st>>>(a, w.W, w.lgd, w.Gend, w.dR, NT);
  chunk_bwd_grad_kernel<X, SP><<<dim3(NT, BH), 256, 0, st>>>(a, w.R, w.Hs, w.lgd, w.A, w.Gend, w.dR, w.scr, NT);
  return hipGetLastError();
}

}  // namespace

size_t chunk_bwd_workspace_bytes(int B, int T, int H, int has_sparse) {
  const size_t NT = (T + L - 1) / L, M = has_sparse ? 2 * L : L, BH = (size_t)B * H;
  const size_t per = 4 * (4 * M * DP + 2 * DP * DP + L + M * M) + 6 * 256;
  const size_t scr = 4 * (L * M + 2 * M * DP + 3 * M * M);
  return BH * NT * (per + scr) + 256 * 12;
}

hipError_t launch_chunk_bwd(const ChunkBwdArgs& a, hipStream_t st) {
  const bool sp = a.f.sparse_k != nullptr;
  const BwdWs w = bwd_ws(a.workspace, a.f.B, a.f.T, a.f.H, sp);
  if (hipError_t e = launch_chunk_recompute(a.f, w.W, w.U, w.R, w.Hs, w.lgd, w.A, st)) return e;
  if (a.f.dtype == DT_BF16) return sp ? launch_bwd_t<bf16_t, true>(a, w, st) : launch_bwd_t<bf16_t, false>(a, w, st);
  return sp ? launch_bwd_t<float, true>(a, w, st) : launch_bwd_t<float, false>(a, w, st);
}

}  // namespace sgsa
