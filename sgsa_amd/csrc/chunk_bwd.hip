// Backward of the chunked SGSA forward on gfx950 (chunk_sgsa's gradient).
//
// The reference differentiates chunk_sgsa by recomputing the forward in torch
// under autograd (modelings/sgsa_ops/chunk_bwd.py:12-77; the plan of a kernel
// backward is modelings/sgsa_bwd_derivation.md:699-832).  Here the gradient of
// the chunk form is written out and run on fp32 MFMA, for bf16 or fp32 inputs:
//
//   1. chunk_intra_kernel (chunk.hip): per chunk the WY inverse A = (I+T)^-1,
//      W = A diag(D_tau) kappa, U = A nu and the log-decay prefix l;
//   2. chunk_bwd_maps_kernel, parallel over chunks: the chunk's affine state
//      map S' = Phi S + Pm, Phi = e^l_L I - kappa^T diag(c) W,
//      Pm = kappa^T diag(c) U; a segmented scan (sscan_kernel) over the
//      chunks: the chunk-start states;
//   3. chunk_bwd_pre_kernel, parallel: X1 = P^T dO and the state-independent
//      part of the state gradient's step, Y2 = Q^T diag(e^l) dO - W^T X1;
//      a segmented scan from the last chunk: the state gradient at every
//      chunk end, G <- Phi^T G + Y2 (Phi^T = e^l_L I - W^T diag(c) kappa is
//      the adjoint of the state map);
//   4. chunk_bwd_grad_kernel, parallel over chunks: every input gradient of a
//      chunk from its start state S, its end gradient G and its inputs.
//
// Per chunk (tokens t, samples i at token tau_i, M = 2L samples with the
// sparse write, lambda = beta / alpha per sample):
//
//   P_ti = 1[tau_i <= t] exp(l_t - l_tau_i) lambda_i (q_t . kappa_i)
//   c_i  = lambda_i exp(l_L - l_tau_i),   l_L the chunk's last prefix
//   R    = U - W S,   o = diag(e^l) Q S + P R,   S' = e^l_L S + kappa^T diag(c) R
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
// The intermediates of stage 4 go through a per-chunk workspace (L2 traffic).
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

constexpr int PIT = DP + 4;   // LDS row pitch (floats)
// Waves per workgroup of the per-chunk kernels (maps, pre, grad), whose LDS
// allows one workgroup per CU.
constexpr int GW = 8;

// One 16 x 16 output tile over K (a multiple of 32) with the sum taken four k at
// a time per lane: lane (r, g) of the MFMA takes k = k0 + 4g + j in the j-th of
// four products, so fa4(r, k) / fb4(k, c) return the four consecutive k from k
// (a float4 load where the operand is contiguous along k).  Two accumulators,
// for the k-groups at k0 and k0 + 16, keep two MFMA chains in flight.
template <typename FA, typename FB>
__device__ __forceinline__ f4 mm4(f4 acc, int K, FA&& fa4, FB&& fb4) {
  const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
  f4 acc1 = f4_zero();
  for (int k0 = 0; k0 < K; k0 += 32) {
    const float4 a0 = fa4(lr, k0 + 4 * lg), b0 = fb4(k0 + 4 * lg, lr);
    const float4 a1 = fa4(lr, k0 + 16 + 4 * lg), b1 = fb4(k0 + 16 + 4 * lg, lr);
    acc = mma_f32(a0.x, b0.x, acc);
    acc1 = mma_f32(a1.x, b1.x, acc1);
    acc = mma_f32(a0.y, b0.y, acc);
    acc1 = mma_f32(a1.y, b1.y, acc1);
    acc = mma_f32(a0.z, b0.z, acc);
    acc1 = mma_f32(a1.z, b1.z, acc1);
    acc = mma_f32(a0.w, b0.w, acc);
    acc1 = mma_f32(a1.w, b1.w, acc1);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] += acc1[e];
  return acc;
}
// p[r][k..k+3] (contiguous) and p[k..k+3][c] (a column), for row pitch n
__device__ __forceinline__ float4 rowv(const float* p, int n, int r, int k) {
  return *reinterpret_cast<const float4*>(p + (long)r * n + k);
}
__device__ __forceinline__ float4 colv(const float* p, int n, int k, int c) {
  const float* q = p + (long)k * n + c;
  return make_float4(q[0], q[n], q[2 * n], q[3 * n]);
}


// Stage 2a, parallel over chunks: Phi = e^l_L I - kappa^T diag(c) W and
// Pm = kappa^T diag(c) U, [DP][DP] each.  grid (NT, B*H), GW waves.
template <typename X, bool SP>
__global__ __launch_bounds__(64 * GW) void chunk_bwd_maps_kernel(ChunkBwdArgs a, const float* __restrict__ Wg,
                                                             const float* __restrict__ Ug,
                                                             const float* __restrict__ lgd,
                                                             float* __restrict__ Phig, float* __restrict__ Pmg,
                                                             int NT) {
  constexpr int M = SP ? 2 * L : L;
  __shared__ float kps[M][PIT];   // c_i kappa_i
  __shared__ float ws[M][PIT];    // W, then U
  const int c = blockIdx.x, bh = blockIdx.y;
  const int T = a.f.T, H = a.f.H, D = a.f.D;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lg = lane >> 4;
  const int t0 = c * L;
  const long cb = (long)bh * NT + c;
  const Rows<X> kk{(const X*)a.f.k, b, h, T, H, D}, ks{(const X*)a.f.sparse_k, b, h, T, H, D};
  const float* lg_c = lgd + cb * L;
  const float lL = lg_c[L - 1];
  for (int e = tid; e < M * DP; e += 64 * GW) {
    const int i = e / DP, d = e % DP;
    const int tl = SP ? (i >> 1) : i;
    const int t = t0 + tl;
    float lm = 0.f;
    if (t < T) lm = (SP && (i & 1)) ? a.f.alpha[(long)(b * T + t) * H + h] : a.f.beta[(long)(b * T + t) * H + h];
    const float ci = lm * expf(lL - lg_c[tl]);
    kps[i][d] = ci * ((SP && (i & 1)) ? ks(t, d) : kk(t, d));
    ws[i][d] = Wg[cb * M * DP + e];
  }
  __syncthreads();
  const float eL = expf(lL);
  float* Phi = Phig + cb * DP * DP;
  for (int tile = w; tile < (DP / 16) * (DP / 16); tile += GW) {
    const int I = tile / (DP / 16), J = tile % (DP / 16);
    const f4 x = mm4(f4_zero(), M, [&](int r, int k) { return colv(&kps[0][0], PIT, k, 16 * I + r); },
                     [&](int k, int cc) { return colv(&ws[0][0], PIT, k, 16 * J + cc); });
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = 16 * I + 4 * lg + e, cc = 16 * J + (lane & 15);
      Phi[(long)r * DP + cc] = (r == cc ? eL : 0.f) - x[e];
    }
  }
  __syncthreads();
  for (int e = tid; e < M * DP; e += 64 * GW) ws[e / DP][e % DP] = Ug[cb * M * DP + e];
  __syncthreads();
  float* Pm = Pmg + cb * DP * DP;
  for (int tile = w; tile < (DP / 16) * (DP / 16); tile += GW) {
    const int I = tile / (DP / 16), J = tile % (DP / 16);
    const f4 x = mm4(f4_zero(), M, [&](int r, int k) { return colv(&kps[0][0], PIT, k, 16 * I + r); },
                     [&](int k, int cc) { return colv(&ws[0][0], PIT, k, 16 * J + cc); });
#pragma unroll
    for (int e = 0; e < 4; ++e) Pm[(long)(16 * I + 4 * lg + e) * DP + 16 * J + (lane & 15)] = x[e];
  }
}

// Stage 3a, parallel over chunks: X1 = P^T dO [M][DP] and the state-independent
// part of the state gradient's step, Y2 = Q^T diag(e^l) dO - W^T X1 [DP][DP].
// grid (NT, B*H), GW waves; q, kappa, dO staged in LDS as fp32.
template <typename X, bool SP>
__global__ __launch_bounds__(64 * GW) void chunk_bwd_pre_kernel(ChunkBwdArgs a, const float* __restrict__ Wg,
                                                            const float* __restrict__ lgd,
                                                            float* __restrict__ X1g, float* __restrict__ Y2g,
                                                            int NT) {
  constexpr int M = SP ? 2 * L : L;
  __shared__ __align__(16) float qs[L][PIT];    // q, later P
  __shared__ __align__(16) float kps[M][PIT];
  __shared__ __align__(16) float dos[L][PIT];
  __shared__ float lam[M], logd[L], el[L];

  const int c = blockIdx.x, bh = blockIdx.y;
  const int T = a.f.T, H = a.f.H, D = a.f.D;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lg = lane >> 4;
  const int t0 = c * L;
  const long cb = (long)bh * NT + c;
  const Rows<X> q{(const X*)a.f.q, b, h, T, H, D}, dO{(const X*)a.d_out, b, h, T, H, D};
  const Rows<X> kk{(const X*)a.f.k, b, h, T, H, D}, ks{(const X*)a.f.sparse_k, b, h, T, H, D};
  for (int e = tid; e < L * DP; e += 64 * GW) {
    const int t = e / DP, d = e % DP;
    qs[t][d] = q(t0 + t, d);
    dos[t][d] = dO(t0 + t, d);
  }
  for (int e = tid; e < M * DP; e += 64 * GW) {
    const int i = e / DP, d = e % DP;
    const int tl = SP ? (i >> 1) : i;
    kps[i][d] = (SP && (i & 1)) ? ks(t0 + tl, d) : kk(t0 + tl, d);
  }
  if (tid < L) {
    const float x = lgd[cb * L + tid];
    logd[tid] = x;
    el[tid] = expf(x);
  }
  if (tid < M) {
    const int tl = SP ? (tid >> 1) : tid;
    const int r = SP ? (tid & 1) : 0;
    const int t = t0 + tl;
    float lm = 0.f;
    if (t < T) lm = r ? a.f.alpha[(long)(b * T + t) * H + h] : a.f.beta[(long)(b * T + t) * H + h];
    lam[tid] = lm;
  }
  __syncthreads();
  // P (registers, then over q)
  constexpr int NPT = (L / 16) * (M / 16) / GW;   // tiles per wave
  f4 pt[NPT];
#pragma unroll
  for (int u = 0; u < NPT; ++u) {
    const int tile = w + GW * u, I = tile / (M / 16), J = tile % (M / 16);
    const f4 x = mm4(f4_zero(), DP, [&](int r, int k) { return rowv(&qs[0][0], PIT, 16 * I + r, k); },
                     [&](int k, int cc) { return rowv(&kps[0][0], PIT, 16 * J + cc, k); });
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * I + 4 * lg + e, i = 16 * J + (lane & 15);
      const int ti = SP ? (i >> 1) : i;
      pt[u][e] = ti <= t ? expf(logd[t] - logd[ti]) * lam[i] * x[e] : 0.f;
    }
  }
  // Y2 = Q^T diag(e^l) dO first (q is still in qs)
  float* Y2 = Y2g + cb * DP * DP;
  for (int tile = w; tile < (DP / 16) * (DP / 16); tile += GW) {
    const int I = tile / (DP / 16), J = tile % (DP / 16);
    const f4 x = mm4(f4_zero(), L,
                     [&](int r, int k) {
                       const float4 v = colv(&qs[0][0], PIT, k, 16 * I + r);
                       return make_float4(v.x * el[k], v.y * el[k + 1], v.z * el[k + 2], v.w * el[k + 3]);
                     },
                     [&](int k, int cc) { return colv(&dos[0][0], PIT, k, 16 * J + cc); });
#pragma unroll
    for (int e = 0; e < 4; ++e) Y2[(long)(16 * I + 4 * lg + e) * DP + 16 * J + (lane & 15)] = x[e];
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < NPT; ++u) {
    const int tile = w + GW * u, I = tile / (M / 16), J = tile % (M / 16);
#pragma unroll
    for (int e = 0; e < 4; ++e) qs[16 * I + 4 * lg + e][16 * J + (lane & 15)] = pt[u][e];
  }
  __syncthreads();
  // X1 = P^T dO, kept in LDS (over kappa) for W^T X1
  float* X1 = X1g + cb * M * DP;
  for (int tile = w; tile < (M / 16) * (DP / 16); tile += GW) {
    const int I = tile / (DP / 16), J = tile % (DP / 16);
    const f4 x = mm4(f4_zero(), L, [&](int r, int k) { return colv(&qs[0][0], PIT, k, 16 * I + r); },
                     [&](int k, int cc) { return colv(&dos[0][0], PIT, k, 16 * J + cc); });
#pragma unroll
    for (int e = 0; e < 4; ++e) X1[(long)(16 * I + 4 * lg + e) * DP + 16 * J + (lane & 15)] = x[e];
  }
  __syncthreads();
  for (int e = tid; e < M * DP; e += 64 * GW) kps[e / DP][e % DP] = X1[e];
  __syncthreads();
  // Y2 -= W^T X1
  const float* Wc = Wg + cb * M * DP;
  for (int tile = w; tile < (DP / 16) * (DP / 16); tile += GW) {
    const int I = tile / (DP / 16), J = tile % (DP / 16);
    const f4 x = mm4(f4_zero(), M, [&](int r, int k) { return colv(Wc, DP, k, 16 * I + r); },
                     [&](int k, int cc) { return colv(&kps[0][0], PIT, k, 16 * J + cc); });
#pragma unroll
    for (int e = 0; e < 4; ++e) Y2[(long)(16 * I + 4 * lg + e) * DP + 16 * J + (lane & 15)] -= x[e];
  }
}

// Stage 4.  grid (NT, B*H), GW waves: every gradient of one chunk.  kappa, q
// and dO stay in LDS as fp32 for the whole kernel; the other operands are
// read from the workspace (L2).
template <typename X, bool SP>
__global__ __launch_bounds__(64 * GW) void chunk_bwd_grad_kernel(ChunkBwdArgs a, const float* __restrict__ Wg,
                                                             const float* __restrict__ Ug,
                                                             const float* __restrict__ X1g,
                                                             const float* __restrict__ Hs,
                                                             const float* __restrict__ lgd,
                                                             const float* __restrict__ Ag,
                                                             const float* __restrict__ Gend, float* __restrict__ scr,
                                                             int NT) {
  constexpr int M = SP ? 2 * L : L;
  __shared__ __align__(16) float kps[M][PIT];
  __shared__ __align__(16) float qs[L][PIT];
  __shared__ __align__(16) float dos[L][PIT];
  __shared__ float lam[M], cf[M], etau[M], dlam[M], dcv[M];
  __shared__ float logd[L], el[L], dl[L];
  __shared__ float red[GW];

  const int c = blockIdx.x, bh = blockIdx.y;
  const int T = a.f.T, H = a.f.H, D = a.f.D;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lg = lane >> 4;
  const int t0 = c * L;
  const Rows<X> q{(const X*)a.f.q, b, h, T, H, D}, dO{(const X*)a.d_out, b, h, T, H, D};
  const Rows<X> kk{(const X*)a.f.k, b, h, T, H, D}, ks{(const X*)a.f.sparse_k, b, h, T, H, D};
  const Rows<X> vv{(const X*)a.f.v, b, h, T, H, D}, vs{(const X*)a.f.sparse_v, b, h, T, H, D};
  auto nu4 = [&](int i, int d) __attribute__((always_inline)) {   // nu[i][d..d+3]
    const int tl = SP ? (i >> 1) : i;
    const Rows<X>& src = (SP && (i & 1)) ? vs : vv;
    return make_float4(src(t0 + tl, d), src(t0 + tl, d + 1), src(t0 + tl, d + 2), src(t0 + tl, d + 3));
  };
  auto tau = [](int i) { return SP ? (i >> 1) : i; };
  const float* KS = &kps[0][0];
  const float* QS = &qs[0][0];
  const float* DS = &dos[0][0];

  const long cb = (long)bh * NT + c;
  const float* S = Hs + cb * DP * DP;      // [DP][DP] chunk-start state
  const float* G = Gend + cb * DP * DP;    // [DP][DP] state gradient at the chunk end
  const float* A = Ag + cb * M * M;        // [M][M]
  // per-chunk workspace: R, dR, dW, Z [M][DP], Y [L][M], dA, Tm, Xm [M][M]
  float* R = scr + cb * (size_t)(L * M + 4 * M * DP + 3 * M * M);
  float* dR = R + M * DP;
  float* dW = dR + M * DP;
  float* Z = dW + M * DP;
  float* Y = Z + M * DP;
  float* dA = Y + L * M;
  float* Tm = dA + M * M;
  float* Xm = Tm + M * M;

  for (int e = tid; e < L * DP; e += 64 * GW) {
    const int t = e / DP, d = e % DP;
    qs[t][d] = q(t0 + t, d);
    dos[t][d] = dO(t0 + t, d);
  }
  for (int e = tid; e < M * DP; e += 64 * GW) {
    const int i = e / DP, d = e % DP;
    const int tl = tau(i);
    kps[i][d] = (SP && (i & 1)) ? ks(t0 + tl, d) : kk(t0 + tl, d);
  }
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

  // P0: R = U - W S and dR = X1 + diag(c) kappa G
  {
    const float* Wc = Wg + cb * M * DP;
    const float* Uc = Ug + cb * M * DP;
    const float* X1 = X1g + cb * M * DP;
    for (int tile = w; tile < (M / 16) * (DP / 16); tile += GW) {
      const int I = tile / (DP / 16), J = tile % (DP / 16);
      const f4 ws = mm4(f4_zero(), DP, [&](int r, int k) { return rowv(Wc, DP, 16 * I + r, k); },
                        [&](int k, int cc) { return colv(S, DP, k, 16 * J + cc); });
      const f4 kg = mm4(f4_zero(), DP, [&](int r, int k) { return rowv(KS, PIT, 16 * I + r, k); },
                        [&](int k, int cc) { return colv(G, DP, k, 16 * J + cc); });
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 16 * I + 4 * lg + e, d = 16 * J + (lane & 15);
        const long o = (long)i * DP + d;
        R[o] = Uc[o] - ws[e];
        dR[o] = X1[o] + cf[i] * kg[e];
      }
    }
  }
  __syncthreads();
  // P1: Y, and the P-terms of dlambda and dl
  for (int tile = w; tile < (L / 16) * (M / 16); tile += GW) {
    const int I = tile / (M / 16), J = tile % (M / 16);
    const f4 qk = mm4(f4_zero(), DP, [&](int r, int k) { return rowv(QS, PIT, 16 * I + r, k); },
                      [&](int k, int cc) { return rowv(KS, PIT, 16 * J + cc, k); });
    const f4 dp = mm4(f4_zero(), DP, [&](int r, int k) { return rowv(DS, PIT, 16 * I + r, k); },
                      [&](int k, int cc) { return rowv(R, DP, 16 * J + cc, k); });
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
  for (int tile = w; tile < (M / 16) * (DP / 16); tile += GW) {
    const int I = tile / (DP / 16), J = tile % (DP / 16);
    const f4 x = mm4(f4_zero(), DP, [&](int r, int k) { return rowv(dR, DP, 16 * I + r, k); },
                     [&](int k, int cc) { return rowv(S, DP, 16 * J + cc, k); });
    const f4 y = mm4(f4_zero(), M, [&](int r, int k) { return colv(A, M, k, 16 * I + r); },
                     [&](int k, int cc) { return colv(dR, DP, k, 16 * J + cc); });
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
  for (int tile = w; tile < (M / 16) * (DP / 16); tile += GW) {
    const int I = tile / (DP / 16), J = tile % (DP / 16);
    const f4 z = mm4(f4_zero(), M, [&](int r, int k) { return colv(A, M, k, 16 * I + r); },
                     [&](int k, int cc) { return colv(dW, DP, k, 16 * J + cc); });
    float part[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * I + 4 * lg + e, d = 16 * J + (lane & 15);
      Z[(long)i * DP + d] = z[e];
      part[e] = etau[i] * kps[i][d] * z[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {   // sum over the tile's 16 columns (the 16 lanes of a row)
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) part[e] += __shfl_xor(part[e], o, 64);
      if ((lane & 15) == 0) atomicAdd(&dl[tau(16 * I + 4 * lg + e)], part[e]);
    }
  }
  // P4: dA = dR nu^T + dW (diag(e^l_tau) kappa)^T
  for (int tile = w; tile < (M / 16) * (M / 16); tile += GW) {
    const int I = tile / (M / 16), J = tile % (M / 16);
    f4 x = mm4(f4_zero(), DP, [&](int r, int k) { return rowv(dR, DP, 16 * I + r, k); },
               [&](int k, int cc) { return nu4(16 * J + cc, k); });
    x = mm4(x, DP, [&](int r, int k) { return rowv(dW, DP, 16 * I + r, k); },
            [&](int k, int cc) {
              const float4 v = rowv(KS, PIT, 16 * J + cc, k);
              const float e = etau[16 * J + cc];
              return make_float4(e * v.x, e * v.y, e * v.z, e * v.w);
            });
#pragma unroll
    for (int e = 0; e < 4; ++e) dA[(long)(16 * I + 4 * lg + e) * M + 16 * J + (lane & 15)] = x[e];
  }
  __syncthreads();
  // P5: Tm = dA A^T
  for (int tile = w; tile < (M / 16) * (M / 16); tile += GW) {
    const int I = tile / (M / 16), J = tile % (M / 16);
    const f4 x = mm4(f4_zero(), M, [&](int r, int k) { return rowv(dA, M, 16 * I + r, k); },
                     [&](int k, int cc) { return rowv(A, M, 16 * J + cc, k); });
#pragma unroll
    for (int e = 0; e < 4; ++e) Tm[(long)(16 * I + 4 * lg + e) * M + 16 * J + (lane & 15)] = x[e];
  }
  __syncthreads();
  // P6: dT = -A^T Tm; X = dT on the strictly lower token blocks, times the decay
  // ratio; the T-terms of dlambda and dl
  for (int tile = w; tile < (M / 16) * (M / 16); tile += GW) {
    const int I = tile / (M / 16), J = tile % (M / 16);
    const f4 dt = mm4(f4_zero(), M, [&](int r, int k) { return colv(A, M, k, 16 * I + r); },
                      [&](int k, int cc) { return colv(Tm, M, k, 16 * J + cc); });
    const f4 gk = mm4(f4_zero(), DP, [&](int r, int k) { return rowv(KS, PIT, 16 * I + r, k); },
                      [&](int k, int cc) { return rowv(KS, PIT, 16 * J + cc, k); });
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
  for (int tile = w; tile < (M / 16) * (DP / 16); tile += GW) {
    const int I = tile / (DP / 16), J = tile % (DP / 16);
    f4 x = mm4(f4_zero(), L, [&](int r, int k) { return colv(Y, M, k, 16 * I + r); },
               [&](int k, int cc) { return colv(QS, PIT, k, 16 * J + cc); });
    const f4 rg = mm4(f4_zero(), DP, [&](int r, int k) { return rowv(R, DP, 16 * I + r, k); },
                      [&](int k, int cc) { return rowv(G, DP, 16 * J + cc, k); });
    x = mm4(x, M, [&](int r, int k) {
          const float4 v = rowv(Xm, M, 16 * I + r, k);
          return make_float4(v.x * lam[k], v.y * lam[k + 1], v.z * lam[k + 2], v.w * lam[k + 3]);
        },
        [&](int k, int cc) { return colv(KS, PIT, k, 16 * J + cc); });
    const f4 xt = mm4(f4_zero(), M, [&](int r, int k) { return colv(Xm, M, k, 16 * I + r); },
                      [&](int k, int cc) { return colv(KS, PIT, k, 16 * J + cc); });
    const f4 kg = mm4(f4_zero(), DP, [&](int r, int k) { return rowv(KS, PIT, 16 * I + r, k); },
                      [&](int k, int cc) { return colv(G, DP, k, 16 * J + cc); });
    float part[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * I + 4 * lg + e, d = 16 * J + (lane & 15);
      const float g = x[e] + cf[i] * rg[e] + etau[i] * Z[(long)i * DP + d] + lam[i] * xt[e];
      const int t = t0 + tau(i);
      if (t < T && d < D) {
        X* o = (SP && (i & 1)) ? dsko : dko;
        st(o, ((long)(b * T + t) * H + h) * D + d, g);
      }
      part[e] = kg[e] * R[(long)i * DP + d];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) part[e] += __shfl_xor(part[e], o, 64);
      if ((lane & 15) == 0) atomicAdd(&dcv[16 * I + 4 * lg + e], part[e]);
    }
  }
  // P8: dq = diag(e^l) dO S^T + Y kappa; dl_t += e^l_t q_t . (S dO_t)
  X* dqo = (X*)a.dq;
  for (int tile = w; tile < (L / 16) * (DP / 16); tile += GW) {
    const int I = tile / (DP / 16), J = tile % (DP / 16);
    const f4 ds = mm4(f4_zero(), DP, [&](int r, int k) { return rowv(DS, PIT, 16 * I + r, k); },
                      [&](int k, int cc) { return rowv(S, DP, 16 * J + cc, k); });
    const f4 yk = mm4(f4_zero(), M, [&](int r, int k) { return rowv(Y, M, 16 * I + r, k); },
                      [&](int k, int cc) { return colv(KS, PIT, k, 16 * J + cc); });
    float part[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int tl = 16 * I + 4 * lg + e, d = 16 * J + (lane & 15);
      const int t = t0 + tl;
      if (t < T && d < D) st(dqo, ((long)(b * T + t) * H + h) * D + d, el[tl] * ds[e] + yk[e]);
      part[e] = el[tl] * qs[tl][d] * ds[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) part[e] += __shfl_xor(part[e], o, 64);
      if ((lane & 15) == 0) atomicAdd(&dl[16 * I + 4 * lg + e], part[e]);
    }
  }
  // P9: <G, S>
  float gs = 0.f;
  for (int e = tid; e < DP * DP; e += 64 * GW) gs += G[e] * S[e];
  gs = wave_sum(gs);
  if (lane == 0) red[w] = gs;
  __syncthreads();
  if (tid == 0) {
    float r = 0.f;
#pragma unroll
    for (int i = 0; i < GW; ++i) r += red[i];
    dl[L - 1] += el[L - 1] * r;
  }
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

// ---------------------------------------------------------------------------
// Segmented scans of the state maps (the chunk-start states and the end-of-chunk
// state gradients).  x <- Phi_c x + Y_c over the chunks of a head (TR: Phi_c^T,
// in decreasing chunk order) is split into G segments of CPS chunks:
//   1. each segment's composed map, run from I without Y and from 0 with Y
//      (sscan_kernel over the segment's chunks, all segments in parallel);
//   2. the segment-level scan over those G maps from the initial state, which
//      gives every segment's entering state;
//   3. every segment rerun from its entering state, writing x before each chunk.
// That takes 2 CPS + G dependent steps instead of NT.  A block (512 threads)
// holds the whole DP x DP state, wave w its 16-column tile in the accumulator
// layout (32 VGPRs), so each Phi_c is read once per step; the product runs on
// v_mfma_f32_16x16x4_f32 with Phi_c staged in LDS from registers loaded one step
// ahead and the wave's columns of x staged as the B operand.
// ---------------------------------------------------------------------------
struct SScanArgs {
  const float* phi;   // [BH][NP][DP][DP] row-major
  const float* y;     // same layout, or nullptr
  int NP, CPS, G;
  int init_mode;      // 0: zero, 1: identity, 2: per segment [BH][G][DP][DP], 3: [BH][D][D] (zero past D)
  const float* init;
  int D;
  float* out;         // [BH][NP][DP][DP]: x before each step, or nullptr
  int last_mode;      // 0: none, 1: per segment [BH][G][DP][DP], 2: [BH][D][D] from the scan's last segment
  float* last;
};

template <bool TR, bool INC>
__global__ __launch_bounds__(512) void sscan_kernel(SScanArgs a) {
  constexpr int NW = 8;
  constexpr int EPT = DP * DP / (64 * NW) / 4;   // float4 of Phi per thread
  constexpr int MB = DP * DP * 4;                // bytes of one matrix
  __shared__ __align__(16) float ph[DP][PIT];
  __shared__ float xs[NW][DP][17];
  const int z = blockIdx.x, bh = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int col = 16 * w + lr;
  const int cbeg = z * a.CPS, cend = min(a.NP, cbeg + a.CPS);
  const int nst = cend - cbeg;
  // element (16 rt + 4 lg + e, col) of a matrix: byte offset xoff + 4 DP (16 rt + e), the
  // row part a compile-time constant (scalar offsets of buffer loads and stores)
  const int xoff = 4 * (4 * lg * DP + col);
  auto rsrc = [](const float* base) __attribute__((always_inline)) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, MB, 0x00020000);
  };

  f4 x[DP / 16];
  {
    const bool seg_in = a.init_mode == 2;
    const auto ir = rsrc(seg_in ? a.init + ((long)bh * a.G + z) * DP * DP : a.phi);
#pragma unroll
    for (int rt = 0; rt < DP / 16; ++rt) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * rt + 4 * lg + e;
        float v = 0.f;
        if (a.init_mode == 1) v = row == col ? 1.f : 0.f;
        else if (seg_in) v = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ir, xoff, 4 * DP * (16 * rt + e), 0));
        else if (a.init_mode == 3) v = (row < a.D && col < a.D) ? a.init[((long)bh * a.D + row) * a.D + col] : 0.f;
        x[rt][e] = v;
      }
    }
  }
  uint4 pf[EPT];
  auto prefetch = [&](int c) __attribute__((always_inline)) {
    const auto pr = rsrc(a.phi + ((long)bh * a.NP + c) * DP * DP);
#pragma unroll
    for (int u = 0; u < EPT; ++u) pf[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(pr, 16 * tid, 16 * 64 * NW * u, 0));
  };
  if (nst > 0) prefetch(INC ? cbeg : cend - 1);
  for (int s = 0; s < nst; ++s) {
    const int c = INC ? cbeg + s : cend - 1 - s;
    const long cb = (long)bh * a.NP + c;
#pragma unroll
    for (int u = 0; u < EPT; ++u) {
      const int e4 = tid + 64 * NW * u, r = (4 * e4) / DP, c0 = (4 * e4) % DP;
      *reinterpret_cast<uint4*>(&ph[r][c0]) = pf[u];
    }
#pragma unroll
    for (int rt = 0; rt < DP / 16; ++rt) {
#pragma unroll
      for (int e = 0; e < 4; ++e) xs[w][16 * rt + 4 * lg + e][lr] = x[rt][e];
    }
    if (a.out != nullptr) {   // block-uniform
      float* ob = a.out + cb * DP * DP + (long)(4 * lg) * DP + col;
#pragma unroll
      for (int rt = 0; rt < DP / 16; ++rt) {
#pragma unroll
        for (int e = 0; e < 4; ++e) ob[(16 * rt + e) * DP] = x[rt][e];
      }
    }
    __syncthreads();
    if (s + 1 < nst) prefetch(INC ? c + 1 : c - 1);
    const bool hy = a.y != nullptr;
    const auto yr = rsrc(hy ? a.y + cb * DP * DP : a.phi);
#pragma unroll
    for (int rt = 0; rt < DP / 16; ++rt) {
      f4 acc0 = f4_zero(), acc1 = f4_zero();
#pragma unroll 1
      for (int k0 = 0; k0 < DP; k0 += 32) {
        float av0[4], av1[4];
        if constexpr (TR) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            av0[j] = ph[k0 + 4 * lg + j][16 * rt + lr];
            av1[j] = ph[k0 + 16 + 4 * lg + j][16 * rt + lr];
          }
        } else {
          const float4 p0 = *reinterpret_cast<const float4*>(&ph[16 * rt + lr][k0 + 4 * lg]);
          const float4 p1 = *reinterpret_cast<const float4*>(&ph[16 * rt + lr][k0 + 16 + 4 * lg]);
          av0[0] = p0.x; av0[1] = p0.y; av0[2] = p0.z; av0[3] = p0.w;
          av1[0] = p1.x; av1[1] = p1.y; av1[2] = p1.z; av1[3] = p1.w;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc0 = mma_f32(av0[j], xs[w][k0 + 4 * lg + j][lr], acc0);
          acc1 = mma_f32(av1[j], xs[w][k0 + 16 + 4 * lg + j][lr], acc1);
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float yv = hy ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(yr, xoff, 4 * DP * (16 * rt + e), 0)) : 0.f;
        x[rt][e] = acc0[e] + acc1[e] + yv;
      }
    }
    __syncthreads();   // ph is restaged by the next step
  }
  const bool final_seg = INC ? z == a.G - 1 : z == 0;
  if (a.last_mode == 1 || (a.last_mode == 2 && final_seg)) {
#pragma unroll
    for (int rt = 0; rt < DP / 16; ++rt) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * rt + 4 * lg + e;
        if (a.last_mode == 1) a.last[((long)bh * a.G + z) * DP * DP + (long)row * DP + col] = x[rt][e];
        else if (row < a.D && col < a.D) a.last[((long)bh * a.D + row) * a.D + col] = x[rt][e];
      }
    }
  }
}

// Segments of a head's NT chunks for the segmented scans: up to 16 of at least 8 chunks.
inline void sscan_segments(int NT, int& G, int& CPS) {
  G = NT / 8 < 16 ? NT / 8 : 16;
  if (G < 1) G = 1;
  CPS = (NT + G - 1) / G;
  G = (NT + CPS - 1) / CPS;
}

// One scan (TR, INC as above) by the three launches; seg: 3 x [BH][G][DP][DP] floats.
template <bool TR, bool INC>
hipError_t launch_sscan(const float* phi, const float* y, int BH, int NT, const float* init, int D, float* out,
                        float* last, float* seg, hipStream_t st) {
  int G, CPS;
  sscan_segments(NT, G, CPS);
  const size_t segsz = (size_t)BH * G * DP * DP;
  float* smap = seg;               // the segments' composed maps (from I, no Y)
  float* soff = seg + segsz;       // their offsets (from 0, with Y)
  float* sin = seg + 2 * segsz;    // the segments' entering states
  const dim3 gs(G, BH), g1(1, BH);
  SScanArgs a{};
  a.phi = phi; a.NP = NT; a.CPS = CPS; a.G = G; a.D = D;
  // 1. composed maps and offsets
  a.y = nullptr; a.init_mode = 1; a.init = nullptr; a.out = nullptr; a.last_mode = 1; a.last = smap;
  sscan_kernel<TR, INC><<<gs, 512, 0, st>>>(a);
  a.y = y; a.init_mode = 0; a.last = soff;
  sscan_kernel<TR, INC><<<gs, 512, 0, st>>>(a);
  // 2. the segment-level scan: entering states (the composed maps apply as they are)
  SScanArgs b{};
  b.phi = smap; b.y = soff; b.NP = G; b.CPS = G; b.G = 1; b.D = D;
  b.init_mode = init != nullptr ? 3 : 0; b.init = init; b.out = sin; b.last_mode = 0;
  sscan_kernel<false, INC><<<g1, 512, 0, st>>>(b);
  // 3. every segment from its entering state, x before each chunk
  a.y = y; a.init_mode = 2; a.init = sin; a.out = out; a.last_mode = last != nullptr ? 2 : 0; a.last = last;
  sscan_kernel<TR, INC><<<gs, 512, 0, st>>>(a);
  return hipGetLastError();
}

struct BwdWs {
  float *W, *U, *X1, *A, *lgd, *Phi, *PmY2, *Hs, *Gend, *seg, *scr;
};

size_t bwd_scr_floats(size_t M) { return L * M + 4 * M * DP + 3 * M * M; }

BwdWs bwd_ws(void* base, int B, int T, int H, int sp) {
  const size_t NT = (T + L - 1) / L, M = sp ? 2 * L : L, BH = (size_t)B * H;
  auto al = [](char* p) { return (char*)(((uintptr_t)p + 255) & ~(uintptr_t)255); };
  char* p = al((char*)base);
  BwdWs w;
  w.W = (float*)p; p = al(p + 4 * BH * NT * M * DP);
  w.U = (float*)p; p = al(p + 4 * BH * NT * M * DP);
  w.X1 = (float*)p; p = al(p + 4 * BH * NT * M * DP);
  w.A = (float*)p; p = al(p + 4 * BH * NT * M * M);
  w.lgd = (float*)p; p = al(p + 4 * BH * NT * L);
  w.Phi = (float*)p; p = al(p + 4 * BH * NT * DP * DP);
  w.PmY2 = (float*)p; p = al(p + 4 * BH * NT * DP * DP);
  w.Hs = (float*)p; p = al(p + 4 * BH * NT * DP * DP);
  w.Gend = (float*)p; p = al(p + 4 * BH * NT * DP * DP);
  w.seg = (float*)p; p = al(p + 4 * 3 * BH * 16 * DP * DP);   // the segmented scans' maps and states (G <= 16)
  w.scr = (float*)p;
  return w;
}

template <typename X, bool SP>
hipError_t launch_bwd_t(const ChunkBwdArgs& a, const BwdWs& w, hipStream_t st) {
  const int NT = (a.f.T + L - 1) / L;
  const int BH = a.f.B * a.f.H;
  const dim3 chunks(NT, BH);
  chunk_bwd_maps_kernel<X, SP><<<chunks, 64 * GW, 0, st>>>(a, w.W, w.U, w.lgd, w.Phi, w.PmY2, NT);
  if (hipError_t e = launch_sscan<false, true>(w.Phi, w.PmY2, BH, NT, a.f.initial_state, a.f.D, w.Hs, nullptr,
                                                 w.seg, st))
    return e;
  chunk_bwd_pre_kernel<X, SP><<<chunks, 64 * GW, 0, st>>>(a, w.W, w.lgd, w.X1, w.PmY2, NT);
  if (hipError_t e = launch_sscan<true, false>(w.Phi, w.PmY2, BH, NT, a.d_final_state, a.f.D, w.Gend,
                                                 a.d_initial_state, w.seg, st))
    return e;
  chunk_bwd_grad_kernel<X, SP><<<chunks, 64 * GW, 0, st>>>(a, w.W, w.U, w.X1, w.Hs, w.lgd, w.A, w.Gend, w.scr, NT);
  return hipGetLastError();
}

}  // namespace

size_t chunk_bwd_workspace_bytes(int B, int T, int H, int has_sparse) {
  const size_t NT = (T + L - 1) / L, M = has_sparse ? 2 * L : L, BH = (size_t)B * H;
  const size_t per = 4 * (3 * M * DP + M * M + L + 4 * DP * DP + bwd_scr_floats(M));
  return BH * NT * per + 4 * 3 * BH * 16 * DP * DP + 256 * 13;
}

hipError_t launch_chunk_bwd(const ChunkBwdArgs& a, hipStream_t st) {
  const bool sp = a.f.sparse_k != nullptr;
  const BwdWs w = bwd_ws(a.workspace, a.f.B, a.f.T, a.f.H, sp);
  if (hipError_t e = launch_chunk_intra(a.f, w.W, w.U, w.lgd, w.A, st)) return e;
  if (a.f.dtype == DT_BF16) return sp ? launch_bwd_t<bf16_t, true>(a, w, st) : launch_bwd_t<bf16_t, false>(a, w, st);
  return sp ? launch_bwd_t<float, true>(a, w, st) : launch_bwd_t<float, false>(a, w, st);
}

}  // namespace sgsa
