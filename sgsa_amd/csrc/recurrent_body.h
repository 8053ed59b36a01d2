// The body of K6 (recurrent_kernel in recurrent.hip), shared with the decode
// step's merge-then-update kernel (gather.hip): one block of 256 threads per
// (batch, head) -- blockIdx.x -- and tile of 128 / CS state columns -- blockIdx.y.
// recurrent.hip describes the layout.
#pragma once

#include "common.h"
#include "kernels.h"

namespace sgsa {

template <typename X, bool SP, int CS>
__device__ __forceinline__ void recurrent_body(const RecurrentArgs& a) {
  constexpr int RC = 128 / CS;     // columns per block
  constexpr int NG = 256 / RC;     // row groups
  constexpr int RR = 128 / NG;     // rows per thread
  __shared__ float vq[128], vk[128], vkh[128];   // q, k, kh of the current token (all rows)
  __shared__ float vv[RC], vvh[RC];              // v, vh (this tile's columns)
  __shared__ float part[3][NG][RC];              // partial base^T k, base^T kh, S^T q per row group
  __shared__ float scal[3];                      // beta, gamma, alpha

  const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x, jl = tid % RC, g = tid / RC;
  const int j = blockIdx.y * RC + jl;
  const int D = a.D, T = a.T, H = a.H;
  const bool colv = j < D;
  const X* q = reinterpret_cast<const X*>(a.q);
  const X* k = reinterpret_cast<const X*>(a.k);
  const X* v = reinterpret_cast<const X*>(a.v);
  const X* sk = reinterpret_cast<const X*>(a.sparse_k);
  const X* sv = reinterpret_cast<const X*>(a.sparse_v);

  float S[RR];
#pragma unroll
  for (int r = 0; r < RR; ++r) {
    const int i = RR * g + r;
    S[r] = (a.initial_state != nullptr && colv && i < D) ? a.initial_state[((long)bh * D + i) * D + j] : 0.f;
  }

  // prefetch registers: thread t < 128 loads element t of q, k, kh; thread 128 + c
  // (c < RC) element c of this tile's v, vh; thread 255 the three scalars
  float pv[3] = {0.f, 0.f, 0.f};
  float ps[3] = {0.f, 1.f, 0.f};
  const int vc = blockIdx.y * RC + (tid - 128);
  auto fetch = [&](int t) __attribute__((always_inline)) {
    const long row = ((long)(b * T + t) * H + h);
    if (tid < 128) {
      if (tid < D) {
        pv[0] = ld(q, row * D + tid);
        pv[1] = ld(k, row * D + tid);
        if constexpr (SP) pv[2] = ld(sk, row * D + tid);
      }
    } else if (tid < 128 + RC) {
      if (vc < D) {
        pv[0] = ld(v, row * D + vc);
        if constexpr (SP) pv[1] = ld(sv, row * D + vc);
      }
    }
    if (tid == 255) {
      ps[0] = a.beta[row];
      ps[1] = a.gamma[row];
      ps[2] = SP ? a.alpha[row] : 0.f;
    }
  };

  fetch(0);
  for (int t = 0; t < T; ++t) {
    // publish token t (the previous token's readers passed the last barrier)
    if (tid < 128) {
      vq[tid] = pv[0];
      vk[tid] = pv[1];
      vkh[tid] = pv[2];
    } else if (tid < 128 + RC) {
      vv[tid - 128] = pv[0];
      vvh[tid - 128] = pv[1];
    }
    if (tid == 255) { scal[0] = ps[0]; scal[1] = ps[1]; scal[2] = ps[2]; }
    __syncthreads();
    if (t + 1 < T) fetch(t + 1);
    const float gam = scal[1];
    // base = gamma S; predictions base^T k and base^T kh over this thread's rows
    float pk = 0.f, ph = 0.f;
#pragma unroll
    for (int r = 0; r < RR; ++r) {
      S[r] *= gam;
      pk = fmaf(S[r], vk[RR * g + r], pk);
      if constexpr (SP) ph = fmaf(S[r], vkh[RR * g + r], ph);
    }
    part[0][g][jl] = pk;
    if constexpr (SP) part[1][g][jl] = ph;
    __syncthreads();
    float sk_ = 0.f, sh_ = 0.f;
#pragma unroll
    for (int u = 0; u < NG; ++u) {
      sk_ += part[0][u][jl];
      if constexpr (SP) sh_ += part[1][u][jl];
    }
    const float dl = scal[0] * (vv[jl] - sk_);
    const float ds = SP ? scal[2] * (vvh[jl] - sh_) : 0.f;
    // rank-1 writes, then the readout o = S^T q
    float po = 0.f;
#pragma unroll
    for (int r = 0; r < RR; ++r) {
      const int i = RR * g + r;
      S[r] = fmaf(vk[i], dl, S[r]);
      if constexpr (SP) S[r] = fmaf(vkh[i], ds, S[r]);
      po = fmaf(S[r], vq[i], po);
    }
    part[2][g][jl] = po;
    __syncthreads();
    if (g == 0 && colv) {
      float o = 0.f;
#pragma unroll
      for (int u = 0; u < NG; ++u) o += part[2][u][jl];
      st(reinterpret_cast<X*>(a.out), ((long)(b * T + t) * H + h) * D + j, o);
    }
  }

  if (a.final_state != nullptr && colv) {
#pragma unroll
    for (int r = 0; r < RR; ++r) {
      const int i = RR * g + r;
      if (i < D) a.final_state[((long)bh * D + i) * D + j] = S[r];
    }
  }
}

}  // namespace sgsa
