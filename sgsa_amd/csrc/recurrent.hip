// K6: recurrent SGSA, one token after another (decode step and the reference's
// "recurrent" backend).
//
// Replaces fused_recurrent_sgsa / recurrent_sgsa_fwd_triton
// (modelings/sgsa_ops/recurrent.py:138-175, recurrent_fwd_triton.py:25-145)
// with the semantics of naive_recurrent_sgsa (naive.py:34-57): per token
//   base = gamma_t S
//   S    = base + k_t (beta_t (v_t - base^T k_t))^T
//   S   += kh_t (alpha_t (vh_t - base^T kh_t))^T      (reads base, not the updated S)
//   o_t  = S^T q_t
// One block of 256 threads per (batch, head).  The D x D fp32 state stays in
// registers for the whole sequence: thread t owns column j = t % 128 and rows
// [64 (t / 128), +64).  Both predictions base^T k and base^T kh are formed from
// the same registers before either update; the two row halves are combined
// through LDS.  The next token's vectors are prefetched into registers while
// the current token runs.  Decode (T = 1) is bound by reading and writing the
// state: 2 D^2 * 4 bytes per head.
#include "common.h"
#include "kernels.h"

namespace sgsa {

namespace {
constexpr int RC = 128;   // columns (value dim) per block, padded
constexpr int RR = 64;    // rows (key dim) per thread
}  // namespace

template <typename X, bool SP>
__global__ __launch_bounds__(256) void recurrent_kernel(RecurrentArgs a) {
  __shared__ float vecs[5][RC];   // q, k, v, kh, vh of the current token
  __shared__ float part[3][2][RC];  // partial base^T k, base^T kh, S^T q per row half
  __shared__ float scal[3];         // beta, gamma, alpha

  const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x, j = tid & (RC - 1), half = tid >> 7;
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
    const int i = RR * half + r;
    S[r] = (a.initial_state != nullptr && colv && i < D) ? a.initial_state[((long)bh * D + i) * D + j] : 0.f;
  }

  // prefetch registers: thread j (< D) of the first row half loads element j
  // of the five vectors, thread 0 of the second half the three scalars
  float pv[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
  float ps[3] = {0.f, 1.f, 0.f};
  auto fetch = [&](int t) __attribute__((always_inline)) {
    const long row = ((long)(b * T + t) * H + h);
    if (half == 0 && colv) {
      pv[0] = ld(q, row * D + j);
      pv[1] = ld(k, row * D + j);
      pv[2] = ld(v, row * D + j);
      if constexpr (SP) {
        pv[3] = ld(sk, row * D + j);
        pv[4] = ld(sv, row * D + j);
      }
    }
    if (half == 1 && j == 0) {
      ps[0] = a.beta[row];
      ps[1] = a.gamma[row];
      ps[2] = SP ? a.alpha[row] : 0.f;
    }
  };

  fetch(0);
  for (int t = 0; t < T; ++t) {
    // publish token t (the previous token's readers passed the last barrier)
    if (half == 0) {
#pragma unroll
      for (int c = 0; c < 5; ++c) vecs[c][j] = colv ? pv[c] : 0.f;
    }
    if (half == 1 && j == 0) { scal[0] = ps[0]; scal[1] = ps[1]; scal[2] = ps[2]; }
    __syncthreads();
    if (t + 1 < T) fetch(t + 1);
    const float gam = scal[1];
    // base = gamma S; predictions base^T k and base^T kh over this thread's rows
    float pk = 0.f, ph = 0.f;
#pragma unroll
    for (int r = 0; r < RR; ++r) {
      S[r] *= gam;
      pk = fmaf(S[r], vecs[1][RR * half + r], pk);
      if constexpr (SP) ph = fmaf(S[r], vecs[3][RR * half + r], ph);
    }
    part[0][half][j] = pk;
    if constexpr (SP) part[1][half][j] = ph;
    __syncthreads();
    const float dl = scal[0] * (vecs[2][j] - (part[0][0][j] + part[0][1][j]));
    const float ds = SP ? scal[2] * (vecs[4][j] - (part[1][0][j] + part[1][1][j])) : 0.f;
    // rank-1 writes, then the readout o = S^T q
    float po = 0.f;
#pragma unroll
    for (int r = 0; r < RR; ++r) {
      const int i = RR * half + r;
      S[r] = fmaf(vecs[1][i], dl, S[r]);
      if constexpr (SP) S[r] = fmaf(vecs[3][i], ds, S[r]);
      po = fmaf(S[r], vecs[0][i], po);
    }
    part[2][half][j] = po;
    __syncthreads();
    if (half == 0 && colv) st(reinterpret_cast<X*>(a.out), ((long)(b * T + t) * H + h) * D + j, part[2][0][j] + part[2][1][j]);
  }

  if (a.final_state != nullptr && colv) {
#pragma unroll
    for (int r = 0; r < RR; ++r) {
      const int i = RR * half + r;
      if (i < D) a.final_state[((long)bh * D + i) * D + j] = S[r];
    }
  }
}

hipError_t launch_recurrent(const RecurrentArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)(a.B * a.H));
  const bool sp = a.sparse_k != nullptr;
  if (a.dtype == DT_F32) {
    if (sp) recurrent_kernel<float, true><<<grid, 256, 0, st>>>(a);
    else recurrent_kernel<float, false><<<grid, 256, 0, st>>>(a);
  } else {
    if (sp) recurrent_kernel<bf16_t, true><<<grid, 256, 0, st>>>(a);
    else recurrent_kernel<bf16_t, false><<<grid, 256, 0, st>>>(a);
  }
  return hipGetLastError();
}

}  // namespace sgsa
