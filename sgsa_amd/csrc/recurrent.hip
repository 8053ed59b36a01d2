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
// One block of 256 threads per (batch, head) and tile of RC = 128 / CS columns
// (the columns of the state, the value dim, evolve independently).  The D x D fp32
// state stays in registers for the whole sequence: thread t owns column j = t % RC
// of its tile and RR = RC / 2 rows ([RR (t / RC), +RR)).  Both predictions base^T k
// and base^T kh are formed from the same registers before either update; the row
// groups are combined through LDS in a fixed order.  The next token's vectors are
// prefetched into registers while the current token runs.  Decode (T = 1) is bound
// by reading and writing the state, 2 D^2 * 4 bytes per head: with few heads the
// columns are split over CS = 4 blocks so that the whole chip moves it.
#include "common.h"
#include "kernels.h"
#include "recurrent_body.h"

namespace sgsa {

template <typename X, bool SP, int CS>
__global__ __launch_bounds__(256) void recurrent_kernel(RecurrentArgs a) {
  recurrent_body<X, SP, CS>(a);
}

template <typename X, bool SP>
static void launch_rec_t(const RecurrentArgs& a, hipStream_t st) {
  if (a.B * a.H < 256) recurrent_kernel<X, SP, 4><<<dim3((unsigned)(a.B * a.H), 4), 256, 0, st>>>(a);
  else recurrent_kernel<X, SP, 1><<<dim3((unsigned)(a.B * a.H), 1), 256, 0, st>>>(a);
}

hipError_t launch_recurrent(const RecurrentArgs& a, hipStream_t st) {
  const bool sp = a.sparse_k != nullptr;
  if (a.dtype == DT_F32) {
    if (sp) launch_rec_t<float, true>(a, st);
    else launch_rec_t<float, false>(a, st);
  } else {
    if (sp) launch_rec_t<bf16_t, true>(a, st);
    else launch_rec_t<bf16_t, false>(a, st);
  }
  return hipGetLastError();
}

}  // namespace sgsa
