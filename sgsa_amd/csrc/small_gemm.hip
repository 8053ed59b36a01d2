// y = x W^T (+ bias) for a handful of rows: the decode step's projections
// (nn.Linear at B <= 16 tokens), where a library GEMM's host dispatch costs
// more than the kernel.  bf16 in, fp32 accumulation, bf16 out.
//
// One workgroup per 16 output columns, its eight waves splitting K in eight
// interleaved ranges of 32-element steps; each wave runs
// v_mfma_f32_16x16x32_bf16 with the x rows (zero past M) as the A operand and
// 16 weight rows as the B operand, both loaded from global memory straight
// into registers, four steps ahead.  The waves' 16x16 tiles meet in LDS.

#include "common.h"
#include "kernels.h"

namespace sgsa {
namespace {

typedef uint16_t sg_u16x8 __attribute__((ext_vector_type(8)));

constexpr int SG_W = 8;   // waves per workgroup

__global__ __launch_bounds__(64 * SG_W) void small_gemm_kernel(const bf16_t* __restrict__ x, long xs, const bf16_t* __restrict__ W,
                                                         const bf16_t* __restrict__ bias, int M, int N, int K,
                                                         bf16_t* __restrict__ y, long ys) {
  __shared__ f4 red[SG_W][64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int n = min(n0 + lr, N - 1);    // columns past N re-read the last row and are not stored
  const int row = lr;                   // A operand row; rows >= M read row 0 and are zeroed
  const bool live = row < M;
  const uint16_t* xr = reinterpret_cast<const uint16_t*>(x) + (long)(live ? row : 0) * xs + 8 * lg;
  const uint16_t* wr = reinterpret_cast<const uint16_t*>(W) + (long)n * K + 8 * lg;
  const int nsteps = K / 32;
  f4 acc = f4_zero();
  // wave w takes steps w, w + SG_W, ...
  int s = w;
  for (; s + 3 * SG_W < nsteps; s += 4 * SG_W) {
    sg_u16x8 a[4], b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      a[u] = *reinterpret_cast<const sg_u16x8*>(xr + 32 * (s + SG_W * u));
      b[u] = *reinterpret_cast<const sg_u16x8*>(wr + 32 * (s + SG_W * u));
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const sg_u16x8 av = live ? a[u] : (sg_u16x8){0, 0, 0, 0, 0, 0, 0, 0};
      acc = mma_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, b[u]), acc);
    }
  }
  for (; s < nsteps; s += SG_W) {
    sg_u16x8 a = *reinterpret_cast<const sg_u16x8*>(xr + 32 * s);
    const sg_u16x8 b = *reinterpret_cast<const sg_u16x8*>(wr + 32 * s);
    if (!live) a = (sg_u16x8){0, 0, 0, 0, 0, 0, 0, 0};
    acc = mma_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc);
  }
  red[w][lane] = acc;
  __syncthreads();
  if (w == 0) {
    // acc element i of lane (lr, lg): output row 4 lg + i, column n0 + lr
    f4 t = red[0][lane];
#pragma unroll
    for (int v = 1; v < SG_W; ++v) {
      const f4 o = red[v][lane];
      t[0] += o[0]; t[1] += o[1]; t[2] += o[2]; t[3] += o[3];
    }
    const int col = n0 + lr;
    if (col < N) {
      const float bv = bias != nullptr ? bf16_to_f32(bias[col].bits) : 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * lg + i;
        if (r < M) y[(long)r * ys + col].bits = f32_to_bf16(t[i] + bv);
      }
    }
  }
}

}  // namespace

hipError_t launch_small_gemm(const void* x, long xs, const void* W, const void* bias, int M, int N, int K, void* y,
                             long ys, hipStream_t st) {
  small_gemm_kernel<<<dim3((unsigned)((N + 15) / 16)), 64 * SG_W, 0, st>>>((const bf16_t*)x, xs, (const bf16_t*)W,
                                                                     (const bf16_t*)bias, M, N, K, (bf16_t*)y, ys);
  return hipGetLastError();
}

}  // namespace sgsa
