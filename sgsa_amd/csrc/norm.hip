// RMSNorm of the model shells (SGSAForCausalLM, the hybrid decoder) in one
// launch per call: y = x * rsqrt(mean(x^2) + eps) * weight, evaluated in fp32
// and stored in x's dtype.  The torch form of the same expression takes about
// eight launches (cast, square, mean, add, rsqrt, two products, cast), which at
// decode's few rows cost more host time than the arithmetic.
#include "common.h"
#include "kernels.h"

namespace sgsa {

// One workgroup of 256 threads per row.
template <typename X, typename W>
__global__ __launch_bounds__(256) void rms_norm_kernel(const X* __restrict__ x, const W* __restrict__ w, int C,
                                                       float eps, X* __restrict__ y) {
  __shared__ float part[4];
  const long row = blockIdx.x;
  const X* xr = x + row * C;
  float ss = 0.f;
  for (int c = threadIdx.x; c < C; c += 256) {
    const float v = ld(xr, c);
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float mean = (part[0] + part[1] + part[2] + part[3]) / (float)C;
  const float r = 1.0f / sqrtf(mean + eps);
  X* yr = y + row * C;
  for (int c = threadIdx.x; c < C; c += 256) st(yr, c, ld(xr, c) * r * ld(w, c));
}

hipError_t launch_rms_norm(int dtype, int w_f32, long rows, int C, const void* x, const void* w, float eps, void* y,
                           hipStream_t st) {
  const dim3 grid((unsigned)rows);
  if (dtype == DT_F32) {
    rms_norm_kernel<float, float><<<grid, 256, 0, st>>>((const float*)x, (const float*)w, C, eps, (float*)y);
  } else if (w_f32) {
    rms_norm_kernel<bf16_t, float><<<grid, 256, 0, st>>>((const bf16_t*)x, (const float*)w, C, eps, (bf16_t*)y);
  } else {
    rms_norm_kernel<bf16_t, bf16_t><<<grid, 256, 0, st>>>((const bf16_t*)x, (const bf16_t*)w, C, eps, (bf16_t*)y);
  }
  return hipGetLastError();
}

}  // namespace sgsa
