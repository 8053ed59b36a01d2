// Small fused ops of the model shells (SGSAForCausalLM, the hybrid decoder), one
// launch each where the torch form takes several, which at decode's few rows
// cost more host time than the arithmetic:
//   RMSNorm  y = x * rsqrt(mean(x^2) + eps) * weight, in fp32, stored in x's
//            dtype (torch: cast, square, mean, add, rsqrt, two products, cast);
//   gates    beta = max(sigmoid(b), 1e-4), gamma = sigmoid(g), budget = u in
//            fp32 from the three H-wide logit groups of a projection row
//            (torch: three casts, two sigmoids, a clamp);
//   RoPE     q and k of a dense layer rotated (rotate-half form) straight from
//            the fused projection row into [B, heads, T, D], rounding to x's
//            dtype after each product and the sum as torch's elementwise ops do
//            (torch: a negation, a concatenation, two casts, two products and a
//            sum per tensor, then the transposing copies).
#include "common.h"
#include "kernels.h"

namespace sgsa {

__device__ __forceinline__ float round_to(float v, float) { return v; }
__device__ __forceinline__ float round_to(float v, bf16_t) { return bf16_to_f32(f32_to_bf16(v)); }

// One workgroup of 256 threads per row.  ADD: the row is first a + b, rounded
// to X and stored to sum (the residual add before the norm).
//   NE > 0 (bf16 rows, C a multiple of 8, 16-byte aligned, C <= 2048 NE / 8):
//     thread t holds elements 2048 j + 8 t + e (j < NE / 8, e < 8), read as one
//     16-byte load per j, and its weights, all loaded before the reduction; the
//     squares are summed in (j, e) order, then over the wave and the 4 waves.
//   NE = 0 walks the row twice (thread t: elements t, t + 256, ..).
template <typename X, typename W, bool ADD = false, int NE = 0>
__global__ __launch_bounds__(256) void rms_norm_kernel(const X* __restrict__ x, const W* __restrict__ w, int C,
                                                       float eps, X* __restrict__ y, const X* __restrict__ b = nullptr,
                                                       X* __restrict__ sum = nullptr) {
  __shared__ float part[4];
  const long row = blockIdx.x;
  const X* xr = x + row * C;
  X* yr = y + row * C;
  float ss = 0.f;
  if constexpr (NE > 0) {
    constexpr int NJ = NE / 8;
    float v[NJ][8], wv[NJ][8];
    const X tag{};
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
      const int c0 = 2048 * jj + 8 * threadIdx.x;
      if (c0 < C) {
        const uint4 xv = *reinterpret_cast<const uint4*>(xr + c0);
        uint4 bv = make_uint4(0, 0, 0, 0);
        if constexpr (ADD) bv = *reinterpret_cast<const uint4*>(b + row * C + c0);
        const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, bw[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t xs_ = (e & 1) ? (xw[e >> 1] & 0xffff0000u) : (xw[e >> 1] << 16);
          v[jj][e] = __uint_as_float(xs_);
          if constexpr (ADD) {
            const uint32_t bs_ = (e & 1) ? (bw[e >> 1] & 0xffff0000u) : (bw[e >> 1] << 16);
            v[jj][e] = round_to(v[jj][e] + __uint_as_float(bs_), tag);
          }
          wv[jj][e] = ld(w, c0 + e);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) { v[jj][e] = 0.f; wv[jj][e] = 0.f; }
      }
    }
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
      const int c0 = 2048 * jj + 8 * threadIdx.x;
      if (c0 < C) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if constexpr (ADD) st(sum + row * C, c0 + e, v[jj][e]);
          ss = fmaf(v[jj][e], v[jj][e], ss);
        }
      }
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float mean = (part[0] + part[1] + part[2] + part[3]) / (float)C;
    const float r = 1.0f / sqrtf(mean + eps);
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
      const int c0 = 2048 * jj + 8 * threadIdx.x;
      if (c0 < C) {
#pragma unroll
        for (int e = 0; e < 8; ++e) st(yr, c0 + e, v[jj][e] * r * wv[jj][e]);
      }
    }
    return;
  }
  if constexpr (ADD) {
    const X* br = b + row * C;
    X* sr = sum + row * C;
    for (int c = threadIdx.x; c < C; c += 256) {
      st(sr, c, ld(xr, c) + ld(br, c));
      const float v = ld(sr, c);
      ss = fmaf(v, v, ss);
    }
    xr = sr;
  } else {
    for (int c = threadIdx.x; c < C; c += 256) {
      const float v = ld(xr, c);
      ss = fmaf(v, v, ss);
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float mean = (part[0] + part[1] + part[2] + part[3]) / (float)C;
  const float r = 1.0f / sqrtf(mean + eps);
  for (int c = threadIdx.x; c < C; c += 256) st(yr, c, ld(xr, c) * r * ld(w, c));
}

// The row form: 16-byte register chunks for bf16 rows with C % 8 == 0 (16-byte aligned
// rows) and C <= 4096, else the two walks.
template <typename X, typename W, bool ADD>
hipError_t launch_norm_rows(long rows, int C, const X* x, const W* w, float eps, X* y, const X* b, X* sum,
                            hipStream_t st) {
  const dim3 grid((unsigned)rows);
  const bool chunks = sizeof(X) == 2 && C % 8 == 0 && ((uintptr_t)x | (uintptr_t)b) % 16 == 0;
  if (chunks && C <= 2048) rms_norm_kernel<X, W, ADD, 8><<<grid, 256, 0, st>>>(x, w, C, eps, y, b, sum);
  else if (chunks && C <= 4096) rms_norm_kernel<X, W, ADD, 16><<<grid, 256, 0, st>>>(x, w, C, eps, y, b, sum);
  else rms_norm_kernel<X, W, ADD, 0><<<grid, 256, 0, st>>>(x, w, C, eps, y, b, sum);
  return hipGetLastError();
}

// One thread per (row, head).  Row r's logits start at src + r * stride: beta's
// H, then gamma's H, then the budget's H.
template <typename X>
__global__ __launch_bounds__(256) void gates_kernel(const X* __restrict__ src, long stride, long rows, int H,
                                                    float* __restrict__ beta, float* __restrict__ gamma,
                                                    float* __restrict__ budget) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * H) return;
  const long r = i / H;
  const int h = (int)(i % H);
  const X* p = src + r * stride + h;
  const float bl = ld(p, 0), gl = ld(p, H), ul = ld(p, 2 * H);
  beta[i] = fmaxf(1.0f / (1.0f + expf(-bl)), 1e-4f);
  gamma[i] = 1.0f / (1.0f + expf(-gl));
  budget[i] = ul;
}

hipError_t launch_gates(int dtype, const void* src, long stride, long rows, int H, float* beta, float* gamma,
                        float* budget, hipStream_t st) {
  const dim3 grid((unsigned)((rows * H + 255) / 256));
  if (dtype == DT_F32) gates_kernel<float><<<grid, 256, 0, st>>>((const float*)src, stride, rows, H, beta, gamma, budget);
  else gates_kernel<bf16_t><<<grid, 256, 0, st>>>((const bf16_t*)src, stride, rows, H, beta, gamma, budget);
  return hipGetLastError();
}

// One decode token's projection row per sequence, split for the kernels: row b
// (src + b * stride) holds q, k, v, q_ret (HD = H * D each), then the gate
// logits b, g, u (H each).  Threads i < 4 B HD copy one element each into the
// contiguous [B, HD] outputs (k and v also into cache row pos of their
// sequence when the caches are given); the next B H threads make the gates as
// gates_kernel does.
template <typename X>
__global__ __launch_bounds__(256) void decode_split_kernel(const X* __restrict__ src, long stride, int B, int H, int D,
                                                           X* __restrict__ q, X* __restrict__ k, X* __restrict__ v,
                                                           X* __restrict__ qr, float* __restrict__ beta,
                                                           float* __restrict__ gamma, float* __restrict__ budget,
                                                           X* __restrict__ kc, X* __restrict__ vc, long cache_len,
                                                           long pos) {
  const long HD = (long)H * D;
  const long ncopy = 4L * B * HD;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i < ncopy) {
    const long b = i / (4 * HD), j = i % (4 * HD);
    const int grp = (int)(j / HD);
    const long e = j % HD;
    const X x = src[b * stride + j];
    X* dst = grp == 0 ? q : grp == 1 ? k : grp == 2 ? v : qr;
    dst[b * HD + e] = x;
    if (grp == 1 && kc != nullptr) kc[(b * cache_len + pos) * HD + e] = x;
    if (grp == 2 && vc != nullptr) vc[(b * cache_len + pos) * HD + e] = x;
    return;
  }
  const long g = i - ncopy;
  if (g >= (long)B * H) return;
  const long b = g / H;
  const int h = (int)(g % H);
  const X* p = src + b * stride + 4 * HD + h;
  const float bl = ld(p, 0), gl = ld(p, H), ul = ld(p, 2 * H);
  beta[g] = fmaxf(1.0f / (1.0f + expf(-bl)), 1e-4f);
  gamma[g] = 1.0f / (1.0f + expf(-gl));
  budget[g] = ul;
}

hipError_t launch_decode_split(int dtype, const void* src, long stride, int B, int H, int D, void* q, void* k, void* v,
                               void* qr, float* beta, float* gamma, float* budget, void* kc, void* vc, long cache_len,
                               long pos, hipStream_t st) {
  const long n = 4L * B * H * D + (long)B * H;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (dtype == DT_F32)
    decode_split_kernel<float><<<grid, 256, 0, st>>>((const float*)src, stride, B, H, D, (float*)q, (float*)k,
                                                     (float*)v, (float*)qr, beta, gamma, budget, (float*)kc,
                                                     (float*)vc, cache_len, pos);
  else
    decode_split_kernel<bf16_t><<<grid, 256, 0, st>>>((const bf16_t*)src, stride, B, H, D, (bf16_t*)q, (bf16_t*)k,
                                                      (bf16_t*)v, (bf16_t*)qr, beta, gamma, budget, (bf16_t*)kc,
                                                      (bf16_t*)vc, cache_len, pos);
  return hipGetLastError();
}

// One thread per output element.  Row (b, t) of the projection output starts at
// src + (b T + t) stride: q's Hq heads of D, then k's Hk heads (then, when vo is
// given, v's Hk heads, copied unrotated).  q goes to qo [B, Hq, T, D]; k (and v)
// to row koff + t of a [B, Hk, klen, D] buffer: the k_out tensor itself (klen =
// T, koff = 0) or a decode step's cache (klen = cache_len, koff = pos).

template <typename X>
__global__ __launch_bounds__(256) void rope_qk_kernel(const X* __restrict__ src, long stride, int B, int T, int Hq,
                                                      int Hk, int D, int pos0, const float* __restrict__ cosv,
                                                      const float* __restrict__ sinv, X* __restrict__ qo,
                                                      X* __restrict__ ko, long klen, long koff, X* __restrict__ vo) {
#pragma clang fp contract(off)
  const int nh = Hq + Hk + (vo != nullptr ? Hk : 0);
  const long n = (long)B * T * nh * D;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int d = (int)(i % D);
  const long r = i / D;
  const int hh = (int)(r % nh);
  const long bt = r / nh;
  const int t = (int)(bt % T), b = (int)(bt / T);
  const X* xr = src + bt * stride + (long)hh * D;
  if (hh >= Hq + Hk) {   // v: copied as it is
    vo[(((long)b * Hk + (hh - Hq - Hk)) * klen + koff + t) * D + d] = xr[d];
    return;
  }
  const int half = D / 2;
  const float x = ld(xr, d);
  const float xr_ = d < half ? -ld(xr, d + half) : ld(xr, d - half);
  const X tag{};
  const float c = round_to(cosv[(long)(pos0 + t) * D + d], tag);
  const float s = round_to(sinv[(long)(pos0 + t) * D + d], tag);
  const float y = round_to(round_to(x * c, tag) + round_to(xr_ * s, tag), tag);
  if (hh < Hq) st(qo, (((long)b * Hq + hh) * T + t) * D + d, y);
  else st(ko, (((long)b * Hk + (hh - Hq)) * klen + koff + t) * D + d, y);
}

hipError_t launch_rope_qk(int dtype, const void* src, long stride, int B, int T, int Hq, int Hk, int D, int pos0,
                          const float* cosv, const float* sinv, void* qo, void* ko, hipStream_t st, long klen,
                          long koff, void* vo) {
  if (klen < 0) klen = T;
  const long n = (long)B * T * (Hq + Hk + (vo != nullptr ? Hk : 0)) * D;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (dtype == DT_F32)
    rope_qk_kernel<float><<<grid, 256, 0, st>>>((const float*)src, stride, B, T, Hq, Hk, D, pos0, cosv, sinv,
                                                (float*)qo, (float*)ko, klen, koff, (float*)vo);
  else
    rope_qk_kernel<bf16_t><<<grid, 256, 0, st>>>((const bf16_t*)src, stride, B, T, Hq, Hk, D, pos0, cosv, sinv,
                                                 (bf16_t*)qo, (bf16_t*)ko, klen, koff, (bf16_t*)vo);
  return hipGetLastError();
}

hipError_t launch_add_rms_norm(int dtype, int w_f32, long rows, int C, const void* a, const void* b, void* sum,
                               const void* w, float eps, void* y, hipStream_t st) {
  if (dtype == DT_F32)
    return launch_norm_rows<float, float, true>(rows, C, (const float*)a, (const float*)w, eps, (float*)y,
                                                (const float*)b, (float*)sum, st);
  if (w_f32)
    return launch_norm_rows<bf16_t, float, true>(rows, C, (const bf16_t*)a, (const float*)w, eps, (bf16_t*)y,
                                                 (const bf16_t*)b, (bf16_t*)sum, st);
  return launch_norm_rows<bf16_t, bf16_t, true>(rows, C, (const bf16_t*)a, (const bf16_t*)w, eps, (bf16_t*)y,
                                                (const bf16_t*)b, (bf16_t*)sum, st);
}

// silu(gate) * up of a fused gate | up projection row, in X's roundings: silu
// rounded to X, then the product rounded to X.  One thread per output element;
// VEC (bf16, I % 8 == 0, 16-byte aligned rows): eight elements per thread, read
// and written as 16-byte pieces.
template <typename X>
__global__ __launch_bounds__(256) void silu_mul_kernel(const X* __restrict__ src, long stride, long rows, int I,
                                                       X* __restrict__ y) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * I) return;
  const long r = i / I;
  const int c = (int)(i % I);
  const X tag{};
  const float g = ld(src, r * stride + c), u = ld(src, r * stride + I + c);
  st(y, i, round_to(g / (1.0f + expf(-g)), tag) * u);
}

__global__ __launch_bounds__(256) void silu_mul8_kernel(const bf16_t* __restrict__ src, long stride, long rows, int I,
                                                        bf16_t* __restrict__ y) {
  const long i = ((long)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i >= rows * I) return;
  const long r = i / I;
  const int c = (int)(i % I);
  const uint4 gv = *reinterpret_cast<const uint4*>(src + r * stride + c);
  const uint4 uv = *reinterpret_cast<const uint4*>(src + r * stride + I + c);
  const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
  uint32_t o[4];
#pragma unroll
  for (int e2 = 0; e2 < 4; ++e2) {
    const float g0 = __uint_as_float(gw[e2] << 16), g1 = __uint_as_float(gw[e2] & 0xffff0000u);
    const float u0 = __uint_as_float(uw[e2] << 16), u1 = __uint_as_float(uw[e2] & 0xffff0000u);
    const float s0 = bf16_to_f32(f32_to_bf16(g0 / (1.0f + expf(-g0))));
    const float s1 = bf16_to_f32(f32_to_bf16(g1 / (1.0f + expf(-g1))));
    o[e2] = (uint32_t)f32_to_bf16(s0 * u0) | ((uint32_t)f32_to_bf16(s1 * u1) << 16);
  }
  *reinterpret_cast<uint4*>(y + i) = make_uint4(o[0], o[1], o[2], o[3]);
}

hipError_t launch_silu_mul(int dtype, const void* src, long stride, long rows, int I, void* y, hipStream_t st) {
  if (dtype != DT_F32 && I % 8 == 0 && stride % 8 == 0 && ((uintptr_t)src | (uintptr_t)y) % 16 == 0) {
    const dim3 grid((unsigned)((rows * I / 8 + 255) / 256));
    silu_mul8_kernel<<<grid, 256, 0, st>>>((const bf16_t*)src, stride, rows, I, (bf16_t*)y);
    return hipGetLastError();
  }
  const dim3 grid((unsigned)((rows * I + 255) / 256));
  if (dtype == DT_F32) silu_mul_kernel<float><<<grid, 256, 0, st>>>((const float*)src, stride, rows, I, (float*)y);
  else silu_mul_kernel<bf16_t><<<grid, 256, 0, st>>>((const bf16_t*)src, stride, rows, I, (bf16_t*)y);
  return hipGetLastError();
}

hipError_t launch_rms_norm(int dtype, int w_f32, long rows, int C, const void* x, const void* w, float eps, void* y,
                           hipStream_t st) {
  if (dtype == DT_F32)
    return launch_norm_rows<float, float, false>(rows, C, (const float*)x, (const float*)w, eps, (float*)y, nullptr,
                                                 nullptr, st);
  if (w_f32)
    return launch_norm_rows<bf16_t, float, false>(rows, C, (const bf16_t*)x, (const float*)w, eps, (bf16_t*)y,
                                                  nullptr, nullptr, st);
  return launch_norm_rows<bf16_t, bf16_t, false>(rows, C, (const bf16_t*)x, (const bf16_t*)w, eps, (bf16_t*)y,
                                                 nullptr, nullptr, st);
}

}  // namespace sgsa
