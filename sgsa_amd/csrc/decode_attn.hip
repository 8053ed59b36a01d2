// Dense GQA attention for one decode token per sequence (the hybrid decoder's
// dense layers, modelings/hybrid_dense_delta_topk.py:178-192 at q_len = 1):
// o = softmax(q K^T / sqrt(d)) V over the cached keys [0, kend), with the
// reference's rounding points in bf16: the score product rounded to bf16, the
// scaling in bf16, the softmax in fp32, the probabilities rounded to bf16 and
// their product with V accumulated in fp32.
//
// Split over key blocks of 256, three launches:
//   scores  (block, b*Hkv + kh): the G = H / Hkv query heads sharing kv head kh
//           against the block's keys (bf16: on MFMA, 16 keys per product; fp32:
//           one key per thread); the rounded scores go
//           to the workspace, and each head's block maximum and sum of
//           exp(s - max) to a partial.
//   pv      (block, b*Hkv + kh): each head's softmax normaliser from all the
//           partials, the block's probabilities (rounded to the dtype) in LDS,
//           then their product with the block's value rows, one dimension
//           pair per thread, into an fp32 partial output.
//   reduce  (b*H): the partial outputs summed in block order, stored in dtype.
// K and V are each read once; the workspace holds the scores, the partials
// and the partial outputs.

#include "common.h"
#include "kernels.h"

namespace sgsa {
namespace {

constexpr int DA_KB = 256;   // keys per block
constexpr int DA_D = 128;    // head dimension

__device__ __forceinline__ float da_round(float v, float) { return v; }
__device__ __forceinline__ float da_round(float v, bf16_t) { return bf16_to_f32(f32_to_bf16(v)); }

template <typename X>
__device__ __forceinline__ void load8f(const X* p, float (&f)[8]) {
  if constexpr (sizeof(X) == 2) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
    const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  }
}

template <typename X, int G>
__global__ __launch_bounds__(256) void dattn_scores_kernel(const X* __restrict__ q, const X* __restrict__ kc, int H,
                                                           int Hkv, long Tmax, int kend, int nblk, float scale,
                                                           X* __restrict__ sws, float2* __restrict__ part) {
  __shared__ float qs[G][DA_D];
  __shared__ float red[G][4][2];
  const int blk = blockIdx.x, bk = blockIdx.y;
  const int b = bk / Hkv, kh = bk % Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const X tag{};
  for (int i = tid; i < G * DA_D; i += 256) qs[i / DA_D][i % DA_D] = ld(q, ((long)b * H + kh * G + i / DA_D) * DA_D + i % DA_D);
  __syncthreads();
  const int j = blk * DA_KB + tid;
  const bool valid = j < kend;
  const X* kr = kc + ((long)bk * Tmax + (valid ? j : 0)) * DA_D;
  float acc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g] = 0.f;
#pragma unroll 4
  for (int d0 = 0; d0 < DA_D; d0 += 8) {
    float kf[8];
    load8f(kr + d0, kf);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float4 qa = *reinterpret_cast<const float4*>(&qs[g][d0]);
      const float4 qb = *reinterpret_cast<const float4*>(&qs[g][d0 + 4]);
      acc[g] = fmaf(kf[0], qa.x, acc[g]); acc[g] = fmaf(kf[1], qa.y, acc[g]);
      acc[g] = fmaf(kf[2], qa.z, acc[g]); acc[g] = fmaf(kf[3], qa.w, acc[g]);
      acc[g] = fmaf(kf[4], qb.x, acc[g]); acc[g] = fmaf(kf[5], qb.y, acc[g]);
      acc[g] = fmaf(kf[6], qb.z, acc[g]); acc[g] = fmaf(kf[7], qb.w, acc[g]);
    }
  }
  float s[G], m[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    s[g] = da_round(da_round(acc[g], tag) * scale, tag);   // matmul output, then the scaling, in dtype
    if (valid) st(sws, ((long)b * H + kh * G + g) * kend + j, s[g]);
    m[g] = valid ? s[g] : -INFINITY;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m[g] = fmaxf(m[g], __shfl_xor(m[g], o, 64));
    if (lane == 0) red[g][w][0] = m[g];
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = fmaxf(fmaxf(red[g][0][0], red[g][1][0]), fmaxf(red[g][2][0], red[g][3][0]));
    float e = valid ? expf(s[g] - m[g]) : 0.f;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) e += __shfl_xor(e, o, 64);
    if (lane == 0) red[g][w][1] = e;
  }
  __syncthreads();
  if (tid < G) {
    const int g = tid;
    const float mx = fmaxf(fmaxf(red[g][0][0], red[g][1][0]), fmaxf(red[g][2][0], red[g][3][0]));
    const float l = (red[g][0][1] + red[g][1][1]) + (red[g][2][1] + red[g][3][1]);
    part[((long)b * H + kh * G + g) * nblk + blk] = make_float2(mx, l);
  }
}

// bf16 form of dattn_scores_kernel, the products on v_mfma_f32_16x16x32_bf16: A = the
// group's G query heads (rows past G zero), B = 16 keys, dims 32 s + 8 lg + e at
// k-position 8 lg + e of step s.  Lane (lc, lg) loads 64-byte pieces of 16 key rows per
// instruction (16 rows x 64 B) where the one-key-per-thread form touches 64 rows x 16 B,
// and holds C[4 lg + e][lc], head 4 lg + e's score of key 16 kg + lc.  The rounding
// points, the stores and the per-head block statistics are those of the fp32 form.
template <int G>
__global__ __launch_bounds__(256) void dattn_scores_mfma_kernel(const bf16_t* __restrict__ q,
                                                                const bf16_t* __restrict__ kc, int H, int Hkv,
                                                                long Tmax, int kend, int nblk, float scale,
                                                                bf16_t* __restrict__ sws, float2* __restrict__ part) {
  static_assert(G <= 16, "one 16-row A operand holds the group's heads");
  __shared__ float red[G][4][2];
  const int blk = blockIdx.x, bk = blockIdx.y;
  const int b = bk / Hkv, kh = bk % Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int lc = lane & 15, lg = lane >> 4;
  const bf16_t tag{};
  const uint16_t* qh = reinterpret_cast<const uint16_t*>(q) + ((long)b * H + kh * G + min(lc, G - 1)) * DA_D + 8 * lg;
  const uint16_t* kb = reinterpret_cast<const uint16_t*>(kc) + (long)bk * Tmax * DA_D + 8 * lg;
  const int j0 = blk * DA_KB + 64 * w;   // the wave's 64 keys, 16 kg + lc
  u16x8 kr[4][4];
#pragma unroll
  for (int kg = 0; kg < 4; ++kg) {
    const int j = min(j0 + 16 * kg + lc, kend - 1);   // keys past kend re-read the last one and are not used
#pragma unroll
    for (int s = 0; s < 4; ++s) kr[kg][s] = *reinterpret_cast<const u16x8*>(kb + (long)j * DA_D + 32 * s);
  }
  bf16x8 qa[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const u16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
    qa[s] = __builtin_bit_cast(bf16x8, lc < G ? *reinterpret_cast<const u16x8*>(qh + 32 * s) : z);
  }
  constexpr int NE = G < 4 ? G : 4;   // heads 4 lg + e < G held per lane
  float sc[4][NE], mh[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) mh[e] = -INFINITY;
  const bool hl = 4 * lg < G;          // lanes whose rows are real heads
#pragma unroll
  for (int kg = 0; kg < 4; ++kg) {
    f4 c = f4_zero();
#pragma unroll
    for (int s = 0; s < 4; ++s) c = mma_bf16(qa[s], __builtin_bit_cast(bf16x8, kr[kg][s]), c);
    const int j = j0 + 16 * kg + lc;
    const bool valid = j < kend;
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      const int g = 4 * lg + e;
      const float s = da_round(da_round(c[e], tag) * scale, tag);
      sc[kg][e] = s;
      if (hl && valid) st(sws, ((long)b * H + kh * G + g) * kend + j, s);
      mh[e] = valid ? fmaxf(mh[e], s) : mh[e];
    }
  }
  // head g = 4 lg + e: its 64 scores of the wave sit in lanes 16 lg .. 16 lg + 15 (4 each)
#pragma unroll
  for (int e = 0; e < NE; ++e) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) mh[e] = fmaxf(mh[e], __shfl_xor(mh[e], o, 64));
    if (hl && lc == 0) red[4 * lg + e][w][0] = mh[e];
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const int g = min(4 * lg + e, G - 1);
    const float m = fmaxf(fmaxf(red[g][0][0], red[g][1][0]), fmaxf(red[g][2][0], red[g][3][0]));
    float x = 0.f;
#pragma unroll
    for (int kg = 0; kg < 4; ++kg) x += j0 + 16 * kg + lc < kend ? expf(sc[kg][e] - m) : 0.f;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) x += __shfl_xor(x, o, 64);
    if (hl && lc == 0) red[4 * lg + e][w][1] = x;
  }
  __syncthreads();
  if (tid < G) {
    const int g = tid;
    const float mx = fmaxf(fmaxf(red[g][0][0], red[g][1][0]), fmaxf(red[g][2][0], red[g][3][0]));
    const float l = (red[g][0][1] + red[g][1][1]) + (red[g][2][1] + red[g][3][1]);
    part[((long)b * H + kh * G + g) * nblk + blk] = make_float2(mx, l);
  }
}

template <typename X, int G>
__global__ __launch_bounds__(256) void dattn_pv_kernel(const X* __restrict__ sws, const float2* __restrict__ part,
                                                       const X* __restrict__ vc, int H, int Hkv, long Tmax, int kend,
                                                       int nblk, float* __restrict__ opart) {
  __shared__ float pl[G][DA_KB];
  __shared__ float wsum[4 * G * DA_D];   // the waves' partial sums [w][g][d]
  __shared__ float nm[G][2];
  const int blk = blockIdx.x, bk = blockIdx.y;
  const int b = bk / Hkv, kh = bk % Hkv;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const X tag{};
  // softmax normaliser of each head: wave w < G takes head w's partials
  if (w < G) {
    const float2* pp = part + ((long)b * H + kh * G + w) * nblk;
    float mx = -INFINITY;
    for (int i = lane; i < nblk; i += 64) mx = fmaxf(mx, pp[i].x);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    float sum = 0.f;
    for (int i = lane; i < nblk; i += 64) sum += pp[i].y * expf(pp[i].x - mx);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    if (lane == 0) { nm[w][0] = mx; nm[w][1] = sum; }
  }
  if (G > 4) {   // heads 4.. by the waves again
    __syncthreads();
    if (w + 4 < G) {
      const int g = w + 4;
      const float2* pp = part + ((long)b * H + kh * G + g) * nblk;
      float mx = -INFINITY;
      for (int i = lane; i < nblk; i += 64) mx = fmaxf(mx, pp[i].x);
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
      float sum = 0.f;
      for (int i = lane; i < nblk; i += 64) sum += pp[i].y * expf(pp[i].x - mx);
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
      if (lane == 0) { nm[g][0] = mx; nm[g][1] = sum; }
    }
  }
  __syncthreads();
  const int j = blk * DA_KB + tid;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float p = 0.f;
    if (j < kend) p = da_round(expf(ld(sws, ((long)b * H + kh * G + g) * kend + j) - nm[g][0]) / nm[g][1], tag);
    pl[g][tid] = p;
  }
  __syncthreads();
  // wave w: keys 64 w .. 64 w + 63 of the block for every head; lane l: dimensions 2l, 2l + 1.
  // Each value pair is loaded once and used by all G heads; the waves' sums meet in LDS.
  const int dp = 2 * lane;
  const int nk = min(DA_KB, kend - blk * DA_KB);
  const int j0 = 64 * w, j1 = min(nk, j0 + 64);
  const X* vr = vc + ((long)bk * Tmax + blk * DA_KB) * DA_D + dp;
  float o0[G], o1[G];
#pragma unroll
  for (int g = 0; g < G; ++g) { o0[g] = 0.f; o1[g] = 0.f; }
  auto vload = [&](int jj, float& v0, float& v1) __attribute__((always_inline)) {
    if constexpr (sizeof(X) == 2) {
      const uint32_t u2 = *reinterpret_cast<const uint32_t*>(vr + (long)jj * DA_D);
      v0 = __uint_as_float(u2 << 16);
      v1 = __uint_as_float(u2 & 0xffff0000u);
    } else {
      const float2 f2 = *reinterpret_cast<const float2*>(vr + (long)jj * DA_D);
      v0 = f2.x; v1 = f2.y;
    }
  };
  int jj = j0;
  for (; jj + 8 <= j1; jj += 8) {   // eight rows' loads in flight at a time
    float v0[8], v1[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) vload(jj + u, v0[u], v1[u]);
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float p = pl[g][jj + u];
        o0[g] = fmaf(p, v0[u], o0[g]);
        o1[g] = fmaf(p, v1[u], o1[g]);
      }
  }
  for (; jj < j1; ++jj) {
    float v0, v1;
    vload(jj, v0, v1);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float p = pl[g][jj];
      o0[g] = fmaf(p, v0, o0[g]);
      o1[g] = fmaf(p, v1, o1[g]);
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    wsum[(w * G + g) * DA_D + dp] = o0[g];
    wsum[(w * G + g) * DA_D + dp + 1] = o1[g];
  }
  __syncthreads();
  // thread t: element t of the G x 128 block output, the waves' sums in wave order
  for (int e = tid; e < G * DA_D; e += 256) {
    const int g = e / DA_D, d = e % DA_D;
    const float o = (wsum[(0 * G + g) * DA_D + d] + wsum[(1 * G + g) * DA_D + d]) +
                    (wsum[(2 * G + g) * DA_D + d] + wsum[(3 * G + g) * DA_D + d]);
    opart[(((long)b * H + kh * G + g) * nblk + blk) * DA_D + d] = o;
  }
}

template <typename X>
__global__ __launch_bounds__(128) void dattn_reduce_kernel(const float* __restrict__ opart, int nblk,
                                                           X* __restrict__ out) {
  const long bh = blockIdx.x;
  const int d = threadIdx.x;
  const float* op = opart + bh * nblk * DA_D + d;
  float o = 0.f;
  int i = 0;
  for (; i + 8 <= nblk; i += 8) {   // eight loads in flight, summed in block order
    float x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = op[(long)(i + u) * DA_D];
#pragma unroll
    for (int u = 0; u < 8; ++u) o += x[u];
  }
  for (; i < nblk; ++i) o += op[(long)i * DA_D];
  st(out, bh * DA_D + d, o);
}

template <typename X, int G>
hipError_t launch_t(int B, int H, int Hkv, const void* q, const void* kc, const void* vc, long Tmax, int kend,
                    void* out, char* ws, hipStream_t st) {
  const int nblk = (kend + DA_KB - 1) / DA_KB;
  const long BH = (long)B * H;
  X* sws = reinterpret_cast<X*>(ws);
  char* p = ws + ((BH * kend * sizeof(X) + 255) & ~(size_t)255);
  float2* part = reinterpret_cast<float2*>(p);
  p += (BH * nblk * sizeof(float2) + 255) & ~(size_t)255;
  float* opart = reinterpret_cast<float*>(p);
  const dim3 grid((unsigned)nblk, (unsigned)(B * Hkv));
  const float scale = (float)(1.0 / 11.313708498984761);   // 1 / sqrt(128), as the fp32 of the double
  const bool al16 = (((uintptr_t)q | (uintptr_t)kc) & 15u) == 0;
  if constexpr (sizeof(X) == 2) {
    if (al16)
      dattn_scores_mfma_kernel<G><<<grid, 256, 0, st>>>((const bf16_t*)q, (const bf16_t*)kc, H, Hkv, Tmax, kend, nblk,
                                                         scale, sws, part);
    else
      dattn_scores_kernel<X, G><<<grid, 256, 0, st>>>((const X*)q, (const X*)kc, H, Hkv, Tmax, kend, nblk, scale, sws,
                                                      part);
  } else {
    dattn_scores_kernel<X, G><<<grid, 256, 0, st>>>((const X*)q, (const X*)kc, H, Hkv, Tmax, kend, nblk, scale, sws,
                                                    part);
  }
  dattn_pv_kernel<X, G><<<grid, 256, 0, st>>>(sws, part, (const X*)vc, H, Hkv, Tmax, kend, nblk, opart);
  dattn_reduce_kernel<X><<<dim3((unsigned)BH), 128, 0, st>>>(opart, nblk, (X*)out);
  return hipGetLastError();
}

template <typename X>
hipError_t launch_g(int B, int H, int Hkv, const void* q, const void* kc, const void* vc, long Tmax, int kend,
                    void* out, char* ws, hipStream_t st) {
  switch (H / Hkv) {
    case 1: return launch_t<X, 1>(B, H, Hkv, q, kc, vc, Tmax, kend, out, ws, st);
    case 2: return launch_t<X, 2>(B, H, Hkv, q, kc, vc, Tmax, kend, out, ws, st);
    case 4: return launch_t<X, 4>(B, H, Hkv, q, kc, vc, Tmax, kend, out, ws, st);
    case 8: return launch_t<X, 8>(B, H, Hkv, q, kc, vc, Tmax, kend, out, ws, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

size_t decode_attn_workspace_bytes(int dtype, int B, int H, int kend) {
  const size_t es = dtype == DT_F32 ? 4 : 2;
  const size_t BH = (size_t)B * H;
  const size_t nblk = ((size_t)kend + DA_KB - 1) / DA_KB;
  return ((BH * kend * es + 255) & ~(size_t)255) + ((BH * nblk * sizeof(float2) + 255) & ~(size_t)255) +
         BH * nblk * DA_D * sizeof(float) + 256;
}

hipError_t launch_decode_attn(int dtype, int B, int H, int Hkv, const void* q, const void* kc, const void* vc,
                              long Tmax, int kend, void* out, void* ws, hipStream_t st) {
  char* w = reinterpret_cast<char*>(((uintptr_t)ws + 255) & ~(uintptr_t)255);
  if (dtype == DT_F32) return launch_g<float>(B, H, Hkv, q, kc, vc, Tmax, kend, out, w, st);
  return launch_g<bf16_t>(B, H, Hkv, q, kc, vc, Tmax, kend, out, w, st);
}

}  // namespace sgsa
