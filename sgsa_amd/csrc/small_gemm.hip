// y = x W^T (+ bias) for a handful of rows: the decode step's projections
// (nn.Linear at B <= 16 tokens), where a library GEMM's host dispatch costs
// more than the kernel.  bf16 in, fp32 accumulation, bf16 out.
//
// The product reads W once and is bound by that read (N K bf16).  One
// workgroup per 16 output columns, its 16 waves splitting K in interleaved
// 32-element steps: wave w takes steps w, w + 16, ...  W comes row-major
// [N, K] or pre-tiled (TL): tile t (columns 16t .. 16t + 15), step s, lane l
// holds the 8 elements W[16t + l % 16][32s + 8 (l / 16) ..] at
// ((t * K/32 + s) * 64 + l) * 8, so that one step of a wave reads 1 KB in one
// piece instead of 64 bytes from each of 16 rows (the same products in the
// same order: bit-identical, and 20-25% faster at the decode shapes; rows past
// N are zero).  Each wave issues the
// loads of up to D steps (W rows and the x rows, straight into registers)
// before the first product, so a workgroup pays about one memory latency per
// D steps rather than one per step; steps past K re-read the last step with
// the x operand zeroed, which keeps the loads free of branches.  (Measured at
// the decode shapes: 16 waves with every load in one batch beat 8 waves with
// one batch and 8 waves with two batches at twice the occupancy.)  The
// products run on v_mfma_f32_16x16x32_bf16 (A operand: the x rows, zero past
// M; B operand: 16 rows of W), and the 16 waves' partial 16x16 tiles meet in
// LDS, where 256 threads sum one output element each and apply the epilogue:
//   plain     y = bf16(acc + bias), then with a residual operand
//             bf16(y + res) (the model's h + mlp(x), as two bf16 tensor ops
//             compute it);
//   split     the SGSA decode projection's row q | k | v | q_ret | b | g | u
//             routed as sgsa_decode_split routes it: the bf16 values to the
//             contiguous q, k, v, q_ret and to cache row pos, the gates
//             beta = max(sigmoid(b), 1e-4), gamma = sigmoid(g), budget = u in
//             fp32 from the bf16 logits;
//   swiglu    W's rows interleaved in groups of 8 (gate rows 8b .. 8b + 7,
//             then the up rows 8b .. 8b + 7), so a workgroup's 16 columns
//             hold 8 gate and the matching 8 up values; it writes
//             bf16(bf16(silu(gate)) * up) for those 8 columns of y [M, N / 2]
//             (sgsa_silu_mul's roundings on the bf16 projection values).

#include <math.h>

#include "common.h"
#include "kernels.h"

namespace sgsa {
namespace {

typedef uint16_t sg_u16x8 __attribute__((ext_vector_type(8)));

constexpr int SG_W = 16;   // waves per workgroup

template <int D, int EPI, bool TL>
__global__ __launch_bounds__(64 * SG_W) void small_gemm_kernel(const bf16_t* __restrict__ x, long xs,
                                                               const bf16_t* __restrict__ W,
                                                               const bf16_t* __restrict__ bias, int M, int N, int K,
                                                               bf16_t* __restrict__ y, long ys,
                                                               const bf16_t* __restrict__ res, long rs, SgSplit sp) {
  __shared__ f4 red[SG_W][64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int n = min(n0 + lr, N - 1);    // columns past N re-read the last row and are not stored
  const bool live = lr < M;             // A operand row lr; rows >= M read row 0 and are zeroed
  const uint16_t* xr = reinterpret_cast<const uint16_t*>(x) + (long)(live ? lr : 0) * xs + 8 * lg;
  const int nsteps = K / 32;
  const uint16_t* wr = reinterpret_cast<const uint16_t*>(W) +
                       (TL ? (long)blockIdx.x * nsteps * 512 + 8 * lane : (long)n * K + 8 * lg);
  constexpr int wstep = TL ? 512 : 32;   // elements between a lane's consecutive steps
  f4 acc = f4_zero();
  for (int s0 = w; s0 < nsteps; s0 += SG_W * D) {
    sg_u16x8 a[D], b[D];
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const int s = min(s0 + SG_W * u, nsteps - 1);
      a[u] = (sg_u16x8){0, 0, 0, 0, 0, 0, 0, 0};
      if (live) a[u] = *reinterpret_cast<const sg_u16x8*>(xr + 32 * s);   // rows past M load nothing
      b[u] = *reinterpret_cast<const sg_u16x8*>(wr + (long)wstep * s);
    }
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const bool on = live && s0 + SG_W * u < nsteps;
      const sg_u16x8 av = on ? a[u] : (sg_u16x8){0, 0, 0, 0, 0, 0, 0, 0};
      acc = mma_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, b[u]), acc);
    }
  }
  red[w][lane] = acc;
  __syncthreads();
  if (tid >= 256) return;
  // output row r, column n0 + c: element r % 4 of lane c + 16 (r / 4) in every wave's tile
  const int r = tid >> 4, c = tid & 15;
  const int l = c + 16 * (r >> 2), e = r & 3;
  float t = 0.f;
#pragma unroll
  for (int v = 0; v < SG_W; ++v) t += red[v][l][e];
  const int col = n0 + c;
  const float bv = (bias != nullptr && col < N) ? bf16_to_f32(bias[col].bits) : 0.f;
  const uint16_t o = f32_to_bf16(t + bv);
  if constexpr (EPI == 2) {
    // c < 8: gate column 8 blockIdx.x + c; its up value is column c + 8 of the same
    // row, held by the lane 8 on (lanes 16 r' + c of one wave hold row r')
    const float up = __shfl_down(bf16_to_f32(o), 8, 16);
    if (c < 8 && r < M && col < N) {
      const float g = bf16_to_f32(o);
      const float sg = bf16_to_f32(f32_to_bf16(g / (1.0f + expf(-g))));
      y[(long)r * ys + 8 * blockIdx.x + c].bits = f32_to_bf16(sg * up);
    }
    return;
  }
  if (r >= M || col >= N) return;
  if constexpr (EPI == 0) {
    uint16_t ov = o;
    if (res != nullptr) ov = f32_to_bf16(bf16_to_f32(o) + bf16_to_f32(res[(long)r * rs + col].bits));
    y[(long)r * ys + col].bits = ov;
  } else {
    const long HD = sp.HD;
    if (col < 4 * HD) {
      const int grp = (int)(col / HD);
      const long e2 = col % HD;
      uint16_t* dst = grp == 0 ? sp.q : grp == 1 ? sp.k : grp == 2 ? sp.v : sp.qr;
      dst[(long)r * HD + e2] = o;
      if (grp == 1) sp.kc[((long)r * sp.cache_len + sp.pos) * HD + e2] = o;
      if (grp == 2) sp.vc[((long)r * sp.cache_len + sp.pos) * HD + e2] = o;
    } else {
      const int j = (int)(col - 4 * HD), H = sp.H;
      const float lv = bf16_to_f32(o);
      if (j < H) sp.beta[(long)r * H + j] = fmaxf(1.0f / (1.0f + expf(-lv)), 1e-4f);
      else if (j < 2 * H) sp.gamma[(long)r * H + j - H] = 1.0f / (1.0f + expf(-lv));
      else sp.budget[(long)r * H + j - 2 * H] = lv;
    }
  }
}

// W [N, K] row-major -> the tiled layout, one 16-byte piece per thread
__global__ __launch_bounds__(256) void tile_rows_kernel(const uint16_t* __restrict__ W, int N, int K,
                                                        uint16_t* __restrict__ out, long pieces) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= pieces) return;
  const int nsteps = K / 32;
  const int l = (int)(i & 63);
  const long ts = i >> 6;
  const long t = ts / nsteps;
  const int s = (int)(ts % nsteps);
  const long n = 16 * t + (l & 15);
  sg_u16x8 v = (sg_u16x8){0, 0, 0, 0, 0, 0, 0, 0};
  if (n < N) v = *reinterpret_cast<const sg_u16x8*>(W + n * K + 32 * s + 8 * (l >> 4));
  *reinterpret_cast<sg_u16x8*>(out + 8 * i) = v;
}

template <int EPI, bool TL>
hipError_t launch_gemm(const void* x, long xs, const void* W, const void* bias, int M, int N, int K, void* y, long ys,
                       hipStream_t st, const void* res, long rs, const SgSplit& sp) {
  const dim3 grid((unsigned)((N + 15) / 16));
  const int spw = (K / 32 + SG_W - 1) / SG_W;   // steps per wave
  const bf16_t* xp = (const bf16_t*)x;
  const bf16_t* wp = (const bf16_t*)W;
  const bf16_t* bp = (const bf16_t*)bias;
  const bf16_t* rp = (const bf16_t*)res;
  bf16_t* yp = (bf16_t*)y;
  if (spw <= 4) small_gemm_kernel<4, EPI, TL><<<grid, 64 * SG_W, 0, st>>>(xp, xs, wp, bp, M, N, K, yp, ys, rp, rs, sp);
  else if (spw <= 8) small_gemm_kernel<8, EPI, TL><<<grid, 64 * SG_W, 0, st>>>(xp, xs, wp, bp, M, N, K, yp, ys, rp, rs, sp);
  else small_gemm_kernel<11, EPI, TL><<<grid, 64 * SG_W, 0, st>>>(xp, xs, wp, bp, M, N, K, yp, ys, rp, rs, sp);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_small_gemm(const void* x, long xs, const void* W, const void* bias, int M, int N, int K, void* y,
                             long ys, hipStream_t st, const void* res, long rs, bool tiled) {
  if (tiled) return launch_gemm<0, true>(x, xs, W, bias, M, N, K, y, ys, st, res, rs, SgSplit{});
  return launch_gemm<0, false>(x, xs, W, bias, M, N, K, y, ys, st, res, rs, SgSplit{});
}

hipError_t launch_small_gemm_split(const void* x, long xs, const void* W, const void* bias, int M, int N, int K,
                                   const SgSplit& sp, hipStream_t st) {
  return launch_gemm<1, true>(x, xs, W, bias, M, N, K, nullptr, 0, st, nullptr, 0, sp);
}

hipError_t launch_small_gemm_swiglu(const void* x, long xs, const void* W, int M, int N, int K, void* y, long ys,
                                    hipStream_t st) {
  return launch_gemm<2, true>(x, xs, W, nullptr, M, N, K, y, ys, st, nullptr, 0, SgSplit{});
}

hipError_t launch_tile_rows(const void* W, int N, int K, void* out, hipStream_t st) {
  const long pieces = (long)((N + 15) / 16) * (K / 32) * 64;
  tile_rows_kernel<<<dim3((unsigned)((pieces + 255) / 256)), 256, 0, st>>>((const uint16_t*)W, N, K, (uint16_t*)out,
                                                                            pieces);
  return hipGetLastError();
}

}  // namespace sgsa
