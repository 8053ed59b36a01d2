// Chunked SGSA forward, bf16-input path (gfx950: v_mfma_f32_16x16x32_bf16,
// v_mfma_f32_16x16x4_f32, ds_read_b64_tr_b16).
//
// Per chunk of L = 64 tokens with M = 2L virtual write samples (sample i = 2t + r:
// r = 0 the local write k, v, beta; r = 1 the sparse write k~, v^, alpha;
// chunk_fwd.py:49-61; without the sparse write M = L and i = t), the chunk-local
// log-decay prefix l_t = sum_{p <= t} log max(gamma_p, 1e-6), sample keys kappa,
// values nu and write strengths lam, and the chunk-start state S [d_k][d_v]:
//
//   T_ij = 1[tau_j < tau_i] lam_j e^{l_tau_i - l_tau_j} (kappa_i . kappa_j),    A = (I + T)^-1
//   X = kappa S,   B_i = nu_i - e^{l_tau_i} X_i,   R = A B
//   o_t = e^{l_t} (q_t S) + sum_{tau_i <= t} lam_i e^{l_t - l_tau_i} (q_t . kappa_i) R_i
//   S'  = e^{l_L} S + kappa^T R',   R'_i = lam_i e^{l_L - l_tau_i} R_i
//
// which is chunk_fwd.py:70-126 with the UT/WY inverse kept as A (R = U - W S for
// W = A e^{l_tau} kappa and U = A nu).
//
// K3 chunk_inv_bf16      grid (NT, B*H), 8 waves: Gram of kappa (bf16 MFMA, exact in fp32), T, and A by
//                        blocked inversion on fp32 MFMA: each 16x16 diagonal block as the product
//                        (I - T)(I + T^2)(I + T^4)(I + T^8) (T^16 = 0 in a block), then the
//                        off-diagonal blocks by doubling, A_RC = -A_RR T_RC A_CC for 16-, 32- and
//                        64-row halves.  A goes to the workspace as the bf16 rounding of its
//                        lower 16x16 tiles (18 KB per chunk), the only intermediate of the chunk.
// K4 chunk_maps2_bf16    grid (B*H*G)    the affine maps S_end = Phi S_start + P of G segments of
//                        consecutive chunks (Phi: from I with nu = 0; P: from 0), both in one
//                        block (D = 128; chunk_maps_bf16 builds them in two blocks for D < 128)
//    chunk_seg_scan_bf16 grid (B*H)      the segment start states
//    chunk_replay_bf16   grid (B*H, G)   each segment reruns its chunks from its start state and
//                        writes the output rows; the last segment writes the final state.
//
// In K4 a wave owns 32 columns of the state (the value dimension).  Every product of a
// chunk -- kappa S, A B, kappa^T R', q S, P R -- contracts over an index the wave holds
// whole, so a wave's chain of MFMAs never waits for another wave: the accumulator tiles
// of one product are the B operand of the next.  A 16x16x32 B operand made of two
// accumulator tiles (rows 32s..32s+15 and 32s+16..32s+31) holds in lane (lr, lg) the k
// rows 32s + 4lg + e and 32s + 16 + 4lg + e (e = 0..3); the A operand of such a product
// is read in the same k order.  The shared operands of a chunk (kappa, nu and q rows, the
// A tiles) are staged in LDS once per chunk; kappa^T operands are read from the kappa
// rows with ds_read_b64_tr_b16.  The state stays fp32 in registers.  fp32 operands enter
// the bf16 MFMAs as hi + lo bf16 pairs, which keeps about 16 mantissa bits -- hi.Y + lo.Y
// against a bf16 Y, hi.hi + hi.lo + lo.hi between two fp32 ones -- where the result carries
// the state or the output: S in q S, R' in the update kappa^T R', B in A B (against A's bf16
// rounding), P and R in P R.  Two products take one bf16 operand: X = kappa S reads S's bf16
// rounding, and A is stored as bf16.  Measured on a CPU emulation of these roundings (one
// head, T = 2048 and 8192, the north-star input distribution): output and final state within
// 7e-4 of the fp64 recurrence, against 8e-6 and 4e-6 with hi + lo in every product and the
// 2e-2 bound for bf16 inputs; X and A B with all hi + lo terms cost 52 more MFMAs per wave
// and chunk and twice the A staging.
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace sgsa {

namespace {

constexpr int L = 64;
constexpr int DP = 128;
constexpr int PK = DP + 8;     // bf16 pitch of a staged kappa / nu / q row (272 B)
constexpr int AP = 24;         // bf16 pitch of a staged A tile row (48 B: a tile's row reads hit distinct banks)
constexpr int TP = 17;         // fp32 pitch of a 16x16 tile in K3

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ bf16x8 as_bf8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

__device__ __forceinline__ uint4 zero4() { return make_uint4(0, 0, 0, 0); }

// 8 consecutive bf16 of an input row starting at d0 (zero outside [0,D) or !valid).
__device__ __forceinline__ uint4 load8(const bf16_t* row, int d0, int D, bool valid) {
  if (!valid || d0 >= D) return zero4();
  if ((D & 7) == 0) return *reinterpret_cast<const uint4*>(row + d0);
  u16x8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = (d0 + j < D) ? row[d0 + j].bits : (uint16_t)0;
  return __builtin_bit_cast(uint4, r);
}

// Two floats to two bf16 (round to nearest even) in one v_cvt_pk_bf16_f32; a in bits 0-15.
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2_t));
}

// x = hi + lo: hi the bf16 rounding of x, lo the bf16 rounding of the remainder (4 values each).
__device__ __forceinline__ void split4(const f4& x, uint2& hi, uint2& lo) {
  const uint32_t h0 = pack2(x[0], x[1]), h1 = pack2(x[2], x[3]);
  hi = make_uint2(h0, h1);
  lo = make_uint2(pack2(x[0] - __uint_as_float(h0 << 16), x[1] - __uint_as_float(h0 & 0xffff0000u)),
                  pack2(x[2] - __uint_as_float(h1 << 16), x[3] - __uint_as_float(h1 & 0xffff0000u)));
}

__device__ __forceinline__ f4 unsplit4(uint2 hi, uint2 lo) {
  f4 x;
  x[0] = __uint_as_float(hi.x << 16) + __uint_as_float(lo.x << 16);
  x[1] = __uint_as_float(hi.x & 0xffff0000u) + __uint_as_float(lo.x & 0xffff0000u);
  x[2] = __uint_as_float(hi.y << 16) + __uint_as_float(lo.y << 16);
  x[3] = __uint_as_float(hi.y & 0xffff0000u) + __uint_as_float(lo.y & 0xffff0000u);
  return x;
}

// B operand from two accumulator tiles (k rows 32s + 4lg + e, then 32s + 16 + 4lg + e).
__device__ __forceinline__ bf16x8 cat(uint2 a, uint2 b) { return as_bf8(make_uint4(a.x, a.y, b.x, b.y)); }

// A operand of step s from a row-major bf16 row in LDS, in that k order.
__device__ __forceinline__ bf16x8 rowop_p(const uint16_t* row, int s, int lg) {
  const uint2 a = *reinterpret_cast<const uint2*>(row + 32 * s + 4 * lg);
  const uint2 b = *reinterpret_cast<const uint2*>(row + 32 * s + 16 + 4 * lg);
  return cat(a, b);
}

// A or B operand of step s in the MFMA's own k order (both operands read from rows).
__device__ __forceinline__ bf16x8 rowop(const uint16_t* row, int s, int lg) {
  return as_bf8(*reinterpret_cast<const uint4*>(row + 32 * s + 8 * lg));
}

__device__ __forceinline__ s16x4 lds_tr(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
}

// ds_read_b64_tr_b16: within 16 lanes, lane i receives element i % 4 of the 8 bytes
// lane 4e + i / 4 addresses (e = 0..3).  Lane m addressing row j0 + m / 4 at column
// d0 + 4 (m % 4) therefore hands lane i the column d0 + i of rows j0 .. j0 + 3.

// e^x through v_exp_f32 (2^x): one multiply and the hardware exponential.
__device__ __forceinline__ float fexp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// sample i of a chunk -> (token offset, which input)
template <bool SP> __device__ __forceinline__ int samp_t(int i) { return SP ? (i >> 1) : i; }
template <bool SP> __device__ __forceinline__ int samp_r(int i) { return SP ? (i & 1) : 0; }

__device__ __host__ constexpr int tri(int I, int J) { return I * (I + 1) / 2 + J; }

// K4 stages the kappa / nu rows of a chunk input-major: the local-write rows (tokens
// 0..63) first, the sparse-write rows after them, shifted by 16 bytes so that the rows
// of one sample pair sit in different banks.  Element offset of sample i's row:
template <bool SP> __device__ __forceinline__ int krow(int i) {
  return SP ? ((i & 1) ? (64 + (i >> 1)) * PK + 8 : (i >> 1) * PK) : i * PK;
}
template <int M> constexpr int krows_elems() { return M * PK + (M == 2 * L ? 8 : 0); }

// kappa^T as the A operand of step s (rows: dims 16r .. 16r + 15; k: samples in the
// accumulator k order): two transposing reads of the staged kappa rows.
template <bool SP>
__device__ __forceinline__ bf16x8 kapT_op(const uint16_t* kap, int r, int s, int lr, int lg) {
  const int d = 16 * r + 4 * (lr & 3);
  const s16x4 a = lds_tr(kap + krow<SP>(32 * s + 4 * lg + (lr >> 2)) + d);
  const s16x4 b = lds_tr(kap + krow<SP>(32 * s + 16 + 4 * lg + (lr >> 2)) + d);
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}


// ---------------------------------------------------------------------------
// K3
// ---------------------------------------------------------------------------

// Z = X Y for 16x16 fp32 tiles (row-major, pitch TP): four v_mfma_f32_16x16x4_f32 (lane l
// supplies X[l%16][4s + l/16] and Y[4s + l/16][l%16]); result in the accumulator layout.
__device__ __forceinline__ f4 mm16(const float* X, const float* Y, f4 acc, int lr, int lg) {
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = mma_f32(X[lr * TP + 4 * s + lg], Y[(4 * s + lg) * TP + lr], acc);
  return acc;
}

__device__ __forceinline__ void st16(float* Z, const f4& v, int lr, int lg) {
#pragma unroll
  for (int e = 0; e < 4; ++e) Z[(4 * lg + e) * TP + lr] = v[e];
}

__device__ __forceinline__ f4 ld16(const float* Z, int lr, int lg) {
  f4 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = Z[(4 * lg + e) * TP + lr];
  return v;
}

constexpr int K3W = 8;   // waves of a chunk_inv_bf16 block

// The backward's per-chunk operands (chunk_bwd.hip), fp32: A [M][M] row-major (zero
// above the diagonal), W = A diag(e^{l_tau}) kappa and U = A nu [M][DP], the log-decay
// prefix [L].  Samples past T have zero kappa and nu rows.
struct K3Bwd {
  float* A;
  float* W;
  float* U;
  float* logd;
  const bf16_t* v;
  const bf16_t* sv;
};

// BWD: the backward's form -- the same Gram and inverse, then K3Bwd's outputs in place
// of the bf16 A tiles.
template <int M, bool FULL, bool BWD = false>
__global__ __launch_bounds__(64 * K3W) void chunk_inv_bf16(const bf16_t* __restrict__ k, const bf16_t* __restrict__ sk,
                                                    const float* __restrict__ beta, const float* __restrict__ alpha,
                                                    const float* __restrict__ gamma, int T, int H, int D, int NT,
                                                    uint16_t* __restrict__ Aout, K3Bwd bw = K3Bwd{}) {
  constexpr bool SP = M == 2 * L;
  constexpr int NB = M / 16;
  constexpr int NTL = NB * (NB + 1) / 2;
  constexpr int UNION = M * PK * 2;                      // bytes: kappa rows; later the product scratch
  constexpr int NDW = K3W < NB ? K3W : NB;               // waves holding a diagonal block
  static_assert(NDW * 4 * 16 * TP * 4 <= UNION && 16 * 16 * TP * 4 <= UNION, "scratch exceeds the union");
  __shared__ __align__(16) unsigned char un[UNION];
  __shared__ __align__(16) float Tt[NTL * 16 * TP];      // lower tiles of T, then of A
  __shared__ float lam[M];
  __shared__ float logd[L];
  __shared__ float dtau[BWD ? M : 1];   // BWD: e^{l_tau_i} per sample
  uint16_t* kap = reinterpret_cast<uint16_t*>(un);

  const int c = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const int lr = lane & 15, lg = lane >> 4;
  const int t0 = c * L;

  if (tid < L) {
    const int t = t0 + tid;
    float x = 0.f;
    if (t < T) x = logf(fmaxf(gamma[(long)(b * T + t) * H + h], 1e-6f));
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float n = __shfl_up(x, o, 64);
      if (lane >= o) x += n;
    }
    logd[tid] = x;
  }
  if (tid < M) {
    const int t = t0 + samp_t<SP>(tid);
    float lm = 0.f;
    if (t < T) lm = samp_r<SP>(tid) ? alpha[(long)(b * T + t) * H + h] : beta[(long)(b * T + t) * H + h];
    lam[tid] = lm;
  }
  {
    constexpr int NK = M * (DP / 8) / (64 * K3W);   // all of a thread's loads in flight before its stores
    uint4 kx[NK];
#pragma unroll
    for (int j = 0; j < NK; ++j) {
      const int e = tid + 64 * K3W * j;
      const int i = e / (DP / 8), cv = e % (DP / 8);
      const int t = t0 + samp_t<SP>(i);
      const bf16_t* src = samp_r<SP>(i) ? sk : k;
      if constexpr (FULL)   // a token past T reads token T - 1: its samples have lam = 0 (zero T column)
        kx[j] = *reinterpret_cast<const uint4*>(src + ((long)(b * T + min(t, T - 1)) * H + h) * DP + 8 * cv);
      else kx[j] = load8(src + ((long)(b * T + (t < T ? t : 0)) * H + h) * D, 8 * cv, D, t < T);
    }
#pragma unroll
    for (int j = 0; j < NK; ++j) {
      const int e = tid + 64 * K3W * j;
      *reinterpret_cast<uint4*>(&kap[(e / (DP / 8)) * PK + 8 * (e % (DP / 8))]) = kx[j];
    }
  }
  __syncthreads();

  // Gram on the lower tiles -> T
  for (int ti = w; ti < NTL; ti += K3W) {
    int I = 0;
    while (tri(I + 1, 0) <= ti) ++I;
    const int J = ti - tri(I, 0);
    f4 acc = f4_zero();
#pragma unroll
    for (int s = 0; s < DP / 32; ++s)
      acc = mma_bf16(rowop(kap + (16 * I + lr) * PK, s, lg), rowop(kap + (16 * J + lr) * PK, s, lg), acc);
    const int j = 16 * J + lr, tJ = samp_t<SP>(j);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * I + 4 * lg + e, tI = samp_t<SP>(i);
      acc[e] = (tJ < tI) ? lam[j] * expf(logd[tI] - logd[tJ]) * acc[e] : 0.f;
    }
    st16(Tt + ti * 16 * TP, acc, lr, lg);
  }
  __syncthreads();   // kappa rows are dead from here on: the union becomes product scratch

  // Diagonal blocks: A_II = (I - T)(I + T^2)(I + T^4)(I + T^8), T strictly lower (T^16 = 0).
  {
    float* sc = reinterpret_cast<float*>(un) + w * 4 * 16 * TP;   // this wave's four scratch tiles
    float* s0 = sc;
    float* s1 = sc + 16 * TP;
    float* s2 = sc + 2 * 16 * TP;
    float* s3 = sc + 3 * 16 * TP;
    for (int Ib = w; Ib < NB; Ib += K3W) {
      float* Tb = Tt + tri(Ib, Ib) * 16 * TP;
      const f4 t1 = ld16(Tb, lr, lg);
      const f4 t2 = mm16(Tb, Tb, f4_zero(), lr, lg);
      st16(s0, t2, lr, lg);
      wave_lds_sync();
      const f4 t3 = mm16(Tb, s0, f4_zero(), lr, lg);
      const f4 t4 = mm16(s0, s0, f4_zero(), lr, lg);
      st16(s1, t4, lr, lg);
      wave_lds_sync();
      st16(s2, mm16(s1, s1, f4_zero(), lr, lg), lr, lg);   // T^8
      f4 p1;
#pragma unroll
      for (int e = 0; e < 4; ++e) p1[e] = (4 * lg + e == lr ? 1.f : 0.f) - t1[e] + t2[e] - t3[e];
      st16(s3, p1, lr, lg);
      wave_lds_sync();
      const f4 p2 = mm16(s3, s1, p1, lr, lg);   // P1 + P1 T^4
      st16(s0, p2, lr, lg);
      wave_lds_sync();
      const f4 a = mm16(s0, s2, p2, lr, lg);    // P2 + P2 T^8
      st16(Tb, a, lr, lg);
      wave_lds_sync();
    }
  }
  __syncthreads();

  // Off-diagonal blocks by doubling: for halves of nb tiles, rows R = (2p+1)nb.., cols
  // C = 2p nb..: Z = T_RC A_CC, then A_RC = -A_RR Z.
  float* Zs = reinterpret_cast<float*>(un);
#pragma unroll
  for (int nb = 1; nb < NB; nb <<= 1) {
    const int npair = NB / (2 * nb);
    const int items = npair * nb * nb;
    for (int it = w; it < items; it += K3W) {
      const int p = it / (nb * nb), i = (it / nb) % nb, j = it % nb;
      const int Ri = (2 * p + 1) * nb + i, C0 = 2 * p * nb;
      f4 z = f4_zero();
      for (int kk = j; kk < nb; ++kk)
        z = mm16(Tt + tri(Ri, C0 + kk) * 16 * TP, Tt + tri(C0 + kk, C0 + j) * 16 * TP, z, lr, lg);
      st16(Zs + it * 16 * TP, z, lr, lg);
    }
    __syncthreads();
    for (int it = w; it < items; it += K3W) {
      const int p = it / (nb * nb), i = (it / nb) % nb, j = it % nb;
      const int R0 = (2 * p + 1) * nb, C0 = 2 * p * nb;
      f4 a = f4_zero();
      for (int kk = 0; kk <= i; ++kk)
        a = mm16(Tt + tri(R0 + i, R0 + kk) * 16 * TP, Zs + ((p * nb + kk) * nb + j) * 16 * TP, a, lr, lg);
      st16(Tt + tri(R0 + i, C0 + j) * 16 * TP, -a, lr, lg);
    }
    __syncthreads();
  }

  if constexpr (!BWD) {
    // A -> workspace: [NTL tiles][16][16] bf16 (round to nearest)
    uint16_t* dst = Aout + ((long)bh * NT + c) * NTL * 256;
    for (int e = tid; e < NTL * 64; e += 64 * K3W) {
      const int tl = e >> 6, r = (e >> 2) & 15, cg = e & 3;
      const float* src = Tt + tl * 16 * TP + r * TP + 4 * cg;
      *reinterpret_cast<uint2*>(dst + tl * 256 + r * 16 + 4 * cg) = make_uint2(pack2(src[0], src[1]), pack2(src[2], src[3]));
    }
  } else {
    const long cid = (long)bh * NT + c;
    if (tid < L) bw.logd[cid * L + tid] = logd[tid];
    // A: [M][M] fp32, row-major, zero above the diagonal
    float* Ac = bw.A + cid * M * M;
    for (int e = tid; e < M * M; e += 64 * K3W) {
      const int i = e / M, j = e % M, I = i >> 4, J = j >> 4;
      Ac[e] = (J < I || (J == I && (j & 15) <= (i & 15))) ? Tt[tri(I, J) * 16 * TP + (i & 15) * TP + (j & 15)] : 0.f;
    }
    // W = A diag(e^{l_tau}) kappa, then U = A nu: the rows staged again in the union
    // (zero past T and past D), fp32 MFMA (A fp32, the bf16 rows exact in fp32).
    // Output tile (I, n), I < NB, n < DP / 16: wave w takes tiles w, w + K3W, ..
    float* dt = dtau;
    for (int pass = 0; pass < 2; ++pass) {
      __syncthreads();   // the union's previous contents are no longer read
      const bf16_t* lo_src = pass == 0 ? k : bw.v;
      const bf16_t* sp_src = pass == 0 ? sk : bw.sv;
      for (int e = tid; e < M * (DP / 8); e += 64 * K3W) {
        const int i = e / (DP / 8), cv = e % (DP / 8);
        const int t = t0 + samp_t<SP>(i);
        const bf16_t* src = samp_r<SP>(i) ? sp_src : lo_src;
        *reinterpret_cast<uint4*>(&kap[i * PK + 8 * cv]) =
            load8(src + ((long)(b * T + (t < T ? t : 0)) * H + h) * D, 8 * cv, D, t < T);
      }
      if (pass == 0 && tid < M) dt[tid] = expf(logd[samp_t<SP>(tid)]);
      __syncthreads();
      float* dst = (pass == 0 ? bw.W : bw.U) + cid * M * DP;
      for (int ot = w; ot < NB * (DP / 16); ot += K3W) {
        const int I = ot / (DP / 16), n = ot % (DP / 16);
        f4 acc = f4_zero();
        for (int J = 0; J <= I; ++J) {
          const float* At = Tt + tri(I, J) * 16 * TP;
#pragma unroll
          for (int s4 = 0; s4 < 4; ++s4) {
            const int kk = 16 * J + 4 * s4 + lg;
            float bb = bf16_to_f32(kap[kk * PK + 16 * n + lr]);
            if (pass == 0) bb *= dt[kk];
            const float aa = (J == I && 4 * s4 + lg > lr) ? 0.f : At[lr * TP + 4 * s4 + lg];
            acc = mma_f32(aa, bb, acc);
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[(long)(16 * I + 4 * lg + e) * DP + 16 * n + lr] = acc[e];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// K4: the state passes.
// ---------------------------------------------------------------------------

// Number of segments of the state pass: enough (b*h, segment) blocks to fill
// the GPU, at least 8 chunks per segment, at most 16 segments.
inline int seg_count(int BH, int NT) {
  int g = (256 + BH - 1) / BH;
  g = g < 16 ? g : 16;
  const int gmax = (NT + 7) / 8;
  g = g < gmax ? g : gmax;
  return g < 1 ? 1 : g;
}

// Per-chunk gate tables in LDS: the chunk-local log-decay prefix l_t, e^{l_t}, and per
// sample the write strength lam_i and the factor lam_i e^{l_L - l_tau_i} of R'.
template <int M>
struct GateTab {
  float logd[L];
  float el[L];
  float lam[M];
  float fac[M];
};

// The gate inputs of chunk token t0 + lane (wave 0, one token per lane), loaded into
// registers ahead of use: gamma, beta and alpha (tokens past T: gamma 1, no write).
struct GateIn {
  float g, b, a;
};
template <bool SP>
__device__ __forceinline__ GateIn load_gates(const float* __restrict__ beta, const float* __restrict__ alpha,
                                             const float* __restrict__ gamma, int T, int H, int b, int h, int t0,
                                             int lane) {
  GateIn gi{1.f, 0.f, 0.f};
  const int t = t0 + lane;
  if (t < T) {
    const long o = (long)(b * T + t) * H + h;
    gi.g = gamma[o];
    gi.b = beta[o];
    if (SP) gi.a = alpha[o];
  }
  return gi;
}
// Fills the tables from load_gates' registers (wave 0).
template <int M>
__device__ __forceinline__ void store_gates(const GateIn& gi, int lane, GateTab<M>& gt) {
  constexpr bool SP = M == 2 * L;
  float x = __logf(fmaxf(gi.g, 1e-6f));
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float n = __shfl_up(x, o, 64);
    if (lane >= o) x += n;
  }
  gt.logd[lane] = x;
  gt.el[lane] = fexp(x);
  const float dec = fexp(__shfl(x, 63, 64) - x);   // e^{l_L - l_t}
#pragma unroll
  for (int r = 0; r < (SP ? 2 : 1); ++r) {
    const int i = SP ? 2 * lane + r : lane;
    const float lm = r ? gi.a : gi.b;
    gt.lam[i] = lm;
    gt.fac[i] = lm * dec;
  }
}

// Fills the tables (tokens past T: no decay, no write); wave 0 does it all, one token per
// lane, so the factors come from the scan in registers.
template <int M>
__device__ __forceinline__ void stage_gates(const float* __restrict__ beta, const float* __restrict__ alpha,
                                            const float* __restrict__ gamma, int T, int H, int b, int h, int t0,
                                            int tid, GateTab<M>& gt) {
  constexpr bool SP = M == 2 * L;
  if (tid < 64) {
    const int t = t0 + tid;
    float x = 0.f;
    if (t < T) x = __logf(fmaxf(gamma[(long)(b * T + t) * H + h], 1e-6f));
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float n = __shfl_up(x, o, 64);
      if (tid >= o) x += n;
    }
    gt.logd[tid] = x;
    gt.el[tid] = fexp(x);
    const float dec = fexp(__shfl(x, 63, 64) - x);   // e^{l_L - l_t}
#pragma unroll
    for (int r = 0; r < (SP ? 2 : 1); ++r) {
      const int i = SP ? 2 * tid + r : tid;
      float lm = 0.f;
      if (t < T) lm = r ? alpha[(long)(b * T + t) * H + h] : beta[(long)(b * T + t) * H + h];
      gt.lam[i] = lm;
      gt.fac[i] = lm * dec;
    }
  }
}

// Stage chunk c's shared operands in LDS: kappa rows, nu rows (USE_NU), q rows (USE_Q),
// the A tiles (rows padded to AP), the log-decay prefix and the write strengths.  Each
// thread issues all of its global loads before its first LDS store, so the chunk's
// loads are in flight together.  FULL (D = DP): rows are read without conditions -- a
// token past T reads token T - 1 instead of zeros, which is harmless: such a sample's
// write strength is 0 (no write, no T_ij column), A rows of valid samples only involve
// earlier samples, and it only reaches output rows t >= T, which are not stored.  For
// D < DP, dims >= D must read as 0, and rows past T do too.
template <int M, int NTHR, bool USE_NU, bool USE_Q, bool FULL>
__device__ __forceinline__ void stage_chunk(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                                            const bf16_t* __restrict__ v, const bf16_t* __restrict__ sk,
                                            const bf16_t* __restrict__ sv, const float* __restrict__ beta,
                                            const float* __restrict__ alpha, const float* __restrict__ gamma,
                                            const uint16_t* __restrict__ Ain, int T, int H, int D, int NT, int b,
                                            int h, int bh, int c, int tid, uint16_t* kap, uint16_t* nuv,
                                            uint16_t* qr, uint16_t* At, GateTab<M>& gt) {
  constexpr bool SP = M == 2 * L;
  constexpr int NB = M / 16;
  constexpr int NTL = NB * (NB + 1) / 2;
  constexpr int NK = M * (DP / 8) / NTHR;              // 16-byte row pieces per thread
  constexpr int NQ = L * (DP / 8) / NTHR;
  constexpr int NA = (NTL * 32 + NTHR - 1) / NTHR;     // 16-byte A tile pieces per thread
  static_assert(NK * NTHR == M * (DP / 8) && NQ * NTHR == L * (DP / 8), "row pieces must divide evenly");
  const int t0 = c * L;
  uint4 kx[NK], nx[USE_NU ? NK : 1], qx[USE_Q ? NQ : 1], ax[NA];
  const uint16_t* src = Ain + ((long)bh * NT + c) * NTL * 256;
#pragma unroll
  for (int j = 0; j < NA; ++j) {
    const int e = tid + j * NTHR;   // tile tp, row r, 16-byte half hf
    const int tp = e >> 5, r = (e >> 1) & 15, hf = e & 1;
    if constexpr (NTL * 32 % NTHR == 0) ax[j] = *reinterpret_cast<const uint4*>(src + tp * 256 + r * 16 + 8 * hf);
    else ax[j] = e < NTL * 32 ? *reinterpret_cast<const uint4*>(src + tp * 256 + r * 16 + 8 * hf) : zero4();
  }
#pragma unroll
  for (int j = 0; j < NK; ++j) {
    const int e = tid + j * NTHR;
    const int i = e / (DP / 8), cv = e % (DP / 8);
    const int t = t0 + samp_t<SP>(i);
    const bool r1 = samp_r<SP>(i);
    if constexpr (FULL) {
      const long roff = ((long)(b * T + min(t, T - 1)) * H + h) * DP + 8 * cv;
      kx[j] = *reinterpret_cast<const uint4*>((r1 ? sk : k) + roff);
      if constexpr (USE_NU) nx[j] = *reinterpret_cast<const uint4*>((r1 ? sv : v) + roff);
    } else {
      const long roff = ((long)(b * T + (t < T ? t : 0)) * H + h) * D;
      kx[j] = load8((r1 ? sk : k) + roff, 8 * cv, D, t < T);
      if constexpr (USE_NU) nx[j] = load8((r1 ? sv : v) + roff, 8 * cv, D, t < T);
    }
  }
  if constexpr (USE_Q) {
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const int e = tid + j * NTHR;
      const int i = e / (DP / 8), cv = e % (DP / 8);
      const int t = t0 + i;
      if constexpr (FULL) qx[j] = *reinterpret_cast<const uint4*>(q + ((long)(b * T + min(t, T - 1)) * H + h) * DP + 8 * cv);
      else qx[j] = load8(q + ((long)(b * T + (t < T ? t : 0)) * H + h) * D, 8 * cv, D, t < T);
    }
  }
  stage_gates<M>(beta, alpha, gamma, T, H, b, h, t0, tid, gt);
#pragma unroll
  for (int j = 0; j < NA; ++j) {
    const int e = tid + j * NTHR;
    const int tp = e >> 5, r = (e >> 1) & 15, hf = e & 1;
    if (e < NTL * 32) *reinterpret_cast<uint4*>(&At[(tp * 16 + r) * AP + 8 * hf]) = ax[j];
  }
#pragma unroll
  for (int j = 0; j < NK; ++j) {
    const int e = tid + j * NTHR;
    const int i = e / (DP / 8), cv = e % (DP / 8);
    *reinterpret_cast<uint4*>(&kap[krow<SP>(i) + 8 * cv]) = kx[j];
    if constexpr (USE_NU) *reinterpret_cast<uint4*>(&nuv[krow<SP>(i) + 8 * cv]) = nx[j];
  }
  if constexpr (USE_Q) {
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const int e = tid + j * NTHR;
      const int i = e / (DP / 8), cv = e % (DP / 8);
      *reinterpret_cast<uint4*>(&qr[i * PK + 8 * cv]) = qx[j];
    }
  }
}

// The staging of stage_chunk for D = DP as direct-to-LDS buffer loads (buffer_load_dwordx4
// ... lds: lane l of an instruction fills the 16 bytes at its LDS base + 16 l), which
// hold no data registers, so all of a chunk's loads are issued back to back; in pieces, so
// that a chunk's operands can load while the previous chunk still computes.  One buffer
// resource per input covers its head's rows [0, T): a token past T reads as zeros.  A
// 272-byte kappa / nu / q row is 17 slots (the 17th is its pad and re-reads the first);
// a 48-byte A tile row is 3 (2 data, 1 pad).  The caller waits for the loads (vmcnt) and
// then publishes them with a barrier.
struct DmaCtx {
  int T, H, NT, b, h, bh, lane, w;
  // per-lane byte offsets, the same for every chunk: row slots of load i = w + 8 u
  // (row (64 i + lane) / 17 of the chunk, 16-byte piece (64 i + lane) % 17) and A
  // tile slots (row (64 i + lane) / 3, piece (64 i + lane) % 3); the chunk's start
  // is added per load (rows) or is the buffer's base (A tiles)
  unsigned ro[3], ao[4];
  __device__ DmaCtx(int T_, int H_, int NT_, int b_, int h_, int bh_, int lane_, int w_)
      : T(T_), H(H_), NT(NT_), b(b_), h(h_), bh(bh_), lane(lane_), w(w_) {
    const int rbytes = H * DP * 2;
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      const int sl = 64 * (w + 8 * u) + lane;
      const int row = sl / 17, pc = sl % 17;
      ro[u] = (unsigned)(row * rbytes + 16 * (pc < 16 ? pc : 0));
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int sl = 64 * (w + 8 * u) + lane;
      const int row = sl / 3, pc = sl % 3;
      ao[u] = (unsigned)(row * 32 + 16 * (pc < 2 ? pc : 0));
    }
  }
};
// 64 rows of one input, tokens c L .. c L + 63, into dst (rows of PK elements)
template <int NW>
__device__ __forceinline__ void dma_rows(const DmaCtx& x, const bf16_t* base, int c, uint16_t* dst) {
  static_assert(NW == 8, "the per-lane offsets are laid out for 8 waves");
  constexpr int RI = L * 17 / 64;
  const long hoff = ((long)x.b * x.T * x.H + x.h) * DP;
  const int rbytes = x.H * DP * 2;
  const int nrec = (x.T - 1) * rbytes + DP * 2;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(base + hoff), 0, nrec, 0x00020000);
  const unsigned coff = (unsigned)(c * L * rbytes);
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    const int i = x.w + NW * u;
    if (i < RI)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(dst + 512 * i), 16,
                                               x.ro[u] + coff, 0, 0, 0);
  }
}
// kappa (or nu) rows of chunk c: the local rows, then (SP) the sparse rows 16 bytes on
template <int M, int NW>
__device__ __forceinline__ void dma_pair(const DmaCtx& x, const bf16_t* a, const bf16_t* sa, int c, uint16_t* dst) {
  dma_rows<NW>(x, a, c, dst);
  if constexpr (M == 2 * L) dma_rows<NW>(x, sa, c, dst + 64 * PK + 8);
}
// The A tile area: the tiles' rows, rounded up to whole DMA instructions (every lane of
// the last one writes; its slots past the tiles read past the buffer, as zeros).
template <int M> constexpr int a_instr() { return ((M / 16) * (M / 16 + 1) / 2 * 16 * 3 + 63) / 64; }
template <int M> constexpr int at_elems() {
  return a_instr<M>() * 512 > (M / 16) * (M / 16 + 1) / 2 * 16 * AP ? a_instr<M>() * 512
                                                                      : (M / 16) * (M / 16 + 1) / 2 * 16 * AP;
}
// the A tiles of chunk c
template <int M, int NW>
__device__ __forceinline__ void dma_A(const DmaCtx& x, const uint16_t* Ain, int c, uint16_t* At) {
  static_assert(NW == 8, "the per-lane offsets are laid out for 8 waves");
  constexpr int NB = M / 16;
  constexpr int NTL = NB * (NB + 1) / 2;
  constexpr int AI = a_instr<M>();
  static_assert(AI <= 4 * NW, "A tiles beyond the per-lane offsets");
  const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(Ain + ((long)x.bh * x.NT + c) * NTL * 256), 0, NTL * 512, 0x00020000);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = x.w + NW * u;
    if (i < AI)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ars, (__attribute__((address_space(3))) void*)(At + 512 * i), 16,
                                               x.ao[u], 0, 0, 0);
  }
}

// A wave's state is kept in 16-column tiles: S[r] holds S[16r + 4lg + e][col + lr] of the
// tile's columns col .. col + 15 (r: d_k row tile).  fp32 operands enter the products as
// Op pairs, each the B operand of one k step of 32 (hi and lo bf16 halves of two
// accumulator tiles, in the k order of cat()).
struct Op {
  uint4 h, l;
};

// Tiles 2s and 2s + 1 of x as the operand of step s.
template <int N>
__device__ __forceinline__ void pack_ops(const f4 (&x)[N], Op (&op)[N / 2]) {
#pragma unroll
  for (int s = 0; s < N / 2; ++s) {
    uint2 ha, la, hb, lb;
    split4(x[2 * s], ha, la);
    split4(x[2 * s + 1], hb, lb);
    op[s].h = make_uint4(ha.x, ha.y, hb.x, hb.y);
    op[s].l = make_uint4(la.x, la.y, lb.x, lb.y);
  }
}

// R = A B for one 16-column tile at column col, with X = kappa S and
// B = nu - e^{l_tau} X (nu = 0 for !USE_NU); Sop is the state tile as operands.
template <int M, bool USE_NU>
__device__ __forceinline__ void tile_residual(const Op (&Sop)[DP / 32], const uint16_t* kap, const uint16_t* nuv,
                                              const uint16_t* At, const float* el, int col, int lr, int lg,
                                              f4 (&R)[M / 16]) {
  constexpr bool SP = M == 2 * L;
  constexpr int NB = M / 16;
  Op Bop[NB / 2];
#pragma unroll
  for (int sp = 0; sp < NB / 2; ++sp) {
    f4 y[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int I = 2 * sp + hf;
      f4 x = f4_zero();
      const uint16_t* kr = kap + krow<SP>(16 * I + lr);
#pragma unroll
      for (int s = 0; s < DP / 32; ++s) x = mma_bf16(rowop_p(kr, s, lg), as_bf8(Sop[s].h), x);
      float ef[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) ef[e] = el[samp_t<SP>(16 * I + 4 * lg + e)];
      if constexpr (USE_NU) {
        const s16x4 nv = lds_tr(nuv + krow<SP>(16 * I + 4 * lg + (lr >> 2)) + col + 4 * (lr & 3));
#pragma unroll
        for (int e = 0; e < 4; ++e) y[hf][e] = bf16_to_f32((uint16_t)nv[e]) - ef[e] * x[e];
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) y[hf][e] = -ef[e] * x[e];
      }
    }
    uint2 ha, la, hb, lb;
    split4(y[0], ha, la);
    split4(y[1], hb, lb);
    Bop[sp].h = make_uint4(ha.x, ha.y, hb.x, hb.y);
    Bop[sp].l = make_uint4(la.x, la.y, lb.x, lb.y);
    __builtin_amdgcn_sched_barrier(0);   // one pair of tile rows at a time
  }
  // tile row I takes the A tiles (I, J <= I)
#pragma unroll
  for (int I = 0; I < NB; ++I) {
    R[I] = f4_zero();
#pragma unroll
    for (int s = 0; 2 * s <= I; ++s) {
      const uint2 h0 = *reinterpret_cast<const uint2*>(At + tri(I, 2 * s) * 16 * AP + lr * AP + 4 * lg);
      uint2 h1 = make_uint2(0, 0);
      if (2 * s + 1 <= I) h1 = *reinterpret_cast<const uint2*>(At + tri(I, 2 * s + 1) * 16 * AP + lr * AP + 4 * lg);
      const bf16x8 ah = cat(h0, h1);
      R[I] = mma_bf16(ah, as_bf8(Bop[s].h), R[I]);
      R[I] = mma_bf16(ah, as_bf8(Bop[s].l), R[I]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// R' = lam e^{l_L - l_tau} R (the per-sample factors from the gate table) as operands.
template <int M>
__device__ __forceinline__ void scaled_ops(const f4 (&R)[M / 16], const float* facg, int lg, Op (&op)[M / 32]) {
  f4 y[M / 16];
#pragma unroll
  for (int I = 0; I < M / 16; ++I) {
    const float4 f = *reinterpret_cast<const float4*>(facg + 16 * I + 4 * lg);
    y[I][0] = R[I][0] * f.x;
    y[I][1] = R[I][1] * f.y;
    y[I][2] = R[I][2] * f.z;
    y[I][3] = R[I][3] * f.w;
  }
  pack_ops<M / 16>(y, op);
}

// S <- e^{l_L} S + kappa^T R' for one 16-column tile.
template <int M>
__device__ __forceinline__ void tile_update(f4 (&S)[DP / 16], const Op (&Rop)[M / 32], const uint16_t* kap, float DL,
                                            int lr, int lg) {
#pragma unroll
  for (int r = 0; r < DP / 16; ++r) {
    f4 acc = S[r] * DL;
#pragma unroll
    for (int s = 0; s < M / 32; ++s) {
      const bf16x8 a = kapT_op<M == 2 * L>(kap, r, s, lr, lg);
      acc = mma_bf16(a, as_bf8(Rop[s].h), acc);
      acc = mma_bf16(a, as_bf8(Rop[s].l), acc);
    }
    S[r] = acc;
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The chunks of segment g for one state: PHI = false runs P (start 0, with nu), PHI = true
// runs Phi (start I, nu = 0), each wave over one 16-column tile of the state.  kapb holds
// two kappa buffers and gtb two gate tables: with D = DP the next chunk's kappa rows and
// gates load while the current chunk computes, and its nu rows and A tiles as soon as
// every wave has formed R (their buffers are free then); D < DP stages each chunk in turn.
template <int M, bool FULL, bool PHI>
__device__ __forceinline__ void maps_pass(const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
                                          const bf16_t* __restrict__ sk, const bf16_t* __restrict__ sv,
                                          const float* __restrict__ beta, const float* __restrict__ alpha,
                                          const float* __restrict__ gamma, int T, int H, int D, int NT, int CPS,
                                          const uint16_t* __restrict__ Ain, float* __restrict__ dst, uint16_t* kapb,
                                          uint16_t* nuv, uint16_t* At, GateTab<M>* gtb, int bh, int g) {
  constexpr bool SP = M == 2 * L;
  constexpr int NB = M / 16;
  constexpr int KE = krows_elems<M>();
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const int lr = lane & 15, lg = lane >> 4;
  const int col = 16 * w;
  const int cb = g * CPS, ce = min(NT, cb + CPS);

  f4 S[DP / 16];
#pragma unroll
  for (int r = 0; r < DP / 16; ++r)
#pragma unroll
    for (int e = 0; e < 4; ++e) S[r][e] = (PHI && 16 * r + 4 * lg + e == col + lr) ? 1.f : 0.f;

  if constexpr (FULL) {
    const DmaCtx x{T, H, NT, b, h, bh, lane, w};
    if (cb < ce) {
      dma_pair<M, 8>(x, k, sk, cb, kapb);
      if constexpr (!PHI) dma_pair<M, 8>(x, v, sv, cb, nuv);
      dma_A<M, 8>(x, Ain, cb, At);
      if (w == 0) store_gates<M>(load_gates<SP>(beta, alpha, gamma, T, H, b, h, cb * L, lane), lane, gtb[0]);
      __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's loads have landed in LDS
    }
    __syncthreads();
    for (int c = cb; c < ce; ++c) {
      const int cur = (c - cb) & 1;
      const uint16_t* kap = kapb + cur * KE;
      const GateTab<M>& gt = gtb[cur];
      const bool more = c + 1 < ce;   // block-uniform
      GateIn gn{1.f, 0.f, 0.f};
      if (more) {
        dma_pair<M, 8>(x, k, sk, c + 1, kapb + (cur ^ 1) * KE);
        if (w == 0) gn = load_gates<SP>(beta, alpha, gamma, T, H, b, h, (c + 1) * L, lane);
      }
      Op Sop[DP / 32];
      pack_ops<DP / 16>(S, Sop);
      f4 R[NB];
      tile_residual<M, !PHI>(Sop, kap, nuv, At, gt.el, col, lr, lg, R);
      __syncthreads();   // every wave is done with nu and the A tiles
      if (more) {
        if constexpr (!PHI) dma_pair<M, 8>(x, v, sv, c + 1, nuv);
        dma_A<M, 8>(x, Ain, c + 1, At);
      }
      Op Rop[NB / 2];
      scaled_ops<M>(R, gt.fac, lg, Rop);
      tile_update<M>(S, Rop, kap, gt.el[L - 1], lr, lg);
      if (more && w == 0) store_gates<M>(gn, lane, gtb[cur ^ 1]);
      __builtin_amdgcn_s_waitcnt(0x0f70);
      __syncthreads();   // the next chunk's operands are in place; this chunk's are free
    }
  } else {
    GateTab<M>& gt = gtb[0];
    for (int c = cb; c < ce; ++c) {
      __syncthreads();   // every wave is done with the previous chunk's operands
      stage_chunk<M, 512, !PHI, false, FULL>(nullptr, k, v, sk, sv, beta, alpha, gamma, Ain, T, H, D, NT, b, h, bh,
                                             c, tid, kapb, nuv, nullptr, At, gt);
      __syncthreads();
      Op Sop[DP / 32];
      pack_ops<DP / 16>(S, Sop);
      f4 R[NB];
      tile_residual<M, !PHI>(Sop, kapb, nuv, At, gt.el, col, lr, lg, R);
      Op Rop[NB / 2];
      scaled_ops<M>(R, gt.fac, lg, Rop);
      tile_update<M>(S, Rop, kapb, gt.el[L - 1], lr, lg);
    }
  }
#pragma unroll
  for (int r = 0; r < DP / 16; ++r)
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[(long)(16 * r + 4 * lg + e) * DP + col + lr] = S[r][e];
}

// The maps: one block builds P, one Phi, for each (b*h, segment) pair; the end states go
// to sout ([P; Phi] x [B*H][G][DP][DP] fp32).  Block ids go to the XCDs round-robin, so
// the P and Phi blocks of a pair get ids i and i + 8: the same XCD, running side by side,
// so the second reads the chunk operands from that XCD's L2.  1-D grid of
// 16 ceil(B*H*G / 8) blocks.
template <int M, bool FULL>
__global__ __launch_bounds__(512, 1) void chunk_maps_bf16(const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
                                                        const bf16_t* __restrict__ sk, const bf16_t* __restrict__ sv,
                                                        const float* __restrict__ beta, const float* __restrict__ alpha,
                                                        const float* __restrict__ gamma, int T, int H, int D, int NT,
                                                        int CPS, int BH, int G, const uint16_t* __restrict__ Ain,
                                                        float* __restrict__ sout) {
  constexpr int NB = M / 16;
  __shared__ __align__(16) uint16_t kap[(FULL ? 2 : 1) * krows_elems<M>()];
  __shared__ __align__(16) uint16_t nuv[krows_elems<M>()];
  __shared__ __align__(16) uint16_t At[at_elems<M>()];
  __shared__ __align__(16) GateTab<M> gt[FULL ? 2 : 1];
  const int pid = blockIdx.x;
  const int z = (pid >> 3) & 1;                       // 0: P, 1: Phi
  const int pair = (pid >> 4) * 8 + (pid & 7);        // (b*h, segment) pair, b*h fastest
  if (pair >= BH * G) return;                         // block-uniform
  const int bh = pair % BH, g = pair / BH;
  float* dst = sout + (long)((z * BH + bh) * G + g) * DP * DP;
  if (z == 1)
    maps_pass<M, FULL, true>(k, v, sk, sv, beta, alpha, gamma, T, H, D, NT, CPS, Ain, dst, kap, nuv, At, gt, bh, g);
  else
    maps_pass<M, FULL, false>(k, v, sk, sv, beta, alpha, gamma, T, H, D, NT, CPS, Ain, dst, kap, nuv, At, gt, bh, g);
}

// Both maps of a (b*h, segment) pair in one block (D = DP): P (from 0, with nu) and
// Phi (from I, nu = 0) share every chunk's staged kappa, nu and A tiles, so a chunk's
// operands are loaded and published once for the two states, and the pairs run in
// one round of workgroups.  Each wave carries its 16-column tile of both states;
// per chunk: P's residual and update, Phi's residual, the barrier that frees nu and
// the A tiles for the next chunk's loads, then Phi's update.  1-D grid of B*H*G
// blocks; sout as chunk_maps_bf16.
template <int M>
__global__ __launch_bounds__(512, 1) void chunk_maps2_bf16(const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
                                                         const bf16_t* __restrict__ sk, const bf16_t* __restrict__ sv,
                                                         const float* __restrict__ beta, const float* __restrict__ alpha,
                                                         const float* __restrict__ gamma, int T, int H, int NT, int CPS,
                                                         int BH, int G, const uint16_t* __restrict__ Ain,
                                                         float* __restrict__ sout) {
  constexpr bool SP = M == 2 * L;
  constexpr int NB = M / 16;
  constexpr int KE = krows_elems<M>();
  __shared__ __align__(16) uint16_t kapb[2 * KE];
  __shared__ __align__(16) uint16_t nuv[KE];
  __shared__ __align__(16) uint16_t At[at_elems<M>()];
  __shared__ __align__(16) GateTab<M> gtb[2];
  const int pair = blockIdx.x;
  if (pair >= BH * G) return;   // block-uniform
  const int bh = pair % BH, g = pair / BH;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const int lr = lane & 15, lg = lane >> 4;
  const int col = 16 * w;
  const int cb = g * CPS, ce = min(NT, cb + CPS);

  f4 S0[DP / 16], S1[DP / 16];   // P (from 0) and Phi (from I)
#pragma unroll
  for (int r = 0; r < DP / 16; ++r)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      S0[r][e] = 0.f;
      S1[r][e] = (16 * r + 4 * lg + e == col + lr) ? 1.f : 0.f;
    }

  const DmaCtx x{T, H, NT, b, h, bh, lane, w};
  if (cb < ce) {
    dma_pair<M, 8>(x, k, sk, cb, kapb);
    dma_pair<M, 8>(x, v, sv, cb, nuv);
    dma_A<M, 8>(x, Ain, cb, At);
    if (w == 0) store_gates<M>(load_gates<SP>(beta, alpha, gamma, T, H, b, h, cb * L, lane), lane, gtb[0]);
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's loads have landed in LDS
  }
  __syncthreads();
  for (int c = cb; c < ce; ++c) {
    const int cur = (c - cb) & 1;
    const uint16_t* kap = kapb + cur * KE;
    const GateTab<M>& gt = gtb[cur];
    const bool more = c + 1 < ce;   // block-uniform
    GateIn gn{1.f, 0.f, 0.f};
    if (more) {
      dma_pair<M, 8>(x, k, sk, c + 1, kapb + (cur ^ 1) * KE);
      if (w == 0) gn = load_gates<SP>(beta, alpha, gamma, T, H, b, h, (c + 1) * L, lane);
    }
    f4 R[NB];
    Op Rop[NB / 2];
    {
      Op Sop[DP / 32];
      pack_ops<DP / 16>(S0, Sop);
      tile_residual<M, true>(Sop, kap, nuv, At, gt.el, col, lr, lg, R);
    }
    scaled_ops<M>(R, gt.fac, lg, Rop);
    tile_update<M>(S0, Rop, kap, gt.el[L - 1], lr, lg);
    {
      Op Sop[DP / 32];
      pack_ops<DP / 16>(S1, Sop);
      tile_residual<M, false>(Sop, kap, nuv, At, gt.el, col, lr, lg, R);
    }
    __syncthreads();   // every wave is done with nu and the A tiles
    if (more) {
      dma_pair<M, 8>(x, v, sv, c + 1, nuv);
      dma_A<M, 8>(x, Ain, c + 1, At);
    }
    scaled_ops<M>(R, gt.fac, lg, Rop);
    tile_update<M>(S1, Rop, kap, gt.el[L - 1], lr, lg);
    if (more && w == 0) store_gates<M>(gn, lane, gtb[cur ^ 1]);
    __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();   // the next chunk's operands are in place; this chunk's are free
  }
  float* d0 = sout + (long)(bh * G + g) * DP * DP;
  float* d1 = sout + (long)((BH + bh) * G + g) * DP * DP;
#pragma unroll
  for (int r = 0; r < DP / 16; ++r)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      d0[(long)(16 * r + 4 * lg + e) * DP + col + lr] = S0[r][e];
      d1[(long)(16 * r + 4 * lg + e) * DP + col + lr] = S1[r][e];
    }
}

// The segment start states: sinit[bh*G + g] for g < G, from h0 ([B*H][D][D] or
// NULL) and the maps of chunk_maps_bf16 (maps[0]: P, maps[1]: Phi), as
// S(g+1) = Phi_g S(g) + P_g in fp32 (Phi and S enter the MFMAs as hi + lo bf16).
// Grid (B*H, DP/16): block y owns the 16 state columns 16y.., wave w the row tiles 2w,
// 2w+1 of them; the column tile passes between the waves through LDS as B operands,
// and each wave loads the next step's Phi rows and P tile while the current step runs.
__global__ __launch_bounds__(256) void chunk_seg_scan_bf16(int G, int D, const float* __restrict__ h0,
                                                         const float* __restrict__ maps, float* __restrict__ sinit) {
  __shared__ __align__(16) uint4 sop[DP / 32][64][2];   // the column tile as the operand of each k step
  const int bh = blockIdx.x, BH = gridDim.x;
  const int col = 16 * blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const float* P = maps;
  const float* Phi = maps + (long)BH * G * DP * DP;
  f4 S[2];   // row tiles 2w, 2w+1: S[16(2w+u) + 4lg + e][col + lr]
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 16 * (2 * w + u) + 4 * lg + e, cc = col + lr;
      S[u][e] = (h0 != nullptr && row < D && cc < D) ? h0[((long)bh * D + row) * D + cc] : 0.f;
    }
  // Phi rows of the wave's row tiles in the accumulator k order (step s: columns
  // 32s + 4lg .. +3 and 32s + 16 + 4lg .. +3), and the P tile
  float4 fa[2][DP / 32][2];
  f4 pa[2];
  auto load = [&](int g) __attribute__((always_inline)) {
    const float* Fg = Phi + (long)(bh * G + g) * DP * DP;
    const float* Pg = P + (long)(bh * G + g) * DP * DP;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float* fr = Fg + (long)(16 * (2 * w + u) + lr) * DP;
#pragma unroll
      for (int s = 0; s < DP / 32; ++s) {
        fa[u][s][0] = *reinterpret_cast<const float4*>(fr + 32 * s + 4 * lg);
        fa[u][s][1] = *reinterpret_cast<const float4*>(fr + 32 * s + 16 + 4 * lg);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) pa[u][e] = Pg[(long)(16 * (2 * w + u) + 4 * lg + e) * DP + col + lr];
    }
  };
  if (G > 1) load(0);
  for (int g = 0; g < G; ++g) {
    float* dst = sinit + (long)(bh * G + g) * DP * DP;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[(long)(16 * (2 * w + u) + 4 * lg + e) * DP + col + lr] = S[u][e];
    if (g + 1 == G) break;
    // this wave's row tiles 2w, 2w+1 are the halves of k step w
    {
      uint2 ha, la, hb, lb;
      split4(S[0], ha, la);
      split4(S[1], hb, lb);
      sop[w][lane][0] = make_uint4(ha.x, ha.y, hb.x, hb.y);
      sop[w][lane][1] = make_uint4(la.x, la.y, lb.x, lb.y);
    }
    __syncthreads();
    uint4 ah[2][DP / 32], al[2][DP / 32];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int s2 = 0; s2 < DP / 32; ++s2) {
        uint2 h0_, l0_, h1_, l1_;
        const float4 x0 = fa[u][s2][0], x1 = fa[u][s2][1];
        split4((f4){x0.x, x0.y, x0.z, x0.w}, h0_, l0_);
        split4((f4){x1.x, x1.y, x1.z, x1.w}, h1_, l1_);
        ah[u][s2] = make_uint4(h0_.x, h0_.y, h1_.x, h1_.y);
        al[u][s2] = make_uint4(l0_.x, l0_.y, l1_.x, l1_.y);
      }
    const f4 p0 = pa[0], p1 = pa[1];
    if (g + 2 < G) load(g + 1);
    f4 acc[2] = {p0, p1};
#pragma unroll
    for (int s2 = 0; s2 < DP / 32; ++s2) {
      const uint4 bh_ = sop[s2][lane][0], bl_ = sop[s2][lane][1];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        acc[u] = mma_bf16(as_bf8(ah[u][s2]), as_bf8(bh_), acc[u]);
        acc[u] = mma_bf16(as_bf8(ah[u][s2]), as_bf8(bl_), acc[u]);
        acc[u] = mma_bf16(as_bf8(al[u][s2]), as_bf8(bh_), acc[u]);
      }
    }
    S[0] = acc[0];
    S[1] = acc[1];
    __syncthreads();   // sop is rewritten next step
  }
}

// Segment g reruns its chunks from its start state (sinit[bh*G + g], leading dimension
// sld; rows / columns >= sld read as 0) and writes the output rows; the last segment
// writes the final state to ht ([B*H][D][D], rows / columns < D).  Eight waves, one
// 16-column tile of the state (and of the output) each.  With D = DP the next chunk's
// operands load while the current one computes: its kappa rows (a second buffer) and
// gates from the start, its nu rows once every wave has formed R, its q rows once the P
// operands are built and its A tiles once the output rows are done.
template <int M, bool FULL>
__global__ __launch_bounds__(512, 1) void chunk_replay_bf16(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const bf16_t* __restrict__ sk, const bf16_t* __restrict__ sv, const float* __restrict__ beta,
    const float* __restrict__ alpha, const float* __restrict__ gamma, int T, int H, int D, int NT, int CPS,
    const uint16_t* __restrict__ Ain, const float* __restrict__ sinit, int sld, float* __restrict__ ht,
    bf16_t* __restrict__ out) {
  constexpr bool SP = M == 2 * L;
  constexpr int NB = M / 16;
  constexpr int KE = krows_elems<M>();
  __shared__ __align__(16) uint16_t kapb[(FULL ? 2 : 1) * KE];
  __shared__ __align__(16) uint16_t nuv[KE];
  __shared__ __align__(16) uint16_t qr[L * PK];
  constexpr int NCBX = SP ? 10 : 6;   // the P operand blocks that later pass through At
  __shared__ __align__(16) uint16_t At[(at_elems<M>() > NCBX * 1024) ? at_elems<M>() : NCBX * 1024];
  __shared__ __align__(16) GateTab<M> gtb[FULL ? 2 : 1];

  const int bh = blockIdx.x, g = blockIdx.y, G = gridDim.y;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const int lr = lane & 15, lg = lane >> 4;
  const int col = 16 * w;
  const int cb = g * CPS, ce = min(NT, cb + CPS);
  const DmaCtx x{T, H, NT, b, h, bh, lane, w};

  f4 S[DP / 16];
  {
    const float* s0 = sinit != nullptr ? sinit + (long)(bh * G + g) * sld * sld : nullptr;
#pragma unroll
    for (int r = 0; r < DP / 16; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * r + 4 * lg + e, cc = col + lr;
        S[r][e] = (s0 != nullptr && row < sld && cc < sld) ? s0[(long)row * sld + cc] : 0.f;
      }
  }

  if constexpr (FULL) {
    if (cb < ce) {
      dma_pair<M, 8>(x, k, sk, cb, kapb);
      dma_pair<M, 8>(x, v, sv, cb, nuv);
      dma_rows<8>(x, q, cb, qr);
      dma_A<M, 8>(x, Ain, cb, At);
      if (w == 0) store_gates<M>(load_gates<SP>(beta, alpha, gamma, T, H, b, h, cb * L, lane), lane, gtb[0]);
      __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's loads have landed in LDS
    }
    __syncthreads();
  }
  for (int c = cb; c < ce; ++c) {
    const int cur = FULL ? (c - cb) & 1 : 0;
    const uint16_t* kap = kapb + cur * KE;
    const GateTab<M>& gt = gtb[cur];
    const bool more = FULL && c + 1 < ce;   // block-uniform
    GateIn gn{1.f, 0.f, 0.f};
    if constexpr (FULL) {
      if (more) {
        dma_pair<M, 8>(x, k, sk, c + 1, kapb + (cur ^ 1) * KE);
        if (w == 0) gn = load_gates<SP>(beta, alpha, gamma, T, H, b, h, (c + 1) * L, lane);
      }
    } else {
      __syncthreads();   // every wave is done with the previous chunk's operands
      stage_chunk<M, 512, true, true, FULL>(q, k, v, sk, sv, beta, alpha, gamma, Ain, T, H, D, NT, b, h, bh, c, tid,
                                            kapb, nuv, qr, At, gtb[0]);
      __syncthreads();
    }
    Op Sop[DP / 32];
    pack_ops<DP / 16>(S, Sop);
    // q S for the chunk's 64 rows (rows 16 tt + 4 lg + e of the accumulator)
    f4 qs[L / 16];
#pragma unroll
    for (int tt = 0; tt < L / 16; ++tt) {
      qs[tt] = f4_zero();
      const uint16_t* qrow = qr + (16 * tt + lr) * PK;
#pragma unroll
      for (int s = 0; s < DP / 32; ++s) {
        const bf16x8 a = rowop_p(qrow, s, lg);
        qs[tt] = mma_bf16(a, as_bf8(Sop[s].h), qs[tt]);
        qs[tt] = mma_bf16(a, as_bf8(Sop[s].l), qs[tt]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    f4 R[NB];
    tile_residual<M, true>(Sop, kap, nuv, At, gt.el, col, lr, lg, R);
    Op Rop[NB / 2];
    pack_ops<NB>(R, Rop);

    // o = e^{l_t} q S + P R, P_ti = 1[tau_i <= t] lam_i e^{l_t - l_tau_i} (q_t . kappa_i).
    // The P operands depend only on the chunk: the waves share them out -- the operand of
    // (row tile tt, sample step s) is built from P^T tiles 2s, 2s+1 (kappa q^T, whose
    // accumulator layout is P's A operand layout) -- and pass them through the A tile
    // area, free once every wave has formed R.
    constexpr int NCB = SP ? 10 : 6;   // (tt, s) pairs: s < tt + 1 (SP) or s < tt / 2 + 1
    static_assert(NCB == NCBX, "the P operand area must fit At");
    uint4* pst = reinterpret_cast<uint4*>(At);   // [NCB][64 lanes][hi, lo]
    __syncthreads();   // every wave is done with the A tiles and nu
    if (more) dma_pair<M, 8>(x, v, sv, c + 1, nuv);
    for (int cb2 = w; cb2 < NCB; cb2 += 8) {
      int tt = 0, s0 = cb2;
      while (s0 >= (SP ? tt + 1 : tt / 2 + 1)) { s0 -= (SP ? tt + 1 : tt / 2 + 1); ++tt; }
      const int t = 16 * tt + lr;                // P^T column of this lane
      const uint16_t* qrow = qr + (16 * tt + lr) * PK;
      f4 p[2];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int J = 2 * s0 + hf;
        p[hf] = f4_zero();
#pragma unroll
        for (int s2 = 0; s2 < DP / 32; ++s2)
          p[hf] = mma_bf16(rowop(kap + krow<SP>(16 * J + lr), s2, lg), rowop(qrow, s2, lg), p[hf]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = 16 * J + 4 * lg + e, tj = samp_t<SP>(j);
          p[hf][e] = (tj <= t) ? gt.lam[j] * fexp(gt.logd[t] - gt.logd[tj]) * p[hf][e] : 0.f;
        }
      }
      Op Pop[1];
      pack_ops<2>(p, Pop);
      pst[(cb2 * 64 + lane) * 2] = Pop[0].h;
      pst[(cb2 * 64 + lane) * 2 + 1] = Pop[0].l;
    }
    __syncthreads();   // the P operands are in place; q is free
    if (more) dma_rows<8>(x, q, c + 1, qr);
    const int t0 = c * L;
    const bool whole = t0 + L <= T;   // block-uniform: every output row of the chunk exists
    bf16_t* orow = out + ((long)(b * T + t0) * H + h) * D + col + lr;
    const long ostep = (long)H * D;   // between consecutive tokens
#pragma unroll
    for (int tt = 0; tt < L / 16; ++tt) {
      const int ns = SP ? tt + 1 : tt / 2 + 1;
      const int cbase = SP ? tt * (tt + 1) / 2 : (tt < 2 ? tt : 2 + 2 * (tt - 2));
      f4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = gt.el[16 * tt + 4 * lg + e] * qs[tt][e];
#pragma unroll
      for (int s = 0; s < NB / 2; ++s) {
        if (s < ns) {
          const uint4 ph = pst[((cbase + s) * 64 + lane) * 2], pl = pst[((cbase + s) * 64 + lane) * 2 + 1];
          o = mma_bf16(as_bf8(ph), as_bf8(Rop[s].h), o);
          o = mma_bf16(as_bf8(ph), as_bf8(Rop[s].l), o);
          o = mma_bf16(as_bf8(pl), as_bf8(Rop[s].h), o);
        }
      }
      if (FULL && whole) {
#pragma unroll
        for (int e = 0; e < 4; ++e) orow[(16 * tt + 4 * lg + e) * ostep].bits = f32_to_bf16(o[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int tl = 16 * tt + 4 * lg + e;
          if (t0 + tl < T && col + lr < D) orow[tl * ostep].bits = f32_to_bf16(o[e]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (more) {
      __syncthreads();   // every wave is done with the P operands: the A area is free
      dma_A<M, 8>(x, Ain, c + 1, At);
    }

    // R' from the residual operands (R = hi + lo to about 16 bits)
#pragma unroll
    for (int sp = 0; sp < NB / 2; ++sp) {
      const float4 f0 = *reinterpret_cast<const float4*>(gt.fac + 32 * sp + 4 * lg);
      const float4 f1 = *reinterpret_cast<const float4*>(gt.fac + 32 * sp + 16 + 4 * lg);
      f4 y[2] = {unsplit4(make_uint2(Rop[sp].h.x, Rop[sp].h.y), make_uint2(Rop[sp].l.x, Rop[sp].l.y)),
                 unsplit4(make_uint2(Rop[sp].h.z, Rop[sp].h.w), make_uint2(Rop[sp].l.z, Rop[sp].l.w))};
      y[0][0] *= f0.x; y[0][1] *= f0.y; y[0][2] *= f0.z; y[0][3] *= f0.w;
      y[1][0] *= f1.x; y[1][1] *= f1.y; y[1][2] *= f1.z; y[1][3] *= f1.w;
      Op o1[1];
      pack_ops<2>(y, o1);
      Rop[sp] = o1[0];
    }
    tile_update<M>(S, Rop, kap, gt.el[L - 1], lr, lg);
    if constexpr (FULL) {
      if (more && w == 0) store_gates<M>(gn, lane, gtb[cur ^ 1]);
      __builtin_amdgcn_s_waitcnt(0x0f70);
      __syncthreads();   // the next chunk's operands are in place; this chunk's are free
    }
  }

  if (ht != nullptr && g == G - 1) {
#pragma unroll
    for (int r = 0; r < DP / 16; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * r + 4 * lg + e, cc = col + lr;
        if (row < D && cc < D) ht[((long)bh * D + row) * D + cc] = S[r][e];
      }
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

size_t chunk_bf16_workspace_bytes(int B, int T, int H, int has_sparse) {
  const size_t NT = (T + L - 1) / L;
  const size_t NB = has_sparse ? 2 * L / 16 : L / 16;
  const size_t ntl = NB * (NB + 1) / 2;
  const size_t n = (size_t)B * H * NT;
  size_t total = n * ntl * 512;    // A tiles, bf16
  const size_t G = seg_count(B * H, (int)NT);
  if (G > 1) total += 3 * (size_t)B * H * G * DP * DP * 4;   // segment maps P, Phi and start states
  return total + 256 * 4;
}

template <int M, bool FULL>
static hipError_t launch_intra_bwd_t(const ChunkArgs& a, float* W, float* U, float* lgd, float* A, hipStream_t st) {
  const int NT = (a.T + L - 1) / L;
  const K3Bwd bw{A, W, U, lgd, (const bf16_t*)a.v, (const bf16_t*)a.sparse_v};
  chunk_inv_bf16<M, FULL, true><<<dim3(NT, a.B * a.H), 64 * K3W, 0, st>>>(
      (const bf16_t*)a.k, (const bf16_t*)a.sparse_k, a.beta, a.alpha, a.gamma, a.T, a.H, a.D, NT, nullptr, bw);
  return hipGetLastError();
}

// The backward's per-chunk operands for bf16 inputs (see K3Bwd).
hipError_t launch_chunk_intra_bf16(const ChunkArgs& a, float* W, float* U, float* lgd, float* A, hipStream_t st) {
  const bool sp = a.sparse_k != nullptr, full = a.D == DP;
  if (sp) return full ? launch_intra_bwd_t<2 * L, true>(a, W, U, lgd, A, st) : launch_intra_bwd_t<2 * L, false>(a, W, U, lgd, A, st);
  return full ? launch_intra_bwd_t<L, true>(a, W, U, lgd, A, st) : launch_intra_bwd_t<L, false>(a, W, U, lgd, A, st);
}

template <int M, bool FULL>
static hipError_t launch_bf16_t(const ChunkArgs& a, hipStream_t st) {
  constexpr int NB = M / 16;
  constexpr int NTL = NB * (NB + 1) / 2;
  const int NT = (a.T + L - 1) / L;
  const size_t n = (size_t)a.B * a.H * NT;
  auto align = [](char* p) { return (char*)(((uintptr_t)p + 255) & ~(uintptr_t)255); };
  char* p = align((char*)a.workspace);
  uint16_t* Aws = (uint16_t*)p;
  p = align(p + n * NTL * 512);
  const int BH = a.B * a.H;
  const int G = seg_count(BH, NT);
  const int CPS = (NT + G - 1) / G;
  float* maps = (float*)p;   // [2][BH][G][DP][DP]: P, Phi
  float* sinit = maps + 2 * (size_t)BH * G * DP * DP;
  const bf16_t* q = (const bf16_t*)a.q;
  const bf16_t* k = (const bf16_t*)a.k;
  const bf16_t* v = (const bf16_t*)a.v;
  const bf16_t* sk = (const bf16_t*)a.sparse_k;
  const bf16_t* sv = (const bf16_t*)a.sparse_v;
  chunk_inv_bf16<M, FULL><<<dim3(NT, BH), 64 * K3W, 0, st>>>(k, sk, a.beta, a.alpha, a.gamma, a.T, a.H, a.D, NT, Aws);
  if (G == 1) {
    chunk_replay_bf16<M, FULL><<<dim3(BH, 1), 512, 0, st>>>(q, k, v, sk, sv, a.beta, a.alpha, a.gamma, a.T, a.H, a.D, NT,
                                                      NT, Aws, a.initial_state, a.D, a.final_state, (bf16_t*)a.out);
  } else {
    if constexpr (FULL)
      chunk_maps2_bf16<M><<<dim3(BH * G), 512, 0, st>>>(k, v, sk, sv, a.beta, a.alpha, a.gamma, a.T, a.H, NT, CPS, BH,
                                                        G, Aws, maps);
    else
      chunk_maps_bf16<M, FULL><<<dim3(16 * ((BH * G + 7) / 8)), 512, 0, st>>>(
          k, v, sk, sv, a.beta, a.alpha, a.gamma, a.T, a.H, a.D, NT, CPS, BH, G, Aws, maps);
    chunk_seg_scan_bf16<<<dim3(BH, DP / 16), 256, 0, st>>>(G, a.D, a.initial_state, maps, sinit);
    chunk_replay_bf16<M, FULL><<<dim3(BH, G), 512, 0, st>>>(q, k, v, sk, sv, a.beta, a.alpha, a.gamma, a.T, a.H, a.D, NT,
                                                      CPS, Aws, sinit, DP, a.final_state, (bf16_t*)a.out);
  }
  return hipGetLastError();
}

hipError_t launch_chunk_bf16(const ChunkArgs& a, hipStream_t st) {
  const bool sp = a.sparse_k != nullptr;
  // direct-to-LDS staging addresses a head's rows with 32-bit byte offsets
  const long span = (long)(a.T + L) * a.H * DP * 2;
  if (a.D == DP && span < 0x7fffffffL) return sp ? launch_bf16_t<2 * L, true>(a, st) : launch_bf16_t<L, true>(a, st);
  return sp ? launch_bf16_t<2 * L, false>(a, st) : launch_bf16_t<L, false>(a, st);
}

}  // namespace sgsa
