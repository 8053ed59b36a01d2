// Shared device helpers for the SGSA gfx950 kernels: element types, bf16
// rounding, MFMA fragment wrappers and wave-level primitives.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sgsa {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

struct bf16_t {
  uint16_t bits;
};

// --- scalar conversions -------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even, the rounding torch uses for float -> bfloat16.
// Round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

template <typename X> struct elem;
template <> struct elem<float> {
  __device__ __forceinline__ static float load(const float* p, long i) { return p[i]; }
  __device__ __forceinline__ static void store(float* p, long i, float v) { p[i] = v; }
};
template <> struct elem<bf16_t> {
  __device__ __forceinline__ static float load(const bf16_t* p, long i) { return bf16_to_f32(p[i].bits); }
  __device__ __forceinline__ static void store(bf16_t* p, long i, float v) { p[i].bits = f32_to_bf16(v); }
};

template <typename X>
__device__ __forceinline__ float ld(const X* p, long i) { return elem<X>::load(p, i); }
template <typename X>
__device__ __forceinline__ void st(X* p, long i, float v) { elem<X>::store(p, i, v); }

// Order-preserving map fp32 -> uint32 (larger float => larger key).  -0.0 is
// folded onto +0.0 first so the two compare equal, as IEEE comparison does.
__device__ __forceinline__ uint32_t f32_order_key(float f) {
  f = f + 0.0f;
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inverse of f32_order_key.
__device__ __forceinline__ float key_to_f32(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// --- MFMA fragments -------------------------------------------------------
// v_mfma_f32_16x16x4_f32 (one block): lane l supplies A[l%16][l/16] and
// B[l/16][l%16]; the accumulator holds C[4*(l/16)+i][l%16] in element i.
__device__ __forceinline__ f4 mma_f32(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// v_mfma_f32_16x16x32_bf16 (gfx950): lane l supplies A[l%16][8*(l/16)+j] and
// B[8*(l/16)+j][l%16], j=0..7; same accumulator layout as above.
__device__ __forceinline__ f4 mma_bf16(bf16x8 a, bf16x8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// fp32 score of an accumulated q.k product: acc * (1/scale), with -0.0 folded
// onto +0.0.  Every kernel that selects on scores or recomputes them goes
// through this one expression, so their scores agree bit for bit.
__device__ __forceinline__ f4 score_of(f4 acc, float mscale) {
#pragma clang fp contract(off)
  return acc * mscale + 0.0f;
}

// Smallest float above x (x finite or -inf; +inf stays +inf).  For scores s
// (never -0.0 or NaN): s > x  <=>  s >= next_up(x).
__device__ __forceinline__ float next_up(float x) {
  uint32_t u = __float_as_uint(x);
  if (u == 0x7f800000u) return x;
  if (u == 0x80000000u) u = 0u;
  return __uint_as_float((int32_t)u >= 0 ? u + 1u : u - 1u);
}

__device__ __forceinline__ f4 f4_zero() {
  f4 z = {0.f, 0.f, 0.f, 0.f};
  return z;
}

// --- wave primitives ------------------------------------------------------

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Sum over the aligned group of `w` lanes containing this lane (w a power of 2, <= 64).
__device__ __forceinline__ float group_sum(float v, int w) {
  for (int o = w >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ int popc64(uint64_t x) { return __popcll(x); }

// Wave ballot straight from the predicate's lane mask (no int round trip).
__device__ __forceinline__ uint64_t ballot64(bool p) { return __builtin_amdgcn_ballot_w64(p); }
// Inclusive prefix sum over the 64 lanes: row_shr 1/2/4/8 within each row of 16
// lanes (lanes past the row edge read 0), then row_bcast 15 adds the last lane
// of rows 0 and 2 to rows 1 and 3 and row_bcast 31 adds lane 31 to rows 2 and 3.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
  int v = (int)x;
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);
  return (uint32_t)v;
}
// Number of set bits of m below this lane.
__device__ __forceinline__ uint32_t lane_rank(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

}  // namespace sgsa
