// Block retrieval modes of the retriever on its torch path
// (modelings/modeling_sgsa.py:167-195 block selection, :302-359 candidates,
// :444-463 dispatch).  Three kernels, then the row gather of gather.hip:
//
//   block_max_kernel     block scores: per query row and key block of
//   (or _mfma_kernel)    block_size keys, the max causal score (-FLT_MAX when
//                        the block has no causal key), fp32, block-major;
//   block_select_kernel  per row, the top `top_blocks` blocks (score desc,
//                        lowest index on ties) and the row's candidate count;
//   block_cand_kernel    per row, the causal keys of the kept blocks with
//                        their scores: block_token sorts them in LDS and emits
//                        the masked top-k slots; block_only emits them all.
//
// With a padding mask (mask [B,T], the same for keys and queries, :421-428)
// a row sees the valid keys <= its position, a padded query row sees none;
// block_mask_prep_kernel lays out per batch the valid keys' prefix counts and
// order, the mask as bits and each row's count of blocks holding a key it sees,
// from which the rows' k_q (:159-160) follows.
//
// Scores here are acc * (1/sqrt(D)).  bf16 inputs with D % 32 == 0: acc from
// v_mfma_f32_16x16x32_bf16 over d in steps of 32 (the MFMA sweep and scorer);
// fp32 inputs with D % 16 == 0: acc from v_mfma_f32_16x16x4_f32 in the steps of
// block_max_f32mfma_kernel; otherwise acc is an fp32 fma chain over d = 0..D-1
// in ascending order.  The
// block sweep and the candidate scorer of one call use the same form, so a
// candidate's score is bit-identical to the value its block max was taken on.
#include <float.h>

#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace sgsa {

__device__ __forceinline__ float block_score(float acc, float mscale) {
#pragma clang fp contract(off)
  return acc * mscale + 0.0f;
}

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---- padding masks ----------------------------------------------------------
// One 1024-thread workgroup per batch b, over the positions in tiles of 1024:
// pass 1 writes pc[t] = valid keys before t (pc[T] = all of them), perm[pc[t]]
// = t for valid t and the mask bits; pass 2 flags each block's first valid key
// (a valid t with no valid key in [block start, t)), and the inclusive prefix
// of the flags is the number of blocks holding a valid key <= t.  nvb[t] is
// that count (the count over all keys when not causal) for a valid query row,
// 0 for a padded one.
__global__ __launch_bounds__(1024) void block_mask_prep_kernel(BlockArgs a) {
  __shared__ int wsum[16];
  const int b = blockIdx.x, T = a.T, bs = a.bs;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint8_t* m = a.mask + (long)b * T;
  int32_t* pc = a.mpc + (long)b * (T + 1);
  int32_t* perm = a.mperm + (long)b * T;
  int32_t* nvb = a.mnvb + (long)b * T;
  uint32_t* bits = a.mbits + (long)b * a.nmw;
  // prefix of a per-position flag over the workgroup: (exclusive count, total)
  auto scan = [&](bool f, int carry, int& before) {
    const uint64_t bal = ballot64(f);
    if (lane == 0) wsum[w] = popc64(bal);
    __syncthreads();
    int lo = carry, tot = carry;
    for (int i = 0; i < 16; ++i) {
      lo += i < w ? wsum[i] : 0;
      tot += wsum[i];
    }
    before = lo + (int)lane_rank(bal);
    __syncthreads();
    return tot;
  };
  int carry = 0;
  for (int t0 = 0; t0 < T; t0 += 1024) {
    const int t = t0 + tid;
    const bool v = t < T && m[t] != 0;
    const uint64_t bal = ballot64(v);
    if (t < T && (lane & 31) == 0) bits[t >> 5] = (uint32_t)(bal >> (lane & 32));
    int before;
    carry = scan(v, carry, before);
    if (t < T) {
      pc[t] = before;
      if (v) perm[before] = t;
    }
  }
  if (tid == 0) pc[T] = carry;
  __syncthreads();
  carry = 0;
  for (int t0 = 0; t0 < T; t0 += 1024) {
    const int t = t0 + tid;
    const bool v = t < T && m[t] != 0;
    const bool first = v && pc[t] == pc[(t / bs) * bs];
    int before;
    carry = scan(first, carry, before);
    if (t < T) nvb[t] = v ? before + (first ? 1 : 0) : 0;
  }
  if (!a.causal) {
    __syncthreads();
    for (int t = tid; t < T; t += 1024) nvb[t] = m[t] != 0 ? carry : 0;
  }
}

// kqb[t] = min(eb, max(1, max over b of nvb[b][t])), the masked top-k's k_q
// over the block scores of position t (:159-160).
__global__ __launch_bounds__(256) void block_mask_kq_kernel(BlockArgs a) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= a.T) return;
  int mx = 1;
  for (int b = 0; b < a.B; ++b) mx = max(mx, a.mnvb[(long)b * a.T + t]);
  a.mkqb[t] = min(a.eb, mx);
}

__device__ __forceinline__ bool mask_bit(const uint32_t* bits, int j) { return (bits[j >> 5] >> (j & 31)) & 1u; }

// ---- block maxima ----------------------------------------------------------
// Block scores are held block-major, [B,H,nb,T] (entry (b,h,j,t) at
// ((b*H+h)*nb + j)*T + t), so the 16 or 64 query rows of a store are
// consecutive; the caller's [B,H,T,nb] copy is a transpose, made only on request.
//
// fp32 / generic sweep: one workgroup per (64 query rows, b, h).  The q tile
// stays in LDS as fp32; keys come in tiles of 64 keys x 32 dims.  Thread
// (ty, tx) owns rows ty+16i and keys tx+16j (i, j < 4).  After a key tile, its
// 64x64 scores go to LDS and each (row, block) pair the tile touches is folded
// into the block score with a max.  The workgroup owns its rows, and the
// barrier between key tiles orders the read-modify-writes of a block that
// spans two tiles.
constexpr int BM_DC = 32;   // dims per key chunk

template <typename X>
__global__ __launch_bounds__(256) void block_max_kernel(BlockArgs a, float mscale) {
  __shared__ float qs[64 * (BLK_MAX_D + 1)];
  __shared__ float ks[64 * (BM_DC + 1)];
  __shared__ float ss[64 * 65];
  const int D = a.D, DP = D + 1, T = a.T, H = a.H, bs = a.bs, nb = a.nb;
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  const int r0 = blockIdx.x * 64;
  const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
  const X* Q = reinterpret_cast<const X*>(a.q);
  const X* K = reinterpret_cast<const X*>(a.k);
  const uint32_t* mb = a.mask ? a.mbits + (long)b * a.nmw : nullptr;

  for (int e = tid; e < 64 * D; e += 256) {
    const int r = e / D, d = e % D, t = r0 + r;
    qs[r * DP + d] = t < T ? ld(Q, ((long)(b * T + t) * H + h) * D + d) : 0.f;
  }
  float* bsc = a.block_scores + (long)bh * nb * T;
  for (long e = tid; e < 64L * nb; e += 256) {
    const int t = r0 + (int)(e % 64);
    if (t < T) bsc[(e / 64) * T + t] = -FLT_MAX;
  }

  const int kend = a.causal ? min(T, r0 + 64) : T;
  for (int k0 = 0; k0 < kend; k0 += 64) {
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
    for (int d0 = 0; d0 < D; d0 += BM_DC) {
      const int dc = min(BM_DC, D - d0);
      __syncthreads();
      for (int e = tid; e < 64 * dc; e += 256) {
        const int r = e / dc, d = e % dc, key = k0 + r;
        ks[r * (BM_DC + 1) + d] = key < T ? ld(K, ((long)(b * T + key) * H + h) * D + d0 + d) : 0.f;
      }
      __syncthreads();
      for (int d = 0; d < dc; ++d) {
        float qa[4], kb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) qa[i] = qs[(ty + 16 * i) * DP + d0 + d];
#pragma unroll
        for (int j = 0; j < 4; ++j) kb[j] = ks[(tx + 16 * j) * (BM_DC + 1) + d];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(qa[i], kb[j], acc[i][j]);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = ty + 16 * i, c = tx + 16 * j, t = r0 + r, key = k0 + c;
        bool ok = t < T && key < T && (!a.causal || key <= t);
        if (ok && a.mask) ok = mask_bit(mb, t) && mask_bit(mb, key);
        ss[r * 65 + c] = ok ? block_score(acc[i][j], mscale) : -FLT_MAX;
      }
    __syncthreads();
    const int kt_end = min(k0 + 64, T);
    const int bA = k0 / bs, nbt = (kt_end - 1) / bs - bA + 1;
    for (int it = tid; it < 64 * nbt; it += 256) {
      const int r = it % 64, bb = bA + it / 64, t = r0 + r;
      if (t >= T) continue;
      const int lo = max(bb * bs, k0), hi = min(bb * bs + bs, kt_end);
      float m = -FLT_MAX;
      for (int key = lo; key < hi; ++key) m = fmaxf(m, ss[r * 65 + key - k0]);
      float* p = bsc + (long)bb * T + t;
      *p = fmaxf(*p, m);
    }
  }
}

// bf16 form of the sweep on MFMA (v_mfma_f32_16x16x32_bf16), for D % 32 == 0.
// A workgroup takes 128 query rows (wave w owns rows r0+32w..+31 as two
// 16-row B operands, fragments in registers) and sweeps 64-key tiles; the
// longest causal sweeps are issued first.  A key tile sits in LDS (row pitch
// D+8 bf16, so the 16 keys of a fragment read fall in distinct banks) as four
// 16-key A operands, and the next tile is loaded into registers while the
// current one is multiplied.  Lane (lg, lc) ends with the scores of keys 4lg+i
// of each 16-key column block for query lc of each row set.
// REG (block_size % 16 == 0): every column block lies in one key block, so a
// block's max for a query is an in-lane max over i and the column blocks, then
// two swaps over lg; lanes lg == 0 store the queries' values (a plain store
// when the block starts in this tile, else a max with what the same lane
// stored for the previous tile).  Otherwise the scores go through LDS and each
// (row, block) pair the tile touches is reduced key by key.  Blocks with no key
// below the tile's causal end are only written when fill_invalid is set: the
// select kernel never reads them.
constexpr int BMM_KP = BLK_MAX_D + 8;
constexpr int BMM_ROWS = 128;

// fp32 form of the MFMA sweep (v_mfma_f32_16x16x4_f32), D % 16 == 0: the bf16 kernel's
// tiles, rows, operand roles and reductions with one fp32 element per lane and k-step.
// Step s = 4j + e of a 16x16 tile multiplies dimension 16j + 4lg + e in lane group lg, so
// a lane's four consecutive steps read four consecutive floats of its key row (one 16-byte
// LDS read) and of its query row (registers).  block_cand_kernel's fp32 scorer runs the
// same steps in the same order, so a candidate's score is bit for bit the value its
// block max was taken on.
constexpr int BMF_KP = BLK_MAX_D + 4;   // key tile row pitch, floats

template <bool REG>
__global__ __launch_bounds__(256) void block_max_f32mfma_kernel(BlockArgs a, float mscale) {
  __shared__ __attribute__((aligned(16))) float kt[64 * BMF_KP];
  __shared__ float ss[REG ? 1 : 128 * 65];
  constexpr int ROWS = 128;
  const int D = a.D, T = a.T, H = a.H, bs = a.bs, nb = a.nb, nj = D / 16;
  const int nrb = (T + ROWS - 1) / ROWS;
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  const int r0 = (nrb - 1 - (int)blockIdx.x) * ROWS;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, lg = l >> 4, lc = l & 15;
  const float* Q = reinterpret_cast<const float*>(a.q);
  const float* K = reinterpret_cast<const float*>(a.k) + ((long)b * T * H + h) * D;
  const long kstride = (long)H * D;

  float4 qf[2][BLK_MAX_D / 16];
  int qrow[2];
#pragma unroll
  for (int rs = 0; rs < 2; ++rs) {
    qrow[rs] = r0 + 32 * w + 16 * rs + lc;
#pragma unroll
    for (int j = 0; j < BLK_MAX_D / 16; ++j) {
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (j < nj && qrow[rs] < T)
        v = *reinterpret_cast<const float4*>(Q + ((long)(b * T + qrow[rs]) * H + h) * D + 16 * j + 4 * lg);
      qf[rs][j] = v;
    }
  }
  float* bsc = a.block_scores + (long)bh * nb * T;
  const int kend = a.causal ? min(T, r0 + ROWS) : T;
  if (a.fill_invalid) {
    const int fb = (kend + bs - 1) / bs, nfill = nb - fb;
    for (long e = tid; e < (long)ROWS * nfill; e += 256) {
      const int t = r0 + (int)(e % ROWS);
      if (t < T) bsc[(fb + e / ROWS) * T + t] = -FLT_MAX;
    }
  }
  const uint32_t* mb = a.mask ? a.mbits + (long)b * a.nmw : nullptr;
  bool qok[2];
#pragma unroll
  for (int rs = 0; rs < 2; ++rs) qok[rs] = !mb || (qrow[rs] < T && mask_bit(mb, qrow[rs]));

  const int cpr = D / 4;       // 16-byte chunks per key row
  const int nch = 64 * cpr;    // chunks per tile, <= 2048
  float4 pf[8];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = tid + 256 * u, r = e / cpr, c = e % cpr, key = k0 + r;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (e < nch && key < T) v = *reinterpret_cast<const float4*>(K + key * kstride + 4 * c);
      pf[u] = v;
    }
  };
  fetch(0);
  for (int k0 = 0; k0 < kend; k0 += 64) {
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = tid + 256 * u;
      if (e < nch) *reinterpret_cast<float4*>(kt + (e / cpr) * BMF_KP + 4 * (e % cpr)) = pf[u];
    }
    __syncthreads();
    if (k0 + 64 < kend) fetch(k0 + 64);
    const int kt_end = min(k0 + 64, T);
    uint64_t kbits = ~0ull;
    if (mb) {
      const int w0 = k0 >> 5;
      kbits = (uint64_t)mb[w0] | (w0 + 1 < a.nmw ? (uint64_t)mb[w0 + 1] << 32 : 0ull);
    }
    float sc[2][4][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f4 acc[2] = {f4_zero(), f4_zero()};
#pragma unroll
      for (int j = 0; j < BLK_MAX_D / 16; ++j) {
        if (j < nj) {
          const float4 kv = *reinterpret_cast<const float4*>(kt + (16 * kb + lc) * BMF_KP + 16 * j + 4 * lg);
#pragma unroll
          for (int rs = 0; rs < 2; ++rs) {
            acc[rs] = mma_f32(kv.x, qf[rs][j].x, acc[rs]);
            acc[rs] = mma_f32(kv.y, qf[rs][j].y, acc[rs]);
            acc[rs] = mma_f32(kv.z, qf[rs][j].z, acc[rs]);
            acc[rs] = mma_f32(kv.w, qf[rs][j].w, acc[rs]);
          }
        }
      }
#pragma unroll
      for (int rs = 0; rs < 2; ++rs) {
        const f4 v = score_of(acc[rs], mscale);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = k0 + 16 * kb + 4 * lg + i;
          const bool ok = qrow[rs] < T && key < T && (!a.causal || key <= qrow[rs]) && qok[rs] &&
                          ((kbits >> (key - k0)) & 1ull);
          sc[rs][kb][i] = ok ? v[i] : -FLT_MAX;
        }
      }
    }
    if (REG) {
#pragma unroll
      for (int rs = 0; rs < 2; ++rs) {
        float run = -FLT_MAX;
        int cur = k0 / bs;
        auto flush = [&](int bb) {
          float m = fmaxf(run, __shfl_xor(run, 16, 64));
          m = fmaxf(m, __shfl_xor(m, 32, 64));
          if (lg == 0 && qrow[rs] < T) {
            float* p = bsc + (long)bb * T + qrow[rs];
            *p = bb * bs >= k0 ? m : fmaxf(*p, m);
          }
        };
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          const int c0 = k0 + 16 * kb;
          if (c0 >= kt_end) break;
          const int bb = c0 / bs;
          if (bb != cur) {
            flush(cur);
            run = -FLT_MAX;
            cur = bb;
          }
          run = fmaxf(run, fmaxf(fmaxf(sc[rs][kb][0], sc[rs][kb][1]), fmaxf(sc[rs][kb][2], sc[rs][kb][3])));
        }
        flush(cur);
      }
    } else {
#pragma unroll
      for (int rs = 0; rs < 2; ++rs)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) ss[(32 * w + 16 * rs + lc) * 65 + 16 * kb + 4 * lg + i] = sc[rs][kb][i];
      __syncthreads();
      const int bA = k0 / bs, nbt = (kt_end - 1) / bs - bA + 1;
      for (int it = tid; it < ROWS * nbt; it += 256) {
        const int r = it % ROWS, bb = bA + it / ROWS, t = r0 + r;
        if (t >= T) continue;
        const int lo = max(bb * bs, k0), hi = min(bb * bs + bs, kt_end);
        float m = -FLT_MAX;
        for (int key = lo; key < hi; ++key) m = fmaxf(m, ss[r * 65 + key - k0]);
        float* p = bsc + (long)bb * T + t;
        *p = bb * bs >= k0 ? m : fmaxf(*p, m);
      }
    }
  }
}

template <bool REG>
__global__ __launch_bounds__(256) void block_max_mfma_kernel(BlockArgs a, float mscale) {
  __shared__ __attribute__((aligned(16))) uint16_t kt[64 * BMM_KP];
  __shared__ float ss[REG ? 1 : BMM_ROWS * 65];
  const int D = a.D, T = a.T, H = a.H, bs = a.bs, nb = a.nb, nks = D / 32;
  const int nrb = (T + BMM_ROWS - 1) / BMM_ROWS;
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  const int r0 = (nrb - 1 - (int)blockIdx.x) * BMM_ROWS;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, lg = l >> 4, lc = l & 15;
  const uint16_t* Q = reinterpret_cast<const uint16_t*>(a.q);
  const uint16_t* K = reinterpret_cast<const uint16_t*>(a.k) + ((long)b * T * H + h) * D;
  const long kstride = (long)H * D;

  bf16x8 qf[2][BLK_MAX_D / 32];
  int qrow[2];
#pragma unroll
  for (int rs = 0; rs < 2; ++rs) {
    qrow[rs] = r0 + 32 * w + 16 * rs + lc;
#pragma unroll
    for (int s = 0; s < BLK_MAX_D / 32; ++s) {
      u16x8 raw = {0, 0, 0, 0, 0, 0, 0, 0};
      if (s < nks && qrow[rs] < T)
        raw = *reinterpret_cast<const u16x8*>(Q + ((long)(b * T + qrow[rs]) * H + h) * D + 32 * s + 8 * lg);
      qf[rs][s] = __builtin_bit_cast(bf16x8, raw);
    }
  }
  float* bsc = a.block_scores + (long)bh * nb * T;
  const int kend = a.causal ? min(T, r0 + BMM_ROWS) : T;
  if (a.fill_invalid) {
    const int fb = (kend + bs - 1) / bs, nfill = nb - fb;
    for (long e = tid; e < (long)BMM_ROWS * nfill; e += 256) {
      const int t = r0 + (int)(e % BMM_ROWS);
      if (t < T) bsc[(fb + e / BMM_ROWS) * T + t] = -FLT_MAX;
    }
  }
  const uint32_t* mb = a.mask ? a.mbits + (long)b * a.nmw : nullptr;
  bool qok[2];
#pragma unroll
  for (int rs = 0; rs < 2; ++rs) qok[rs] = !mb || (qrow[rs] < T && mask_bit(mb, qrow[rs]));

  const int cpr = D / 8;       // 16-byte chunks per key row
  const int nch = 64 * cpr;    // chunks per tile, <= 1024
  u16x8 pf[4];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = tid + 256 * u, r = e / cpr, c = e % cpr, key = k0 + r;
      u16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
      if (e < nch && key < T) v = *reinterpret_cast<const u16x8*>(K + key * kstride + 8 * c);
      pf[u] = v;
    }
  };
  fetch(0);
  for (int k0 = 0; k0 < kend; k0 += 64) {
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = tid + 256 * u;
      if (e < nch) *reinterpret_cast<u16x8*>(kt + (e / cpr) * BMM_KP + 8 * (e % cpr)) = pf[u];
    }
    __syncthreads();
    if (k0 + 64 < kend) fetch(k0 + 64);
    const int kt_end = min(k0 + 64, T);
    // the tile's 64 mask bits (keys k0.., k0 a multiple of 64)
    uint64_t kbits = ~0ull;
    if (mb) {
      const int w0 = k0 >> 5;
      kbits = (uint64_t)mb[w0] | (w0 + 1 < a.nmw ? (uint64_t)mb[w0 + 1] << 32 : 0ull);
    }
    float sc[2][4][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f4 acc[2] = {f4_zero(), f4_zero()};
#pragma unroll
      for (int s = 0; s < BLK_MAX_D / 32; ++s) {
        if (s < nks) {
          const bf16x8 kf = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8*>(kt + (16 * kb + lc) * BMM_KP + 32 * s + 8 * lg));
          acc[0] = mma_bf16(kf, qf[0][s], acc[0]);
          acc[1] = mma_bf16(kf, qf[1][s], acc[1]);
        }
      }
#pragma unroll
      for (int rs = 0; rs < 2; ++rs) {
        const f4 v = score_of(acc[rs], mscale);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = k0 + 16 * kb + 4 * lg + i;
          const bool ok = qrow[rs] < T && key < T && (!a.causal || key <= qrow[rs]) && qok[rs] &&
                          ((kbits >> (key - k0)) & 1ull);
          sc[rs][kb][i] = ok ? v[i] : -FLT_MAX;
        }
      }
    }
    if (REG) {
#pragma unroll
      for (int rs = 0; rs < 2; ++rs) {
        float run = -FLT_MAX;
        int cur = k0 / bs;
        auto flush = [&](int bb) {
          float m = fmaxf(run, __shfl_xor(run, 16, 64));
          m = fmaxf(m, __shfl_xor(m, 32, 64));
          if (lg == 0 && qrow[rs] < T) {
            float* p = bsc + (long)bb * T + qrow[rs];
            *p = bb * bs >= k0 ? m : fmaxf(*p, m);
          }
        };
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          const int c0 = k0 + 16 * kb;
          if (c0 >= kt_end) break;
          const int bb = c0 / bs;
          if (bb != cur) {
            flush(cur);
            run = -FLT_MAX;
            cur = bb;
          }
          run = fmaxf(run, fmaxf(fmaxf(sc[rs][kb][0], sc[rs][kb][1]), fmaxf(sc[rs][kb][2], sc[rs][kb][3])));
        }
        flush(cur);
      }
    } else {
#pragma unroll
      for (int rs = 0; rs < 2; ++rs)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) ss[(32 * w + 16 * rs + lc) * 65 + 16 * kb + 4 * lg + i] = sc[rs][kb][i];
      __syncthreads();
      const int bA = k0 / bs, nbt = (kt_end - 1) / bs - bA + 1;
      for (int it = tid; it < BMM_ROWS * nbt; it += 256) {
        const int r = it % BMM_ROWS, bb = bA + it / BMM_ROWS, t = r0 + r;
        if (t >= T) continue;
        const int lo = max(bb * bs, k0), hi = min(bb * bs + bs, kt_end);
        float m = -FLT_MAX;
        for (int key = lo; key < hi; ++key) m = fmaxf(m, ss[r * 65 + key - k0]);
        float* p = bsc + (long)bb * T + t;
        *p = bb * bs >= k0 ? m : fmaxf(*p, m);
      }
    }
  }
}

// bf16 sweep for block_size 16 or 32 with the keys straight into registers
// (the K1 threshold kernel's sweep, without its LDS): a workgroup takes 128
// query rows, resident as eight 16-row B operands per wave, and sweeps
// 128-key tiles; wave w takes keys [32w, 32w+32) of a tile as two 16-key A
// operands, loaded into registers one tile ahead (MFMA row rho holds key
// rho/4 + 4 (rho%4), so lane (lg, lr) ends with rows 16g + lr against keys
// 32w + 16u + lg + 4i).  A wave's keys are whole blocks, so a block's max for a
// row is an in-lane max and two swaps over lg, stored by the lanes lg == 0
// (16 consecutive rows per store); blocks never span tiles, and nothing is
// shared between waves.  Same operands, k-position order and score_of() as
// block_cand_kernel's scorer, so scores agree bit for bit.
// MK: the call has a padding mask (a separate instantiation keeps the unmasked
// sweep's registers as they are).  NKS = D / 32 is a template argument: with D
// known, the k-steps' loads and MFMAs are straight-line code with no branch
// each, and the compiler interleaves them.
template <bool MK, int NKS>
__global__ __launch_bounds__(256, 2) void block_max_reg_kernel(BlockArgs a, float mscale) {
  constexpr int QR = BMM_ROWS, NG = QR / 16, TK = 128;
  const int D = NKS * 32, T = a.T, H = a.H, bs = a.bs, nb = a.nb;
  const int nrb = (T + QR - 1) / QR;
  // grid (B*H, row blocks): consecutive workgroups take different heads, so the XCDs they are dealt
  // to in turn each see a few heads' keys in their L2; the latest (heaviest) row blocks go first
  const int bh = blockIdx.x, b = bh / H, h = bh % H;
  const int r0 = (nrb - 1 - (int)blockIdx.y) * QR;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const uint16_t* Q = reinterpret_cast<const uint16_t*>(a.q);
  const uint16_t* K = reinterpret_cast<const uint16_t*>(a.k) + ((long)b * T * H + h) * D;
  const long kstride = (long)H * D;

  bf16x8 qf[NG][NKS];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const int qr = r0 + 16 * g + lr;
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      u16x8 raw = {0, 0, 0, 0, 0, 0, 0, 0};
      if (qr < T) raw = *reinterpret_cast<const u16x8*>(Q + ((long)(b * T + qr) * H + h) * D + 32 * s + 8 * lg);
      qf[g][s] = __builtin_bit_cast(bf16x8, raw);
    }
  }
  float* bsc = a.block_scores + (long)bh * nb * T;
  const int kend = a.causal ? min(T, r0 + QR) : T;
  if (a.fill_invalid) {
    const int fb = (kend + bs - 1) / bs, nfill = nb - fb;
    for (long e = tid; e < (long)QR * nfill; e += 256) {
      const int t = r0 + (int)(e % QR);
      if (t < T) bsc[(fb + e / QR) * T + t] = -FLT_MAX;
    }
  }
  const int minvalid = a.causal ? min(T, r0 + 1) : T;   // keys below it are valid for every row
  const uint32_t* mb = MK ? a.mbits + (long)b * a.nmw : nullptr;
  uint32_t qok = 0;   // bit g: row r0 + 16 g + lr is a real token
  if (MK) {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int qr = r0 + 16 * g + lr;
      if (qr < T && mask_bit(mb, qr)) qok |= 1u << g;
    }
  }
  const int ntile = (kend + TK - 1) / TK;
  const int krow = (lr >> 2) + 4 * (lr & 3);
  // key operands of one tile; without a mask two of them, the next tile's loads issued before
  // the current tile's MFMAs (the masked form has no registers to spare for it)
  bf16x8 kf[2][NKS], kn[2][NKS];
  auto kload = [&](bf16x8 (&kb)[2][NKS], int kt) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = kt * TK + 32 * w + 16 * u + krow;
      const uint16_t* p = K + (long)(j < T ? j : 0) * kstride + 8 * lg;
#pragma unroll
      for (int s = 0; s < NKS; ++s) kb[u][s] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8*>(p + 32 * s));
    }
  };
  float m[2][NG];
  // the block maxima of the wave's keys for each row; FULL: every key of the wave is valid for every row
  auto tile = [&](const bf16x8 (&kb)[2][NKS], int kw, uint32_t kbits, auto fullt) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(fullt)::value;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        f4 c = f4_zero();
#pragma unroll
        for (int s = 0; s < NKS; ++s) c = mma_bf16(kb[u][s], qf[g][s], c);
        const f4 sc = score_of(c, mscale);
        float mx = -FLT_MAX;
        if constexpr (FULL) {
          mx = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), sc[2]), sc[3]);   // the masked chain's order
        } else {
          const int qr = r0 + 16 * g + lr;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kw + 16 * u + lg + 4 * i;
            bool ok = qr < T && key < T && (!a.causal || key <= qr);
            if (MK) ok = ok && ((qok >> g) & 1u) && ((kbits >> (key - kw)) & 1u);
            mx = fmaxf(mx, ok ? sc[i] : -FLT_MAX);
          }
        }
        m[u][g] = mx;
      }
    }
  };
  auto sweep = [&](const bf16x8 (&kb)[2][NKS], int kt) __attribute__((always_inline)) {
    const int kw = kt * TK + 32 * w;   // the wave's first key
    const bool full = !MK && kw + 32 <= minvalid;
    const uint32_t kbits = MK ? (kw < T ? mb[kw >> 5] : 0u) : ~0u;   // keys kw..kw+31
    if (full) tile(kb, kw, kbits, std::true_type{});
    else tile(kb, kw, kbits, std::false_type{});
    return kw;
  };
  auto store = [&](int kw) __attribute__((always_inline)) {
    if (kw < kend) {   // wave-uniform: the wave's keys hold a block the rows may see
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        if (bs == 32 && u == 1) break;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          float v = bs == 32 ? fmaxf(m[0][g], m[1][g]) : m[u][g];
          v = fmaxf(v, __shfl_xor(v, 16, 64));
          v = fmaxf(v, __shfl_xor(v, 32, 64));
          const int t = r0 + 16 * g + lr;
          const int bb = (kw + 16 * u) / bs;
          if (lg == 0 && t < T && kw + 16 * u < kend) bsc[(long)bb * T + t] = v;
        }
      }
    }
  };
  if (ntile > 0) kload(kf, 0);
  if constexpr (!MK) {
    for (int kt = 0; kt < ntile; kt += 2) {
      if (kt + 1 < ntile) kload(kn, kt + 1);
      store(sweep(kf, kt));
      if (kt + 1 >= ntile) break;
      if (kt + 2 < ntile) kload(kf, kt + 2);
      store(sweep(kn, kt + 1));
    }
  } else {
    for (int kt = 0; kt < ntile; ++kt) {
      const int kw = sweep(kf, kt);
      if (kt + 1 < ntile) kload(kf, kt + 1);
      store(kw);
    }
  }
}

// [B,H,nb,T] -> [B,H,T,nb], for callers that ask for the block scores.
__global__ __launch_bounds__(256) void block_scores_transpose_kernel(const float* __restrict__ src, long bhn, int T,
                                                                     int nb, float* __restrict__ dst) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;   // over dst
  if (i >= bhn) return;
  const int j = (int)(i % nb);
  const long rt = i / nb;            // bh * T + t
  const long bh = rt / T;
  const int t = (int)(rt % T);
  dst[i] = src[(bh * nb + j) * T + t];
}

// ---- top blocks per row ----------------------------------------------------
// One lane per row; the lanes of a wave take consecutive query positions, so
// each block-score read is coalesced.  Blocks 0..lim/bs hold a key <= lim
// (lim = t causal, else T-1); without a mask they are the valid blocks of
// :188-189, the same count for every (b, h) of a row, so the masked top-k
// keeps kqb = min(eb, that count) of them (:159-160) and pads the rest with
// index 0 (:151-152).  With a mask the valid blocks are those holding a key
// the row sees (score > -FLT_MAX), kqb comes from block_mask_kq_kernel (at
// most the lim/bs + 1 blocks scanned), and a row with fewer valid blocks takes
// its invalid ones, -FLT_MAX, in ascending index.  A pass keeps, in
// registers, the best BS_R blocks after the last one taken, in (score desc,
// index asc) order; passes repeat until kqb are taken.
constexpr int BS_R = 4;
constexpr int BS_AHEAD = 16;   // block scores a lane loads before inserting them

__global__ __launch_bounds__(256) void block_select_kernel(BlockArgs a) {
  const long row = (long)blockIdx.x * 256 + threadIdx.x;
  const long nrows = (long)a.B * a.H * a.T;
  if (row >= nrows) return;
  const int T = a.T, t = (int)(row % T), bs = a.bs, eb = a.eb;
  const long bh = row / T;
  const int lim = a.causal ? t : T - 1;
  const int nvb = lim / bs + 1;
  const int kqb = a.mask ? a.mkqb[t] : min(eb, nvb);
  const int b = (int)(bh / a.H);
  const int32_t* pc = a.mask ? a.mpc + (long)b * (T + 1) : nullptr;
  const bool qok = !a.mask || a.mask[(long)b * T + t] != 0;
  const float* col = a.block_scores + bh * a.nb * T + t;
  int32_t* bi = a.block_indices + row * eb;
  float ls = INFINITY;
  int lj = -1, ncand = 0, first = 0, second = 0;
  for (int got = 0; got < kqb;) {
    float bv[BS_R];
    int bj[BS_R];
#pragma unroll
    for (int r = 0; r < BS_R; ++r) { bv[r] = -INFINITY; bj[r] = 0x7fffffff; }
    // block j's score into the kept list if it ranks after the last block taken
    auto insert = [&](float cv, int cj) __attribute__((always_inline)) {
      if (!(cv < ls || (cv == ls && cj > lj))) return;
#pragma unroll
      for (int r = 0; r < BS_R; ++r) {
        if (cv > bv[r] || (cv == bv[r] && cj < bj[r])) {
          const float tv = bv[r];
          const int tj = bj[r];
          bv[r] = cv; bj[r] = cj; cv = tv; cj = tj;
        }
      }
    };
    // BS_AHEAD scores loaded ahead of their insertions (one load at a time leaves the loop latency-bound)
    int j = 0;
    for (; j + BS_AHEAD <= nvb; j += BS_AHEAD) {
      float cvs[BS_AHEAD];
#pragma unroll
      for (int u = 0; u < BS_AHEAD; ++u) cvs[u] = col[(long)(j + u) * T];
#pragma unroll
      for (int u = 0; u < BS_AHEAD; ++u) insert(cvs[u], j + u);
    }
    for (; j < nvb; ++j) insert(col[(long)j * T], j);
    const int take = min(BS_R, kqb - got);
#pragma unroll
    for (int r = 0; r < BS_R; ++r) {
      if (r < take) {
        int j = bj[r];
        if (j == 0x7fffffff) j = 0;   // only NaN scores left: keep block 0 so every key stays in range
        bi[got + r] = j;
        const int hi = min(j * bs + bs, lim + 1);
        ncand += pc ? (qok ? pc[hi] - pc[j * bs] : 0) : hi - j * bs;
        if (got + r == 0) first = j;
        if (got + r == 1) second = j;
        ls = bv[r];
        lj = j;
      }
    }
    got += take;
  }
  for (int s = kqb; s < eb; ++s) bi[s] = 0;
  a.ncand[row] = ncand;
  if (a.bmargin) a.bmargin[row] = eb >= 2 ? (float)first - (float)second : 0.f;
}

// q . k over d = 0..D-1 as one fp32 fma chain (16-byte loads when VEC).
template <typename X, bool VEC> struct KeyDot;
template <bool VEC> struct KeyDot<float, VEC> {
  __device__ __forceinline__ static float run(const float* qrow, const float* kp, int D) {
    float acc = 0.f;
    if (VEC) {
      for (int d0 = 0; d0 < D; d0 += 4) {
        const float4 v = *reinterpret_cast<const float4*>(kp + d0);
        acc = fmaf(qrow[d0], v.x, acc);
        acc = fmaf(qrow[d0 + 1], v.y, acc);
        acc = fmaf(qrow[d0 + 2], v.z, acc);
        acc = fmaf(qrow[d0 + 3], v.w, acc);
      }
    } else {
      for (int d = 0; d < D; ++d) acc = fmaf(qrow[d], kp[d], acc);
    }
    return acc;
  }
};
template <bool VEC> struct KeyDot<bf16_t, VEC> {
  __device__ __forceinline__ static float run(const float* qrow, const bf16_t* kp, int D) {
    float acc = 0.f;
    if (VEC) {
      for (int d0 = 0; d0 < D; d0 += 8) {
        const uint4 v = *reinterpret_cast<const uint4*>(kp + d0);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc = fmaf(qrow[d0 + 2 * e], __uint_as_float(w[e] << 16), acc);
          acc = fmaf(qrow[d0 + 2 * e + 1], __uint_as_float(w[e] & 0xffff0000u), acc);
        }
      }
    } else {
      for (int d = 0; d < D; ++d) acc = fmaf(qrow[d], bf16_to_f32(kp[d].bits), acc);
    }
    return acc;
  }
};

// ---- candidates of the kept blocks -----------------------------------------
// One wave (workgroup) per row.  Candidate c maps to a kept slot by binary
// search over the slots' prefix counts; its key is scored by the lane.
// block_token (:322-344): sort keys (~order(score) << 32 | key) ascending in
// LDS (bitonic), i.e. score desc, key asc; the row keeps kq = min(kk, max over
// (b, h) of the position's candidate count) slots (:159-160); slots past the
// row's own candidates but below kq take the lowest-index keys outside the
// candidate set with score -FLT_MAX and are invalid (what the masked top-k over
// -FLT_MAX ties returns under the lowest-index rule); slots >= kq hold index 0.
// block_only (:346-359): every candidate becomes a slot, in generation order.
// LDS of block_cand_kernel, sized per launch: the query row, the kept slots'
// prefix counts and (block_token) the sort keys of the candidates.
constexpr size_t CAND_Q_BYTES = BLK_MAX_D * sizeof(float);
__host__ __device__ inline size_t cand_pre_bytes(int eb) { return ((size_t)(eb + 1) * sizeof(int) + 7) & ~(size_t)7; }
inline int cand_npad(int ks) {
  int n = 1;
  while (n < ks) n <<= 1;
  return n;
}

template <typename X, bool VEC, bool TOKEN, bool MF>
__global__ __launch_bounds__(64) void block_cand_kernel(BlockArgs a, float mscale) {
  extern __shared__ __align__(16) char cand_lds[];
  float* qrow = reinterpret_cast<float*>(cand_lds);
  int* pre = reinterpret_cast<int*>(cand_lds + CAND_Q_BYTES);
  uint64_t* keys = reinterpret_cast<uint64_t*>(cand_lds + CAND_Q_BYTES + cand_pre_bytes(a.eb));
  const long row = blockIdx.x;
  const int lane = threadIdx.x;
  const int T = a.T, H = a.H, D = a.D, bs = a.bs, eb = a.eb;
  const int t = (int)(row % T);
  const long bh = row / T;
  const int b = (int)(bh / H), h = (int)(bh % H);
  const int lim = a.causal ? t : T - 1;
  const int nvb = lim / bs + 1;
  const bool masked = a.mask != nullptr;
  const int kqb = masked ? a.mkqb[t] : min(eb, nvb);
  const int32_t* pc = masked ? a.mpc + (long)b * (T + 1) : nullptr;
  const int32_t* perm = masked ? a.mperm + (long)b * T : nullptr;
  const uint8_t* mrow = masked ? a.mask + (long)b * T : nullptr;
  const bool qok = !masked || mrow[t] != 0;
  const int32_t* bi = a.block_indices + row * eb;
  const X* Q = reinterpret_cast<const X*>(a.q);
  const X* K = reinterpret_cast<const X*>(a.k);

  for (int d = lane; d < D; d += 64) qrow[d] = ld(Q, ((long)(b * T + t) * H + h) * D + d);
  // candidates of kept block s: its keys <= lim (with a mask, its valid ones)
  int run = 0;
  for (int s0 = 0; s0 < kqb; s0 += 64) {
    const int s = s0 + lane;
    int c = 0;
    if (s < kqb) {
      const int bj = bi[s];
      const int hi = min(bj * bs + bs, lim + 1);
      c = masked ? (qok ? pc[hi] - pc[bj * bs] : 0) : hi - bj * bs;
    }
    const int inc = (int)wave_incl_scan((uint32_t)c);
    if (s < kqb) pre[s] = run + inc - c;
    run += __shfl(inc, 63, 64);
  }
  const int ncand = run;
  wave_sync_lds();

  auto key_of = [&](int c) {
    int lo = 0, hi = kqb - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (pre[mid] <= c) lo = mid;
      else hi = mid - 1;
    }
    // the (c - pre[lo])-th candidate of block bi[lo]
    return masked ? perm[pc[bi[lo] * bs] + (c - pre[lo])] : bi[lo] * bs + (c - pre[lo]);
  };
  float m1 = -FLT_MAX;
  if constexpr (MF && sizeof(X) == 4) {
    // fp32: block_max_f32mfma_kernel's steps -- step 4j + e multiplies dimension 16j + 4lg + e,
    // A row lc = candidate c0 + lc, every B column the query -- so the scores agree bit for bit
    const int nj = D / 16, lg = lane >> 4, lc = lane & 15;
    const float* Qf = reinterpret_cast<const float*>(a.q) + ((long)(b * T + t) * H + h) * D;
    const float* Kf = reinterpret_cast<const float*>(a.k);
    float4 qa[BLK_MAX_D / 16];
#pragma unroll
    for (int j = 0; j < BLK_MAX_D / 16; ++j)
      qa[j] = j < nj ? *reinterpret_cast<const float4*>(Qf + 16 * j + 4 * lg) : make_float4(0.f, 0.f, 0.f, 0.f);
    for (int c0 = 0; c0 < ncand; c0 += 16) {
      const int ca = c0 + lc;
      const int key = ca < ncand ? key_of(ca) : 0;
      const float* kp = Kf + ((long)(b * T + key) * H + h) * D;
      f4 acc = f4_zero();
#pragma unroll
      for (int j = 0; j < BLK_MAX_D / 16; ++j) {
        if (j < nj) {
          const float4 kv = *reinterpret_cast<const float4*>(kp + 16 * j + 4 * lg);
          acc = mma_f32(kv.x, qa[j].x, acc);
          acc = mma_f32(kv.y, qa[j].y, acc);
          acc = mma_f32(kv.z, qa[j].z, acc);
          acc = mma_f32(kv.w, qa[j].w, acc);
        }
      }
      const f4 sv4 = score_of(acc, mscale);
      const float sv = lc == 0 ? sv4[0] : lc == 1 ? sv4[1] : lc == 2 ? sv4[2] : sv4[3];
      const int c = c0 + 4 * lg + lc;
      const int ckey = __shfl(key, 4 * lg + lc, 64);
      if (lc < 4 && c < ncand) {
        if (TOKEN) {
          keys[c] = ((uint64_t)(~f32_order_key(sv)) << 32) | (uint32_t)ckey;
        } else {
          a.slot_idx[row * a.ks + c] = ckey;
          a.slot_sc[row * a.ks + c] = sv;
          m1 = fmaxf(m1, sv);
        }
      }
    }
  } else if (MF) {
    // 16 candidates per MFMA group as the A operand (row lc = candidate c0+lc),
    // every B column the query: the same operand roles and instruction
    // sequence as block_max_mfma_kernel, so the scores agree bit for bit.
    const int nks = D / 32, lg = lane >> 4, lc = lane & 15;
    const uint16_t* Qb = reinterpret_cast<const uint16_t*>(a.q) + ((long)(b * T + t) * H + h) * D;
    const uint16_t* Kb = reinterpret_cast<const uint16_t*>(a.k);
    bf16x8 qa[BLK_MAX_D / 32];
#pragma unroll
    for (int s = 0; s < BLK_MAX_D / 32; ++s) {
      u16x8 raw = {0, 0, 0, 0, 0, 0, 0, 0};
      if (s < nks) raw = *reinterpret_cast<const u16x8*>(Qb + 32 * s + 8 * lg);
      qa[s] = __builtin_bit_cast(bf16x8, raw);
    }
    // NK = D / 32 when it is 4 (straight-line k-steps), 0 for D / 32 at run time
    auto score_groups = [&](auto nkt) __attribute__((always_inline)) {
      constexpr int NK = decltype(nkt)::value;
      for (int c0 = 0; c0 < ncand; c0 += 16) {
        const int ca = c0 + lc;   // the candidate this lane loads as A row lc
        const int key = ca < ncand ? key_of(ca) : 0;
        const uint16_t* kp = Kb + ((long)(b * T + key) * H + h) * D;
        f4 acc = f4_zero();
#pragma unroll
        for (int s = 0; s < BLK_MAX_D / 32; ++s)
          if (NK ? s < NK : s < nks) acc = mma_bf16(__builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8*>(kp + 32 * s + 8 * lg)), qa[s], acc);
        // accumulator element i holds A row 4lg+i, i.e. candidate c0+4lg+i; lane lc == i reports it
        const f4 sv4 = score_of(acc, mscale);
        const float sv = lc == 0 ? sv4[0] : lc == 1 ? sv4[1] : lc == 2 ? sv4[2] : sv4[3];
        const int c = c0 + 4 * lg + lc;
        const int ckey = __shfl(key, 4 * lg + lc, 64);   // key of candidate c (lane 4lg+lc loaded it)
        if (lc < 4 && c < ncand) {
          if (TOKEN) {
            keys[c] = ((uint64_t)(~f32_order_key(sv)) << 32) | (uint32_t)ckey;
          } else {
            a.slot_idx[row * a.ks + c] = ckey;
            a.slot_sc[row * a.ks + c] = sv;
            m1 = fmaxf(m1, sv);
          }
        }
      }
    };
    if (nks == 4) score_groups(std::integral_constant<int, 4>{});
    else score_groups(std::integral_constant<int, 0>{});
  }
  for (int c = MF ? ncand : lane; c < ncand; c += 64) {
    const int key = key_of(c);
    const float s = block_score(KeyDot<X, VEC>::run(qrow, K + ((long)(b * T + key) * H + h) * D, D), mscale);
    if (TOKEN) {
      keys[c] = ((uint64_t)(~f32_order_key(s)) << 32) | (uint32_t)key;
    } else {
      a.slot_idx[row * a.ks + c] = key;
      a.slot_sc[row * a.ks + c] = s;
      m1 = fmaxf(m1, s);
    }
  }

  if (!TOKEN) {
    m1 = wave_max(m1);
    if (lane == 0) {
      a.counts[row] = ncand;
      a.top2[2 * row] = m1;
      a.top2[2 * row + 1] = -FLT_MAX;
    }
    return;
  }

  int npad = 1;
  while (npad < ncand) npad <<= 1;
  for (int c = ncand + lane; c < npad; c += 64) keys[c] = ~0ull;
  wave_sync_lds();
  for (int span = 2; span <= npad; span <<= 1) {
    for (int j = span >> 1; j > 0; j >>= 1) {
      for (int i = lane; i < npad; i += 64) {
        const int p = i ^ j;
        if (p > i) {
          const uint64_t x = keys[i], y = keys[p];
          if ((x > y) == ((i & span) == 0)) {
            keys[i] = y;
            keys[p] = x;
          }
        }
      }
      wave_sync_lds();
    }
  }

  int mc = 1;
  for (int e = lane; e < a.B * a.H; e += 64) mc = max(mc, a.ncand[(long)e * T + t]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mc = max(mc, __shfl_xor(mc, o, 64));
  const int kk = a.kk, kq = min(kk, mc), nv = min(ncand, kq);
  int32_t* oi = a.slot_idx + row * kk;
  float* os = a.slot_sc + row * kk;
  uint8_t* ov = a.slot_valid + row * kk;
  for (int i = lane; i < kk; i += 64) {
    if (i < nv) {
      const uint64_t x = keys[i];
      oi[i] = (int)(uint32_t)x;
      os[i] = key_to_f32(~(uint32_t)(x >> 32));
      ov[i] = 1;
    } else if (i >= kq) {
      oi[i] = 0;
      os[i] = -FLT_MAX;
      ov[i] = 0;
    }
  }
  if (nv < kq) {
    const int need = kq - nv;
    const bool all_kept = kqb == nvb;
    int found = 0;
    for (int j0 = 0; found < need && j0 < T; j0 += 64) {
      const int j = j0 + lane;
      bool member = false;
      if (j < T && j <= lim && (!masked || (qok && mrow[j] != 0))) {
        if (all_kept) {
          member = true;
        } else {
          const int bj = j / bs;
          for (int s = 0; s < kqb; ++s) member |= bi[s] == bj;
        }
      }
      const bool outside = j < T && !member;
      const uint64_t m = ballot64(outside);
      const int r = found + (int)lane_rank(m);
      if (outside && r < need) {
        oi[nv + r] = j;
        os[nv + r] = -FLT_MAX;
        ov[nv + r] = 0;
      }
      found += popc64(m);
    }
  }
  if (lane == 0) {
    a.counts[row] = kq;
    a.top2[2 * row] = nv >= 1 ? key_to_f32(~(uint32_t)(keys[0] >> 32)) : -FLT_MAX;
    a.top2[2 * row + 1] = nv >= 2 ? key_to_f32(~(uint32_t)(keys[1] >> 32)) : -FLT_MAX;
  }
}

// block_only weights as the reference returns them, dense [B,H,T,T]: zero the
// row, then place each slot's weight at its key (keys of a row are distinct).
__global__ __launch_bounds__(256) void block_dense_weights_kernel(int T, int ks, const int32_t* __restrict__ idx,
                                                                  const float* __restrict__ w,
                                                                  const int32_t* __restrict__ counts,
                                                                  float* __restrict__ dense) {
  const long row = blockIdx.x;
  float* out = dense + row * T;
  for (int j = threadIdx.x; j < T; j += 256) out[j] = 0.f;
  __syncthreads();
  const int n = counts[row];
  for (int s = threadIdx.x; s < n; s += 256) out[idx[row * ks + s]] = w[row * ks + s];
}

template <typename X, bool MF>
static void launch_cand(const BlockArgs& a, float ms, bool vec, hipStream_t st) {
  const dim3 grid((unsigned)((long)a.B * a.H * a.T));
  // ncand <= ks = eb * min(bs, T): the sort needs next_pow2(ks) keys (<= BLK_MAXC)
  const size_t lds = CAND_Q_BYTES + cand_pre_bytes(a.eb) + (a.mode == 1 ? (size_t)cand_npad(a.ks) * 8 : 0);
  if (a.mode == 1) {
    if (vec) block_cand_kernel<X, true, true, MF><<<grid, 64, lds, st>>>(a, ms);
    else block_cand_kernel<X, false, true, MF><<<grid, 64, lds, st>>>(a, ms);
  } else {
    if (vec) block_cand_kernel<X, true, false, MF><<<grid, 64, lds, st>>>(a, ms);
    else block_cand_kernel<X, false, false, MF><<<grid, 64, lds, st>>>(a, ms);
  }
}

bool block_uses_mfma(const BlockArgs& a) {
  auto aligned = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  return a.dtype == DT_BF16 && a.D % 32 == 0 && aligned(a.q) && aligned(a.k);
}

// fp32 inputs with D % 16 == 0 (at most BLK_MAX_D) take the fp32 MFMA sweep and scorer
static bool block_uses_f32_mfma(const BlockArgs& a) {
  auto aligned = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  return a.dtype == DT_F32 && a.D % 16 == 0 && a.D <= BLK_MAX_D && aligned(a.q) && aligned(a.k);
}

hipError_t launch_block_select(const BlockArgs& a, hipStream_t st) {
  const float ms = score_multiplier((float)sqrt((double)a.D), 0);
  if (a.mask) {
    block_mask_prep_kernel<<<dim3((unsigned)a.B), 1024, 0, st>>>(a);
    block_mask_kq_kernel<<<dim3((unsigned)((a.T + 255) / 256)), 256, 0, st>>>(a);
  }
  const dim3 g1((unsigned)((a.T + 63) / 64), (unsigned)(a.B * a.H));
  const dim3 g2((unsigned)((a.T + BMM_ROWS - 1) / BMM_ROWS), (unsigned)(a.B * a.H));
  const bool mf = block_uses_mfma(a), mf32 = block_uses_f32_mfma(a);
  if (mf && (a.bs == 16 || a.bs == 32)) {
    // D is a multiple of 32 and at most BLK_MAX_D (block_uses_mfma, the entry points' checks)
    const dim3 gh(g2.y, g2.x);   // (B*H, row blocks)
    switch ((a.mask ? 8 : 0) + a.D / 32) {
      case 1: block_max_reg_kernel<false, 1><<<gh, 256, 0, st>>>(a, ms); break;
      case 2: block_max_reg_kernel<false, 2><<<gh, 256, 0, st>>>(a, ms); break;
      case 3: block_max_reg_kernel<false, 3><<<gh, 256, 0, st>>>(a, ms); break;
      case 4: block_max_reg_kernel<false, 4><<<gh, 256, 0, st>>>(a, ms); break;
      case 9: block_max_reg_kernel<true, 1><<<gh, 256, 0, st>>>(a, ms); break;
      case 10: block_max_reg_kernel<true, 2><<<gh, 256, 0, st>>>(a, ms); break;
      case 11: block_max_reg_kernel<true, 3><<<gh, 256, 0, st>>>(a, ms); break;
      case 12: block_max_reg_kernel<true, 4><<<gh, 256, 0, st>>>(a, ms); break;
      default: return hipErrorInvalidValue;
    }
  }
  else if (mf && a.bs % 16 == 0) block_max_mfma_kernel<true><<<g2, 256, 0, st>>>(a, ms);
  else if (mf) block_max_mfma_kernel<false><<<g2, 256, 0, st>>>(a, ms);
  else if (mf32 && a.bs % 16 == 0) block_max_f32mfma_kernel<true><<<g2, 256, 0, st>>>(a, ms);
  else if (mf32) block_max_f32mfma_kernel<false><<<g2, 256, 0, st>>>(a, ms);
  else if (a.dtype == DT_F32) block_max_kernel<float><<<g1, 256, 0, st>>>(a, ms);
  else block_max_kernel<bf16_t><<<g1, 256, 0, st>>>(a, ms);
  const long rows = (long)a.B * a.H * a.T;
  block_select_kernel<<<dim3((unsigned)((rows + 255) / 256)), 256, 0, st>>>(a);
  const int epv = a.dtype == DT_F32 ? 4 : 8;
  const bool vec = a.D % epv == 0 && ((uintptr_t)a.k & 15u) == 0;
  if (mf) launch_cand<bf16_t, true>(a, ms, vec, st);
  else if (mf32) launch_cand<float, true>(a, ms, vec, st);
  else if (a.dtype == DT_F32) launch_cand<float, false>(a, ms, vec, st);
  else launch_cand<bf16_t, false>(a, ms, vec, st);
  return hipGetLastError();
}

hipError_t launch_block_scores_transpose(const float* src, int B, int H, int T, int nb, float* dst, hipStream_t st) {
  const long n = (long)B * H * T * nb;
  block_scores_transpose_kernel<<<dim3((unsigned)((n + 255) / 256)), 256, 0, st>>>(src, n, T, nb, dst);
  return hipGetLastError();
}

hipError_t launch_block_dense_weights(int B, int H, int T, int ks, const int32_t* idx, const float* w,
                                      const int32_t* counts, float* dense, hipStream_t st) {
  block_dense_weights_kernel<<<dim3((unsigned)((long)B * H * T)), 256, 0, st>>>(T, ks, idx, w, counts, dense);
  return hipGetLastError();
}

}  // namespace sgsa
