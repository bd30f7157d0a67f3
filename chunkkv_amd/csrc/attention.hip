// Attention of the active rows over the whole cache, with the causal mask given by positions:
// query row i (absolute position pos[i]) attends to cache rows j <= pos[i] of its KV head.
//
// Reference semantics (src/chunkkv/engine/torch_engine.py): the mask is materialised as a
// boolean (n_active x N) tensor, mask = active[:, None] >= arange(N)[None, :] (:157), and
// F.scaled_dot_product_attention(q, K, V, attn_mask=mask, enable_gqa=True) (:68-72) runs with
// the default scale 1/sqrt(head_dim); query head h reads KV head h / (Hq / Hkv). This kernel
// computes the same function from the positions alone: no mask tensor, no KV-head expansion.
//
// Design (gfx950, flash-attention forward): one workgroup = 4 wavefronts = 128 queries of one
// query head; it walks the cache in 64-row tiles up to the largest position among its queries
// (tiles past a wavefront's own queries are skipped by that wavefront). Both products run on
// the bf16 matrix cores (v_mfma_f32_16x16x32_bf16) in transposed form:
//   S^T = K Q^T   (A = K rows from LDS, B = the wavefront's Q rows held in registers)
//   O^T = V^T P^T (A = V^T rows from LDS, B = P straight from the S^T accumulators)
// so that every lane owns one query (lane % 16) for the whole computation: the online-softmax
// max/sum and the output rows live in that lane and only two xor-shuffles per tile combine the
// four lane groups. K/V tiles go from global memory straight into double-buffered LDS (no
// register staging, one barrier per tile), in swizzled rows that make the fragment reads
// conflict-free; V^T comes out of row-major V through transposing LDS reads. Scores and the output accumulate in
// fp32; P is rounded to bf16 for the second product (as fused SDPA kernels do). When a launch
// would have too few workgroups to fill the chip (decode: one query, long cache) the cache range
// is split over more workgroups (flash-decoding): each writes unnormalised fp32 rows with their
// running max and sum to a caller-provided workspace, and a small kernel merges the splits. Built with the
// MFMA VGPR form (no accumulator-register copies around the online-softmax rescale).
#include <algorithm>

#include "ckv_common.hpp"

namespace ckv {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#ifndef CKV_ATTN_QG
#define CKV_ATTN_QG 2
#endif
constexpr int kAttnWaves = 4;
constexpr int kAttnQG = CKV_ATTN_QG;                // 16-query groups per wavefront
constexpr int kAttnBM = kAttnWaves * kAttnQG * 16;  // queries per workgroup
constexpr int kAttnBN = 64;                         // cache rows per tile

// Combine a lane's value with the lanes 16 and 32 away (the four lane groups of one query), with
// gfx950's row-swap permutes (VALU, no LDS round trip): each returns the lane's own value and
// its partner's, in an order that depends on the lane, so only order-free combinations are used.
__device__ __forceinline__ float group_max(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float group_sum(float v) {  // fp32 addition commutes: every lane agrees
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

typedef short v4i16 __attribute__((ext_vector_type(4)));

// LDS tiles (K and V, 64 cache rows each) are unpadded rows of D x 2 bytes, CPR 16-byte chunks,
// filled by direct-to-LDS loads. Spreading over the banks comes from swizzles of the chunk index:
// chunk c of slot s holds logical chunk c ^ swz(s).
//  - K: swz_k(s) = s % CPR. The 16 lanes of one lane group read one logical chunk of 16
//    consecutive slots for an S^T operand (16-byte reads): 16 distinct physical chunks.
//  - V: swz_v(s) = 2 (s % 4) + 8 ((s / 8) % 2) (CPR = 16; 2 (s % 4) for CPR = 8). A transposing
//    read of a lane group covers 4 consecutive slots x 2 adjacent chunks x 2 halves; the swizzle
//    puts them, and the next lane group's 4 slots 8 rows on, on distinct 8-byte bank ranges.
//  - K slot s of a 32-row block holds cache row kslot_row(s): slot 16 t + 4 a + b <- row
//    8 a + 4 t + b, so the 16 slots one S^T operand reads give each lane 8 consecutive rows of
//    the output (the rows its P^T operand pairs with V). V slots hold rows in order.
// Without the swizzles the kernel takes 0.405 ms instead of 0.220 ms on the 2976-row case.
template <int CPR>
__device__ __forceinline__ int swz_k(int s) { return s % CPR; }
template <int CPR>
__device__ __forceinline__ int swz_v(int s) { return CPR >= 16 ? 2 * (s % 4) + 8 * ((s / 8) % 2) : 2 * (s % 4); }
__device__ __forceinline__ int kslot_row(int s) {
  const int k = s & 31;
  return (s & ~31) + 8 * ((k >> 2) & 3) + 4 * (k >> 4) + (k & 3);
}

#ifndef CKV_ATTN_PRIO
#define CKV_ATTN_PRIO 0  // 1: raise the wavefront's issue priority around its matrix-core sections
#endif
#ifndef CKV_ATTN_MFMA_SUM
#define CKV_ATTN_MFMA_SUM 1  // softmax row sums on the matrix cores (a ones operand) instead of VALU adds
#endif
#ifndef CKV_ATTN_XCD
#define CKV_ATTN_XCD 1  // place the workgroups of one KV head on the same XCDs
#endif
constexpr int kXcds = 8;  // MI355X: workgroups go round-robin to 8 XCDs, each with its own L2

// Work item (query block qb, query head hq, cache split z) of this workgroup. The hardware hands
// workgroup L (x fastest, then y, then z) to XCD L % 8, so items are assigned through L: the
// XCDs split evenly over the KV heads (8 / Hkv XCDs each), every item of one KV head lands on
// that head's XCDs (its K/V stay in their L2s and are read there by all `group` query heads
// together), consecutive items of an XCD cycle through the group's query heads on one query
// block and split, and query blocks go latest position first, alternating between the head's
// XCDs so their work stays balanced. Items that do not fill a last round of 8 are dealt to the
// workgroups of that round. A bijection of the grid; with a KV-head count that does not divide 8
// the plain order is kept.
__device__ __forceinline__ void attn_work_item(int nqb, int Hq, int group, int& qb, int& hq, int& z) {
  qb = nqb - 1 - (int)blockIdx.x;  // latest positions (most keys) first
  hq = (int)blockIdx.y;
  z = (int)blockIdx.z;
  const int Hkv = Hq / group;
  if (!CKV_ATTN_XCD || kXcds % Hkv != 0) return;
  const int L = (int)blockIdx.x + ((int)blockIdx.y + (int)blockIdx.z * Hq) * nqb;
  const int xpk = kXcds / Hkv, P = group * nqb * (int)gridDim.z;  // XCDs, items per KV head
  const int per = P * Hkv / kXcds, full = per * kXcds;              // complete rounds of 8 workgroups
  int kv, j;
  if (L < full) {
    const int xcd = L % kXcds, idx = L / kXcds;
    kv = xcd / xpk;
    j = idx * xpk + xcd % xpk;
  } else {
    const int left = P - xpk * per;  // items per KV head past the complete rounds (> 0 here)
    const int t = L - full;
    kv = t / left;
    j = xpk * per + t % left;
  }
  const int rest = j / group;
  hq = kv * group + j % group;
  qb = nqb - 1 - rest % nqb;
  z = rest / nqb;
}

// GROUPED (few queries, decode): a workgroup's query rows are (token, query head) pairs of ONE KV
// head, row r = token r / group, head hk * group + r % group, so the group's query heads share
// every K/V tile the workgroup loads (grid y = KV heads); otherwise rows are tokens of one query
// head (grid y = query heads).
template <int D, bool GROUPED>
__global__ __launch_bounds__(kAttnWaves * 64) void attn_active_kernel(
    char* __restrict__ out, const char* __restrict__ q, int64_t q_hs_b, int64_t q_ts_b,
    const char* __restrict__ kc, const char* __restrict__ vc, int64_t kv_hs_b,
    const int64_t* __restrict__ pos, int n, int N, int Hq, int group, float scale_log2, int split_tiles,
    float* __restrict__ ws, int32_t* __restrict__ err) {
  constexpr int DS = D / 32;          // k-steps of S^T = K Q^T
  constexpr int DT = D / 16;          // 16-row tiles of O^T
  constexpr int CPR = D / 8;          // 16-byte chunks per cache row
  constexpr int ROWB = D * 2;        // bytes per cache row (and LDS slot)
  constexpr int NT = kAttnWaves * 64;
  static_assert(D % 32 == 0, "head_dim must be a multiple of 32");
  static_assert((kAttnBN * CPR) % NT == 0, "tile loads must tile the workgroup");
  static_assert((CPR & (CPR - 1)) == 0 && CPR >= 8, "swizzles need a power-of-two chunk count");

  // Two buffers per tensor: tile t + 1 loads into one while tile t is read from the other.
  __shared__ __attribute__((aligned(1024))) char k_lds0[kAttnBN * ROWB];
  __shared__ __attribute__((aligned(1024))) char k_lds1[kAttnBN * ROWB];
  __shared__ __attribute__((aligned(1024))) char v_lds0[kAttnBN * ROWB];
  __shared__ __attribute__((aligned(1024))) char v_lds1[kAttnBN * ROWB];
  __shared__ int blk_max_s[kAttnWaves];

  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int g = lane / 16, lm = lane % 16;
  int qb, hq, z;
  if (GROUPED) {
    int hk0;
    attn_work_item((int)gridDim.x, Hq / group, 1, qb, hk0, z);
    hq = hk0 * group;  // the group's first query head
  } else {
    attn_work_item((int)gridDim.x, Hq, group, qb, hq, z);
  }
  const int hk = hq / group;
  const int q0 = qb * kAttnBM + wave * kAttnQG * 16;
  const int n_rows = GROUPED ? n * group : n;
  // This lane's query rows: token row_m and query head row_h (row_m >= n: no query).
  int row_m[kAttnQG], row_h[kAttnQG];
#pragma unroll
  for (int qg = 0; qg < kAttnQG; ++qg) {
    const int r = q0 + qg * 16 + lm;
    row_m[qg] = r < n_rows ? (GROUPED ? r / group : r) : n;
    row_h[qg] = GROUPED ? hq + r % group : hq;
  }

  // Positions of this lane's queries (-1 = no query); out-of-range positions are flagged and
  // clamped so that every read stays inside the cache.
  int my_pos[kAttnQG];
  int wmax = -1, wmin = N;
#pragma unroll
  for (int qg = 0; qg < kAttnQG; ++qg) {
    const int m = row_m[qg];
    int p = -1;
    if (m < n) {
      const int64_t p64 = pos[m];
      if (p64 < 0 || p64 >= N) {
        flag_error(err, CKV_DEVICE_ERR_RANGE);
        p = p64 < 0 ? 0 : N - 1;
      } else {
        p = (int)p64;
      }
      wmin = min(wmin, p);
    }
    my_pos[qg] = p;
    wmax = max(wmax, p);
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) {
    wmax = max(wmax, __shfl_xor(wmax, s, 64));
    wmin = min(wmin, __shfl_xor(wmin, s, 64));
  }
  if (lane == 0) blk_max_s[wave] = wmax;
  __syncthreads();
  int bmax = blk_max_s[0];
#pragma unroll
  for (int w = 1; w < kAttnWaves; ++w) bmax = max(bmax, blk_max_s[w]);
  // This workgroup's share of the cache tiles: all of them, or split z of the key range when the
  // launch is split (flash-decoding: few queries, long cache) and partials go to ws.
  const int all_tiles = bmax < 0 ? 0 : bmax / kAttnBN + 1;
  const int tile_begin = ws != nullptr ? z * split_tiles : 0;
  const int n_tiles = ws != nullptr ? min(all_tiles, tile_begin + split_tiles) : all_tiles;

  // Q fragments (B operand of S^T): query q0 + 16 qg + lm, head-dim 32 s + 8 g .. + 8.
  bf16x8 qf[kAttnQG][DS];
#pragma unroll
  for (int qg = 0; qg < kAttnQG; ++qg) {
    const int m = row_m[qg];
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      vec16 v = {0, 0, 0, 0};
      if (m < n) v = ld16(q + (int64_t)row_h[qg] * q_hs_b + (int64_t)m * q_ts_b + (32 * s + 8 * g) * 2);
      qf[qg][s] = __builtin_bit_cast(bf16x8, v);
    }
  }

  f32x4 o[kAttnQG][DT];
  float m_run[kAttnQG], l_run[kAttnQG];
  // With CKV_ATTN_MFMA_SUM the row sums come from one more MFMA per key block with an all-ones A
  // operand: every row of its output is sum_k P^T[k][query], the sum of the bf16 weights that
  // multiply V (lane (g, lm) gets query lm's sum in each of its four values).
  f32x4 l_acc[kAttnQG];
  const bf16x8 ones = {(__bf16)1.f, (__bf16)1.f, (__bf16)1.f, (__bf16)1.f,
                       (__bf16)1.f, (__bf16)1.f, (__bf16)1.f, (__bf16)1.f};
#pragma unroll
  for (int qg = 0; qg < kAttnQG; ++qg) {
    m_run[qg] = -INFINITY;
    l_run[qg] = 0.f;
    l_acc[qg] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[qg][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const char* kh = kc + (int64_t)hk * kv_hs_b;
  const char* vh = vc + (int64_t)hk * kv_hs_b;

  // Tile loads go straight from global memory to LDS (global_load_lds_dwordx4): load
  // instruction i of wavefront w fills the 1 KB block w * KI + i of a tile buffer, lane l its 16
  // bytes at l * 16, i.e. position P = (w KI + i) 64 + l = slot P / CPR, chunk P % CPR. No
  // registers stage the tile and no LDS store instructions run; rows past the cache load row
  // N - 1 instead (every query's position is below them, so they are masked).
  constexpr int KI = (kAttnBN * CPR) / NT;  // load instructions per wavefront, tile and tensor
  static_assert(KI >= 1 && (kAttnBN * CPR) % NT == 0, "a tile must fill whole load instructions");
  int grow_k[KI], gcol_k[KI], gcol_v[KI];
#pragma unroll
  for (int i = 0; i < KI; ++i) {
    const int P = (wave * KI + i) * 64 + lane;
    const int slot = P / CPR, pc = P % CPR;
    grow_k[i] = kslot_row(slot);
    gcol_k[i] = (pc ^ swz_k<CPR>(slot)) * 16;
    gcol_v[i] = (pc ^ swz_v<CPR>(slot)) * 16;
  }
  typedef __attribute__((address_space(1))) void gvoid;
  typedef __attribute__((address_space(3))) void lvoid;
  auto issue = [&](int n0, char* kb, char* vb) {
#pragma unroll
    for (int i = 0; i < KI; ++i) {
      const int slot = ((wave * KI + i) * 64 + lane) / CPR;
      const int rk = min(n0 + grow_k[i], N - 1), rv = min(n0 + slot, N - 1);
      __builtin_amdgcn_global_load_lds((gvoid*)(kh + (int64_t)rk * ROWB + gcol_k[i]),
                                       (lvoid*)(kb + (wave * KI + i) * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((gvoid*)(vh + (int64_t)rv * ROWB + gcol_v[i]),
                                       (lvoid*)(vb + (wave * KI + i) * 1024), 16, 0, 0);
    }
  };
  // S^T operand of (kb, t, ds) for lane (g, lm): slot 32 kb + 16 t + lm, logical chunk 4 ds + g.
  int k_rd[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) k_rd[ds] = lm * ROWB + (((4 * ds + g) ^ swz_k<CPR>(lm)) * 16);
  // O^T's A operand (V^T rows) comes from row-major V through transposing 64-bit LDS loads:
  // in each 16-lane group, lane m names row 4h + m / 4 (of the group's 8 keys 8 g ..) at column
  // 4 (m % 4) of the 16-column tile, and lane 4a + b receives column 4a + b of rows 4h + 0..3.
  // So lane (g, lm) holds V[8 g + 4 h + e][16 dt + lm], e = 0..3: two loads (h = 0, 1) give the
  // eight keys 8 g + e' the B operand (P^T) pairs with that lane. Element 16 dt + 4 (lm % 4) is
  // logical chunk 2 dt + (lm % 4) / 2, byte 8 (lm % 2).
  auto v_rd = [&](int h, int dt) {
    const int row = 8 * g + 4 * h + lm / 4;
    return row * ROWB + (((2 * dt + (lm % 4) / 2) ^ swz_v<CPR>(row)) * 16) + 8 * (lm % 2);
  };
  if (tile_begin < n_tiles) issue(tile_begin * kAttnBN, k_lds0, v_lds0);

  // One tile; the loop below alternates the buffers (each call names its buffers directly, so
  // the compiler sees that the loads in flight never alias the buffer being read).
  auto body = [&](int tile, const char* k_lds, const char* v_lds, char* k_nxt, char* v_nxt) {
    const int n0 = tile * kAttnBN;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wavefront's loads of the tile landed
    __syncthreads();  // every wavefront's loads landed and every wavefront is done with the other buffer
    if (tile + 1 < n_tiles) issue(n0 + kAttnBN, k_nxt, v_nxt);  // lands during the MFMAs below

    if (n0 > wmax) return;  // uniform per wavefront: no query of this wavefront reaches the tile
    const bool need_mask = n0 + kAttnBN - 1 > wmin;

    // S^T for the tile: lane (g, lm) gets query lm, rows n0 + 32 kb + 8 g + 4 t + e.
    constexpr int KB = kAttnBN / 32;
    f32x4 s[kAttnQG][KB][2];
    if (CKV_ATTN_PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
          const bf16x8 a = *(const bf16x8*)(k_lds + (kb * 32 + 16 * t) * ROWB + k_rd[ds]);
#pragma unroll
          for (int qg = 0; qg < kAttnQG; ++qg)
            s[qg][kb][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[qg][ds], ds == 0 ? f32x4{0.f, 0.f, 0.f, 0.f}
                                                                                       : s[qg][kb][t], 0, 0, 0);
        }
      }
    if (CKV_ATTN_PRIO) __builtin_amdgcn_s_setprio(0);

    // Online softmax over the tile. The running max is only raised when a query's tile max
    // exceeds it by more than 2^8 (log2 domain): weights stay <= 256, the output rescale is
    // skipped for the whole wavefront otherwise, and the result is unchanged (the final division
    // uses the same max).
    bf16x8 pb[kAttnQG][KB];
#pragma unroll
    for (int qg = 0; qg < kAttnQG; ++qg) {
      // Raw scores of this lane (query lm, rows n0 + 32 kb + 8 g + 4 t + e); rows past the query's
      // position become -inf, on the tiles that reach past the lowest position only (uniform).
      float x[KB][8];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int e = 0; e < 4; ++e) x[kb][4 * t + e] = s[qg][kb][t][e];
      if (need_mask) {
        const int lim = my_pos[qg] - n0 - 8 * g;  // row offset 32 kb + 4 t + e must stay <= lim
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (32 * kb + j > lim) x[kb][j] = -INFINITY;
      }
      float bm = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j) bm = fmaxf(bm, x[kb][j]);
      bm = group_max(bm) * scale_log2;  // the scale is > 0: max commutes
      const bool raise = bm > m_run[qg] + 8.f;  // also true on the first visible tile (m_run = -inf)
      if (__builtin_amdgcn_ballot_w64(raise)) {  // uniform branch
        const float m_new = raise ? bm : m_run[qg];
        const float alpha = m_run[qg] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run[qg] - m_new);
        l_run[qg] *= alpha;
        l_acc[qg] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[qg][dt] *= alpha;
        m_run[qg] = m_new;
      }
      // p = 2^(score * scale - max) in one fma; with no visible row yet (absent queries) every
      // score is -inf and subtracting 0 keeps p = 0.
      const float msub = m_run[qg] == -INFINITY ? 0.f : m_run[qg];
      float psum = 0.f;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(x[kb][e], scale_log2, -msub));
          if (!CKV_ATTN_MFMA_SUM) psum += p;
          pb[qg][kb][e] = (__bf16)p;
        }
      if (!CKV_ATTN_MFMA_SUM) l_run[qg] += psum;
    }

    // O^T += V^T P^T: A = V^T rows dt*16 + lm, columns 32 kb + 8 g .. + 8.
    if (CKV_ATTN_PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
        const char* vb = v_lds + kb * 32 * ROWB;
        const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vb + v_rd(0, dt)));
        const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vb + v_rd(1, dt)));
        const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int qg = 0; qg < kAttnQG; ++qg)
          o[qg][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[qg][kb], o[qg][dt], 0, 0, 0);
        if (CKV_ATTN_MFMA_SUM && dt == DT - 1) {
#pragma unroll
          for (int qg = 0; qg < kAttnQG; ++qg)
            l_acc[qg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[qg][kb], l_acc[qg], 0, 0, 0);
        }
      }
    if (CKV_ATTN_PRIO) __builtin_amdgcn_s_setprio(0);
  };
  for (int tile = tile_begin; tile < n_tiles; tile += 2) {
    body(tile, k_lds0, v_lds0, k_lds1, v_lds1);
    if (tile + 1 < n_tiles) body(tile + 1, k_lds1, v_lds1, k_lds0, v_lds0);
  }

  // Normalise and write: lane (g, lm) holds O[query][dt*16 + 4g + e], 4 bf16 = 8 bytes per tile.
  // A split launch writes the unnormalised fp32 rows with their (max, sum) instead; the combine
  // kernel merges the splits.
#pragma unroll
  for (int qg = 0; qg < kAttnQG; ++qg) {
    const float l = CKV_ATTN_MFMA_SUM ? l_acc[qg][0] : group_sum(l_run[qg]);
    const int m = row_m[qg], h = row_h[qg];
    if (m >= n) continue;
    if (ws != nullptr) {
      float* prow = ws + (((int64_t)z * Hq + h) * n + m) * (D + 4);  // 16-byte aligned rows
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) *(float4*)(prow + dt * 16 + 4 * g) = make_float4(o[qg][dt][0], o[qg][dt][1],
                                                                                    o[qg][dt][2], o[qg][dt][3]);
      if (g == 0) {
        prow[D] = m_run[qg];
        prow[D + 1] = l;
      }
      continue;
    }
    const float inv = 1.f / l;
    char* orow = out + ((int64_t)m * Hq + h) * (D * 2);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      unsigned w[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) w[h] = f32x2_to_bf16x2_bits(o[qg][dt][2 * h] * inv, o[qg][dt][2 * h + 1] * inv);
      *(uint2*)(orow + (dt * 16 + 4 * g) * 2) = uint2{w[0], w[1]};
    }
  }
}

// Merge the splits of a split launch: for query m and head h, with (M_z, L_z, O_z) the partials
// of split z (max in the log2 domain, sum and unnormalised rows relative to M_z):
//   out = sum_z 2^(M_z - M) O_z / sum_z 2^(M_z - M) L_z,  M = max_z M_z  (splits with M_z = -inf
// saw no visible row and weigh 0). One workgroup of kCombineWaves wavefronts per (query, head):
// wavefront w folds splits w*4 .. w*4+3, then every (4 x kCombineWaves)-th group after them,
// loading each group's four partials together and merging them into a running (max, sum, row)
// with the online rescale; the wavefronts' results are merged through LDS. Lane d covers
// head-dim columns d, d + 64.
constexpr int kCombineWaves = 4;

template <int D>
__global__ __launch_bounds__(kCombineWaves * 64) void attn_combine_kernel(char* __restrict__ out,
                                                                          const float* __restrict__ ws, int n, int Hq,
                                                                          int splits) {
  constexpr int CW = D / 64;  // columns per lane
  constexpr int U = 4;        // partials in flight per wavefront
  const int m = blockIdx.x, hq = blockIdx.y, lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const int64_t stride = (int64_t)Hq * n * (D + 4);
  const float* base = ws + ((int64_t)hq * n + m) * (D + 4);
  float M = -INFINITY, L = 0.f, acc[CW];
#pragma unroll
  for (int j = 0; j < CW; ++j) acc[j] = 0.f;
  for (int z0 = wave * U; z0 < splits; z0 += U * kCombineWaves) {
    float mz[U], lz[U], oz[U][CW];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      mz[u] = -INFINITY;
      lz[u] = 0.f;
#pragma unroll
      for (int j = 0; j < CW; ++j) oz[u][j] = 0.f;
      if (z0 + u < splits) {
        const float* pz = base + (int64_t)(z0 + u) * stride;
        mz[u] = pz[D];
        lz[u] = pz[D + 1];
#pragma unroll
        for (int j = 0; j < CW; ++j) oz[u][j] = pz[lane + 64 * j];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (mz[u] == -INFINITY) continue;  // uniform: the same partial for every lane
      const float mn = fmaxf(M, mz[u]);
      const float a = __builtin_amdgcn_exp2f(M - mn);  // 0 while M is still -inf
      const float b = __builtin_amdgcn_exp2f(mz[u] - mn);
      L = L * a + lz[u] * b;
#pragma unroll
      for (int j = 0; j < CW; ++j) acc[j] = acc[j] * a + oz[u][j] * b;
      M = mn;
    }
  }
  __shared__ float s_m[kCombineWaves], s_l[kCombineWaves], s_o[kCombineWaves][D];
  if (lane == 0) {
    s_m[wave] = M;
    s_l[wave] = L;
  }
#pragma unroll
  for (int j = 0; j < CW; ++j) s_o[wave][lane + 64 * j] = acc[j];
  __syncthreads();
  if (wave != 0) return;
  float mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < kCombineWaves; ++w) mx = fmaxf(mx, s_m[w]);
  float lt = 0.f, o[CW];
#pragma unroll
  for (int j = 0; j < CW; ++j) o[j] = 0.f;
#pragma unroll
  for (int w = 0; w < kCombineWaves; ++w) {
    if (s_m[w] == -INFINITY) continue;
    const float sw = __builtin_amdgcn_exp2f(s_m[w] - mx);
    lt += sw * s_l[w];
#pragma unroll
    for (int j = 0; j < CW; ++j) o[j] += sw * s_o[w][lane + 64 * j];
  }
  const float inv = 1.f / lt;
  uint16_t* orow = reinterpret_cast<uint16_t*>(out + ((int64_t)m * Hq + hq) * (D * 2));
#pragma unroll
  for (int j = 0; j < CW; ++j) orow[lane + 64 * j] = (uint16_t)f32_to_bf16_bits(o[j] * inv);
}

}  // namespace ckv

namespace ckv {

#ifndef CKV_ATTN_GSPLIT
#define CKV_ATTN_GSPLIT 3
#endif
constexpr int kGroupedSplitTiles = CKV_ATTN_GSPLIT;  // cache tiles per split of a grouped launch

// Split plan of a launch whose rows are tokens of one query head: split only launches too small
// to fill the chip (decode-like), into about 1024 workgroups of >= 4 tiles each.
static void row_split_plan(int n_queries, int n_tokens, int n_q_heads, int& splits, int& split_tiles) {
  splits = 1;
  split_tiles = 0;
  const int64_t blocks = (int64_t)((n_queries + kAttnBM - 1) / kAttnBM) * n_q_heads;
  const int tiles = (n_tokens + kAttnBN - 1) / kAttnBN;
  constexpr int64_t kTarget = 1024;  // workgroups that fill the 256 CUs a few times over
  if (blocks < kTarget / 2 && tiles >= 8) {
    const int want = (int)std::min<int64_t>((kTarget + blocks - 1) / blocks, tiles / 4);
    split_tiles = (tiles + want - 1) / want;
    splits = (tiles + split_tiles - 1) / split_tiles;
  }
}

// Grouped launches (queries that share KV heads fit one workgroup's rows): every
// kGroupedSplitTiles cache tiles are one split. Usable when n_queries * group <= kAttnBM.
static void grouped_split_plan(int n_queries, int n_tokens, int& splits) {
  const int tiles = (n_tokens + kAttnBN - 1) / kAttnBN;
  splits = (2 * n_queries <= kAttnBM && tiles >= 2) ? (tiles + kGroupedSplitTiles - 1) / kGroupedSplitTiles : 1;
}

}  // namespace ckv

extern "C" int64_t ckv_attention_workspace_bytes(int32_t n_queries, int32_t n_tokens, int32_t n_q_heads,
                                                 int32_t head_dim, int32_t* splits_out, int32_t* split_tiles_out) {
  using namespace ckv;
  int splits = 1, split_tiles = 0, gsplits = 1;
  if (n_queries > 0 && n_tokens > 0 && n_q_heads > 0 && head_dim > 0) {
    row_split_plan(n_queries, n_tokens, n_q_heads, splits, split_tiles);
    grouped_split_plan(n_queries, n_tokens, gsplits);
  }
  if (splits_out != nullptr) *splits_out = splits;
  if (split_tiles_out != nullptr) *split_tiles_out = split_tiles;
  const int64_t row = (int64_t)n_q_heads * n_queries * (head_dim + 4) * 4;
  const int64_t most = std::max(splits > 1 ? splits : 0, gsplits > 1 ? gsplits : 0);
  return most * row;
}

extern "C" int32_t ckv_attention_active(void* out, const void* q, int64_t q_head_stride, int64_t q_token_stride,
                                        const void* k_cache, const void* v_cache, int64_t kv_head_stride,
                                        const int64_t* positions, int32_t n_queries, int32_t n_tokens,
                                        int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int32_t dtype,
                                        double scale, void* workspace, int64_t workspace_bytes, int32_t* err,
                                        void* stream) {
  using namespace ckv;
  if (out == nullptr || q == nullptr || k_cache == nullptr || v_cache == nullptr || positions == nullptr)
    return CKV_ERR_INVALID_ARGUMENT;
  if (dtype != CKV_DTYPE_BF16 || (head_dim != 64 && head_dim != 128)) return CKV_ERR_INVALID_ARGUMENT;
  if (n_queries < 0 || n_tokens <= 0 || n_q_heads <= 0 || n_kv_heads <= 0 || n_q_heads % n_kv_heads != 0 ||
      !(scale > 0.0))
    return CKV_ERR_INVALID_ARGUMENT;
  if (q_token_stride % 8 || q_head_stride % 8 || kv_head_stride % 8) return CKV_ERR_INVALID_ARGUMENT;  // 16-byte rows
  if (((uintptr_t)out | (uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16) return CKV_ERR_INVALID_ARGUMENT;
  if (q_token_stride < head_dim || kv_head_stride < (int64_t)n_tokens * head_dim) return CKV_ERR_OUT_OF_RANGE;
  if (n_queries == 0) return CKV_OK;
  if (n_q_heads > 65535) return CKV_ERR_TOO_LARGE;
  const float scale_log2 = (float)(scale * 1.4426950408889634);  // exp(x) = exp2(x log2 e)
  const int group = n_q_heads / n_kv_heads;
  hipStream_t st = (hipStream_t)stream;
  const int64_t row_b = (int64_t)n_q_heads * n_queries * (head_dim + 4) * 4;
  const bool ws_ok = workspace != nullptr && (uintptr_t)workspace % 16 == 0;
  auto launch = [&](auto kernel, auto combine, dim3 grid, int split_tiles, float* ws, int splits) {
    hipLaunchKernelGGL(kernel, grid, dim3(kAttnWaves * 64), 0, st, (char*)out, (const char*)q, q_head_stride * 2,
                       q_token_stride * 2, (const char*)k_cache, (const char*)v_cache, kv_head_stride * 2, positions,
                       n_queries, n_tokens, n_q_heads, group, scale_log2, split_tiles, ws, err);
    if (ws != nullptr)
      hipLaunchKernelGGL(combine, dim3((unsigned)n_queries, (unsigned)n_q_heads), dim3(kCombineWaves * 64), 0, st,
                         (char*)out, ws,
                         n_queries, n_q_heads, splits);
  };
  // Queries that share KV heads and fit one workgroup's rows (decode): one workgroup per
  // (KV head, split), all of the group's query heads on each loaded K/V tile.
  int gsplits = 1;
  grouped_split_plan(n_queries, n_tokens, gsplits);
  if (group > 1 && (int64_t)n_queries * group <= kAttnBM && gsplits > 1 && ws_ok &&
      workspace_bytes >= gsplits * row_b) {
    const dim3 grid(1u, (unsigned)n_kv_heads, (unsigned)gsplits);
    if (head_dim == 128)
      launch(attn_active_kernel<128, true>, attn_combine_kernel<128>, grid, kGroupedSplitTiles, (float*)workspace, gsplits);
    else
      launch(attn_active_kernel<64, true>, attn_combine_kernel<64>, grid, kGroupedSplitTiles, (float*)workspace, gsplits);
    CKV_RETURN_IF_LAUNCH_FAILED();
    return CKV_OK;
  }
  int splits = 1, split_tiles = 0;
  row_split_plan(n_queries, n_tokens, n_q_heads, splits, split_tiles);
  float* ws = (splits > 1 && ws_ok && workspace_bytes >= splits * row_b) ? (float*)workspace : nullptr;
  if (ws == nullptr) splits = 1;
  const dim3 grid((unsigned)((n_queries + kAttnBM - 1) / kAttnBM), (unsigned)n_q_heads, (unsigned)splits);
  if (head_dim == 128)
    launch(attn_active_kernel<128, false>, attn_combine_kernel<128>, grid, split_tiles, ws, splits);
  else
    launch(attn_active_kernel<64, false>, attn_combine_kernel<64>, grid, split_tiles, ws, splits);
  CKV_RETURN_IF_LAUNCH_FAILED();
  return CKV_OK;
}
