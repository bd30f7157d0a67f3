// Fresh-token RoPE of the projected q and k rows, written where their consumers read them: q in
// the layout of the attention kernel, k (and v, copied) either straight into the cache rows of
// their positions or into a separate tensor.
//
// Reference semantics (src/chunkkv/engine/torch_engine.py): _qkv (:61-66) views the q/k/v
// projections as heads and applies _rope (:53-54) to q and k: angles = positions.float()[:, None]
// * inv_freq[None, :], then _rotate (:46-51) in fp32 with one rounding to the element type; the
// cache rows of the active positions are then overwritten with k and v (:155-156). Here the
// rotation of token t uses the fp32 angle fl32(fl32(pos[t]) * inv_freq_i) with the correctly
// rounded fp32 cos/sin of that angle (evaluated in fp64), the same rotation ckv_shift_keys
// applies for a shift by pos[t]; products and sums are separately rounded fp32 operations.
//
// Design (gfx950): no cos/sin table by default. cos/sin come from the inverse frequencies (host,
// from theta, passed by value in the kernel arguments) and each token's position, evaluated in
// fp64 with the short reduction + series of cos_sin.hpp. A k/v-only launch (the cache repair)
// runs one wavefront per token, each lane evaluating one frequency once and the lanes sharing
// them through ds_bpermute; a launch with q shares each evaluation over 4 heads. A caller-kept
// per-position table (ckv_rope_table) is also accepted. All accesses are 16 bytes. The ~20 elementwise torch
// launches of the reference's RoPE (fp32 temporaries, cat, cast) and the separate scatter of k/v
// into the cache become one pass over the projection output.
#include <algorithm>

#include "ckv_common.hpp"

namespace ckv {

constexpr int kRopeThreads = 256;
// The k/v cache-row write: one wavefront (one token) per workgroup. In the 8k request step
// (26 launches of 2976 rows) 0.258 ms against 0.261 ms at 256 threads and 0.263 ms at 128.
constexpr int kRopeKvThreads = kWave;

// Without a table, k/v only (the cache-repair launch): one wavefront per token (TW tokens when
// D/2 < 64). An item is a 16-byte column pair (col, col + D/2) of one head row, rotated for k
// heads and copied for v heads; a token of Hkv k and Hkv v heads has 2 Hkv D/2/VEC items (64 at
// Hkv = 4, D = 128: one per lane). Lane l evaluates frequency l of its token once, from the
// position (loaded first: vector loads complete in order) while the lane's row data is still in
// flight, and the lanes fetch the VEC frequencies of their column from the evaluating lanes with
// ds_bpermute: every (token, frequency) is evaluated exactly once, with no LDS and no barrier.
constexpr int kWaveBatch = 2;  // items per lane whose loads go out before the cos/sin are built

template <int DTYPE, int D>
__global__ __launch_bounds__(kRopeThreads) void rope_wave_kernel(
    char* __restrict__ q_out, int64_t qo_hs_b, int64_t qo_ts_b, char* __restrict__ k_out, int64_t ko_hs_b,
    int64_t ko_ts_b, char* __restrict__ v_out, int64_t vo_hs_b, int64_t vo_ts_b, const int64_t* __restrict__ rows,
    int n_out, const char* __restrict__ q_in, int64_t qi_hs_b, int64_t qi_ts_b, const char* __restrict__ k_in,
    int64_t ki_hs_b, int64_t ki_ts_b, const char* __restrict__ v_in, int64_t vi_hs_b, int64_t vi_ts_b,
    const int64_t* __restrict__ pos, const InvFreq inv, int n, int Hq, int Hkv, int32_t* __restrict__ err) {
  using E = Elem<DTYPE>;
  constexpr int VEC = E::kVec;
  constexpr int HALF = D / 2;
  constexpr int TPR = HALF / VEC;  // items per head row
  constexpr int HALF_B = HALF * E::kBytes;
  constexpr int TW = HALF >= kWave ? 1 : kWave / HALF;   // tokens per wavefront
  constexpr int EVL = HALF >= kWave ? HALF / kWave : 1;  // evaluations per lane
  static_assert(kWave % TPR == 0 && (HALF % kWave == 0 || kWave % HALF == 0), "head_dim out of range");

  const int lane = threadIdx.x & (kWave - 1);
  const int t0 = (int)((blockIdx.x * (kRopeThreads / kWave) + threadIdx.x / kWave) * TW);
  if (t0 >= n) return;  // uniform per wavefront
  const int ntok = min(TW, n - t0);
  const int n_rk = Hq + Hkv;                                    // rotated heads: q, then k
  const int per = (n_rk + (v_out != nullptr ? Hkv : 0)) * TPR;  // items per token
  const int total = ntok * per;

  // 1. positions and rows of the wavefront's tokens
  int64_t pv[TW], rv[TW];
#pragma unroll
  for (int tl = 0; tl < TW; ++tl) {
    const int t = t0 + min(tl, ntok - 1);
    pv[tl] = pos[t];
    rv[tl] = rows != nullptr ? rows[t] : t;
  }
  // 2. the first kWaveBatch items' data, unconditionally (a lane past the end reloads the last
  // item), so that no branch hides a load from the wait counters
  auto src_of = [&](int it) {
    const int tl = it / per, k = it - tl * per;
    const int h = k / TPR, col = k % TPR;
    const int t = t0 + tl;
    const char* base = h < Hq    ? q_in + h * qi_hs_b + t * qi_ts_b
                       : h < n_rk ? k_in + (h - Hq) * ki_hs_b + t * ki_ts_b
                                  : v_in + (h - n_rk) * vi_hs_b + t * vi_ts_b;
    return base + col * 16;
  };
  vec16 a[kWaveBatch], b[kWaveBatch];
#pragma unroll
  for (int j = 0; j < kWaveBatch; ++j) {
    const char* src = src_of(min(lane + j * kWave, total - 1));
    a[j] = ld16(src);
    b[j] = ld16(src + HALF_B);
  }
  // 3. this lane's frequencies: token etl, frequencies lane (+ 64 j)
  const int etl = HALF >= kWave ? 0 : lane / HALF;
  int64_t pe = pv[0];
#pragma unroll
  for (int tl = 1; tl < TW; ++tl) pe = etl == tl ? pv[tl] : pe;
  const int pp = pe >= INT32_MIN && pe <= INT32_MAX ? (int)pe : 0;
  float ang[EVL], cv[EVL], sv[EVL];
#pragma unroll
  for (int j = 0; j < EVL; ++j) ang[j] = (float)pp * inv.v[HALF >= kWave ? lane + j * kWave : lane % HALF];
  angles_cos_sin<EVL>(ang, cv, sv);
  // 4. the VEC frequencies of this lane's column (the same column for all its items), per token
  const int col = lane % TPR;
  float c[TW][VEC], sn[TW][VEC];
#pragma unroll
  for (int tl = 0; tl < TW; ++tl) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const int f = col * VEC + e;
      const int src = HALF >= kWave ? f % kWave : tl * HALF + f;
      float cc = __shfl(cv[0], src), ss = __shfl(sv[0], src);
#pragma unroll
      for (int j = 1; j < EVL; ++j) {
        const float cj = __shfl(cv[j], src), sj = __shfl(sv[j], src);
        cc = f / kWave == j ? cj : cc;
        ss = f / kWave == j ? sj : ss;
      }
      c[tl][e] = cc;
      sn[tl][e] = ss;
    }
  }
  bool ok[TW];
#pragma unroll
  for (int tl = 0; tl < TW; ++tl) {
    ok[tl] = tl < ntok && pv[tl] >= INT32_MIN && pv[tl] <= INT32_MAX && rv[tl] >= 0 && rv[tl] < n_out;
    if (tl < ntok && !ok[tl] && lane == 0) flag_error(err, CKV_DEVICE_ERR_RANGE);
  }
  // 5. rotate k (and q), copy v, store; items past the first kWaveBatch of a lane load here
  for (int j0 = 0; lane + j0 * kWave < total; j0 += kWaveBatch) {
#pragma unroll
    for (int j = 0; j < kWaveBatch; ++j) {
      const int it = lane + (j0 + j) * kWave;
      if (it >= total) break;
      if (j0 > 0) {
        const char* src = src_of(it);
        a[j] = ld16(src);
        b[j] = ld16(src + HALF_B);
      }
      const int tl = it / per, h = (it - tl * per) / TPR;
      bool okt = ok[0];
      int64_t row = rv[0];
#pragma unroll
      for (int u = 1; u < TW; ++u) {
        okt = tl == u ? ok[u] : okt;
        row = tl == u ? rv[u] : row;
      }
      if (!okt) continue;
      const int t = t0 + tl;
      char* d = (h < Hq    ? q_out + h * qo_hs_b + t * qo_ts_b
                 : h < n_rk ? k_out + (h - Hq) * ko_hs_b + row * ko_ts_b
                            : v_out + (h - n_rk) * vo_hs_b + row * vo_ts_b) +
                col * 16;
      vec16 y1 = a[j], y2 = b[j];
      if (h < n_rk) {
        float cc[VEC], ss[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          cc[e] = c[0][e];
          ss[e] = sn[0][e];
#pragma unroll
          for (int u = 1; u < TW; ++u) {
            cc[e] = tl == u ? c[u][e] : cc[e];
            ss[e] = tl == u ? sn[u][e] : ss[e];
          }
        }
        rotate_pairs<DTYPE>(a[j], b[j], cc, ss, y1, y2);
      }
      st16(d, y1);
      st16(d + HALF_B, y2);
    }
  }
}

// k/v only with head_dim <= 128 and both k and v (the cache-repair launch of every layer): one
// wavefront per token and no integer division. Item i of a token is the 16-byte column pair
// (col, col + D/2) of head row i / TPR: k heads first (rotated), then v heads (copied). Lane f
// evaluates frequency f of the token's position once; the lanes fetch their column's VEC
// frequencies with ds_bpermute. The rows are stored non-temporally: a launch leaves no dirty
// lines in L2 for the next kernel boundary to write back (measured: ~0.9 us less per 2976-row
// launch in a chain of them).
// SHAPE: kKvLoop = items strided over the wavefront; kKvOne = at most one item per lane;
// kKvFull = exactly one item per lane (2 * Hkv * TPR == 64, Hkv a compile-time constant: the
// k/v split is lane < 32). RM: where a token's row goes: kRowToken (rows NULL: row = token),
// kRowPos (rows are the positions: no second load), kRowIndexed (row = rows[t]). Both are
// template parameters because the runtime forms cost ~0.3-0.4 us per 2976-row launch.
constexpr int kKvLoop = 0, kKvOne = 1, kKvFull = 2;
constexpr int kRowToken = 0, kRowPos = 1, kRowIndexed = 2;

#ifndef CKV_KV_TPW
#define CKV_KV_TPW 1
#endif
constexpr int kKvTpw = CKV_KV_TPW;  // tokens per wavefront of the k/v write

// The arguments come in the order a wavefront needs them: the first 64 bytes (what the token
// count check and the first loads use) fit the 16 SGPRs the library preloads, the frequency table
// comes last. TPW tokens per wavefront (TPW > 1 only with SHAPE != kKvLoop): every token's loads
// go out first, then the positions, then each lane evaluates its frequency for every token.
template <int DTYPE, int D, int SHAPE, int RM, int TPW>
__global__ __launch_bounds__(kRopeKvThreads) void rope_kv_kernel(
    int n, int n_kv_heads, const int64_t* __restrict__ pos, const char* __restrict__ k_in,
    const char* __restrict__ v_in, int64_t ki_hs_b, int64_t ki_ts_b, int64_t vi_hs_b, int64_t vi_ts_b,
    char* __restrict__ k_out, char* __restrict__ v_out, int64_t ko_hs_b, int64_t ko_ts_b, int64_t vo_hs_b,
    int64_t vo_ts_b, const int64_t* __restrict__ rows, int n_out, int32_t* __restrict__ err, const InvFreq inv) {
  using E = Elem<DTYPE>;
  constexpr int VEC = E::kVec;
  constexpr int HALF = D / 2;
  constexpr int TPR = HALF / VEC;  // column pairs per head row (a power of two)
  constexpr int HALF_B = HALF * E::kBytes;
  static_assert(HALF <= kWave && kWave % HALF == 0 && (TPR & (TPR - 1)) == 0, "head_dim out of range");
  static_assert(TPW == 1 || SHAPE != kKvLoop, "several tokens per wavefront need one item per lane at most");
  const int Hkv = SHAPE == kKvFull ? kWave / 2 / TPR : n_kv_heads;
  const int lane = threadIdx.x & (kWave - 1);
  const int t0 = (int)(blockIdx.x * (kRopeKvThreads / kWave) + threadIdx.x / kWave) * TPW;
  if (t0 >= n) return;  // uniform per wavefront
  const int items = 2 * Hkv * TPR;
  const int col = lane & (TPR - 1);
  // item it: head row it / TPR (TPR is a power of two: a shift), k rows first. Base pointer,
  // strides and head index are picked by value, so the k and v lanes share one address path.
  auto src_of = [&](int hh, int t) {
    const bool k = hh < Hkv;
    return (k ? k_in : v_in) + (k ? hh : hh - Hkv) * (k ? ki_hs_b : vi_hs_b) + t * (k ? ki_ts_b : vi_ts_b) + col * 16;
  };
  // the tokens past n (the last wavefront) load token n - 1 again and store nothing
  int tt[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) tt[j] = min(t0 + j, n - 1);
  // the first item's data goes out before anything waits on the position load
  const int h0 = (SHAPE == kKvFull ? lane : min(lane, items - 1)) / TPR;
  vec16 a[TPW], b[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const char* s0 = src_of(h0, tt[j]);
    // non-temporal loads: each input row is read once (the request step 0.258 -> 0.244 ms)
    a[j] = ld16_stream(s0);
    b[j] = ld16_stream(s0 + HALF_B);
  }
  int64_t p[TPW], row[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) p[j] = pos[tt[j]];
#pragma unroll
  for (int j = 0; j < TPW; ++j) row[j] = RM == kRowToken ? (int64_t)tt[j] : RM == kRowPos ? p[j] : rows[tt[j]];
  bool ok[TPW];
  float angs[TPW], cv[TPW], sv[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    ok[j] = p[j] >= INT32_MIN && p[j] <= INT32_MAX && row[j] >= 0 && row[j] < n_out;
    angs[j] = (float)(ok[j] ? (int)p[j] : 0) * inv.v[lane & (HALF - 1)];
  }
  angles_cos_sin<TPW>(angs, cv, sv);
  auto dst_of = [&](int hh, int64_t r) {
    const bool k = hh < Hkv;
    return (k ? k_out : v_out) + (k ? hh : hh - Hkv) * (k ? ko_hs_b : vo_hs_b) + r * (k ? ko_ts_b : vo_ts_b) +
           col * 16;
  };
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    if (j > 0 && t0 + j >= n) break;  // uniform
    float c[VEC], sn[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      c[e] = __shfl(cv[j], col * VEC + e);
      sn[e] = __shfl(sv[j], col * VEC + e);
    }
    if (!ok[j]) {  // uniform
      if (lane == 0) flag_error(err, CKV_DEVICE_ERR_RANGE);
      continue;
    }
    if constexpr (SHAPE != kKvLoop) {  // items <= one wavefront: a single pass, no loop
      char* d = dst_of(h0, row[j]);
      vec16 y1 = a[j], y2 = b[j];
      if (h0 < Hkv) rotate_pairs<DTYPE>(a[j], b[j], c, sn, y1, y2);
      if (SHAPE == kKvFull || lane < items) {
        st16_stream(d, y1);
        st16_stream(d + HALF_B, y2);
      }
    } else {
      vec16 aa = a[0], bb = b[0];
      for (int it = lane; it < items; it += kWave) {
        const int hh = it / TPR;
        if (it != lane) {
          const char* si = src_of(hh, tt[0]);
          aa = ld16_stream(si);
          bb = ld16_stream(si + HALF_B);
        }
        char* d = dst_of(hh, row[0]);
        vec16 y1 = aa, y2 = bb;
        if (hh < Hkv) rotate_pairs<DTYPE>(aa, bb, c, sn, y1, y2);
        st16_stream(d, y1);
        st16_stream(d + HALF_B, y2);
      }
    }
  }
}

// Without a table, with q (32+ rotated heads share each token's cos/sin): one thread per
// (token, 16-byte column, group of kRopeFreeHG heads), grid-stride, evaluating its VEC
// frequencies itself (kRopeFreeHG-fold sharing), v copied in 16-byte chunks. The thread's loads go
// out in the order their values are needed (position, row, inverse frequencies, data) and it
// branches on none of them before its stores.
constexpr int kRopeFreeHG = 4;

template <int DTYPE, int D>
__global__ __launch_bounds__(kRopeThreads) void rope_free_kernel(
    char* __restrict__ q_out, int64_t qo_hs_b, int64_t qo_ts_b, char* __restrict__ k_out, int64_t ko_hs_b,
    int64_t ko_ts_b, char* __restrict__ v_out, int64_t vo_hs_b, int64_t vo_ts_b, const int64_t* __restrict__ rows,
    int n_out, const char* __restrict__ q_in, int64_t qi_hs_b, int64_t qi_ts_b, const char* __restrict__ k_in,
    int64_t ki_hs_b, int64_t ki_ts_b, const char* __restrict__ v_in, int64_t vi_hs_b, int64_t vi_ts_b,
    const int64_t* __restrict__ pos, const InvFreq inv, int n, int Hq, int Hkv, int32_t* __restrict__ err) {
  using E = Elem<DTYPE>;
  constexpr int VEC = E::kVec;
  constexpr int HALF = D / 2;
  constexpr int TPR = HALF / VEC;
  constexpr int HALF_B = HALF * E::kBytes;
  constexpr int CPR = D * E::kBytes / 16;
  constexpr int HG = kRopeFreeHG;
  typedef __attribute__((address_space(1))) const int64_t gi64;
  const int n_heads = Hq + Hkv;
  const unsigned n_rot = (unsigned)((n_heads + HG - 1) / HG * TPR);  // rotation items per token
  const unsigned n_cp = v_out != nullptr ? (unsigned)(Hkv * CPR) : 0u;  // copy items per token
  const unsigned rot_total = (unsigned)n * n_rot;
  const unsigned total = rot_total + (unsigned)n * n_cp;  // < 2^31, checked by the host
  for (unsigned idx = blockIdx.x * kRopeThreads + threadIdx.x; idx < total; idx += gridDim.x * kRopeThreads) {
    const bool rot = idx < rot_total;
    const unsigned j = rot ? idx : idx - rot_total;
    const unsigned per = rot ? n_rot : n_cp;
    const int t = (int)(j / per), it = (int)(j - (unsigned)t * per);
    const int64_t p = *(gi64*)(pos + t);
    const int64_t row = rows != nullptr ? *(gi64*)(rows + t) : t;
    if (rot) {
      const int h0 = (it / TPR) * HG, col = it % TPR;
      float iv[VEC];
#pragma unroll
      for (int e = 0; e < VEC; e += 4) {
        const vec16 w = *reinterpret_cast<const vec16*>(&inv.v[col * VEC + e]);
        iv[e] = __uint_as_float(w[0]);
        iv[e + 1] = __uint_as_float(w[1]);
        iv[e + 2] = __uint_as_float(w[2]);
        iv[e + 3] = __uint_as_float(w[3]);
      }
      vec16 a[HG], b[HG];
#pragma unroll
      for (int jj = 0; jj < HG; ++jj) {
        const int h = min(h0 + jj, n_heads - 1);
        const char* s = (h < Hq ? q_in + h * qi_hs_b + t * qi_ts_b : k_in + (h - Hq) * ki_hs_b + t * ki_ts_b) +
                        col * 16;
        a[jj] = ld16(s);
        b[jj] = ld16(s + HALF_B);
      }
      const bool ok = p >= INT32_MIN && p <= INT32_MAX && row >= 0 && row < n_out;
      const int pp = ok ? (int)p : 0;
      float ang[VEC], c[VEC], sn[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) ang[e] = (float)pp * iv[e];
      angles_cos_sin<VEC>(ang, c, sn);
#pragma unroll
      for (int jj = 0; jj < HG; ++jj) {
        const int h = h0 + jj;
        vec16 y1, y2;
        rotate_pairs<DTYPE>(a[jj], b[jj], c, sn, y1, y2);
        if (ok && h < n_heads) {
          char* d = (h < Hq ? q_out + h * qo_hs_b + t * qo_ts_b : k_out + (h - Hq) * ko_hs_b + row * ko_ts_b) +
                    col * 16;
          st16(d, y1);
          st16(d + HALF_B, y2);
        }
      }
      if (!ok && it == 0) flag_error(err, CKV_DEVICE_ERR_RANGE);
    } else {
      const int h = it / CPR, c = it % CPR;
      const vec16 x = ld16(v_in + h * vi_hs_b + t * vi_ts_b + c * 16);
      const bool ok = p >= INT32_MIN && p <= INT32_MAX && row >= 0 && row < n_out;
      if (ok) st16(v_out + h * vo_hs_b + row * vo_ts_b + c * 16, x);
    }
  }
}

// With a cos/sin table a token needs no shared state, so the work is flattened: one thread per
// (token, item), item = a rotated 16-byte column pair of kRopeHG consecutive q/k heads (one load
// of the column's cos/sin for all of them) or a copied 16-byte chunk of a v row, grid-stride over
// all of them (every thread busy, whatever the head counts), rotation items first.
#ifndef CKV_ROPE_HG
#define CKV_ROPE_HG 2
#endif
constexpr int kRopeHG = CKV_ROPE_HG;  // heads per rotation item (one cos/sin load for all of them)

template <int DTYPE, int D>
__global__ __launch_bounds__(kRopeThreads) void rope_qkv_flat_kernel(
    char* __restrict__ q_out, int64_t qo_hs_b, int64_t qo_ts_b, char* __restrict__ k_out, int64_t ko_hs_b,
    int64_t ko_ts_b, char* __restrict__ v_out, int64_t vo_hs_b, int64_t vo_ts_b, const int64_t* __restrict__ rows,
    int n_out, const char* __restrict__ q_in, int64_t qi_hs_b, int64_t qi_ts_b, const char* __restrict__ k_in,
    int64_t ki_hs_b, int64_t ki_ts_b, const char* __restrict__ v_in, int64_t vi_hs_b, int64_t vi_ts_b,
    const int64_t* __restrict__ pos, const float2* __restrict__ cs_table, int64_t n_table, int n, int Hq, int Hkv,
    int32_t* __restrict__ err) {
  using E = Elem<DTYPE>;
  constexpr int VEC = E::kVec;
  constexpr int HALF = D / 2;
  constexpr int TPR = HALF / VEC;
  constexpr int HALF_B = HALF * E::kBytes;
  constexpr int CPR = D * E::kBytes / 16;
  typedef __attribute__((address_space(1))) const int64_t gi64;
  const int n_heads = Hq + Hkv;
  const unsigned n_rot = (unsigned)((n_heads + kRopeHG - 1) / kRopeHG * TPR);  // rotation items per token
  const unsigned n_cp = v_out != nullptr ? (unsigned)(Hkv * CPR) : 0u;  // copy items per token
  const unsigned rot_total = (unsigned)n * n_rot;
  const unsigned total = rot_total + (unsigned)n * n_cp;  // < 2^31, checked by the host
  // Items are ordered by kind (every rotation item, then every copy item) so that a wavefront
  // runs one kind only.
  for (unsigned idx = blockIdx.x * kRopeThreads + threadIdx.x; idx < total; idx += gridDim.x * kRopeThreads) {
    const bool rot = idx < rot_total;
    const unsigned j = rot ? idx : idx - rot_total;
    const unsigned per = rot ? n_rot : n_cp;
    const int t = (int)(j / per), it = (int)(j - (unsigned)t * per);
    const int64_t p = *(gi64*)(pos + t);
    const int64_t row = rows != nullptr ? *(gi64*)(rows + t) : t;
    if (p < 0 || p >= n_table || row < 0 || row >= n_out) {
      if (it == 0 && rot) flag_error(err, CKV_DEVICE_ERR_RANGE);
      continue;
    }
    if (rot) {
      const int h0 = (it / TPR) * kRopeHG, col = it % TPR;
      vec16 a[kRopeHG], b[kRopeHG];
#pragma unroll
      for (int j = 0; j < kRopeHG; ++j) {  // the heads' loads first, all in flight together
        const int h = h0 + j;
        if (h < n_heads) {
          const char* s = (h < Hq ? q_in + h * qi_hs_b + t * qi_ts_b : k_in + (h - Hq) * ki_hs_b + t * ki_ts_b) +
                          col * 16;
          a[j] = ld16(s);
          b[j] = ld16(s + HALF_B);
        }
      }
      const float2* tr = cs_table + p * HALF + col * VEC;  // VEC pairs = VEC/2 16-byte loads
      float c[VEC], sn[VEC];
#pragma unroll
      for (int e = 0; e < VEC; e += 2) {
        const vec16 w = ld16(tr + e);
        c[e] = __uint_as_float(w[0]);
        sn[e] = __uint_as_float(w[1]);
        c[e + 1] = __uint_as_float(w[2]);
        sn[e + 1] = __uint_as_float(w[3]);
      }
#pragma unroll
      for (int j = 0; j < kRopeHG; ++j) {
        const int h = h0 + j;
        if (h < n_heads) {
          char* d = (h < Hq ? q_out + h * qo_hs_b + t * qo_ts_b : k_out + (h - Hq) * ko_hs_b + row * ko_ts_b) +
                    col * 16;
          vec16 y1, y2;
          rotate_pairs<DTYPE>(a[j], b[j], c, sn, y1, y2);
          st16(d, y1);
          st16(d + HALF_B, y2);
        }
      }
    } else {
      const int h = it / CPR, c = it % CPR;
      st16(v_out + h * vo_hs_b + row * vo_ts_b + c * 16, ld16(v_in + h * vi_hs_b + t * vi_ts_b + c * 16));
    }
  }
}

template <int DTYPE, int D>
static void launch_rope(int n, hipStream_t st, char* qo, int64_t qo_hs, int64_t qo_ts, char* ko, int64_t ko_hs,
                        int64_t ko_ts, char* vo, int64_t vo_hs, int64_t vo_ts, const int64_t* rows, int n_out,
                        const char* qi, int64_t qi_hs, int64_t qi_ts, const char* ki, int64_t ki_hs, int64_t ki_ts,
                        const char* vi, int64_t vi_hs, int64_t vi_ts, const int64_t* pos, const float2* tab,
                        int64_t n_tab, int Hq, int Hkv, double theta, int32_t* err) {
  if (tab != nullptr) {
    using E = Elem<DTYPE>;
    const int64_t per_tok = (int64_t)(Hq + Hkv + kRopeHG - 1) / kRopeHG * (D / 2 / E::kVec) +
                            (vo != nullptr ? Hkv * (D * E::kBytes / 16) : 0);
    const int64_t blocks = std::min<int64_t>((n * per_tok + kRopeThreads - 1) / kRopeThreads, 1 << 20);
    hipLaunchKernelGGL((rope_qkv_flat_kernel<DTYPE, D>), dim3((unsigned)blocks), dim3(kRopeThreads), 0, st, qo, qo_hs,
                       qo_ts, ko, ko_hs, ko_ts, vo, vo_hs, vo_ts, rows, n_out, qi, qi_hs, qi_ts, ki, ki_hs, ki_ts, vi,
                       vi_hs, vi_ts, pos, tab, n_tab, n, Hq, Hkv, err);
    return;
  }
  const InvFreq& inv = host_inv_freq(D, theta);
  if constexpr (D <= 2 * kWave) {
    if (Hq == 0 && vo != nullptr) {
      constexpr int TPR = D / 2 / Elem<DTYPE>::kVec;
      const int items = 2 * Hkv * TPR;
      const int shape = items == kWave ? kKvFull : items < kWave ? kKvOne : kKvLoop;
      const int per_wg = kRopeKvThreads / kWave * (shape == kKvLoop ? 1 : kKvTpw);
      const dim3 grid((unsigned)((n + per_wg - 1) / per_wg));
      const int rm = rows == nullptr ? kRowToken : rows == pos ? kRowPos : kRowIndexed;
      auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(kRopeKvThreads), 0, st, n, Hkv, pos, ki, vi, ki_hs, ki_ts, vi_hs, vi_ts, ko,
                           vo, ko_hs, ko_ts, vo_hs, vo_ts, rows, n_out, err, inv);
      };
#define CKV_KV(S, R) \
  if (shape == S && rm == R) go(rope_kv_kernel<DTYPE, D, S, R, S == kKvLoop ? 1 : kKvTpw>);
      CKV_KV(kKvFull, kRowToken) CKV_KV(kKvFull, kRowPos) CKV_KV(kKvFull, kRowIndexed)
      CKV_KV(kKvOne, kRowToken) CKV_KV(kKvOne, kRowPos) CKV_KV(kKvOne, kRowIndexed)
      CKV_KV(kKvLoop, kRowToken) CKV_KV(kKvLoop, kRowPos) CKV_KV(kKvLoop, kRowIndexed)
#undef CKV_KV
      return;
    }
  }
  if (Hq == 0) {
    constexpr int TW = D / 2 >= kWave ? 1 : kWave / (D / 2);
    const int per_wg = (kRopeThreads / kWave) * TW;
    hipLaunchKernelGGL((rope_wave_kernel<DTYPE, D>), dim3((unsigned)((n + per_wg - 1) / per_wg)), dim3(kRopeThreads),
                       0, st, qo, qo_hs, qo_ts, ko, ko_hs, ko_ts, vo, vo_hs, vo_ts, rows, n_out, qi, qi_hs, qi_ts, ki,
                       ki_hs, ki_ts, vi, vi_hs, vi_ts, pos, inv, n, Hq, Hkv, err);
    return;
  }
  using E = Elem<DTYPE>;
  const int64_t per_tok = (int64_t)(Hq + Hkv + kRopeFreeHG - 1) / kRopeFreeHG * (D / 2 / E::kVec) +
                          (vo != nullptr ? Hkv * (D * E::kBytes / 16) : 0);
  const int64_t blocks = std::min<int64_t>((n * per_tok + kRopeThreads - 1) / kRopeThreads, 1 << 20);
  hipLaunchKernelGGL((rope_free_kernel<DTYPE, D>), dim3((unsigned)blocks), dim3(kRopeThreads), 0, st, qo, qo_hs, qo_ts,
                     ko, ko_hs, ko_ts, vo, vo_hs, vo_ts, rows, n_out, qi, qi_hs, qi_ts, ki, ki_hs, ki_ts, vi, vi_hs,
                     vi_ts, pos, inv, n, Hq, Hkv, err);
}

typedef void (*RopeLaunch)(int, hipStream_t, char*, int64_t, int64_t, char*, int64_t, int64_t, char*, int64_t,
                           int64_t, const int64_t*, int, const char*, int64_t, int64_t, const char*, int64_t, int64_t,
                           const char*, int64_t, int64_t, const int64_t*, const float2*, int64_t, int, int, double,
                           int32_t*);

static RopeLaunch pick_rope(int dtype, int head_dim) {
#define CKV_CASE(DT, HD) \
  if (dtype == DT && head_dim == HD) return &launch_rope<DT, HD>;
  CKV_CASE(CKV_DTYPE_BF16, 64)
  CKV_CASE(CKV_DTYPE_BF16, 128)
  CKV_CASE(CKV_DTYPE_BF16, 256)
  CKV_CASE(CKV_DTYPE_F32, 64)
  CKV_CASE(CKV_DTYPE_F32, 128)
  CKV_CASE(CKV_DTYPE_F32, 256)
#undef CKV_CASE
  return nullptr;
}

// table[p][i] = (cos, sin) of the fp32 angle fl32(fl32(p) * inv_freq_i), correctly rounded.
__global__ void rope_table_kernel(float2* __restrict__ tab, int64_t n_pos, int head_dim, const InvFreq inv) {
  const int half = head_dim / 2;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n_pos * half) tab[i] = shift_cos_sin(inv.v[i % half], (int)(i / half));
}

}  // namespace ckv

extern "C" int32_t ckv_rope_table(void* table, int64_t n_positions, int32_t head_dim, double theta, void* stream) {
  using namespace ckv;
  if (table == nullptr || n_positions < 0 || head_dim <= 0 || (head_dim & 1) || head_dim > 2 * kMaxHalf ||
      !(theta > 0.0))
    return CKV_ERR_INVALID_ARGUMENT;
  if (n_positions > 0x7fffffff) return CKV_ERR_TOO_LARGE;
  const int64_t total = n_positions * (head_dim / 2);
  if (total == 0) return CKV_OK;
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (float2*)table, n_positions, (int)head_dim, host_inv_freq(head_dim, theta));
  CKV_RETURN_IF_LAUNCH_FAILED();
  return CKV_OK;
}

extern "C" int32_t ckv_rope_qkv(void* q_out, int64_t qo_head_stride, int64_t qo_token_stride, void* k_out,
                                int64_t ko_head_stride, int64_t ko_token_stride, void* v_out, int64_t vo_head_stride,
                                int64_t vo_token_stride, const int64_t* rows, int32_t n_out_rows, const void* q_in,
                                int64_t qi_head_stride, int64_t qi_token_stride, const void* k_in,
                                int64_t ki_head_stride, int64_t ki_token_stride, const void* v_in,
                                int64_t vi_head_stride, int64_t vi_token_stride, const int64_t* positions,
                                const void* cs_table, int64_t n_table, int32_t n_tokens, int32_t n_q_heads,
                                int32_t n_kv_heads, int32_t head_dim, int32_t dtype, double theta, int32_t* err,
                                void* stream) {
  using namespace ckv;
  RopeLaunch fn = pick_rope(dtype, head_dim);
  if (fn == nullptr || k_out == nullptr || k_in == nullptr || positions == nullptr ||
      (v_out == nullptr) != (v_in == nullptr) || (n_q_heads > 0 && (q_out == nullptr || q_in == nullptr)))
    return CKV_ERR_INVALID_ARGUMENT;
  if (n_tokens < 0 || n_q_heads < 0 || n_kv_heads <= 0 || n_out_rows < 0 || !(theta > 0.0))
    return CKV_ERR_INVALID_ARGUMENT;
  if (rows == nullptr && n_out_rows < n_tokens) return CKV_ERR_OUT_OF_RANGE;
  if (cs_table != nullptr && (n_table < 0 || (uintptr_t)cs_table % 16)) return CKV_ERR_INVALID_ARGUMENT;
  if ((int64_t)n_tokens * ((n_q_heads + n_kv_heads) * 64 + n_kv_heads * 64) >= (1ll << 31))
    return CKV_ERR_TOO_LARGE;  // the flattened (token, item) index stays below 2^31
  const int64_t eb = dtype == CKV_DTYPE_BF16 ? 2 : 4;
  const int64_t strides[] = {qo_head_stride, qo_token_stride, ko_head_stride, ko_token_stride, vo_head_stride,
                             vo_token_stride, qi_head_stride, qi_token_stride, ki_head_stride, ki_token_stride,
                             vi_head_stride, vi_token_stride};
  for (int64_t s : strides)
    if ((s * eb) % 16) return CKV_ERR_INVALID_ARGUMENT;  // every row starts on a 16-byte boundary
  if (((uintptr_t)q_out | (uintptr_t)q_in | (uintptr_t)k_out | (uintptr_t)k_in | (uintptr_t)v_out | (uintptr_t)v_in) %
      16)
    return CKV_ERR_INVALID_ARGUMENT;
  if (n_tokens == 0) return CKV_OK;
  if (n_tokens > 0x7fffffff) return CKV_ERR_TOO_LARGE;
  fn(n_tokens, (hipStream_t)stream, (char*)q_out, qo_head_stride * eb, qo_token_stride * eb, (char*)k_out,
     ko_head_stride * eb, ko_token_stride * eb, (char*)v_out, vo_head_stride * eb, vo_token_stride * eb, rows,
     n_out_rows, (const char*)q_in, qi_head_stride * eb, qi_token_stride * eb, (const char*)k_in,
     ki_head_stride * eb, ki_token_stride * eb, (const char*)v_in, vi_head_stride * eb, vi_token_stride * eb,
     positions, (const float2*)cs_table, n_table, n_q_heads, n_kv_heads, theta, err);
  CKV_RETURN_IF_LAUNCH_FAILED();
  return CKV_OK;
}
