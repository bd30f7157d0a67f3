// Layer-1 fresh-vs-cached K/V deviation of token positions, one 64-lane wavefront per position:
// the arithmetic shared by ckv_deviation and ckv_deviation_select.
//
// Reference semantics (src/chunkkv/engine/torch_engine.py:117-124):
//   d_act  = ((k - K[:, :, active]).float() ** 2).sum(dim=(0, 1, 3))
//   d_act += ((v - V[:, :, active]).float() ** 2).sum(dim=(0, 1, 3))
//   n_act  = (k.float() ** 2).sum(dim=(0, 1, 3)) + (v.float() ** 2).sum(dim=(0, 1, 3))
//   diff[active] = d_act; norm[active] = n_act   (zeros elsewhere)
// The subtraction happens in the element type (one rounding); squares and sums are fp32.
// K/V rows outside every placement are zero in the reference (base_kv zero-fills them).
//
// Each lane loads 16 bytes of each of the four rows (fresh k, cached K, fresh v, cached V) of
// every one of its tokens before any arithmetic, so a token's H*D elements (1 KiB per tensor at
// H=4, D=128, bf16) arrive in one coalesced pass. 16-byte vector q of a tensor goes to lane
// q mod 64, each lane adds in ascending q from +0, and four fp32 partial sums per lane are
// combined by a xor butterfly: the summation contract the oracle restates bit for bit.
#pragma once

#include "ckv_common.hpp"

namespace ckv {

struct DevArgs {
  const char* kf;  // fresh k rows: head stride kf_hs_b, token stride kf_ts_b (bytes)
  int64_t kf_hs_b, kf_ts_b;
  const char* vf;  // fresh v rows
  int64_t vf_hs_b, vf_ts_b;
  const char* kc;  // cached K, V: (H, N, D), head stride c_hs_b (bytes)
  const char* vc;
  int64_t c_hs_b;
  const uint8_t* flags;
  const int32_t* local;  // row of each position in the fresh tensors, -1 = not computed
  int n_tokens, n_fresh, n_heads, head_dim;
  int32_t* err;
};

// Deviation and norm of positions p_base .. p_base + T - 1, computed by the calling wavefront.
// Every lane returns the totals; positions outside the active set (local < 0) or past n_tokens
// give 0. fl[t] returns the position's flag byte (0 past n_tokens). Requires n_tokens >= 1.
//
// One memory round trip when the active set is every position (local[p] == p: the layer-1 case
// without exact placements): the local indices, the flags, the cached rows at p and the fresh
// rows at row p go out together (indices clamped into range, values dropped where they are
// used), and a position whose local index turns out to be another row loads that row again.
template <int DTYPE, int T>
__device__ __forceinline__ void deviation_wave(const DevArgs& a, int p_base, float (&diff)[T], float (&norm)[T],
                                               uint32_t (&fl)[T]) {
  using E = Elem<DTYPE>;
  constexpr int VEC = E::kVec;
  const int lane = threadIdx.x % kWave;
  const int64_t row_b = (int64_t)a.head_dim * E::kBytes;
  const int vecs_per_row = a.head_dim / VEC;
  const int n_vecs = a.n_heads * vecs_per_row;
  const int N = a.n_tokens;

  // Lane t < T loads position p_base + t's local index and flag byte. The addresses differ per
  // lane, so these are vector loads, which complete in issue order: the row loads below go out
  // right behind them and only the first read of an index waits. (Read as wave-uniform values
  // they became a scalar load and a byte load plus readfirstlane that every row load waited for:
  // one whole memory round trip more per wavefront.)
  const int lp = min(p_base + min(lane, T - 1), N - 1);
  const int j_lane = a.local[lp];
  const uint32_t f_lane = a.flags[lp];
  int jraw[T];
  uint32_t fraw[T];
  float sk[T], sv[T], nk[T], nv[T];
#pragma unroll
  for (int t = 0; t < T; ++t) sk[t] = sv[t] = nk[t] = nv[t] = 0.0f;
  int jj[T];
  bool cached[T], bad = false;
  auto checks = [&]() {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      jraw[t] = __builtin_amdgcn_readlane(j_lane, t);
      fraw[t] = (uint32_t)__builtin_amdgcn_readlane((int)f_lane, t);
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const bool valid = p_base + t < N;
      fl[t] = valid ? fraw[t] : 0u;
      cached[t] = (fl[t] & CKV_POS_CACHED) != 0;
      bad = bad || (valid && jraw[t] >= a.n_fresh);
      jj[t] = valid && jraw[t] >= 0 && jraw[t] < a.n_fresh ? jraw[t] : -1;
    }
  };
  auto accumulate = [&](int t, const vec16& k16, const vec16& v16, const vec16& kc16, const vec16& vc16) {
    float kx[VEC], vx[VEC], kcx[VEC], vcx[VEC];
    E::unpack(k16, kx);
    E::unpack(v16, vx);
    E::unpack(kc16, kcx);
    E::unpack(vc16, vcx);
    // the differences rounded to the element type two at a time (NaN payloads unspecified: a NaN
    // total is canonicalized below)
    float dk[VEC], dv[VEC];
#pragma unroll
    for (int e = 0; e < VEC; e += 2) {
      const float ck0 = cached[t] ? kcx[e] : 0.0f, ck1 = cached[t] ? kcx[e + 1] : 0.0f;  // rows outside
      const float cv0 = cached[t] ? vcx[e] : 0.0f, cv1 = cached[t] ? vcx[e + 1] : 0.0f;  // every placement: 0
      E::round_trip2(kx[e] - ck0, kx[e + 1] - ck1, dk[e], dk[e + 1]);
      E::round_trip2(vx[e] - cv0, vx[e + 1] - cv1, dv[e], dv[e + 1]);
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      sk[t] = sk[t] + dk[e] * dk[e];
      sv[t] = sv[t] + dv[e] * dv[e];
      nk[t] = nk[t] + kx[e] * kx[e];
      nv[t] = nv[t] + vx[e] * vx[e];
    }
  };

  // every row is read once here: non-temporal loads (config 3's deviation 9.2 -> 8.4 us)
  if (a.n_fresh <= 0) {  // uniform: no fresh rows, every position outside the active set
    checks();
  } else if (n_vecs <= kWave) {  // uniform: one 16-byte vector of each row per lane
    const bool lane_on = lane < n_vecs;
    const int q = min(lane, n_vecs - 1);
    const int h = q / vecs_per_row;
    const int64_t cb = (int64_t)(q % vecs_per_row) * 16;
    vec16 k16[T], v16[T], kc16[T], vc16[T];
    int js[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int pc = min(p_base + t, N - 1);
      js[t] = min(pc, a.n_fresh - 1);  // the fresh row when local[p] == p
      const int64_t co = h * a.c_hs_b + (int64_t)pc * row_b + cb;
      kc16[t] = ld16_stream(a.kc + co);
      vc16[t] = ld16_stream(a.vc + co);
      k16[t] = ld16_stream(a.kf + h * a.kf_hs_b + js[t] * a.kf_ts_b + cb);
      v16[t] = ld16_stream(a.vf + h * a.vf_hs_b + js[t] * a.vf_ts_b + cb);
    }
    __builtin_amdgcn_sched_barrier(0);  // the row loads stay ahead of the first index read
    checks();
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if (jj[t] >= 0 && jj[t] != js[t]) {  // uniform: another row after all
        k16[t] = ld16_stream(a.kf + h * a.kf_hs_b + jj[t] * a.kf_ts_b + cb);
        v16[t] = ld16_stream(a.vf + h * a.vf_hs_b + jj[t] * a.vf_ts_b + cb);
      }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if (lane_on && jj[t] >= 0) accumulate(t, k16[t], v16[t], kc16[t], vc16[t]);
    }
  } else {  // several vectors of each row per lane: q = lane, lane + 64, ... ascending
    checks();
    for (int q = lane; q < n_vecs; q += kWave) {
      const int h = q / vecs_per_row;
      const int64_t cb = (int64_t)(q % vecs_per_row) * 16;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        if (jj[t] < 0) continue;  // uniform
        const int64_t co = h * a.c_hs_b + (int64_t)(p_base + t) * row_b + cb;
        accumulate(t, ld16_stream(a.kf + h * a.kf_hs_b + jj[t] * a.kf_ts_b + cb),
                   ld16_stream(a.vf + h * a.vf_hs_b + jj[t] * a.vf_ts_b + cb), ld16_stream(a.kc + co), ld16_stream(a.vc + co));
      }
    }
  }
  if (bad && lane == 0) flag_error(a.err, CKV_DEVICE_ERR_RANGE);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const float x = wave_butterfly_sum(sk[t]);
    const float y = wave_butterfly_sum(sv[t]);
    const float z = wave_butterfly_sum(nk[t]);
    const float w = wave_butterfly_sum(nv[t]);
    diff[t] = jj[t] < 0 ? 0.0f : canonical_nan(x + y);
    norm[t] = jj[t] < 0 ? 0.0f : canonical_nan(z + w);
  }
}

}  // namespace ckv
