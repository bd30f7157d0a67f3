// Layer-1 KV repair in one call (ckv_layer1_repair): layer 1's base cache, the fresh-vs-cached
// deviation, the per-chunk relative deviation and escalation, the pooled top-k with forced sinks,
// the compaction of the new active set and the scatter of the kept rows, as three launches:
//   1. layer1_gather_deviation_kernel: every position's rows (the chunk's row re-rotated by the
//      placement's shift, the fresh row), the cached row written into the cache, the deviation,
//      and the candidates counted into the selection's top-digit histogram (top_bin: 4096 bins
//      of 1/64 octave of deviation);
//   2. the selection (select_common.hpp) in one workgroup, its threshold's bin read off that
//      histogram, so only the candidates of one bin are ranked;
//   3. the kept rows scattered from the fresh rows, their count read on the device.
// Nothing is read back on the host.
//
// Reference semantics (src/chunkkv/engine/torch_engine.py):
//   base_kv(1)          :96-103   zero-filled K/V, each placement's chunk rows with keys
//                                 re-rotated by delta (shift_keys :56-59, _rotate :46-51)
//   deviation           :117-124  diff = sum (k - K)^2 + sum (v - V)^2, norm = sum k^2 + sum v^2
//   rel / escalation    :125-142  per non-exact placement, budget = sum int(round(ratio * len))
//   pooled top-k, sinks :143-147  the budget largest deviations among pool & ~keep
//   compaction          :148-153  keep_abs = keep.nonzero(), sel = local[keep_abs]
//   scatter             :155-156  K[:, :, keep_abs] = k[:, :, sel], V likewise
// The outputs are bit-identical to ckv_rerope_gather_layers (this layer, every cached row),
// ckv_deviation, ckv_select and ckv_scatter_kept_rows issued in that order: the same rotation,
// summation order and ranking (larger deviation first, then lower position; NaN last).
//
// Design of the first launch (gfx950): a wavefront owns T consecutive positions and lane l the
// 16-byte vector l of each of a position's four rows (fresh k, fresh v, cached K, cached V): the
// deviation's summation contract maps vector q to lane q, so the sums need no data movement. A
// lane gets its rotation partner's vector (l ^ (vectors per row / 2)) by a lane exchange, and the
// (cos, sin) of its frequencies from lanes that evaluate one frequency each. Many small
// workgroups keep every CU busy with loads in flight (the launch is bound by HBM latency and
// bandwidth); a workgroup adds each distinct histogram bin of its positions' candidates with one
// atomic.
#include <algorithm>
#include <mutex>

#include "ckv_common.hpp"
#include "launch.hpp"
#include "scatter_common.hpp"
#include "select_slices.hpp"

namespace ckv {

constexpr int kL1Threads = 256;
constexpr int kL1Waves = kL1Threads / kWave;
// Positions per wavefront. One: in the 8k request step 0.262 ms against 0.264 ms with two and
// 0.266 ms with four (more wavefronts, each with fewer loads in flight, overlap the pass's
// dependent load chain better).
#ifndef CKV_L1_T
#define CKV_L1_T 1
#endif
constexpr int kL1T = CKV_L1_T;
constexpr int kL1MaxSegs = 64 * 60;  // segment search: 64 samples, then a window of stride + T

// per-position class bits
constexpr uint32_t kCValid = 1u, kCCached = 2u, kCNoLocal = 16u, kCSink = 32u, kCPooled = 128u;

struct L1Args {
  char* dk;  // layer cache (H, N, D), head stride d_hs_b bytes
  char* dv;
  int64_t d_hs_b;
  const uint64_t* tab;  // [chunk][n_layers][2] K/V base addresses
  int tab_chunks, n_layers, layer;
  const ckv_segment* segs;  // cached runs, sorted by dst_start, disjoint
  int n_segs;
  const char* kf;  // fresh k/v rows, strides in bytes
  int64_t kf_hs_b, kf_ts_b;
  const char* vf;
  int64_t vf_hs_b, vf_ts_b;
  int n_fresh;
  const uint8_t* flags;
  const int32_t* local;
  int n_tokens, n_heads, head_dim;
  int vpr_log2;  // log2(16-byte vectors per row)
  float* diff;
  float* norm;
  uint32_t* hist;  // NULL: no histogram (the selection runs its full passes)
  int32_t* zero_word;  // NULL, or a word the launch sets to 0 (a count the next launch adds to)
  int32_t* err;
};

// cos/sin of one fp32 angle per lane, each the correctly rounded fp32 value (angle_cos_sin):
// the short reduction inline, the library sincos out of line for |angle| >= 2^31, so that its
// registers do not count against the kernel's.
__device__ __attribute__((noinline)) float2 library_cos_sin(float ang) {
  double sd, cd;
  sincos((double)ang, &sd, &cd);
  return make_float2((float)cd, (float)sd);
}
__device__ __forceinline__ float2 lane_cos_sin(float ang) {
  float c, s;
  if (!cos_sin_fast(ang, c, s)) return library_cos_sin(ang);
  return make_float2(c, s);
}

// ---- one wavefront's positions: rows, rotation, deviation ------------------------------------

template <int DTYPE, int T>
struct WaveRows {
  vec16 kf[T], vf[T], kc[T], vc[T];  // fresh k, fresh v, cached K (re-rotated, rounded), cached V
};

// Loads the rows of positions pb .. pb + T - 1 (this wavefront's), re-rotates the cached keys and
// computes the deviations. cls gets kCValid / kCCached / kCNoLocal; diff and norm are 0 at
// positions without a fresh row.
// FULL: every lane holds a vector of every row (n_heads x 16-byte vectors per row == 64).
template <int DTYPE, int T, bool FULL>
__device__ __forceinline__ void wave_rows(const L1Args& a, const InvFreq& inv, int pb, WaveRows<DTYPE, T>& r,
                                          uint32_t (&cls)[T], float (&dv)[T], float (&nv)[T], int (&li)[T]) {
  using E = Elem<DTYPE>;
  constexpr int VEC = E::kVec;
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const int vpr = 1 << a.vpr_log2;
  const int64_t rowb = (int64_t)vpr * 16;
  const bool lane_on = FULL || lane < (a.n_heads << a.vpr_log2);
  const int h = lane >> a.vpr_log2, col = lane & (vpr - 1);
  const int64_t colb = (int64_t)col * 16;
  const int N = a.n_tokens;

  // 1. every first-level load at once, unconditionally: indices are clamped into range and the
  // results masked where they are used. (A load behind a condition made the compiler wait for it
  // before the next one went out: flags, local indices, segments, inverse frequencies and the
  // chunk addresses were eight memory round trips in a row.)
  const int half = a.head_dim >> 1;
  const float my_inv = inv.v[lane & (half - 1)];
  uint32_t fl[T];
  int lraw[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int pc = min(pb + t, N - 1);  // N >= 1
    fl[t] = a.flags[pc];
    lraw[t] = a.local[pc];
  }
  const int n_segs = a.n_segs;
  const int stride = (n_segs + kWave - 1) / kWave;
  int st1 = 0x7fffffff;
  if (n_segs > kWave) {  // uniform: 64 samples first, then the window that holds the positions
    const int si = lane * stride;
    st1 = a.segs[min(si, n_segs - 1)].dst_start;
    st1 = si < n_segs ? st1 : 0x7fffffff;
  }

  // 2. the segment records around the positions (the chain to the cached rows: record, chunk
  // address, row) go out before the fresh rows: vector loads complete in issue order, so a
  // record loaded after the fresh rows could not be used before they had arrived
  int sbase = 0, scount = n_segs;
  if (n_segs > kWave) {
    const uint64_t m = __ballot(st1 <= pb);
    const int bk = m ? 63 - __builtin_clzll(m) : 0;
    sbase = bk * stride;
    scount = min(stride + T, n_segs - sbase);
  }
  // unconditional (segs is readable even without segments: the host passes the workspace), so
  // no branch merges paths with different loads in flight
  ckv_segment sd = a.segs[sbase + max(min(lane, scount - 1), 0)];

  // 3. the fresh rows: lanes past the rows and positions without a fresh row load a valid row
  // and drop it where it is used
  const int hc = FULL ? h : min(h, a.n_heads - 1);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int p = pb + t;
    const bool okl = p < N && lraw[t] >= 0 && lraw[t] < a.n_fresh;
    li[t] = okl ? lraw[t] : -1;
    r.kc[t] = r.vc[t] = vec16{0u, 0u, 0u, 0u};
    const int64_t lc = okl ? lraw[t] : 0;  // kf/vf are readable with n_fresh == 0: the workspace
    r.kf[t] = ld16_stream(a.kf + hc * a.kf_hs_b + lc * a.kf_ts_b + colb);  // read once: non-temporal
    r.vf[t] = ld16_stream(a.vf + hc * a.vf_hs_b + lc * a.vf_ts_b + colb);
  }

  // 4. each position's segment (the last with dst_start <= p) and its chunk's base addresses
  sd.dst_start = lane < scount ? sd.dst_start : 0x7fffffff;
  int delta[T];
  bool have[T];
  const char* kb[T];
  const char* vb[T];
  int64_t soff[T];
  bool bad = false;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int p = pb + t;
    const uint32_t f = __builtin_amdgcn_readfirstlane(fl[t]) & (p < N ? 0xffu : 0u);  // every lane loaded the same byte
    const uint64_t m = __ballot(lane < scount && sd.dst_start <= p);
    const int L = m ? 63 - __builtin_clzll(m) : 0;
    const int dst = __builtin_amdgcn_readlane(sd.dst_start, L);
    const int n = __builtin_amdgcn_readlane(sd.n_tokens, L);
    const int ch = __builtin_amdgcn_readlane(sd.chunk, L);
    const int ss = __builtin_amdgcn_readlane(sd.src_start, L);
    const int sl = __builtin_amdgcn_readlane(sd.src_len, L);
    delta[t] = __builtin_amdgcn_readlane(sd.delta, L);
    const bool cached = p < N && (f & CKV_POS_CACHED);
    const bool found = m != 0ull && p < dst + n;
    const bool seg_ok = found && dst >= 0 && ss >= 0 && ch >= 0 && ch < a.tab_chunks && (int64_t)dst + n <= N &&
                        (int64_t)ss + n <= sl;
    bad = bad || (cached && !seg_ok);
    have[t] = cached && seg_ok;
    soff[t] = (int64_t)hc * sl * rowb + (int64_t)(ss + (p - dst)) * rowb + colb;
    // unconditional (entry 0 when there is no row to load; the host passes a readable table),
    // so both positions' address loads are in flight together
    const int64_t ti = have[t] ? ((int64_t)ch * a.n_layers + a.layer) * 2 : 0;
    kb[t] = reinterpret_cast<const char*>(a.tab[ti]);
    vb[t] = reinterpret_cast<const char*>(a.tab[ti + 1]);
    bad = bad || (p < N && lraw[t] >= a.n_fresh);
    cls[t] = (p < N ? kCValid : 0u) | (cached ? kCCached : 0u) | (li[t] < 0 ? kCNoLocal : 0u) |
             ((f & CKV_POS_SINK) ? kCSink : 0u) | ((f & CKV_POS_POOLED) ? kCPooled : 0u);
  }
  if (bad && lane == 0) flag_error(a.err, CKV_DEVICE_ERR_RANGE);

  // 5. the chunk's K/V at the segment's source row; cos/sin of each position's shift while they
  // arrive: lane f evaluates frequency f (mod D/2) once per distinct shift, the rotation fetches
  // its column's VEC frequencies from the evaluating lanes
#pragma unroll
  for (int t = 0; t < T; ++t) {
    if (have[t]) {  // uniform
      r.kc[t] = ld16_stream(kb[t] + soff[t]);
      r.vc[t] = ld16_stream(vb[t] + soff[t]);
    }
  }
  float cv[T], sv[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    cv[t] = 1.0f;
    sv[t] = 0.0f;
    if (!have[t] || delta[t] == 0) continue;  // uniform; delta 0 copies the row bit for bit
    if (t > 0 && have[t - 1] && delta[t - 1] == delta[t]) {
      cv[t] = cv[t - 1];
      sv[t] = sv[t - 1];
      continue;
    }
    const float2 cs = lane_cos_sin((float)delta[t] * my_inv);
    cv[t] = cs.x;
    sv[t] = cs.y;
  }

  // 6. re-rotate the cached keys: the partner half comes from lane l ^ (vpr / 2). With u the
  // lane's own elements and w its partner's (same frequencies, other half), both halves are
  // y = fl(u c) + fl(w s'), s' = -s in the first half: the first half's x1 c - x2 s and the second
  // half's x1 s + x2 c with the same roundings (negation is exact, addition commutes), with no
  // per-lane branch; every cos/sin is fetched before the products use them.
  const int half_v = vpr >> 1;
  const uint32_t sgn = col < half_v ? 0x80000000u : 0u;
  const int f0 = (col & (half_v - 1)) * VEC;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    if (!have[t] || delta[t] == 0) continue;  // uniform
    const vec16 mine = r.kc[t];
    vec16 other;
    other.x = __shfl_xor(mine.x, half_v);
    other.y = __shfl_xor(mine.y, half_v);
    other.z = __shfl_xor(mine.z, half_v);
    other.w = __shfl_xor(mine.w, half_v);
    float c[VEC], s[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      c[e] = __shfl(cv[t], f0 + e);
      s[e] = __uint_as_float(__float_as_uint(__shfl(sv[t], f0 + e)) ^ sgn);
    }
    float u[VEC], w[VEC], y[VEC];
    E::unpack(mine, u);
    E::unpack(other, w);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float p1 = u[e] * c[e];
      const float p2 = w[e] * s[e];
      y[e] = p1 + p2;
    }
    if (lane_on) r.kc[t] = E::pack(y);
  }

  // 7. deviations in the contract's order: lane q adds its vector's elements in ascending order,
  // then the xor butterfly; diff = Sk + Sv, norm = Nk + Nv. The differences are rounded to the
  // element type two at a time (NaN payloads unspecified), so a NaN result is canonicalized.
#pragma unroll
  for (int t = 0; t < T; ++t) {
    float kx[VEC], vx[VEC], kcx[VEC], vcx[VEC];
    const vec16 zero = {0u, 0u, 0u, 0u};  // lanes past the rows add nothing
    E::unpack(lane_on ? r.kf[t] : zero, kx);
    E::unpack(lane_on ? r.vf[t] : zero, vx);
    E::unpack(lane_on ? r.kc[t] : zero, kcx);
    E::unpack(lane_on ? r.vc[t] : zero, vcx);
    float dk[VEC], dw[VEC];
#pragma unroll
    for (int e = 0; e < VEC; e += 2) {
      E::round_trip2(kx[e] - kcx[e], kx[e + 1] - kcx[e + 1], dk[e], dk[e + 1]);
      E::round_trip2(vx[e] - vcx[e], vx[e + 1] - vcx[e + 1], dw[e], dw[e + 1]);
    }
    float sk = 0.0f, sv = 0.0f, nk = 0.0f, nw = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      sk = sk + dk[e] * dk[e];
      sv = sv + dw[e] * dw[e];
      nk = nk + kx[e] * kx[e];
      nw = nw + vx[e] * vx[e];
    }
    const float x = wave_butterfly_sum(sk);
    const float y = wave_butterfly_sum(sv);
    const float z = wave_butterfly_sum(nk);
    const float w = wave_butterfly_sum(nw);
    dv[t] = li[t] < 0 ? 0.0f : canonical_nan(x + y);
    nv[t] = li[t] < 0 ? 0.0f : canonical_nan(z + w);
  }
}


// Launch 1: the positions of kL1Waves wavefronts (P consecutive ones) per workgroup. Cached rows
// go into the cache (sinks excepted: always kept, the scatter writes them), deviations out, and
// the positions flagged cached, pooled and not sink (the candidates when no chunk escalates)
// counted by their key's top_bin, one atomic per distinct bin of the workgroup.
// The pointers and sizes the first loads use lead the argument list: the library preloads the
// first 16 argument dwords into SGPRs, but only up to the first argument passed by reference
// (the L1Args struct), and every other argument takes a scalar load at wave start.
template <int DTYPE, int T, bool FULL>
__global__ __launch_bounds__(kL1Threads) void layer1_gather_deviation_kernel(
    const uint8_t* flags, const int32_t* local, const ckv_segment* segs, const uint64_t* tab, int n_tokens, int n_segs,
    const char* kf, const char* vf, L1Args a, const InvFreq inv) {
  a.flags = flags;
  a.local = local;
  a.segs = segs;
  a.tab = tab;
  a.n_tokens = n_tokens;
  a.n_segs = n_segs;
  a.kf = kf;
  a.vf = vf;
  constexpr int P = kL1Waves * T;
  __shared__ uint32_t s_bin[P];
  const int tid = (int)threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pb = (int)blockIdx.x * P + wave * T;
  const int N = a.n_tokens;
  WaveRows<DTYPE, T> r;
  uint32_t cls[T];
  float dv[T], nv[T];
  int li[T];
  wave_rows<DTYPE, T, FULL>(a, inv, pb, r, cls, dv, nv, li);

  const int vpr = 1 << a.vpr_log2;
  const int64_t rowb = (int64_t)vpr * 16;
  const bool lane_on = FULL || lane < (a.n_heads << a.vpr_log2);
  const int64_t hoff = (int64_t)(lane >> a.vpr_log2) * a.d_hs_b + (int64_t)(lane & (vpr - 1)) * 16;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int p = pb + t;
    if ((cls[t] & kCCached) && !(cls[t] & kCSink) && lane_on) {  // cls: p < N
      const int64_t off = hoff + (int64_t)p * rowb;
      st16_stream(a.dk + off, r.kc[t]);  // non-temporal, as every cache-row writer here
      st16_stream(a.dv + off, r.vc[t]);
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int p = pb + t;
      if (p < N) {
        a.diff[p] = dv[t];
        a.norm[p] = nv[t];
      }
      const bool cand = (cls[t] & kCCached) && (cls[t] & kCPooled) && !(cls[t] & kCSink);
      s_bin[wave * T + t] = cand ? top_bin(dev_key(dv[t])) : ~0u;
    }
  }
  if (a.zero_word != nullptr && blockIdx.x == 0 && tid == 0) *a.zero_word = 0;
  if (a.hist == nullptr) return;  // uniform
  __syncthreads();
  if (wave == 0) {
    const uint32_t bin = lane < P ? s_bin[lane] : ~0u;
    uint32_t cnt = 0u;
    bool first = true;
#pragma unroll
    for (int j = 0; j < P; ++j) {
      const uint32_t bj = s_bin[j];
      cnt += bj == bin ? 1u : 0u;
      first = first && !(j < lane && bj == bin);
    }
    if (bin != ~0u && first) atomicAdd(hist_copy(a.hist, hist_copies_l1(a.n_tokens)) + bin, cnt);
  }
}

}  // namespace ckv

namespace ckv {

// The dropped-row gather that ckv_layer1_repair_gather carries in its last launch: the K/V slabs
// (layer l's cache at l * layer_stride elements), the layers and the segments' longest run.
struct GatherTail {
  void* k_slab;
  void* v_slab;
  int64_t layer_stride;
  int32_t begin, end, max_seg_tokens;
};

static int32_t layer1_repair_impl(
    void* dst_k, void* dst_v, int64_t dst_head_stride, const uint64_t* src_tab, int32_t n_tab_chunks,
    int32_t n_layers, int32_t layer, const ckv_segment* segs, int32_t n_segs, const void* k_fresh,
    int64_t kf_head_stride, int64_t kf_token_stride, const void* v_fresh, int64_t vf_head_stride,
    int64_t vf_token_stride, int32_t n_fresh, const uint8_t* pos_flags, const int32_t* local, int32_t n_tokens,
    int32_t n_heads, int32_t head_dim, int32_t dtype, double theta, const ckv_chunk_span* chunks, int32_t n_chunks,
    int32_t has_threshold, double escalate_threshold, float* diff, float* norm, int64_t* keep_abs,
    int64_t* keep_local, int32_t* keep_rank, float* rel_dev, uint8_t* escalated, int32_t* counts, void* workspace,
    int64_t workspace_bytes, int32_t* err, void* stream, const GatherTail* tail) {
  if (dtype != CKV_DTYPE_BF16 && dtype != CKV_DTYPE_F32) return CKV_ERR_INVALID_ARGUMENT;
  const int eb = dtype == CKV_DTYPE_BF16 ? 2 : 4;
  if (n_heads <= 0 || head_dim <= 0 || n_tokens < 0 || n_fresh < 0 || n_segs < 0 || n_chunks < 0 ||
      n_tab_chunks < 0 || n_layers <= 0 || layer < 0 || layer >= n_layers || !(theta > 0.0))
    return CKV_ERR_INVALID_ARGUMENT;
  const int rowb = head_dim * eb;
  if (head_dim > 128 || rowb % 32 != 0 || (rowb & (rowb - 1)) != 0) return CKV_ERR_INVALID_ARGUMENT;
  const int vpr = rowb / 16;
  int vpr_log2 = 0;
  while ((1 << vpr_log2) < vpr) ++vpr_log2;
  if ((int64_t)n_heads * vpr > kWave) return CKV_ERR_TOO_LARGE;  // one 16-byte vector per lane and row
  if (dst_k == nullptr || dst_v == nullptr || pos_flags == nullptr || local == nullptr || diff == nullptr ||
      norm == nullptr || keep_abs == nullptr || keep_local == nullptr || counts == nullptr || workspace == nullptr ||
      (n_segs > 0 && (segs == nullptr || src_tab == nullptr)) ||
      (n_fresh > 0 && (k_fresh == nullptr || v_fresh == nullptr)) ||
      (n_chunks > 0 && (chunks == nullptr || rel_dev == nullptr || escalated == nullptr)))
    return CKV_ERR_INVALID_ARGUMENT;
  if (workspace_bytes < CKV_LAYER1_REPAIR_WORKSPACE_BYTES || (uintptr_t)workspace % 16) return CKV_ERR_INVALID_ARGUMENT;
  const int64_t strides[] = {dst_head_stride, kf_head_stride, kf_token_stride, vf_head_stride, vf_token_stride};
  for (int64_t s : strides)
    if ((s * eb) % 16) return CKV_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)dst_k | (uintptr_t)dst_v | (uintptr_t)k_fresh | (uintptr_t)v_fresh) % 16)
    return CKV_ERR_INVALID_ARGUMENT;
  if (dst_head_stride < (int64_t)n_tokens * head_dim) return CKV_ERR_OUT_OF_RANGE;
  if (n_tokens > CKV_SELECT_MAX_TOKENS || n_segs > kL1MaxSegs) return CKV_ERR_TOO_LARGE;
  hipStream_t st = (hipStream_t)stream;
  const SelectArgs sel{diff,          norm,     pos_flags,  local,      (int)n_tokens,
                       chunks,        (int)n_chunks,        (int)(has_threshold != 0),
                       escalate_threshold, keep_abs, keep_local, keep_rank, rel_dev,
                       escalated,     counts,   hist_copies_l1((int)n_tokens)};
  if (tail != nullptr && (keep_rank == nullptr || tail->begin < 0 || tail->end < tail->begin || tail->end > n_layers ||
                          tail->max_seg_tokens < 0 || (tail->begin < tail->end && (layer >= tail->begin &&
                                                                                  layer < tail->end))))
    return CKV_ERR_INVALID_ARGUMENT;
  if (n_tokens == 0) return select_launch(sel, nullptr, st);  // nothing to repair: counts and span stats

  // Without a threshold the selection and the kept rows' scatter are one launch of many
  // workgroups (select_slices.hpp) started from the histogram; with one, the single-workgroup
  // selection (the register-resident form takes the histogram; above it, the L2 form counts
  // itself) and the scatter. With a dropped-row gather to carry (tail) and no threshold, up to
  // 16384 positions: the single-workgroup selection with whole layers of the gather beside it
  // (select_gather.hip), then the kept rows with the rest of the gather.
  const bool pre = tail != nullptr && has_threshold == 0 && n_tokens <= kSelRegMax * kSelThreads && n_segs > 0 &&
                   tail->begin < tail->end;
  const bool spread = !pre && has_threshold == 0 && select_slices_fits(n_tokens);
  uint32_t* hist = spread || n_tokens <= kSelRegMax * kSelThreads ? (uint32_t*)workspace : nullptr;
  L1Args args{};
  args.dk = (char*)dst_k;
  args.dv = (char*)dst_v;
  args.d_hs_b = dst_head_stride * eb;
  args.tab = n_tab_chunks > 0 && src_tab != nullptr ? src_tab : (const uint64_t*)workspace;
  args.tab_chunks = args.tab == src_tab ? n_tab_chunks : 0;
  args.n_layers = n_layers;
  args.layer = layer;
  // the first launch loads a segment record and the fresh rows without branching on their
  // counts: with none, it reads the workspace (16 KB, 16-byte aligned) and drops what it read
  args.segs = n_segs > 0 ? segs : (const ckv_segment*)workspace;
  args.n_segs = n_segs;
  const bool fresh = n_fresh > 0;
  args.kf = fresh ? (const char*)k_fresh : (const char*)workspace;
  args.kf_hs_b = fresh ? kf_head_stride * eb : 0;
  args.kf_ts_b = fresh ? kf_token_stride * eb : 0;
  args.vf = fresh ? (const char*)v_fresh : (const char*)workspace;
  args.vf_hs_b = fresh ? vf_head_stride * eb : 0;
  args.vf_ts_b = fresh ? vf_token_stride * eb : 0;
  args.n_fresh = n_fresh;
  args.flags = pos_flags;
  args.local = local;
  args.n_tokens = n_tokens;
  args.n_heads = n_heads;
  args.head_dim = head_dim;
  args.vpr_log2 = vpr_log2;
  args.diff = diff;
  args.norm = norm;
  args.hist = hist;
  args.zero_word = spread ? counts + CKV_COUNT_UNCOMPUTED : nullptr;
  args.err = err;
  const InvFreq& inv = host_inv_freq(head_dim, theta);
  constexpr int P = kL1Waves * kL1T;
  const unsigned blocks = (unsigned)((n_tokens + P - 1) / P);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(kL1Threads), 0, st, args.flags, args.local, args.segs, args.tab,
                       args.n_tokens, args.n_segs, args.kf, args.vf, args, inv);
  };
  const bool full = (int64_t)n_heads * vpr == kWave;  // every lane holds a vector of every row
  if (dtype == CKV_DTYPE_BF16) {
    if (full) go(layer1_gather_deviation_kernel<CKV_DTYPE_BF16, kL1T, true>);
    else go(layer1_gather_deviation_kernel<CKV_DTYPE_BF16, kL1T, false>);
  } else {
    if (full) go(layer1_gather_deviation_kernel<CKV_DTYPE_F32, kL1T, true>);
    else go(layer1_gather_deviation_kernel<CKV_DTYPE_F32, kL1T, false>);
  }
  CKV_RETURN_IF_LAUNCH_FAILED();
  if (tail != nullptr) {
    // the selection (with the first n_pre layers of [begin, end) gathered whole beside it), then
    // one launch: the kept rows of this layer beside the gather of the dropped rows of the other
    // layers (keep_rank >= 0 marks the kept positions)
    int32_t n_pre = 0, rc;
    if (pre) {
      PreGather g{};
      g.dk = (char*)tail->k_slab;
      g.dv = (char*)tail->v_slab;
      g.ls_b = tail->layer_stride * eb;
      g.hs_b = dst_head_stride * eb;
      g.tab = src_tab;
      g.segs = segs;
      g.n_tab_chunks = n_tab_chunks;
      g.n_segs = n_segs;
      g.n_layers = n_layers;
      g.layer_begin = tail->begin;
      g.n_heads = n_heads;
      g.n_tokens = n_tokens;
      g.err = err;
      rc = select_gather_launch(sel, hist, g, tail->end - tail->begin, tail->max_seg_tokens, head_dim, dtype, theta,
                                &n_pre, st);
    } else {
      rc = spread ? select_slices_launch(sel, hist, nullptr, err, st) : select_launch(sel, hist, st);
    }
    if (rc != CKV_OK) return rc;
    const RowScatter kept{(char*)dst_k,   (char*)dst_v,   dst_head_stride * eb,      args.kf,
                          args.kf_hs_b,   args.kf_ts_b,   args.vf,                   args.vf_hs_b,
                          args.vf_ts_b,   keep_abs,       keep_local,                counts + CKV_COUNT_KEEP,
                          (int)n_tokens,  (int)n_fresh,   (int)n_tokens,             (int)n_heads,
                          vpr,            (int64_t)rowb};
    return gather_layers_launch(tail->k_slab, tail->v_slab, tail->layer_stride, dst_head_stride,
                                n_segs > 0 ? src_tab : (const uint64_t*)workspace, n_tab_chunks, n_layers,
                                tail->begin + n_pre, tail->end, n_segs > 0 ? segs : (const ckv_segment*)workspace, n_segs,
                                tail->max_seg_tokens, keep_rank, n_heads, n_tokens, head_dim, dtype, theta, err,
                                stream, &kept);
  }
  if (spread) {
    // with no fresh rows no source row is in range (a kept row then flags the range error)
    const SliceRows rows{(char*)dst_k,          (char*)dst_v,        dst_head_stride * eb,
                         (const char*)args.kf, args.kf_hs_b,        args.kf_ts_b,
                         (const char*)args.vf, args.vf_hs_b,        args.vf_ts_b,
                         (int)n_fresh,         (int)n_heads,        vpr};
    return select_slices_launch(sel, hist, &rows, err, st);
  }
  int32_t rc = select_launch(sel, hist, st);
  if (rc != CKV_OK) return rc;
  // the kept rows from the fresh rows: K[keep_abs[j]] = k[keep_local[j]], j < counts[KEEP]. With
  // no fresh rows no source row is in range (a kept row then flags the range error) and nothing
  // is read: the workspace stands in for k/v.
  return scatter_launch(dst_k, dst_v, dst_head_stride, fresh ? k_fresh : workspace, kf_head_stride, kf_token_stride,
                        fresh ? v_fresh : workspace, vf_head_stride, vf_token_stride, keep_abs, keep_local, n_tokens,
                        n_fresh, n_tokens, n_heads, head_dim, dtype, counts + CKV_COUNT_KEEP, err, stream);
}

}  // namespace ckv

extern "C" int32_t ckv_layer1_repair(
    void* dst_k, void* dst_v, int64_t dst_head_stride, const uint64_t* src_tab, int32_t n_tab_chunks,
    int32_t n_layers, int32_t layer, const ckv_segment* segs, int32_t n_segs, const void* k_fresh,
    int64_t kf_head_stride, int64_t kf_token_stride, const void* v_fresh, int64_t vf_head_stride,
    int64_t vf_token_stride, int32_t n_fresh, const uint8_t* pos_flags, const int32_t* local, int32_t n_tokens,
    int32_t n_heads, int32_t head_dim, int32_t dtype, double theta, const ckv_chunk_span* chunks, int32_t n_chunks,
    int32_t has_threshold, double escalate_threshold, float* diff, float* norm, int64_t* keep_abs,
    int64_t* keep_local, int32_t* keep_rank, float* rel_dev, uint8_t* escalated, int32_t* counts, void* workspace,
    int64_t workspace_bytes, int32_t* err, void* stream) {
  return ckv::layer1_repair_impl(dst_k, dst_v, dst_head_stride, src_tab, n_tab_chunks, n_layers, layer, segs, n_segs,
                                 k_fresh, kf_head_stride, kf_token_stride, v_fresh, vf_head_stride, vf_token_stride,
                                 n_fresh, pos_flags, local, n_tokens, n_heads, head_dim, dtype, theta, chunks, n_chunks,
                                 has_threshold, escalate_threshold, diff, norm, keep_abs, keep_local, keep_rank,
                                 rel_dev, escalated, counts, workspace, workspace_bytes, err, stream, nullptr);
}

extern "C" int32_t ckv_layer1_repair_gather(
    void* k_slab, void* v_slab, int64_t layer_stride, int64_t head_stride, const uint64_t* src_tab,
    int32_t n_tab_chunks, int32_t n_layers, int32_t layer, int32_t gather_begin, int32_t gather_end,
    const ckv_segment* segs, int32_t n_segs, int32_t max_seg_tokens, const void* k_fresh, int64_t kf_head_stride,
    int64_t kf_token_stride, const void* v_fresh, int64_t vf_head_stride, int64_t vf_token_stride, int32_t n_fresh,
    const uint8_t* pos_flags, const int32_t* local, int32_t n_tokens, int32_t n_heads, int32_t head_dim,
    int32_t dtype, double theta, const ckv_chunk_span* chunks, int32_t n_chunks, int32_t has_threshold,
    double escalate_threshold, float* diff, float* norm, int64_t* keep_abs, int64_t* keep_local, int32_t* keep_rank,
    float* rel_dev, uint8_t* escalated, int32_t* counts, void* workspace, int64_t workspace_bytes, int32_t* err,
    void* stream) {
  using namespace ckv;
  if (k_slab == nullptr || v_slab == nullptr || n_layers <= 0 || layer < 0 || layer >= n_layers || head_dim <= 0 ||
      n_heads <= 0 || (dtype != CKV_DTYPE_BF16 && dtype != CKV_DTYPE_F32))
    return CKV_ERR_INVALID_ARGUMENT;
  if (layer_stride < head_stride * n_heads) return CKV_ERR_OUT_OF_RANGE;
  const int64_t eb = dtype == CKV_DTYPE_BF16 ? 2 : 4;
  const GatherTail tail{k_slab, v_slab, layer_stride, gather_begin, gather_end, max_seg_tokens};
  char* dk = (char*)k_slab + (int64_t)layer * layer_stride * eb;
  char* dv = (char*)v_slab + (int64_t)layer * layer_stride * eb;
  return layer1_repair_impl(dk, dv, head_stride, src_tab, n_tab_chunks, n_layers, layer, segs, n_segs, k_fresh,
                            kf_head_stride, kf_token_stride, v_fresh, vf_head_stride, vf_token_stride, n_fresh,
                            pos_flags, local, n_tokens, n_heads, head_dim, dtype, theta, chunks, n_chunks, has_threshold,
                            escalate_threshold, diff, norm, keep_abs, keep_local, keep_rank, rel_dev, escalated,
                            counts, workspace, workspace_bytes, err, stream, &tail);
}
