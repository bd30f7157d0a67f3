// Layer-1 KV repair in one launch (ckv_layer1_repair): layer 1's base cache, the fresh-vs-cached
// deviation, the per-chunk relative deviation and escalation, the pooled top-k with forced sinks,
// the compaction of the new active set and the write of layer 1's cache (the fresh row at every
// kept position, the re-rotated cached row at every other cached position). Every fresh and
// cached row is read once and every cache row written once.
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
// Design (gfx950):
//  * Tiles of P = 8 T consecutive positions (T <= 6), one per workgroup of 512 threads (one
//    workgroup per CU, so each wavefront has 256 VGPRs for the rows of its T positions);
//    wavefront w of a tile owns positions w T .. w T + T - 1 and lane l the 16-byte vector l of
//    each of a position's four rows (fresh k, fresh v, cached K, cached V): the deviation's
//    summation contract maps vector q to lane q. A lane holds its rotation partner's vector after
//    one lane exchange, and the (cos, sin) of its frequencies after the lanes evaluate one
//    frequency each and exchange them.
//  * The rows stay in registers while the selection runs over the whole grid: a grid barrier
//    after the deviations (each workgroup has added its candidates to a 4096-bin histogram of
//    their keys' top 12 bits), further 12- and 8-bit rounds only while the threshold's bin holds
//    more than 4096 candidates, then each workgroup publishes its tile's kept count (and appends
//    the candidates of the threshold's bin to a list) and a last barrier hands every workgroup
//    what it needs to rank its own positions and place its kept rows in the compacted order.
//    Typically two barriers; an escalation threshold adds two (the chunk sums come first).
//  * Deadlock-free whatever the residency: a workgroup claims its tile with an atomic exchange,
//    tiles beyond the grid go to workgroups through a counter, and a workgroup that waits too
//    long at the first barrier claims the tiles of workgroups that have not started; a tile
//    processed that way (and every tile beyond the first of a workgroup) keeps no rows in
//    registers and reloads its rows at the end. Every wait is bounded: past its limit the kernel
//    flags CKV_DEVICE_ERR_SYNC and runs to its end with unspecified outputs, every index checked.
//  * Cross-workgroup values (deviations, histogram counts, tile counts, the list) go through
//    device-scope stores, atomics and loads, which are coherent across the XCDs' L2 caches.
//  * The workspace holds two parity sets of histograms and claim flags: a call uses one and
//    clears the other for the next call; the last workgroup to leave resets the control words and
//    flips the parity. The caller zeroes the workspace once, before its first use.
#include <algorithm>
#include <mutex>

#include "ckv_common.hpp"
#include "select_common.hpp"

namespace ckv {

constexpr int kL1Threads = 512;                // one workgroup per CU: 256 VGPRs per wavefront
constexpr int kL1Waves = kL1Threads / kWave;  // 8
constexpr int kL1MaxSlots = 17;               // tiles a workgroup may hold: its own + 16
constexpr int kL1ListMax = 4096;              // threshold-bin candidates ranked in LDS
constexpr int kL1MaxGrid = 1024;
constexpr int kL1MaxTiles = 4096;
constexpr int kL1MaxSpans = 4096;
constexpr int kL1SegStride = 60;  // segment search: 64 samples, then a window of stride + T
constexpr int kL1MaxSegs = 64 * kL1SegStride;

// workspace layout, in 32-bit words
constexpr int kWsBar = 0;        // barrier arrivals (tiles), cumulative over the call
constexpr int kWsExit = 1;       // workgroups that have left
constexpr int kWsListN = 2;      // list entries appended
constexpr int kWsParity = 3;     // which histogram / claim set this call uses
constexpr int kWsNextExtra = 4;  // tickets for tiles beyond the grid
constexpr int kWsSelCached = 5;  // kept cached positions (summed at the end)
constexpr int kWsUncomp = 6;     // kept positions without a fresh row
constexpr int kWsHist = 64;                                // [2][3][4096]
constexpr int kWsClaim = kWsHist + 2 * 3 * 4096;           // [2][kL1MaxGrid]
constexpr int kWsEsc = kWsClaim + 2 * kL1MaxGrid;          // [kL1MaxSpans]
constexpr int kWsPub = kWsEsc + kL1MaxSpans;               // [kL1MaxTiles]
constexpr int kWsList = kWsPub + kL1MaxTiles;              // uint64_t [kL1ListMax]
constexpr int kWsWords = kWsList + 2 * kL1ListMax;
static_assert(kWsList % 2 == 0, "list entries are 8-byte aligned");
static_assert(kWsWords * 4 == CKV_LAYER1_REPAIR_WORKSPACE_BYTES, "workspace size");

// per-position class bits kept in LDS
constexpr uint32_t kCValid = 1u, kCCached = 2u, kCStatic = 4u, kCCand = 8u, kCNoLocal = 16u, kCSink = 32u,
                   kCKept = 64u;

enum { kModeNone = 0, kModeAll = 1, kModeList = 2, kModeTies = 3, kModeRefine = 4 };

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
  const ckv_chunk_span* spans;
  int n_spans, has_thr;
  double thr;
  float* diff;
  float* norm;
  int64_t* keep_abs;
  int64_t* keep_local;
  int32_t* keep_rank;
  float* rel_out;
  uint8_t* esc_out;
  int32_t* counts;
  uint32_t* ws;
  int32_t* err;
  int n_tiles, spin_limit, steal_after;
};

__device__ __forceinline__ uint32_t ld_dev(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class V>
__device__ __forceinline__ void st_dev(V* p, V v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t add_dev(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until this wavefront's global loads, stores and atomics have completed.
__device__ __forceinline__ void drain_vmem() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  asm volatile("" ::: "memory");
}

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
template <int DTYPE, int T>
__device__ __forceinline__ void wave_rows(const L1Args& a, const InvFreq& inv, int pb, WaveRows<DTYPE, T>& r,
                                          uint32_t (&cls)[T], float (&dv)[T], float (&nv)[T], int (&li)[T]) {
  using E = Elem<DTYPE>;
  constexpr int VEC = E::kVec;
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const int vpr = 1 << a.vpr_log2;
  const int64_t rowb = (int64_t)vpr * 16;
  const bool lane_on = lane < (a.n_heads << a.vpr_log2);
  const int h = lane >> a.vpr_log2, col = lane & (vpr - 1);
  const int64_t colb = (int64_t)col * 16;
  const int N = a.n_tokens;

  // 1. flags, local indices and the segment descriptors around the positions, all in flight
  uint32_t fl[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int p = pb + t;
    fl[t] = p < N ? a.flags[p] : 0u;
    li[t] = p < N ? a.local[p] : -1;
  }
  int sbase = 0, scount = a.n_segs;
  if (a.n_segs > kWave) {  // 64 samples, then the window that holds every position's segment
    const int stride = (a.n_segs + kWave - 1) / kWave;
    const int si = lane * stride;
    const int st = si < a.n_segs ? a.segs[si].dst_start : 0x7fffffff;
    const uint64_t m = __ballot(st <= pb);
    const int bk = m ? 63 - __builtin_clzll(m) : 0;
    sbase = bk * stride;
    scount = min(stride + T, a.n_segs - sbase);
  }
  ckv_segment sd{0x7fffffff, 0, -1, 0, 0, 0};
  if (lane < scount) sd = a.segs[sbase + lane];

  // 2. each position's segment (the last with dst_start <= p) and its chunk's base addresses
  int delta[T];
  bool have[T];
  const char* kb[T];
  const char* vb[T];
  int64_t soff[T];
  bool bad = false;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int p = pb + t;
    const uint64_t m = __ballot(lane < scount && sd.dst_start <= p);
    const int L = m ? 63 - __builtin_clzll(m) : 0;
    const int dst = __builtin_amdgcn_readlane(sd.dst_start, L);
    const int n = __builtin_amdgcn_readlane(sd.n_tokens, L);
    const int ch = __builtin_amdgcn_readlane(sd.chunk, L);
    const int ss = __builtin_amdgcn_readlane(sd.src_start, L);
    const int sl = __builtin_amdgcn_readlane(sd.src_len, L);
    delta[t] = __builtin_amdgcn_readlane(sd.delta, L);
    const bool cached = p < N && (fl[t] & CKV_POS_CACHED);
    const bool found = m != 0ull && p < dst + n;
    const bool seg_ok = found && dst >= 0 && ss >= 0 && ch >= 0 && ch < a.tab_chunks && (int64_t)dst + n <= N &&
                        (int64_t)ss + n <= sl;
    bad = bad || (cached && !seg_ok);
    have[t] = cached && seg_ok;
    kb[t] = vb[t] = nullptr;
    soff[t] = (int64_t)h * sl * rowb + (int64_t)(ss + (p - dst)) * rowb + colb;
    if (have[t]) {
      const int64_t ti = ((int64_t)ch * a.n_layers + a.layer) * 2;
      kb[t] = reinterpret_cast<const char*>(a.tab[ti]);
      vb[t] = reinterpret_cast<const char*>(a.tab[ti + 1]);
    }
    bad = bad || li[t] >= a.n_fresh;
    li[t] = li[t] >= a.n_fresh ? -1 : li[t];
    cls[t] = (p < N ? kCValid : 0u) | (cached ? kCCached : 0u) | (li[t] < 0 ? kCNoLocal : 0u) |
             ((fl[t] & CKV_POS_SINK) ? kCSink : 0u);
  }
  if (bad && lane == 0) flag_error(a.err, CKV_DEVICE_ERR_RANGE);

  // 3. cos/sin of each position's shift while the chunk addresses arrive: lane f evaluates
  // frequency f (mod D/2) once per distinct shift; the rotation fetches its column's VEC
  // frequencies from the evaluating lanes
  const int half = a.head_dim >> 1;
  const float my_inv = inv.v[lane & (half - 1)];
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

  // 4. the rows: fresh k/v at the local index, the chunk's K/V at the segment's source row
#pragma unroll
  for (int t = 0; t < T; ++t) {
    r.kf[t] = r.vf[t] = r.kc[t] = r.vc[t] = vec16{0u, 0u, 0u, 0u};
    if (li[t] >= 0 && lane_on) {
      r.kf[t] = ld16(a.kf + h * a.kf_hs_b + (int64_t)li[t] * a.kf_ts_b + colb);
      r.vf[t] = ld16(a.vf + h * a.vf_hs_b + (int64_t)li[t] * a.vf_ts_b + colb);
    }
    if (have[t] && lane_on) {
      r.kc[t] = ld16(kb[t] + soff[t]);
      r.vc[t] = ld16(vb[t] + soff[t]);
    }
  }

  // 5. re-rotate the cached keys: the partner half comes from lane l ^ (vpr / 2)
  const int half_v = vpr >> 1;
  const bool first_half = col < half_v;
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
    float x1[VEC], x2[VEC], y[VEC];
    E::unpack(first_half ? mine : other, x1);
    E::unpack(first_half ? other : mine, x2);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float c = __shfl(cv[t], f0 + e), s = __shfl(sv[t], f0 + e);
      const float p1 = x1[e] * c;
      const float p2 = x2[e] * s;
      const float p3 = x1[e] * s;
      const float p4 = x2[e] * c;
      y[e] = first_half ? p1 - p2 : p3 + p4;
    }
    if (lane_on) r.kc[t] = E::pack(y);
  }

  // 6. deviations in the contract's order: lane q adds its vector's elements in ascending order,
  // then the xor butterfly; diff = Sk + Sv, norm = Nk + Nv
#pragma unroll
  for (int t = 0; t < T; ++t) {
    float kx[VEC], vx[VEC], kcx[VEC], vcx[VEC];
    E::unpack(r.kf[t], kx);
    E::unpack(r.vf[t], vx);
    E::unpack(r.kc[t], kcx);
    E::unpack(r.vc[t], vcx);
    float sk = 0.0f, sv = 0.0f, nk = 0.0f, nw = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float dk = E::round_trip(kx[e] - kcx[e]);
      const float dw = E::round_trip(vx[e] - vcx[e]);
      sk = sk + dk * dk;
      sv = sv + dw * dw;
      nk = nk + kx[e] * kx[e];
      nw = nw + vx[e] * vx[e];
    }
    const float x = wave_butterfly_sum(sk);
    const float y = wave_butterfly_sum(sv);
    const float z = wave_butterfly_sum(nk);
    const float w = wave_butterfly_sum(nw);
    dv[t] = li[t] < 0 ? 0.0f : x + y;
    nv[t] = li[t] < 0 ? 0.0f : z + w;
  }
}

// Span coverage of the wavefront's positions pb .. pb + T - 1: pool (inside an in-range pooled span
// that does not escalate) and esc (inside an escalated span). esc_ws NULL: no span escalates.
template <int T>
__device__ __forceinline__ void wave_spans(const L1Args& a, int pb, const uint32_t* esc_ws, bool (&pool)[T],
                                           bool (&escd)[T]) {
  const int lane = (int)(threadIdx.x & (kWave - 1));
#pragma unroll
  for (int t = 0; t < T; ++t) pool[t] = escd[t] = false;
  for (int c0 = 0; c0 < a.n_spans; c0 += kWave) {
    const int c = c0 + lane;
    ckv_chunk_span sp{0, 0, 0, 0};
    if (c < a.n_spans) sp = a.spans[c];
    const bool ok = c < a.n_spans && sp.start >= 0 && sp.length >= 0 && (int64_t)sp.start + sp.length <= a.n_tokens;
    const bool e = ok && esc_ws != nullptr && ld_dev(esc_ws + c) != 0u;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int p = pb + t;
      const bool in = ok && sp.start <= p && p < sp.start + sp.length;
      pool[t] = pool[t] || __ballot(in && !e && sp.pooled != 0) != 0ull;
      escd[t] = escd[t] || __ballot(in && e) != 0ull;
    }
  }
}

// The pooled budget requested by the in-range spans that do not escalate, and the number of spans
// outside [0, n_tokens); every lane of the calling wavefront gets both.
__device__ __forceinline__ void wave_budget(const L1Args& a, const uint32_t* esc_ws, int& budget_req, int& n_bad) {
  const int lane = (int)(threadIdx.x & (kWave - 1));
  uint32_t breq = 0u, nb = 0u;
  for (int c0 = 0; c0 < a.n_spans; c0 += kWave) {
    const int c = c0 + lane;
    ckv_chunk_span sp{0, 0, 0, 0};
    if (c < a.n_spans) sp = a.spans[c];
    const bool ok = c < a.n_spans && sp.start >= 0 && sp.length >= 0 && (int64_t)sp.start + sp.length <= a.n_tokens;
    const bool e = ok && esc_ws != nullptr && ld_dev(esc_ws + c) != 0u;
    breq += (ok && !e && sp.pooled != 0) ? (uint32_t)sp.budget : 0u;
    nb += (c < a.n_spans && !ok) ? 1u : 0u;
  }
  budget_req = (int)__builtin_amdgcn_readlane((int)wave_incl_scan(breq), kWave - 1);
  n_bad = (int)__builtin_amdgcn_readlane((int)wave_incl_scan(nb), kWave - 1);
}

// Final class bits from the load classes and the span coverage (torch_engine.py:125-143):
// keep = ~cached | sink | escalated span; candidate = pooled span & ~keep.
__device__ __forceinline__ uint32_t classify(uint32_t cls, bool pool, bool esc) {
  const bool valid = cls & kCValid, cached = cls & kCCached, sink = cls & kCSink;
  const bool stat = valid && (!cached || sink || esc);
  const bool cand = valid && !stat && pool;
  return (cls & (kCValid | kCCached | kCNoLocal | kCSink)) | (stat ? kCStatic : 0u) | (cand ? kCCand : 0u);
}

// ---- the grid ---------------------------------------------------------------------------------

// All threads call. Adds `add` arrivals and waits, bounded, until the barrier's arrival count
// reaches `target`. Returns 0 (reached), 1 (steal_after polls passed: the caller may take over
// unstarted tiles) or 2 (spin limit passed: CKV_DEVICE_ERR_SYNC is flagged).
__device__ __forceinline__ int grid_wait(const L1Args& a, int spin_limit, uint32_t add, uint32_t target,
                                         int steal_after, int* s_res) {
  drain_vmem();
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t* bar = a.ws + kWsBar;
    if (add != 0u) add_dev(bar, add);
    int res = 0;
    for (int it = 0; ld_dev(bar) < target; ++it) {
      if (steal_after > 0 && it >= steal_after) {
        res = 1;
        break;
      }
      if (it >= spin_limit) {
        res = 2;
        flag_error(a.err, CKV_DEVICE_ERR_SYNC);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    *s_res = res;
  }
  __syncthreads();
  return *s_res;
}

// Exclusive workgroup scan of one int per thread in thread order, and the total, with ONE
// barrier: each call in flight gets its own `slots` (kL1Waves ints).
__device__ __forceinline__ int l1_block_scan(int v, int* slots, int& total) {
  const int lane = (int)(threadIdx.x & (kWave - 1)), wave = (int)(threadIdx.x >> 6);
  const int x = (int)wave_incl_scan((uint32_t)v);
  if (lane == kWave - 1) slots[wave] = x;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kL1Waves; ++w) {
    const int t = slots[w];
    before += w < wave ? t : 0;
    all += t;
  }
  total = all;
  return before + x - v;
}

// Counts of a radix round's bins: thread t owns bins nb - kB t - 1 .. nb - kB (t + 1) (descending
// bin order = thread order); `before` counts the bins above its own, `total` every bin.
constexpr int kB = 4096 / kL1Threads;
struct BinScan {
  uint32_t h[kB];
  int before, total;
};

template <bool COH>
__device__ __forceinline__ BinScan scan_bins(const uint32_t* hist, int nb, int* slots) {
  BinScan b;
  int sum = 0;
#pragma unroll
  for (int i = 0; i < kB; ++i) {
    b.h[i] = 0u;
    if (kB * (int)threadIdx.x < nb) {
      const uint32_t* q = hist + (nb - kB * (int)threadIdx.x - 1 - i);
      b.h[i] = COH ? ld_dev(q) : *q;
    }
    sum += (int)b.h[i];
  }
  b.before = l1_block_scan(sum, slots, b.total);
  return b;
}

// The bin holding the need-th largest key (1 <= need <= total): its digit, the count in the bins
// above it and its own count, through s_out (cleared by the caller before scan_bins).
__device__ __forceinline__ void locate_bin(const BinScan& b, int nb, int need, int* s_out, int& digit, int& above,
                                           int& count) {
  int ab = b.before;
#pragma unroll
  for (int i = 0; i < kB; ++i) {
    if (ab < need && need <= ab + (int)b.h[i]) {
      s_out[0] = nb - kB * (int)threadIdx.x - 1 - i;
      s_out[1] = ab;
      s_out[2] = (int)b.h[i];
    }
    ab += (int)b.h[i];
  }
  __syncthreads();
  digit = s_out[0];
  above = s_out[1];
  count = s_out[2];
}

template <int DTYPE, int T>
__global__ __launch_bounds__(kL1Threads) void layer1_repair_kernel(L1Args a, const InvFreq inv) {
  constexpr int P = kL1Waves * T;                // positions per tile
  constexpr int kPer = kL1ListMax / kL1Threads;  // list entries per thread
  __shared__ uint32_t s_key[kL1MaxSlots][P];     // held tiles: keys, class bits, tile index
  __shared__ uint32_t s_cls[kL1MaxSlots][P];
  __shared__ int s_tile[kL1MaxSlots];
  __shared__ uint32_t s_lh[4096];          // LDS histograms; per-tile tie counts
  __shared__ uint32_t s_cnt[kL1MaxTiles];  // per-tile kept counts, then offsets
  __shared__ int s_above[kL1MaxSlots], s_tie[kL1MaxSlots], s_tb[kL1MaxSlots];
  __shared__ int s_misc[16];
  __shared__ int slots[4][kL1Waves];
  __shared__ uint64_t s_or[kL1Waves];
  __shared__ uint64_t s_cstar;

  const int tid = (int)threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = (int)gridDim.x, wg = (int)blockIdx.x;
  const int N = a.n_tokens, n_tiles = a.n_tiles;
  uint32_t* ws = a.ws;
  const int par = (int)(ld_dev(ws + kWsParity) & 1u);
  uint32_t* hist = ws + kWsHist + par * 3 * 4096;
  uint32_t* claim = ws + kWsClaim + par * kL1MaxGrid;
  uint32_t* pub = ws + kWsPub;
  uint64_t* list = reinterpret_cast<uint64_t*>(ws + kWsList);
  uint32_t* esc_ws = ws + kWsEsc;
  const bool thr = a.has_thr != 0;
  // workspace words 8 and 9, when nonzero, override the wait limits
  const uint32_t spin_o = ld_dev(ws + 8), steal_o = ld_dev(ws + 9);
  const int spin_limit = spin_o != 0u ? (int)spin_o : a.spin_limit;
  const int steal_after = steal_o != 0u ? (int)steal_o : a.steal_after;

  // claim this workgroup's tile (its rows load meanwhile); clear the other parity's set
  uint32_t claimed = 1u;
  if (tid == 0) claimed = __hip_atomic_exchange(claim + wg, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  {
    uint32_t* z = ws + kWsHist + (par ^ 1) * 3 * 4096;
    for (int i = wg * kL1Threads + tid; i < 3 * 4096; i += G * kL1Threads) z[i] = 0u;
    uint32_t* zc = ws + kWsClaim + (par ^ 1) * kL1MaxGrid;
    for (int i = wg * kL1Threads + tid; i < kL1MaxGrid; i += G * kL1Threads) zc[i] = 0u;
  }
  for (int i = tid; i < 4096; i += kL1Threads) s_lh[i] = 0u;
  if (tid < 16) s_misc[tid] = 0;

  // Commits one computed tile into slot `slot`: deviations out, class bits and keys into LDS, and
  // (without a threshold) its candidates into the round-0 histogram.
  auto commit = [&](int slot, int tile, const uint32_t (&cls0)[T], const float (&dv)[T], const float (&nv)[T]) __attribute__((always_inline)) {
    const int pb = tile * P + wave * T;
    bool pool[T], escd[T];
    wave_spans<T>(a, pb, nullptr, pool, escd);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int p = pb + t;
      if (lane == 0) {
        if (p < N) {
          st_dev(a.diff + p, dv[t]);
          st_dev(a.norm + p, nv[t]);
        }
        s_key[slot][wave * T + t] = dev_key(dv[t]);
        s_cls[slot][wave * T + t] = classify(cls0[t], pool[t], escd[t]);
      }
    }
    if (tid == 0) s_tile[slot] = tile;
    lds_barrier();
    if (!thr && wave == 0) {  // one atomic per distinct top-12-bit bin of the tile's candidates
      const uint32_t bin = lane < P && (s_cls[slot][lane] & kCCand) ? s_key[slot][lane] >> 20 : ~0u;
      uint32_t cnt = 0u;
      bool first = true;
      for (int j = 0; j < P; ++j) {
        const uint32_t bj = (s_cls[slot][j] & kCCand) ? s_key[slot][j] >> 20 : ~0u;
        cnt += bj == bin ? 1u : 0u;
        first = first && !(j < lane && bj == bin);
      }
      if (bin != ~0u && first) add_dev(hist + bin, cnt);
    }
  };

  // 1. this workgroup's own tile, rows kept in registers
  WaveRows<DTYPE, T> rows;
  int li0[T];
  {
    uint32_t cls[T];
    float dv[T], nv[T];
    wave_rows<DTYPE, T>(a, inv, wg * P + wave * T, rows, cls, dv, nv, li0);
    if (tid == 0) s_misc[0] = (int)claimed;
    __syncthreads();
    if (s_misc[0] == 0) commit(0, wg, cls, dv, nv);
  }
  const bool own = s_misc[0] == 0;
  int held = own ? 1 : 0;
  if (wave == 0 && !thr) {  // without a threshold the budget follows from the spans alone
    int breq, nbd;
    wave_budget(a, nullptr, breq, nbd);
    if (lane == 0) {
      s_misc[4] = breq;
      s_misc[5] = nbd;
    }
  }

  // A tile held without registers (beyond the grid, or taken over): one position at a time.
  auto memory_tile = [&](int tile) __attribute__((always_inline)) {
    uint32_t cls[T];
    float dv[T], nv[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      WaveRows<DTYPE, 1> r1;
      uint32_t c1[1];
      float d1[1], n1[1];
      int l1[1];
      wave_rows<DTYPE, 1>(a, inv, tile * P + wave * T + t, r1, c1, d1, n1, l1);
      cls[t] = c1[0];
      dv[t] = d1[0];
      nv[t] = n1[0];
    }
    commit(held, tile, cls, dv, nv);
    ++held;
  };

  // 2. tiles beyond the grid, by ticket
  if (own && n_tiles > G) {
    while (held < kL1MaxSlots) {
      __syncthreads();
      if (tid == 0) s_misc[1] = G + (int)add_dev(ws + kWsNextExtra, 1u);
      __syncthreads();
      const int t = s_misc[1];
      if (t >= n_tiles) break;
      memory_tile(t);
    }
  }

  // 3. first barrier: every tile's deviations are out. A workgroup that waits long takes over a
  // ticket beyond the grid or a tile whose workgroup has not started.
  uint32_t target = (uint32_t)n_tiles;
  bool failed = false;
  {
    uint32_t add = (uint32_t)held;
    bool steal = true;
    for (;;) {
      const int res = grid_wait(a, spin_limit, add, target, steal ? steal_after : 0, &s_misc[2]);
      add = 0u;
      if (res == 0) break;
      if (res == 2) {
        failed = true;
        break;
      }
      if (wave == 0) {
        int t = -1;
        if (held < kL1MaxSlots) {
          if (n_tiles > G && lane == 0) {
            const int e = G + (int)add_dev(ws + kWsNextExtra, 1u);
            t = e < n_tiles ? e : -1;
          }
          t = __builtin_amdgcn_readfirstlane(t);
          for (int c0 = 0; c0 < G && t < 0; c0 += kWave) {
            const int c = c0 + lane;
            const bool free_t = c < G && ld_dev(claim + c) == 0u;
            uint64_t m = __ballot(free_t);
            while (m != 0ull && t < 0) {
              const int l = (int)__ffsll((unsigned long long)m) - 1;
              m &= m - 1ull;
              uint32_t old = 1u;
              if (lane == l) old = __hip_atomic_exchange(claim + c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              old = (uint32_t)__builtin_amdgcn_readlane((int)old, l);
              if (old == 0u) t = c0 + l;
            }
          }
        }
        if (lane == 0) s_misc[3] = t;
      }
      __syncthreads();
      const int t = s_misc[3];
      if (t < 0) {
        steal = false;  // nothing left to take: wait for the others
        continue;
      }
      memory_tile(t);
      add = 1u;
    }
  }

  // per-chunk rel / escalation (torch_engine.py:128-141), one wavefront per span, in the lane-strided
  // order of the selection's contract
  auto chunk_sums = [&]() __attribute__((always_inline)) {
    for (int c = wave * G + wg; c < a.n_spans; c += G * kL1Waves) {
      const ckv_chunk_span sp = a.spans[c];
      const bool ok = sp.start >= 0 && sp.length >= 0 && (int64_t)sp.start + sp.length <= N;
      float sd = 0.0f, sn = 0.0f;
      if (ok) {
        for (int q0 = 0; q0 < sp.length; q0 += 8 * kWave) {
          float bd[8], bn[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int q = q0 + j * kWave + lane;
            bd[j] = q < sp.length ? ld_dev(a.diff + sp.start + q) : 0.0f;
            bn[j] = q < sp.length ? ld_dev(a.norm + sp.start + q) : 0.0f;
          }
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            if (q0 + j * kWave + lane < sp.length) {
              sd = sd + bd[j];
              sn = sn + bn[j];
            }
          }
        }
      }
      sd = wave_butterfly_sum(sd);
      sn = wave_butterfly_sum(sn);
      const float rel = sd / sn;
      const bool esc = ok && thr && ((double)rel > a.thr);
      if (lane == 0) {
        a.rel_out[c] = rel;
        a.esc_out[c] = esc ? 1 : 0;
        if (thr) st_dev(esc_ws + c, esc ? 1u : 0u);
      }
    }
  };

  // 4. with an escalation threshold the chunk sums come first: escalated spans keep every
  // position and leave the pool, so the classes and the round-0 histogram follow them
  if (thr) {
    if (!failed) {
      chunk_sums();
      target += (uint32_t)n_tiles;
      failed = grid_wait(a, spin_limit, (uint32_t)held, target, 0, &s_misc[2]) == 2;
    }
    if (wave == 0) {
      int breq, nbd;
      wave_budget(a, esc_ws, breq, nbd);
      if (lane == 0) {
        s_misc[4] = breq;
        s_misc[5] = nbd;
      }
    }
    for (int s = 0; s < held; ++s) {
      const int pb = s_tile[s] * P + wave * T;
      bool pool[T], escd[T];
      wave_spans<T>(a, pb, esc_ws, pool, escd);
      if (lane == 0) {
#pragma unroll
        for (int t = 0; t < T; ++t) s_cls[s][wave * T + t] = classify(s_cls[s][wave * T + t], pool[t], escd[t]);
      }
    }
    lds_barrier();
    for (int i = tid; i < held * P; i += kL1Threads) {
      const int s = i / P, j = i % P;
      if (s_cls[s][j] & kCCand) atomicAdd(&s_lh[s_key[s][j] >> 20], 1u);
    }
    __syncthreads();
    for (int b = tid; b < 4096; b += kL1Threads) {
      const uint32_t v = s_lh[b];
      if (v != 0u) add_dev(hist + b, v);
      s_lh[b] = 0u;
    }
    target += (uint32_t)n_tiles;
    if (!failed) failed = grid_wait(a, spin_limit, (uint32_t)held, target, 0, &s_misc[2]) == 2;
  }

  // 5. the threshold: the top 12 bits from the round-0 histogram, 12 and 8 more while its bin
  // holds more candidates than the list takes
  const int budget_req = s_misc[4], n_bad = s_misc[5];
  int mode = kModeNone, need = 0, count = 0, rounds = 1, budget = 0, n_cand = 0;
  uint32_t prefix = 0u, pmask = 0u;
  {
    if (tid < 3) s_misc[8 + tid] = 0;
    const BinScan bs = scan_bins<true>(hist, 4096, slots[0]);
    n_cand = bs.total;
    budget = max(0, min(budget_req, n_cand));
    if (budget == 0) {
      mode = kModeNone;
    } else if (budget >= n_cand) {
      mode = kModeAll;
    } else {
      int digit, above;
      locate_bin(bs, 4096, budget, s_misc + 8, digit, above, count);
      prefix = (uint32_t)digit << 20;
      pmask = 0xfff00000u;
      need = budget - above;
      mode = count <= kL1ListMax ? kModeList : kModeRefine;
    }
  }
  for (int r = 1; r <= 2 && mode == kModeRefine; ++r) {
    const int shift = r == 1 ? 8 : 0;
    const int nb = r == 1 ? 4096 : 256;
    __syncthreads();
    for (int i = tid; i < held * P; i += kL1Threads) {
      const int s = i / P, j = i % P;
      const uint32_t k = s_key[s][j];
      if ((s_cls[s][j] & kCCand) && (k & pmask) == prefix) atomicAdd(&s_lh[(k >> shift) & (uint32_t)(nb - 1)], 1u);
    }
    __syncthreads();
    for (int b = tid; b < nb; b += kL1Threads) {
      const uint32_t v = s_lh[b];
      if (v != 0u) add_dev(hist + r * 4096 + b, v);
      s_lh[b] = 0u;
    }
    target += (uint32_t)n_tiles;
    if (!failed) failed = grid_wait(a, spin_limit, (uint32_t)held, target, 0, &s_misc[2]) == 2;
    if (tid < 3) s_misc[8 + tid] = 0;
    const BinScan bs = scan_bins<true>(hist + r * 4096, nb, slots[r & 1]);
    int digit, above;
    locate_bin(bs, nb, need, s_misc + 8, digit, above, count);
    prefix |= (uint32_t)digit << shift;
    pmask |= (uint32_t)(nb - 1) << shift;
    need -= above;
    rounds = r + 1;
    mode = count <= kL1ListMax ? kModeList : (r == 2 ? kModeTies : kModeRefine);
  }
  if (failed) mode = kModeNone;

  // 6. publication: each held tile's kept count outside the threshold's bin (static keeps and
  // candidates above it) and its candidates in the bin; the bin's candidates join the list
  const bool in_mode = mode == kModeList || mode == kModeTies;
  auto is_above = [&](uint32_t cl, uint32_t k) __attribute__((always_inline)) {
    return (cl & kCStatic) || ((cl & kCCand) && (mode == kModeAll || (in_mode && (k & pmask) > prefix)));
  };
  auto is_inbin = [&](uint32_t cl, uint32_t k) __attribute__((always_inline)) { return in_mode && (cl & kCCand) && (k & pmask) == prefix; };
  __syncthreads();
  if (tid < kL1MaxSlots) {
    s_above[tid] = 0;
    s_tie[tid] = 0;
  }
  __syncthreads();
  int my_in = 0;
  for (int i = tid; i < held * P; i += kL1Threads) {
    const int s = i / P, j = i % P;
    const uint32_t cl = s_cls[s][j], k = s_key[s][j];
    if (is_above(cl, k)) atomicAdd(&s_above[s], 1);
    if (is_inbin(cl, k)) {
      atomicAdd(&s_tie[s], 1);
      ++my_in;
    }
  }
  if (mode == kModeList) {
    int tot = 0;
    int idx = l1_block_scan(my_in, slots[2], tot);
    if (tid == 0) s_misc[6] = tot > 0 ? (int)add_dev(ws + kWsListN, (uint32_t)tot) : 0;
    __syncthreads();
    const int base = s_misc[6];
    for (int i = tid; i < held * P; i += kL1Threads) {
      const int s = i / P, j = i % P;
      const uint32_t cl = s_cls[s][j], k = s_key[s][j];
      if (is_inbin(cl, k)) {
        const uint32_t p = (uint32_t)(s_tile[s] * P + j);
        if (base + idx < kL1ListMax) st_dev(list + base + idx, ((uint64_t)k << 32) | (uint64_t)(~p));
        ++idx;
      }
    }
  }
  __syncthreads();
  if (tid < held && s_tile[tid] < n_tiles)
    st_dev(pub + s_tile[tid], (uint32_t)s_above[tid] | ((uint32_t)s_tie[tid] << 16));
  target += (uint32_t)n_tiles;
  if (!failed) failed = grid_wait(a, spin_limit, (uint32_t)held, target, 0, &s_misc[2]) == 2;
  if (failed) mode = kModeNone;

  // 7. every tile's kept count, then the offsets of the compacted outputs
  for (int t = tid; t < n_tiles; t += kL1Threads) {
    const uint32_t w = ld_dev(pub + t);
    s_cnt[t] = w & 0xffffu;
    s_lh[t] = w >> 16;
  }
  __syncthreads();
  uint64_t cstar = 0ull;
  if (mode == kModeList) {
    // the need-th largest (key, -position) in the list: MSB radix over the bits where entries
    // differ, 8 bits and one LDS histogram per pass, until a digit isolates one entry
    const int M = min(count, kL1ListMax);
    uint64_t e[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int j = tid + k * kL1Threads;
      e[k] = j < M ? ld_dev(list + j) : 0ull;
    }
    if (tid == 0) s_cstar = e[0];
    __syncthreads();
    const uint64_t e0 = s_cstar;
    uint64_t x = 0ull;
#pragma unroll
    for (int k = 0; k < kPer; ++k)
      if (tid + k * kL1Threads < M) x |= e[k] ^ e0;
    uint32_t xl = (uint32_t)x, xh = (uint32_t)(x >> 32);
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) {
      xl |= (uint32_t)__shfl_xor((int)xl, m);
      xh |= (uint32_t)__shfl_xor((int)xh, m);
    }
    if (lane == 0) s_or[wave] = ((uint64_t)xh << 32) | xl;
    __syncthreads();
    uint64_t dbits = 0ull;
#pragma unroll
    for (int w = 0; w < kL1Waves; ++w) dbits |= s_or[w];
    cstar = e0;
    if (dbits != 0ull) {
      const int hb = 63 - __builtin_clzll(dbits);
      const uint64_t low = (2ull << hb) - 1ull;  // bits 0 .. hb (all of them for hb = 63)
      uint64_t pre = e0 & ~low, pm = ~low;
      int nd = need;
      for (int i = tid; i < 8 * 256; i += kL1Threads) s_lh[2048 + i] = 0u;
      __syncthreads();
      int pass = 0;
      for (int shift = (hb >> 3) << 3; shift >= 0; shift -= 8, ++pass) {
        uint32_t* hp = s_lh + 2048 + pass * 256;
#pragma unroll
        for (int k = 0; k < kPer; ++k)
          if (tid + k * kL1Threads < M && (e[k] & pm) == pre) atomicAdd(&hp[(uint32_t)(e[k] >> shift) & 255u], 1u);
        lds_barrier();
        // every wavefront finds the digit: lane l owns digits 255 - 4l .. 252 - 4l
        uint32_t h4[4], ls = 0u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          h4[i] = hp[255 - (lane * 4 + i)];
          ls += h4[i];
        }
        uint32_t ab = wave_incl_scan(ls) - ls;
        int my_digit = -1, my_cnt = 0;
        uint32_t my_ab = 0u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if ((int)ab < nd && nd <= (int)(ab + h4[i])) {
            my_digit = 255 - (lane * 4 + i);
            my_ab = ab;
            my_cnt = (int)h4[i];
          }
          ab += h4[i];
        }
        const uint64_t fnd = __ballot(my_digit >= 0);
        const int src = fnd ? (int)__ffsll((unsigned long long)fnd) - 1 : 0;
        const int dg = __builtin_amdgcn_readlane(my_digit, src);
        const int cnt = __builtin_amdgcn_readlane(my_cnt, src);
        nd -= __builtin_amdgcn_readlane((int)my_ab, src);
        pre |= (uint64_t)(uint32_t)max(dg, 0) << shift;
        pm |= 255ull << shift;
        if (cnt <= 1 || shift == 0) break;  // uniform
      }
#pragma unroll
      for (int k = 0; k < kPer; ++k)
        if (tid + k * kL1Threads < M && (e[k] & pm) == pre) s_cstar = e[k];
      __syncthreads();
      cstar = s_cstar;
    }
    // the kept entries count for their tiles
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      if (tid + k * kL1Threads < M && e[k] >= cstar) {
        const uint32_t tile = (~(uint32_t)e[k]) / (uint32_t)P;
        if (tile < (uint32_t)n_tiles) atomicAdd(&s_cnt[tile], 1u);
      }
    }
    __syncthreads();
  } else if (mode == kModeTies) {
    // every candidate in the bin has the same key: the lowest positions are taken
    const int per = (n_tiles + kL1Threads - 1) / kL1Threads;
    int sum = 0;
    for (int i = 0; i < per; ++i) {
      const int t = tid * per + i;
      if (t < n_tiles) sum += (int)s_lh[t];
    }
    int tot = 0;
    int run = l1_block_scan(sum, slots[3], tot);
    for (int i = 0; i < per; ++i) {
      const int t = tid * per + i;
      if (t < n_tiles) {
        const int tie = (int)s_lh[t];
        s_cnt[t] += (uint32_t)max(0, min(need - run, tie));
        s_lh[t] = (uint32_t)run;  // ties before this tile
        run += tie;
      }
    }
    __syncthreads();
    if (tid < held && s_tile[tid] < n_tiles) s_tb[tid] = (int)s_lh[s_tile[tid]];
    __syncthreads();
  }
  int n_keep = 0;
  {
    const int per = (n_tiles + kL1Threads - 1) / kL1Threads;
    int sum = 0;
    for (int i = 0; i < per; ++i) {
      const int t = tid * per + i;
      if (t < n_tiles) sum += (int)s_cnt[t];
    }
    int run = l1_block_scan(sum, slots[0], n_keep);
    for (int i = 0; i < per; ++i) {
      const int t = tid * per + i;
      if (t < n_tiles) {
        const int c = (int)s_cnt[t];
        s_cnt[t] = (uint32_t)run;
        run += c;
      }
    }
    __syncthreads();
  }

  // 8. each held tile (one wavefront each): the kept positions, their ranks, the compacted
  // outputs
  uint32_t kept_cached = 0u, uncomputed = 0u;
  const uint64_t lt = (1ull << lane) - 1ull;
  for (int s = wave; s < held; s += kL1Waves) {
    const int tile = s_tile[s];
    const bool on = lane < P;
    const uint32_t cl = on ? s_cls[s][lane] : 0u;
    const uint32_t k = on ? s_key[s][lane] : 0u;
    const int p = tile * P + lane;
    const bool valid = on && (cl & kCValid) && tile < n_tiles;
    bool kept = valid && is_above(cl, k);
    const bool ib = valid && is_inbin(cl, k);
    if (mode == kModeList) {
      kept = kept || (ib && ((((uint64_t)k << 32) | (uint64_t)(~(uint32_t)p)) >= cstar));
    } else if (mode == kModeTies) {
      const int r = __popcll(__ballot(ib) & lt);
      kept = kept || (ib && s_tb[s] + r < need);
    }
    const uint64_t km = __ballot(kept);
    const int rank = (tile < n_tiles ? (int)s_cnt[tile] : 0) + __popcll(km & lt);
    if (valid) {
      const int32_t lc = a.local[p];
      if (kept && rank < N) {
        a.keep_abs[rank] = p;
        a.keep_local[rank] = lc < 0 ? 0 : lc;
      }
      if (a.keep_rank != nullptr) a.keep_rank[p] = kept ? rank : -1;
      kept_cached += (kept && (cl & kCCached)) ? 1u : 0u;
      uncomputed += (kept && lc < 0) ? 1u : 0u;
    }
    if (on) s_cls[s][lane] = cl | (kept ? kCKept : 0u);
  }
  lds_barrier();

  // 9. the cache rows: the fresh row at a kept position, the cached row (keys re-rotated) at any
  // other; the own tile's rows from registers, the others reloaded
  {
    const int vpr = 1 << a.vpr_log2;
    const int64_t rowb = (int64_t)vpr * 16;
    const bool lane_on = lane < (a.n_heads << a.vpr_log2);
    const int64_t hoff = (int64_t)(lane >> a.vpr_log2) * a.d_hs_b + (int64_t)(lane & (vpr - 1)) * 16;
    auto put = [&](int p, bool kept, int li, const vec16& kf, const vec16& vf, const vec16& kc, const vec16& vc) __attribute__((always_inline)) {
      if (p >= N || !lane_on) return;
      const bool fresh = kept && li >= 0;
      const int64_t off = hoff + (int64_t)p * rowb;
      st16(a.dk + off, fresh ? kf : kc);
      st16(a.dv + off, fresh ? vf : vc);
    };
    if (own) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int j = wave * T + t;
        put(wg * P + j, (s_cls[0][j] & kCKept) != 0u, li0[t], rows.kf[t], rows.vf[t], rows.kc[t], rows.vc[t]);
      }
    }
    for (int s = own ? 1 : 0; s < held; ++s) {
      const int tile = s_tile[s];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int j = wave * T + t;
        WaveRows<DTYPE, 1> r1;
        uint32_t c1[1];
        float d1[1], n1[1];
        int l1[1];
        wave_rows<DTYPE, 1>(a, inv, tile * P + j, r1, c1, d1, n1, l1);
        put(tile * P + j, (s_cls[s][j] & kCKept) != 0u, l1[0], r1.kf[0], r1.vf[0], r1.kc[0], r1.vc[0]);
      }
    }
  }

  if (!thr) chunk_sums();

  // 10. totals; the last workgroup to leave writes the counts and resets the control words
  kept_cached = (uint32_t)__builtin_amdgcn_readlane((int)wave_incl_scan(kept_cached), kWave - 1);
  uncomputed = (uint32_t)__builtin_amdgcn_readlane((int)wave_incl_scan(uncomputed), kWave - 1);
  if (lane == 0 && kept_cached != 0u) add_dev(ws + kWsSelCached, kept_cached);
  if (lane == 0 && uncomputed != 0u) add_dev(ws + kWsUncomp, uncomputed);
  drain_vmem();
  __syncthreads();
  if (tid == 0) {
    const uint32_t ticket = add_dev(ws + kWsExit, 1u);
    if (ticket == (uint32_t)G - 1u) {
      int32_t* counts = a.counts;
      counts[CKV_COUNT_KEEP] = n_keep;
      counts[CKV_COUNT_SELECTED_CACHED] = (int32_t)ld_dev(ws + kWsSelCached);
      counts[CKV_COUNT_BUDGET] = budget;
      counts[CKV_COUNT_CANDIDATES] = n_cand;
      counts[CKV_COUNT_UNCOMPUTED] = (int32_t)ld_dev(ws + kWsUncomp);
      counts[CKV_COUNT_BUDGET_REQUESTED] = budget_req;
      counts[CKV_COUNT_BAD_SPANS] = n_bad;
      counts[CKV_COUNT_TOP_HISTOGRAM] = rounds;
      st_dev(ws + kWsBar, 0u);
      st_dev(ws + kWsListN, 0u);
      st_dev(ws + kWsNextExtra, 0u);
      st_dev(ws + kWsSelCached, 0u);
      st_dev(ws + kWsUncomp, 0u);
      st_dev(ws + kWsParity, (uint32_t)(par ^ 1));
      st_dev(ws + kWsExit, 0u);
    }
  }
}

// ---- host -------------------------------------------------------------------------------------

template <int DTYPE, int T>
static const void* l1_kernel() {
  return reinterpret_cast<const void*>(&layer1_repair_kernel<DTYPE, T>);
}

constexpr int kL1Ts[] = {2, 4, 6};  // positions per wavefront of the instantiations (8 would spill)

template <int DTYPE>
static const void* l1_kernel_for(int T) {
  return T == 2 ? l1_kernel<DTYPE, 2>() : T == 4 ? l1_kernel<DTYPE, 4>() : l1_kernel<DTYPE, 6>();
}

// Workgroups of one instantiation a CU holds at once (1 by design), cached.
static int l1_occupancy(int dtype, int T) {
  static std::mutex mu;
  static int cache[2][9] = {};
  std::lock_guard<std::mutex> lock(mu);
  int& c = cache[dtype == CKV_DTYPE_BF16 ? 1 : 0][T];
  if (c == 0) {
    const void* k = dtype == CKV_DTYPE_BF16 ? l1_kernel_for<CKV_DTYPE_BF16>(T) : l1_kernel_for<CKV_DTYPE_F32>(T);
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, kL1Threads, 0) != hipSuccess) return 0;
    c = n;
  }
  return c;
}

template <int DTYPE>
static int32_t launch_l1(int T, int G, hipStream_t st, const L1Args& args, const InvFreq& inv) {
#define CKV_L1(TT)                                                                                              \
  if (T == TT) {                                                                                                \
    hipLaunchKernelGGL((layer1_repair_kernel<DTYPE, TT>), dim3((unsigned)G), dim3(kL1Threads), 0, st, args, inv); \
    CKV_RETURN_IF_LAUNCH_FAILED();                                                                              \
    return CKV_OK;                                                                                              \
  }
  CKV_L1(2)
  CKV_L1(4)
  CKV_L1(6)
#undef CKV_L1
  return CKV_ERR_INVALID_ARGUMENT;
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
  using namespace ckv;
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
  if (n_tokens > CKV_SELECT_MAX_TOKENS || n_segs > kL1MaxSegs || n_chunks > kL1MaxSpans) return CKV_ERR_TOO_LARGE;
  if (n_tokens == 0)  // nothing to repair: the selection writes the counts and the spans' stats
    return ckv_select(diff, norm, pos_flags, local, 0, chunks, n_chunks, has_threshold, escalate_threshold, keep_abs,
                      keep_local, keep_rank, rel_dev, escalated, counts, stream);

  int dev = 0, n_cu = 0;
  if (hipStreamGetDevice((hipStream_t)stream, &dev) != hipSuccess ||
      hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
    return CKV_ERR_HIP;
  // the fewest positions per wavefront whose tiles fit one resident grid; else 6 and extra tiles
  int T = 0, G = 0, n_tiles = 0;
  for (int t : kL1Ts) {
    const int occ = l1_occupancy(dtype, t);
    if (occ <= 0) return CKV_ERR_HIP;
    const int gmax = std::min(n_cu * occ, kL1MaxGrid);
    const int nt = (n_tokens + kL1Waves * t - 1) / (kL1Waves * t);
    T = t;
    n_tiles = nt;
    G = std::min(nt, gmax);
    if (nt <= gmax) break;
  }
  if (n_tiles > kL1MaxTiles || n_tiles > G * kL1MaxSlots) return CKV_ERR_TOO_LARGE;

  L1Args args{};
  args.dk = (char*)dst_k;
  args.dv = (char*)dst_v;
  args.d_hs_b = dst_head_stride * eb;
  args.tab = src_tab;
  args.tab_chunks = n_tab_chunks;
  args.n_layers = n_layers;
  args.layer = layer;
  args.segs = segs;
  args.n_segs = n_segs;
  args.kf = (const char*)k_fresh;
  args.kf_hs_b = kf_head_stride * eb;
  args.kf_ts_b = kf_token_stride * eb;
  args.vf = (const char*)v_fresh;
  args.vf_hs_b = vf_head_stride * eb;
  args.vf_ts_b = vf_token_stride * eb;
  args.n_fresh = n_fresh;
  args.flags = pos_flags;
  args.local = local;
  args.n_tokens = n_tokens;
  args.n_heads = n_heads;
  args.head_dim = head_dim;
  args.vpr_log2 = vpr_log2;
  args.spans = chunks;
  args.n_spans = n_chunks;
  args.has_thr = has_threshold != 0;
  args.thr = escalate_threshold;
  args.diff = diff;
  args.norm = norm;
  args.keep_abs = keep_abs;
  args.keep_local = keep_local;
  args.keep_rank = keep_rank;
  args.rel_out = rel_dev;
  args.esc_out = escalated;
  args.counts = counts;
  args.ws = (uint32_t*)workspace;
  args.err = err;
  args.n_tiles = n_tiles;
  args.spin_limit = 1 << 21;  // about a second of polls: far beyond any barrier of a healthy run
  args.steal_after = 256;     // polls (a few hundred microseconds) before taking over unstarted tiles
  const InvFreq& inv = host_inv_freq(head_dim, theta);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == CKV_DTYPE_BF16) return launch_l1<CKV_DTYPE_BF16>(T, G, st, args, inv);
  return launch_l1<CKV_DTYPE_F32>(T, G, st, args, inv);
}
