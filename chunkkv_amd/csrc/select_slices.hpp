// The layer-1 selection without an escalation threshold, spread over the chip: one launch of
// many workgroups, each of which finds the threshold of the pooled top-k itself (from the
// candidate histogram the deviation launch counted, or by radix passes where that histogram
// cannot be used), counts the kept positions before its slice of positions, and compacts its
// slice: keep_abs / keep_local / keep_rank, and optionally the scatter of the slice's kept rows
// from the fresh rows into the layer's cache. No workgroup waits for another: no grid barrier,
// no spin wait, no second launch.
//
// Reference semantics (src/chunkkv/engine/torch_engine.py:125-156) with no escalation threshold:
//   keep = ~cached | sink                                          (:125-127)
//   pool = union of the spans of placements with ratio > 0; budget = sum int(round(ratio * len))
//   budget = min(budget, (pool & ~keep).sum())                     (:142)
//   top = argsort(-where(pool & ~keep, diff, -1))[:budget]; keep[top] = True   (:143-145)
//   keep_abs = keep.nonzero(); sel = local[keep_abs]               (:146-152)
//   K[:, :, keep_abs] = k[:, :, sel]; V likewise                   (:155-156)
// with the ties torch's unstable argsort leaves open fixed as elsewhere in this library: larger
// deviation first, then lower position; NaN last. The outputs are bit-identical to
// select_reg_kernel followed by scatter_rows_kernel.
//
// Layout (gfx950): 1024 threads (four wavefronts per SIMD, which hide each other's latencies);
// thread t owns G groups of four consecutive positions, group i = positions 4 (t + 1024 i) .. +3,
// so every load instruction of a wavefront reads 64 consecutive groups. Right after its loads a
// thread reduces each position to a code, ordered as the selection ranks positions. With up to
// 3 groups per thread (12288 positions) the code is 32-bit:
//   0xffffffff / 0xfffffffe   not cached / sink: always kept
//   ((bin + 1) << 17) | k     a candidate (cached, not sink, inside a pooled span) whose key
//                             (the order-preserving image of its deviation) lies in histogram
//                             bin `bin` with k its low 17 bits (an interior bin is a key prefix)
//   0                         neither (or past n_tokens)
// and above it (registers permitting) 16-bit: 0xffff / 0xfffe, bin + 1, 0.
// A position is kept iff code > Tc, or code == Tc and p <= p*, or its bit in the taken bitmap
// (LDS) is set (forced codes exceed every Tc).
//  - Histogram path: the bin b* holding the budget-th largest key comes from a suffix scan of the
//    histogram; the candidates of b* (a few dozen at the 8k request) are listed in LDS (their
//    keys from the 32-bit codes, or read from L2) and ranked directly (up to kSlRankMax), or by
//    radix passes over the list (up to kSlListMax). With 32-bit codes the need-th entry gives Tc
//    and p*; with 16-bit codes Tc = bin + 1 and the taken entries are marked in the bitmap.
//  - Otherwise (no histogram, an edge bin, a histogram that does not match the candidates, a
//    longer list): radix passes over every candidate's key, re-read from L2 in each pass, and
//    the taken candidates marked in the bitmap.
#pragma once

#include "select_common.hpp"

namespace ckv {

constexpr int kSlThreads = 1024;
constexpr int kSlWaves = kSlThreads / kWave;
constexpr int kSlRankMax = 128;   // threshold-bin candidates ranked directly
constexpr int kSlListMax = 4096;  // threshold-bin candidates refined by radix passes over an LDS list
constexpr int kSlHists = 4;       // digit histograms per pass buffer (wavefront w counts into w % 4)
constexpr int kSlWideCodes = 3;   // groups per thread up to which the codes are 32-bit

// Per-position codes of a thread's G groups: 32-bit (C32) or 16-bit, two per register.
template <int G, bool C32>
struct Codes {
  static constexpr uint32_t kUncached = C32 ? 0xffffffffu : 0xffffu;
  static constexpr uint32_t kForcedMin = kUncached - 1u;  // the sink code
  uint32_t w[G][C32 ? 4 : 2];
  __device__ __forceinline__ uint32_t get(int i, int j) const {
    if constexpr (C32) return w[i][j];
    else return (w[i][j >> 1] >> (16 * (j & 1))) & 0xffffu;
  }
  __device__ __forceinline__ void set(int i, int j, uint32_t c) {
    if constexpr (C32) {
      w[i][j] = c;
    } else if (j & 1) {
      w[i][j >> 1] |= c << 16;
    } else {
      w[i][j >> 1] = c;
    }
  }
  __device__ __forceinline__ static bool cand(uint32_t c) { return c != 0u && c < kForcedMin; }
};

// The scatter of a slice's kept rows (optional): the layer's cache (H, N, D) and the fresh rows.
struct SliceRows {
  char* dk;
  char* dv;
  int64_t d_hs_b;  // cache head stride, bytes
  const char* kf;
  int64_t kf_hs_b, kf_ts_b;
  const char* vf;
  int64_t vf_hs_b, vf_ts_b;
  int n_fresh, n_heads, vpr;  // 16-byte vectors per row (a power of two)
};

// Exclusive workgroup prefix of a 64-bit value with its total; `slots` (kSlWaves entries) must
// not be read by any other call in flight since the previous barrier. One LDS-only barrier.
__device__ __forceinline__ uint64_t sl_scan_u64(uint64_t v, uint64_t* slots, uint64_t& total) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const uint64_t x = wave_incl_scan(v);
  if (lane == kWave - 1) slots[wave] = x;
  lds_barrier();
  uint64_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kSlWaves; ++w) {
    const uint64_t t = slots[w];
    before += (w < wave) ? t : 0;
    all += t;
  }
  total = all;
  return before + x - v;
}

// One MSB-first digit pass: each(visit) calls visit(value) for this thread's live values; among
// those with (value & pmask) == prefix, the digit (value >> shift) & dmask holding the need-th
// largest is appended to prefix / pmask, need becomes the rank within that digit, and the
// digit's count is returned. h: kSlHists cleared histograms of 256 bins, cleared again before
// this returns. Two LDS barriers.
template <class Each>
__device__ __forceinline__ uint32_t sl_pass(Each each, uint32_t& prefix, uint32_t& pmask, int& need, int shift,
                                            uint32_t dmask, uint32_t (*h)[256]) {
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  uint32_t* hw = h[wave % kSlHists];
  const uint32_t pf = prefix, pm = pmask;
  each([&](uint32_t v) {
    if ((v & pm) == pf) atomicAdd(&hw[(v >> shift) & dmask], 1u);
  });
  lds_barrier();
  // every wavefront folds the histograms and finds the digit: lane l owns digits 255-4l .. 252-4l
  uint32_t h4[4];
  uint32_t local_sum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = 255 - (lane * 4 + i);
    h4[i] = h[0][d] + h[1][d] + h[2][d] + h[3][d];
    local_sum += h4[i];
  }
  const uint32_t incl = wave_incl_scan(local_sum);
  uint32_t above = incl - local_sum;
  int my_digit = -1;
  uint32_t my_above = 0u, my_count = 0u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (above < (uint32_t)need && (uint32_t)need <= above + h4[i]) {
      my_digit = 255 - (lane * 4 + i);
      my_above = above;
      my_count = h4[i];
    }
    above += h4[i];
  }
  const uint64_t found = __ballot(my_digit >= 0);
  const int src = found ? (int)__ffsll((unsigned long long)found) - 1 : 0;  // wavefront-uniform
  const int digit = __builtin_amdgcn_readlane(my_digit, src);
  need -= (int)__builtin_amdgcn_readlane((int)my_above, src);
  const uint32_t count = (uint32_t)__builtin_amdgcn_readlane((int)my_count, src);
  prefix |= (uint32_t)digit << shift;
  pmask |= dmask << shift;
  lds_barrier();  // every wavefront has read the histograms: clear them for the next pass
  for (int b = tid; b < kSlHists * 256; b += kSlThreads) (&h[0][0])[b] = 0u;
  return count;
}

// Grid: n_slices selecting workgroups (slice s = positions [s S, min((s + 1) S, N))), then
// workgroups of chunk sums (rel_dev, escalated = 0; one wavefront per chunk). S is a power of two
// from 32 to 256, so a slice's groups belong to S/4 consecutive lanes of one wavefront.
// counts[CKV_COUNT_UNCOMPUTED] must be zero before the launch (the launch before it clears it);
// the workgroups add their slices' counts. ghist (may be NULL) is the candidate histogram, with a
// ticket word right after its kTopBins bins, zero before the launch: each selecting workgroup
// takes a ticket once its histogram loads have landed, and the last one clears the histogram
// and the ticket for the next call.
// The pointers and sizes the first loads use lead the argument list (preloaded into SGPRs).
template <int G, bool ROWS, bool C32 = (G <= kSlWideCodes)>
__global__ __launch_bounds__(kSlThreads) void select_slices_kernel(
    const float* diff, const uint8_t* flags, uint32_t* ghist, const int32_t* local, int n_tokens, int n_chunks,
    const ckv_chunk_span* chunks, int slice_len_copies, int n_slices, SelectArgs a, SliceRows rw, int32_t* err) {
  constexpr int NT = kSlThreads;
  constexpr int BPT = kTopBins / NT;  // histogram bins per thread (4: one 16-byte load)
  static_assert(BPT == 4, "a thread's bins are one 16-byte load");
  // pool bitmask, then the taken-candidate bitmask, each covering the workgroup's capacity (MW
  // words): group i of thread t is 4 bits of word t / 8 + 128 i (an immediate offset from one base)
  extern __shared__ uint32_t lds_dyn[];
  constexpr int MW = NT / 8 * G;
  __shared__ uint32_t hist[2][kSlHists][256];
  __shared__ uint64_t slots64[2][kSlWaves];
  __shared__ uint2 lst[kSlListMax];  // the threshold bin's candidates: (key, position)
  __shared__ int s_budget_req, s_bad, s_n, s_last, s_nrows;
  __shared__ int s_top[3];  // threshold bin, rank within it, its count
  __shared__ uint32_t s_T;
  __shared__ int s_pstar;
  __shared__ int2 s_rows[256];  // the slice's kept positions in rank order: (position, fresh row)

  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int N = n_tokens;
  if ((int)blockIdx.x >= n_slices) {  // chunk sums beside the selection
    a.diff = diff;
    a.n_tokens = N;
    a.chunks = chunks;
    a.n_chunks = n_chunks;
    for (int c = ((int)blockIdx.x - n_slices) * kSlWaves + wave; c < n_chunks;
         c += ((int)gridDim.x - n_slices) * kSlWaves)
      chunk_sums_wave(a, c);
    return;
  }
  uint32_t* poolw = lds_dyn;
  uint32_t* takew = lds_dyn + MW;
  const uint32_t* pool_t = poolw + (tid >> 3);  // this thread's words (group i: pool_t[128 i])
  const uint32_t* take_t = takew + (tid >> 3);
  const int nib = (4 * tid) & 31;
  // slice length in the low 16 bits, the histogram's copies above them: both among the
  // preloaded arguments, so the first loads wait for no scalar load of the struct arguments
  const int slice_len = slice_len_copies & 0xffff;
  const int hcopies = slice_len_copies >> 16;
  const int s0 = (int)blockIdx.x * slice_len;
  const bool aligned = ((uintptr_t)diff % 16 == 0) && ((uintptr_t)flags % 4 == 0);

  // Group i of this thread: the wavefront's 64 groups of row i in range (uniform) load as
  // 16-byte / 4-byte vectors, the wavefront crossing n_tokens element by element, clamped
  // (values past n_tokens are never used: their codes are 0).
  auto load_group = [&](int i, float (&d)[4], uint32_t& f) {
    const int base = 4 * (tid + NT * i);
    const bool whole = aligned && __builtin_amdgcn_readfirstlane(4 * ((wave + 1) * kWave + NT * i)) <= N;
    if (whole) {
      const float4 x = *(const float4*)(diff + base);
      d[0] = x.x;
      d[1] = x.y;
      d[2] = x.z;
      d[3] = x.w;
      f = *(const uint32_t*)(flags + base);
    } else {
      f = 0u;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t pc = clamp_pos(base + j, N);
        d[j] = ld_at(diff, pc);
        f |= (uint32_t)ld_at(flags, pc) << (8 * j);
      }
    }
  };

  // ---- phase 0: every load up front. The chunk spans go first: phase 1 uses them before anything
  // else loaded here (vector loads complete in issue order), so it runs while the rest are in
  // flight. Their index is clamped instead of the load sitting behind tid < n_chunks: entries
  // past n_chunks are never read (phase 1 tests c < n_chunks first).
  ckv_chunk_span sp = {0, 0, 0, 0};
  if (n_chunks > 0) {  // uniform
    const vec16 v = ld16(chunks + min(tid, n_chunks - 1));
    sp = ckv_chunk_span{(int32_t)v.x, (int32_t)v.y, (int32_t)v.z, (int32_t)v.w};
  }
  float dv[G][4];
  uint32_t fw[G];
#pragma unroll
  for (int i = 0; i < G; ++i) load_group(i, dv[i], fw[i]);
  // the histogram's copies, as the counting launch spread it
  const vec16 g4 =
      ghist != nullptr ? hist_load4_n(ghist + (kTopBins - BPT * (tid + 1)), hcopies) : vec16{0u, 0u, 0u, 0u};
  // the slice's groups: S/4 consecutive threads at group row ig
  const int sg0 = s0 >> 2;
  const int ig = sg0 / NT, t_first = sg0 % NT;
  const bool slice_owner = tid >= t_first && tid < t_first + (slice_len >> 2);
  int lv[4] = {0, 0, 0, 0};
  auto load_local = [&]() {
    if (slice_owner) {
      const int base = 4 * (tid + NT * ig);
      if (base + 4 <= N && (uintptr_t)local % 16 == 0) {
        const int4 l = *(const int4*)(local + base);
        lv[0] = l.x;
        lv[1] = l.y;
        lv[2] = l.z;
        lv[3] = l.w;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) lv[j] = ld_at(local, clamp_pos(base + j, N));
      }
    }
  };
  // with 9 groups per thread the local indices come late (registers), otherwise with the first loads
  constexpr bool kLateLocal = G > 6;
  if constexpr (!kLateLocal) load_local();

  // ---- phase 1: LDS state; the pool bitmask from the spans
  if (tid == 0) {
    s_budget_req = 0;
    s_bad = 0;
    s_n = 0;
    s_nrows = 0;
    s_top[0] = 0;  // an edge bin (radix passes) unless a thread finds the threshold's bin
  }
  for (int w = tid; w < 2 * MW; w += NT) lds_dyn[w] = 0u;
  for (int b = tid; b < 2 * kSlHists * 256; b += NT) (&hist[0][0][0])[b] = 0u;
  lds_barrier();
  for (int c0 = 0; c0 < n_chunks; c0 += NT) {
    const int c = c0 + tid;
    if (c0 > 0) {
      sp = ckv_chunk_span{0, 0, 0, 0};
      if (c < n_chunks) sp = span_at(chunks, c);
    }
    const bool in = c < n_chunks;
    const bool ok = in && sp.start >= 0 && sp.length >= 0 && (int64_t)sp.start + sp.length <= N;
    if (in && !ok) atomicAdd(&s_bad, 1);
    if (ok && sp.pooled && sp.length > 0) {
      atomicAdd(&s_budget_req, sp.budget);
      const int a0 = sp.start, b0 = sp.start + sp.length;
      for (int word = a0 >> 5; word <= (b0 - 1) >> 5; ++word) {
        const int lo = max(a0, word << 5) - (word << 5);
        const int hi = min(b0, (word << 5) + 32) - (word << 5);
        atomicOr(&poolw[word], (hi - lo == 32) ? 0xffffffffu : (((1u << (hi - lo)) - 1u) << lo));
      }
    }
  }
  lds_barrier();

  // ---- phase 2: codes; candidate and mismatch counts; the histogram's share of this thread
  using CD = Codes<G, C32>;
  CD code;
  int n_cand = 0, mism = 0;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int base = 4 * (tid + NT * i);
    const uint32_t pool4 = (pool_t[(NT / 8) * i] >> nib) & 0xfu;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool valid = base + j < N;
      const uint32_t f = (fw[i] >> (8 * j)) & 0xffu;
      const bool cached = (f & CKV_POS_CACHED) != 0, sink = (f & CKV_POS_SINK) != 0;
      const bool open = valid && cached && !sink;
      const bool c = open && ((pool4 >> j) & 1u);
      const bool hc = open && (f & CKV_POS_POOLED);
      const uint32_t key = dev_key(dv[i][j]);
      const uint32_t bin1 = top_bin(key) + 1u;
      const uint32_t cc = C32 ? (bin1 << kTopShift) | (key & ((1u << kTopShift) - 1u)) : bin1;
      code.set(i, j, !valid ? 0u : !cached ? CD::kUncached : sink ? CD::kForcedMin : c ? cc : 0u);
      n_cand += c ? 1 : 0;
      mism += c != hc ? 1 : 0;
    }
  }
  const uint32_t gsum = g4.x + g4.y + g4.z + g4.w;
  uint64_t scan_tot = 0;
  const uint64_t scan_ex =
      sl_scan_u64((uint64_t)n_cand | ((uint64_t)mism << 21) | ((uint64_t)gsum << 42), slots64[0], scan_tot);
  // the workgroup's ticket (every thread's histogram load landed before the scan's barrier); its
  // value is first read in phase 4, so no barrier before then waits for the atomic's round trip.
  // The address carries threadIdx.y, 0 in this one-dimensional launch but a per-lane value to
  // the compiler: at a provably uniform address its atomic optimizer broadcasts the returned
  // value right after the atomic, and phase 3's first barrier then waited for the round trip.
  // Every load above has landed before it (an explicit wait, free here: the histogram loads, which
  // the scan needed, were issued after the deviations and flags, and vector loads complete in
  // order): otherwise a value used after it, such as a code computed late, waits for every memory
  // operation of the wavefront, the atomic included.
  const int opaque0 = (int)threadIdx.y;
  uint32_t ticket = 0u;
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt and lgkmcnt at their maxima (no wait)
  if (ghist != nullptr && tid == 0) ticket = atomicAdd(ghist + kHistWords + opaque0, 1u);
  const int cand_total = (int)(scan_tot & kField);
  const int budget_req = s_budget_req;
  const int budget = max(0, min(budget_req, cand_total));
  bool use_top = ghist != nullptr && ((scan_tot >> 21) & kField) == 0 && (int)((scan_tot >> 42) & kField) == cand_total;

  // ---- phase 3: the threshold (Tc, p*), or the taken candidates' bitmap
  uint32_t Tc = CD::kForcedMin - 1u;  // with no budget: only the forced positions are kept
  int pstar = -1;
  bool marked = false;  // the taken candidates are marked in takew instead
  bool ranked = false;
  if (budget > 0) {  // uniform
    bool listed = false;
    if (use_top) {
      // the bin holding the budget-th largest key: the thread whose bins hold it writes it
      const uint32_t above = (uint32_t)((scan_ex >> 42) & kField);
      const uint32_t need0 = (uint32_t)budget;
      if (above < need0 && need0 <= above + gsum) {
        const uint32_t a3 = above + g4.w, a2 = a3 + g4.z, a1 = a2 + g4.y;  // above bins b0+2, b0+1, b0
        const int e = need0 <= a3 ? 0 : need0 <= a2 ? 1 : need0 <= a1 ? 2 : 3;  // bin b0 + 3 - e
        const uint32_t before = e == 0 ? above : e == 1 ? a3 : e == 2 ? a2 : a1;
        s_top[0] = kTopBins - BPT * tid - 1 - e;
        s_top[1] = (int)(need0 - before);
        s_top[2] = (int)(e == 0 ? g4.w : e == 1 ? g4.z : e == 2 ? g4.y : g4.x);
      }
      lds_barrier();
      const int tb = s_top[0], need = s_top[1], m = s_top[2];
      if (tb > 0 && tb < kTopBins - 1 && m <= kSlListMax) {  // uniform: an interior bin, listable
        // list the bin's candidates (key from the code), then find the need-th
        const uint32_t target = (uint32_t)(tb + 1);
        auto in_bin = [&](uint32_t cd) { return CD::cand(cd) && (C32 ? cd >> kTopShift : cd) == target; };
        int mine = 0;
#pragma unroll
        for (int i = 0; i < G; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) mine += in_bin(code.get(i, j)) ? 1 : 0;
        const int incl = (int)wave_incl_scan((uint32_t)mine);
        int wbase = 0;
        if (lane == kWave - 1) wbase = atomicAdd(&s_n, incl);
        int off = __builtin_amdgcn_readlane(wbase, kWave - 1) + incl - mine;
        const uint32_t pfx = top_bin_prefix((uint32_t)tb);
#pragma unroll
        for (int i = 0; i < G; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t cd = code.get(i, j);
            if (in_bin(cd)) {
              if (off < kSlListMax)
                lst[off] = make_uint2(pfx | (cd & ((1u << kTopShift) - 1u)), (uint32_t)(4 * (tid + NT * i) + j));
              ++off;
            }
          }
        lds_barrier();
        if (s_n == m) {  // uniform: the listed entries are the histogram's count
          listed = true;
          if constexpr (!C32) {  // 16-bit codes hold no key bits: the listed keys from L2
            constexpr int kG = 4;
            for (int e0 = tid; e0 < m; e0 += kG * NT) {
              float d[kG];
#pragma unroll
              for (int u = 0; u < kG; ++u) d[u] = e0 + u * NT < m ? ld_at(diff, lst[e0 + u * NT].y) : 0.0f;
#pragma unroll
              for (int u = 0; u < kG; ++u)
                if (e0 + u * NT < m) lst[e0 + u * NT].x = dev_key(d[u]);
            }
            lds_barrier();
          }
          if (m <= kSlRankMax) {
            // entry e's rank (entries ahead of it in (key desc, position asc)) by 8 lanes
            constexpr int LPE = NT / kSlRankMax, PER = kSlRankMax / LPE;
            const int e = tid / LPE, part = tid % LPE;
            int ahead = 0;
            uint2 me = make_uint2(0u, 0u);
            if (e < m) {
              me = lst[e];
              uint2 o[PER];
#pragma unroll
              for (int k = 0; k < PER; ++k) o[k] = lst[part + LPE * k];  // inside the list's storage
#pragma unroll
              for (int k = 0; k < PER; ++k)
                ahead += (part + LPE * k < m && (o[k].x > me.x || (o[k].x == me.x && o[k].y < me.y))) ? 1 : 0;
            }
#pragma unroll
            for (int s = 1; s < LPE; s <<= 1) ahead += __shfl_xor(ahead, s);
            if (e < m && part == 0 && ahead == need - 1) {
              s_T = me.x;
              s_pstar = (int)me.y;
            }
            lds_barrier();
            ranked = true;
          } else {
            // radix passes over the listed keys' 17 low bits, then over the ties' positions
            uint32_t prefix = pfx, pmask = 0xffffffffu << kTopShift;
            int nd = need;
            auto each_key = [&](auto visit) {
              for (int e = tid; e < m; e += NT) visit(lst[e].x);
            };
            sl_pass(each_key, prefix, pmask, nd, 9, 255u, hist[0]);
            sl_pass(each_key, prefix, pmask, nd, 1, 255u, hist[1]);
            const int ties = (int)sl_pass(each_key, prefix, pmask, nd, 0, 1u, hist[0]);
            int ps = 0x7fffffff;
            if (nd < ties) {  // the nd lowest positions among the ties: the nd-th largest of 0xffff - p
              const uint32_t T = prefix;
              auto each_pos = [&](auto visit) {
                for (int e = tid; e < m; e += NT) {
                  const uint2 x = lst[e];
                  if (x.x == T) visit(0xffffu - x.y);
                }
              };
              uint32_t pp = 0u, pm = 0xffff0000u;
              sl_pass(each_pos, pp, pm, nd, 8, 255u, hist[1]);
              sl_pass(each_pos, pp, pm, nd, 0, 255u, hist[0]);
              ps = (int)(0xffffu - pp);
            }
            if (tid == 0) {
              s_T = prefix;
              s_pstar = ps;
            }
            lds_barrier();
          }
          if constexpr (C32) {  // the code of the threshold key
            Tc = (target << kTopShift) | (s_T & ((1u << kTopShift) - 1u));
            pstar = s_pstar;
          } else {  // higher bins by code, this bin's taken entries marked
            const uint32_t T = s_T;
            const int ps = s_pstar;
            for (int e = tid; e < m; e += NT) {
              const uint2 x = lst[e];
              if (x.x > T || (x.x == T && (int)x.y <= ps)) atomicOr(&takew[x.y >> 5], 1u << (x.y & 31));
            }
            lds_barrier();
            Tc = target;
            marked = true;
          }
        }
      }
      if (!listed) use_top = false;
    }
    if (!listed) {
      // radix passes over every candidate's key, re-read from L2 in each pass one group at a time
      // (candidacy recomputed from the flags and the pool bitmap: no register array is indexed)
      auto each_group = [&](auto fn) {
#pragma unroll 1
        for (int i = 0; i < G; ++i) {
          float d[4];
          uint32_t f;
          load_group(i, d, f);
          const int base = 4 * (tid + NT * i);
          const uint32_t pool4 = (pool_t[(NT / 8) * i] >> nib) & 0xfu;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t fj = (f >> (8 * j)) & 0xffu;
            const bool c = base + j < N && (fj & CKV_POS_CACHED) && !(fj & CKV_POS_SINK) && ((pool4 >> j) & 1u);
            if (c) fn(base + j, dev_key(d[j]));
          }
        }
      };
      auto each_cand = [&](auto visit) { each_group([&](int, uint32_t k) { visit(k); }); };
      uint32_t prefix = 0u, pmask = 0u;
      int nd = budget;
      int ties = 0;
#pragma unroll 1
      for (int shift = 24; shift >= 0; shift -= 8)
        ties = (int)sl_pass(each_cand, prefix, pmask, nd, shift, 255u, hist[(shift >> 3) & 1]);
      const uint32_t T = prefix;
      int ps = 0x7fffffff;
      if (nd < ties) {
        auto each_pos = [&](auto visit) {
          each_group([&](int p, uint32_t k) {
            if (k == T) visit(0xffffu - (uint32_t)p);
          });
        };
        uint32_t pp = 0u, pm = 0xffff0000u;
        sl_pass(each_pos, pp, pm, nd, 8, 255u, hist[1]);
        sl_pass(each_pos, pp, pm, nd, 0, 255u, hist[0]);
        ps = (int)(0xffffu - pp);
      }
      // mark the taken candidates
      each_group([&](int p, uint32_t k) {
        if (k > T || (k == T && p <= ps)) atomicOr(&takew[p >> 5], 1u << (p & 31));
      });
      lds_barrier();
      marked = true;
    }
  }

  // ---- phase 4: kept positions before the slice; totals
  int n_before = 0, n_kept = 0, n_unc = 0;
  uint32_t k4s = 0u;  // the slice group's kept bits
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int base = 4 * (tid + NT * i);
    const uint32_t t4 = marked ? (take_t[(NT / 8) * i] >> nib) & 0xfu : 0u;
    uint32_t k4 = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t cd = code.get(i, j);
      const bool kept = cd > Tc || (cd == Tc && base + j <= pstar) || ((t4 >> j) & 1u);
      k4 |= (uint32_t)kept << j;
      n_unc += cd == CD::kUncached ? 1 : 0;
    }
    const int nb = min(max(s0 - base, 0), 4);
    n_before += __popc(k4 & ((1u << nb) - 1u));
    n_kept += __popc(k4);
    k4s = i == ig ? k4 : k4s;
  }
  if (ghist != nullptr && tid == 0) s_last = ticket == (uint32_t)(n_slices - 1) ? 1 : 0;  // the scan's barrier publishes it
  uint64_t red_tot = 0;
  sl_scan_u64((uint64_t)n_before | ((uint64_t)n_kept << 21) | ((uint64_t)n_unc << 42), slots64[1], red_tot);
  const int prefix_keep = (int)(red_tot & kField);
  if (blockIdx.x == 0 && tid == 0) {
    int32_t* counts = a.counts;
    const int total = (int)((red_tot >> 21) & kField);
    counts[CKV_COUNT_KEEP] = total;
    counts[CKV_COUNT_SELECTED_CACHED] = total - (int)((red_tot >> 42) & kField);
    counts[CKV_COUNT_BUDGET] = budget;
    counts[CKV_COUNT_CANDIDATES] = cand_total;
    counts[CKV_COUNT_BUDGET_REQUESTED] = budget_req;
    counts[CKV_COUNT_BAD_SPANS] = s_bad;
    counts[CKV_COUNT_TOP_HISTOGRAM] = (use_top ? 1 : 0) | (ranked ? 2 : 0);
  }
  if (ghist != nullptr && s_last) {  // uniform: the last ticket; every workgroup has read the histogram
    hist_zero4_n(ghist + (kTopBins - BPT * (tid + 1)), hcopies);
    if (tid == 0) ghist[kHistWords] = 0u;
  }

  // ---- phase 5: the slice (its owners are S/4 consecutive lanes of one wavefront)
  if constexpr (kLateLocal) load_local();
  if (__builtin_amdgcn_readfirstlane((int)(t_first / kWave)) == wave) {  // uniform
    const uint32_t k4 = slice_owner ? k4s : 0u;
    const uint32_t incl = wave_incl_scan((uint32_t)__popc(k4));
    int rank = prefix_keep + (int)(incl - (uint32_t)__popc(k4));
    if (slice_owner) {
      const int base = 4 * (tid + NT * ig);
      int kr[4];
      int unc = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool k = (k4 >> j) & 1u;
        kr[j] = k ? rank : -1;
        if (k) {
          a.keep_abs[rank] = base + j;
          a.keep_local[rank] = lv[j] < 0 ? 0 : lv[j];
          unc += lv[j] < 0;
          if constexpr (ROWS) s_rows[rank - prefix_keep] = make_int2(base + j, lv[j]);
          ++rank;
        }
      }
      if (a.keep_rank != nullptr) {
        if (base + 4 <= N && (uintptr_t)a.keep_rank % 16 == 0) {
          *(int4*)(a.keep_rank + base) = make_int4(kr[0], kr[1], kr[2], kr[3]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (base + j < N) a.keep_rank[base + j] = kr[j];
        }
      }
      if (unc > 0) atomicAdd(a.counts + CKV_COUNT_UNCOMPUTED, unc);
    }
    if (ROWS && lane == kWave - 1) s_nrows = (int)incl;
  }

  // ---- phase 6: the slice's kept rows from the fresh rows into the cache. Thread t copies 16-byte
  // vector t % per_row (K rows first, then V) of rows t / per_row, + rpr, ...
  if constexpr (ROWS) {
    lds_barrier();
    const int n_rows = s_nrows;
    const int hv = rw.n_heads * rw.vpr;  // vectors per K (or V) row set
    const int per_row = 2 * hv;
    const int rpr = NT / per_row;  // rows per round (per_row <= 128)
    const int r0 = tid / per_row, it = tid - r0 * per_row;
    if (r0 < rpr) {
      const bool is_v = it >= hv;
      const int r2 = is_v ? it - hv : it;
      const int h = r2 >> __builtin_ctz(rw.vpr);
      const int64_t cb = (int64_t)(r2 & (rw.vpr - 1)) * 16;
      const char* src = (is_v ? rw.vf + h * rw.vf_hs_b : rw.kf + h * rw.kf_hs_b) + cb;
      const int64_t sts = is_v ? rw.vf_ts_b : rw.kf_ts_b;
      char* dst = (is_v ? rw.dv : rw.dk) + h * rw.d_hs_b + cb;
      const int64_t row_b = (int64_t)rw.vpr * 16;
      constexpr int kU = 8;  // rows in flight per thread
      for (int j0 = r0; j0 < n_rows; j0 += kU * rpr) {
        vec16 x[kU];
        int64_t drow[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          const int j = j0 + u * rpr;
          drow[u] = -1;
          if (j < n_rows) {
            const int2 pr = s_rows[j];
            if (pr.y >= 0 && pr.y < rw.n_fresh) {
              x[u] = ld16_stream(src + pr.y * sts);
              drow[u] = pr.x;
            } else if (it == 0) {
              flag_error(err, CKV_DEVICE_ERR_RANGE);  // a kept position with no fresh row
            }
          }
        }
#pragma unroll
        for (int u = 0; u < kU; ++u)
          if (drow[u] >= 0) st16_stream(dst + drow[u] * row_b, x[u]);  // non-temporal, as every cache-row writer
      }
    }
  }
}

}  // namespace ckv
