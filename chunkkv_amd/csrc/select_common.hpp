// Layer-1 selection machinery shared by ckv_select and ckv_deviation_select: per-chunk relative
// deviation and escalation, pooled budget, pooled top-k with forced sinks, and compaction of the
// new active set, run by one 1024-thread workgroup.
//
// Reference semantics (src/chunkkv/engine/torch_engine.py:125-153):
//   keep = ~cached | sink
//   for each non-exact placement p:                              (:128-140)
//     rel = diff[span].sum() / norm[span].sum()                   (fp32, .item())
//     escalated = thr is not None and rel > thr                   (Python float compare)
//     if escalated: keep[span] = True
//     elif ratio > 0: pool[span] = True; budget += int(round(ratio * len))
//   budget = min(budget, (pool & ~keep).sum())                    (:142)
//   top = argsort(-where(pool & ~keep, diff, -1))[:budget]; keep[top] = True   (:143-145)
//   keep_abs = keep.nonzero(); sel = local[keep_abs]              (:146-152)
// torch's argsort is not stable, so the reference leaves the order of equal deviations open;
// these kernels fix it: larger diff first, then lower token index (NaN ranks last).
//
// Design (gfx950): 16 wavefronts; keep/pool spans live as N-bit masks in LDS. Chunk sums: one
// wavefront per chunk, lane-strided fp32 partials + xor butterfly (the order the oracle
// restates). Top-k: MSB-first radix select over order-preserving 32-bit keys, which yields the
// exact threshold key T and how many ties at T to take; then key > T plus the lowest-index ties
// are taken and the kept positions compacted in token order. Each thread owns a contiguous run
// of KPT <= 33 positions whose keys stay in registers for every pass. A caller that already
// counted the candidates by top_bin (ckv_deviation_select and ckv_layer1_repair do so while they
// compute the deviations) hands that histogram in: the threshold's bin then comes from one
// workgroup scan over it, and only the few candidates in that bin are ranked (directly, up to
// kRankMax of them, else by radix passes over the remaining 17 key bits).
#pragma once

#include "ckv_common.hpp"

namespace ckv {

constexpr int kSelThreads = 1024;
#ifndef CKV_SEL_REG_MAX
#define CKV_SEL_REG_MAX 16
#endif
constexpr int kSelRegMax = CKV_SEL_REG_MAX;  // positions per thread up to which the keys stay in registers
constexpr int kSelWaves = kSelThreads / kWave;
// Top-digit histogram: kTopBins bins over a window of the keys of positive deviations. Interior
// bin b (1 <= b <= kTopBins - 2) holds the keys [kTopLo + (b - 1) 2^kTopShift, kTopLo + b 2^kTopShift),
// i.e. the keys whose top 32 - kTopShift bits equal those of kTopLo + (b - 1) 2^kTopShift: 1/64 of an
// octave of deviation each (the sign, the exponent and 6 mantissa bits), 4094 of them covering
// 2^-24 <= diff < 2^39.97. Bin 0 holds every key below the window (smaller deviations, zero, NaN)
// and bin kTopBins - 1 every key above it; they are not key prefixes, so a threshold that falls
// into one is found by full radix passes instead. (Deviations are sums of squares, so the window
// spends no bins on negative values, and deviations of one chunk, which cluster within a few
// percent of each other, spread over several bins.)
constexpr int kTopShift = 17;
constexpr int kTopBins = 4096;
constexpr uint32_t kTopLo = 0x80000000u | (103u << 23);  // key of 2^-24
static_assert(kTopBins == 4 * kSelThreads, "each thread owns four top-digit bins");
static_assert((kTopLo & ((1u << kTopShift) - 1u)) == 0u, "interior bins are key prefixes");
static_assert((uint64_t)kTopLo + ((uint64_t)(kTopBins - 2) << kTopShift) <= 0xffffffffull, "window inside the key range");

// The histogram can be held as kHistCopies copies of kTopBins words (the workspace's first
// kHistWords words; the spread selection's ticket word follows them): workgroup w of the counting
// launch adds into copy w % kHistCopies, so its atomics land on four addresses per bin instead of
// one, and a reader sums the copies of its bins. With uncorrelated fresh rows most candidates
// share a handful of bins and atomics on one address serialise: a 32,832-position layer-1 pass
// took 96 us with one copy, 55 us with two, 35 us (as with correlated rows) with four or eight,
// and the 8k request's layer-1 repair 129.5 us with one copy against 115.4 us with four (114.2 us
// with correlated rows either way). Reading four copies costs a selection up to ~0.8 us where it
// is on the critical path. So the layer-1 pass (four positions a workgroup, the engine's path)
// counts into four copies above 2048 positions (hist_copies_l1); the deviation launch of
// ckv_deviation_select (eight positions a workgroup) above 16384 (hist_copies): its 8192-position
// selection would pay 0.7 us for the copies (config 3: 25.2 against 26.0 us). The selection
// reads as many copies as SelectArgs::hist_copies says.
constexpr int kHistCopies = 4;
constexpr int kHistWords = kHistCopies * kTopBins;
static_assert(kHistWords * 4 + 4 <= CKV_DEVIATION_SELECT_WORKSPACE_BYTES &&
                  CKV_DEVIATION_SELECT_WORKSPACE_BYTES == CKV_LAYER1_REPAIR_WORKSPACE_BYTES,
              "the histogram copies and the ticket fit the workspaces");
__host__ __device__ constexpr int hist_copies(int n_tokens) { return n_tokens > 16384 ? kHistCopies : 1; }
__host__ __device__ constexpr int hist_copies_l1(int n_tokens) { return n_tokens > 2048 ? kHistCopies : 1; }

// This workgroup's copy of a histogram held as `copies` copies.
__device__ __forceinline__ uint32_t* hist_copy(uint32_t* h, int copies) {
  return h + ((int)blockIdx.x % copies) * kTopBins;
}
// Four adjacent bins (p = their first word in copy 0), summed over C copies.
template <int C>
__device__ __forceinline__ vec16 hist_load4(const uint32_t* p) {
  vec16 s = ld16(p);
#pragma unroll
  for (int c = 1; c < C; ++c) s += ld16(p + c * kTopBins);
  return s;
}
// Clear four adjacent bins in each of C copies.
template <int C>
__device__ __forceinline__ void hist_zero4(uint32_t* p) {
#pragma unroll
  for (int c = 0; c < C; ++c) st16(p + c * kTopBins, vec16{0u, 0u, 0u, 0u});
}
// The same for `copies` copies (1 or kHistCopies, uniform): each form's loads go out together.
__device__ __forceinline__ vec16 hist_load4_n(const uint32_t* p, int copies) {
  return copies > 1 ? hist_load4<kHistCopies>(p) : hist_load4<1>(p);
}
__device__ __forceinline__ void hist_zero4_n(uint32_t* p, int copies) {
  if (copies > 1) hist_zero4<kHistCopies>(p);
  else hist_zero4<1>(p);
}

// Order-preserving key of a deviation: larger float -> larger key; -0 == +0; NaN -> 0.
__device__ __forceinline__ uint32_t dev_key(float f) {
  if (f != f) return 0u;
  if (f == 0.0f) f = 0.0f;
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Histogram bin of a key (monotone in the key).
__device__ __forceinline__ uint32_t top_bin(uint32_t key) {
  if (key < kTopLo) return 0u;
  const uint32_t b = ((key - kTopLo) >> kTopShift) + 1u;
  return b < (uint32_t)kTopBins - 1u ? b : (uint32_t)kTopBins - 1u;
}
// Smallest key of interior bin b.
__device__ __forceinline__ uint32_t top_bin_prefix(uint32_t b) { return kTopLo + ((b - 1u) << kTopShift); }

__device__ __forceinline__ bool bit_of(const uint32_t* w, int p) { return (w[p >> 5] >> (p & 31)) & 1u; }

// Workgroup barrier that orders LDS only: waits for this wavefront's LDS operations (lgkmcnt 0),
// not for its global loads and stores, which __syncthreads() would also drain. Values loaded
// from global memory are still waited for where they are used.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt at their maxima (no wait)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Exclusive prefix count of `pred` over the workgroup in thread order, plus the total.
__device__ __forceinline__ int block_excl_count(bool pred, int* wave_tot, int& total) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const uint64_t m = __ballot(pred);
  const int in_wave = __popcll(m & ((1ull << lane) - 1ull));
  if (lane == 0) wave_tot[wave] = __popcll(m);
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    const int t = wave_tot[w];
    before += (w < wave) ? t : 0;
    all += t;
  }
  __syncthreads();  // wave_tot is reused by the next call
  total = all;
  return before + in_wave;
}

// Set bits [a, b) of an LDS bitmask, spreading the words over the lanes of one wavefront.
__device__ __forceinline__ void set_bit_range(uint32_t* w, int a, int b, int lane) {
  if (a >= b) return;
  for (int word = (a >> 5) + lane; word <= ((b - 1) >> 5); word += kWave) {
    const int lo = max(a, word << 5) - (word << 5);
    const int hi = min(b, (word << 5) + 32) - (word << 5);  // exclusive, 1..32
    const uint32_t m = (hi - lo == 32) ? 0xffffffffu : (((1u << (hi - lo)) - 1u) << lo);
    atomicOr(&w[word], m);
  }
}

// Exclusive workgroup scan of one int per thread with ONE barrier, which orders LDS only (the
// scan exchanges nothing through global memory; a full barrier would wait for this wavefront's
// stores in flight): each call must get its own `slots` array (kSelWaves ints) that no call in
// flight since the previous barrier reads.
__device__ __forceinline__ int block_scan_1b(int v, int* slots, int& total) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int x = (int)wave_incl_scan((uint32_t)v);
  if (lane == kWave - 1) slots[wave] = x;
  lds_barrier();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    const int t = slots[w];
    before += (w < wave) ? t : 0;
    all += t;
  }
  total = all;
  return before + x - v;
}

// block_scan_1b for a 64-bit value (several counts packed in disjoint bit fields).
__device__ __forceinline__ uint64_t block_scan_1b_u64(uint64_t v, uint64_t* slots, uint64_t& total) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const uint64_t x = wave_incl_scan(v);
  if (lane == kWave - 1) slots[wave] = x;
  lds_barrier();
  uint64_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    const uint64_t t = slots[w];
    before += (w < wave) ? t : 0;
    all += t;
  }
  total = all;
  return before + x - v;
}

struct SelectArgs {
  const float* diff;
  const float* norm;
  const uint8_t* flags;
  const int32_t* local;
  int n_tokens;
  const ckv_chunk_span* chunks;
  int n_chunks;
  int has_thr;
  double thr;
  int64_t* keep_abs;
  int64_t* keep_local;
  int32_t* keep_rank;  // may be NULL
  float* rel_out;
  uint8_t* esc_out;
  int32_t* counts;
  int hist_copies;  // copies of the candidate histogram the counting launch used (0 or 1: one)
};

// rel_dev / escalated of chunk c (no threshold: never escalated), computed by the calling
// wavefront in the selection's order: lane l adds positions start + l, start + l + 64, ...
// ascending, then the xor butterfly (what select_run does with SUMS).
__device__ __forceinline__ void chunk_sums_wave(const SelectArgs& a, int c) {
  constexpr int kBatch = 8;
  const int lane = (int)(threadIdx.x % kWave);
  const ckv_chunk_span sp = a.chunks[c];
  const bool ok = sp.start >= 0 && sp.length >= 0 && (int64_t)sp.start + sp.length <= a.n_tokens;
  float sd = 0.0f, sn = 0.0f;
  if (ok) {
    for (int q0 = 0; q0 < sp.length; q0 += kBatch * kWave) {
      float bd[kBatch], bn[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int q = q0 + j * kWave + lane;
        bd[j] = q < sp.length ? a.diff[sp.start + q] : 0.0f;
        bn[j] = q < sp.length ? a.norm[sp.start + q] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        if (q0 + j * kWave + lane < sp.length) {
          sd = sd + bd[j];
          sn = sn + bn[j];
        }
      }
    }
  }
  sd = wave_butterfly_sum(sd);
  sn = wave_butterfly_sum(sn);
  if (lane == 0) {
    a.rel_out[c] = sd / sn;
    a.esc_out[c] = 0;
  }
}

constexpr uint64_t kField = 0x1fffffull;  // 21-bit count fields of the packed workgroup scans
constexpr int kLightPass = 1024;          // candidates in the top bin up to which passes are light
constexpr int kRankMax = 128;             // candidates in the top bin up to which they are ranked directly

// The selection for n_tokens <= KPT * 1024, run by one whole 1024-thread workgroup: thread t owns
// positions [t*KPT, (t+1)*KPT), whose keys stay in registers through every radix pass.
//   ghist  NULL, or the top_bin histogram over the positions flagged cached, pooled and not sink
//          (what the candidates are when no chunk escalates). It is used when it matches the
//          candidate set exactly (same positions, same total) and the threshold falls into an
//          interior bin, else the selection runs its full four passes. Either way it is zeroed
//          before the function returns.
//   masks  2 * ceil(n_tokens / 32) words of LDS.
// Barrier budget: chunk phase 1; candidate scan 1; top-bin broadcast 1 (histogram path);
// 2 per radix pass (double-buffered histograms, every wavefront derives the digit itself); tie
// scan 1 (only when ties at the threshold are split); compaction scan 1.
// Chunks whose spans a wavefront loads before the selection (registers permitting).
template <int KPT>
constexpr int kSelPre = KPT <= 16 ? 2 : 1;

// Spans of the chunks wavefront `wave` handles first (wave + r * 16, r < kSelPre), zero past the
// last chunk: loaded by every workgroup of ckv_deviation_select at its start, so the selecting
// workgroup has them without a dependent round trip.
// Span c (c uniform) through the scalar cache: the spans are constant for the launch, and a
// scalar load leaves the wavefront's vector loads in flight (a vector load would be waited for
// together with every one issued before it).
__device__ __forceinline__ ckv_chunk_span span_at(const ckv_chunk_span* chunks, int c) {
  typedef __attribute__((address_space(4))) const int32_t ci32;
  ci32* f = (ci32*)(chunks + c);
  return ckv_chunk_span{f[0], f[1], f[2], f[3]};
}

// The first spans go out as vector loads, before the selection's other loads: waiting for
// them then waits for nothing issued later (vector loads complete in issue order), while a
// scalar load would hold up the selection's first LDS barrier (which waits for every scalar
// load) until the spans arrive.
template <int KPT>
__device__ __forceinline__ void load_first_spans(const ckv_chunk_span* chunks, int n_chunks, int wave,
                                                 ckv_chunk_span (&sp)[kSelPre<KPT>]) {
#pragma unroll
  for (int r = 0; r < kSelPre<KPT>; ++r) {
    const int c = wave + r * kSelWaves;  // uniform
    sp[r] = ckv_chunk_span{0, 0, 0, 0};
    if (c < n_chunks) {
      const vec16 v = ld16(chunks + c);
      sp[r] = ckv_chunk_span{(int32_t)v.x, (int32_t)v.y, (int32_t)v.z, (int32_t)v.w};
    }
  }
}

// Position p clamped into [0, n_tokens), and element idx of an array whose base address is
// wavefront-uniform, addressed as that base plus a 32-bit offset (the base stays in scalar
// registers; one 64-bit address per position and array put the 33-position bucket's addresses
// into scratch memory).
__device__ __forceinline__ uint32_t clamp_pos(int p, int n_tokens) { return (uint32_t)min(p, n_tokens - 1); }
template <class T>
__device__ __forceinline__ T ld_at(const T* base, uint32_t idx) {
  return *(const T*)((const char*)base + idx * (uint32_t)sizeof(T));
}

// SUMS = false (only without a threshold): the per-chunk sums and rel_dev/escalated are left to
// other workgroups (chunk_sums_wave); the budget and the pool come from the spans alone.
template <int KPT, bool SUMS = true>
__device__ __forceinline__ void select_run(const SelectArgs& a, uint32_t* ghist, uint32_t* masks,
                                           const ckv_chunk_span (&sp0)[kSelPre<KPT>]) {
  static_assert(KPT <= 33, "a run of KPT positions spans at most two mask words and one 64-bit word");
  constexpr int kBatch = 8;  // chunk-sum loads in flight per lane
  __shared__ __align__(16) uint32_t hist[2][kSelWaves][256];  // also the rank list and the store staging
  __shared__ uint32_t hl[3][256];  // one shared histogram per pass after the top digit (few candidates)
  __shared__ int slots[2][kSelWaves];
  __shared__ uint64_t slots64[2][kSelWaves];
  __shared__ int s_budget_req, s_bad_span, s_rk_n;
  __shared__ int s_top[3];  // threshold top digit, ties still to take after it, its bin's count

  const float* __restrict__ diff = a.diff;
  const float* __restrict__ norm = a.norm;
  const uint8_t* __restrict__ flags = a.flags;
  const int32_t* __restrict__ local = a.local;
  const int n_tokens = a.n_tokens;
  const ckv_chunk_span* __restrict__ chunks = a.chunks;
  const int n_chunks = a.n_chunks;
  const int tid = threadIdx.x, lane = tid % kWave;
  // uniform, so the chunk loop below loads its spans through the scalar cache: a vector load
  // there would make the loop wait for every row load issued before it
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int W = (n_tokens + 31) >> 5;
  uint32_t* escw = masks;
  uint32_t* poolw = masks + W;

  // Phase 0, no barrier before it: every global load this workgroup can issue up front, all in
  // flight together (nothing loaded is used before the last load has gone out). The first chunks'
  // spans come in with the call, so their deviation loads go out at once too.
  const int p0 = tid * KPT;
  constexpr int kFlagWords = (KPT + 3) / 4;
  constexpr int kPre = kSelPre<KPT>;
  float dv[KPT];            // the owned positions' deviations (their keys after phase 0)
  uint32_t fl[kFlagWords];  // their flag bytes, four per register
  int lv[KPT];              // their local indices (the compaction's keep_local)
  // From 16 positions per thread the local indices are loaded by the compaction, which alone
  // uses them: held from the start they pushed the 16-position bucket past the 128 registers a
  // thread of a 1024-thread workgroup has, 20-28 bytes per thread into scratch memory.
  constexpr bool kLateLocal = KPT >= 16;
#pragma unroll
  for (int w = 0; w < kFlagWords; ++w) fl[w] = 0u;
  // A thread's run is contiguous, so lanes are KPT elements apart: with KPT % 4 == 0 and aligned
  // arrays, 16-byte (4-byte for flags) loads cut the load instructions and cache-line requests
  // four-fold.
  int32_t* keep_rank = a.keep_rank;
  const bool vec_ok = KPT % 4 == 0 && (((uintptr_t)diff | (uintptr_t)local) % 16 == 0) &&
                      ((uintptr_t)flags % 4 == 0) && (keep_rank == nullptr || (uintptr_t)keep_rank % 16 == 0);
  // One branch per wavefront, not per thread and group: with a per-thread choice the two paths
  // write the same registers, so every vector group had to land before the next could go out
  // (three memory round trips in a row instead of one).
  const int wave_end = __builtin_amdgcn_readfirstlane((wave + 1) * kWave * KPT);
  constexpr int kWin = (KPT + 2) / 4 + 1;   // aligned flag words holding bytes p0 .. p0 + KPT - 1
  constexpr int kFlagOver = 4 * kWin - KPT;  // their bytes past the run at most (p0 % 4 == 0)
  // The loads go out in the order their values are needed (vector loads complete in issue order):
  // the deviations, the top-digit histogram, the flags, and last the local indices, which only
  // the compaction uses.
  // The top-digit bins this thread owns: bins b0 .. b0 + 3, b0 = kTopBins - 4 (tid + 1), so that
  // thread order is descending bin order.
  vec16 g4 = {0u, 0u, 0u, 0u};
  uint32_t* gmine = ghist != nullptr ? ghist + (kTopBins - 4 * (tid + 1)) : nullptr;
  auto load_hist = [&]() {
    if (gmine != nullptr) g4 = hist_load4_n(gmine, a.hist_copies);
  };
  if (vec_ok && wave_end <= n_tokens) {  // uniform: the whole wavefront's runs are in range
#pragma unroll
    for (int i0 = 0; i0 < KPT; i0 += 4) {
      const float4 d = *(const float4*)(diff + p0 + i0);
      dv[i0] = d.x;
      dv[i0 + 1] = d.y;
      dv[i0 + 2] = d.z;
      dv[i0 + 3] = d.w;
    }
    load_hist();
#pragma unroll
    for (int i0 = 0; i0 < KPT; i0 += 4) fl[i0 / 4] = *(const uint32_t*)(flags + p0 + i0);  // flags i0 .. i0 + 3
    if constexpr (!kLateLocal) {
#pragma unroll
      for (int i0 = 0; i0 < KPT; i0 += 4) {
        const int4 l = *(const int4*)(local + p0 + i0);
        lv[i0] = l.x;
        lv[i0 + 1] = l.y;
        lv[i0 + 2] = l.z;
        lv[i0 + 3] = l.w;
      }
    }
  } else if (wave_end + kFlagOver <= n_tokens && (uintptr_t)flags % 4 == 0) {  // uniform
    // Runs in range but not 16-byte loadable (KPT % 4 != 0, or arrays not aligned): one address
    // per array and thread, the positions at immediate offsets from it; the flags as the kWin
    // aligned 32-bit words from p0 rounded down (at most kFlagOver bytes past the run: below
    // n_tokens here), realigned by v_alignbyte (one register per four positions in flight, not
    // one per position).
    const float* d = diff + p0;
#pragma unroll
    for (int i = 0; i < KPT; ++i) dv[i] = d[i];
    load_hist();
    const uint32_t* fw = (const uint32_t*)(flags + (p0 & ~3));
    uint32_t win[kWin + 1];
#pragma unroll
    for (int w = 0; w < kWin; ++w) win[w] = fw[w];
    win[kWin] = 0u;
    const uint32_t sh = (uint32_t)(p0 & 3);
#pragma unroll
    for (int w = 0; w < kFlagWords; ++w) fl[w] = __builtin_amdgcn_alignbyte(win[w + 1], win[w], sh);
    if constexpr (!kLateLocal) {
      const int32_t* l = local + p0;
#pragma unroll
      for (int i = 0; i < KPT; ++i) lv[i] = l[i];
    }
  } else if (__builtin_amdgcn_readfirstlane(wave * kWave * KPT) < n_tokens) {  // uniform
    // The wavefront whose runs cross n_tokens: every load unconditional, its index clamped into
    // range (loads behind per-position branches went out one round trip at a time). The values
    // of positions past the end are never used: every use below is masked by the candidate or
    // kept bits, which only positions below n_tokens get.
#pragma unroll
    for (int i = 0; i < KPT; ++i) dv[i] = ld_at(diff, clamp_pos(p0 + i, n_tokens));
    load_hist();
#pragma unroll
    for (int i = 0; i < KPT; ++i) fl[i / 4] |= (uint32_t)ld_at(flags, clamp_pos(p0 + i, n_tokens)) << (8 * (i % 4));
    if constexpr (!kLateLocal) {
#pragma unroll
      for (int i = 0; i < KPT; ++i) lv[i] = ld_at(local, clamp_pos(p0 + i, n_tokens));
    }
  } else {  // a wavefront past the last position: nothing to load
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      dv[i] = __uint_as_float(0x7fc00000u);
      if constexpr (!kLateLocal) lv[i] = 0;
    }
    load_hist();
  }
  // the first batch of this wavefront's first chunks' deviations
  float bd0[kPre][kBatch], bn0[kPre][kBatch];
#pragma unroll
  for (int r = 0; r < (SUMS ? kPre : 0); ++r) {
    const int c = wave + r * kSelWaves;
    const bool ok0 = sp0[r].start >= 0 && sp0[r].length >= 0 && (int64_t)sp0[r].start + sp0[r].length <= n_tokens;
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int q = j * kWave + lane;
      const bool in = c < n_chunks && ok0 && q < sp0[r].length;
      bd0[r][j] = in ? diff[sp0[r].start + q] : 0.0f;
      bn0[r][j] = in ? norm[sp0[r].start + q] : 0.0f;
    }
  }
  if (tid == 0) {
    s_budget_req = 0;
    s_bad_span = 0;
    s_rk_n = 0;
  }
  for (int w = tid; w < 2 * W; w += kSelThreads) masks[w] = 0u;
  for (int b = tid; b < 2 * kSelWaves * 256; b += kSelThreads) (&hist[0][0][0])[b] = 0u;
  if (tid < 3 * 256) (&hl[0][0])[tid] = 0u;
  lds_barrier();  // the loads above stay in flight

  // Phase 1: per-chunk rel / escalation / budget, one wavefront per chunk, summed in the
  // contract's order (lane-strided, ascending, then the xor butterfly).
  const ckv_chunk_span sp_first = sp0[0], sp_last = sp0[kPre - 1];
  for (int c = wave, r = 0; c < n_chunks; c += kSelWaves, ++r) {
    const bool pre = r < kPre;
    // selected by value, field by field (a select between the addresses would put the spans in
    // scratch memory)
    const ckv_chunk_span ld = pre ? sp_first : span_at(chunks, c);
    const bool f = r == 0;
    ckv_chunk_span sp;
    sp.start = pre ? (f ? sp_first.start : sp_last.start) : ld.start;
    sp.length = pre ? (f ? sp_first.length : sp_last.length) : ld.length;
    sp.budget = pre ? (f ? sp_first.budget : sp_last.budget) : ld.budget;
    sp.pooled = pre ? (f ? sp_first.pooled : sp_last.pooled) : ld.pooled;
    const bool ok = sp.start >= 0 && sp.length >= 0 && (int64_t)sp.start + sp.length <= n_tokens;
    float sd = 0.0f, sn = 0.0f;
    if (SUMS && ok) {
      for (int q0 = 0; q0 < sp.length; q0 += kBatch * kWave) {
        float bd[kBatch], bn[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const int q = q0 + j * kWave + lane;
          if (pre && q0 == 0) {
            bd[j] = r == 0 ? bd0[0][j] : bd0[kPre - 1][j];
            bn[j] = r == 0 ? bn0[0][j] : bn0[kPre - 1][j];
          } else {
            bd[j] = q < sp.length ? diff[sp.start + q] : 0.0f;
            bn[j] = q < sp.length ? norm[sp.start + q] : 0.0f;
          }
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          if (q0 + j * kWave + lane < sp.length) {
            sd = sd + bd[j];
            sn = sn + bn[j];
          }
        }
      }
    }
    bool esc = false;
    if constexpr (SUMS) {
      sd = wave_butterfly_sum(sd);
      sn = wave_butterfly_sum(sn);
      const float rel = sd / sn;
      esc = ok && a.has_thr && ((double)rel > a.thr);
      if (lane == 0) {
        a.rel_out[c] = rel;
        a.esc_out[c] = esc ? 1 : 0;
      }
    }
    if (lane == 0 && !ok) atomicAdd(&s_bad_span, 1);
    if (!ok) continue;
    if (esc) {
      set_bit_range(escw, sp.start, sp.start + sp.length, lane);
    } else if (sp.pooled) {
      set_bit_range(poolw, sp.start, sp.start + sp.length, lane);
      if (lane == 0) atomicAdd(&s_budget_req, sp.budget);
    }
  }
  lds_barrier();  // the rel/escalation stores above need no acknowledgement here

  uint32_t key[KPT];  // order-preserving deviation keys of the owned positions
#pragma unroll
  for (int i = 0; i < KPT; ++i) key[i] = dev_key(dv[i]);

  // Phase 2: keep = ~cached | sink | escalated span; candidates = pooled span minus keep.
  // The run [p0, p0 + KPT) lies in mask words p0 / 32 and p0 / 32 + 1 ((p0 % 32) + KPT <= 64):
  // two reads per mask, bit i of the shifted window is position p0 + i.
  uint64_t esc_bits = 0u, pool_bits = 0u;
  if (p0 < n_tokens) {
    const int w0 = p0 >> 5;
    const bool two = w0 + 1 < W;
    esc_bits = ((uint64_t)escw[w0] | (two ? (uint64_t)escw[w0 + 1] << 32 : 0ull)) >> (p0 & 31);
    pool_bits = ((uint64_t)poolw[w0] | (two ? (uint64_t)poolw[w0 + 1] << 32 : 0ull)) >> (p0 & 31);
  }
  uint64_t cand = 0u, kept_static = 0u;
  uint64_t cached_bits = 0u;  // the compaction's count of kept cached positions (the flags die here)
  int mism = 0;  // positions where the histogram's candidate rule and the true one disagree
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int p = p0 + i;
    if (p < n_tokens) {
      const uint32_t f = (fl[i / 4] >> (8 * (i % 4))) & 0xffu;
      cached_bits |= (uint64_t)((f & CKV_POS_CACHED) ? 1u : 0u) << i;
      const bool k = !(f & CKV_POS_CACHED) || (f & CKV_POS_SINK) || ((esc_bits >> i) & 1u);
      kept_static |= (uint64_t)k << i;
      const bool c = !k && ((pool_bits >> i) & 1u);
      if (c) cand |= 1ull << i;
      const bool hc = (f & CKV_POS_CACHED) && !(f & CKV_POS_SINK) && (f & CKV_POS_POOLED);
      mism += hc != c;
    }
  }
  // One scan: candidates, mismatches, and this thread's share of the top-digit histogram (its
  // exclusive prefix = candidates in higher bins than its own).
  const uint32_t gsum = g4.x + g4.y + g4.z + g4.w;
  if (gmine != nullptr) hist_zero4_n(gmine, a.hist_copies);  // leave the histogram zeroed for the next call
  uint64_t scan_tot = 0;
  const uint64_t scan_ex = block_scan_1b_u64((uint64_t)__popcll(cand) | ((uint64_t)mism << 21) |
                                                 ((uint64_t)gsum << 42), slots64[0], scan_tot);
  const int n_cand = (int)(scan_tot & kField);
  const int budget_req = s_budget_req;
  const int budget = max(0, min(budget_req, n_cand));
  bool use_top = ghist != nullptr && ((scan_tot >> 21) & kField) == 0 &&
                 (int)((scan_tot >> 42) & kField) == n_cand;  // uniform

  // Phase 3: radix select of the budget-th largest candidate key.
  uint32_t prefix = 0u, pmask = 0u;
  int need = budget;
  int tie_count = 0;  // candidates with key == T (the last pass's bin of T)
  int first_pass = 0;
  if (budget > 0 && use_top) {
    // the bin holding the budget-th largest key, from the counted histogram
    // (one thread holds it: it walks its four bins, descending, and writes the result once)
    const uint32_t above = (uint32_t)((scan_ex >> 42) & kField);
    if (above < (uint32_t)need && (uint32_t)need <= above + gsum) {
      const uint32_t a3 = above + g4.w, a2 = a3 + g4.z, a1 = a2 + g4.y;  // candidates above bins b0+2, b0+1, b0
      const uint32_t u = (uint32_t)need;
      const int i = u <= a3 ? 0 : u <= a2 ? 1 : u <= a1 ? 2 : 3;  // bin b0 + 3 - i
      const uint32_t before = i == 0 ? above : i == 1 ? a3 : i == 2 ? a2 : a1;
      const uint32_t cnt = i == 0 ? g4.w : i == 1 ? g4.z : i == 2 ? g4.y : g4.x;
      s_top[0] = kTopBins - 4 * tid - 1 - i;
      s_top[1] = need - (int)before;
      s_top[2] = (int)cnt;
    }
    lds_barrier();
    const uint32_t tb = (uint32_t)s_top[0];
    if (tb == 0u || tb == (uint32_t)kTopBins - 1u) {  // uniform: an edge bin is no key prefix
      use_top = false;
    } else {
      prefix = top_bin_prefix(tb);
      pmask = 0xffffffffu << kTopShift;
      need = s_top[1];
      tie_count = s_top[2];
      first_pass = 1;
    }
  }
  // With the top digit known and at most kRankMax candidates in its bin, the bin's candidates
  // are listed in LDS and each ranked against the others by (key descending, position
  // ascending): the first `need` are taken, ties included, in one pass and two barriers instead
  // of three radix passes and a tie scan. The list and the taken-position bitmap use the
  // per-wavefront histograms' storage, idle on this path (the bitmap half was cleared up front).
  const bool ranked = budget > 0 && use_top && tie_count <= kRankMax;  // uniform
  uint64_t take = 0u, tie = 0u;
  if (ranked) {
    uint2* rk = reinterpret_cast<uint2*>(&hist[0][0][0]);  // (key, position), kRankMax entries
    uint32_t* takebits = &hist[1][0][0];                     // one bit per position, W words
    // the candidates in the threshold's (interior) bin: keys with its prefix
    uint64_t inb = 0u;
#pragma unroll
    for (int i = 0; i < KPT; ++i) inb |= (uint64_t)((key[i] & pmask) == prefix) << i;
    inb &= cand;
    const int mine_n = __popcll(inb);
    const int incl = (int)wave_incl_scan((uint32_t)mine_n);
    int wbase = 0;
    if (lane == kWave - 1) wbase = atomicAdd(&s_rk_n, incl);  // one LDS atomic per wavefront
    int off = __builtin_amdgcn_readlane(wbase, kWave - 1) + incl - mine_n;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      if ((inb >> i) & 1ull) {
        if (off < kRankMax) rk[off] = make_uint2(key[i], (uint32_t)(p0 + i));  // the count says so
        ++off;
      }
    }
    lds_barrier();
    // Entry e's rank (entries ahead of it) is counted by the 8 lanes 8e .. 8e + 7, each over
    // every eighth entry (several LDS reads in flight), then summed over the 8 lanes.
    static_assert(kRankMax * 8 <= kSelThreads, "eight threads per listed entry");
    const int m = tie_count;  // the histogram's count of this bin = entries listed
    {
      const int e = tid >> 3, part = tid & 7;
      int ahead = 0;
      uint2 me = make_uint2(0u, 0u);
      if (e < m) {
        me = rk[e];
        // every eighth entry from `part`, all kRankMax / 8 of them read (inside the list's
        // storage) and those past m dropped: no loop condition between the reads
        uint2 o[kRankMax / 8];
#pragma unroll
        for (int k = 0; k < kRankMax / 8; ++k) o[k] = rk[part + 8 * k];
#pragma unroll
        for (int k = 0; k < kRankMax / 8; ++k)
          ahead += (part + 8 * k < m && (o[k].x > me.x || (o[k].x == me.x && o[k].y < me.y))) ? 1 : 0;
      }
      ahead += __shfl_xor(ahead, 1);
      ahead += __shfl_xor(ahead, 2);
      ahead += __shfl_xor(ahead, 4);
      if (e < m && part == 0 && ahead < need) atomicOr(&takebits[me.y >> 5], 1u << (me.y & 31));
    }
    lds_barrier();
    const uint32_t above_bin = prefix | ((1u << kTopShift) - 1u);  // largest key in the bin
    if (p0 < n_tokens) {
      const int w0 = p0 >> 5;
      const uint64_t tb = ((uint64_t)takebits[w0] | (w0 + 1 < W ? (uint64_t)takebits[w0 + 1] << 32 : 0ull)) >> (p0 & 31);
#pragma unroll
      for (int i = 0; i < KPT; ++i) take |= (uint64_t)(key[i] > above_bin) << i;
      take = (take & cand) | (inb & tb);
    }
  }
  // After the top digit, few candidates share its bin: one shared histogram per pass (its own
  // buffer, cleared up front) and one LDS barrier. Otherwise per-wavefront histograms folded
  // after a second barrier, so hot bins do not serialise LDS atomics.
  const bool light = use_top && tie_count <= kLightPass;
  if (budget > 0 && !ranked) {
    // passes over the bits below the known prefix: 8, 8, 8, 8 from bit 31, or, after the
    // top-digit histogram, 8, 8 and 1 from bit 16
    static_assert(kTopShift == 17, "pass layout below the top digit");
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {
      if (pass < first_pass) continue;
      const int shift = use_top ? (pass == 1 ? 9 : pass == 2 ? 1 : 0) : 24 - 8 * pass;
      const uint32_t dmask = (use_top && pass == 3) ? 1u : 255u;
      uint32_t(*h)[256] = hist[pass & 1];
      uint32_t* hmine = light ? hl[pass > 0 ? pass - 1 : 0] : h[wave];
      // Run-length aggregate equal digits within the thread: in the high passes almost every key
      // shares one or two digits, and unaggregated LDS atomics would serialize.
      uint32_t run_digit = 0u, run_count = 0u;
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        if (((cand >> i) & 1ull) && (key[i] & pmask) == prefix) {
          const uint32_t d = (key[i] >> shift) & dmask;
          if (run_count != 0u && d != run_digit) {
            atomicAdd(&hmine[run_digit], run_count);
            run_count = 0u;
          }
          run_digit = d;
          ++run_count;
        }
      }
      if (run_count != 0u) atomicAdd(&hmine[run_digit], run_count);
      if (light) {
        lds_barrier();
      } else {
        lds_barrier();
        if (tid < 256) {  // fold the per-wavefront histograms into h[0]
          uint32_t t = 0;
#pragma unroll
          for (int w = 0; w < kSelWaves; ++w) t += h[w][tid];
          h[0][tid] = t;
        } else {  // the other buffer was last read before this pass's barrier: clear it for pass+1
          uint32_t* o = &hist[(pass + 1) & 1][0][0];
          for (int b = tid - 256; b < kSelWaves * 256; b += kSelThreads - 256) o[b] = 0u;
        }
        lds_barrier();
      }
      const uint32_t* hsum = light ? hmine : h[0];
      // every wavefront finds the digit: lane l owns digits 255-4l .. 252-4l (descending)
      uint32_t h4[4];
      uint32_t local_sum = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        h4[i] = hsum[255 - (lane * 4 + i)];
        local_sum += h4[i];
      }
      const uint32_t incl = wave_incl_scan(local_sum);
      uint32_t above = incl - local_sum;
      int my_digit = -1;
      uint32_t my_above = 0u;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (above < (uint32_t)need && (uint32_t)need <= above + h4[i]) {
          my_digit = 255 - (lane * 4 + i);
          my_above = above;
        }
        above += h4[i];
      }
      const uint64_t found = __ballot(my_digit >= 0);
      const int src = found ? (int)__ffsll((unsigned long long)found) - 1 : 0;  // wavefront-uniform
      const int digit = __builtin_amdgcn_readlane(my_digit, src);
      need -= (int)__builtin_amdgcn_readlane((int)my_above, src);
      prefix |= (uint32_t)digit << shift;
      pmask |= dmask << shift;
      if (pass == 3) tie_count = (int)hsum[digit];
    }
  }
  const uint32_t T = prefix;

  // Phase 4: take key > T and the first `need` ties at T in token order, then compact.
  if (budget > 0 && !ranked) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      if ((cand >> i) & 1ull) {
        take |= (uint64_t)(key[i] > T) << i;
        tie |= (uint64_t)(key[i] == T) << i;
      }
    }
  }
  if (!ranked && need < tie_count) {  // uniform: only then do ties need ranking (lowest positions first)
    int tie_total = 0;
    int tie_rank = block_scan_1b(__popcll(tie), slots[1], tie_total);
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      if ((tie >> i) & 1ull) {
        take |= (uint64_t)(tie_rank < need) << i;
        ++tie_rank;
      }
    }
  } else {
    take |= tie;  // every tie at T is taken (none when ranked)
  }
  const uint64_t kept = kept_static | take;
  if constexpr (kLateLocal) {  // the local indices, as the first loads took them
    if (vec_ok && wave_end <= n_tokens) {  // uniform
#pragma unroll
      for (int i0 = 0; i0 < KPT; i0 += 4) {
        const int4 l = *(const int4*)(local + p0 + i0);
        lv[i0] = l.x;
        lv[i0 + 1] = l.y;
        lv[i0 + 2] = l.z;
        lv[i0 + 3] = l.w;
      }
    } else if (wave_end <= n_tokens) {  // uniform
      const int32_t* l = local + p0;
#pragma unroll
      for (int i = 0; i < KPT; ++i) lv[i] = l[i];
    } else if (__builtin_amdgcn_readfirstlane(wave * kWave * KPT) < n_tokens) {  // uniform
#pragma unroll
      for (int i = 0; i < KPT; ++i) lv[i] = ld_at(local, clamp_pos(p0 + i, n_tokens));
    } else {
#pragma unroll
      for (int i = 0; i < KPT; ++i) lv[i] = 0;
    }
  }
  // One scan for three counts in 21-bit fields (each total <= n_tokens < 2^21): kept positions
  // (the rank of each), kept cached positions, kept positions absent from the active set.
  uint64_t mine = (uint64_t)__popcll(kept) + ((uint64_t)__popcll(kept & cached_bits) << 21);
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    if ((kept >> i) & 1ull) mine += (uint64_t)(lv[i] < 0) << 42;
  }
  uint64_t all = 0;
  int rank = (int)(block_scan_1b_u64(mine, slots64[1], all) & kField);
  const int n_keep = (int)(all & kField);
  const int sel_cached = (int)((all >> 21) & kField);
  const int uncomputed = (int)((all >> 42) & kField);
  // keep_abs / keep_local go out through LDS, a window of kStage ranks at a time (the radix
  // histograms' space, no longer read): each thread puts its kept positions at their ranks, then
  // the workgroup stores the window in rank order, two entries per 16-byte store, instead of
  // every lane storing 8 bytes at its own rank
  {
    int2* stage = reinterpret_cast<int2*>(&hist[0][0][0]);
    constexpr int kStage = (int)(sizeof(hist) / sizeof(int2));
    const bool st16_ok = (((uintptr_t)a.keep_abs | (uintptr_t)a.keep_local) % 16) == 0;
    for (int w0 = 0; w0 < n_keep; w0 += kStage) {  // uniform
      __syncthreads();  // the histograms' last reads, or the previous window's
      int r = rank;
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        if ((kept >> i) & 1ull) {
          if (r >= w0 && r < w0 + kStage) stage[r - w0] = make_int2(p0 + i, lv[i] < 0 ? 0 : lv[i]);
          ++r;
        }
      }
      __syncthreads();
      const int cnt = min(kStage, n_keep - w0);
      for (int j = 2 * tid; j < cnt; j += 2 * kSelThreads) {
        const int2 e0 = stage[j];
        if (st16_ok && j + 1 < cnt) {
          const int2 e1 = stage[j + 1];
          *(longlong2*)(a.keep_abs + w0 + j) = make_longlong2(e0.x, e1.x);
          *(longlong2*)(a.keep_local + w0 + j) = make_longlong2(e0.y, e1.y);
        } else {
          a.keep_abs[w0 + j] = e0.x;
          a.keep_local[w0 + j] = e0.y;
          if (j + 1 < cnt) {
            const int2 e1 = stage[j + 1];
            a.keep_abs[w0 + j + 1] = e1.x;
            a.keep_local[w0 + j + 1] = e1.y;
          }
        }
      }
    }
  }
  // four positions at a time: the four keep_rank entries
#pragma unroll
  for (int i0 = 0; i0 < KPT; i0 += 4) {
    int kr[4];  // keep_rank of positions i0 .. i0 + 3
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = i0 + j;
      const bool k = i < KPT && ((kept >> i) & 1ull);
      kr[j] = k ? rank : -1;
      if (k) ++rank;
    }
    if (keep_rank != nullptr) {
      if (vec_ok && p0 + i0 + 4 <= n_tokens) {
        *(int4*)(keep_rank + p0 + i0) = make_int4(kr[0], kr[1], kr[2], kr[3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (i0 + j < KPT && p0 + i0 + j < n_tokens) keep_rank[p0 + i0 + j] = kr[j];
      }
    }
  }
  if (tid == 0) {
    int32_t* counts = a.counts;
    counts[CKV_COUNT_KEEP] = n_keep;
    counts[CKV_COUNT_SELECTED_CACHED] = sel_cached;
    counts[CKV_COUNT_BUDGET] = budget;
    counts[CKV_COUNT_CANDIDATES] = n_cand;
    counts[CKV_COUNT_UNCOMPUTED] = uncomputed;
    counts[CKV_COUNT_BUDGET_REQUESTED] = budget_req;
    counts[6] = s_bad_span;
    counts[7] = (use_top ? 1 : 0) | (ranked ? 2 : 0);
  }
}

}  // namespace ckv
