// Layer-1 selection: per-chunk relative deviation and escalation, pooled budget, pooled top-k
// with forced sinks, and compaction of the new active set — one single-workgroup launch, so
// the host never synchronises inside the layer loop.
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
// this kernel fixes it: larger diff first, then lower token index (NaN ranks last).
//
// Design (gfx950): 1024 threads (16 wavefronts). keep/pool live as N-bit masks in LDS.
// Chunk sums: one wavefront per chunk, lane-strided fp32 partials + xor butterfly (the order
// the oracle restates). Top-k: MSB-first radix select over order-preserving 32-bit keys, four
// 8-bit passes, which yields the exact threshold key T and how many ties at T to take; then
// key > T plus the lowest-index ties are taken and the kept positions compacted in token order.
// Up to 33792 tokens (select_reg_kernel) each thread owns a contiguous run of <= 33 positions
// whose keys stay in registers for all passes, histograms are per wavefront (no atomic pile-up
// on the few hot bins), and ties and compaction need one workgroup scan each. Larger requests
// use select_kernel, which re-reads keys from L2 in every pass.
#include "ckv_common.hpp"

namespace ckv {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / kWave;

// Order-preserving key of a deviation: larger float -> larger key; -0 == +0; NaN -> 0.
__device__ __forceinline__ uint32_t dev_key(float f) {
  if (f != f) return 0u;
  if (f == 0.0f) f = 0.0f;
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

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

// Phases shared by both selection kernels: keep = ~cached | sink and pool = 0 as LDS
// bitmasks, then per-chunk relative deviation, escalation and requested budget.
__device__ __forceinline__ void select_prologue(const float* __restrict__ diff, const float* __restrict__ norm,
                                                const uint8_t* __restrict__ flags, int n_tokens,
                                                const ckv_chunk_span* __restrict__ chunks, int n_chunks, int has_thr,
                                                double thr, float* __restrict__ rel_out, uint8_t* __restrict__ esc_out,
                                                uint32_t* keepw, uint32_t* poolw, int W, int* s_budget_req,
                                                int* s_bad_span) {
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  if (tid == 0) {
    *s_budget_req = 0;
    *s_bad_span = 0;
  }
  // Each wavefront covers 64 positions = 2 mask words per step.
  for (int base = wave * kWave; base < W * 32; base += kSelThreads) {
    const int p = base + lane;
    bool k = false;
    if (p < n_tokens) {
      const uint8_t f = flags[p];
      k = !(f & CKV_POS_CACHED) || (f & CKV_POS_SINK);
    }
    const uint64_t m = __ballot(k);
    if (lane == 0) {
      keepw[base >> 5] = (uint32_t)m;
      poolw[base >> 5] = 0u;
    } else if (lane == 32 && ((base >> 5) + 1) < W) {
      keepw[(base >> 5) + 1] = (uint32_t)(m >> 32);
      poolw[(base >> 5) + 1] = 0u;
    }
  }
  __syncthreads();
  for (int c = wave; c < n_chunks; c += kSelWaves) {
    const ckv_chunk_span sp = chunks[c];
    const bool ok = sp.start >= 0 && sp.length >= 0 && (int64_t)sp.start + sp.length <= n_tokens;
    float sd = 0.0f, sn = 0.0f;
    if (ok) {
      for (int q = lane; q < sp.length; q += kWave) {
        sd = sd + diff[sp.start + q];
        sn = sn + norm[sp.start + q];
      }
    }
    sd = wave_butterfly_sum(sd);
    sn = wave_butterfly_sum(sn);
    const float rel = sd / sn;
    const bool esc = ok && has_thr && ((double)rel > thr);
    if (lane == 0) {
      rel_out[c] = rel;
      esc_out[c] = esc ? 1 : 0;
      if (!ok) atomicAdd(s_bad_span, 1);
    }
    if (!ok) continue;
    if (esc) {
      set_bit_range(keepw, sp.start, sp.start + sp.length, lane);
    } else if (sp.pooled) {
      set_bit_range(poolw, sp.start, sp.start + sp.length, lane);
      if (lane == 0) atomicAdd(s_budget_req, sp.budget);
    }
  }
  __syncthreads();
}

// Inclusive wavefront scan + exclusive workgroup scan of one int per thread.
__device__ __forceinline__ int block_excl_scan(int v, int* wave_tot, int& total) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  int x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  if (lane == kWave - 1) wave_tot[wave] = x;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    const int t = wave_tot[w];
    before += (w < wave) ? t : 0;
    all += t;
  }
  __syncthreads();
  total = all;
  return before + x - v;
}

// Exclusive workgroup scan of one int per thread with ONE barrier: each call must get its own
// `slots` array (kSelWaves ints) that no call in flight since the previous barrier reads.
__device__ __forceinline__ int block_scan_1b(int v, int* slots, int& total) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  int x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  if (lane == kWave - 1) slots[wave] = x;
  __syncthreads();
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
  uint64_t x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const uint64_t y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  if (lane == kWave - 1) slots[wave] = x;
  __syncthreads();
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

// Register-resident selection for n_tokens <= KPT * 1024: thread t owns positions
// [t*KPT, (t+1)*KPT); their keys stay in registers through the four radix passes.
// Barrier budget: chunk phase 2, candidate count 1, 2 per radix pass (double-buffered
// histograms, every wavefront derives the digit itself), tie scan 1, compaction scan 1, counts 2.
template <int KPT>
__global__ __launch_bounds__(kSelThreads) void select_reg_kernel(
    const float* __restrict__ diff, const float* __restrict__ norm, const uint8_t* __restrict__ flags,
    const int32_t* __restrict__ local, int n_tokens, const ckv_chunk_span* __restrict__ chunks, int n_chunks,
    int has_thr, double thr, int64_t* __restrict__ keep_abs, int64_t* __restrict__ keep_local,
    int32_t* __restrict__ keep_rank, float* __restrict__ rel_out, uint8_t* __restrict__ esc_out,
    int32_t* __restrict__ counts) {
  static_assert(KPT <= 33, "a run of KPT positions spans at most two mask words and one 64-bit word");
  constexpr int kBatch = 8;            // chunk-sum loads in flight per lane
  extern __shared__ uint32_t masks[];  // esc[W], pool[W]: spans of escalated / pooled chunks
  __shared__ uint32_t hist[2][kSelWaves][256];
  __shared__ int slots[2][kSelWaves];
  __shared__ uint64_t slots64[kSelWaves];
  __shared__ int s_budget_req, s_bad_span;

  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int W = (n_tokens + 31) >> 5;
  uint32_t* escw = masks;
  uint32_t* poolw = masks + W;

  // Phase 0, no barrier before it: every global load this workgroup can issue up front.
  const int p0 = tid * KPT;
  constexpr int kFlagWords = (KPT + 3) / 4;
  uint32_t key[KPT];        // order-preserving deviation keys of the owned positions
  uint32_t fl[kFlagWords];  // their flag bytes, four per register
  int lv[KPT];              // their local indices (the compaction's keep_local)
#pragma unroll
  for (int w = 0; w < kFlagWords; ++w) fl[w] = 0u;
  // A thread's run is contiguous, so lanes are KPT elements apart: with KPT % 4 == 0 and aligned
  // arrays, 16-byte (4-byte for flags) loads cut the load instructions and cache-line requests
  // four-fold.
  const bool vec_ok = KPT % 4 == 0 && (((uintptr_t)diff | (uintptr_t)local) % 16 == 0) &&
                      ((uintptr_t)flags % 4 == 0) && (keep_rank == nullptr || (uintptr_t)keep_rank % 16 == 0);
#pragma unroll
  for (int i0 = 0; i0 < KPT; i0 += 4) {
    if (vec_ok && p0 + i0 + 4 <= n_tokens) {
      const float4 d = *(const float4*)(diff + p0 + i0);
      const int4 l = *(const int4*)(local + p0 + i0);
      const uint32_t f = *(const uint32_t*)(flags + p0 + i0);
      key[i0] = dev_key(d.x);
      key[i0 + 1] = dev_key(d.y);
      key[i0 + 2] = dev_key(d.z);
      key[i0 + 3] = dev_key(d.w);
      lv[i0] = l.x;
      lv[i0 + 1] = l.y;
      lv[i0 + 2] = l.z;
      lv[i0 + 3] = l.w;
      fl[i0 / 4] = f;  // i0 % 4 == 0 here: the word holds flags i0 .. i0 + 3
    } else {
#pragma unroll
      for (int i = i0; i < i0 + 4 && i < KPT; ++i) {
        const int p = p0 + i;
        key[i] = p < n_tokens ? dev_key(diff[p]) : 0u;
        lv[i] = p < n_tokens ? local[p] : 0;
        if (p < n_tokens) fl[i / 4] |= (uint32_t)flags[p] << (8 * (i % 4));
      }
    }
  }
  // this wavefront's first chunk: span and the first batch of its deviations
  ckv_chunk_span sp0{0, 0, 0, 0};
  float bd0[kBatch], bn0[kBatch];
  if (wave < n_chunks) {
    sp0 = chunks[wave];
    const bool ok0 = sp0.start >= 0 && sp0.length >= 0 && (int64_t)sp0.start + sp0.length <= n_tokens;
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int q = j * kWave + lane;
      bd0[j] = (ok0 && q < sp0.length) ? diff[sp0.start + q] : 0.0f;
      bn0[j] = (ok0 && q < sp0.length) ? norm[sp0.start + q] : 0.0f;
    }
  }
  if (tid == 0) {
    s_budget_req = 0;
    s_bad_span = 0;
  }
  for (int w = tid; w < 2 * W; w += kSelThreads) masks[w] = 0u;
  for (int b = tid; b < 2 * kSelWaves * 256; b += kSelThreads) (&hist[0][0][0])[b] = 0u;
  lds_barrier();  // the loads above stay in flight

  // Phase 1: per-chunk rel / escalation / budget, one wavefront per chunk, summed in the
  // contract's order (lane-strided, ascending, then the xor butterfly).
  for (int c = wave; c < n_chunks; c += kSelWaves) {
    const ckv_chunk_span sp = c == wave ? sp0 : chunks[c];
    const bool ok = sp.start >= 0 && sp.length >= 0 && (int64_t)sp.start + sp.length <= n_tokens;
    float sd = 0.0f, sn = 0.0f;
    if (ok) {
      for (int q0 = 0; q0 < sp.length; q0 += kBatch * kWave) {
        float bd[kBatch], bn[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const int q = q0 + j * kWave + lane;
          if (c == wave && q0 == 0) {
            bd[j] = bd0[j];
            bn[j] = bn0[j];
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
    sd = wave_butterfly_sum(sd);
    sn = wave_butterfly_sum(sn);
    const float rel = sd / sn;
    const bool esc = ok && has_thr && ((double)rel > thr);
    if (lane == 0) {
      rel_out[c] = rel;
      esc_out[c] = esc ? 1 : 0;
      if (!ok) atomicAdd(&s_bad_span, 1);
    }
    if (!ok) continue;
    if (esc) {
      set_bit_range(escw, sp.start, sp.start + sp.length, lane);
    } else if (sp.pooled) {
      set_bit_range(poolw, sp.start, sp.start + sp.length, lane);
      if (lane == 0) atomicAdd(&s_budget_req, sp.budget);
    }
  }
  lds_barrier();  // the rel/escalation stores above need no acknowledgement here

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
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int p = p0 + i;
    if (p < n_tokens) {
      const uint32_t f = (fl[i / 4] >> (8 * (i % 4))) & 0xffu;
      const bool k = !(f & CKV_POS_CACHED) || (f & CKV_POS_SINK) || ((esc_bits >> i) & 1u);
      kept_static |= (uint64_t)k << i;
      if (!k && ((pool_bits >> i) & 1u)) cand |= 1ull << i;
    }
  }
  int n_cand = 0;
  block_scan_1b(__popcll(cand), slots[0], n_cand);
  const int budget_req = s_budget_req;
  const int budget = max(0, min(budget_req, n_cand));

  // Phase 3: radix select of the budget-th largest candidate key.
  uint32_t prefix = 0u, pmask = 0u;
  int need = budget;
  int tie_count = 0;  // candidates with key == T (the last pass's bin of T)
  if (budget > 0) {
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {
      const int shift = 24 - 8 * pass;
      uint32_t(*h)[256] = hist[pass & 1];
      // Run-length aggregate equal digits within the thread: in the high passes almost every key
      // shares one or two digits, and unaggregated LDS atomics would serialize.
      uint32_t run_digit = 0u, run_count = 0u;
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        if (((cand >> i) & 1ull) && (key[i] & pmask) == prefix) {
          const uint32_t d = (key[i] >> shift) & 255u;
          if (run_count != 0u && d != run_digit) {
            atomicAdd(&h[wave][run_digit], run_count);
            run_count = 0u;
          }
          run_digit = d;
          ++run_count;
        }
      }
      if (run_count != 0u) atomicAdd(&h[wave][run_digit], run_count);
      __syncthreads();
      if (tid < 256) {  // fold the per-wavefront histograms into h[0]
        uint32_t t = 0;
#pragma unroll
        for (int w = 0; w < kSelWaves; ++w) t += h[w][tid];
        h[0][tid] = t;
      } else {  // the other buffer was last read before this pass's barrier: clear it for pass+1
        uint32_t* o = &hist[(pass + 1) & 1][0][0];
        for (int b = tid - 256; b < kSelWaves * 256; b += kSelThreads - 256) o[b] = 0u;
      }
      __syncthreads();
      // every wavefront finds the digit: lane l owns digits 255-4l .. 252-4l (descending)
      uint32_t h4[4];
      uint32_t local_sum = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        h4[i] = h[0][255 - (lane * 4 + i)];
        local_sum += h4[i];
      }
      uint32_t incl = local_sum;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const uint32_t t = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += t;
      }
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
      const int src = found ? (int)__ffsll((unsigned long long)found) - 1 : 0;
      const int digit = __shfl(my_digit, src, kWave);
      need -= (int)__shfl(my_above, src, kWave);
      prefix |= (uint32_t)digit << shift;
      pmask |= 255u << shift;
      if (pass == 3) tie_count = (int)h[0][digit];
    }
  }
  const uint32_t T = prefix;

  // Phase 4: take key > T and the first `need` ties at T in token order, then compact.
  uint64_t take = 0u, tie = 0u;
  if (budget > 0) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      if ((cand >> i) & 1ull) {
        take |= (uint64_t)(key[i] > T) << i;
        tie |= (uint64_t)(key[i] == T) << i;
      }
    }
  }
  if (need < tie_count) {  // uniform: only then do ties need ranking (lowest positions first)
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
    take |= tie;  // every tie at T is taken
  }
  const uint64_t kept = kept_static | take;
  // One scan for three counts in 21-bit fields (each total <= n_tokens < 2^21): kept positions
  // (the rank of each), kept cached positions, kept positions absent from the active set.
  uint64_t mine = (uint64_t)__popcll(kept);
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    if ((kept >> i) & 1ull) {
      mine += (((fl[i / 4] >> (8 * (i % 4))) & CKV_POS_CACHED) ? 1ull : 0ull) << 21;
      mine += (uint64_t)(lv[i] < 0) << 42;
    }
  }
  uint64_t all = 0;
  int rank = (int)(block_scan_1b_u64(mine, slots64, all) & 0x1fffffu);
  const int n_keep = (int)(all & 0x1fffffu);
  const int sel_cached = (int)((all >> 21) & 0x1fffffu);
  const int uncomputed = (int)((all >> 42) & 0x1fffffu);
  int kr[KPT];  // keep_rank of the owned positions
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    kr[i] = ((kept >> i) & 1ull) ? rank : -1;
    if ((kept >> i) & 1ull) {
      const int p = p0 + i;
      keep_abs[rank] = p;
      keep_local[rank] = lv[i] < 0 ? 0 : lv[i];
      ++rank;
    }
  }
  if (keep_rank != nullptr) {
#pragma unroll
    for (int i0 = 0; i0 < KPT; i0 += 4) {
      if (vec_ok && p0 + i0 + 4 <= n_tokens) {
        *(int4*)(keep_rank + p0 + i0) = make_int4(kr[i0], kr[i0 + 1], kr[i0 + 2], kr[i0 + 3]);
      } else {
#pragma unroll
        for (int i = i0; i < i0 + 4 && i < KPT; ++i)
          if (p0 + i < n_tokens) keep_rank[p0 + i] = kr[i];
      }
    }
  }
  if (tid == 0) {
    counts[CKV_COUNT_KEEP] = n_keep;
    counts[CKV_COUNT_SELECTED_CACHED] = sel_cached;
    counts[CKV_COUNT_BUDGET] = budget;
    counts[CKV_COUNT_CANDIDATES] = n_cand;
    counts[CKV_COUNT_UNCOMPUTED] = uncomputed;
    counts[CKV_COUNT_BUDGET_REQUESTED] = budget_req;
    counts[6] = s_bad_span;
    counts[7] = 0;
  }
}

// Selection for any n_tokens <= CKV_SELECT_MAX_TOKENS: keys are re-read from global memory
// (L2) in every pass and positions are walked in 1024-wide tiles.
__global__ __launch_bounds__(kSelThreads) void select_kernel(
    const float* __restrict__ diff, const float* __restrict__ norm, const uint8_t* __restrict__ flags,
    const int32_t* __restrict__ local, int n_tokens, const ckv_chunk_span* __restrict__ chunks,
    int n_chunks, int has_thr, double thr, int64_t* __restrict__ keep_abs,
    int64_t* __restrict__ keep_local, int32_t* __restrict__ keep_rank, float* __restrict__ rel_out,
    uint8_t* __restrict__ esc_out, int32_t* __restrict__ counts) {
  extern __shared__ uint32_t masks[];  // keep[W], pool[W]
  __shared__ uint32_t hist[256];
  __shared__ int wave_tot[kSelWaves];
  __shared__ int s_budget_req, s_bad_span, s_digit, s_above;

  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int W = (n_tokens + 31) >> 5;
  uint32_t* keepw = masks;
  uint32_t* poolw = masks + W;

  if (tid == 0) {
    s_budget_req = 0;
    s_bad_span = 0;
  }
  // keep = ~cached | sink; pool = 0. Each wavefront covers 64 positions = 2 words per step.
  for (int base = wave * kWave; base < W * 32; base += kSelThreads) {
    const int p = base + lane;
    bool k = false;
    if (p < n_tokens) {
      const uint8_t f = flags[p];
      k = !(f & CKV_POS_CACHED) || (f & CKV_POS_SINK);
    }
    const uint64_t m = __ballot(k);
    if (lane == 0) {
      keepw[base >> 5] = (uint32_t)m;
      poolw[base >> 5] = 0u;
    } else if (lane == 32 && ((base >> 5) + 1) < W) {
      keepw[(base >> 5) + 1] = (uint32_t)(m >> 32);
      poolw[(base >> 5) + 1] = 0u;
    }
  }
  __syncthreads();

  // Per-chunk relative deviation, escalation and budget (one wavefront per chunk).
  for (int c = wave; c < n_chunks; c += kSelWaves) {
    const ckv_chunk_span sp = chunks[c];
    const bool ok = sp.start >= 0 && sp.length >= 0 && (int64_t)sp.start + sp.length <= n_tokens;
    float sd = 0.0f, sn = 0.0f;
    if (ok) {
      for (int q = lane; q < sp.length; q += kWave) {
        sd = sd + diff[sp.start + q];
        sn = sn + norm[sp.start + q];
      }
    }
    sd = wave_butterfly_sum(sd);
    sn = wave_butterfly_sum(sn);
    const float rel = sd / sn;
    const bool esc = ok && has_thr && ((double)rel > thr);
    if (lane == 0) {
      rel_out[c] = rel;
      esc_out[c] = esc ? 1 : 0;
      if (!ok) atomicAdd(&s_bad_span, 1);
    }
    if (!ok) continue;
    if (esc) {
      set_bit_range(keepw, sp.start, sp.start + sp.length, lane);
    } else if (sp.pooled) {
      set_bit_range(poolw, sp.start, sp.start + sp.length, lane);
      if (lane == 0) atomicAdd(&s_budget_req, sp.budget);
    }
  }
  __syncthreads();

  // Candidates = pool & ~keep; budget = min(requested, #candidates).
  int my_cand = 0;
  for (int w = tid; w < W; w += kSelThreads) my_cand += __popc(poolw[w] & ~keepw[w]);
  int n_cand = 0;
  {
    // integer block sum via the count helper is not applicable (counts > 1 per thread)
    int v = my_cand;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
    if (lane == 0) wave_tot[wave] = v;
    __syncthreads();
    for (int w = 0; w < kSelWaves; ++w) n_cand += wave_tot[w];
    __syncthreads();
  }
  const int budget_req = s_budget_req;
  const int budget = max(0, min(budget_req, n_cand));

  // Radix select of the budget-th largest key among candidates.
  uint32_t prefix = 0u, pmask = 0u;
  int need = budget;  // after the passes: ties at T still to take
  if (budget > 0) {
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int b = tid; b < 256; b += kSelThreads) hist[b] = 0u;
      __syncthreads();
      for (int p = tid; p < n_tokens; p += kSelThreads) {
        if (bit_of(poolw, p) && !bit_of(keepw, p)) {
          const uint32_t key = dev_key(diff[p]);
          if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
        }
      }
      __syncthreads();
      if (wave == 0) {
        // lane l owns digits 255-4l .. 252-4l (descending); inclusive scan from the top.
        uint32_t h4[4];
        uint32_t local_sum = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          h4[i] = hist[255 - (lane * 4 + i)];
          local_sum += h4[i];
        }
        uint32_t incl = local_sum;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
          const uint32_t t = __shfl_up(incl, off, kWave);
          if (lane >= off) incl += t;
        }
        uint32_t above = incl - local_sum;  // keys with a larger digit than this lane's first
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (above < (uint32_t)need && (uint32_t)need <= above + h4[i]) {
            s_digit = 255 - (lane * 4 + i);
            s_above = (int)above;
          }
          above += h4[i];
        }
      }
      __syncthreads();
      need -= s_above;
      prefix |= (uint32_t)s_digit << shift;
      pmask |= 255u << shift;
      __syncthreads();
    }
  }
  const uint32_t T = prefix;

  // Final pass in token order: take key > T and the first `need` ties, then compact keep.
  int tie_carry = 0, keep_carry = 0, my_cached = 0, my_bad = 0;
  for (int base = 0; base < n_tokens; base += kSelThreads) {
    const int p = base + tid;
    const bool valid = p < n_tokens;
    bool take = false, tie = false;
    if (valid && budget > 0 && bit_of(poolw, p) && !bit_of(keepw, p)) {
      const uint32_t key = dev_key(diff[p]);
      take = key > T;
      tie = key == T;
    }
    int tie_total = 0;
    const int tie_rank = block_excl_count(tie, wave_tot, tie_total) + tie_carry;
    tie_carry += tie_total;
    take = take || (tie && tie_rank < need);
    const bool kept = valid && (bit_of(keepw, p) || take);
    int keep_total = 0;
    const int rank = block_excl_count(kept, wave_tot, keep_total) + keep_carry;
    keep_carry += keep_total;
    if (valid && keep_rank != nullptr) keep_rank[p] = kept ? rank : -1;
    if (kept) {
      const int l = local[p];
      keep_abs[rank] = p;
      keep_local[rank] = l < 0 ? 0 : l;
      my_bad += l < 0;
      my_cached += (flags[p] & CKV_POS_CACHED) ? 1 : 0;
    }
  }

  // Reduce the per-thread counters.
  int v1 = my_cached, v2 = my_bad;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    v1 += __shfl_xor(v1, m, kWave);
    v2 += __shfl_xor(v2, m, kWave);
  }
  __shared__ int red1[kSelWaves], red2[kSelWaves];
  if (lane == 0) {
    red1[wave] = v1;
    red2[wave] = v2;
  }
  __syncthreads();
  if (tid == 0) {
    int c1 = 0, c2 = 0;
    for (int w = 0; w < kSelWaves; ++w) {
      c1 += red1[w];
      c2 += red2[w];
    }
    counts[CKV_COUNT_KEEP] = keep_carry;
    counts[CKV_COUNT_SELECTED_CACHED] = c1;
    counts[CKV_COUNT_BUDGET] = budget;
    counts[CKV_COUNT_CANDIDATES] = n_cand;
    counts[CKV_COUNT_UNCOMPUTED] = c2;
    counts[CKV_COUNT_BUDGET_REQUESTED] = budget_req;
    counts[6] = s_bad_span;
    counts[7] = 0;
  }
}

}  // namespace ckv

extern "C" int32_t ckv_select(const float* diff, const float* norm, const uint8_t* pos_flags,
                              const int32_t* local, int32_t n_tokens, const ckv_chunk_span* chunks,
                              int32_t n_chunks, int32_t has_threshold, double escalate_threshold,
                              int64_t* keep_abs, int64_t* keep_local, int32_t* keep_rank, float* rel_dev,
                              uint8_t* escalated, int32_t* counts, void* stream) {
  using namespace ckv;
  if (diff == nullptr || norm == nullptr || pos_flags == nullptr || local == nullptr || keep_abs == nullptr ||
      keep_local == nullptr || counts == nullptr || n_tokens < 0 || n_chunks < 0)
    return CKV_ERR_INVALID_ARGUMENT;
  if (n_chunks > 0 && (chunks == nullptr || rel_dev == nullptr || escalated == nullptr))
    return CKV_ERR_INVALID_ARGUMENT;
  if (n_tokens > CKV_SELECT_MAX_TOKENS) return CKV_ERR_TOO_LARGE;
  const int W = (n_tokens + 31) / 32;
  const size_t lds = (size_t)(W > 0 ? W : 1) * 2 * sizeof(uint32_t);
  hipStream_t st = (hipStream_t)stream;
  const int kpt = (n_tokens + kSelThreads - 1) / kSelThreads;
#define CKV_SEL_REG(K)                                                                                        \
  if (kpt <= K) {                                                                                             \
    hipLaunchKernelGGL(select_reg_kernel<K>, dim3(1), dim3(kSelThreads), lds, st, diff, norm, pos_flags, local, \
                       (int)n_tokens, chunks, (int)n_chunks, (int)(has_threshold != 0), escalate_threshold,      \
                       keep_abs, keep_local, keep_rank, rel_dev, escalated, counts);                            \
    CKV_RETURN_IF_LAUNCH_FAILED();                                                                            \
    return CKV_OK;                                                                                            \
  }
  CKV_SEL_REG(4)
  CKV_SEL_REG(8)
  CKV_SEL_REG(12)
  CKV_SEL_REG(16)
  CKV_SEL_REG(24)
  CKV_SEL_REG(33)
#undef CKV_SEL_REG
  hipLaunchKernelGGL(select_kernel, dim3(1), dim3(kSelThreads), lds, st, diff, norm, pos_flags, local, (int)n_tokens,
                     chunks, (int)n_chunks, (int)(has_threshold != 0), escalate_threshold, keep_abs, keep_local,
                     keep_rank, rel_dev, escalated, counts);
  CKV_RETURN_IF_LAUNCH_FAILED();
  return CKV_OK;
}
