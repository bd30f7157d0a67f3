// Layer-1 selection entry point (ckv_select): per-chunk relative deviation and escalation,
// pooled budget, pooled top-k with forced sinks, and compaction of the new active set — one
// single-workgroup launch, so the host never synchronises inside the layer loop. The semantics
// and the register-resident algorithm are in select_common.hpp (shared with the fused
// ckv_deviation_select); requests above 33792 tokens use select_kernel below, which re-reads
// keys from L2 in every pass.
#include "launch.hpp"
#include "select_slices.hpp"

namespace ckv {

// Register-resident selection (select_run) for n_tokens <= KPT * 1024; ghist (may be NULL) is a
// top_bin candidate histogram counted by an earlier launch, left zeroed. Without a threshold
// (SUMS = false) workgroup 0 selects and the others compute the chunks' rel_dev, one wavefront
// per chunk, beside it.
// The pointers and sizes the first loads use lead the argument list: the library preloads the
// first 16 argument dwords into SGPRs, but only up to the first argument passed by reference
// (the SelectArgs struct), and every other argument takes a scalar load at wave start.
template <int KPT, bool SUMS>
__global__ __launch_bounds__(kSelThreads) void select_reg_kernel(const float* diff, const uint8_t* flags,
                                                                 const int32_t* local, uint32_t* ghist,
                                                                 const ckv_chunk_span* chunks, int n_tokens,
                                                                 int n_chunks, int hist_copies, SelectArgs a) {
  extern __shared__ uint32_t masks[];  // esc[W], pool[W]: spans of escalated / pooled chunks
  a.diff = diff;
  a.flags = flags;
  a.local = local;
  a.chunks = chunks;
  a.n_tokens = n_tokens;
  a.n_chunks = n_chunks;
  a.hist_copies = hist_copies;
  if (!SUMS && blockIdx.x > 0) {
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
    for (int c = ((int)blockIdx.x - 1) * kSelWaves + wave; c < a.n_chunks; c += ((int)gridDim.x - 1) * kSelWaves)
      chunk_sums_wave(a, c);
    return;
  }
  ckv_chunk_span sp[kSelPre<KPT>];
  load_first_spans<KPT>(a.chunks, a.n_chunks, __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), sp);
  select_run<KPT, SUMS>(a, ghist, masks, sp);
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

// The spread selection: 1024-thread workgroups of G groups of 4 positions per thread (the
// smallest G from 1, 2, 3, 4, 6, 9 that covers n_tokens), slices of S positions (a power of two
// from 32 to 256, so a slice's groups are S/4 lanes of one wavefront), the smallest S for which
// the selecting and the chunk-sum workgroups fit one workgroup per CU.
bool select_slices_fits(int n_tokens) { return n_tokens >= 1 && n_tokens <= kSlicesMaxTokens; }

int32_t select_slices_launch(const SelectArgs& args, uint32_t* ghist, const SliceRows* rows, int32_t* err,
                             hipStream_t st) {
  const int N = args.n_tokens;
  if (!select_slices_fits(N) || args.has_thr) return CKV_ERR_INVALID_ARGUMENT;
  if (rows != nullptr && (2 * rows->n_heads * rows->vpr > kSlThreads || (rows->vpr & (rows->vpr - 1)) != 0))
    return CKV_ERR_INVALID_ARGUMENT;
  const int G = (N + 4 * kSlThreads - 1) / (4 * kSlThreads);
  const int Gb = G <= 4 ? G : G <= 6 ? 6 : 9;  // the instantiated group counts
  const size_t lds = (size_t)2 * (kSlThreads / 8) * Gb * sizeof(uint32_t);  // pool and taken bitmaps
  const int sum_groups = (args.n_chunks + kSlWaves - 1) / kSlWaves;
  int S = 32;
  while ((N + S - 1) / S + sum_groups > 256 && S < 256) S *= 2;
  const int n_slices = (N + S - 1) / S;
  const dim3 grid((unsigned)(n_slices + sum_groups));
  SliceRows rw = rows != nullptr ? *rows : SliceRows{};
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(kSlThreads), lds, st, args.diff, args.flags, ghist, args.local, N,
                       args.n_chunks, args.chunks, S | (args.hist_copies > 1 ? kHistCopies : 1) << 16, n_slices, args,
                       rw, err);
  };
#define CKV_SL(G)                                                   \
  if (N <= kSlThreads * 4 * G) {                                    \
    if (rows != nullptr) go(select_slices_kernel<G, true>);         \
    else go(select_slices_kernel<G, false>);                        \
    CKV_RETURN_IF_LAUNCH_FAILED();                                  \
    return CKV_OK;                                                  \
  }
  CKV_SL(1)
  CKV_SL(2)
  CKV_SL(3)
  CKV_SL(4)
  CKV_SL(6)
  CKV_SL(9)
#undef CKV_SL
  return CKV_ERR_INVALID_ARGUMENT;
}

int32_t select_launch(const SelectArgs& args, uint32_t* ghist, hipStream_t st) {
  const int n_tokens = args.n_tokens;
  const int W = (n_tokens + 31) / 32;
  const size_t lds = (size_t)(W > 0 ? W : 1) * 2 * sizeof(uint32_t);
  const int kpt = (n_tokens + kSelThreads - 1) / kSelThreads;
  // without a threshold the chunk sums run in workgroups of their own beside the selection
  const unsigned sum_groups = args.has_thr ? 0u : (unsigned)((args.n_chunks + kSelWaves - 1) / kSelWaves);
#define CKV_SEL_REG(K)                                                                                    \
  if (kpt <= K) {                                                                                         \
    if (args.has_thr)                                                                                     \
      hipLaunchKernelGGL((select_reg_kernel<K, true>), dim3(1), dim3(kSelThreads), lds, st, args.diff, args.flags, \
                         args.local, ghist, args.chunks, args.n_tokens, args.n_chunks, args.hist_copies, args);  \
    else                                                                                                  \
      hipLaunchKernelGGL((select_reg_kernel<K, false>), dim3(1 + sum_groups), dim3(kSelThreads), lds, st,  \
                         args.diff, args.flags, args.local, ghist, args.chunks, args.n_tokens, args.n_chunks, \
                         args.hist_copies, args);                                                         \
    CKV_RETURN_IF_LAUNCH_FAILED();                                                                        \
    return CKV_OK;                                                                                        \
  }
  CKV_SEL_REG(4)
  CKV_SEL_REG(8)
  CKV_SEL_REG(12)
  CKV_SEL_REG(16)
  static_assert(kSelRegMax == 16, "the largest register bucket");
#undef CKV_SEL_REG
  if (ghist != nullptr) return CKV_ERR_INVALID_ARGUMENT;  // the L2 form takes no histogram
  hipLaunchKernelGGL(select_kernel, dim3(1), dim3(kSelThreads), lds, st, args.diff, args.norm, args.flags,
                     args.local, n_tokens, args.chunks, args.n_chunks, args.has_thr, args.thr, args.keep_abs,
                     args.keep_local, args.keep_rank, args.rel_out, args.esc_out, args.counts);
  CKV_RETURN_IF_LAUNCH_FAILED();
  return CKV_OK;
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
  const SelectArgs args{diff,     norm,     pos_flags, local,      (int)n_tokens, chunks,   (int)n_chunks,
                        (int)(has_threshold != 0), escalate_threshold, keep_abs, keep_local, keep_rank, rel_dev,
                        escalated, counts};
  return select_launch(args, nullptr, (hipStream_t)stream);
}
