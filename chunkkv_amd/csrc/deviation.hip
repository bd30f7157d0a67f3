// Layer-1 fresh-vs-cached K/V deviation per token position (ckv_deviation), and the two launches
// of ckv_deviation_select (the deviation counting the selection's candidate histogram, then the
// selection starting from it). The semantics and the summation contract are in
// deviation_common.hpp.
//
// Design (gfx950): one 64-lane wavefront per kDevTokens token positions, four wavefronts per
// workgroup; every load of a token is issued before its arithmetic.
#include "deviation_common.hpp"
#include "launch.hpp"
#include "select_slices.hpp"

namespace ckv {

constexpr int kDevThreads = 256;
constexpr int kDevWaves = kDevThreads / kWave;
#ifndef CKV_DEV_TOKENS
#define CKV_DEV_TOKENS 2
#endif
constexpr int kDevTokens = CKV_DEV_TOKENS;  // token positions per wavefront
constexpr int kDevPerGroup = kDevWaves * kDevTokens;
static_assert(kDevPerGroup <= kWave, "one lane of wavefront 0 per position of the workgroup");

// HIST: positions flagged cached, pooled and not sink (the candidates when no chunk escalates)
// are counted by top_bin into hist, one atomic per distinct bin of the workgroup.
// The pointers and sizes the first loads use lead the argument list: the library preloads the
// first 16 argument dwords into SGPRs, but only up to the first argument passed by reference
// (the DevArgs struct), and every other argument takes a scalar load at wave start.
// zero_word (may be NULL) is set to 0 by the launch (a count the next launch adds to).
template <int DTYPE, bool HIST>
__global__ __launch_bounds__(kDevThreads) void deviation_kernel(const int32_t* local, const uint8_t* flags,
                                                                const char* kc, const char* vc, const char* kf,
                                                                const char* vf, int n_tokens, int n_fresh, DevArgs a,
                                                                float* __restrict__ diff, float* __restrict__ norm,
                                                                uint32_t* __restrict__ hist,
                                                                int32_t* __restrict__ zero_word) {
  a.local = local;
  a.flags = flags;
  a.kc = kc;
  a.vc = vc;
  a.kf = kf;
  a.vf = vf;
  a.n_tokens = n_tokens;
  a.n_fresh = n_fresh;
  __shared__ uint32_t s_bin[kDevPerGroup];
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
  const int lane = (int)threadIdx.x % kWave;
  const int p_base = ((int)blockIdx.x * kDevWaves + wave) * kDevTokens;
  float d[kDevTokens], n[kDevTokens];
  uint32_t fl[kDevTokens];
  if (zero_word != nullptr && blockIdx.x == 0 && threadIdx.x == 0) *zero_word = 0;
  deviation_wave<DTYPE, kDevTokens>(a, p_base, d, n, fl);
  if (lane == 0) {
#pragma unroll
    for (int t = 0; t < kDevTokens; ++t) {
      if (p_base + t < a.n_tokens) {
        diff[p_base + t] = d[t];
        norm[p_base + t] = n[t];
      }
      if constexpr (HIST) {
        const bool cand = (fl[t] & CKV_POS_CACHED) && (fl[t] & CKV_POS_POOLED) && !(fl[t] & CKV_POS_SINK);
        s_bin[wave * kDevTokens + t] = cand ? top_bin(dev_key(d[t])) : ~0u;
      }
    }
  }
  if constexpr (HIST) {
    __syncthreads();
    if (wave == 0) {
      const uint32_t bin = lane < kDevPerGroup ? s_bin[lane] : ~0u;
      uint32_t cnt = 0u;
      bool first = true;
#pragma unroll
      for (int j = 0; j < kDevPerGroup; ++j) {
        const uint32_t bj = s_bin[j];
        cnt += bj == bin ? 1u : 0u;
        first = first && !(j < lane && bj == bin);
      }
      if (bin != ~0u && first) atomicAdd(hist_copy(hist, hist_copies(a.n_tokens)) + bin, cnt);
    }
  }
}

template <int DTYPE, bool HIST>
static void launch_deviation(const DevArgs& args, float* diff, float* norm, uint32_t* hist, hipStream_t st,
                             int32_t* zero_word = nullptr) {
  const unsigned blocks = (unsigned)((args.n_tokens + kDevPerGroup - 1) / kDevPerGroup);
  hipLaunchKernelGGL((deviation_kernel<DTYPE, HIST>), dim3(blocks), dim3(kDevThreads), 0, st, args.local, args.flags,
                     args.kc, args.vc, args.kf, args.vf, args.n_tokens, args.n_fresh, args, diff, norm, hist,
                     zero_word);
}

static int32_t check_deviation_args(const void* k_fresh, const void* v_fresh, const void* k_cache, const void* v_cache,
                                    int64_t cache_head_stride, const uint8_t* pos_flags, const int32_t* local,
                                    int32_t n_tokens, int32_t n_fresh, int32_t n_heads, int32_t head_dim,
                                    int32_t dtype, const float* diff, const float* norm) {
  if (dtype != CKV_DTYPE_BF16 && dtype != CKV_DTYPE_F32) return CKV_ERR_INVALID_ARGUMENT;
  const int vec = dtype == CKV_DTYPE_BF16 ? 8 : 4;
  if (head_dim <= 0 || head_dim % vec != 0 || n_heads <= 0 || n_tokens < 0 || n_fresh < 0)
    return CKV_ERR_INVALID_ARGUMENT;
  if (pos_flags == nullptr || local == nullptr || diff == nullptr || norm == nullptr || k_cache == nullptr ||
      v_cache == nullptr || (n_fresh > 0 && (k_fresh == nullptr || v_fresh == nullptr)))
    return CKV_ERR_INVALID_ARGUMENT;
  if (cache_head_stride < (int64_t)n_tokens * head_dim) return CKV_ERR_OUT_OF_RANGE;
  return CKV_OK;
}

static DevArgs deviation_args(const void* k_fresh, int64_t kf_head_stride, int64_t kf_token_stride, const void* v_fresh,
                              int64_t vf_head_stride, int64_t vf_token_stride, const void* k_cache,
                              const void* v_cache, int64_t cache_head_stride, const uint8_t* pos_flags,
                              const int32_t* local, int32_t n_tokens, int32_t n_fresh, int32_t n_heads,
                              int32_t head_dim, int32_t dtype, int32_t* err) {
  const int64_t eb = dtype == CKV_DTYPE_BF16 ? 2 : 4;
  return DevArgs{(const char*)k_fresh, kf_head_stride * eb, kf_token_stride * eb, (const char*)v_fresh,
                 vf_head_stride * eb, vf_token_stride * eb, (const char*)k_cache, (const char*)v_cache,
                 cache_head_stride * eb, pos_flags, local, (int)n_tokens, (int)n_fresh, (int)n_heads,
                 (int)head_dim, err};
}

}  // namespace ckv

extern "C" int32_t ckv_deviation(const void* k_fresh, int64_t kf_head_stride, int64_t kf_token_stride,
                                 const void* v_fresh, int64_t vf_head_stride, int64_t vf_token_stride,
                                 const void* k_cache, const void* v_cache, int64_t cache_head_stride,
                                 const uint8_t* pos_flags, const int32_t* local, int32_t n_tokens,
                                 int32_t n_fresh, int32_t n_heads, int32_t head_dim, int32_t dtype,
                                 float* diff, float* norm, int32_t* err, void* stream) {
  using namespace ckv;
  const int32_t rc = check_deviation_args(k_fresh, v_fresh, k_cache, v_cache, cache_head_stride, pos_flags, local,
                                          n_tokens, n_fresh, n_heads, head_dim, dtype, diff, norm);
  if (rc != CKV_OK) return rc;
  if (n_tokens == 0) return CKV_OK;
  const DevArgs args = deviation_args(k_fresh, kf_head_stride, kf_token_stride, v_fresh, vf_head_stride,
                                      vf_token_stride, k_cache, v_cache, cache_head_stride, pos_flags, local,
                                      n_tokens, n_fresh, n_heads, head_dim, dtype, err);
  if (dtype == CKV_DTYPE_BF16)
    launch_deviation<CKV_DTYPE_BF16, false>(args, diff, norm, nullptr, (hipStream_t)stream);
  else
    launch_deviation<CKV_DTYPE_F32, false>(args, diff, norm, nullptr, (hipStream_t)stream);
  CKV_RETURN_IF_LAUNCH_FAILED();
  return CKV_OK;
}

extern "C" int32_t ckv_deviation_select(
    const void* k_fresh, int64_t kf_head_stride, int64_t kf_token_stride, const void* v_fresh, int64_t vf_head_stride,
    int64_t vf_token_stride, const void* k_cache, const void* v_cache, int64_t cache_head_stride,
    const uint8_t* pos_flags, const int32_t* local, int32_t n_tokens, int32_t n_fresh, int32_t n_heads,
    int32_t head_dim, int32_t dtype, const ckv_chunk_span* chunks, int32_t n_chunks, int32_t has_threshold,
    double escalate_threshold, float* diff, float* norm, int64_t* keep_abs, int64_t* keep_local, int32_t* keep_rank,
    float* rel_dev, uint8_t* escalated, int32_t* counts, void* workspace, int64_t workspace_bytes, int32_t* err,
    void* stream) {
  using namespace ckv;
  int32_t rc = check_deviation_args(k_fresh, v_fresh, k_cache, v_cache, cache_head_stride, pos_flags, local, n_tokens,
                                    n_fresh, n_heads, head_dim, dtype, diff, norm);
  if (rc != CKV_OK) return rc;
  if (n_chunks < 0 || keep_abs == nullptr || keep_local == nullptr || counts == nullptr)
    return CKV_ERR_INVALID_ARGUMENT;
  if (n_chunks > 0 && (chunks == nullptr || rel_dev == nullptr || escalated == nullptr))
    return CKV_ERR_INVALID_ARGUMENT;
  if (n_tokens > CKV_SELECT_MAX_TOKENS) return CKV_ERR_TOO_LARGE;
  // Without a threshold: the selection spread over many workgroups (select_slices.hpp); with one,
  // the single-workgroup selection (the register-resident form takes the histogram).
  const bool spread = has_threshold == 0 && select_slices_fits(n_tokens);
  const bool with_hist = n_tokens > 0 && (spread || n_tokens <= kSelRegMax * kSelThreads);
  if (with_hist && (workspace == nullptr || workspace_bytes < CKV_DEVIATION_SELECT_WORKSPACE_BYTES ||
                    (uintptr_t)workspace % 16))
    return CKV_ERR_INVALID_ARGUMENT;
  hipStream_t st = (hipStream_t)stream;
  uint32_t* hist = with_hist ? (uint32_t*)workspace : nullptr;
  int32_t* zero = spread ? counts + CKV_COUNT_UNCOMPUTED : nullptr;
  if (n_tokens > 0) {
    const DevArgs args = deviation_args(k_fresh, kf_head_stride, kf_token_stride, v_fresh, vf_head_stride,
                                        vf_token_stride, k_cache, v_cache, cache_head_stride, pos_flags, local,
                                        n_tokens, n_fresh, n_heads, head_dim, dtype, err);
    if (dtype == CKV_DTYPE_BF16) {
      if (with_hist) launch_deviation<CKV_DTYPE_BF16, true>(args, diff, norm, hist, st, zero);
      else launch_deviation<CKV_DTYPE_BF16, false>(args, diff, norm, nullptr, st);
    } else {
      if (with_hist) launch_deviation<CKV_DTYPE_F32, true>(args, diff, norm, hist, st, zero);
      else launch_deviation<CKV_DTYPE_F32, false>(args, diff, norm, nullptr, st);
    }
    CKV_RETURN_IF_LAUNCH_FAILED();
  }
  const SelectArgs sel{diff,     norm,     pos_flags, local,      (int)n_tokens, chunks,   (int)n_chunks,
                       (int)(has_threshold != 0), escalate_threshold, keep_abs, keep_local, keep_rank, rel_dev,
                       escalated, counts, hist_copies((int)n_tokens)};
  if (spread) return select_slices_launch(sel, hist, nullptr, err, st);
  return select_launch(sel, hist, st);
}
