// Layer-1 fresh-vs-cached K/V deviation per token position (ckv_deviation). The semantics and
// the summation contract are in deviation_common.hpp, shared with ckv_deviation_select.
//
// Design (gfx950): one 64-lane wavefront per kDevTokens token positions, four wavefronts per
// workgroup; every load of a token is issued before its arithmetic.
#include "deviation_common.hpp"

namespace ckv {

constexpr int kDevThreads = 256;
constexpr int kDevWaves = kDevThreads / kWave;
#ifndef CKV_DEV_TOKENS
#define CKV_DEV_TOKENS 1
#endif
constexpr int kDevTokens = CKV_DEV_TOKENS;  // token positions per wavefront

template <int DTYPE>
__global__ __launch_bounds__(kDevThreads) void deviation_kernel(DevArgs a, float* __restrict__ diff,
                                                                float* __restrict__ norm) {
  const int p_base = (blockIdx.x * kDevWaves + threadIdx.x / kWave) * kDevTokens;
  float d[kDevTokens], n[kDevTokens];
  uint32_t fl[kDevTokens];
  deviation_wave<DTYPE, kDevTokens>(a, p_base, d, n, fl);
  if (threadIdx.x % kWave == 0) {
#pragma unroll
    for (int t = 0; t < kDevTokens; ++t) {
      if (p_base + t < a.n_tokens) {
        diff[p_base + t] = d[t];
        norm[p_base + t] = n[t];
      }
    }
  }
}

}  // namespace ckv

extern "C" int32_t ckv_deviation(const void* k_fresh, int64_t kf_head_stride, int64_t kf_token_stride,
                                 const void* v_fresh, int64_t vf_head_stride, int64_t vf_token_stride,
                                 const void* k_cache, const void* v_cache, int64_t cache_head_stride,
                                 const uint8_t* pos_flags, const int32_t* local, int32_t n_tokens,
                                 int32_t n_fresh, int32_t n_heads, int32_t head_dim, int32_t dtype,
                                 float* diff, float* norm, int32_t* err, void* stream) {
  using namespace ckv;
  if (dtype != CKV_DTYPE_BF16 && dtype != CKV_DTYPE_F32) return CKV_ERR_INVALID_ARGUMENT;
  const int vec = dtype == CKV_DTYPE_BF16 ? 8 : 4;
  if (head_dim <= 0 || head_dim % vec != 0 || n_heads <= 0 || n_tokens < 0 || n_fresh < 0)
    return CKV_ERR_INVALID_ARGUMENT;
  if (pos_flags == nullptr || local == nullptr || diff == nullptr || norm == nullptr || k_cache == nullptr ||
      v_cache == nullptr || (n_fresh > 0 && (k_fresh == nullptr || v_fresh == nullptr)))
    return CKV_ERR_INVALID_ARGUMENT;
  if (cache_head_stride < (int64_t)n_tokens * head_dim) return CKV_ERR_OUT_OF_RANGE;
  if (n_tokens == 0) return CKV_OK;
  const int64_t eb = dtype == CKV_DTYPE_BF16 ? 2 : 4;
  const int per_block = kDevWaves * kDevTokens;
  const unsigned blocks = (unsigned)((n_tokens + per_block - 1) / per_block);
  hipStream_t st = (hipStream_t)stream;
  const DevArgs args{(const char*)k_fresh, kf_head_stride * eb, kf_token_stride * eb, (const char*)v_fresh,
                     vf_head_stride * eb, vf_token_stride * eb, (const char*)k_cache, (const char*)v_cache,
                     cache_head_stride * eb, pos_flags, local, (int)n_tokens, (int)n_fresh, (int)n_heads,
                     (int)head_dim, err};
  if (dtype == CKV_DTYPE_BF16)
    hipLaunchKernelGGL(deviation_kernel<CKV_DTYPE_BF16>, dim3(blocks), dim3(kDevThreads), 0, st, args, diff, norm);
  else
    hipLaunchKernelGGL(deviation_kernel<CKV_DTYPE_F32>, dim3(blocks), dim3(kDevThreads), 0, st, args, diff, norm);
  CKV_RETURN_IF_LAUNCH_FAILED();
  return CKV_OK;
}
