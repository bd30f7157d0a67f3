// Layer-1 fresh-vs-cached K/V deviation per token position.
//
// Reference semantics (src/chunkkv/engine/torch_engine.py:117-124):
//   d_act  = ((k - K[:, :, active]).float() ** 2).sum(dim=(0, 1, 3))
//   d_act += ((v - V[:, :, active]).float() ** 2).sum(dim=(0, 1, 3))
//   n_act  = (k.float() ** 2).sum(dim=(0, 1, 3)) + (v.float() ** 2).sum(dim=(0, 1, 3))
//   diff[active] = d_act; norm[active] = n_act   (zeros elsewhere)
// The subtraction happens in the element type (one rounding); squares and sums are fp32.
// K/V rows outside every placement are zero in the reference (base_kv zero-fills them).
//
// Design (gfx950): one 64-lane wavefront per kDevTokens token positions; each lane loads 16 bytes
// of each of the four rows (fresh k, cached K, fresh v, cached V) of every one of its tokens
// before any arithmetic, so a token's H*D elements (1 KiB per tensor at H=4, D=128, bf16)
// arrive in one coalesced pass. Four fp32 partial sums
// per lane are combined by a xor butterfly; the lane/butterfly order is the summation contract
// that the oracle restates bit-for-bit.
#include "ckv_common.hpp"

namespace ckv {

constexpr int kDevThreads = 256;
constexpr int kDevWaves = kDevThreads / kWave;
#ifndef CKV_DEV_TOKENS
#define CKV_DEV_TOKENS 1
#endif
constexpr int kDevTokens = CKV_DEV_TOKENS;  // token positions per wavefront

template <int DTYPE>
__global__ __launch_bounds__(kDevThreads) void deviation_kernel(
    const char* __restrict__ kf, int64_t kf_hs_b, int64_t kf_ts_b, const char* __restrict__ vf,
    int64_t vf_hs_b, int64_t vf_ts_b, const char* __restrict__ kc, const char* __restrict__ vc,
    int64_t c_hs_b, const uint8_t* __restrict__ flags, const int32_t* __restrict__ local,
    int n_tokens, int n_fresh, int n_heads, int head_dim, float* __restrict__ diff,
    float* __restrict__ norm, int32_t* __restrict__ err) {
  using E = Elem<DTYPE>;
  constexpr int VEC = E::kVec;
  const int lane = threadIdx.x % kWave;
  const int p_base = (blockIdx.x * kDevWaves + threadIdx.x / kWave) * kDevTokens;
  const int64_t row_b = (int64_t)head_dim * E::kBytes;
  const int vecs_per_row = head_dim / VEC;
  const int n_vecs = n_heads * vecs_per_row;

  int jj[kDevTokens];
  bool cached[kDevTokens];
  float sk[kDevTokens], sv[kDevTokens], nk[kDevTokens], nv[kDevTokens];
#pragma unroll
  for (int t = 0; t < kDevTokens; ++t) {
    const int p = p_base + t;
    jj[t] = p < n_tokens ? local[p] : -1;
    cached[t] = p < n_tokens && (flags[p] & CKV_POS_CACHED) != 0;
    if (jj[t] >= n_fresh) {
      if (lane == 0) flag_error(err, CKV_DEVICE_ERR_RANGE);
      jj[t] = -1;
    }
    sk[t] = sv[t] = nk[t] = nv[t] = 0.0f;
  }
  for (int q = lane; q < n_vecs; q += kWave) {
    const int h = q / vecs_per_row;
    const int64_t cb = (int64_t)(q % vecs_per_row) * 16;
    vec16 k16[kDevTokens], v16[kDevTokens], kc16[kDevTokens], vc16[kDevTokens];
#pragma unroll
    for (int t = 0; t < kDevTokens; ++t) {
      if (jj[t] >= 0) {
        k16[t] = ld16(kf + h * kf_hs_b + jj[t] * kf_ts_b + cb);
        v16[t] = ld16(vf + h * vf_hs_b + jj[t] * vf_ts_b + cb);
        if (cached[t]) {
          const int64_t co = h * c_hs_b + (int64_t)(p_base + t) * row_b + cb;
          kc16[t] = ld16(kc + co);
          vc16[t] = ld16(vc + co);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < kDevTokens; ++t) {
      if (jj[t] < 0) continue;
      float kx[VEC], vx[VEC], kcx[VEC], vcx[VEC];
      E::unpack(k16[t], kx);
      E::unpack(v16[t], vx);
      if (cached[t]) {
        E::unpack(kc16[t], kcx);
        E::unpack(vc16[t], vcx);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) kcx[e] = vcx[e] = 0.0f;
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float dk = E::round_trip(kx[e] - kcx[e]);
        const float dv = E::round_trip(vx[e] - vcx[e]);
        sk[t] = sk[t] + dk * dk;
        sv[t] = sv[t] + dv * dv;
        nk[t] = nk[t] + kx[e] * kx[e];
        nv[t] = nv[t] + vx[e] * vx[e];
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kDevTokens; ++t) {
    const int p = p_base + t;
    if (p >= n_tokens) continue;  // uniform across the wavefront
    const float a = wave_butterfly_sum(sk[t]);
    const float b = wave_butterfly_sum(sv[t]);
    const float c = wave_butterfly_sum(nk[t]);
    const float d = wave_butterfly_sum(nv[t]);
    if (lane == 0) {
      diff[p] = jj[t] < 0 ? 0.0f : a + b;
      norm[p] = jj[t] < 0 ? 0.0f : c + d;
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
  if (dtype == CKV_DTYPE_BF16)
    hipLaunchKernelGGL(deviation_kernel<CKV_DTYPE_BF16>, dim3(blocks), dim3(kDevThreads), 0, st,
                       (const char*)k_fresh, kf_head_stride * eb, kf_token_stride * eb, (const char*)v_fresh,
                       vf_head_stride * eb, vf_token_stride * eb, (const char*)k_cache, (const char*)v_cache,
                       cache_head_stride * eb, pos_flags, local, n_tokens, n_fresh, n_heads, head_dim, diff,
                       norm, err);
  else
    hipLaunchKernelGGL(deviation_kernel<CKV_DTYPE_F32>, dim3(blocks), dim3(kDevThreads), 0, st,
                       (const char*)k_fresh, kf_head_stride * eb, kf_token_stride * eb, (const char*)v_fresh,
                       vf_head_stride * eb, vf_token_stride * eb, (const char*)k_cache, (const char*)v_cache,
                       cache_head_stride * eb, pos_flags, local, n_tokens, n_fresh, n_heads, head_dim, diff,
                       norm, err);
  CKV_RETURN_IF_LAUNCH_FAILED();
  return CKV_OK;
}
