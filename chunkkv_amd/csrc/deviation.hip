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
// Design (gfx950): one 64-lane wavefront per token position; each lane loads 16 bytes of each
// of the four rows (fresh k, cached K, fresh v, cached V) per step, so a token's H*D elements
// (1 KiB per tensor at H=4, D=128, bf16) arrive in one coalesced pass. Four fp32 partial sums
// per lane are combined by a xor butterfly; the lane/butterfly order is the summation contract
// that the oracle restates bit-for-bit.
#include "ckv_common.hpp"

namespace ckv {

constexpr int kDevThreads = 256;
constexpr int kDevWaves = kDevThreads / kWave;

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
  const int p = blockIdx.x * kDevWaves + threadIdx.x / kWave;
  if (p >= n_tokens) return;
  const int j = local[p];
  if (j < 0 || j >= n_fresh) {
    if (j >= n_fresh && lane == 0) flag_error(err, CKV_DEVICE_ERR_RANGE);
    if (lane == 0) {
      diff[p] = 0.0f;
      norm[p] = 0.0f;
    }
    return;
  }
  const bool cached = (flags[p] & CKV_POS_CACHED) != 0;
  const int64_t row_b = (int64_t)head_dim * E::kBytes;
  const int vecs_per_row = head_dim / VEC;
  const int n_vecs = n_heads * vecs_per_row;

  float sk = 0.0f, sv = 0.0f, nk = 0.0f, nv = 0.0f;
  for (int q = lane; q < n_vecs; q += kWave) {
    const int h = q / vecs_per_row;
    const int64_t cb = (int64_t)(q % vecs_per_row) * 16;
    const vec16 k16 = ld16(kf + h * kf_hs_b + j * kf_ts_b + cb);
    const vec16 v16 = ld16(vf + h * vf_hs_b + j * vf_ts_b + cb);
    float kx[VEC], vx[VEC], kcx[VEC], vcx[VEC];
    E::unpack(k16, kx);
    E::unpack(v16, vx);
    if (cached) {
      const int64_t co = h * c_hs_b + (int64_t)p * row_b + cb;
      E::unpack(ld16(kc + co), kcx);
      E::unpack(ld16(vc + co), vcx);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) kcx[e] = vcx[e] = 0.0f;
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float dk = E::round_trip(kx[e] - kcx[e]);
      const float dv = E::round_trip(vx[e] - vcx[e]);
      sk = sk + dk * dk;
      sv = sv + dv * dv;
      nk = nk + kx[e] * kx[e];
      nv = nv + vx[e] * vx[e];
    }
  }
  sk = wave_butterfly_sum(sk);
  sv = wave_butterfly_sum(sv);
  nk = wave_butterfly_sum(nk);
  nv = wave_butterfly_sum(nv);
  if (lane == 0) {
    diff[p] = sk + sv;
    norm[p] = nk + nv;
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
  const unsigned blocks = (unsigned)((n_tokens + kDevWaves - 1) / kDevWaves);
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
