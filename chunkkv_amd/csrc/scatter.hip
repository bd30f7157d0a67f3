// Scatter freshly computed K/V rows of the active set into one layer's cache.
//
// Reference semantics (src/chunkkv/engine/torch_engine.py:155-156):
//   K[:, :, active] = k;  V[:, :, active] = v      (row overwrite, bit-exact copy)
// and, with a source row map (ckv_scatter_kept_rows), the compaction before it (:152):
//   k, v = k[:, :, sel], v[:, :, sel]  folded into the same pass (k/v are read at rows sel[j]).
//
// Design (gfx950): each thread moves kScatterUnroll 16-byte vectors of K and the matching
// vectors of V (all loads issued before any store; grid-stride so each load instruction of a
// wavefront is contiguous).
// Consecutive threads walk one row (D elements), then the next head, then the next active
// token, so the destination writes of a row are one contiguous 256-byte burst (D = 128, bf16)
// and the source reads follow the fresh tensor's own strides.
#include "launch.hpp"

namespace ckv {

constexpr int kScatterThreads = 256;
#ifndef CKV_SCATTER_UNROLL
#define CKV_SCATTER_UNROLL 1
#endif
constexpr int kScatterUnroll = CKV_SCATTER_UNROLL;  // 16-byte K/V vector pairs per thread

__global__ __launch_bounds__(kScatterThreads) void scatter_rows_kernel(
    char* dst_k, char* dst_v, int64_t d_hs_b, const char* __restrict__ sk, int64_t sk_hs_b,
    int64_t sk_ts_b, const char* __restrict__ sv, int64_t sv_hs_b, int64_t sv_ts_b,
    const int64_t* __restrict__ rows, const int64_t* __restrict__ src_rows, int n_rows, int n_src, int n_tokens,
    int n_heads, int vecs_per_row, int64_t row_b, const int32_t* __restrict__ n_rows_dev, int32_t* __restrict__ err) {
  if (n_rows_dev != nullptr) n_rows = min(n_rows, max(0, *n_rows_dev));  // a count only the device knows
  const int64_t per_tok = (int64_t)n_heads * vecs_per_row;
  const int64_t total = (int64_t)n_rows * per_tok;
  const int64_t stride = (int64_t)gridDim.x * kScatterThreads;
  const int64_t g0 = (int64_t)blockIdx.x * kScatterThreads + threadIdx.x;
  vec16 a[kScatterUnroll], b[kScatterUnroll];
  int64_t dst_o[kScatterUnroll];
#pragma unroll
  for (int u = 0; u < kScatterUnroll; ++u) {
    const int64_t g = g0 + u * stride;
    dst_o[u] = -1;
    if (g < total) {
      const int64_t j = g / per_tok;
      const int rem = (int)(g - j * per_tok);
      const int h = rem / vecs_per_row;
      const int64_t cb = (int64_t)(rem % vecs_per_row) * 16;
      const int64_t t = rows[j];
      const int64_t js = src_rows != nullptr ? src_rows[j] : j;
      const bool src_ok = js >= 0 && js < n_src;
      if (src_ok) {
        a[u] = ld16_stream(sk + h * sk_hs_b + js * sk_ts_b + cb);  // read once: non-temporal
        b[u] = ld16_stream(sv + h * sv_hs_b + js * sv_ts_b + cb);
      }
      if (src_ok && t >= 0 && t < n_tokens) {
        dst_o[u] = h * d_hs_b + t * row_b + cb;
      } else if (rem == 0) {
        flag_error(err, CKV_DEVICE_ERR_RANGE);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < kScatterUnroll; ++u) {
    if (dst_o[u] >= 0) {  // non-temporal: no dirty L2 lines left for the kernel boundary
      st16_stream(dst_k + dst_o[u], a[u]);
      st16_stream(dst_v + dst_o[u], b[u]);
    }
  }
}

int32_t scatter_launch(void* dst_k, void* dst_v, int64_t dst_head_stride, const void* src_k, int64_t sk_head_stride,
                       int64_t sk_token_stride, const void* src_v, int64_t sv_head_stride, int64_t sv_token_stride,
                       const int64_t* rows, const int64_t* src_rows, int32_t n_rows, int32_t n_src, int32_t n_tokens,
                       int32_t n_heads, int32_t head_dim, int32_t dtype, const int32_t* n_rows_dev, int32_t* err,
                       void* stream) {
  if (dtype != CKV_DTYPE_BF16 && dtype != CKV_DTYPE_F32) return CKV_ERR_INVALID_ARGUMENT;
  const int64_t eb = dtype == CKV_DTYPE_BF16 ? 2 : 4;
  if (head_dim <= 0 || (head_dim * eb) % 16 != 0 || n_heads <= 0 || n_rows < 0 || n_tokens < 0 || n_src < 0)
    return CKV_ERR_INVALID_ARGUMENT;
  if (n_rows > 0 && (dst_k == nullptr || dst_v == nullptr || src_k == nullptr || src_v == nullptr || rows == nullptr))
    return CKV_ERR_INVALID_ARGUMENT;
  if (dst_head_stride < (int64_t)n_tokens * head_dim) return CKV_ERR_OUT_OF_RANGE;
  if (n_rows == 0) return CKV_OK;
  const int vecs_per_row = (int)(head_dim * eb / 16);
  const int64_t total = (int64_t)n_rows * n_heads * vecs_per_row;
  const int64_t per_block = (int64_t)kScatterThreads * kScatterUnroll;
  const int64_t blocks = (total + per_block - 1) / per_block;
  if (blocks > 0x7fffffffLL) return CKV_ERR_TOO_LARGE;
  hipLaunchKernelGGL(scatter_rows_kernel, dim3((unsigned)blocks), dim3(kScatterThreads), 0, (hipStream_t)stream,
                     (char*)dst_k, (char*)dst_v, dst_head_stride * eb, (const char*)src_k, sk_head_stride * eb,
                     sk_token_stride * eb, (const char*)src_v, sv_head_stride * eb, sv_token_stride * eb, rows,
                     src_rows, (int)n_rows, (int)n_src, (int)n_tokens, (int)n_heads, vecs_per_row,
                     (int64_t)head_dim * eb, n_rows_dev, err);
  CKV_RETURN_IF_LAUNCH_FAILED();
  return CKV_OK;
}

}  // namespace ckv

extern "C" int32_t ckv_scatter_rows(void* dst_k, void* dst_v, int64_t dst_head_stride, const void* src_k,
                                    int64_t sk_head_stride, int64_t sk_token_stride, const void* src_v,
                                    int64_t sv_head_stride, int64_t sv_token_stride, const int64_t* rows,
                                    int32_t n_rows, int32_t n_tokens, int32_t n_heads, int32_t head_dim,
                                    int32_t dtype, int32_t* err, void* stream) {
  return ckv::scatter_launch(dst_k, dst_v, dst_head_stride, src_k, sk_head_stride, sk_token_stride, src_v,
                             sv_head_stride, sv_token_stride, rows, nullptr, n_rows, n_rows, n_tokens, n_heads, head_dim,
                             dtype, nullptr, err, stream);
}

extern "C" int32_t ckv_scatter_kept_rows(void* dst_k, void* dst_v, int64_t dst_head_stride, const void* src_k,
                                         int64_t sk_head_stride, int64_t sk_token_stride, const void* src_v,
                                         int64_t sv_head_stride, int64_t sv_token_stride, const int64_t* dst_rows,
                                         const int64_t* src_rows, int32_t n_rows, int32_t n_src, int32_t n_tokens,
                                         int32_t n_heads, int32_t head_dim, int32_t dtype, int32_t* err,
                                         void* stream) {
  if (n_rows > 0 && src_rows == nullptr) return CKV_ERR_INVALID_ARGUMENT;
  return ckv::scatter_launch(dst_k, dst_v, dst_head_stride, src_k, sk_head_stride, sk_token_stride, src_v,
                             sv_head_stride, sv_token_stride, dst_rows, src_rows, n_rows, n_src, n_tokens, n_heads,
                             head_dim, dtype, nullptr, err, stream);
}
