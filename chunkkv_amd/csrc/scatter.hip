// Scatter freshly computed K/V rows of the active set into one layer's cache.
//
// Reference semantics (src/chunkkv/engine/torch_engine.py:155-156):
//   K[:, :, active] = k;  V[:, :, active] = v      (row overwrite, bit-exact copy)
// and, with a source row map (ckv_scatter_kept_rows), the compaction before it (:152):
//   k, v = k[:, :, sel], v[:, :, sel]  folded into the same pass (k/v are read at rows sel[j]).
//
// Design (gfx950): each thread moves kScatterUnroll 16-byte vectors of K and the matching
// vectors of V (scatter_common.hpp: all loads issued before any store; grid-stride so each load
// instruction of a wavefront is contiguous).
#include "launch.hpp"
#include "scatter_common.hpp"

namespace ckv {

constexpr int kScatterThreads = 256;
#ifndef CKV_SCATTER_UNROLL
#define CKV_SCATTER_UNROLL 1
#endif
constexpr int kScatterUnroll = CKV_SCATTER_UNROLL;  // 16-byte K/V vector pairs per thread

__global__ __launch_bounds__(kScatterThreads) void scatter_rows_kernel(RowScatter s, int32_t* __restrict__ err) {
  scatter_items<kScatterUnroll>(s, (int64_t)blockIdx.x * kScatterThreads + threadIdx.x,
                                (int64_t)gridDim.x * kScatterThreads, err);
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
  const RowScatter rs{(char*)dst_k,          (char*)dst_v,          dst_head_stride * eb, (const char*)src_k,
                      sk_head_stride * eb,    sk_token_stride * eb,  (const char*)src_v,   sv_head_stride * eb,
                      sv_token_stride * eb,   rows,                  src_rows,             n_rows_dev,
                      (int)n_rows,            (int)n_src,            (int)n_tokens,        (int)n_heads,
                      vecs_per_row,           (int64_t)head_dim * eb};
  hipLaunchKernelGGL(scatter_rows_kernel, dim3((unsigned)blocks), dim3(kScatterThreads), 0, (hipStream_t)stream, rs,
                     err);
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
