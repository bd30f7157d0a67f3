// ckv_deviation_select for callers that cannot allocate (ckv_deviation_select_noalloc): the same
// two launches as ckv_deviation_select (deviation.hip), with the candidate histogram in a static
// per-GPU device array instead of a caller's workspace.
#include <mutex>

#include "chunkkv_amd.h"
#include <hip/hip_runtime.h>

// The workspace is this file-scope array, one copy per GPU (zero at load; every call leaves it
// zero). In host code the name `scratch` only stands in for the symbol: its device address on
// each GPU comes from hipGetSymbolAddress, once per device with that device current, and only
// that address reaches a kernel.
static __device__ __align__(256) uint32_t scratch[CKV_DEVIATION_SELECT_WORKSPACE_BYTES / 4];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device; nullptr until looked up

int32_t scratch_address(hipStream_t stream, void** out) {
  int dev = 0;
  if (hipStreamGetDevice(stream, &dev) != hipSuccess) return CKV_ERR_HIP;
  if (dev < 0 || dev >= kMaxDevices) return CKV_ERR_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return CKV_ERR_HIP;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return CKV_ERR_HIP;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev && hipSetDevice(cur) != hipSuccess) return CKV_ERR_HIP;
    if (e != hipSuccess || p == nullptr) return CKV_ERR_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return CKV_OK;
}

}  // namespace

extern "C" int32_t ckv_deviation_select_noalloc(
    const void* k_fresh, int64_t kf_head_stride, int64_t kf_token_stride, const void* v_fresh, int64_t vf_head_stride,
    int64_t vf_token_stride, const void* k_cache, const void* v_cache, int64_t cache_head_stride,
    const uint8_t* pos_flags, const int32_t* local, int32_t n_tokens, int32_t n_fresh, int32_t n_heads,
    int32_t head_dim, int32_t dtype, const ckv_chunk_span* chunks, int32_t n_chunks, int32_t has_threshold,
    double escalate_threshold, float* diff, float* norm, int64_t* keep_abs, int64_t* keep_local, int32_t* keep_rank,
    float* rel_dev, uint8_t* escalated, int32_t* counts, int32_t* err, void* stream) {
  if (n_tokens > CKV_SELECT_MAX_TOKENS) return CKV_ERR_TOO_LARGE;
  void* ws = nullptr;
  const int32_t rc = scratch_address((hipStream_t)stream, &ws);
  if (rc != CKV_OK) return rc;
  return ckv_deviation_select(k_fresh, kf_head_stride, kf_token_stride, v_fresh, vf_head_stride, vf_token_stride,
                              k_cache, v_cache, cache_head_stride, pos_flags, local, n_tokens, n_fresh, n_heads,
                              head_dim, dtype, chunks, n_chunks, has_threshold, escalate_threshold, diff, norm,
                              keep_abs, keep_local, keep_rank, rel_dev, escalated, counts, ws,
                              CKV_DEVIATION_SELECT_WORKSPACE_BYTES, err, stream);
}
