// Store-put extraction: copy token rows [start, start + len) of every layer's K and V out of the
// request's cache slabs into one new contiguous buffer per segment, for every reusable segment of
// the request in one launch.
//
// Reference semantics (src/chunkkv/engine/base.py:55-60): PrefillResult.chunk(start, end) builds
// a ChunkKV whose keys/values are `copy(k[:, :, start:end, :])` per layer, copy being
// `.contiguous()` for the torch engine (torch_engine.py:177); the runtime calls it once per
// reusable segment after every prefill (runtime.py:83-92), i.e. 2 x n_layers copy launches per
// segment. Here one launch moves all of them; the bytes are identical (a bit copy).
//
// Destination layout per segment s: [2][n_layers][H][len_s][D] (K layers, then V layers), so
// that layer l's keys (and values) are a contiguous (1, H, len_s, D) view.
//
// Design (gfx950): one workgroup = one (segment, 8-token tile, layer); 16-byte loads and
// stores; a thread walks (K/V, head, token, 16-byte column) items with the column fastest, so a
// wavefront reads and writes whole rows. Grid x = tile (fastest), y = segment, z = layer: the
// workgroups in flight together copy neighbouring tiles of one segment (159 -> 150 us for the
// 8k request's 24 segments x 28 layers against segment-fastest order with 16-token tiles).
#include "ckv_common.hpp"

namespace ckv {

constexpr int kExtractThreads = 256;
constexpr int kExtractTile = 8;

__global__ __launch_bounds__(kExtractThreads) void extract_kernel(
    const char* __restrict__ src_k, const char* __restrict__ src_v, int64_t ls_b, int64_t hs_b, int row_b,
    const uint64_t* __restrict__ dst_tab, const int32_t* __restrict__ spans, int n_layers, int n_heads, int n_tokens,
    int32_t* __restrict__ err) {
  typedef __attribute__((address_space(1))) const int32_t gi32;
  const int seg = blockIdx.y, layer = blockIdx.z;
  const int start = *(gi32*)(spans + 2 * seg), len = *(gi32*)(spans + 2 * seg + 1);
  const int t0 = blockIdx.x * kExtractTile;
  if (start < 0 || len < 0 || (int64_t)start + len > n_tokens) {
    if (threadIdx.x == 0 && blockIdx.x == 0 && layer == 0) flag_error(err, CKV_DEVICE_ERR_RANGE);
    return;
  }
  if (t0 >= len) return;  // uniform
  const int ntok = min(kExtractTile, len - t0);
  const int cpr = row_b / 16;
  const int items = 2 * n_heads * ntok * cpr;
  char* dst = reinterpret_cast<char*>(dst_tab[seg]);
  const int64_t head_b = (int64_t)len * row_b;  // one (head) block of the destination
  for (int i = threadIdx.x; i < items; i += kExtractThreads) {
    const int c = i % cpr;
    const int r = i / cpr;             // (kv, head, token) row
    const int tok = r % ntok;
    const int kh = r / ntok;           // kv * n_heads + head
    const int kv = kh / n_heads, h = kh % n_heads;
    const char* s = (kv ? src_v : src_k) + layer * ls_b + h * hs_b + (int64_t)(start + t0 + tok) * row_b + c * 16;
    char* d = dst + ((int64_t)(kv * n_layers + layer) * n_heads + h) * head_b + (int64_t)(t0 + tok) * row_b + c * 16;
    st16_stream(d, ld16_stream(s));
  }
}

}  // namespace ckv

extern "C" int32_t ckv_extract_chunks(const void* k_slab, const void* v_slab, int64_t layer_stride,
                                      int64_t head_stride, const uint64_t* dst_tab, const int32_t* spans,
                                      int32_t n_spans, int32_t max_len, int32_t n_layers, int32_t n_heads,
                                      int32_t n_tokens, int32_t head_dim, int32_t dtype, int32_t* err,
                                      void* stream) {
  using namespace ckv;
  if (k_slab == nullptr || v_slab == nullptr || dst_tab == nullptr || spans == nullptr) return CKV_ERR_INVALID_ARGUMENT;
  if ((dtype != CKV_DTYPE_BF16 && dtype != CKV_DTYPE_F32) || head_dim <= 0 || n_spans < 0 || max_len < 0 ||
      n_layers <= 0 || n_heads <= 0 || n_tokens < 0)
    return CKV_ERR_INVALID_ARGUMENT;
  const int64_t eb = dtype == CKV_DTYPE_BF16 ? 2 : 4;
  const int64_t row_b = head_dim * eb;
  if (row_b % 16 || ((uintptr_t)k_slab | (uintptr_t)v_slab) % 16) return CKV_ERR_INVALID_ARGUMENT;
  if (head_stride < (int64_t)n_tokens * head_dim || layer_stride < head_stride * n_heads) return CKV_ERR_OUT_OF_RANGE;
  if (n_spans == 0 || max_len == 0) return CKV_OK;
  const int tiles = (max_len + kExtractTile - 1) / kExtractTile;
  if (n_spans > 65535 || n_layers > 65535) return CKV_ERR_TOO_LARGE;  // grid y and z
  hipLaunchKernelGGL(extract_kernel, dim3((unsigned)tiles, (unsigned)n_spans, (unsigned)n_layers),
                     dim3(kExtractThreads), 0, (hipStream_t)stream, (const char*)k_slab, (const char*)v_slab,
                     layer_stride * eb, head_stride * eb, (int)row_b, dst_tab, spans, n_layers, n_heads, n_tokens, err);
  CKV_RETURN_IF_LAUNCH_FAILED();
  return CKV_OK;
}
