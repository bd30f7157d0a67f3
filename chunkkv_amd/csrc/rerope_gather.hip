// Re-RoPE + gather: rebuild every layer's base K/V cache from cached chunks moved to new
// offsets, in one launch for all layers (or a range of layers) and placements. An optional skip
// map leaves the rows of active positions alone, for callers that write those rows from the
// fresh K/V themselves (the overwrite of torch_engine.py:155-156 makes the gathered copy of such
// a row dead).
//
// Reference semantics: torch_engine.py:33 (inv_freq), :46-51 (_rotate), :56-59 (shift_keys),
// :96-103 (base_kv); the per-tile work and its rounding are in gather_common.hpp.
// (MLX twin: src/chunkkv/scheduler/rerope.py:31-61.)
//
// Design (gfx950): one workgroup = one (segment, token tile, layer); the launch shapes below.
#include <algorithm>

#include "ckv_common.hpp"
#include "gather_common.hpp"
#include "launch.hpp"
#include "scatter_common.hpp"

namespace ckv {

// Launch shapes (threads, tokens per tile, row slots in flight per thread, grid order), measured
// on MI355X at the Qwen2.5-7B KV shape (4 heads x 128, bf16).
//  - Tile-fastest grid (x = tile, y = segment): the workgroups in flight together stream
//    neighbouring tiles of one segment. Dense gathers (every row of a segment): 256 threads x 8
//    tokens x 2 slots. Gathers with a skip map (a selection leaves rows out at scattered
//    positions): 512 x 16 x 1; the 8k request's dropped rows of 26 layers (24 segments) take
//    95 us, against 112 us with the segment-fastest grid, and 108 / 114 us with 256 threads x
//    16 tokens x 2 slots / 32 tokens x 4 slots.
//  - Segment-fastest grid (x = segment, y = tile), 256 x 16 x 4, for launches of 64 segments or
//    more: the replay's 4 concurrent 32k requests (128 segments each) reach 75.0 % of HBM peak
//    with it, 68.2 % with the tile-fastest shapes above.
// Stores (a StorePolicy per shape; rows are loaded non-temporally by every shape): the skip and
// dense shapes store the key rows with device scope (sc1: written through the L2, nothing of
// them left for the end-of-launch writeback) and the value rows with device scope and
// non-temporally; the wide shape stores both non-temporally. Measured, same box each: the 8k
// request's dropped rows of layers 4-27 with layer 1's kept rows 88.0 us against 90.1-90.4 us
// with regular key rows and non-temporal value rows (the request step 219.5-219.8 against 222.7
// us; earlier: 98.5 us with both non-temporal, 112.0 us both regular); config 2's dense gather
// 77.3-77.9 against 77.8-78.3 us with both non-temporal; config 5's rounds 2.908-2.919 ms with
// both non-temporal against 3.015-3.024 ms with either device-scope form.
struct GatherDense {
  static constexpr int kThreads = 256, kTile = 8, kUnroll = 2;
  static constexpr bool kSegFastest = false;
  static constexpr int kStK = kStAgent, kStV = kStAgentStream;
};
struct GatherSkip {
  static constexpr int kThreads = 512, kTile = 16, kUnroll = 1;
  static constexpr bool kSegFastest = false;
  static constexpr int kStK = kStAgent, kStV = kStAgentStream;
};
struct GatherWide {
  static constexpr int kThreads = 256, kTile = 16, kUnroll = 4;
  static constexpr bool kSegFastest = true;
  static constexpr int kStK = kStStream, kStV = kStStream;
};
constexpr int kGatherWideSegs = 64;  // segment count from which GatherWide is used

// Grid: (tile, segment) in the order of S (x fastest), z = layer. With ROWS, the first scat_z
// z-slices scatter rows (another layer's kept rows, rs) instead, items grid-stride over them:
// dispatched first, they run beside the gather's first tiles.
template <int DTYPE, int D, class S, bool ROWS>
__global__ __launch_bounds__(S::kThreads) void rerope_gather_kernel(
    char* __restrict__ dst_k, char* __restrict__ dst_v, int64_t dst_layer_stride_b,
    int64_t dst_head_stride_b, const uint64_t* __restrict__ src_tab, int n_chunks,
    const ckv_segment* __restrict__ segs, ckv_segment one_seg, uint64_t one_src_k,
    uint64_t one_src_v, int64_t one_src_head_stride_b, int n_layers, int layer_begin, int n_heads,
    int n_tokens, const int32_t* __restrict__ skip, const InvFreq inv, int32_t* __restrict__ err,
    const RowScatter rs, int scat_z) {
  int zl = (int)blockIdx.z;
  if constexpr (ROWS) {
    if (zl < scat_z) {  // uniform: a scatter block
      const int64_t per_z = (int64_t)gridDim.x * gridDim.y;
      const int64_t stride = (int64_t)scat_z * per_z * S::kThreads;
      int n_rows = rs.n_rows;
      if (rs.n_rows_dev != nullptr) n_rows = min(n_rows, max(0, *rs.n_rows_dev));
      const int64_t total = (int64_t)n_rows * rs.n_heads * rs.vecs_per_row;
      for (int64_t g = (((int64_t)zl * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * S::kThreads + threadIdx.x;
           g < total; g += stride)
        scatter_items<1>(rs, g, 0, err);
      return;
    }
    zl -= scat_z;
  }
  gather_tile<DTYPE, D, S::kThreads, S::kTile, S::kUnroll, true, S::kStK, S::kStV>(
      dst_k, dst_v, dst_layer_stride_b, dst_head_stride_b, src_tab, n_chunks, segs,
      (int)(S::kSegFastest ? blockIdx.x : blockIdx.y), one_seg, one_src_k, one_src_v, one_src_head_stride_b, n_layers,
      layer_begin + zl, (int)(S::kSegFastest ? blockIdx.y : blockIdx.x), n_heads, n_tokens, skip, inv, err);
}

// Writes the D/2 inverse frequencies the kernels above take in their arguments.
__global__ void inv_freq_kernel(float* out, int head_dim, const InvFreq inv) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < head_dim / 2) out[i] = inv.v[i];
}

template <int DTYPE, int D>
static void launch_gather(char* dk, char* dv, int64_t ls_b, int64_t hs_b, const uint64_t* tab,
                          int n_chunks, const ckv_segment* segs, ckv_segment one, uint64_t one_k, uint64_t one_v,
                          int64_t one_hs_b, int n_segs, int max_seg_tokens, int n_layers, int layer_begin,
                          int layer_count, int n_heads, int n_tokens, const int32_t* skip, double theta,
                          int32_t* err, hipStream_t st, const RowScatter* rs) {
  auto go = [&](auto shape) {
    using S = decltype(shape);
    const unsigned tiles = (unsigned)((max_seg_tokens + S::kTile - 1) / S::kTile);
    // scatter z-slices: about two items per thread for the most rows the scatter can have
    int scat_z = 0;
    if (rs != nullptr) {
      const int64_t per_z = (int64_t)tiles * n_segs * S::kThreads;
      const int64_t items = (int64_t)rs->n_rows * rs->n_heads * rs->vecs_per_row;
      scat_z = (int)std::min<int64_t>(std::max<int64_t>(1, (items + 2 * per_z - 1) / (2 * per_z)), 1024);
    }
    const unsigned zs = (unsigned)(layer_count + scat_z);
    const dim3 grid = S::kSegFastest ? dim3((unsigned)n_segs, tiles, zs) : dim3(tiles, (unsigned)n_segs, zs);
    if (rs != nullptr)
      hipLaunchKernelGGL((rerope_gather_kernel<DTYPE, D, S, true>), grid, dim3(S::kThreads), 0, st, dk, dv, ls_b, hs_b,
                         tab, n_chunks, segs, one, one_k, one_v, one_hs_b, n_layers, layer_begin, n_heads, n_tokens,
                         skip, host_inv_freq(D, theta), err, *rs, scat_z);
    else
      hipLaunchKernelGGL((rerope_gather_kernel<DTYPE, D, S, false>), grid, dim3(S::kThreads), 0, st, dk, dv, ls_b,
                         hs_b, tab, n_chunks, segs, one, one_k, one_v, one_hs_b, n_layers, layer_begin, n_heads,
                         n_tokens, skip, host_inv_freq(D, theta), err, RowScatter{}, 0);
  };
  if (n_segs >= kGatherWideSegs) go(GatherWide{});
  else if (skip != nullptr) go(GatherSkip{});
  else go(GatherDense{});
}

using GatherFn = void (*)(char*, char*, int64_t, int64_t, const uint64_t*, int, const ckv_segment*,
                          ckv_segment, uint64_t, uint64_t, int64_t, int, int, int, int, int, int, int,
                          const int32_t*, double, int32_t*, hipStream_t, const RowScatter*);

static GatherFn pick_gather(int dtype, int head_dim) {
#define CKV_CASE(DT, HD) \
  if (dtype == DT && head_dim == HD) return &launch_gather<DT, HD>;
  CKV_CASE(CKV_DTYPE_BF16, 64)
  CKV_CASE(CKV_DTYPE_BF16, 128)
  CKV_CASE(CKV_DTYPE_BF16, 256)
  CKV_CASE(CKV_DTYPE_F32, 64)
  CKV_CASE(CKV_DTYPE_F32, 128)
  CKV_CASE(CKV_DTYPE_F32, 256)
#undef CKV_CASE
  return nullptr;
}

static int elem_bytes(int dtype) { return dtype == CKV_DTYPE_BF16 ? 2 : 4; }

}  // namespace ckv

extern "C" int32_t ckv_inv_freq(float* out, int32_t head_dim, double theta, void* stream) {
  if (out == nullptr || head_dim <= 0 || (head_dim & 1) || head_dim > 2 * ckv::kMaxHalf || !(theta > 0.0))
    return CKV_ERR_INVALID_ARGUMENT;
  const int half = head_dim / 2;
  hipLaunchKernelGGL(ckv::inv_freq_kernel, dim3((half + 63) / 64), dim3(64), 0, (hipStream_t)stream, out,
                     (int)head_dim, ckv::host_inv_freq(head_dim, theta));
  CKV_RETURN_IF_LAUNCH_FAILED();
  return CKV_OK;
}

namespace ckv {

int32_t gather_layers_launch(void* dst_k, void* dst_v, int64_t dst_layer_stride, int64_t dst_head_stride,
                             const uint64_t* src_tab, int32_t n_chunks, int32_t n_layers, int32_t layer_begin,
                             int32_t layer_end, const ckv_segment* segs, int32_t n_segs, int32_t max_seg_tokens,
                             const int32_t* skip, int32_t n_heads, int32_t n_tokens, int32_t head_dim, int32_t dtype,
                             double theta, int32_t* err, void* stream, const RowScatter* rows) {
  GatherFn fn = pick_gather(dtype, head_dim);
  if (fn == nullptr || dst_k == nullptr || dst_v == nullptr || src_tab == nullptr || segs == nullptr)
    return CKV_ERR_INVALID_ARGUMENT;
  if (n_chunks < 0 || n_segs < 0 || max_seg_tokens < 0 || n_layers <= 0 || n_heads <= 0 || n_tokens < 0 ||
      !(theta > 0.0) || layer_begin < 0 || layer_end < layer_begin || layer_end > n_layers)
    return CKV_ERR_INVALID_ARGUMENT;
  if (dst_head_stride < (int64_t)n_tokens * head_dim || dst_layer_stride < dst_head_stride * n_heads)
    return CKV_ERR_OUT_OF_RANGE;
  if (n_segs == 0 || max_seg_tokens == 0 || layer_end == layer_begin) {
    if (rows == nullptr || rows->n_rows == 0) return CKV_OK;
    // nothing to gather: the rows alone, one tile of one segment per z-slice
    max_seg_tokens = 1;
    n_segs = 1;
    layer_end = layer_begin;
  }
  // grid y (tiles of the segment-fastest shape, segments below kGatherWideSegs) and z (layers)
  if ((max_seg_tokens + 15) / 16 > 65535 || layer_end - layer_begin > 64000) return CKV_ERR_TOO_LARGE;
  const int64_t eb = elem_bytes(dtype);
  fn((char*)dst_k, (char*)dst_v, dst_layer_stride * eb, dst_head_stride * eb, src_tab, n_chunks, segs, ckv_segment{},
     0, 0, 0, n_segs, max_seg_tokens, n_layers, layer_begin, layer_end - layer_begin, n_heads, n_tokens, skip, theta, err,
     (hipStream_t)stream, rows);
  CKV_RETURN_IF_LAUNCH_FAILED();
  return CKV_OK;
}

}  // namespace ckv

extern "C" int32_t ckv_rerope_gather_layers(void* dst_k, void* dst_v, int64_t dst_layer_stride,
                                            int64_t dst_head_stride, const uint64_t* src_tab,
                                            int32_t n_chunks, int32_t n_layers, int32_t layer_begin,
                                            int32_t layer_end, const ckv_segment* segs, int32_t n_segs,
                                            int32_t max_seg_tokens, const int32_t* skip, int32_t n_heads,
                                            int32_t n_tokens, int32_t head_dim, int32_t dtype, double theta,
                                            int32_t* err, void* stream) {
  return ckv::gather_layers_launch(dst_k, dst_v, dst_layer_stride, dst_head_stride, src_tab, n_chunks, n_layers,
                                   layer_begin, layer_end, segs, n_segs, max_seg_tokens, skip, n_heads, n_tokens,
                                   head_dim, dtype, theta, err, stream, nullptr);
}

// The gather of ckv_rerope_gather_layers with another layer's kept rows scattered in the same
// launch (the z-slices in front of the gather's, as ckv_layer1_repair_gather issues it).
extern "C" int32_t ckv_rerope_gather_layers_kept(
    void* dst_k, void* dst_v, int64_t dst_layer_stride, int64_t dst_head_stride, const uint64_t* src_tab,
    int32_t n_chunks, int32_t n_layers, int32_t layer_begin, int32_t layer_end, const ckv_segment* segs,
    int32_t n_segs, int32_t max_seg_tokens, const int32_t* skip, int32_t kept_layer, const void* k_fresh,
    int64_t kf_head_stride, int64_t kf_token_stride, const void* v_fresh, int64_t vf_head_stride,
    int64_t vf_token_stride, const int64_t* keep_abs, const int64_t* keep_local, int32_t n_keep,
    const int32_t* n_keep_dev, int32_t n_fresh, int32_t n_heads, int32_t n_tokens, int32_t head_dim, int32_t dtype,
    double theta, int32_t* err, void* stream) {
  using namespace ckv;
  if (dst_k == nullptr || dst_v == nullptr || n_layers <= 0 || kept_layer < 0 || kept_layer >= n_layers ||
      (kept_layer >= layer_begin && kept_layer < layer_end) || n_keep < 0 || n_fresh < 0 || n_heads <= 0 ||
      head_dim <= 0)
    return CKV_ERR_INVALID_ARGUMENT;
  // with no fresh rows no source row is in range: nothing is read from k/v (they may be NULL)
  if (n_keep > 0 && (keep_abs == nullptr || keep_local == nullptr ||
                     (n_fresh > 0 && (k_fresh == nullptr || v_fresh == nullptr))))
    return CKV_ERR_INVALID_ARGUMENT;
  if (n_segs == 0 || max_seg_tokens == 0 || layer_end == layer_begin) {
    // nothing to gather: the table and descriptors are never read (they may be NULL)
    if (src_tab == nullptr) src_tab = (const uint64_t*)dst_k;
    if (segs == nullptr) segs = (const ckv_segment*)dst_k;
  }
  const int64_t eb = elem_bytes(dtype);
  const RowScatter kept{(char*)dst_k + kept_layer * dst_layer_stride * eb,
                        (char*)dst_v + kept_layer * dst_layer_stride * eb,
                        dst_head_stride * eb,
                        (const char*)k_fresh,
                        kf_head_stride * eb,
                        kf_token_stride * eb,
                        (const char*)v_fresh,
                        vf_head_stride * eb,
                        vf_token_stride * eb,
                        keep_abs,
                        keep_local,
                        n_keep_dev,
                        (int)n_keep,
                        (int)n_fresh,
                        (int)n_tokens,
                        (int)n_heads,
                        (int)(head_dim * eb / 16),
                        (int64_t)head_dim * eb};
  return gather_layers_launch(dst_k, dst_v, dst_layer_stride, dst_head_stride, src_tab, n_chunks, n_layers,
                              layer_begin, layer_end, segs, n_segs, max_seg_tokens, skip, n_heads, n_tokens, head_dim,
                              dtype, theta, err, stream, &kept);
}

extern "C" int32_t ckv_rerope_gather(void* dst_k, void* dst_v, int64_t dst_layer_stride,
                                     int64_t dst_head_stride, const uint64_t* src_tab,
                                     int32_t n_chunks, const ckv_segment* segs, int32_t n_segs,
                                     int32_t max_seg_tokens, int32_t n_layers, int32_t n_heads,
                                     int32_t n_tokens, int32_t head_dim, int32_t dtype,
                                     double theta, int32_t* err, void* stream) {
  return ckv_rerope_gather_layers(dst_k, dst_v, dst_layer_stride, dst_head_stride, src_tab, n_chunks, n_layers, 0,
                                  n_layers, segs, n_segs, max_seg_tokens, nullptr, n_heads, n_tokens, head_dim, dtype,
                                  theta, err, stream);
}

extern "C" int32_t ckv_shift_keys(void* dst, int64_t dst_head_stride, const void* src,
                                  int64_t src_head_stride, int32_t n_heads, int32_t n_rows,
                                  int32_t head_dim, int32_t dtype, int32_t delta, double theta,
                                  void* stream) {
  using namespace ckv;
  GatherFn fn = pick_gather(dtype, head_dim);
  if (fn == nullptr || dst == nullptr || src == nullptr || n_heads <= 0 || n_rows < 0 || !(theta > 0.0))
    return CKV_ERR_INVALID_ARGUMENT;
  if (dst_head_stride < (int64_t)n_rows * head_dim || src_head_stride < (int64_t)n_rows * head_dim)
    return CKV_ERR_OUT_OF_RANGE;
  if (n_rows == 0) return CKV_OK;
  const int64_t eb = elem_bytes(dtype);
  ckv_segment one{0, n_rows, 0, 0, n_rows, delta};
  fn((char*)dst, nullptr, 0, dst_head_stride * eb, nullptr, 1, nullptr, one, (uint64_t)(uintptr_t)src, 0,
     src_head_stride * eb, 1, n_rows, 1, 0, 1, n_heads, n_rows, nullptr, theta, nullptr, (hipStream_t)stream, nullptr);
  CKV_RETURN_IF_LAUNCH_FAILED();
  return CKV_OK;
}
