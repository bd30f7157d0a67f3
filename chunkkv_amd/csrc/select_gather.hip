// The layer-1 selection's launch with gather workgroups beside it.
//
// The register-resident selection (select_common.hpp) runs in one workgroup, bound by that CU's
// issue rate, for ~10 us at 8k positions while the rest of the chip idles. The dropped-row gather
// that follows it (layers after layer 1, rows of positions the selection did not keep) needs the
// selection's rank map, but a layer gathered in full (every cached row, as the reference's
// base_kv writes it, torch_engine.py:96-103) does not: its kept rows are overwritten by the fresh
// rows when that layer is computed (:155-156). This launch therefore gathers the first layers of
// the range in full, one (segment, 64-token tile, layer) per 1024-thread workgroup, in the CUs
// the selection leaves free; the gather launch after it takes the remaining layers with the rank
// map. Workgroup 0 selects, workgroups 1..sum_groups compute the chunks' relative deviations (as
// in select.hip), the rest gather.
#include <atomic>

#include "gather_common.hpp"
#include "launch.hpp"

namespace ckv {

#ifndef CKV_PREGATHER_TILE
#define CKV_PREGATHER_TILE 64
#endif
constexpr int kPreTile = CKV_PREGATHER_TILE, kPreUnroll = 2;  // tokens per gather workgroup, row slots per thread
#ifndef CKV_PREGATHER_BYTES_PER_POS
#define CKV_PREGATHER_BYTES_PER_POS 8192
#endif

template <int KPT, int DTYPE, int D>
__global__ __launch_bounds__(kSelThreads) void select_gather_kernel(const float* diff, const uint8_t* flags,
                                                                    const int32_t* local, uint32_t* ghist,
                                                                    const ckv_chunk_span* chunks, int n_tokens,
                                                                    int n_chunks, SelectArgs a, const PreGather g) {
  extern __shared__ uint32_t masks[];  // esc[W], pool[W]: spans of escalated / pooled chunks
  const int sel_blocks = 1 + g.sum_groups;
  if ((int)blockIdx.x >= sel_blocks) {  // uniform: a gather workgroup
    // items (tile, segment, layer), tile fastest, strided over the gather workgroups: the
    // workgroups in flight together stream neighbouring tiles
    const int n_blocks = (int)gridDim.x - sel_blocks;
    for (int it = (int)blockIdx.x - sel_blocks; it < g.n_items; it += n_blocks) {
      const int rest = it / g.tiles;
      gather_tile<DTYPE, D, kSelThreads, kPreTile, kPreUnroll, false>(
          g.dk, g.dv, g.ls_b, g.hs_b, g.tab, g.n_tab_chunks, g.segs, rest % g.n_segs, ckv_segment{}, 0, 0, 0,
          g.n_layers, g.layer_begin + rest / g.n_segs, it % g.tiles, g.n_heads, g.n_tokens, nullptr, g.inv, g.err);
      __syncthreads();  // the next item rewrites the cos/sin table
    }
    return;
  }
  a.diff = diff;
  a.flags = flags;
  a.local = local;
  a.chunks = chunks;
  a.n_tokens = n_tokens;
  a.n_chunks = n_chunks;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
  if (blockIdx.x > 0) {
    for (int c = ((int)blockIdx.x - 1) * kSelWaves + wave; c < a.n_chunks; c += g.sum_groups * kSelWaves)
      chunk_sums_wave(a, c);
    return;
  }
  ckv_chunk_span sp[kSelPre<KPT>];
  load_first_spans<KPT>(a.chunks, a.n_chunks, wave, sp);
  select_run<KPT, false>(a, ghist, masks, sp);
}

static int cu_count() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int32_t pregather_layers(int32_t n_tokens, int32_t n_chunks, int32_t has_threshold, int32_t n_segs,
                         int32_t max_seg_tokens, int32_t max_layers, int32_t n_heads, int32_t head_dim, int32_t dtype) {
  const int64_t kpt = ((int64_t)n_tokens + kSelThreads - 1) / kSelThreads;
  const bool shape_ok = (dtype == CKV_DTYPE_BF16 || dtype == CKV_DTYPE_F32) && (head_dim == 64 || head_dim == 128);
  if (has_threshold != 0 || n_tokens <= 0 || kpt > kSelRegMax || !shape_ok || max_layers <= 0 || max_seg_tokens <= 0 ||
      n_segs <= 0 || n_heads <= 0 || n_chunks < 0)
    return 0;
  // whole layers of about CKV_PREGATHER_BYTES_PER_POS bytes per position in all (the HBM traffic
  // that fits the selection's time), on the CUs the selection leaves free
  const int64_t sum_groups = ((int64_t)n_chunks + kSelWaves - 1) / kSelWaves;
  const int64_t per_layer_tiles = ((int64_t)max_seg_tokens + kPreTile - 1) / kPreTile * n_segs;
  const int64_t eb = dtype == CKV_DTYPE_BF16 ? 2 : 4;
  const int64_t per_layer_bytes = per_layer_tiles * kPreTile * n_heads * head_dim * eb * 4;
  if (cu_count() - 1 - sum_groups <= 0 || per_layer_tiles > (1 << 24)) return 0;
  const int64_t k = std::min<int64_t>(max_layers, (int64_t)n_tokens * CKV_PREGATHER_BYTES_PER_POS / per_layer_bytes);
  return (int32_t)std::max<int64_t>(k, 0);
}

int32_t select_gather_launch(const SelectArgs& args, uint32_t* ghist, PreGather g, int32_t max_layers,
                             int32_t max_seg_tokens, int32_t head_dim, int32_t dtype, double theta, int32_t* n_pre,
                             hipStream_t st) {
  *n_pre = 0;
  const int n_tokens = args.n_tokens;
  const int k = pregather_layers(n_tokens, args.n_chunks, args.has_thr, g.n_segs, max_seg_tokens, max_layers,
                                 g.n_heads, head_dim, dtype);
  if (k <= 0) return select_launch(args, ghist, st);
  const int kpt = (n_tokens + kSelThreads - 1) / kSelThreads;
  const int W = (n_tokens + 31) / 32;
  const size_t lds = (size_t)W * 2 * sizeof(uint32_t);
  g.sum_groups = (args.n_chunks + kSelWaves - 1) / kSelWaves;
  g.tiles = (max_seg_tokens + kPreTile - 1) / kPreTile;
  g.n_items = k * g.tiles * g.n_segs;
  // one 1024-thread workgroup per CU the selection leaves free (no more than there are items)
  const int blocks = std::min<int>(g.n_items, cu_count() - 1 - g.sum_groups);
  g.inv = host_inv_freq(head_dim, theta);
  const dim3 grid((unsigned)(1 + g.sum_groups + blocks));
#define CKV_SG(K, DT, HD)                                                                                      \
  if (kpt <= K && dtype == DT && head_dim == HD) {                                                              \
    hipLaunchKernelGGL((select_gather_kernel<K, DT, HD>), grid, dim3(kSelThreads), lds, st, args.diff, args.flags, \
                       args.local, ghist, args.chunks, args.n_tokens, args.n_chunks, args, g);                   \
    CKV_RETURN_IF_LAUNCH_FAILED();                                                                              \
    *n_pre = k;                                                                                                 \
    return CKV_OK;                                                                                              \
  }
#define CKV_SG_K(K) \
  CKV_SG(K, CKV_DTYPE_BF16, 128) CKV_SG(K, CKV_DTYPE_BF16, 64) CKV_SG(K, CKV_DTYPE_F32, 128) CKV_SG(K, CKV_DTYPE_F32, 64)
  CKV_SG_K(4)
  CKV_SG_K(8)
  CKV_SG_K(12)
  CKV_SG_K(16)
  static_assert(kSelRegMax == 16, "the largest register bucket");
#undef CKV_SG_K
#undef CKV_SG
  return CKV_ERR_INVALID_ARGUMENT;
}

}  // namespace ckv

extern "C" int32_t ckv_layer1_repair_gather_whole_layers(int32_t n_tokens, int32_t n_chunks, int32_t has_threshold,
                                                        int32_t n_segs, int32_t max_seg_tokens, int32_t gather_layers,
                                                        int32_t n_heads, int32_t head_dim, int32_t dtype) {
  return ckv::pregather_layers(n_tokens, n_chunks, has_threshold, n_segs, max_seg_tokens, gather_layers, n_heads,
                               head_dim, dtype);
}
