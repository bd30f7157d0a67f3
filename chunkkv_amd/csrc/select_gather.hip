// The layer-1 selection's launch with gather workgroups beside it.
//
// The register-resident selection (select_common.hpp) runs in one workgroup, bound by that CU's
// issue rate, for ~10 us at 8k positions while the rest of the chip idles. The dropped-row gather
// that follows it (layers after layer 1, rows of positions the selection did not keep) needs the
// selection's rank map, but a layer gathered in full (every cached row, as the reference's
// base_kv writes it, torch_engine.py:96-103) does not: its kept rows are overwritten by the fresh
// rows when that layer is computed (:155-156). This launch therefore gathers the first layers of
// the range in full in the CUs the selection leaves free (one 1024-thread workgroup per CU), and
// the gather launch after it takes the remaining layers with the rank map. Workgroup 0 selects,
// workgroups 1..sum_groups compute the chunks' relative deviations (as in select.hip), the rest
// gather.
//
// The gather's work items are one pass of the workgroup each (RPP rows: every head of RPP / H
// consecutive tokens of one segment and layer), tile fastest, strided over the gather
// workgroups; each workgroup keeps two items in flight: the next item's loads (and its cos/sin
// table) go out before the current item's rotation and stores, so reads and writes overlap
// (measured against the previous form, whose next-item loads waited on a vector descriptor load
// and on register moves: the three launches of ckv_layer1_repair_gather 0.7-0.9 us shorter at
// 8k positions). The per-item work and rounding are rerope_gather's (gather_common.hpp).
#include <atomic>

#include "gather_common.hpp"
#include "launch.hpp"

namespace ckv {

// rows per item (one per thread group of D/2 / VEC threads): kSelThreads / that
template <int DTYPE, int D>
constexpr int pre_rows() {
  return kSelThreads / (D / 2 / Elem<DTYPE>::kVec);
}

template <int DTYPE, int D>
__device__ __forceinline__ void pregather_items(const PreGather& g, int it, int stride) {
  using E = Elem<DTYPE>;
  constexpr int VEC = E::kVec;
  constexpr int HALF = D / 2;
  constexpr int TPR = HALF / VEC;
  constexpr int RPP = pre_rows<DTYPE, D>();
  constexpr int RPW = kWave / TPR;  // rows per wavefront
  constexpr int ROW_B = D * E::kBytes;
  constexpr int HALF_B = HALF * E::kBytes;
  static_assert(kSelThreads % TPR == 0 && kSelThreads >= HALF && kWave % TPR == 0, "rows must tile the workgroup");
  typedef __attribute__((address_space(4))) const int32_t ci32;
  typedef __attribute__((address_space(4))) const uint64_t cu64;
  __shared__ float2 cs_tab[2][HALF];  // the cos/sin tables of the two items in flight

  // each cos/sin lane's inverse frequency from the argument scalars (no vector load)
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
  const int ln = (int)threadIdx.x % kWave;
  float my_inv = 0.0f;
#pragma unroll
  for (int k = 0; k < HALF; ++k) {
    if (k / kWave == wave) my_inv = ln == k % kWave ? g.inv.v[k] : my_inv;  // uniform test, scalar operand
  }
  // row r = threadIdx.x / TPR of an item: head r / tpi, token r % tpi. The host checks that
  // n_heads divides kSelWaves, so tpi is a multiple of RPW and a wavefront's rows are
  // consecutive tokens of one head.
  const int col = (int)threadIdx.x % TPR;
  const int tpi = RPP / g.n_heads;  // tokens per item
  const int head = __builtin_amdgcn_readfirstlane((wave * RPW) / tpi);
  const int wtok = __builtin_amdgcn_readfirstlane((wave * RPW) % tpi);  // the wavefront's first token
  const int wrow = ln / TPR;                                            // this lane's row in the wavefront
  const int tok = wtok + wrow;

  // Rows move through buffer loads and stores: a slot's source and destination are a
  // per-wavefront base (scalar) plus a small per-lane offset, and a lane with no row (past the
  // segment, no item) takes an offset past the buffer's range, which the hardware drops (loads
  // return 0, no memory access). The loads are then unconditional: no branch joins the
  // registers of the item in flight, which would make the compiler wait for its loads there.
  // Descriptors and chunk addresses come through the constant address space as scalar loads
  // (nothing in the launch writes them), so waiting for them never waits for row loads.
  constexpr unsigned kRange = (unsigned)(RPW * ROW_B);  // bytes a wavefront's rows span
  constexpr unsigned kDead = 0x40000000u;               // an offset past every range
  constexpr int kNt = 2;                                // non-temporal (read / written once)
  // base is the same in every lane; read it from the first one so the descriptor is built in
  // scalar registers (through uint32_t: an int would sign-extend the low word into the high one)
  auto rsrc = [](const void* base) {
    const uint64_t v = (uint64_t)base;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), (short)0, (int)kRange, 0x00020000);
  };
  struct Slot {
    vec16 k1, k2, v1, v2;
    char* dk;  // the wavefront's destination rows (K, V)
    char* dv;
    unsigned off;  // this lane's offset in them (kDead: no row)
    bool rot;
  };
  // item -> (tile, segment, layer): its loads and its cos/sin table
  auto prepare = [&](int item, Slot& sl, float2* tab) {
    const bool in = item < g.n_items;  // uniform
    const int itc = in ? item : 0;
    const int tile = itc % g.tiles, rest = itc / g.tiles;
    const int layer = g.layer_begin + rest / g.n_segs;
    ci32* f = (ci32*)(g.segs + rest % g.n_segs);
    const ckv_segment s{f[0], f[1], f[2], f[3], f[4], f[5]};
    const int t0 = tile * tpi;
    bool ok = in && t0 < s.n_tokens;  // uniform: an item inside its segment
    if (ok && (s.dst_start < 0 || s.src_start < 0 || s.chunk < 0 || s.chunk >= g.n_tab_chunks ||
               (int64_t)s.dst_start + s.n_tokens > g.n_tokens || (int64_t)s.src_start + s.n_tokens > s.src_len)) {
      if (threadIdx.x == 0) flag_error(g.err, CKV_DEVICE_ERR_RANGE);
      ok = false;
    }
    const char* src_k = g.dk;  // any address: a lane with no row touches no memory
    const char* src_v = g.dk;
    if (ok) {  // uniform
      const int64_t ti = ((int64_t)s.chunk * g.n_layers + layer) * 2;
      const int64_t so = ((int64_t)head * s.src_len + s.src_start + t0 + wtok) * ROW_B;
      src_k = reinterpret_cast<const char*>(((cu64*)g.tab)[ti]) + so;
      src_v = reinterpret_cast<const char*>(((cu64*)g.tab)[ti + 1]) + so;
    }
    const int64_t d = (int64_t)layer * g.ls_b + (int64_t)head * g.hs_b + (int64_t)(s.dst_start + t0 + wtok) * ROW_B;
    sl.dk = g.dk + (ok ? d : 0);
    sl.dv = g.dv + (ok ? d : 0);
    sl.rot = ok && s.delta != 0;
    if (sl.rot && (int)threadIdx.x < HALF) tab[threadIdx.x] = shift_cos_sin(my_inv, s.delta);
    const bool live = ok && tok < s.n_tokens - t0;
    sl.off = live ? (unsigned)(wrow * ROW_B + col * 16) : kDead;
    const auto rk = rsrc(src_k), rv = rsrc(src_v);
    sl.k1 = __builtin_amdgcn_raw_buffer_load_b128(rk, sl.off, 0, kNt);
    sl.k2 = __builtin_amdgcn_raw_buffer_load_b128(rk, sl.off + HALF_B, 0, kNt);
    sl.v1 = __builtin_amdgcn_raw_buffer_load_b128(rv, sl.off, 0, kNt);
    sl.v2 = __builtin_amdgcn_raw_buffer_load_b128(rv, sl.off + HALF_B, 0, kNt);
  };
  auto finish = [&](const Slot& sl, const float2* tab) {
    vec16 y1 = sl.k1, y2 = sl.k2;
    if (sl.rot) {  // uniform
      float c[VEC], sn[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float2 t = tab[col * VEC + e];
        c[e] = t.x;
        sn[e] = t.y;
      }
      rotate_pairs<DTYPE>(sl.k1, sl.k2, c, sn, y1, y2);
    }
    const auto rk = rsrc(sl.dk), rv = rsrc(sl.dv);
    __builtin_amdgcn_raw_buffer_store_b128(y1, rk, sl.off, 0, kNt);
    __builtin_amdgcn_raw_buffer_store_b128(y2, rk, sl.off + HALF_B, 0, kNt);
    __builtin_amdgcn_raw_buffer_store_b128(sl.v1, rv, sl.off, 0, kNt);
    __builtin_amdgcn_raw_buffer_store_b128(sl.v2, rv, sl.off + HALF_B, 0, kNt);
  };

  // Slots a and b alternate (the loop body twice, no copy between them: a copy of a slot whose
  // loads are in flight would wait for them). The barriers order LDS only (the cos/sin tables),
  // so the next item's row loads stay in flight across them.
  Slot a, b;
  prepare(it, a, cs_tab[0]);
  for (;;) {
    it += stride;
    prepare(it, b, cs_tab[1]);  // the next item's loads go out before this item's stores
    lds_barrier();              // this item's table written
    finish(a, cs_tab[0]);
    if (it >= g.n_items) break;  // uniform
    lds_barrier();               // this item's table read: the next prepare may rewrite it
    it += stride;
    prepare(it, a, cs_tab[0]);
    lds_barrier();
    finish(b, cs_tab[1]);
    if (it >= g.n_items) break;
    lds_barrier();
  }
}
#ifndef CKV_PREGATHER_BYTES_PER_POS
#define CKV_PREGATHER_BYTES_PER_POS 8192
#endif

template <int KPT, int DTYPE, int D>
__global__ __launch_bounds__(kSelThreads) void select_gather_kernel(const float* diff, const uint8_t* flags,
                                                                    const int32_t* local, uint32_t* ghist,
                                                                    const ckv_chunk_span* chunks, int n_tokens,
                                                                    int n_chunks, int hist_copies, SelectArgs a,
                                                                    const PreGather g) {
  extern __shared__ uint32_t masks[];  // esc[W], pool[W]: spans of escalated / pooled chunks
  const int sel_blocks = 1 + g.sum_groups;
  if ((int)blockIdx.x >= sel_blocks) {  // uniform: a gather workgroup
    pregather_items<DTYPE, D>(g, (int)blockIdx.x - sel_blocks, (int)gridDim.x - sel_blocks);
    return;
  }
  a.diff = diff;
  a.flags = flags;
  a.local = local;
  a.chunks = chunks;
  a.n_tokens = n_tokens;
  a.n_chunks = n_chunks;
  a.hist_copies = hist_copies;
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

static int pre_rows_of(int dtype, int head_dim) {
  if (dtype == CKV_DTYPE_BF16) return head_dim == 64 ? pre_rows<CKV_DTYPE_BF16, 64>() : pre_rows<CKV_DTYPE_BF16, 128>();
  return head_dim == 64 ? pre_rows<CKV_DTYPE_F32, 64>() : pre_rows<CKV_DTYPE_F32, 128>();
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
  const int rows = pre_rows_of(dtype, head_dim);
  // an item is every head of rows / n_heads tokens, a wavefront's rows one head's
  if (rows % n_heads != 0 || kSelWaves % n_heads != 0) return 0;
  const int tpi = rows / n_heads;
  // whole layers of about CKV_PREGATHER_BYTES_PER_POS bytes per position in all (the HBM traffic
  // that fits the selection's time), on the CUs the selection leaves free
  const int64_t sum_groups = ((int64_t)n_chunks + kSelWaves - 1) / kSelWaves;
  const int64_t per_layer_tiles = ((int64_t)max_seg_tokens + tpi - 1) / tpi * n_segs;
  const int64_t eb = dtype == CKV_DTYPE_BF16 ? 2 : 4;
  const int64_t per_layer_bytes = per_layer_tiles * tpi * n_heads * head_dim * eb * 4;
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
  const int tpi = pre_rows_of(dtype, head_dim) / g.n_heads;
  g.tiles = (max_seg_tokens + tpi - 1) / tpi;
  g.n_items = k * g.tiles * g.n_segs;
  // one 1024-thread workgroup per CU the selection leaves free (no more than there are items)
  const int blocks = std::min<int>(g.n_items, cu_count() - 1 - g.sum_groups);
  g.inv = host_inv_freq(head_dim, theta);
  const dim3 grid((unsigned)(1 + g.sum_groups + blocks));
#define CKV_SG(K, DT, HD)                                                                                      \
  if (kpt <= K && dtype == DT && head_dim == HD) {                                                              \
    hipLaunchKernelGGL((select_gather_kernel<K, DT, HD>), grid, dim3(kSelThreads), lds, st, args.diff, args.flags, \
                       args.local, ghist, args.chunks, args.n_tokens, args.n_chunks, args.hist_copies, args, g); \
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
