// Layer-1 repair decision in one launch (ckv_deviation_select): the fresh-vs-cached deviation of
// every active position, fused with the per-chunk relative deviation and escalation, the pooled
// top-k with forced sinks, and the compaction of the new active set.
//
// Reference semantics: src/chunkkv/engine/torch_engine.py:117-153; deviation_common.hpp and
// select_common.hpp restate them step by step. Results are bit-identical to ckv_deviation
// followed by ckv_select.
//
// Design (gfx950): 1024-thread workgroups, at most one per CU, each wavefront kDsTok token
// positions of a tile at a time.
//  1. Every workgroup computes its tiles' deviations in the fixed summation order, writes
//     diff/norm, and counts each position that is cached, pooled and not a sink (a candidate
//     when no chunk escalates) into the selection's top_bin histogram (4096 bins) in the workspace, one
//     global atomic per distinct bin of a tile.
//  2. The writes are device-scope stores and atomics (the L2s of the XCDs are not coherent with
//     each other) and each wavefront waits for its own to complete; then one atomic ticket per
//     workgroup finds the last workgroup to finish. The others exit; none waits for another.
//  3. The last workgroup acquires and runs the selection (select_run) with the histogram: the
//     threshold's bin comes from one scan over it and only that bin's candidates are ranked.
//     If the histogram does not match the candidate set (a chunk escalated, or the flags'
//     pooled bit disagrees with the spans), or the threshold falls outside the histogram's
//     window, the selection runs its full four passes.
//  4. The last workgroup leaves the histogram and the ticket zeroed: the workspace needs
//     clearing once, before its first use, and never again.
// Up to 33792 positions (33 per thread of the selecting workgroup); larger requests run
// ckv_deviation and ckv_select as two launches.
#include <mutex>

#include "deviation_common.hpp"
#include "select_common.hpp"

namespace ckv {

constexpr int kWsTicket = kTopBins;  // workspace word index of the ticket (after the histogram)
static_assert((kTopBins + 64) * 4 == CKV_DEVIATION_SELECT_WORKSPACE_BYTES, "workspace layout");

#ifndef CKV_DEVSEL_TOK
#define CKV_DEVSEL_TOK 3
#endif
constexpr int kDsTok = CKV_DEVSEL_TOK;                // token positions per wavefront
constexpr int kDsTokPerGroup = kSelWaves * kDsTok;   // per workgroup
static_assert(kDsTokPerGroup <= kWave, "one lane of wavefront 0 per position of the workgroup");

__device__ __forceinline__ void wait_vmem() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wavefront's stores and atomics have completed
  asm volatile("" ::: "memory");
}

template <int DTYPE, int KPT>
__global__ __launch_bounds__(kSelThreads) void deviation_select_kernel(DevArgs d, SelectArgs s, float* __restrict__ diff,
                                                                       float* __restrict__ norm, uint32_t* ws) {
  extern __shared__ uint32_t masks[];  // the selection's esc[W], pool[W]
  __shared__ uint32_t s_bin[kDsTokPerGroup];  // each position's histogram bin, or ~0u
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  uint32_t* ghist = ws;
  uint32_t* ticket = ws + kWsTicket;
  // the spans the selection's wavefront `wave` starts from, loaded while the deviations run
  ckv_chunk_span sp[kSelPre<KPT>];
  load_first_spans<KPT>(s.chunks, s.n_chunks, __builtin_amdgcn_readfirstlane(wave), sp);

  // Tiles of kDsTokPerGroup consecutive positions, strided over a grid of at most one workgroup
  // per CU (the selection's registers leave room for one 1024-thread workgroup per CU): a grid
  // just above the CU count would run its last workgroups as a second round.
  const int n_tiles = (d.n_tokens + kDsTokPerGroup - 1) / kDsTokPerGroup;
  for (int tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {  // uniform per workgroup
    const int p0 = tile * kDsTokPerGroup + wave * kDsTok;
    float dv[kDsTok], nv[kDsTok];
    uint32_t fl[kDsTok];
    deviation_wave<DTYPE, kDsTok>(d, p0, dv, nv, fl);
    // diff/norm go out as device-scope stores (global_store sc1: coherent across the XCDs once
    // complete), waited for (vmcnt 0) before the ticket below. An agent-scope release fence
    // would instead write back the XCD's whole L2 (buffer_wbl2), once per wavefront: ~130 us
    // per launch at 8192 positions, against the writes' few kilobytes.
    if (lane == 0) {
#pragma unroll
      for (int t = 0; t < kDsTok; ++t) {
        const int p = p0 + t;
        uint32_t bin = ~0u;
        if (p < d.n_tokens) {
          __hip_atomic_store(diff + p, dv[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(norm + p, nv[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if ((fl[t] & CKV_POS_CACHED) && !(fl[t] & CKV_POS_SINK) && (fl[t] & CKV_POS_POOLED))
            bin = top_bin(dev_key(dv[t]));
        }
        s_bin[wave * kDsTok + t] = bin;
      }
    }
    lds_barrier();
    if (wave == 0) {
      // One device-scope atomic per distinct bin of the tile, adding its count: neighbouring
      // positions mostly share a bin, and same-address device atomics serialise far from the CU
      // (one atomic per position cost ~25 us per launch at 8192 positions).
      const uint32_t bin = lane < kDsTokPerGroup ? s_bin[lane] : ~0u;
      uint32_t count = 0;
      bool first = true;
#pragma unroll
      for (int j = 0; j < kDsTokPerGroup; ++j) {
        const uint32_t b = s_bin[j];
        count += b == bin;
        first = first && !(j < lane && b == bin);
      }
      if (bin != ~0u && first)
        __hip_atomic_fetch_add(&ghist[bin], count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    lds_barrier();  // s_bin is rewritten by the next tile
  }
  wait_vmem();  // this wavefront's stores and atomics have completed
  __syncthreads();
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
  __syncthreads();
  if (!s_last) return;  // uniform per workgroup
  // The other workgroups' diff/norm and histogram counts completed before their tickets.
  // Acquire: invalidate this XCD's caches, which may hold stale lines of those buffers from
  // earlier launches (~2 us). Reading them with device-scope loads instead measured slower: those
  // loads did not overlap (7 us for the selection's first loads against 3.7 us).
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  select_run<KPT>(s, ghist, masks, sp);
  if (tid == 0) __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int DTYPE>
static int32_t launch_devsel(int kpt, unsigned blocks, size_t lds, hipStream_t st, const DevArgs& d,
                             const SelectArgs& s, float* diff, float* norm, uint32_t* ws) {
#define CKV_DEVSEL(K)                                                                                       \
  if (kpt <= K) {                                                                                           \
    hipLaunchKernelGGL((deviation_select_kernel<DTYPE, K>), dim3(blocks), dim3(kSelThreads), lds, st, d, s, \
                       diff, norm, ws);                                                                     \
    CKV_RETURN_IF_LAUNCH_FAILED();                                                                          \
    return CKV_OK;                                                                                          \
  }
  CKV_DEVSEL(4)
  CKV_DEVSEL(8)
  CKV_DEVSEL(12)
  CKV_DEVSEL(16)
  CKV_DEVSEL(24)
  CKV_DEVSEL(33)
#undef CKV_DEVSEL
  return CKV_ERR_TOO_LARGE;
}

}  // namespace ckv

extern "C" int32_t ckv_deviation_select(
    const void* k_fresh, int64_t kf_head_stride, int64_t kf_token_stride, const void* v_fresh, int64_t vf_head_stride,
    int64_t vf_token_stride, const void* k_cache, const void* v_cache, int64_t cache_head_stride,
    const uint8_t* pos_flags, const int32_t* local, int32_t n_tokens, int32_t n_fresh, int32_t n_heads,
    int32_t head_dim, int32_t dtype, const ckv_chunk_span* chunks, int32_t n_chunks, int32_t has_threshold,
    double escalate_threshold, float* diff, float* norm, int64_t* keep_abs, int64_t* keep_local, int32_t* keep_rank,
    float* rel_dev, uint8_t* escalated, int32_t* counts, void* workspace, int64_t workspace_bytes, int32_t* err,
    void* stream) {
  using namespace ckv;
  if (dtype != CKV_DTYPE_BF16 && dtype != CKV_DTYPE_F32) return CKV_ERR_INVALID_ARGUMENT;
  const int vec = dtype == CKV_DTYPE_BF16 ? 8 : 4;
  if (head_dim <= 0 || head_dim % vec != 0 || n_heads <= 0 || n_tokens < 0 || n_fresh < 0 || n_chunks < 0)
    return CKV_ERR_INVALID_ARGUMENT;
  if (pos_flags == nullptr || local == nullptr || diff == nullptr || norm == nullptr || k_cache == nullptr ||
      v_cache == nullptr || (n_fresh > 0 && (k_fresh == nullptr || v_fresh == nullptr)) || keep_abs == nullptr ||
      keep_local == nullptr || counts == nullptr)
    return CKV_ERR_INVALID_ARGUMENT;
  if (n_chunks > 0 && (chunks == nullptr || rel_dev == nullptr || escalated == nullptr))
    return CKV_ERR_INVALID_ARGUMENT;
  if (cache_head_stride < (int64_t)n_tokens * head_dim) return CKV_ERR_OUT_OF_RANGE;
  if (n_tokens > CKV_SELECT_MAX_TOKENS) return CKV_ERR_TOO_LARGE;
  const int kpt = (n_tokens + kSelThreads - 1) / kSelThreads;
  if (n_tokens == 0 || kpt > 33) {  // beyond the one-launch form: the two launches it fuses
    const int32_t rc = ckv_deviation(k_fresh, kf_head_stride, kf_token_stride, v_fresh, vf_head_stride,
                                     vf_token_stride, k_cache, v_cache, cache_head_stride, pos_flags, local,
                                     n_tokens, n_fresh, n_heads, head_dim, dtype, diff, norm, err, stream);
    if (rc != CKV_OK) return rc;
    return ckv_select(diff, norm, pos_flags, local, n_tokens, chunks, n_chunks, has_threshold, escalate_threshold,
                      keep_abs, keep_local, keep_rank, rel_dev, escalated, counts, stream);
  }
  if (workspace == nullptr || workspace_bytes < CKV_DEVIATION_SELECT_WORKSPACE_BYTES || (uintptr_t)workspace % 16)
    return CKV_ERR_INVALID_ARGUMENT;
  const int64_t eb = dtype == CKV_DTYPE_BF16 ? 2 : 4;
  const DevArgs d{(const char*)k_fresh, kf_head_stride * eb, kf_token_stride * eb, (const char*)v_fresh,
                  vf_head_stride * eb, vf_token_stride * eb, (const char*)k_cache, (const char*)v_cache,
                  cache_head_stride * eb, pos_flags, local, (int)n_tokens, (int)n_fresh, (int)n_heads,
                  (int)head_dim, err};
  const SelectArgs s{diff,     norm,     pos_flags, local,      (int)n_tokens, chunks,   (int)n_chunks,
                     (int)(has_threshold != 0), escalate_threshold, keep_abs, keep_local, keep_rank, rel_dev,
                     escalated, counts};
  int dev = 0, n_cu = 0;
  if (hipStreamGetDevice((hipStream_t)stream, &dev) != hipSuccess ||
      hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
    return CKV_ERR_HIP;
  const int n_tiles = (n_tokens + kDsTokPerGroup - 1) / kDsTokPerGroup;
  const unsigned blocks = (unsigned)(n_tiles < n_cu ? n_tiles : n_cu);
  const size_t lds = (size_t)((n_tokens + 31) / 32) * 2 * sizeof(uint32_t);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == CKV_DTYPE_BF16)
    return launch_devsel<CKV_DTYPE_BF16>(kpt, blocks, lds, st, d, s, diff, norm, (uint32_t*)workspace);
  return launch_devsel<CKV_DTYPE_F32>(kpt, blocks, lds, st, d, s, diff, norm, (uint32_t*)workspace);
}

// ---- the same call for callers that cannot allocate (ckv_deviation_select_noalloc) ----------
//
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
