// One workgroup's tile of the re-RoPE gather (the body of rerope_gather_kernel, also run by the
// selection launch's gather workgroups): the rows of tokens [tile * TILE, +TILE) of segment
// seg_index (or of one_seg when segs is NULL), every head, of one layer, re-rotated by the
// segment's shift. With SKIP, skip (may be NULL) leaves the rows of positions with skip[p] >= 0
// alone (tiles of at most 32 tokens); without, every row of the tile is written and skip unused.
//
// Reference semantics (src/chunkkv/engine/torch_engine.py):
//   inv_freq           :33   base ** (-arange(0, D, 2) / D)            (fp32)
//   _rotate            :46-51  y1 = x1*cos - x2*sin, y2 = x1*sin + x2*cos in fp32, rounded
//                               once to the element type; halves are [0, D/2) and [D/2, D)
//   shift_keys         :56-59  angles = delta * inv_freq, same for every token; delta == 0
//                               returns the keys unchanged
//   base_kv            :96-103 per layer, per placement: K[:, :, s:e] = shift_keys(chunk K),
//                               V[:, :, s:e] = chunk V
//
// The workgroup builds a D/2-entry cos/sin table in LDS once, from the inverse frequencies
// (computed from theta on the host, passed by value in the kernel arguments), while its first
// 16-byte loads are in flight. The table holds the correctly rounded fp32 cos/sin of the fp32
// angle (evaluated in fp64, rounded once). Every thread then rotates VEC frequency pairs (the 16
// bytes at column c of the first half and the matching 16 bytes of the second half) of UNROLL
// rows per pass. Memory traffic is one read and one write of every gathered byte. Products and
// sums are separately rounded fp32 operations (built with -ffp-contract=off).
#pragma once

#include "ckv_common.hpp"

namespace ckv {

#ifndef CKV_GATHER_NT_LOAD
#define CKV_GATHER_NT_LOAD 1
#endif

__device__ __forceinline__ vec16 gather_ld(const void* p) {
  if constexpr (CKV_GATHER_NT_LOAD) return ld16_stream(p);
  else return ld16(p);
}

// ST_K / ST_V: the StorePolicy of the key rows' and the value rows' stores.
template <int DTYPE, int D, int THREADS, int TILE, int UNROLL, bool SKIP, int ST_K = kStStream,
          int ST_V = kStStream>
__device__ __forceinline__ void gather_tile(
    char* __restrict__ dst_k, char* __restrict__ dst_v, int64_t dst_layer_stride_b, int64_t dst_head_stride_b,
    const uint64_t* __restrict__ src_tab, int n_chunks, const ckv_segment* __restrict__ segs, int seg_index,
    ckv_segment one_seg, uint64_t one_src_k, uint64_t one_src_v, int64_t one_src_head_stride_b, int n_layers,
    int layer, int tile, int n_heads, int n_tokens, const int32_t* __restrict__ skip, const InvFreq& inv,
    int32_t* __restrict__ err) {
  using E = Elem<DTYPE>;
  constexpr int VEC = E::kVec;
  constexpr int HALF = D / 2;
  static_assert(HALF % VEC == 0, "head_dim/2 must be a multiple of the vector width");
  constexpr int TPR = HALF / VEC;                  // threads per row
  constexpr int kGatherThreads = THREADS, kGatherTile = TILE, kGatherUnroll = UNROLL;
  constexpr int RPP = kGatherThreads / TPR;        // rows per pass of the workgroup
  constexpr int64_t ROW_B = (int64_t)D * E::kBytes;
  constexpr int HALF_B = HALF * E::kBytes;
  static_assert(kGatherThreads % TPR == 0, "rows must tile the workgroup");
  static_assert(kGatherThreads >= HALF, "one thread per cos/sin table entry");

  __shared__ float2 cs_tab[HALF];  // this workgroup's cos/sin of the shift

  // the inverse frequency of each cos/sin lane, assembled from the argument segment's scalars
  // (lane k of the evaluating wavefront gets inv[k]): the evaluation below then depends on no
  // vector load, so it runs while the row loads are in flight (a vector load of its own would
  // wait for every row load issued before it)
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
  const int ln = (int)threadIdx.x % kWave;
  float my_inv = 0.0f;
#pragma unroll
  for (int k = 0; k < HALF; ++k) {
    if (k / kWave == wave) my_inv = ln == k % kWave ? inv.v[k] : my_inv;  // uniform test, scalar operand
  }

  ckv_segment s = one_seg;
  if (segs != nullptr) {
    typedef __attribute__((address_space(1))) const int32_t gi32;
    gi32* f = (gi32*)(segs + seg_index);
    s = ckv_segment{f[0], f[1], f[2], f[3], f[4], f[5]};
  }
  const int t0 = tile * kGatherTile;
  if (t0 >= s.n_tokens) return;  // uniform: tile past this segment's end
  if (s.dst_start < 0 || s.src_start < 0 || s.chunk < 0 || s.chunk >= n_chunks ||
      (int64_t)s.dst_start + s.n_tokens > n_tokens ||
      (int64_t)s.src_start + s.n_tokens > s.src_len) {
    if (threadIdx.x == 0) flag_error(err, CKV_DEVICE_ERR_RANGE);
    return;
  }

  const char* src_k;
  const char* src_v;
  int64_t src_head_b;
  if (segs != nullptr) {
    const int64_t ti = ((int64_t)s.chunk * n_layers + layer) * 2;
    src_k = reinterpret_cast<const char*>(src_tab[ti]);
    src_v = reinterpret_cast<const char*>(src_tab[ti + 1]);
    src_head_b = (int64_t)s.src_len * ROW_B;
  } else {
    src_k = reinterpret_cast<const char*>(one_src_k);
    src_v = reinterpret_cast<const char*>(one_src_v);
    src_head_b = one_src_head_stride_b;
  }
  const bool with_v = src_v != nullptr && dst_v != nullptr;

  const int ntok = min(kGatherTile, s.n_tokens - t0);
  const int rows = n_heads * kGatherTile;  // (head, token) grid of the tile; tokens >= ntok idle
  const int col = threadIdx.x % TPR;
  const int rl = threadIdx.x / TPR;
  const int64_t col_b = (int64_t)col * 16;

  const char* sk0 = src_k + (int64_t)(s.src_start + t0) * ROW_B + col_b;
  const char* sv0 = with_v ? src_v + (int64_t)(s.src_start + t0) * ROW_B + col_b : nullptr;
  char* dk0 = dst_k + (int64_t)layer * dst_layer_stride_b + (int64_t)(s.dst_start + t0) * ROW_B + col_b;
  char* dv0 = with_v ? dst_v + (int64_t)layer * dst_layer_stride_b + (int64_t)(s.dst_start + t0) * ROW_B + col_b
                     : nullptr;

  vec16 kx1[kGatherUnroll], kx2[kGatherUnroll], vx1[kGatherUnroll], vx2[kGatherUnroll];
  bool live[kGatherUnroll];

  // A row is gathered unless its token lies past the segment or skip marks it (skip[p] >= 0:
  // an active position whose row the fresh K/V provides). The tile's skip entries come in
  // together as scalar loads beside the chunk addresses (indices clamped into the segment) and
  // make one mask, so no row load waits for a skip load of its own.
  static_assert(!SKIP || kGatherTile <= 32, "the skip mask holds 32 tokens");
  uint32_t skipped = 0u;  // bit t: token t0 + t is skipped
  if (SKIP && skip != nullptr) {  // uniform
    const int base = s.dst_start + t0;
    int sv[kGatherTile];
    if (base + kGatherTile <= n_tokens) {  // adjacent entries: merged into wide scalar loads
#pragma unroll
      for (int t = 0; t < kGatherTile; ++t) sv[t] = skip[base + t];
    } else {  // the request's last tile: indices clamped (entries past the tile are not used)
#pragma unroll
      for (int t = 0; t < kGatherTile; ++t) sv[t] = skip[min(base + t, n_tokens - 1)];
    }
#pragma unroll
    for (int t = 0; t < kGatherTile; ++t) skipped |= (sv[t] >= 0 ? 1u : 0u) << t;
  }
  auto row_ok = [&](int r) {
    const int tok = r % kGatherTile;
    return r < rows && tok < ntok && !(SKIP && ((skipped >> (SKIP ? tok : 0)) & 1u));
  };
  auto src_off = [&](int r) { return (int64_t)(r / kGatherTile) * src_head_b + (int64_t)(r % kGatherTile) * ROW_B; };
  auto dst_off = [&](int r) { return (int64_t)(r / kGatherTile) * dst_head_stride_b + (int64_t)(r % kGatherTile) * ROW_B; };

  auto issue_loads = [&](int r0) {
#pragma unroll
    for (int u = 0; u < kGatherUnroll; ++u) {
      const int r = r0 + u * RPP + rl;
      live[u] = row_ok(r);
      if (live[u]) {
        const int64_t o = src_off(r);
        kx1[u] = gather_ld(sk0 + o);
        kx2[u] = gather_ld(sk0 + o + HALF_B);
        if (with_v) {
          vx1[u] = gather_ld(sv0 + o);
          vx2[u] = gather_ld(sv0 + o + HALF_B);
        }
      }
    }
  };

  issue_loads(0);

  // cos/sin of this segment's shift for every frequency, computed once per workgroup.
  const bool rotate = s.delta != 0;
  float c[VEC], sn[VEC];
  if (rotate) {
    if (threadIdx.x < HALF) cs_tab[threadIdx.x] = shift_cos_sin(my_inv, s.delta);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float2 t = cs_tab[col * VEC + e];
      c[e] = t.x;
      sn[e] = t.y;
    }
  }

  for (int r0 = 0;;) {
#pragma unroll
    for (int u = 0; u < kGatherUnroll; ++u) {
      const int r = r0 + u * RPP + rl;
      if (live[u]) {
        const int64_t o = dst_off(r);
        // one store per half whichever the shift (stores in both arms of a branch get merged by
        // the compiler, which then drops a non-temporal hint the arms share)
        vec16 y1 = kx1[u], y2 = kx2[u];
        if (rotate) rotate_pairs<DTYPE>(kx1[u], kx2[u], c, sn, y1, y2);
        st16_policy<ST_K>(dk0 + o, y1);
        st16_policy<ST_K>(dk0 + o + HALF_B, y2);
        if (with_v) {
          st16_policy<ST_V>(dv0 + o, vx1[u]);
          st16_policy<ST_V>(dv0 + o + HALF_B, vx2[u]);
        }
      }
    }
    r0 += kGatherUnroll * RPP;
    if (r0 >= rows) break;
    issue_loads(r0);
  }
}

}  // namespace ckv
