// Assemble one layer's K/V cache: every row written exactly once, either the freshly computed
// row of an active position or the cached chunk row re-rotated to its new offset.
//
// Reference semantics (src/chunkkv/engine/torch_engine.py): per layer the reference first builds
// the base cache (:96-103, every cached row shifted and copied, uncached rows zero) and then
// overwrites the active rows with the fresh K/V (:155-156). The result of that pair is, row by
// row: fresh row if the position is active, else the re-rotated cached row. Uncached positions
// are always active, so no zero row survives. This kernel produces that result directly, so
// rows of active positions are never gathered only to be overwritten (at layer 0 of a request
// without exact placements that is every row).
//
// Design (gfx950): segments cover the request: cached runs (chunk >= 0, same descriptors as the
// gather) and uncached runs (chunk == -1). One workgroup = one (segment, 16-token tile). Each
// thread looks up local[] for its token, then issues 16-byte loads from the fresh tensors or
// from the chunk store, and rotates cached keys with the segment's cos/sin table (built in LDS
// while the loads are in flight). Same arithmetic as the gather: bit-identical rows.
#include "ckv_common.hpp"

namespace ckv {

#ifndef CKV_ASM_THREADS
#define CKV_ASM_THREADS 256
#endif
#ifndef CKV_ASM_TILE
#define CKV_ASM_TILE 16
#endif
#ifndef CKV_ASM_UNROLL
#define CKV_ASM_UNROLL 2
#endif
constexpr int kAsmThreads = CKV_ASM_THREADS;
constexpr int kAsmTile = CKV_ASM_TILE;  // tokens per workgroup
constexpr int kAsmUnroll = CKV_ASM_UNROLL;  // rows in flight per thread

enum : int { kRowSkip = 0, kRowFresh = 1, kRowCached = 2 };

template <int DTYPE, int D>
__global__ __launch_bounds__(kAsmThreads) void assemble_kernel(
    char* dst_k, char* dst_v, int64_t dst_head_stride_b, const uint64_t* __restrict__ src_tab, int n_chunks,
    int n_layers, int layer, const ckv_segment* __restrict__ segs, const char* __restrict__ kf,
    int64_t kf_hs_b, int64_t kf_ts_b, const char* __restrict__ vf, int64_t vf_hs_b, int64_t vf_ts_b,
    int n_fresh, const int32_t* __restrict__ local, int n_heads, int n_tokens, const InvFreq inv,
    int32_t* __restrict__ err) {
  using E = Elem<DTYPE>;
  constexpr int VEC = E::kVec;
  constexpr int HALF = D / 2;
  static_assert(HALF % VEC == 0, "head_dim/2 must be a multiple of the vector width");
  constexpr int TPR = HALF / VEC;
  constexpr int RPP = kAsmThreads / TPR;
  constexpr int64_t ROW_B = (int64_t)D * E::kBytes;
  constexpr int HALF_B = HALF * E::kBytes;

  __shared__ float2 cs_tab[HALF];

  typedef __attribute__((address_space(1))) const int32_t gi32;
  gi32* f = (gi32*)(segs + blockIdx.x);
  const ckv_segment s{f[0], f[1], f[2], f[3], f[4], f[5]};
  const int t0 = blockIdx.y * kAsmTile;
  if (t0 >= s.n_tokens) return;  // uniform
  const bool has_src = s.chunk >= 0;
  if (s.dst_start < 0 || s.chunk < -1 || s.chunk >= n_chunks || (int64_t)s.dst_start + s.n_tokens > n_tokens ||
      (has_src && (s.src_start < 0 || (int64_t)s.src_start + s.n_tokens > s.src_len))) {
    if (threadIdx.x == 0) flag_error(err, CKV_DEVICE_ERR_RANGE);
    return;
  }
  const char* sk = nullptr;
  const char* sv = nullptr;
  if (has_src) {
    const int64_t ti = ((int64_t)s.chunk * n_layers + layer) * 2;
    sk = reinterpret_cast<const char*>(src_tab[ti]) + (int64_t)s.src_start * ROW_B;
    sv = reinterpret_cast<const char*>(src_tab[ti + 1]) + (int64_t)s.src_start * ROW_B;
  }
  const int64_t src_head_b = (int64_t)s.src_len * ROW_B;

  const int ntok = min(kAsmTile, s.n_tokens - t0);
  const int rows = n_heads * kAsmTile;
  const int col = threadIdx.x % TPR;
  const int rl = threadIdx.x / TPR;
  const int64_t col_b = (int64_t)col * 16;

  const bool rotate = has_src && s.delta != 0;
  float c[VEC], sn[VEC];

  for (int r0 = 0; r0 < rows; r0 += kAsmUnroll * RPP) {
    int mode[kAsmUnroll];
    int64_t src_o[kAsmUnroll], dst_o[kAsmUnroll];
    vec16 kx1[kAsmUnroll], kx2[kAsmUnroll], vx1[kAsmUnroll], vx2[kAsmUnroll];
#pragma unroll
    for (int u = 0; u < kAsmUnroll; ++u) {
      const int r = r0 + u * RPP + rl;
      const int tok = r % kAsmTile, h = r / kAsmTile;
      mode[u] = kRowSkip;
      if (r < rows && tok < ntok) {
        const int p = s.dst_start + t0 + tok;
        const int lp = local != nullptr ? local[p] : -1;
        dst_o[u] = (int64_t)h * dst_head_stride_b + (int64_t)p * ROW_B + col_b;
        if (lp >= 0 && lp < n_fresh) {
          mode[u] = kRowFresh;
          src_o[u] = 0;
          const char* kr = kf + h * kf_hs_b + (int64_t)lp * kf_ts_b + col_b;
          const char* vr = vf + h * vf_hs_b + (int64_t)lp * vf_ts_b + col_b;
          kx1[u] = ld16_stream(kr);
          kx2[u] = ld16_stream(kr + HALF_B);
          vx1[u] = ld16_stream(vr);
          vx2[u] = ld16_stream(vr + HALF_B);
        } else if (lp < 0 && has_src) {
          mode[u] = kRowCached;
          src_o[u] = (int64_t)h * src_head_b + (int64_t)(t0 + tok) * ROW_B + col_b;
          kx1[u] = ld16_stream(sk + src_o[u]);
          kx2[u] = ld16_stream(sk + src_o[u] + HALF_B);
          vx1[u] = ld16_stream(sv + src_o[u]);
          vx2[u] = ld16_stream(sv + src_o[u] + HALF_B);
        } else if (local != nullptr && col == 0) {
          flag_error(err, CKV_DEVICE_ERR_RANGE);  // active index out of range, or no source row
        }
      }
    }
    if (rotate && r0 == 0) {  // uniform; the table is built once, behind the first loads
      if (threadIdx.x < HALF) cs_tab[threadIdx.x] = shift_cos_sin(inv.v[threadIdx.x], s.delta);
      __syncthreads();
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float2 t = cs_tab[col * VEC + e];
        c[e] = t.x;
        sn[e] = t.y;
      }
    }
#pragma unroll
    for (int u = 0; u < kAsmUnroll; ++u) {
      if (mode[u] == kRowSkip) continue;
      char* dk = dst_k + dst_o[u];
      char* dv = dst_v + dst_o[u];
      if (mode[u] == kRowCached && rotate) {
        vec16 y1, y2;
        rotate_pairs<DTYPE>(kx1[u], kx2[u], c, sn, y1, y2);
        st16_stream(dk, y1);
        st16_stream(dk + HALF_B, y2);
      } else {
        st16_stream(dk, kx1[u]);
        st16_stream(dk + HALF_B, kx2[u]);
      }
      st16_stream(dv, vx1[u]);
      st16_stream(dv + HALF_B, vx2[u]);
    }
  }
}

template <int DTYPE, int D>
static void launch_assemble(char* dk, char* dv, int64_t hs_b, const uint64_t* tab, int n_chunks, int n_layers,
                            int layer, const ckv_segment* segs, int n_segs, int max_tiles, const char* kf,
                            int64_t kf_hs_b, int64_t kf_ts_b, const char* vf, int64_t vf_hs_b, int64_t vf_ts_b,
                            int n_fresh, const int32_t* local, int n_heads, int n_tokens, double theta, int32_t* err,
                            hipStream_t st) {
  hipLaunchKernelGGL((assemble_kernel<DTYPE, D>), dim3((unsigned)n_segs, (unsigned)max_tiles), dim3(kAsmThreads), 0,
                     st, dk, dv, hs_b, tab, n_chunks, n_layers, layer, segs, kf, kf_hs_b, kf_ts_b, vf, vf_hs_b,
                     vf_ts_b, n_fresh, local, n_heads, n_tokens, host_inv_freq(D, theta), err);
}

using AssembleFn = void (*)(char*, char*, int64_t, const uint64_t*, int, int, int, const ckv_segment*, int, int,
                            const char*, int64_t, int64_t, const char*, int64_t, int64_t, int, const int32_t*, int,
                            int, double, int32_t*, hipStream_t);

static AssembleFn pick_assemble(int dtype, int head_dim) {
#define CKV_CASE(DT, HD) \
  if (dtype == DT && head_dim == HD) return &launch_assemble<DT, HD>;
  CKV_CASE(CKV_DTYPE_BF16, 64)
  CKV_CASE(CKV_DTYPE_BF16, 128)
  CKV_CASE(CKV_DTYPE_BF16, 256)
  CKV_CASE(CKV_DTYPE_F32, 64)
  CKV_CASE(CKV_DTYPE_F32, 128)
  CKV_CASE(CKV_DTYPE_F32, 256)
#undef CKV_CASE
  return nullptr;
}

}  // namespace ckv

extern "C" int32_t ckv_assemble_layer(void* dst_k, void* dst_v, int64_t dst_head_stride, const uint64_t* src_tab,
                                      int32_t n_chunks, int32_t n_layers, int32_t layer, const ckv_segment* segs,
                                      int32_t n_segs, int32_t max_seg_tokens, const void* k_fresh,
                                      int64_t kf_head_stride, int64_t kf_token_stride, const void* v_fresh,
                                      int64_t vf_head_stride, int64_t vf_token_stride, int32_t n_fresh,
                                      const int32_t* local, int32_t n_tokens, int32_t n_heads, int32_t head_dim,
                                      int32_t dtype, double theta, int32_t* err, void* stream) {
  using namespace ckv;
  AssembleFn fn = pick_assemble(dtype, head_dim);
  if (fn == nullptr || dst_k == nullptr || dst_v == nullptr || segs == nullptr) return CKV_ERR_INVALID_ARGUMENT;
  if (n_chunks < 0 || n_layers <= 0 || layer < 0 || layer >= n_layers || n_segs < 0 || max_seg_tokens < 0 ||
      n_fresh < 0 || n_tokens < 0 || n_heads <= 0 || !(theta > 0.0))
    return CKV_ERR_INVALID_ARGUMENT;
  if (n_chunks > 0 && src_tab == nullptr) return CKV_ERR_INVALID_ARGUMENT;
  if (local != nullptr && n_fresh > 0 && (k_fresh == nullptr || v_fresh == nullptr)) return CKV_ERR_INVALID_ARGUMENT;
  if (dst_head_stride < (int64_t)n_tokens * head_dim) return CKV_ERR_OUT_OF_RANGE;
  if (n_segs == 0 || max_seg_tokens == 0) return CKV_OK;
  const int max_tiles = (max_seg_tokens + kAsmTile - 1) / kAsmTile;
  if (max_tiles > 65535) return CKV_ERR_TOO_LARGE;
  const int64_t eb = dtype == CKV_DTYPE_BF16 ? 2 : 4;
  fn((char*)dst_k, (char*)dst_v, dst_head_stride * eb, src_tab, n_chunks, n_layers, layer, segs, n_segs, max_tiles,
     (const char*)k_fresh, kf_head_stride * eb, kf_token_stride * eb, (const char*)v_fresh, vf_head_stride * eb,
     vf_token_stride * eb, local != nullptr ? n_fresh : 0, local, n_heads, n_tokens, theta, err, (hipStream_t)stream);
  CKV_RETURN_IF_LAUNCH_FAILED();
  return CKV_OK;
}
