// Row scatter shared by the scatter kernel (scatter.hip) and the gather launch that carries a
// layer's kept rows beside the dropped rows of the other layers (rerope_gather.hip).
//
// Reference semantics (src/chunkkv/engine/torch_engine.py:152, :155-156):
//   k, v = k[:, :, sel], v[:, :, sel];  K[:, :, active] = k;  V[:, :, active] = v
// as one bit-exact copy per row: K[h, rows[j]] = k[h, src_rows[j]] (src_rows NULL: j), V likewise.
//
// Item g moves one 16-byte vector of K and the matching vector of V: consecutive items walk a row
// (D elements), then the next head, then the next row, so a row's writes are one contiguous burst
// and the reads follow the source tensor's own strides.
#pragma once

#include "ckv_common.hpp"

namespace ckv {

struct RowScatter {
  char* dk;  // destination cache (H, n_tokens, D), head stride d_hs_b bytes
  char* dv;
  int64_t d_hs_b;
  const char* sk;  // source rows, strides in bytes
  int64_t sk_hs_b, sk_ts_b;
  const char* sv;
  int64_t sv_hs_b, sv_ts_b;
  const int64_t* rows;      // destination row of each scattered row
  const int64_t* src_rows;  // source row of each (NULL: j)
  const int32_t* n_rows_dev;  // NULL, or a row count only the device knows (min with n_rows)
  int n_rows, n_src, n_tokens, n_heads, vecs_per_row;
  int64_t row_b;
};

// Items g0, g0 + stride, ... (U of them) of the scatter: every load before any store;
// non-temporal loads (read once) and stores (no dirty L2 lines left for the kernel boundary).
// A row whose source or destination is out of range is skipped and flagged in err.
template <int U>
__device__ __forceinline__ void scatter_items(const RowScatter& s, int64_t g0, int64_t stride, int32_t* err) {
  int n_rows = s.n_rows;
  if (s.n_rows_dev != nullptr) n_rows = min(n_rows, max(0, *s.n_rows_dev));
  const int64_t per_tok = (int64_t)s.n_heads * s.vecs_per_row;
  const int64_t total = (int64_t)n_rows * per_tok;
  vec16 a[U], b[U];
  int64_t dst_o[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t g = g0 + u * stride;
    dst_o[u] = -1;
    if (g < total) {
      const int64_t j = g / per_tok;
      const int rem = (int)(g - j * per_tok);
      const int h = rem / s.vecs_per_row;
      const int64_t cb = (int64_t)(rem % s.vecs_per_row) * 16;
      const int64_t t = s.rows[j];
      const int64_t js = s.src_rows != nullptr ? s.src_rows[j] : j;
      const bool src_ok = js >= 0 && js < s.n_src;
      if (src_ok) {
        a[u] = ld16_stream(s.sk + h * s.sk_hs_b + js * s.sk_ts_b + cb);
        b[u] = ld16_stream(s.sv + h * s.sv_hs_b + js * s.sv_ts_b + cb);
      }
      if (src_ok && t >= 0 && t < s.n_tokens) {
        dst_o[u] = h * s.d_hs_b + t * s.row_b + cb;
      } else if (rem == 0) {
        flag_error(err, CKV_DEVICE_ERR_RANGE);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (dst_o[u] >= 0) {
      st16_stream(s.dk + dst_o[u], a[u]);
      st16_stream(s.dv + dst_o[u], b[u]);
    }
  }
}

}  // namespace ckv
