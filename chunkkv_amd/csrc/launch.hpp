// Launchers shared between translation units of the library (host code; no device code here).
#pragma once

#include "select_common.hpp"

namespace ckv {

// The selection (select.hip): the register-resident form up to 33792 positions, with ghist (may
// be NULL) a top_bin candidate histogram that the launch leaves zeroed; the L2 form above
// (ghist must then be NULL).
int32_t select_launch(const SelectArgs& args, uint32_t* ghist, hipStream_t st);

// Row scatter (scatter.hip): K[h, rows[j]] = k[h, src_rows[j]] (src_rows NULL: j), V likewise,
// for j < n_rows, or j < min(n_rows, *n_rows_dev) when n_rows_dev is given (a count only the
// device knows).
int32_t scatter_launch(void* dst_k, void* dst_v, int64_t dst_head_stride, const void* src_k, int64_t sk_head_stride,
                       int64_t sk_token_stride, const void* src_v, int64_t sv_head_stride, int64_t sv_token_stride,
                       const int64_t* rows, const int64_t* src_rows, int32_t n_rows, int32_t n_src, int32_t n_tokens,
                       int32_t n_heads, int32_t head_dim, int32_t dtype, const int32_t* n_rows_dev, int32_t* err,
                       void* stream);

}  // namespace ckv
