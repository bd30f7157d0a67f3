// Launchers shared between translation units of the library (host code; no device code here).
#pragma once

#include "select_common.hpp"

namespace ckv {

// The selection (select.hip): the register-resident form up to 16384 positions, with ghist (may
// be NULL) a top_bin candidate histogram that the launch leaves zeroed; the L2 form above
// (ghist must then be NULL).
int32_t select_launch(const SelectArgs& args, uint32_t* ghist, hipStream_t st);

// The selection without an escalation threshold spread over many workgroups
// (select_slices.hpp), for 1 <= n_tokens <= kSlicesMaxTokens: ghist (may be NULL) is the candidate
// histogram followed by its ticket word, both zero, left zero; rows (may be NULL) adds the
// scatter of the kept rows. counts[CKV_COUNT_UNCOMPUTED] must be zero before the launch.
constexpr int kSlicesMaxTokens = 1024 * 4 * 9;
struct SliceRows;
bool select_slices_fits(int n_tokens);
int32_t select_slices_launch(const SelectArgs& args, uint32_t* ghist, const SliceRows* rows, int32_t* err,
                             hipStream_t st);

// The selection's launch with dense gather workgroups beside it (select_gather.hip): the
// register-resident selection without a threshold, plus every cached row (skip map ignored) of
// layers [g.layer_begin, g.layer_begin + *n_pre) of the slabs g.dk/g.dv, *n_pre chosen here
// (0..max_layers: what fits the CUs the selection leaves free and its time). Any other request
// (a threshold, more than 16384 positions, head_dim not 64/128, no segment) gets select_launch
// and *n_pre = 0. The caller fills g but for tiles, n_items, sum_groups and inv.
struct PreGather {
  char* dk;
  char* dv;
  int64_t ls_b;  // layer stride of the slabs, bytes
  int64_t hs_b;  // head stride, bytes
  const uint64_t* tab;
  const ckv_segment* segs;
  int n_tab_chunks, n_segs, tiles, n_items, n_layers, layer_begin, n_heads, n_tokens, sum_groups;
  int32_t* err;
  InvFreq inv;
};
int32_t pregather_layers(int32_t n_tokens, int32_t n_chunks, int32_t has_threshold, int32_t n_segs,
                         int32_t max_seg_tokens, int32_t max_layers, int32_t n_heads, int32_t head_dim, int32_t dtype);
int32_t select_gather_launch(const SelectArgs& args, uint32_t* ghist, PreGather g, int32_t max_layers,
                             int32_t max_seg_tokens, int32_t head_dim, int32_t dtype, double theta, int32_t* n_pre,
                             hipStream_t st);

// ckv_rerope_gather_layers (rerope_gather.hip), with rows (may be NULL) a scatter of another
// layer's rows carried in the same launch (its blocks dispatched first).
struct RowScatter;
int32_t gather_layers_launch(void* dst_k, void* dst_v, int64_t dst_layer_stride, int64_t dst_head_stride,
                             const uint64_t* src_tab, int32_t n_chunks, int32_t n_layers, int32_t layer_begin,
                             int32_t layer_end, const ckv_segment* segs, int32_t n_segs, int32_t max_seg_tokens,
                             const int32_t* skip, int32_t n_heads, int32_t n_tokens, int32_t head_dim, int32_t dtype,
                             double theta, int32_t* err, void* stream, const RowScatter* rows);

// Row scatter (scatter.hip): K[h, rows[j]] = k[h, src_rows[j]] (src_rows NULL: j), V likewise,
// for j < n_rows, or j < min(n_rows, *n_rows_dev) when n_rows_dev is given (a count only the
// device knows).
int32_t scatter_launch(void* dst_k, void* dst_v, int64_t dst_head_stride, const void* src_k, int64_t sk_head_stride,
                       int64_t sk_token_stride, const void* src_v, int64_t sv_head_stride, int64_t sv_token_stride,
                       const int64_t* rows, const int64_t* src_rows, int32_t n_rows, int32_t n_src, int32_t n_tokens,
                       int32_t n_heads, int32_t head_dim, int32_t dtype, const int32_t* n_rows_dev, int32_t* err,
                       void* stream);

}  // namespace ckv
