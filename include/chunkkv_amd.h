/*
 * chunkkv_amd — C ABI of the MI355X (gfx950) blend-prefill KV-repair kernels.
 *
 * The reference engine has no FFI: its KV repair is a sequence of PyTorch ops inside
 * TorchEngine.prefill (src/chunkkv/engine/torch_engine.py:80-178). Each entry point below
 * replaces one group of those ops; the comment on each names the lines it stands in for.
 *
 * Conventions shared by every entry point
 *  - All array arguments are DEVICE addresses (hipMalloc / torch CUDA tensors) unless the
 *    comment says otherwise. Pointers are borrowed: nothing is freed or retained.
 *  - Every launch goes to `stream` (a hipStream_t; NULL = the legacy default stream). No entry
 *    point synchronises, allocates or keeps global mutable state, so calls are re-entrant and
 *    may run concurrently on different streams.
 *  - K/V rows are head_dim contiguous elements. A "cache" tensor has layout (H, N, D): head
 *    stride given in elements, token stride == head_dim.
 *  - Element type is one of ckv_dtype. Arithmetic is fp32; results are rounded to the element
 *    type with round-to-nearest-even, matching torch's `.to(dtype)`.
 *  - Return value is a ckv_status. Argument errors are detected on the host before any
 *    launch. Descriptor errors that only the device can see (an index or a placement outside
 *    the cache) make the kernel skip that item and OR CKV_DEVICE_ERR_RANGE into `*err` when
 *    `err` is non-NULL; the caller reads `err` whenever it next synchronises.
 */
#ifndef CHUNKKV_AMD_H
#define CHUNKKV_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CKV_ABI_VERSION 5

typedef enum ckv_status {
  CKV_OK = 0,
  CKV_ERR_INVALID_ARGUMENT = 1, /* NULL pointer, unknown dtype, unsupported head_dim, bad count */
  CKV_ERR_OUT_OF_RANGE = 2,     /* a host-visible size or index outside its range              */
  CKV_ERR_TOO_LARGE = 3,        /* the request exceeds a kernel's capacity (see limits below)   */
  CKV_ERR_HIP = 4               /* the HIP runtime rejected a launch                            */
} ckv_status;

typedef enum ckv_dtype {
  CKV_DTYPE_F32 = 0,
  CKV_DTYPE_BF16 = 1
} ckv_dtype;

/* Bits a kernel ORs into the optional device status word `err`. */
#define CKV_DEVICE_ERR_RANGE 1u

/* Per-position flags (one byte per token position), built by the host planner.
 * Mirrors the lists returned by plan_positions (src/chunkkv/engine/base.py:63-73). */
#define CKV_POS_CACHED 1u /* covered by a placement                                   */
#define CKV_POS_SINK 2u   /* one of the first n_sink tokens of a non-exact placement    */
#define CKV_POS_EXACT 4u  /* covered by an exact placement (never recomputed)          */
#define CKV_POS_POOLED 8u /* inside a non-exact placement with ratio > 0 (the layer-1 pool,
                           * torch_engine.py:137-139); read by ckv_deviation_select only     */

/* Supported head dimensions (template instantiations). */
#define CKV_SELECT_MAX_TOKENS 131072 /* ckv_select keeps two N-bit masks in LDS */

/*
 * One run of destination rows filled from one cached chunk: destination token positions
 * [dst_start, dst_start + n_tokens) of every layer receive source tokens
 * [src_start, src_start + n_tokens) of chunk `chunk`, keys re-rotated by `delta` positions.
 * A placement (src/chunkkv/engine/base.py:26-33) becomes one segment; overlapping
 * placements are split by the host so that the last placement wins, as in the reference's
 * sequential slice assignment (torch_engine.py:99-102).
 */
typedef struct ckv_segment {
  int32_t dst_start;
  int32_t n_tokens;
  int32_t chunk;     /* index into the source pointer table                       */
  int32_t src_start; /* first source token inside the chunk                         */
  int32_t src_len;   /* chunk length = token count between two heads in the source */
  int32_t delta;     /* placement start - chunk start (torch_engine.py:101)         */
} ckv_segment;

/*
 * One non-exact placement as the layer-1 selection sees it (torch_engine.py:128-140):
 * its span, the token budget it adds to the pool, and whether it joins the pool at all.
 * `budget` = int(round(ratio * length)) with Python's round-half-even; `pooled` = ratio > 0.
 */
typedef struct ckv_chunk_span {
  int32_t start;
  int32_t length;
  int32_t budget;
  int32_t pooled;
} ckv_chunk_span;

/* Indices of the `counts` output of ckv_select. */
#define CKV_COUNT_KEEP 0            /* tokens in the new active set                         */
#define CKV_COUNT_SELECTED_CACHED 1 /* cached tokens in it (stats recomputed_cached_tokens)  */
#define CKV_COUNT_BUDGET 2          /* pooled budget after the cap (torch_engine.py:142)     */
#define CKV_COUNT_CANDIDATES 3      /* pooled tokens not already kept                       */
#define CKV_COUNT_UNCOMPUTED 4      /* kept tokens absent from the previous active set      */
#define CKV_COUNT_BUDGET_REQUESTED 5
#define CKV_COUNT_BAD_SPANS 6       /* spans outside [0, n_tokens), skipped                  */
#define CKV_COUNT_TOP_HISTOGRAM 7   /* bit 0: the selection started from the counted
                                       candidate histogram (ckv_deviation_select,
                                       ckv_layer1_repair): 4096 bins of 1/64 octave of
                                       deviation over 2^-24 .. 2^40, the threshold inside;
                                       bit 1: the threshold bin's candidates (at most 128)
                                       were ranked directly instead of by radix passes      */
#define CKV_COUNT_N 8

/* Bytes of the workspace ckv_deviation_select takes: the 16 KB candidate histogram, as four
   copies above 16384 positions (the counting launch's workgroups spread their atomics over
   them), then the word that counts the selection's workgroups done reading them (the rest is not
   used). */
#define CKV_DEVIATION_SELECT_WORKSPACE_BYTES 65792

/* Bytes of the workspace ckv_layer1_repair and ckv_layer1_repair_gather take (the same layout;
   their counting launch uses the four copies above 2048 positions). */
#define CKV_LAYER1_REPAIR_WORKSPACE_BYTES 65792

/* ABI version compiled into the library (CKV_ABI_VERSION). */
int32_t ckv_abi_version(void);

/* Static text for a ckv_status value. */
const char* ckv_status_string(int32_t status);

/*
 * Rotary inverse frequencies, the values every rotary kernel of this library takes in its
 * arguments: out[i] = fp32(theta_f ** e_i), evaluated on the host in fp64 (libm pow) and
 * rounded once, with theta_f = fp32(theta) and e_i = fp32(-(2i) / head_dim),
 * i in [0, head_dim/2), head_dim <= 256. Written to out on the stream.
 * Replaces: TorchEngine.__init__ inv_freq (torch_engine.py:33); scheduler/rerope.py:31-33.
 * out: head_dim/2 floats.
 */
int32_t ckv_inv_freq(float* out, int32_t head_dim, double theta, void* stream);

/*
 * Re-RoPE + gather for every layer in one launch: builds each layer's base K/V cache from
 * cached chunks placed at new offsets.
 *   dst_k/dst_v  per-layer caches; layer l, head h, token t lives at
 *                base + l*dst_layer_stride + h*dst_head_stride + t*head_dim (elements).
 *   src_tab      device table of source addresses, src_tab[(chunk*n_layers + l)*2 + 0] = keys
 *                and [...+1] = values of chunk `chunk` at layer l; each is a contiguous
 *                (H, src_len, D) tensor of dtype `dtype`. n_chunks = table rows; a segment
 *                naming a chunk outside [0, n_chunks) is skipped and flagged.
 *   segs         n_segs device descriptors; max_seg_tokens >= every segs[i].n_tokens.
 *                max_seg_tokens is at most 1,048,560 and the layer count at most 65535
 *                (CKV_ERR_TOO_LARGE beyond).
 *   Keys are re-rotated by delta (delta == 0 copies bit-for-bit); values are copied.
 * Destination rows covered by no segment are left untouched (the engine always overwrites
 * them with freshly computed rows).
 * Replaces: base_kv (torch_engine.py:96-103) with shift_keys/_rotate (:46-59);
 *           scheduler/rerope.py:36-47, :56-61.
 */
int32_t ckv_rerope_gather(void* dst_k, void* dst_v, int64_t dst_layer_stride,
                          int64_t dst_head_stride, const uint64_t* src_tab, int32_t n_chunks,
                          const ckv_segment* segs, int32_t n_segs, int32_t max_seg_tokens,
                          int32_t n_layers, int32_t n_heads, int32_t n_tokens,
                          int32_t head_dim, int32_t dtype, double theta, int32_t* err,
                          void* stream);

/*
 * ckv_rerope_gather restricted to layers [layer_begin, layer_end) of the n_layers in src_tab
 * and, when skip is not NULL, to the rows of positions p with skip[p] < 0 (skip: int32
 * (n_tokens,), e.g. the rank map ckv_select writes). Rows of positions with skip[p] >= 0 are
 * left untouched: in the reference those rows of layers >= 2 are gathered and then overwritten
 * by the fresh K/V (torch_engine.py:96-103 then :155-156), so only the survivors are moved.
 * dst_k/dst_v address layer 0 of the slab, as for ckv_rerope_gather.
 * Replaces: the same reference lines as ckv_rerope_gather.
 */
int32_t ckv_rerope_gather_layers(void* dst_k, void* dst_v, int64_t dst_layer_stride,
                                 int64_t dst_head_stride, const uint64_t* src_tab,
                                 int32_t n_chunks, int32_t n_layers, int32_t layer_begin,
                                 int32_t layer_end, const ckv_segment* segs, int32_t n_segs,
                                 int32_t max_seg_tokens, const int32_t* skip, int32_t n_heads,
                                 int32_t n_tokens, int32_t head_dim, int32_t dtype, double theta,
                                 int32_t* err, void* stream);

/*
 * Re-rotate one key tensor by delta positions: dst = shift_keys(src, delta).
 * src and dst are (n_heads, n_rows, head_dim) with the given head strides (elements) and
 * token stride head_dim; dst may equal src. delta == 0 copies.
 * Replaces: TorchEngine.shift_keys (torch_engine.py:56-59); scheduler/rerope.py:56-61.
 */
int32_t ckv_shift_keys(void* dst, int64_t dst_head_stride, const void* src,
                       int64_t src_head_stride, int32_t n_heads, int32_t n_rows,
                       int32_t head_dim, int32_t dtype, int32_t delta, double theta,
                       void* stream);

/*
 * Layer-1 fresh-vs-cached deviation, one value pair per token position p in [0, n_tokens):
 *   j = local[p] (row of p in the fresh tensors, -1 when p is not in the active set)
 *   diff[p] = sum_{h,d} fp32(round(k[h,j,d] - K[h,p,d]))^2 + same for v     (0 when j < 0)
 *   norm[p] = sum_{h,d} fp32(k[h,j,d])^2 + fp32(v[h,j,d])^2                (0 when j < 0)
 * where round() is rounding to `dtype` (torch subtracts in the element type) and K/V read
 * as zero at positions without CKV_POS_CACHED (the reference zero-fills them).
 * Summation order (the bit-exact contract): the H*D products of one tensor are split into
 * 16-byte vectors; vector q goes to lane q mod 64 of a 64-lane wavefront, each lane adds
 * its elements in ascending order into an fp32 accumulator starting at +0, then the lanes
 * are combined by a butterfly (xor 32, 16, 8, 4, 2, 1). diff = Sk + Sv, norm = Nk + Nv.
 *   k_fresh/v_fresh  strides in elements (head, token); rows contiguous.
 *   k_cache/v_cache  (H, n_tokens, D) with head stride cache_head_stride.
 * Replaces: torch_engine.py:117-124.
 */
int32_t ckv_deviation(const void* k_fresh, int64_t kf_head_stride, int64_t kf_token_stride,
                      const void* v_fresh, int64_t vf_head_stride, int64_t vf_token_stride,
                      const void* k_cache, const void* v_cache, int64_t cache_head_stride,
                      const uint8_t* pos_flags, const int32_t* local, int32_t n_tokens,
                      int32_t n_fresh, int32_t n_heads, int32_t head_dim, int32_t dtype,
                      float* diff, float* norm, int32_t* err, void* stream);

/*
 * Per-chunk relative deviation, escalation, pooled budget, pooled top-k with forced sinks,
 * and compaction of the new active set, in one single-workgroup launch.
 *   rel_dev[c]   = fp32(S_diff / S_norm) over chunk c's span (S = the lane-strided sum:
 *                  lane l adds positions start+l, start+l+64, ... then a xor butterfly)
 *   escalated[c] = has_threshold && (double)rel_dev[c] > escalate_threshold
 *   keep         = !cached | sink | spans of escalated chunks | top-`budget` candidates,
 *                  candidates = pooled spans minus keep, ranked by diff descending and
 *                  token index ascending (NaN ranks last),
 *                  budget = min(sum of budget over pooled non-escalated chunks, #candidates)
 *   keep_abs[i]  = i-th kept position in ascending order, i < counts[CKV_COUNT_KEEP]
 *   keep_local[i]= local[keep_abs[i]] (0 where local is -1; counted in CKV_COUNT_UNCOMPUTED)
 *   keep_rank[p] = i where keep_abs[i] == p, else -1, for every p < n_tokens (optional, may be
 *                  NULL): the local index map of the new active set, as ckv_assemble_layer takes it
 *   counts       CKV_COUNT_N int32 values (indices CKV_COUNT_*).
 * keep_abs and keep_local must hold n_tokens entries. n_tokens <= CKV_SELECT_MAX_TOKENS.
 * Replaces: torch_engine.py:125-153 (rel/escalation/budget :128-142, argsort top-k :143-146,
 *           keep.nonzero and local compaction :146-153).
 */
int32_t ckv_select(const float* diff, const float* norm, const uint8_t* pos_flags,
                   const int32_t* local, int32_t n_tokens, const ckv_chunk_span* chunks,
                   int32_t n_chunks, int32_t has_threshold, double escalate_threshold,
                   int64_t* keep_abs, int64_t* keep_local, int32_t* keep_rank, float* rel_dev,
                   uint8_t* escalated, int32_t* counts, void* stream);

/*
 * ckv_deviation followed by ckv_select with the top-k's first digit fused into the deviation:
 * the layer-1 repair decision (torch_engine.py:117-153) from the fresh and cached rows to the new
 * active set, with outputs and results bit-identical to the two calls (same arguments, same
 * meaning; see both above). Two launches: the deviation kernel also counts every position
 * flagged CKV_POS_CACHED | CKV_POS_POOLED and not CKV_POS_SINK into a histogram of its deviation
 * (4096 bins of 1/64 octave) in the workspace; the selection starts from that histogram and
 * ranks only the candidates of the threshold's bin. Without an escalation threshold and up to
 * 36864 positions the selection is spread over many workgroups, each finding the threshold
 * itself and compacting one slice of positions; with a threshold it runs in one workgroup. When
 * the pooled flags disagree with the pooled spans, a chunk escalates, or the threshold lies
 * outside 2^-24 .. 2^40, the selection ignores the histogram (same result, slower);
 * counts[CKV_COUNT_TOP_HISTOGRAM] says which path ran.
 *   workspace        device memory of >= CKV_DEVIATION_SELECT_WORKSPACE_BYTES, 16-byte aligned,
 *                    ZERO before its first use; every call leaves it zero again. Calls that
 *                    share a workspace must be ordered (one stream, or events): concurrent
 *                    calls on one workspace race.
 * n_tokens <= CKV_SELECT_MAX_TOKENS; the workspace is not touched above 36864 positions, nor
 * above 16384 with a threshold (the deviation then counts no histogram and the selection runs
 * its L2 form).
 * Replaces: torch_engine.py:117-153 (the deviation :117-124, rel/escalation/budget :128-142,
 *           argsort top-k :143-146, keep.nonzero and local compaction :146-153).
 */
int32_t ckv_deviation_select(const void* k_fresh, int64_t kf_head_stride, int64_t kf_token_stride,
                             const void* v_fresh, int64_t vf_head_stride, int64_t vf_token_stride,
                             const void* k_cache, const void* v_cache, int64_t cache_head_stride,
                             const uint8_t* pos_flags, const int32_t* local, int32_t n_tokens,
                             int32_t n_fresh, int32_t n_heads, int32_t head_dim, int32_t dtype,
                             const ckv_chunk_span* chunks, int32_t n_chunks, int32_t has_threshold,
                             double escalate_threshold, float* diff, float* norm, int64_t* keep_abs,
                             int64_t* keep_local, int32_t* keep_rank, float* rel_dev, uint8_t* escalated,
                             int32_t* counts, void* workspace, int64_t workspace_bytes, int32_t* err,
                             void* stream);

/*
 * ckv_deviation_select without the workspace argument, for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart
 * in the reference. The workspace is a static device array of the library,
 * CKV_DEVIATION_SELECT_WORKSPACE_BYTES (65,792 bytes) per GPU, enough for every n_tokens the call
 * takes (n_tokens > CKV_SELECT_MAX_TOKENS returns CKV_ERR_TOO_LARGE); its device address is looked
 * up once per GPU on the first call there. The call allocates nothing. All calls on one GPU share
 * that array, which every call leaves zeroed: calls that overlap on one GPU (different streams
 * without ordering) race and must not be issued. Same arguments, results and errors as
 * ckv_deviation_select otherwise.
 */
int32_t ckv_deviation_select_noalloc(const void* k_fresh, int64_t kf_head_stride, int64_t kf_token_stride,
                                     const void* v_fresh, int64_t vf_head_stride, int64_t vf_token_stride,
                                     const void* k_cache, const void* v_cache, int64_t cache_head_stride,
                                     const uint8_t* pos_flags, const int32_t* local, int32_t n_tokens,
                                     int32_t n_fresh, int32_t n_heads, int32_t head_dim, int32_t dtype,
                                     const ckv_chunk_span* chunks, int32_t n_chunks, int32_t has_threshold,
                                     double escalate_threshold, float* diff, float* norm, int64_t* keep_abs,
                                     int64_t* keep_local, int32_t* keep_rank, float* rel_dev, uint8_t* escalated,
                                     int32_t* counts, int32_t* err, void* stream);

/*
 * Layer 1's whole KV repair in one call: its base cache, the deviation, the selection and the
 * scatter of the kept rows, with every output bit-identical to
 *   ckv_rerope_gather_layers(layer, every cached row) -> ckv_deviation -> ckv_select ->
 *   ckv_scatter_kept_rows(keep_abs, keep_local)
 * (same arguments, same meaning; see each above). dst_k/dst_v are the layer's (H, n_tokens, D)
 * cache, head stride dst_head_stride; src_tab/n_tab_chunks/n_layers/layer select the chunks' rows
 * as in ckv_assemble_layer; segs are the cached runs, sorted by dst_start and disjoint (the
 * planner's segments, n_segs <= 3840), read for every position flagged CKV_POS_CACHED. segs and
 * src_tab may be NULL with n_segs == 0, k_fresh and v_fresh with n_fresh == 0 (every position
 * exact: a kept position then flags CKV_DEVICE_ERR_RANGE, as an out-of-range local index does).
 * Nothing is read back on the host. Launch (1): every position's rows, the cached rows written
 * into the cache, the deviations, and the positions flagged CKV_POS_CACHED | CKV_POS_POOLED and
 * not CKV_POS_SINK counted into the deviation histogram. Without an escalation threshold and up
 * to 36864 positions, launch (2) is the selection and the kept rows' scatter in one launch of
 * many workgroups, each finding the threshold from that count and compacting and scattering one
 * slice of positions. Otherwise (2) is the selection in one workgroup (as ckv_deviation_select's)
 * and (3) the kept rows, their count read on the device. Both give the same result when the
 * flags disagree with the spans or a chunk escalates, just slower.
 *   workspace  >= CKV_LAYER1_REPAIR_WORKSPACE_BYTES, 16-byte aligned, ZERO before its first use;
 *              each call leaves it zeroed. Calls that share a workspace must be ordered (one
 *              stream, or events).
 * Limits: H * D * elem <= 1024 bytes per row (CKV_ERR_TOO_LARGE beyond: use the four calls),
 * head_dim <= 128 and a power of two, n_tokens <= CKV_SELECT_MAX_TOKENS (above 36864, or above
 * 16384 with a threshold, the selection counts its own histogram).
 * Replaces: base_kv for layer 1 (torch_engine.py:96-103, with shift_keys :56-59), the deviation
 *           (:117-124), rel/escalation/budget (:125-142), the top-k (:143-147), the compaction
 *           (:148-153) and the scatter (:155-156).
 */
int32_t ckv_layer1_repair(void* dst_k, void* dst_v, int64_t dst_head_stride, const uint64_t* src_tab,
                          int32_t n_tab_chunks, int32_t n_layers, int32_t layer, const ckv_segment* segs,
                          int32_t n_segs, const void* k_fresh, int64_t kf_head_stride,
                          int64_t kf_token_stride, const void* v_fresh, int64_t vf_head_stride,
                          int64_t vf_token_stride, int32_t n_fresh, const uint8_t* pos_flags,
                          const int32_t* local, int32_t n_tokens, int32_t n_heads, int32_t head_dim,
                          int32_t dtype, double theta, const ckv_chunk_span* chunks, int32_t n_chunks,
                          int32_t has_threshold, double escalate_threshold, float* diff, float* norm,
                          int64_t* keep_abs, int64_t* keep_local, int32_t* keep_rank, float* rel_dev,
                          uint8_t* escalated, int32_t* counts, void* workspace, int64_t workspace_bytes,
                          int32_t* err, void* stream);

/*
 * ckv_layer1_repair of layer `layer` followed by the base cache of layers [gather_begin,
 * gather_end): layer `layer` and the selection bit-identical to ckv_layer1_repair; in the gathered
 * layers every row of a position the selection dropped bit-identical to ckv_rerope_gather_layers
 * (the re-rotated cached row), rows of uncached positions untouched. Rows of kept cached
 * positions: in the first W layers of the range (W = ckv_layer1_repair_gather_whole_layers of the
 * same arguments), the re-rotated cached row (whole layers, as base_kv writes them); in the other
 * layers untouched (ckv_rerope_gather_layers' skip map keep_rank). The caller writes the fresh
 * rows of the kept positions into every gathered layer afterwards (as the engine does when it
 * computes that layer), which makes both forms the same cache.
 * Launches: the layer-1 pass; the selection, with the W whole layers gathered by workgroups
 * beside it (the CUs the single-workgroup selection leaves idle); the kept rows' scatter with the
 * gather of the dropped rows of the other layers.
 * k_slab/v_slab hold every layer's (H, n_tokens, D) cache, layer l at l * layer_stride elements,
 * head stride head_stride; max_seg_tokens is the longest segment (as for the gather). The other
 * arguments are ckv_layer1_repair's. keep_rank must not be NULL, and `layer` must lie outside
 * [gather_begin, gather_end).
 * Replaces: base_kv for layer 1 and the layer-1 repair (torch_engine.py:96-103, :117-156), and
 *           base_kv of the later layers (:96-103) up to the overwrite of the kept rows (:155-156).
 */
int32_t ckv_layer1_repair_gather(void* k_slab, void* v_slab, int64_t layer_stride, int64_t head_stride,
                                 const uint64_t* src_tab, int32_t n_tab_chunks, int32_t n_layers, int32_t layer,
                                 int32_t gather_begin, int32_t gather_end, const ckv_segment* segs, int32_t n_segs,
                                 int32_t max_seg_tokens, const void* k_fresh, int64_t kf_head_stride,
                                 int64_t kf_token_stride, const void* v_fresh, int64_t vf_head_stride,
                                 int64_t vf_token_stride, int32_t n_fresh, const uint8_t* pos_flags,
                                 const int32_t* local, int32_t n_tokens, int32_t n_heads, int32_t head_dim,
                                 int32_t dtype, double theta, const ckv_chunk_span* chunks, int32_t n_chunks,
                                 int32_t has_threshold, double escalate_threshold, float* diff, float* norm,
                                 int64_t* keep_abs, int64_t* keep_local, int32_t* keep_rank, float* rel_dev,
                                 uint8_t* escalated, int32_t* counts, void* workspace, int64_t workspace_bytes,
                                 int32_t* err, void* stream);

/*
 * W of ckv_layer1_repair_gather: how many leading layers of the gathered range that call writes
 * whole (kept rows included) beside its selection, for the same n_tokens, n_chunks,
 * has_threshold, n_segs, max_seg_tokens, gather_end - gather_begin, n_heads, head_dim and dtype
 * on the current device. 0 with a threshold, above 16384 positions, head_dim other than 64 or
 * 128, or no segment; otherwise as many whole layers as about 8 KiB of HBM traffic per position
 * covers (what the CUs the selection leaves free move in its time). Host only (reads the
 * device's CU count). No counterpart in the reference.
 */
int32_t ckv_layer1_repair_gather_whole_layers(int32_t n_tokens, int32_t n_chunks, int32_t has_threshold,
                                              int32_t n_segs, int32_t max_seg_tokens, int32_t gather_layers,
                                              int32_t n_heads, int32_t head_dim, int32_t dtype);

/*
 * Assemble one layer's cache with every row written once: for each segment row at position p,
 *   local[p] >= 0  -> K/V[h, p, :] = fresh k/v[h, local[p], :]            (an active position)
 *   otherwise      -> K/V[h, p, :] = the chunk's row, keys re-rotated by delta (as the gather)
 * This is the reference's per-layer pair "base cache, then scatter the active rows" in one pass
 * (torch_engine.py:96-103 + :155-156). segs may include uncached runs with chunk == -1 (their
 * positions must be active). local == NULL gathers only (fresh tensors unused; uncached runs
 * skipped). src_tab is the gather's table (n_chunks x n_layers x 2); `layer` selects its column.
 * k/v_fresh: (H, n_fresh, D) with the given strides; local: n_tokens entries.
 * A row with an active index >= n_fresh, or an inactive position in an uncached run, is left
 * unwritten and flagged. No counterpart in the reference as one call; see above.
 */
int32_t ckv_assemble_layer(void* dst_k, void* dst_v, int64_t dst_head_stride, const uint64_t* src_tab,
                           int32_t n_chunks, int32_t n_layers, int32_t layer, const ckv_segment* segs,
                           int32_t n_segs, int32_t max_seg_tokens, const void* k_fresh,
                           int64_t kf_head_stride, int64_t kf_token_stride, const void* v_fresh,
                           int64_t vf_head_stride, int64_t vf_token_stride, int32_t n_fresh,
                           const int32_t* local, int32_t n_tokens, int32_t n_heads, int32_t head_dim,
                           int32_t dtype, double theta, int32_t* err, void* stream);

/*
 * ckv_rerope_gather_layers and ckv_scatter_kept_rows in ONE launch: the gather of layers
 * [layer_begin, layer_end) (rows with skip[p] >= 0 left alone) and, in the same launch, the
 * kept rows of layer kept_layer of the same slab:
 *   K[kept_layer, h, keep_abs[j], :] = k[h, keep_local[j], :],  V likewise,
 * for j < n_keep, or j < min(n_keep, *n_keep_dev) when n_keep_dev is not NULL (a count only the
 * device knows, e.g. counts + CKV_COUNT_KEEP of a selection; n_keep is then its upper bound and
 * sizes the launch). k/v: n_fresh rows, strides in elements (row contiguous, 16-byte aligned;
 * NULL with n_fresh = 0, when every kept row is out of range).
 * kept_layer must lie outside [layer_begin, layer_end) (CKV_ERR_INVALID_ARGUMENT otherwise), so
 * no row is written twice. A kept row whose source or destination is out of range is skipped and
 * flagged in err. With nothing to gather (n_segs, max_seg_tokens or the layer range empty)
 * src_tab and segs are not read and may be NULL. This is the last launch of
 * ckv_layer1_repair_gather, callable alone (e.g. after ckv_deviation_select).
 * Replaces: base_kv (torch_engine.py:96-103) for layers >= 2 and, for the kept layer, the
 * compaction and scatter of torch_engine.py:152, :155-156.
 */
int32_t ckv_rerope_gather_layers_kept(void* dst_k, void* dst_v, int64_t dst_layer_stride,
                                      int64_t dst_head_stride, const uint64_t* src_tab, int32_t n_chunks,
                                      int32_t n_layers, int32_t layer_begin, int32_t layer_end,
                                      const ckv_segment* segs, int32_t n_segs, int32_t max_seg_tokens,
                                      const int32_t* skip, int32_t kept_layer, const void* k_fresh,
                                      int64_t kf_head_stride, int64_t kf_token_stride, const void* v_fresh,
                                      int64_t vf_head_stride, int64_t vf_token_stride, const int64_t* keep_abs,
                                      const int64_t* keep_local, int32_t n_keep, const int32_t* n_keep_dev,
                                      int32_t n_fresh, int32_t n_heads, int32_t n_tokens, int32_t head_dim,
                                      int32_t dtype, double theta, int32_t* err, void* stream);

/*
 * Scatter freshly computed K/V rows into one layer's cache:
 *   K[h, rows[j], :] = k[h, j, :],  V[h, rows[j], :] = v[h, j, :]   for j < n_rows.
 * rows are distinct positions in [0, n_tokens) (any order).
 * Replaces: torch_engine.py:155-156.
 */
int32_t ckv_scatter_rows(void* dst_k, void* dst_v, int64_t dst_head_stride,
                         const void* src_k, int64_t sk_head_stride, int64_t sk_token_stride,
                         const void* src_v, int64_t sv_head_stride, int64_t sv_token_stride,
                         const int64_t* rows, int32_t n_rows, int32_t n_tokens,
                         int32_t n_heads, int32_t head_dim, int32_t dtype, int32_t* err,
                         void* stream);

/*
 * Scatter the kept rows of the previous active set into one layer's cache, the compaction
 * folded in:
 *   K[h, dst_rows[j], :] = k[h, src_rows[j], :],  V[h, dst_rows[j], :] = v[h, src_rows[j], :]
 * for j < n_rows, with src_rows[j] < n_src (a selection's keep_abs / keep_local).
 * Replaces: the k/v compaction k[:, :, sel], v[:, :, sel] (torch_engine.py:152) and the scatter
 * K[:, :, active] = k, V[:, :, active] = v (:155-156) that follows it.
 */
int32_t ckv_scatter_kept_rows(void* dst_k, void* dst_v, int64_t dst_head_stride,
                              const void* src_k, int64_t sk_head_stride, int64_t sk_token_stride,
                              const void* src_v, int64_t sv_head_stride, int64_t sv_token_stride,
                              const int64_t* dst_rows, const int64_t* src_rows, int32_t n_rows,
                              int32_t n_src, int32_t n_tokens, int32_t n_heads, int32_t head_dim,
                              int32_t dtype, int32_t* err, void* stream);

/*
 * Fresh-token RoPE of projected q/k rows, with the v rows copied alongside:
 *   q_out[h, t] = rope(q_in[h, t], positions[t])                 h < n_q_heads
 *   k_out[h, r] = rope(k_in[h, t], positions[t]),  v_out[h, r] = v_in[h, t]      h < n_kv_heads
 * with r = rows[t] (rows != NULL: e.g. straight into the cache rows of the active positions,
 * r < n_out_rows) or r = t (rows == NULL). rope(x, p) rotates the halves of x by the fp32 angles
 * fl32(fl32(p) * inv_freq_i) with correctly rounded fp32 cos/sin, fp32 products and sums each
 * rounded once, one rounding to dtype: the rotation ckv_shift_keys applies for a shift by p.
 * Element (h, t, d) of each tensor is at base + h*head_stride + t*token_stride + d (elements;
 * rows contiguous and 16-byte aligned), so projection outputs can be passed as token-major views.
 * v_out and v_in are both NULL to skip the copy; with n_q_heads = 0, q_out and q_in may be NULL
 * (k/v only). cs_table: optional ckv_rope_table output with n_table positions (NULL: the kernel
 * evaluates the cos/sin itself). dtype bf16 or f32, head_dim 64, 128 or 256.
 * Replaces: _qkv/_rope/_rotate (torch_engine.py:61-66, :53-54, :46-51) and the scatter of k/v
 * into the cache (:155-156).
 */
int32_t ckv_rope_qkv(void* q_out, int64_t qo_head_stride, int64_t qo_token_stride, void* k_out,
                     int64_t ko_head_stride, int64_t ko_token_stride, void* v_out, int64_t vo_head_stride,
                     int64_t vo_token_stride, const int64_t* rows, int32_t n_out_rows, const void* q_in,
                     int64_t qi_head_stride, int64_t qi_token_stride, const void* k_in,
                     int64_t ki_head_stride, int64_t ki_token_stride, const void* v_in,
                     int64_t vi_head_stride, int64_t vi_token_stride, const int64_t* positions,
                     const void* cs_table, int64_t n_table, int32_t n_tokens, int32_t n_q_heads,
                     int32_t n_kv_heads, int32_t head_dim, int32_t dtype, double theta, int32_t* err,
                     void* stream);

/*
 * The (cos, sin) pairs ckv_rope_qkv uses, for positions [0, n_positions): table[p][i] =
 * (cos, sin) of fl32(fl32(p) * inv_freq_i), correctly rounded fp32, i < head_dim/2; float2
 * entries, n_positions * head_dim/2 of them. Passed to ckv_rope_qkv as cs_table (positions
 * must then lie in [0, n_table)); the results are identical with or without it. No counterpart
 * in the reference (it recomputes cos/sin per call, torch_engine.py:53-54, :47).
 */
int32_t ckv_rope_table(void* table, int64_t n_positions, int32_t head_dim, double theta, void* stream);

/*
 * Store-put extraction: for each of n_spans segments (spans[2s] = start, spans[2s+1] = len),
 * copy token rows [start, start + len) of every layer's K and V out of the request slabs
 * (layer l, head h, token t at base + l*layer_stride + h*head_stride + t*head_dim, elements)
 * into the buffer dst_tab[s] (device address), laid out [2][n_layers][n_heads][len][head_dim]:
 * K layers then V layers, so each layer's keys/values are a contiguous (1, H, len, D) block. The
 * buffer must hold 2 * n_layers * n_heads * len * head_dim elements. max_len >= every len.
 * n_spans and n_layers are at most 65535 (CKV_ERR_TOO_LARGE beyond). A span outside [0, n_tokens) is skipped and flagged in *err. Bit copies (bf16 or f32).
 * Replaces: PrefillResult.chunk's per-layer copies (base.py:55-60, torch_engine.py:177), called
 * per reusable segment by the runtime (runtime.py:83-92): 2 x n_layers launches per segment.
 */
int32_t ckv_extract_chunks(const void* k_slab, const void* v_slab, int64_t layer_stride,
                           int64_t head_stride, const uint64_t* dst_tab, const int32_t* spans,
                           int32_t n_spans, int32_t max_len, int32_t n_layers, int32_t n_heads,
                           int32_t n_tokens, int32_t head_dim, int32_t dtype, int32_t* err,
                           void* stream);

/*
 * Attention of the active rows over the whole cache with the causal mask given by positions:
 *   out[i, h, :] = softmax_j( scale * q[h, i, :] . K[h / G, j, :] ) V[h / G, j, :],
 *   j ranging over [0, positions[i]], G = n_q_heads / n_kv_heads.
 * This is F.scaled_dot_product_attention(q, K, V, attn_mask=active[:, None] >= arange(N),
 * enable_gqa=True) with positions = active (torch_engine.py:157, :68-72), computed without the
 * (n_queries x n_tokens) mask and without expanding the KV heads.
 *   q          bf16 (n_q_heads, n_queries, head_dim) with the given head/token strides (elements,
 *              multiples of 8; rows contiguous)
 *   k_cache,   bf16 (n_kv_heads, n_tokens, head_dim), rows contiguous, head stride kv_head_stride
 *   v_cache
 *   positions  int64 (n_queries,), each in [0, n_tokens) (out-of-range entries are clamped and
 *              flagged in *err); any order, ascending is fastest
 *   out        bf16 (n_queries, n_q_heads, head_dim) contiguous: token-major, the layout the
 *              output projection reads
 * dtype must be CKV_DTYPE_BF16 and head_dim 64 or 128. Scores and the output accumulate in
 * fp32; the softmax weights are rounded to bf16 before they multiply V.
 *   workspace  optional device buffer of workspace_bytes >= ckv_attention_workspace_bytes(...)
 *              (16-byte aligned): with it, launches that are too small to fill the chip (few
 *              queries over a long cache, e.g. decode) split the cache range over more
 *              workgroups and merge the partial results; without it they run unsplit. The
 *              result is the same up to fp32 rounding of the merge.
 * Replaces: the mask construction and SDPA call of torch_engine.py:157, :68-72 (and the decode
 * step's SDPA, :192).
 */
int32_t ckv_attention_active(void* out, const void* q, int64_t q_head_stride, int64_t q_token_stride,
                             const void* k_cache, const void* v_cache, int64_t kv_head_stride,
                             const int64_t* positions, int32_t n_queries, int32_t n_tokens,
                             int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, int32_t dtype,
                             double scale, void* workspace, int64_t workspace_bytes, int32_t* err,
                             void* stream);

/*
 * Bytes of workspace ckv_attention_active uses to split a launch of this shape (0: it never
 * splits this shape), enough for either plan it may take: query heads that share a KV head with
 * n_queries * group <= 128 (decode) go into one workgroup per (KV head, split of 6 cache tiles);
 * other launches split into about 1024 workgroups when they would not fill the chip. The latter
 * plan's split count and cache tiles per split go to *splits and *split_tiles when those are
 * not NULL. Host-only, no device work. No counterpart in the reference.
 */
int64_t ckv_attention_workspace_bytes(int32_t n_queries, int32_t n_tokens, int32_t n_q_heads,
                                      int32_t head_dim, int32_t* splits, int32_t* split_tiles);

/*
 * Residual add and RMSNorm of each row, the elementwise steps around a decoder layer's GEMMs:
 *   s = h_in + delta, rounded to dtype and written to h_out       (delta != NULL)
 *   s = h_in                                                       (delta == NULL; h_out unused)
 *   y = dtype( weight * dtype( s * rsqrt(fl32(sum(s^2)) * fl32(1/hidden) + eps) ) )
 * in fp32 with each product rounded once: the Hugging Face Qwen2/Llama RMSNorm module
 * (x.to(fp32); x * rsqrt(x.pow(2).mean(-1) + eps); weight * x.to(dtype)) after the residual add.
 * The fp32 order of the sum of squares is the kernel's own (a fixed tree). h_out may equal h_in.
 * Rows contiguous: element (r, c) at base + r*hidden + c. hidden a multiple of 8 (bf16) or 4
 * (f32) and at most 8192 (bf16) or 4096 (f32); dtype bf16 or f32.
 * Replaces: `h + attn.o_proj(out)` and `layer.post_attention_layernorm(h)` (torch_engine.py:71-72),
 * the next layer's `layer.input_layernorm(h)` after the MLP's residual add (:72, :113, :191) and
 * `self.inner.norm(h)` (:75).
 */
int32_t ckv_add_rmsnorm(void* h_out, const void* h_in, const void* delta, void* y, const void* weight,
                        int64_t n_rows, int32_t hidden, float eps, int32_t dtype, void* stream);

/*
 * SiLU-gated product of the MLP: out = dtype( dtype(gate / (1 + exp(-gate))) * up ), fp32 math
 * with each step rounded once. Row r of each operand starts at base + r*row_stride (elements,
 * multiples of 8 for bf16 or 4 for f32; base 16-byte aligned), so the halves of one stacked
 * gate|up GEMM output can be passed as two views. dtype bf16 or f32.
 * Replaces: `act_fn(gate_proj(x)) * up_proj(x)` inside layer.mlp (torch_engine.py:72; the Hugging
 * Face Qwen2/Llama MLP with SiLU).
 */
int32_t ckv_silu_mul(void* out, int64_t out_row_stride, const void* gate, int64_t gate_row_stride,
                     const void* up, int64_t up_row_stride, int64_t n_rows, int32_t width, int32_t dtype,
                     void* stream);

/*
 * Token-prefix hashes (host memory, host code): digests[32*i .. 32*i + 32) = SHA-256 of the
 * message LE32(s) || LE32(tokens[0]) || ... || LE32(tokens[s - 1]) with s = starts[i], i.e.
 * the reference's keys.token_hash(tokens[:s]) as raw bytes (its hexdigest is their hex).
 *   tokens     n_tokens ids; every id of a hashed prefix must lie in [0, 2^32)
 *              (CKV_ERR_OUT_OF_RANGE otherwise, where the reference raises OverflowError)
 *   starts     n_starts prefix lengths in [0, n_tokens]
 *   n_threads  host threads to use, 0 = one per available core (at most 16)
 * Replaces: keys.token_hash (src/chunkkv/store/keys.py:15-20) as called per segment by
 *           ReuseGate.decide (src/chunkkv/gate/gate.py:42) and ChunkReuseRuntime.prefill
 *           (src/chunkkv/runtime.py:89).
 */
int32_t ckv_token_hash_prefixes(const int64_t* tokens, int64_t n_tokens, const int64_t* starts,
                                int32_t n_starts, uint8_t* digests, int32_t n_threads);

#ifdef __cplusplus
}
#endif

#endif /* CHUNKKV_AMD_H */
