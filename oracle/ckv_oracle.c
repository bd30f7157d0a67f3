/*
 * ORACLE — test infrastructure only. A plain-C CPU restatement of the reference's blend-prefill
 * KV-repair arithmetic, used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * as the checker of the HIP kernels. It is never part of the product path.
 *
 * Each function cites the reference lines it restates (paths relative to the reference repo):
 *   ckvo_inv_freq        src/chunkkv/engine/torch_engine.py:33 (rerope.py:31-33)
 *   ckvo_rerope_gather   torch_engine.py:46-51 (_rotate), :56-59 (shift_keys), :96-103 (base_kv)
 *   ckvo_shift_keys      torch_engine.py:56-59
 *   ckvo_rope            torch_engine.py:53-54 with :46-51
 *   ckvo_deviation       torch_engine.py:117-124
 *   ckvo_select          torch_engine.py:125-153
 *   ckvo_scatter_rows    torch_engine.py:155-156
 *
 * Arithmetic follows the torch op sequence: fp32 products and sums each rounded once (built
 * with -ffp-contract=off), one rounding to the element type at the end of a rotation, element-
 * type subtraction in the deviation. Two places where torch leaves the result open are fixed by
 * the contract the kernels implement, and restated here from its definition, not from the
 * kernels' code: (1) fp32 sums use the lane-strided order + xor butterfly spelled out in
 * include/chunkkv_amd.h; (2) the top-k breaks ties by the lower token index (a comparison sort
 * here, a radix select on the GPU); (3) cos/sin of the fp32 angle delta*inv_freq and inv_freq
 * itself are the correctly rounded fp32 values (fp64 libm, rounded once), where torch's fp32
 * cos/sin/pow may be an ulp off.
 *
 * Pinning (see tests/test_oracle.py): closed forms (inv_freq vs exact exponents, rotation
 * composition and round trip at the reference's tolerances, Δ=0 identity, fp64 rotation within
 * one bf16 ulp), fp64 brute force for the deviation, an independent numpy lexsort and torch's
 * stable argsort for the selection, and the reference's closed-form stats.
 */
#include <limits.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define DT_F32 0
#define DT_BF16 1

#define POS_CACHED 1u
#define POS_SINK 2u

typedef struct {
  int32_t dst_start, n_tokens, chunk, src_start, src_len, delta;
} seg_t;

typedef struct {
  int32_t start, length, budget, pooled;
} span_t;

/* ---- element conversions ------------------------------------------------------------- */

static float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* round-to-nearest-even; NaN -> 0x7fc0 (torch's c10::BFloat16 rule) */
static uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float ld(const void* base, int64_t i, int dt) {
  if (dt == DT_BF16) return bf16_to_f32(((const uint16_t*)base)[i]);
  return ((const float*)base)[i];
}

static void st(void* base, int64_t i, int dt, float v) {
  if (dt == DT_BF16)
    ((uint16_t*)base)[i] = f32_to_bf16(v);
  else
    ((float*)base)[i] = v;
}

static float round_to(float v, int dt) { return dt == DT_BF16 ? bf16_to_f32(f32_to_bf16(v)) : v; }

static int elem_size(int dt) { return dt == DT_BF16 ? 2 : 4; }

/* ---- a1: inverse frequencies ------------------------------------------------------------ */

void ckvo_inv_freq(int head_dim, double theta, float* out) {
  const float theta_f = (float)theta;
  for (int i = 0; i < head_dim / 2; ++i) {
    const float e = (float)(-2 * i) / (float)head_dim; /* fp32 exponent, as torch builds it */
    out[i] = (float)pow((double)theta_f, (double)e);
  }
}

/* ---- a2: rotation of one row by per-frequency (cos, sin) ----------------------------------- */

static void rotate_row(const void* src, void* dst, int64_t off, int D, int dt, const float* c, const float* s) {
  const int half = D / 2;
  for (int i = 0; i < half; ++i) {
    const float x1 = ld(src, off + i, dt);
    const float x2 = ld(src, off + half + i, dt);
    const float a = x1 * c[i];
    const float b = x2 * s[i];
    const float d = x1 * s[i];
    const float e = x2 * c[i];
    const float y1 = a - b;
    const float y2 = d + e;
    st(dst, off + i, dt, y1);
    st(dst, off + half + i, dt, y2);
  }
}

static void shift_tables(int D, double theta, int32_t delta, float* c, float* s) {
  float inv[1024];
  ckvo_inv_freq(D, theta, inv);
  for (int i = 0; i < D / 2; ++i) {
    const float ang = (float)delta * inv[i];
    c[i] = (float)cos((double)ang); /* correctly rounded fp32 cos/sin of the fp32 angle */
    s[i] = (float)sin((double)ang);
  }
}

/* Fresh-token RoPE: torch_engine.py:53-54 (_rope, angles = positions.float()[:, None] *
 * inv_freq[None, :]) with _rotate (:46-51). Row t of every head is rotated by the fp32 angle
 * fl32(fl32(pos[t]) * inv_freq_i), i.e. the rotation of a shift by pos[t]; the formula is applied
 * at every position (no shortcut at 0, as torch). Element (h, t, d) at h*hs + t*ts + d. */
int ckvo_rope(void* dst, int64_t dst_hs, int64_t dst_ts, const void* src, int64_t src_hs, int64_t src_ts,
              const int64_t* pos, int n_heads, int n_rows, int D, int dt, double theta) {
  if (D <= 0 || D > 2048 || (D & 1)) return 1;
  float c[1024], s[1024];
  const int half = D / 2;
  for (int t = 0; t < n_rows; ++t) {
    if (pos[t] < INT32_MIN || pos[t] > INT32_MAX) return 2;
    shift_tables(D, theta, (int32_t)pos[t], c, s);
    for (int h = 0; h < n_heads; ++h) {
      const int64_t so = (int64_t)h * src_hs + (int64_t)t * src_ts, dof = (int64_t)h * dst_hs + (int64_t)t * dst_ts;
      for (int i = 0; i < half; ++i) {
        const float x1 = ld(src, so + i, dt), x2 = ld(src, so + half + i, dt);
        const float a = x1 * c[i], b = x2 * s[i], d = x1 * s[i], e = x2 * c[i];
        st(dst, dof + i, dt, a - b);
        st(dst, dof + half + i, dt, d + e);
      }
    }
  }
  return 0;
}

/* keys (n_heads, n_rows, D) with head strides in elements; dst may equal src. */
int ckvo_shift_keys(void* dst, int64_t dst_hs, const void* src, int64_t src_hs, int n_heads, int n_rows, int D,
                    int dt, int32_t delta, double theta) {
  if (D <= 0 || D > 2048 || (D & 1)) return 1;
  const int eb = elem_size(dt);
  if (delta == 0) {
    for (int h = 0; h < n_heads; ++h)
      memmove((char*)dst + (size_t)h * dst_hs * eb, (const char*)src + (size_t)h * src_hs * eb, (size_t)n_rows * D * eb);
    return 0;
  }
  float c[1024], s[1024];
  shift_tables(D, theta, delta, c, s);
  for (int h = 0; h < n_heads; ++h)
    for (int t = 0; t < n_rows; ++t) {
      const char* sr = (const char*)src + ((size_t)h * src_hs + (size_t)t * D) * eb;
      char* dr = (char*)dst + ((size_t)h * dst_hs + (size_t)t * D) * eb;
      rotate_row(sr, dr, 0, D, dt, c, s);
    }
  return 0;
}

/* ---- a3: re-RoPE + gather for all layers ------------------------------------------------------
 * src_tab[(chunk*n_layers + l)*2 + {0,1}] = host address of a contiguous (H, src_len, D) tensor.
 * dst layer l, head h, token t at l*layer_stride + h*head_stride + t*D. Returns 1 on a bad
 * descriptor (nothing written for it).                                                     */
int ckvo_rerope_gather(void* dst_k, void* dst_v, int64_t layer_stride, int64_t head_stride, const uint64_t* src_tab,
                       const seg_t* segs, int n_segs, int n_layers, int n_heads, int n_tokens, int D, int dt,
                       double theta) {
  const int eb = elem_size(dt);
  int bad = 0;
  float c[1024], s[1024];
  for (int si = 0; si < n_segs; ++si) {
    const seg_t g = segs[si];
    if (g.dst_start < 0 || g.src_start < 0 || g.n_tokens < 0 || g.chunk < 0 ||
        (int64_t)g.dst_start + g.n_tokens > n_tokens || (int64_t)g.src_start + g.n_tokens > g.src_len) {
      bad = 1;
      continue;
    }
    if (g.delta != 0) shift_tables(D, theta, g.delta, c, s);
    for (int l = 0; l < n_layers; ++l) {
      const char* sk = (const char*)(uintptr_t)src_tab[((size_t)g.chunk * n_layers + l) * 2];
      const char* sv = (const char*)(uintptr_t)src_tab[((size_t)g.chunk * n_layers + l) * 2 + 1];
      for (int h = 0; h < n_heads; ++h)
        for (int t = 0; t < g.n_tokens; ++t) {
          const int64_t so = ((int64_t)h * g.src_len + g.src_start + t) * D;
          const int64_t doff = (int64_t)l * layer_stride + (int64_t)h * head_stride + (int64_t)(g.dst_start + t) * D;
          char* dk = (char*)dst_k + doff * eb;
          if (g.delta == 0)
            memcpy(dk, sk + so * eb, (size_t)D * eb);
          else
            rotate_row(sk + so * eb, dk, 0, D, dt, c, s);
          memcpy((char*)dst_v + doff * eb, sv + so * eb, (size_t)D * eb);
        }
    }
  }
  return bad;
}

/* ---- fixed-order fp32 sums (the contract in include/chunkkv_amd.h) -------------------------- */

static float butterfly64(float* lanes) {
  float tmp[64];
  for (int m = 32; m >= 1; m >>= 1) {
    for (int l = 0; l < 64; ++l) tmp[l] = lanes[l] + lanes[l ^ m];
    memcpy(lanes, tmp, sizeof(tmp));
  }
  return lanes[0];
}

/* ---- a5: deviation ---------------------------------------------------------------------------- */

/* A NaN deviation or norm is reported as the canonical quiet NaN 0x7fc00000: IEEE 754 and torch
 * leave the payload of a NaN result open, and the ranking treats every NaN alike. */
static float canonical_nan(float x) {
  if (x == x) return x;
  const uint32_t u = 0x7fc00000u;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

int ckvo_deviation(const void* kf, int64_t kf_hs, int64_t kf_ts, const void* vf, int64_t vf_hs, int64_t vf_ts,
                   const void* kc, const void* vc, int64_t c_hs, const uint8_t* flags, const int32_t* local,
                   int n_tokens, int n_fresh, int n_heads, int D, int dt, float* diff, float* norm) {
  const int vec = dt == DT_BF16 ? 8 : 4;
  if (D % vec) return 1;
  const int vpr = D / vec, nvec = n_heads * vpr;
  int bad = 0;
  for (int p = 0; p < n_tokens; ++p) {
    const int j = local[p];
    if (j < 0 || j >= n_fresh) {
      bad |= j >= n_fresh;
      diff[p] = 0.0f;
      norm[p] = 0.0f;
      continue;
    }
    const int cached = (flags[p] & POS_CACHED) != 0;
    float sk[64] = {0}, sv[64] = {0}, nk[64] = {0}, nv[64] = {0};
    for (int q = 0; q < nvec; ++q) {
      const int lane = q % 64, h = q / vpr, d0 = (q % vpr) * vec;
      for (int e = 0; e < vec; ++e) {
        const float k = ld(kf, h * kf_hs + (int64_t)j * kf_ts + d0 + e, dt);
        const float v = ld(vf, h * vf_hs + (int64_t)j * vf_ts + d0 + e, dt);
        const float K = cached ? ld(kc, h * c_hs + (int64_t)p * D + d0 + e, dt) : 0.0f;
        const float V = cached ? ld(vc, h * c_hs + (int64_t)p * D + d0 + e, dt) : 0.0f;
        const float dk = round_to(k - K, dt);
        const float dv = round_to(v - V, dt);
        sk[lane] = sk[lane] + dk * dk;
        sv[lane] = sv[lane] + dv * dv;
        nk[lane] = nk[lane] + k * k;
        nv[lane] = nv[lane] + v * v;
      }
    }
    const float a = butterfly64(sk), b = butterfly64(sv), c = butterfly64(nk), d = butterfly64(nv);
    diff[p] = canonical_nan(a + b);
    norm[p] = canonical_nan(c + d);
  }
  return bad;
}

/* ---- a6 + a7 + a8: selection --------------------------------------------------------------- */

static uint32_t dev_key(float f) {
  if (f != f) return 0u;
  if (f == 0.0f) f = 0.0f;
  uint32_t u;
  memcpy(&u, &f, 4);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

typedef struct {
  uint32_t key;
  int32_t pos;
} cand_t;

static int cand_cmp(const void* a, const void* b) {
  const cand_t* x = (const cand_t*)a;
  const cand_t* y = (const cand_t*)b;
  if (x->key != y->key) return x->key > y->key ? -1 : 1; /* larger deviation first */
  return x->pos < y->pos ? -1 : (x->pos > y->pos);       /* then lower token index */
}

int ckvo_select(const float* diff, const float* norm, const uint8_t* flags, const int32_t* local, int n_tokens,
                const span_t* spans, int n_chunks, int has_thr, double thr, int64_t* keep_abs, int64_t* keep_local,
                float* rel_out, uint8_t* esc_out, int32_t* counts) {
  uint8_t* keep = (uint8_t*)calloc((size_t)n_tokens + 1, 1);
  uint8_t* pool = (uint8_t*)calloc((size_t)n_tokens + 1, 1);
  cand_t* cand = (cand_t*)malloc(sizeof(cand_t) * ((size_t)n_tokens + 1));
  if (!keep || !pool || !cand) {
    free(keep);
    free(pool);
    free(cand);
    return 2;
  }
  for (int p = 0; p < n_tokens; ++p) keep[p] = !(flags[p] & POS_CACHED) || (flags[p] & POS_SINK);
  int64_t budget_req = 0;
  int bad_span = 0;
  for (int c = 0; c < n_chunks; ++c) {
    const span_t sp = spans[c];
    const int ok = sp.start >= 0 && sp.length >= 0 && (int64_t)sp.start + sp.length <= n_tokens;
    float ld_[64] = {0}, ln_[64] = {0};
    if (ok)
      for (int q = 0; q < sp.length; ++q) {
        ld_[q % 64] = ld_[q % 64] + diff[sp.start + q];
        ln_[q % 64] = ln_[q % 64] + norm[sp.start + q];
      }
    const float sd = butterfly64(ld_), sn = butterfly64(ln_);
    const float rel = sd / sn;
    const int esc = ok && has_thr && ((double)rel > thr);
    rel_out[c] = rel;
    esc_out[c] = (uint8_t)esc;
    if (!ok) {
      bad_span++;
      continue;
    }
    if (esc) {
      memset(keep + sp.start, 1, (size_t)sp.length);
    } else if (sp.pooled) {
      memset(pool + sp.start, 1, (size_t)sp.length);
      budget_req += sp.budget;
    }
  }
  int n_cand = 0;
  for (int p = 0; p < n_tokens; ++p)
    if (pool[p] && !keep[p]) {
      cand[n_cand].key = dev_key(diff[p]);
      cand[n_cand].pos = p;
      n_cand++;
    }
  int64_t budget = budget_req < n_cand ? budget_req : n_cand;
  if (budget < 0) budget = 0;
  qsort(cand, (size_t)n_cand, sizeof(cand_t), cand_cmp);
  for (int64_t i = 0; i < budget; ++i) keep[cand[i].pos] = 1;
  int n = 0, sel_cached = 0, uncomputed = 0;
  for (int p = 0; p < n_tokens; ++p)
    if (keep[p]) {
      const int l = local[p];
      keep_abs[n] = p;
      keep_local[n] = l < 0 ? 0 : l;
      uncomputed += l < 0;
      sel_cached += (flags[p] & POS_CACHED) != 0;
      n++;
    }
  counts[0] = n;
  counts[1] = sel_cached;
  counts[2] = (int32_t)budget;
  counts[3] = n_cand;
  counts[4] = uncomputed;
  counts[5] = (int32_t)budget_req;
  counts[6] = bad_span;
  counts[7] = 0;
  free(keep);
  free(pool);
  free(cand);
  return 0;
}

/* ---- a9: scatter ---------------------------------------------------------------------------- */

int ckvo_scatter_rows(void* dk, void* dv, int64_t d_hs, const void* sk, int64_t sk_hs, int64_t sk_ts, const void* sv,
                      int64_t sv_hs, int64_t sv_ts, const int64_t* rows, int n_rows, int n_tokens, int n_heads, int D,
                      int dt) {
  const int eb = elem_size(dt);
  int bad = 0;
  for (int j = 0; j < n_rows; ++j) {
    const int64_t t = rows[j];
    if (t < 0 || t >= n_tokens) {
      bad = 1;
      continue;
    }
    for (int h = 0; h < n_heads; ++h) {
      memcpy((char*)dk + ((int64_t)h * d_hs + t * D) * eb, (const char*)sk + ((int64_t)h * sk_hs + (int64_t)j * sk_ts) * eb,
             (size_t)D * eb);
      memcpy((char*)dv + ((int64_t)h * d_hs + t * D) * eb, (const char*)sv + ((int64_t)h * sv_hs + (int64_t)j * sv_ts) * eb,
             (size_t)D * eb);
    }
  }
  return bad;
}
