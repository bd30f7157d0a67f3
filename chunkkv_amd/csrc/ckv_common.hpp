// Shared device helpers for the gfx950 KV-repair kernels: element traits, 16-byte vector
// loads and stores, round-to-nearest-even casts and wavefront reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "chunkkv_amd.h"
#include "cos_sin.hpp"

namespace ckv {

constexpr int kWave = 64;  // CDNA wavefront width

// 16-byte vector: the unit of every global load and store (global_load_dwordx4).
typedef unsigned int vec16 __attribute__((ext_vector_type(4)));

// ---- element conversions --------------------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Two fp32 -> bf16, round-to-nearest-even, packed (lo in bits 0-15): gfx950's packed hardware
// conversion (v_cvt_pk_bf16_f32), which rounds every non-NaN input (denormals, ties, overflow
// to infinity) exactly as adding 0x7fff + lsb to the bit pattern and truncating does, checked
// over all 2^32 inputs in both slots; a NaN becomes the canonical quiet NaN 0x7fc0, which is
// what torch's BFloat16 conversion produces.
typedef __bf16 bf16x2_cvt __attribute__((ext_vector_type(2)));
typedef float f32x2_cvt __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
  const f32x2_cvt v = {lo, hi};
  uint32_t r = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_cvt));
  r = lo != lo ? (r & 0xffff0000u) | 0x7fc0u : r;
  r = hi != hi ? (r & 0x0000ffffu) | 0x7fc00000u : r;
  return r;
}

// Two fp32 values rounded to bf16 (round-to-nearest-even) and back to fp32, for arithmetic only:
// one packed conversion for both. A NaN input gives a NaN (the hardware conversion maps every
// fp32 NaN to a bf16 NaN; checked over all 2^24 NaN patterns in both slots) with an unspecified
// payload, so callers whose results may be NaN canonicalize them (canonical_nan) before storing.
__device__ __forceinline__ void bf16_round_pair(float a, float b, float& ra, float& rb) {
  const f32x2_cvt v = {a, b};
  const uint32_t r = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_cvt));
  ra = __uint_as_float(r << 16);
  rb = __uint_as_float(r & 0xffff0000u);
}

// x, or the canonical quiet NaN 0x7fc00000 if x is a NaN (any sign or payload).
__device__ __forceinline__ float canonical_nan(float x) { return x != x ? __uint_as_float(0x7fc00000u) : x; }

// fp32 -> bf16 bits, round-to-nearest-even, NaN -> 0x7fc0.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) { return f32x2_to_bf16x2_bits(f, 0.0f) & 0xffffu; }

// Element traits: VEC elements per 16-byte vector, unpack to fp32, pack with rounding.
template <int DTYPE>
struct Elem;

template <>
struct Elem<CKV_DTYPE_BF16> {
  static constexpr int kBytes = 2;
  static constexpr int kVec = 8;
  __device__ __forceinline__ static void unpack(const vec16& v, float (&f)[kVec]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = bf16_bits_to_f32(w[i] & 0xffffu);
      f[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
    }
  }
  __device__ __forceinline__ static vec16 pack(const float (&f)[kVec]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = f32x2_to_bf16x2_bits(f[2 * i], f[2 * i + 1]);
    return vec16{w[0], w[1], w[2], w[3]};
  }
  // value after rounding to the element type, back in fp32
  __device__ __forceinline__ static float round_trip(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }
  // two values rounded to the element type and back, for arithmetic (NaN payloads unspecified)
  __device__ __forceinline__ static void round_trip2(float a, float b, float& ra, float& rb) {
    bf16_round_pair(a, b, ra, rb);
  }
};

template <>
struct Elem<CKV_DTYPE_F32> {
  static constexpr int kBytes = 4;
  static constexpr int kVec = 4;
  __device__ __forceinline__ static void unpack(const vec16& v, float (&f)[kVec]) {
    f[0] = __uint_as_float(v.x);
    f[1] = __uint_as_float(v.y);
    f[2] = __uint_as_float(v.z);
    f[3] = __uint_as_float(v.w);
  }
  __device__ __forceinline__ static vec16 pack(const float (&f)[kVec]) {
    return vec16{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3])};
  }
  __device__ __forceinline__ static float round_trip(float f) { return f; }
  __device__ __forceinline__ static void round_trip2(float a, float b, float& ra, float& rb) {
    ra = a;
    rb = b;
  }
};

// ---- memory -----------------------------------------------------------------------------

// All kernel operands live in global memory; saying so (address space 1) makes the compiler
// emit global_load/global_store, which wait on vmcnt alone, instead of flat accesses.
typedef __attribute__((address_space(1))) vec16 gvec16;

__device__ __forceinline__ vec16 ld16(const void* p) { return *(const gvec16*)p; }
__device__ __forceinline__ void st16(void* p, const vec16& v) { *(gvec16*)p = v; }

// Streaming variants: data touched once per launch, so keep it out of the caches' way.
__device__ __forceinline__ vec16 ld16_stream(const void* p) { return __builtin_nontemporal_load((const gvec16*)p); }
__device__ __forceinline__ void st16_stream(void* p, const vec16& v) { __builtin_nontemporal_store(v, (gvec16*)p); }

// Stores with device scope (sc1): written through the L2 as they go, so the end-of-launch release
// has none of their lines left to write back; with nt also non-temporal. No builtin sets sc1 on a
// 16-byte store, so the instruction is written out, and the compiler does not know it is a store:
// a store of more than 8 bytes reads its data registers after it issues, and an instruction that
// overwrites them right after it corrupts the stored data (the compiler pads the stores it emits
// itself). The s_nop after each store supplies those wait states. The memory clobber keeps the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void st16_agent(void* p, const vec16& v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 4" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st16_agent_stream(void* p, const vec16& v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1 nt\n\ts_nop 4" ::"v"(p), "v"(v) : "memory");
}

// A 16-byte store by cache policy (a launch shape's property).
enum StorePolicy { kStRegular = 0, kStStream = 1, kStAgent = 2, kStAgentStream = 3 };
template <int P>
__device__ __forceinline__ void st16_policy(void* p, const vec16& v) {
  if constexpr (P == kStRegular) st16(p, v);
  else if constexpr (P == kStStream) st16_stream(p, v);
  else if constexpr (P == kStAgent) st16_agent(p, v);
  else st16_agent_stream(p, v);
}

// ---- wavefront reductions -----------------------------------------------------------------

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// x of another lane through a DPP row operation (VALU, no LDS round trip); lanes whose source
// is outside the row, or whose row is not in ROW_MASK, read 0.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_or_zero(uint32_t x) {
  return __builtin_amdgcn_update_dpp(0u, x, CTRL, ROW_MASK, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(x), CTRL, 0xf, 0xf, false));
}

// Butterfly sum over the 64 lanes: x_l + x_{l^m} for m = 32, 16, 8, 4, 2, 1, each lane adding
// its own value first. Every lane ends with the same value because fp32 addition commutes; the
// tree is part of the bit-exact contract. The partners come from gfx950's VALU permutes, not
// LDS shuffles: xor 32 and 16 from the row-swap permutes (which return the lane's own value and
// its partner in a lane-dependent order), xor 8 from rotating a 16-lane row by 8, xor 4 from
// rotating it by 4 (lane l+4 of the row holds the same value as lane l^4 once the xor-8 step
// has made lanes 8 apart equal), xor 2 and 1 from quad permutes. Checked against the xor-shuffle
// tree bit for bit on the GPU.
__device__ __forceinline__ float wave_butterfly_sum(float x) {
  const int l = lane_id();
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = x + __uint_as_float(l < 32 ? a[1] : a[0]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = x + __uint_as_float((l & 16) == 0 ? b[1] : b[0]);
  x = x + dpp_f32<0x128>(x);  // row_ror:8
  x = x + dpp_f32<0x124>(x);  // row_ror:4
  x = x + dpp_f32<0x4e>(x);   // quad_perm [2, 3, 0, 1]
  x = x + dpp_f32<0xb1>(x);   // quad_perm [1, 0, 3, 2]
  return x;
}

// Inclusive prefix sum over the 64 lanes in lane order: shifts within 16-lane rows, then row 15
// broadcast into rows 1 and 3 and lane 31 into rows 2 and 3 (integer sums: order-free).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
  x += dpp_or_zero<0x111>(x);  // row_shr:1
  x += dpp_or_zero<0x112>(x);  // row_shr:2
  x += dpp_or_zero<0x114>(x);  // row_shr:4
  x += dpp_or_zero<0x118>(x);  // row_shr:8
  x += dpp_or_zero<0x142, 0xa>(x);  // row_bcast:15
  x += dpp_or_zero<0x143, 0xc>(x);  // row_bcast:31
  return x;
}
__device__ __forceinline__ uint64_t wave_incl_scan(uint64_t x) {
  auto step = [](uint64_t v, auto ctrl) {
    constexpr int C = decltype(ctrl)::value & 0xfff, RM = decltype(ctrl)::value >> 12;
    return v + (((uint64_t)dpp_or_zero<C, RM>((uint32_t)(v >> 32)) << 32) | dpp_or_zero<C, RM>((uint32_t)v));
  };
  x = step(x, std::integral_constant<int, 0xf111>{});
  x = step(x, std::integral_constant<int, 0xf112>{});
  x = step(x, std::integral_constant<int, 0xf114>{});
  x = step(x, std::integral_constant<int, 0xf118>{});
  x = step(x, std::integral_constant<int, 0xa142>{});
  x = step(x, std::integral_constant<int, 0xc143>{});
  return x;
}

__device__ __forceinline__ void flag_error(int32_t* err, uint32_t bits) {
  if (err != nullptr) atomicOr(reinterpret_cast<unsigned int*>(err), bits);
}

// ---- rotary frequencies -------------------------------------------------------------------

// inv_freq_i = fp32(theta_f ** e_i), e_i = fp32(-(2i) / D), i < D/2: the reference's fp32
// expression `base ** (-arange(0, D, 2) / D)` (torch_engine.py:33), evaluated on the host in fp64
// (libm pow) and rounded once, as the reference computes it once per engine. Kernels take the
// D/2 values by value in their arguments (no table in device memory, no pow on the device).
constexpr int kMaxHalf = 128;  // head_dim <= 256
struct alignas(16) InvFreq {
  float v[kMaxHalf];
};

// The last (head_dim, theta) per host thread is kept: launches of one model reuse it.
inline const InvFreq& host_inv_freq(int head_dim, double theta) {
  static thread_local int c_dim = 0;
  static thread_local double c_theta = 0.0;
  static thread_local InvFreq c_val;
  if (head_dim != c_dim || !(theta == c_theta)) {
    const float theta_f = (float)theta;
    for (int i = 0; i < kMaxHalf; ++i) {
      const float e = (float)(-2 * i) / (float)head_dim;
      c_val.v[i] = i < head_dim / 2 ? (float)std::pow((double)theta_f, (double)e) : 0.0f;
    }
    c_dim = head_dim;
    c_theta = theta;
  }
  return c_val;
}

// cos/sin of an fp32 angle, each evaluated in fp64 and rounded once to fp32 (x = cos, y = sin):
// the short reduction + series of cos_sin.hpp for |ang| < 2^31, the library's fp64 sincos beyond.
__device__ __forceinline__ float2 angle_cos_sin(float ang) {
  float c, s;
  if (!cos_sin_fast(ang, c, s)) {
    double sd, cd;
    sincos((double)ang, &sd, &cd);
    c = (float)cd;
    s = (float)sd;
  }
  return make_float2(c, s);
}

// N angles at once: the fast evaluations first, without branches between them, then the library
// sincos for any angle they do not cover (one branch, taken only for |angle| >= 2^31).
template <int N>
__device__ __forceinline__ void angles_cos_sin(const float (&ang)[N], float (&c)[N], float (&s)[N]) {
  bool all = true;
#pragma unroll
  for (int e = 0; e < N; ++e) all = cos_sin_fast(ang[e], c[e], s[e]) && all;
  if (!all) {
#pragma unroll
    for (int e = 0; e < N; ++e) {
      if (!(std::fabs(ang[e]) < 0x1p31f)) {
        double sd, cd;
        sincos((double)ang[e], &sd, &cd);
        c[e] = (float)cd;
        s[e] = (float)sd;
      }
    }
  }
}

// cos/sin of the shift `delta` at inverse frequency inv: the fp32 angle fl32(fl32(delta) * inv),
// as torch forms `delta * inv_freq`, then cos/sin of that angle evaluated in fp64 and rounded
// once, i.e. the correctly rounded fp32 values. (x = cos, y = sin.)
__device__ __forceinline__ float2 shift_cos_sin(float inv, int delta) { return angle_cos_sin((float)delta * inv); }

// Rotate VEC frequency pairs held as two 16-byte vectors: a = first-half elements, b = the
// matching second-half elements. y1 = a*cos - b*sin, y2 = a*sin + b*cos with every product and
// sum rounded separately in fp32 (callers build with -ffp-contract=off), then one rounding to
// the element type.
template <int DTYPE>
__device__ __forceinline__ void rotate_pairs(const vec16& a16, const vec16& b16, const float* c, const float* s,
                                             vec16& y1_16, vec16& y2_16) {
  using E = Elem<DTYPE>;
  float a[E::kVec], b[E::kVec], y1[E::kVec], y2[E::kVec];
  E::unpack(a16, a);
  E::unpack(b16, b);
#pragma unroll
  for (int e = 0; e < E::kVec; ++e) {
    const float p1 = a[e] * c[e];
    const float p2 = b[e] * s[e];
    const float p3 = a[e] * s[e];
    const float p4 = b[e] * c[e];
    y1[e] = p1 - p2;
    y2[e] = p3 + p4;
  }
  y1_16 = E::pack(y1);
  y2_16 = E::pack(y2);
}

}  // namespace ckv

// Host-side status helper shared by the entry points.
#define CKV_RETURN_IF_LAUNCH_FAILED()              \
  do {                                             \
    if (hipGetLastError() != hipSuccess) return CKV_ERR_HIP; \
  } while (0)
