// The elementwise steps between a decoder layer's GEMMs, fused: residual add + RMSNorm, and the
// MLP's SiLU-gated product.
//
// Reference semantics: each layer of the blend prefill runs
//   x = layer.input_layernorm(h)                                (torch_engine.py:113, :191)
//   h = h + attn.o_proj(out)                                     (:71)
//   h = h + layer.mlp(layer.post_attention_layernorm(h))         (:72)
// and the logits read self.inner.norm(h) (:75), with the Hugging Face Qwen2/Llama modules
//   RMSNorm(h) = weight * (h.fp32 * rsqrt(mean(h.fp32^2) + eps)).to(dtype)
//   MLP(x)     = down_proj(silu(gate_proj(x)) * up_proj(x))
// In torch each norm is seven launches over fp32 temporaries and the gated product two.
//
// Design (gfx950): one workgroup per row for the norm. The row (<= 8192 elements) stays in
// registers between the sum of squares and the scaling, so h and delta are read once and h
// and y written once; the sum reduces with a wavefront butterfly and a fixed-order sum of the
// four wave totals. The gated product is one pass over 16-byte vectors of gate and up. Every
// rounding step of the modules is kept: the residual sum rounds to dtype, the normalised row
// rounds to dtype before the weight multiplies it, silu rounds to dtype before the product.
// Only the order of the fp32 sum of squares (torch: its reduction kernel's) and the rsqrt
// routine differ from torch.
#include "ckv_common.hpp"

namespace ckv {

constexpr int kNormThreads = 256;
constexpr int kNormMaxVecs = 4;  // 16-byte vectors per thread: hidden <= 256 * 4 * kVec
constexpr int kGateThreads = 256;
constexpr int kGateMaxRowBlocks = 65535;

template <int DTYPE, int VPT>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(char* h_out, const char* h_in,
                                                                   const char* __restrict__ delta,
                                                                   char* __restrict__ y,
                                                                   const char* __restrict__ weight, int n_vecs,
                                                                   int64_t row_b, float inv_n, float eps) {
  using E = Elem<DTYPE>;
  __shared__ float wave_sum[kNormThreads / kWave];
  const int64_t base = (int64_t)blockIdx.x * row_b;
  const int tid = threadIdx.x;
  float x[VPT][E::kVec];
  vec16 a[VPT], d[VPT];
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    const int v = tid + u * kNormThreads;
    if (v < n_vecs) {
      a[u] = ld16(h_in + base + (int64_t)v * 16);
      if (delta != nullptr) d[u] = ld16(delta + base + (int64_t)v * 16);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    const int v = tid + u * kNormThreads;
    if (v < n_vecs) {
      if (delta != nullptr) {
        float b[E::kVec];
        E::unpack(a[u], x[u]);
        E::unpack(d[u], b);
#pragma unroll
        for (int e = 0; e < E::kVec; ++e) x[u][e] = x[u][e] + b[e];
        a[u] = E::pack(x[u]);  // the residual stream, rounded to dtype
        st16(h_out + base + (int64_t)v * 16, a[u]);
      }
      E::unpack(a[u], x[u]);
#pragma unroll
      for (int e = 0; e < E::kVec; ++e) {
        const float sq = x[u][e] * x[u][e];
        ss = ss + sq;
      }
    }
  }
  ss = wave_butterfly_sum(ss);
  if ((tid & (kWave - 1)) == 0) wave_sum[tid / kWave] = ss;
  __syncthreads();
  float total = wave_sum[0];
#pragma unroll
  for (int w = 1; w < kNormThreads / kWave; ++w) total = total + wave_sum[w];
  const float var = total * inv_n;
  const float r = rsqrtf(var + eps);
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    const int v = tid + u * kNormThreads;
    if (v < n_vecs) {
      float w[E::kVec], o[E::kVec];
      E::unpack(ld16(weight + (int64_t)v * 16), w);
#pragma unroll
      for (int e = 0; e < E::kVec; ++e) o[e] = w[e] * E::round_trip(x[u][e] * r);
      st16(y + base + (int64_t)v * 16, E::pack(o));
    }
  }
}

#ifndef CKV_SILU_FAST
#define CKV_SILU_FAST 1
#endif

template <int DTYPE>
__global__ __launch_bounds__(kGateThreads) void silu_mul_kernel(char* __restrict__ out, int64_t out_rs_b,
                                                                const char* __restrict__ gate, int64_t gate_rs_b,
                                                                const char* __restrict__ up, int64_t up_rs_b,
                                                                int64_t n_rows, int vecs_per_row) {
  using E = Elem<DTYPE>;
  const int v = blockIdx.x * kGateThreads + threadIdx.x;
  if (v >= vecs_per_row) return;
  const int64_t cb = (int64_t)v * 16;
  for (int64_t row = blockIdx.y; row < n_rows; row += gridDim.y) {
    float g[E::kVec], u[E::kVec], o[E::kVec];
    E::unpack(ld16(gate + row * gate_rs_b + cb), g);
    E::unpack(ld16(up + row * up_rs_b + cb), u);
#pragma unroll
    for (int e = 0; e < E::kVec; ++e) {
      if constexpr (CKV_SILU_FAST) {
        // exp(-g) = 2^(-g log2 e) and 1/den on the hardware's exp2 and reciprocal (about 1 ulp
        // each in fp32), not the library's exp and IEEE division: a third of the VALU work,
        // which otherwise bounds the kernel at the 8k request's width
        const float den = 1.0f + __builtin_amdgcn_exp2f(-1.44269504088896341f * g[e]);
        o[e] = E::round_trip(g[e] * __builtin_amdgcn_rcpf(den)) * u[e];
      } else {
        const float den = 1.0f + expf(-g[e]);
        o[e] = E::round_trip(g[e] / den) * u[e];
      }
    }
    st16(out + row * out_rs_b + cb, E::pack(o));
  }
}

template <int DTYPE>
int launch_add_rmsnorm(void* h_out, const void* h_in, const void* delta, void* y, const void* weight,
                       int64_t n_rows, int32_t hidden, float eps, hipStream_t stream) {
  using E = Elem<DTYPE>;
  if (hidden % E::kVec != 0) return CKV_ERR_INVALID_ARGUMENT;
  const int n_vecs = hidden / E::kVec;
  if (n_vecs > kNormThreads * kNormMaxVecs) return CKV_ERR_TOO_LARGE;
  const int vpt = (n_vecs + kNormThreads - 1) / kNormThreads;
  const int64_t row_b = (int64_t)hidden * E::kBytes;
  const float inv_n = 1.0f / (float)hidden;
  auto args = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3((unsigned)n_rows), dim3(kNormThreads), 0, stream, (char*)h_out,
                       (const char*)h_in, (const char*)delta, (char*)y, (const char*)weight, n_vecs, row_b, inv_n,
                       eps);
  };
  switch (vpt) {
    case 1: args(add_rmsnorm_kernel<DTYPE, 1>); break;
    case 2: args(add_rmsnorm_kernel<DTYPE, 2>); break;
    case 3: args(add_rmsnorm_kernel<DTYPE, 3>); break;
    default: args(add_rmsnorm_kernel<DTYPE, 4>); break;
  }
  CKV_RETURN_IF_LAUNCH_FAILED();
  return CKV_OK;
}

template <int DTYPE>
int launch_silu_mul(void* out, int64_t out_rs, const void* gate, int64_t gate_rs, const void* up, int64_t up_rs,
                    int64_t n_rows, int32_t width, hipStream_t stream) {
  using E = Elem<DTYPE>;
  if (width % E::kVec != 0) return CKV_ERR_INVALID_ARGUMENT;
  if (out_rs < width || gate_rs < width || up_rs < width) return CKV_ERR_OUT_OF_RANGE;
  if (out_rs % E::kVec != 0 || gate_rs % E::kVec != 0 || up_rs % E::kVec != 0) return CKV_ERR_INVALID_ARGUMENT;
  const int vpr = width / E::kVec;
  const unsigned col_blocks = (unsigned)((vpr + kGateThreads - 1) / kGateThreads);
  const unsigned row_blocks = (unsigned)(n_rows < kGateMaxRowBlocks ? n_rows : kGateMaxRowBlocks);
  hipLaunchKernelGGL(silu_mul_kernel<DTYPE>, dim3(col_blocks, row_blocks), dim3(kGateThreads), 0, stream,
                     (char*)out, out_rs * E::kBytes, (const char*)gate, gate_rs * E::kBytes, (const char*)up,
                     up_rs * E::kBytes, n_rows, vpr);
  CKV_RETURN_IF_LAUNCH_FAILED();
  return CKV_OK;
}

}  // namespace ckv

extern "C" int32_t ckv_add_rmsnorm(void* h_out, const void* h_in, const void* delta, void* y, const void* weight,
                                   int64_t n_rows, int32_t hidden, float eps, int32_t dtype, void* stream) {
  using namespace ckv;
  if (n_rows < 0 || n_rows > 0x7fffffff || hidden <= 0 || !(eps >= 0.f)) return CKV_ERR_INVALID_ARGUMENT;
  if (n_rows == 0) return CKV_OK;
  if (h_in == nullptr || y == nullptr || weight == nullptr || (delta != nullptr && h_out == nullptr))
    return CKV_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == CKV_DTYPE_BF16) return launch_add_rmsnorm<CKV_DTYPE_BF16>(h_out, h_in, delta, y, weight, n_rows, hidden, eps, s);
  if (dtype == CKV_DTYPE_F32) return launch_add_rmsnorm<CKV_DTYPE_F32>(h_out, h_in, delta, y, weight, n_rows, hidden, eps, s);
  return CKV_ERR_INVALID_ARGUMENT;
}

extern "C" int32_t ckv_silu_mul(void* out, int64_t out_row_stride, const void* gate, int64_t gate_row_stride,
                                const void* up, int64_t up_row_stride, int64_t n_rows, int32_t width, int32_t dtype,
                                void* stream) {
  using namespace ckv;
  if (n_rows < 0 || width <= 0) return CKV_ERR_INVALID_ARGUMENT;
  if (n_rows == 0) return CKV_OK;
  if (out == nullptr || gate == nullptr || up == nullptr) return CKV_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == CKV_DTYPE_BF16)
    return launch_silu_mul<CKV_DTYPE_BF16>(out, out_row_stride, gate, gate_row_stride, up, up_row_stride, n_rows, width, s);
  if (dtype == CKV_DTYPE_F32)
    return launch_silu_mul<CKV_DTYPE_F32>(out, out_row_stride, gate, gate_row_stride, up, up_row_stride, n_rows, width, s);
  return CKV_ERR_INVALID_ARGUMENT;
}
