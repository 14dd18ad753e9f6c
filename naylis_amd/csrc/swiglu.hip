// SwiGLU of the decoder's MLP, fused: transformers' LlamaMLP (inside every
// Naylis decoder layer, model.py:279-345) computes
//     h = silu(gate) * up,   silu(g) = g / (1 + exp(-g))
// as two elementwise launches forward (silu, product) and three backward
// (the product's two gradients, silu's backward).  Here one pass each way,
// rounding like those ops in the activation dtype: silu(g) rounded, then the
// product; backward d_silu = T(dh * up), du = T(dh * T(silu(g))),
// dg = T(d_silu * s * (1 + g * (1 - s))) with s = 1 / (1 + exp(-g)).
#include "common.h"
#include "timing.h"

namespace naylis {

namespace {

template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[4 + i] = b[i];
    }
  }
}

template <typename T>
__device__ __forceinline__ void store8(T* p, const float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    bf16x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (__bf16)v[e];
    *reinterpret_cast<bf16x8*>(p) = r;
  } else {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
}

template <typename T>
__device__ __forceinline__ float rnd(float v) {
  if constexpr (sizeof(T) == 2)
    return bf16_to_f32(f32_to_bf16(v));
  else
    return v;
}

}  // namespace

template <typename T>
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(const T* __restrict__ g, const T* __restrict__ u,
                                                         T* __restrict__ h, long n8) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  float gv[8], uv[8], out[8];
  load8(g + 8 * i, gv);
  load8(u + 8 * i, uv);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float s = rnd<T>(gv[e] / add_rn(1.0f, expf(-gv[e])));
    out[e] = mul_rn(s, uv[e]);
  }
  store8(h + 8 * i, out);
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const T* __restrict__ g, const T* __restrict__ u,
                                                         const T* __restrict__ dh, T* __restrict__ dg,
                                                         T* __restrict__ du, long n8) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  float gv[8], uv[8], dv[8], og[8], ou[8];
  load8(g + 8 * i, gv);
  load8(u + 8 * i, uv);
  load8(dh + 8 * i, dv);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float sig = 1.0f / add_rn(1.0f, expf(-gv[e]));
    const float silu = rnd<T>(gv[e] / add_rn(1.0f, expf(-gv[e])));
    const float ds = rnd<T>(mul_rn(dv[e], uv[e]));
    ou[e] = mul_rn(dv[e], silu);
    og[e] = mul_rn(mul_rn(ds, sig), add_rn(1.0f, mul_rn(gv[e], add_rn(1.0f, -sig))));
  }
  store8(dg + 8 * i, og);
  store8(du + 8 * i, ou);
}

hipError_t launch_swiglu(const void* g, const void* u, const void* dh, void* h_or_dg, void* du, bool bf16, bool bwd,
                         long n, hipStream_t st) {
  const long n8 = n / 8;
  if (n8 == 0) return hipSuccess;
  const dim3 grid((unsigned)((n8 + 255) / 256));
  if (!bwd) {
    if (bf16)
      NAYLIS_TIMED("swiglu_fwd", st, hipLaunchKernelGGL(swiglu_fwd_kernel<bf16_t>, grid, dim3(256), 0, st,
                                                        (const bf16_t*)g, (const bf16_t*)u, (bf16_t*)h_or_dg, n8));
    else
      NAYLIS_TIMED("swiglu_fwd", st, hipLaunchKernelGGL(swiglu_fwd_kernel<float>, grid, dim3(256), 0, st,
                                                        (const float*)g, (const float*)u, (float*)h_or_dg, n8));
  } else {
    if (bf16)
      NAYLIS_TIMED("swiglu_bwd", st, hipLaunchKernelGGL(swiglu_bwd_kernel<bf16_t>, grid, dim3(256), 0, st,
                                                        (const bf16_t*)g, (const bf16_t*)u, (const bf16_t*)dh,
                                                        (bf16_t*)h_or_dg, (bf16_t*)du, n8));
    else
      NAYLIS_TIMED("swiglu_bwd", st, hipLaunchKernelGGL(swiglu_bwd_kernel<float>, grid, dim3(256), 0, st,
                                                        (const float*)g, (const float*)u, (const float*)dh,
                                                        (float*)h_or_dg, (float*)du, n8));
  }
  return hipGetLastError();
}

}  // namespace naylis
