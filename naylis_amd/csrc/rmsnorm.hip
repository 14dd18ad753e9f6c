// RMSNorm of the Naylis decoder, fused: model.py:304-305 builds the MoM
// layer's pre-norm (mom_norm) and the Llama block's norms as LlamaRMSNorm (or
// Liger's fused RMSNorm), computed as
//     h = fp32(x) * rsqrt(mean(fp32(x)^2) + eps),   y = w * h.to(x.dtype)
// In bf16 that is seven elementwise / reduction launches forward and about
// ten backward, each a pass over the (N, D) activations; here one pass each.
//
// One wave per row, 8 consecutive features per lane and chunk (16-byte bf16
// or 32-byte fp32 loads), CH = D / 512 chunks held in registers; the row's
// sum of squares is a butterfly over the wave.  The backward walks rows with
// a fixed grid (a function of N only), keeps the weight-gradient partial of
// its rows in registers, sums the four waves of a workgroup in order and the
// workgroups in order in a second launch: deterministic.
#include <type_traits>

#include "common.h"
#include "timing.h"

namespace naylis {

namespace {

template <typename T>
struct Chunk;  // 8 values of a row

template <>
struct Chunk<bf16_t> {
  uint4 raw;
  __device__ __forceinline__ void load(const bf16_t* p) { raw = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ float get(int e) const {
    const uint32_t w = (&raw.x)[e >> 1];
    return __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
  }
};

template <>
struct Chunk<float> {
  f32x4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = *reinterpret_cast<const f32x4*>(p);
    b = *reinterpret_cast<const f32x4*>(p + 4);
  }
  __device__ __forceinline__ float get(int e) const { return e < 4 ? a[e] : b[e - 4]; }
};

// value as stored in T (round to nearest even for bf16), back in fp32
template <typename T>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (sizeof(T) == 2)
    return bf16_to_f32(f32_to_bf16(v));
  else
    return v;
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

}  // namespace

constexpr int kNormBwdWgs = 512;  // workgroups of the backward (fewer when N is small)

// AT: dtype of the residual branch a (void: no add).  With a, the row is
// first s = x + T(a) (the residual add of the decoder block, a rounded to
// the stream's dtype first), written to s_out, and s is normalised.
template <typename T, typename AT, int CH>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(const T* __restrict__ x, const AT* __restrict__ a,
                                                          const T* __restrict__ w, T* __restrict__ s_out,
                                                          T* __restrict__ y, float* __restrict__ rstd, long N, int D,
                                                          float eps) {
  constexpr bool ADD = !std::is_same<AT, void>::value;
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;
  const T* xr = x + row * D;
  Chunk<T> xc[CH], wc[CH];
  float xv[CH][8];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    xc[c].load(xr + (c * 64 + lane) * 8);
    wc[c].load(w + (c * 64 + lane) * 8);
  }
  if constexpr (ADD) {
    Chunk<AT> ac[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) ac[c].load(a + row * D + (c * 64 + lane) * 8);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[c][e] = round_to<T>(add_rn(xc[c].get(e), round_to<T>(ac[c].get(e))));
      store8(s_out + row * D + (c * 64 + lane) * 8, xv[c]);
    }
  } else {
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[c][e] = xc[c].get(e);
  }
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(xv[c][e], xv[c][e], ss);
  ss = wave_allsum(ss);
  const float r = rsqrtf(add_rn(mul_rn(ss, 1.0f / (float)D), eps));
  T* yr = y + row * D;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = mul_rn(wc[c].get(e), round_to<T>(mul_rn(xv[c][e], r)));
    store8(yr + (c * 64 + lane) * 8, v);
  }
  if (lane == 0) rstd[row] = r;
}

// dres (optional): gradient arriving at x from elsewhere (the residual
// stream), added to the norm's input gradient before the one rounding
template <typename T, int CH>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                          const float* __restrict__ rstd, const T* __restrict__ dy,
                                                          const T* __restrict__ dres, T* __restrict__ dx,
                                                          float* __restrict__ dw_part, long N, int D) {
  __shared__ float red[3][CH * 512];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long stride = (long)gridDim.x * 4;
  Chunk<T> wc[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) wc[c].load(w + (c * 64 + lane) * 8);
  float dwa[CH][8];
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) dwa[c][e] = 0.f;
  for (long row = (long)blockIdx.x * 4 + wave; row < N; row += stride) {
    Chunk<T> xc[CH], gc[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      xc[c].load(x + row * D + (c * 64 + lane) * 8);
      gc[c].load(dy + row * D + (c * 64 + lane) * 8);
    }
    const float r = rstd[row];
    // h = x r; y = w * T(h): dw += dy * T(h), d T(h) = T(dy * w) (the product in the output dtype)
    float h[CH][8], dh[CH][8];
    float m = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        h[c][e] = mul_rn(xc[c].get(e), r);
        dwa[c][e] = fmaf(gc[c].get(e), round_to<T>(h[c][e]), dwa[c][e]);
        dh[c][e] = round_to<T>(mul_rn(gc[c].get(e), wc[c].get(e)));
        m = fmaf(dh[c][e], h[c][e], m);
      }
    m = wave_allsum(m) * (1.0f / (float)D);
    // dx = r (dh - h mean(dh h)) (+ dres)
    Chunk<T> rc[CH];
    if (dres != nullptr) {
#pragma unroll
      for (int c = 0; c < CH; ++c) rc[c].load(dres + row * D + (c * 64 + lane) * 8);
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[e] = r * fmaf(-h[c][e], m, dh[c][e]);
        if (dres != nullptr) v[e] += rc[c].get(e);
      }
      store8(dx + row * D + (c * 64 + lane) * 8, v);
    }
  }
  // the workgroup's weight-gradient partial: waves 0..3 in order
  if (wave > 0) {
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) red[wave - 1][(c * 64 + lane) * 8 + e] = dwa[c][e];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int f = (c * 64 + lane) * 8 + e;
        v[e] = ((dwa[c][e] + red[0][f]) + red[1][f]) + red[2][f];
      }
      float* out = dw_part + (long)blockIdx.x * D + (c * 64 + lane) * 8;
      *reinterpret_cast<f32x4*>(out) = f32x4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<f32x4*>(out + 4) = f32x4{v[4], v[5], v[6], v[7]};
    }
  }
}

// dw = sum of the partials in a fixed order, in the weight's dtype: a
// workgroup takes 64 features (16 lanes of 4), its 16 groups of threads each
// sum every 16th partial (16 loads in flight), then the group sums are added
// in group order
template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_dw_reduce_kernel(const float* __restrict__ dw_part,
                                                                T* __restrict__ dw, int parts, int D) {
  __shared__ f32x4 gsum[16][16];
  const int q = threadIdx.x & 15, grp = threadIdx.x >> 4;
  const int f = blockIdx.x * 64 + 4 * q;
  f32x4 s = f32x4{};
  if (f < D) {
    for (int p0 = grp; p0 < parts; p0 += 16 * 16) {
      f32x4 v[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int p = p0 + 16 * i;
        v[i] = p < parts ? *reinterpret_cast<const f32x4*>(dw_part + (long)p * D + f) : f32x4{};
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) s += v[i];
    }
  }
  gsum[grp][q] = s;
  __syncthreads();
  if (grp == 0 && f < D) {
    f32x4 t = gsum[0][q];
#pragma unroll
    for (int gi = 1; gi < 16; ++gi) t += gsum[gi][q];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (sizeof(T) == 2)
        dw[f + e] = f32_to_bf16(t[e]);
      else
        dw[f + e] = t[e];
    }
  }
}

int rmsnorm_bwd_parts(long N) {
  const long wgs = (N + 3) / 4;
  return (int)(wgs < kNormBwdWgs ? (wgs > 0 ? wgs : 1) : kNormBwdWgs);
}

size_t rmsnorm_ws_bytes(long N, int D) { return (size_t)rmsnorm_bwd_parts(N) * D * sizeof(float); }

template <typename T, typename AT>
static hipError_t fwd_t(const void* x, const void* a, const void* w, void* s_out, void* y, float* rstd, long N, int D,
                        float eps, hipStream_t st) {
  const dim3 grid((unsigned)((N + 3) / 4));
  const int ch = D / 512;
  constexpr bool kAdd = !std::is_same<AT, void>::value;
  const char* kname = kAdd ? "add_rmsnorm_fwd" : "rmsnorm_fwd";
#define NAYLIS_NORM_FWD(C)                                                                                    \
  case C:                                                                                                     \
    NAYLIS_TIMED(kname, st,                                                                                   \
                 hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, AT, C>), grid, dim3(256), 0, st, (const T*)x,      \
                                    (const AT*)a, (const T*)w, (T*)s_out, (T*)y, rstd, N, D, eps));           \
    break;
  switch (ch) {
    NAYLIS_NORM_FWD(1)
    NAYLIS_NORM_FWD(2)
    NAYLIS_NORM_FWD(3)
    NAYLIS_NORM_FWD(4)
    NAYLIS_NORM_FWD(5)
    NAYLIS_NORM_FWD(6)
    NAYLIS_NORM_FWD(7)
    NAYLIS_NORM_FWD(8)
    default:
      return hipErrorInvalidValue;
  }
#undef NAYLIS_NORM_FWD
  return hipGetLastError();
}

template <typename T>
static hipError_t bwd_t(const void* x, const void* w, const float* rstd, const void* dy, const void* dres, void* dx,
                        void* dw, float* part, long N, int D, hipStream_t st) {
  const int parts = rmsnorm_bwd_parts(N);
  const int ch = D / 512;
#define NAYLIS_NORM_BWD(C)                                                                                     \
  case C:                                                                                                      \
    NAYLIS_TIMED("rmsnorm_bwd", st,                                                                            \
                 hipLaunchKernelGGL((rmsnorm_bwd_kernel<T, C>), dim3(parts), dim3(256), 0, st, (const T*)x,    \
                                    (const T*)w, rstd, (const T*)dy, (const T*)dres, (T*)dx, part, N, D));     \
    break;
  switch (ch) {
    NAYLIS_NORM_BWD(1)
    NAYLIS_NORM_BWD(2)
    NAYLIS_NORM_BWD(3)
    NAYLIS_NORM_BWD(4)
    NAYLIS_NORM_BWD(5)
    NAYLIS_NORM_BWD(6)
    NAYLIS_NORM_BWD(7)
    NAYLIS_NORM_BWD(8)
    default:
      return hipErrorInvalidValue;
  }
#undef NAYLIS_NORM_BWD
  NAYLIS_TIMED("rmsnorm_dw_reduce", st,
               hipLaunchKernelGGL((rmsnorm_dw_reduce_kernel<T>), dim3((D + 63) / 64), dim3(256), 0, st, part,
                                  (T*)dw, parts, D));
  return hipGetLastError();
}

hipError_t launch_rmsnorm_fwd(const void* x, bool bf16, const void* w, void* y, float* rstd, long N, int D,
                              float eps, hipStream_t st) {
  if (N == 0) return hipSuccess;
  return bf16 ? fwd_t<bf16_t, void>(x, nullptr, w, nullptr, y, rstd, N, D, eps, st)
              : fwd_t<float, void>(x, nullptr, w, nullptr, y, rstd, N, D, eps, st);
}

hipError_t launch_add_rmsnorm_fwd(const void* x, const void* a, bool a_f32, bool bf16, const void* w, void* s_out,
                                  void* y, float* rstd, long N, int D, float eps, hipStream_t st) {
  if (N == 0) return hipSuccess;
  if (bf16)
    return a_f32 ? fwd_t<bf16_t, float>(x, a, w, s_out, y, rstd, N, D, eps, st)
                 : fwd_t<bf16_t, bf16_t>(x, a, w, s_out, y, rstd, N, D, eps, st);
  return fwd_t<float, float>(x, a, w, s_out, y, rstd, N, D, eps, st);
}

hipError_t launch_rmsnorm_bwd(const void* x, bool bf16, const void* w, const float* rstd, const void* dy,
                              const void* dres, void* dx, void* dw, void* ws, long N, int D, hipStream_t st) {
  float* part = (float*)ws;
  if (N == 0) {
    // no rows: dw = 0 (the reduction over zero partials)
    if (bf16)
      hipLaunchKernelGGL((rmsnorm_dw_reduce_kernel<bf16_t>), dim3((D + 63) / 64), dim3(256), 0, st, part,
                         (bf16_t*)dw, 0, D);
    else
      hipLaunchKernelGGL((rmsnorm_dw_reduce_kernel<float>), dim3((D + 63) / 64), dim3(256), 0, st, part,
                         (float*)dw, 0, D);
    return hipGetLastError();
  }
  return bf16 ? bwd_t<bf16_t>(x, w, rstd, dy, dres, dx, dw, part, N, D, st)
              : bwd_t<float>(x, w, rstd, dy, dres, dx, dw, part, N, D, st);
}

}  // namespace naylis
