// ReZero output gate of the MoM layer (model.py:151 `mom_scale`, applied at
// model.py:239):
//     y = s * z                 z = o_proj output (bf16 or fp32), s = the (1,)
//                               fp32 parameter, y fp32 (type promotion)
// backward:
//     dz = s * dy  (in z's dtype)        ds = sum_i dy_i * z_i  (fp32)
// The backward is one pass over dy and z; ds is reduced through per-workgroup
// partials summed in a fixed order (deterministic).
//
// The same scale with a bf16 (or fp32) result, y = s * x in y's dtype, folds
// the gate into the o projection's weight (s * (o W^T) = o (s W)^T): the
// layer then gets y straight from one GEMM with an fp32 result, and the
// backward's dW = s * dW' and ds = sum(W * dW'), dW' the gradient of the
// scaled weight, are this file's backward run over the weight's elements.
#include "common.h"
#include "launch_rezero.h"
#include "timing.h"

namespace naylis {

constexpr int kRzThreads = 256;
constexpr int kRzVec = 8;                                  // elements per thread and step
constexpr int kRzSteps = 4;                                // steps per thread
constexpr int kRzChunk = kRzThreads * kRzVec * kRzSteps;  // elements per workgroup

template <typename T>
__device__ __forceinline__ void ld8(const T* p, float (&v)[8]);
template <>
__device__ __forceinline__ void ld8<float>(const float* p, float (&v)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = a[e];
    v[4 + e] = b[e];
  }
}
template <>
__device__ __forceinline__ void ld8<bf16_t>(const bf16_t* p, float (&v)[8]) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[2 * e] = __uint_as_float(w[e] << 16);
    v[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
  }
}

template <typename T>
__device__ __forceinline__ void st8(T* p, const float (&v)[8]);
template <>
__device__ __forceinline__ void st8<float>(float* p, const float (&v)[8]) {
  *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
  *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
}
template <>
__device__ __forceinline__ void st8<bf16_t>(bf16_t* p, const float (&v)[8]) {
  uint4 u;
  uint32_t* w = reinterpret_cast<uint32_t*>(&u);
#pragma unroll
  for (int e = 0; e < 4; ++e) w[e] = (uint32_t)f32_to_bf16(v[2 * e]) | ((uint32_t)f32_to_bf16(v[2 * e + 1]) << 16);
  *reinterpret_cast<uint4*>(p) = u;
}

template <typename T>
__device__ __forceinline__ float ld1(const T* p) {
  if constexpr (sizeof(T) == 2)
    return bf16_to_f32(*p);
  else
    return *p;
}
template <typename T>
__device__ __forceinline__ void st1(T* p, float x) {
  if constexpr (sizeof(T) == 2)
    *p = f32_to_bf16(x);
  else
    *p = x;
}

template <typename ZT, typename YT>
__global__ __launch_bounds__(kRzThreads) void rezero_fwd_kernel(const ZT* __restrict__ z, const float* __restrict__ s,
                                                                YT* __restrict__ y, long n, int vec) {
  const float sc = *s;
  const long base = (long)blockIdx.x * kRzChunk;
  if (vec && base + kRzChunk <= n) {  // whole chunk: every load issued before the first store
    float v[kRzSteps][8];
#pragma unroll
    for (int st = 0; st < kRzSteps; ++st) ld8<ZT>(z + base + ((long)st * kRzThreads + threadIdx.x) * kRzVec, v[st]);
#pragma unroll
    for (int st = 0; st < kRzSteps; ++st) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[st][e] *= sc;
      st8<YT>(y + base + ((long)st * kRzThreads + threadIdx.x) * kRzVec, v[st]);
    }
    return;
  }
  for (int st = 0; st < kRzSteps; ++st) {
    const long i = base + ((long)st * kRzThreads + threadIdx.x) * kRzVec;
    for (int e = 0; e < kRzVec; ++e)
      if (i + e < n) st1<YT>(y + i + e, sc * ld1<ZT>(z + i + e));
  }
}

template <typename ZT, typename DT>
__global__ __launch_bounds__(kRzThreads) void rezero_bwd_kernel(const DT* __restrict__ dy, const ZT* __restrict__ z,
                                                                const float* __restrict__ s, ZT* __restrict__ dz,
                                                                float* __restrict__ part, long n, int vec) {
  __shared__ float red[kRzThreads];
  const float sc = *s;
  const long base = (long)blockIdx.x * kRzChunk;
  float acc = 0.f;
  if (vec && base + kRzChunk <= n) {  // whole chunk: every load issued before the first store
    float g[kRzSteps][8], v[kRzSteps][8];
#pragma unroll
    for (int st = 0; st < kRzSteps; ++st) {
      const long i = base + ((long)st * kRzThreads + threadIdx.x) * kRzVec;
      ld8<DT>(dy + i, g[st]);
      ld8<ZT>(z + i, v[st]);
    }
#pragma unroll
    for (int st = 0; st < kRzSteps; ++st) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc = fmaf(g[st][e], v[st][e], acc);
        g[st][e] *= sc;
      }
      if (dz) st8<ZT>(dz + base + ((long)st * kRzThreads + threadIdx.x) * kRzVec, g[st]);
    }
  } else {
    for (int st = 0; st < kRzSteps; ++st) {
      const long i = base + ((long)st * kRzThreads + threadIdx.x) * kRzVec;
      for (int e = 0; e < kRzVec; ++e)
        if (i + e < n) {
          const float g = ld1<DT>(dy + i + e);
          acc = fmaf(g, ld1<ZT>(z + i + e), acc);
          if (dz) st1<ZT>(dz + i + e, sc * g);
        }
    }
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = kRzThreads / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

// ds = sum of the partials: thread t adds partials t, t+256, ... in order,
// then a fixed tree over the 256 thread sums.
__global__ __launch_bounds__(kRzThreads) void rezero_reduce_kernel(const float* __restrict__ part, int nparts,
                                                                   float* __restrict__ ds) {
  __shared__ float red[kRzThreads];
  float acc = 0.f;
  int i = threadIdx.x;
  for (; i + 3 * kRzThreads < nparts; i += 4 * kRzThreads) {  // loads four at a time, adds in order
    float v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = part[i + u * kRzThreads];
#pragma unroll
    for (int u = 0; u < 4; ++u) acc += v[u];
  }
  for (; i < nparts; i += kRzThreads) acc += part[i];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = kRzThreads / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) *ds = red[0];
}

static int n_chunks(long n) { return (int)((n + kRzChunk - 1) / kRzChunk); }

size_t rezero_ws_bytes(long n) { return (size_t)(n_chunks(n) > 0 ? n_chunks(n) : 1) * sizeof(float); }

template <typename ZT, typename YT>
static void fwd_launch(const void* z, const float* s, void* y, long n, int vec, hipStream_t st) {
  NAYLIS_TIMED("rezero_fwd", st,
               hipLaunchKernelGGL((rezero_fwd_kernel<ZT, YT>), dim3(n_chunks(n)), dim3(kRzThreads), 0, st,
                                  (const ZT*)z, s, (YT*)y, n, vec));
}

hipError_t launch_rezero_scale(const void* z, bool z_bf16, const float* s, void* y, bool y_bf16, long n,
                               hipStream_t st) {
  if (n == 0) return hipSuccess;
  const int vec = ((uintptr_t)z & 15) == 0 && ((uintptr_t)y & 15) == 0;
  if (z_bf16 && y_bf16)
    fwd_launch<bf16_t, bf16_t>(z, s, y, n, vec, st);
  else if (z_bf16)
    fwd_launch<bf16_t, float>(z, s, y, n, vec, st);
  else if (y_bf16)
    fwd_launch<float, bf16_t>(z, s, y, n, vec, st);
  else
    fwd_launch<float, float>(z, s, y, n, vec, st);
  return hipGetLastError();
}

hipError_t launch_rezero_fwd(const void* z, bool z_bf16, const float* s, float* y, long n, hipStream_t st) {
  return launch_rezero_scale(z, z_bf16, s, y, false, n, st);
}

template <typename ZT, typename DT>
static void bwd_launch(const void* dy, const void* z, const float* s, void* dz, float* part, long n, int vec,
                       hipStream_t st) {
  NAYLIS_TIMED("rezero_bwd", st,
               hipLaunchKernelGGL((rezero_bwd_kernel<ZT, DT>), dim3(n_chunks(n)), dim3(kRzThreads), 0, st,
                                  (const DT*)dy, (const ZT*)z, s, (ZT*)dz, part, n, vec));
}

hipError_t launch_rezero_reduce(const float* part, int nparts, float* ds, hipStream_t st) {
  NAYLIS_TIMED("rezero_bwd", st,
               hipLaunchKernelGGL(rezero_reduce_kernel, dim3(1), dim3(kRzThreads), 0, st, part, nparts, ds));
  return hipGetLastError();
}

hipError_t launch_rezero_bwd(const void* dy, bool dy_bf16, const void* z, bool z_bf16, const float* s, void* dz,
                             float* ds, void* ws, long n, hipStream_t st) {
  float* part = (float*)ws;
  if (n > 0) {
    const int vec = ((uintptr_t)dy & 15) == 0 && ((uintptr_t)z & 15) == 0 && ((uintptr_t)dz & 15) == 0;
    if (z_bf16 && dy_bf16)
      bwd_launch<bf16_t, bf16_t>(dy, z, s, dz, part, n, vec, st);
    else if (z_bf16)
      bwd_launch<bf16_t, float>(dy, z, s, dz, part, n, vec, st);
    else if (dy_bf16)
      bwd_launch<float, bf16_t>(dy, z, s, dz, part, n, vec, st);
    else
      bwd_launch<float, float>(dy, z, s, dz, part, n, vec, st);
  }
  NAYLIS_TIMED("rezero_bwd", st,
               hipLaunchKernelGGL(rezero_reduce_kernel, dim3(1), dim3(kRzThreads), 0, st, part, n > 0 ? n_chunks(n) : 0,
                                  ds));
  return hipGetLastError();
}

}  // namespace naylis
