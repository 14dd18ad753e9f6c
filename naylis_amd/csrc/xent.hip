// Next-token cross-entropy of the decoder's LM head, fused: the reference
// computes F.cross_entropy(shift_logits.float(), labels, reduction="sum")
// (model.py:536-545): an fp32 copy of the (N, V) logits, log_softmax and the
// label pick forward, and as many full passes backward.  Here the forward
// reads the bf16 logits once per row (max, sum of exp, the label's logit) and
// writes the row's loss and log-sum-exp; the backward reads them once more and
// writes the bf16 gradient (softmax - one_hot) * g_row.  Rows whose label is
// ignore_index have loss 0 and gradient 0.
#include "common.h"
#include "timing.h"

namespace naylis {

namespace {

// workgroup-wide reduction over 4 waves: butterfly per wave, then the four
// wave results in order
template <typename F>
__device__ __forceinline__ float wg_reduce(float v, float* red, F op) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_allreduce_f32(v, op);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return op(op(red[0], red[1]), op(red[2], red[3]));
}

}  // namespace

// one workgroup per row; V a multiple of 2048 (8 values per thread per pass)
__global__ __launch_bounds__(256) void xent_fwd_kernel(const bf16_t* __restrict__ logits,
                                                       const int64_t* __restrict__ labels, float* __restrict__ loss,
                                                       float* __restrict__ lse_out, int V, long ignore_index) {
  __shared__ float red[4];
  const long row = blockIdx.x;
  const bf16_t* x = logits + row * (long)V;
  const long lab = labels[row];
  float mx = -INFINITY;
  for (int j = threadIdx.x * 8; j < V; j += 2048) {
    const uint4 u = *reinterpret_cast<const uint4*>(x + j);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      mx = fmaxf(mx, fmaxf(__uint_as_float(w[i] << 16), __uint_as_float(w[i] & 0xffff0000u)));
  }
  mx = wg_reduce(mx, red, [](float a, float b) { return fmaxf(a, b); });
  float s = 0.f;
  for (int j = threadIdx.x * 8; j < V; j += 2048) {
    const uint4 u = *reinterpret_cast<const uint4*>(x + j);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      s += expf(__uint_as_float(w[i] << 16) - mx) + expf(__uint_as_float(w[i] & 0xffff0000u) - mx);
  }
  s = wg_reduce(s, red, [](float a, float b) { return a + b; });
  if (threadIdx.x == 0) {
    const float lse = mx + logf(s);
    // a label that is neither ignore_index nor a class gives a NaN loss (the
    // reference's F.cross_entropy raises on it): bad data cannot pass silently
    const bool in_range = lab >= 0 && lab < V;
    loss[row] = lab == ignore_index ? 0.f : in_range ? lse - bf16_to_f32(x[in_range ? lab : 0]) : __builtin_nanf("");
    lse_out[row] = lse;
  }
}

// d logits[r, j] = (exp(x - lse) - [j == label]) * g[r * g_stride]
__global__ __launch_bounds__(256) void xent_bwd_kernel(const bf16_t* __restrict__ logits,
                                                       const int64_t* __restrict__ labels,
                                                       const float* __restrict__ lse, const float* __restrict__ g,
                                                       long g_stride, bf16_t* __restrict__ dlogits, int V,
                                                       long ignore_index) {
  const long row = blockIdx.x;
  const bf16_t* x = logits + row * (long)V;
  bf16_t* dx = dlogits + row * (long)V;
  const long lab = labels[row];
  // ignore_index rows get a zero gradient, out-of-range labels a NaN one
  const float gr = lab == ignore_index ? 0.f : (lab >= 0 && lab < V) ? g[row * g_stride] : __builtin_nanf("");
  const float l = lse[row];
  for (int j = threadIdx.x * 8; j < V; j += 2048) {
    const uint4 u = *reinterpret_cast<const uint4*>(x + j);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = __uint_as_float(w[i] << 16), b = __uint_as_float(w[i] & 0xffff0000u);
      const float pa = expf(a - l) - (j + 2 * i == lab ? 1.f : 0.f);
      const float pb = expf(b - l) - (j + 2 * i + 1 == lab ? 1.f : 0.f);
      r[2 * i] = (__bf16)(pa * gr);
      r[2 * i + 1] = (__bf16)(pb * gr);
    }
    *reinterpret_cast<bf16x8*>(dx + j) = r;
  }
}

hipError_t launch_xent(const void* logits, const int64_t* labels, float* loss, float* lse, const float* g,
                       long g_stride, void* dlogits, bool bwd, long N, int V, long ignore_index, hipStream_t st) {
  if (N == 0) return hipSuccess;
  if (!bwd)
    NAYLIS_TIMED("xent_fwd", st, hipLaunchKernelGGL(xent_fwd_kernel, dim3((unsigned)N), dim3(256), 0, st,
                                                    (const bf16_t*)logits, labels, loss, lse, V, ignore_index));
  else
    NAYLIS_TIMED("xent_bwd", st, hipLaunchKernelGGL(xent_bwd_kernel, dim3((unsigned)N), dim3(256), 0, st,
                                                    (const bf16_t*)logits, labels, lse, g, g_stride,
                                                    (bf16_t*)dlogits, V, ignore_index));
  return hipGetLastError();
}

}  // namespace naylis
