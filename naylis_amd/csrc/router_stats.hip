// Load-balance statistics of one MoM layer's routing, model.py:476-517
// (`_collect_mom_aux_loss`): per block e the mean router probability over the
// N tokens and the fraction of tokens whose top-k contains e, the layer's aux
// term E * sum_e frac_e * mean_prob_e, the mean token entropy
// -sum_e p log(max(p, 1e-9)) and the fraction of blocks no token selects.
// The reference builds these from (N, E) / (N, k, E) intermediates in about a
// dozen elementwise and reduction launches per layer; here one pass reads
// probs and top_idx once.
//
// Layout: stats[0, E) mean_prob, [E, 2E) frac, [2E] aux, [2E+1] entropy,
// [2E+2] dead fraction.  Two launches with a fixed-order reduction: each
// 256-token workgroup reduces its tokens per wave (butterfly sums of p and of
// the entropy, ballot counts of the selections) and writes fp64 partials
// (the four waves in order); one workgroup sums the partials in workgroup
// order.
#include "common.h"
#include "launch_router.h"
#include "timing.h"

namespace naylis {

constexpr int kStatsTok = 256;

template <int EMAX>
__global__ __launch_bounds__(256) void router_stats_partial_kernel(const float* __restrict__ probs,
                                                                   const int32_t* __restrict__ top_idx,
                                                                   double* __restrict__ part, long N, int E,
                                                                   int topk) {
  __shared__ float wsum[4][EMAX];
  __shared__ int wcnt[4][EMAX];
  __shared__ float went[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long tok = (long)blockIdx.x * kStatsTok + tid;
  const bool ok = tok < N;
  // this token's probabilities (all loads issued before use)
  float p[EMAX];
  if (E % 4 == 0 && (((uintptr_t)probs) & 15) == 0) {
#pragma unroll
    for (int e = 0; e < EMAX; e += 4) {
      const f32x4 v = (ok && e < E) ? *reinterpret_cast<const f32x4*>(probs + tok * E + e) : f32x4{};
      p[e] = v[0];
      p[e + 1] = v[1];
      p[e + 2] = v[2];
      p[e + 3] = v[3];
    }
  } else {
#pragma unroll
    for (int e = 0; e < EMAX; ++e) p[e] = (ok && e < E) ? probs[tok * E + e] : 0.f;
  }
  unsigned long long mask = 0;
  if (ok)
    for (int t = 0; t < topk; ++t) {
      const int i = top_idx[tok * topk + t];
      if (i >= 0 && i < E) mask |= 1ull << i;
    }
  // entropy term by term in block order, as the reference's fp32 sum over the last axis
  float ent = 0.f;
#pragma unroll
  for (int e = 0; e < EMAX; ++e)
    if (e < E) ent -= mul_rn(p[e], logf(fmaxf(p[e], 1e-9f)));
  if (!ok) ent = 0.f;
  // per wave: column sums (butterfly), selection counts (ballot), entropy sum
#pragma unroll
  for (int e = 0; e < EMAX; ++e) {
    if (e < E) {
      const float s = wave_allsum(p[e]);
      const int c = __popcll(__ballot((mask >> e) & 1ull));
      if (lane == 0) {
        wsum[wave][e] = s;
        wcnt[wave][e] = c;
      }
    }
  }
  const float es = wave_allsum(ent);
  if (lane == 0) went[wave] = es;
  __syncthreads();
  // the workgroup's partials: the four waves in order, in fp64
  const int nv = 2 * E + 1;
  double* out = part + (long)blockIdx.x * nv;
  if (tid < E) {
    out[tid] = (double)wsum[0][tid] + (double)wsum[1][tid] + (double)wsum[2][tid] + (double)wsum[3][tid];
  } else if (tid >= 64 && tid - 64 < E) {
    const int e = tid - 64;
    out[E + e] = (double)(wcnt[0][e] + wcnt[1][e] + wcnt[2][e] + wcnt[3][e]);
  } else if (tid == 128) {
    out[2 * E] = (double)went[0] + (double)went[1] + (double)went[2] + (double)went[3];
  }
}

__global__ __launch_bounds__(256) void router_stats_final_kernel(const double* __restrict__ part,
                                                                 float* __restrict__ stats, int nparts, long N,
                                                                 int E) {
  __shared__ double tot[2 * 64 + 1];
  const int tid = threadIdx.x;
  const int nv = 2 * E + 1;
  if (tid < nv) {
    // partials in workgroup order, 16 loads in flight at a time
    double s = 0.0;
    for (int w0 = 0; w0 < nparts; w0 += 16) {
      double v[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = w0 + i < nparts ? part[(long)(w0 + i) * nv + tid] : 0.0;
#pragma unroll
      for (int i = 0; i < 16; ++i) s += v[i];
    }
    tot[tid] = s;
  }
  __syncthreads();
  const double inv = 1.0 / (double)N;
  if (tid < E) {
    stats[tid] = (float)(tot[tid] * inv);
    stats[E + tid] = (float)(tot[E + tid] * inv);
  }
  if (tid == 0) {
    // aux = E * sum_e frac_e * mean_prob_e over the fp32-rounded means, in block order
    float aux = 0.f;
    int dead = 0;
    for (int e = 0; e < E; ++e) {
      aux = add_rn(aux, mul_rn((float)(tot[E + e] * inv), (float)(tot[e] * inv)));
      dead += tot[E + e] == 0.0;
    }
    stats[2 * E] = mul_rn((float)E, aux);
    stats[2 * E + 1] = (float)(tot[2 * E] * inv);
    stats[2 * E + 2] = (float)dead / (float)E;
  }
}

size_t router_stats_ws_bytes(long N, int E) {
  const long nparts = (N + kStatsTok - 1) / kStatsTok;
  return (size_t)(nparts > 0 ? nparts : 1) * (2 * E + 1) * sizeof(double);
}

hipError_t launch_router_stats(const float* probs, const int32_t* top_idx, float* stats, void* ws, long N, int E,
                               int topk, hipStream_t st) {
  const int nparts = (int)((N + kStatsTok - 1) / kStatsTok);
  double* part = (double*)ws;
  if (nparts > 0) {
    if (E <= 8)
      NAYLIS_TIMED("router_stats", st,
                   hipLaunchKernelGGL(router_stats_partial_kernel<8>, dim3(nparts), dim3(256), 0, st, probs, top_idx,
                                      part, N, E, topk));
    else
      NAYLIS_TIMED("router_stats", st,
                   hipLaunchKernelGGL(router_stats_partial_kernel<64>, dim3(nparts), dim3(256), 0, st, probs, top_idx,
                                      part, N, E, topk));
  }
  NAYLIS_TIMED("router_stats_final", st,
               hipLaunchKernelGGL(router_stats_final_kernel, dim3(1), dim3(256), 0, st, part, stats, nparts, N, E));
  return hipGetLastError();
}

}  // namespace naylis
