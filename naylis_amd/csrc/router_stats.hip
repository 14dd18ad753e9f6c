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
// 256-token workgroup writes fp64 partials (column sums of p, selection
// counts, entropy sum), one workgroup sums them in workgroup order.
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
  constexpr int P = EMAX + 1;
  __shared__ float p_lds[kStatsTok * P];
  __shared__ unsigned long long m_lds[kStatsTok];
  __shared__ float h_lds[kStatsTok];
  const int tid = threadIdx.x;
  const long tok = (long)blockIdx.x * kStatsTok + tid;
  float ent = 0.f;
  unsigned long long mask = 0;
  if (tok < N) {
    // entropy term by term in block order, as the reference's fp32 sum over the last axis
    for (int e = 0; e < E; ++e) {
      const float p = probs[tok * E + e];
      p_lds[tid * P + e] = p;
      ent -= __fmul_rn(p, logf(fmaxf(p, 1e-9f)));
    }
    for (int t = 0; t < topk; ++t) {
      const int i = top_idx[tok * topk + t];
      if (i >= 0 && i < E) mask |= 1ull << i;
    }
  } else {
    for (int e = 0; e < E; ++e) p_lds[tid * P + e] = 0.f;
  }
  m_lds[tid] = mask;
  h_lds[tid] = ent;
  __syncthreads();
  const int nv = 2 * E + 1;
  double* out = part + (long)blockIdx.x * nv;
  if (tid < E) {
    double s = 0.0;
    for (int i = 0; i < kStatsTok; ++i) s += (double)p_lds[i * P + tid];
    out[tid] = s;
  } else if (tid >= 64 && tid - 64 < E) {
    const int e = tid - 64;
    double c = 0.0;
    for (int i = 0; i < kStatsTok; ++i) c += (double)((m_lds[i] >> e) & 1ull);
    out[E + e] = c;
  } else if (tid == 128) {
    double s = 0.0;
    for (int i = 0; i < kStatsTok; ++i) s += (double)h_lds[i];
    out[2 * E] = s;
  }
}

__global__ __launch_bounds__(256) void router_stats_final_kernel(const double* __restrict__ part,
                                                                 float* __restrict__ stats, int nparts, long N,
                                                                 int E) {
  __shared__ double tot[2 * 64 + 1];
  const int tid = threadIdx.x;
  const int nv = 2 * E + 1;
  if (tid < nv) {
    double s = 0.0;
    for (int w = 0; w < nparts; ++w) s += part[(long)w * nv + tid];
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
      aux = __fadd_rn(aux, __fmul_rn((float)(tot[E + e] * inv), (float)(tot[e] * inv)));
      dead += tot[E + e] == 0.0;
    }
    stats[2 * E] = __fmul_rn((float)E, aux);
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
