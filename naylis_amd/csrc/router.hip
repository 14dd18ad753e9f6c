// Fused causal prefix-mean router of the MoM layer (gfx950), forward and
// backward.
//
// Forward (model.py:169-220, mom_kernels/reference.py:32-36,75-84):
//   h_t      = fp32( sum_{s<=t} x_s ) / fp32(t+1)        (prefix mean, fp32)
//   z        = h W_down^T      a = tanh(z)      logits = a W_up^T
//   probs    = softmax(logits)
//   (vals, idx) = topk(logits + noise_scale * noise, k)  (sorted descending)
//   gates    = softmax(vals)
// The prefix sum accumulates in fp64 and is rounded to fp32 once per prefix,
// which is exactly what the CPU reference's torch.cumsum produces for fp32
// input; the divide is IEEE fp32 (correctly rounded), so h is bit-exact.
//
// Launch plan: (1) per 32-token chunk fp64 column sums, (2) exclusive carry
// over chunks, (3) one workgroup per (b, chunk): scan its 32 tokens column by
// column from the carry, stage h in LDS slab by slab (256 features), and
// accumulate the rank-R projection z; then tanh, W_up, softmax, top-k.
//
// Backward: with w_t = dz_t / (t+1) and W~_t = sum_{s>=t} w_s (reverse scan of
// an R-wide array), the two D-wide gradients are plain products
//   dx = W~ W_down          dW_down = W~^T x
// (d h_s = dz_s W_down and dx_t = sum_{s>=t} dh_s / (s+1), so both the
// reverse scan and the recomputation of h fold into W~).
#include "launch_router.h"
#include "common.h"
#include "timing.h"

namespace naylis {

constexpr int kRouterChunk = 32;  // tokens per scan chunk / workgroup
constexpr int kRouterSlab = 256;  // features per LDS slab (one per thread)

template <typename XT>
__device__ __forceinline__ double load_x64(const XT* p);
template <>
__device__ __forceinline__ double load_x64<float>(const float* p) { return (double)*p; }
template <>
__device__ __forceinline__ double load_x64<bf16_t>(const bf16_t* p) { return (double)bf16_to_f32(*p); }

template <typename XT>
__device__ __forceinline__ float load_x32(const XT* p);
template <>
__device__ __forceinline__ float load_x32<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_x32<bf16_t>(const bf16_t* p) { return bf16_to_f32(*p); }

// (1) chunk column sums, fp64: csum[b][c][d] (exact for bf16 input).
// Thread = 8 consecutive features (one 16-byte load of bf16, two of fp32).
template <typename XT>
__global__ __launch_bounds__(256) void router_chunk_sums_kernel(const XT* __restrict__ x, double* __restrict__ csum,
                                                                int T, int D, int n_chunks) {
  const int d = (blockIdx.x * 256 + threadIdx.x) * 8;
  const int c = blockIdx.y;
  const int b = blockIdx.z;
  if (d >= D) return;
  const int t0 = c * kRouterChunk, t1 = min(T, t0 + kRouterChunk);
  double s[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) s[e] = 0.0;
  const bool full = d + 8 <= D;
  for (int t = t0; t < t1; ++t) {
    const XT* p = x + ((long)b * T + t) * D + d;
    if (full) {
      if constexpr (sizeof(XT) == 2) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        const bf16_t* e8 = reinterpret_cast<const bf16_t*>(&v);
#pragma unroll
        for (int e = 0; e < 8; ++e) s[e] += (double)bf16_to_f32(e8[e]);
      } else {
        const f32x4 v0 = *reinterpret_cast<const f32x4*>(p);
        const f32x4 v1 = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s[e] += (double)v0[e];
          s[4 + e] += (double)v1[e];
        }
      }
    } else {
      for (int e = 0; e < 8; ++e)
        if (d + e < D) s[e] += load_x64<XT>(p + e);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (d + e < D) csum[((long)b * n_chunks + c) * D + d + e] = s[e];
}

// (2) exclusive carry over chunks, in place: carry[b][c][d] = sum_{c'<c} csum,
// added in ascending chunk order.  Loads go out 16 at a time so their
// latencies overlap.
__global__ __launch_bounds__(256) void router_chunk_carry_kernel(double* __restrict__ csum, int D, int n_chunks) {
  const int d = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (d >= D) return;
  double run = 0.0;
  for (int c0 = 0; c0 < n_chunks; c0 += 16) {
    double v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = c0 + i < n_chunks ? csum[((long)b * n_chunks + c0 + i) * D + d] : 0.0;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (c0 + i < n_chunks) {
        csum[((long)b * n_chunks + c0 + i) * D + d] = run;
        run += v[i];
      }
  }
}

// (3) main router kernel, one workgroup per (b, kRouterChunk-token chunk).
// For each 256-feature slab: thread f scans its feature over the chunk from
// the fp64 carry and writes h[t][f] to LDS; the 4 waves then each take 64 of
// the slab's features and accumulate z = h W_down^T with fp32 MFMA
// (v_mfma_f32_32x32x2f32: lane l holds A[l%32][l/32] and B[l/32][l%32]).
// The 4 per-wave partial z tiles are summed in LDS in a fixed order.
template <typename XT, int EMAX, int TK>
__global__ __launch_bounds__(256) void router_fwd_kernel(
    const XT* __restrict__ x, const double* __restrict__ carry, const float* __restrict__ w_down,
    const float* __restrict__ w_up, const float* __restrict__ noise, float noise_scale, float* __restrict__ logits,
    float* __restrict__ probs, int32_t* __restrict__ top_idx, float* __restrict__ top_gates,
    float* __restrict__ act, float* __restrict__ h_out, int T, int D, int R, int E, int topk, int n_chunks) {
  constexpr int CT = kRouterChunk;   // 32 tokens: one MFMA row tile
  constexpr int HP = kRouterSlab + 1;
  __shared__ float h_lds[CT * HP];                 // [token][feature] of the slab
  __shared__ float wz_lds[kRouterSlab * 33];       // W_down slab [feature][rank]; then the wave partials of z
  __shared__ float a_lds[CT * 65];                 // tanh activations [token][rank], R <= 64
  __shared__ float wu_lds[EMAX * 65];              // W_up [block][rank]
  float* wd_lds = wz_lds;
  float (*z_lds)[CT * 33] = reinterpret_cast<float (*)[CT * 33]>(wz_lds);
  static_assert(4 * CT * 33 <= kRouterSlab * 33, "z partials must fit in the W_down slab buffer");

  const int c = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t0 = c * CT;
  const int nt = min(CT, T - t0);
  for (int i = tid; i < E * R; i += 256) wu_lds[(i / R) * 65 + i % R] = w_up[i];

  for (int r0 = 0; r0 < R; r0 += 32) {
    f32x16 acc = f32x16{};
    for (int d0 = 0; d0 < D; d0 += kRouterSlab) {
      const int d = d0 + tid;
      __syncthreads();
      // ---- scan this thread's feature over the chunk (fp64, rounded once)
      if (d < D) {
        double run = carry[((long)b * n_chunks + c) * D + d];
        const XT* xp = x + ((long)b * T + t0) * D + d;
        float xv[CT];
#pragma unroll
        for (int t = 0; t < CT; ++t) xv[t] = t < nt ? load_x32<XT>(xp + (long)t * D) : 0.f;
#pragma unroll
        for (int t = 0; t < CT; ++t) {
          float hv = 0.f;
          if (t < nt) {
            run += (double)xv[t];
            const float cs = (float)run;
            hv = cs / (float)(t0 + t + 1);
            if (h_out != nullptr && r0 == 0) h_out[((long)b * T + t0 + t) * D + d] = hv;
          }
          h_lds[t * HP + tid] = hv;
        }
      } else {
#pragma unroll
        for (int t = 0; t < CT; ++t) h_lds[t * HP + tid] = 0.f;
      }
      for (int i = tid; i < kRouterSlab * 32; i += 256) {
        const int r = i / kRouterSlab, f = i % kRouterSlab;  // consecutive threads: consecutive features
        wd_lds[f * 33 + r] = (d0 + f < D && r0 + r < R) ? w_down[(long)(r0 + r) * D + d0 + f] : 0.f;
      }
      __syncthreads();
      // ---- z[t][r] += sum_f h[t][f] Wd[r][f] over this wave's 64 features
      const int fw = wave * 64;
#pragma unroll 8
      for (int k = 0; k < 64; k += 2) {
        const int f = fw + k + (lane >> 5);
        const float av = h_lds[(lane & 31) * HP + f];
        const float bv = wd_lds[f * 33 + (lane & 31)];
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc, 0, 0, 0);
      }
    }
    // ---- sum the 4 wave partials in a fixed order, tanh, stash
    __syncthreads();  // every wave is done reading the W_down slab
#pragma unroll
    for (int v = 0; v < 16; ++v) z_lds[wave][acc_row(lane >> 5, v) * 33 + (lane & 31)] = acc[v];
    __syncthreads();
    for (int i = tid; i < CT * 32; i += 256) {
      const int t = i >> 5, r = i & 31;
      const float z = ((z_lds[0][t * 33 + r] + z_lds[1][t * 33 + r]) + z_lds[2][t * 33 + r]) + z_lds[3][t * 33 + r];
      if (t < nt && r0 + r < R) {
        const float a = tanhf(z);
        act[((long)b * T + t0 + t) * R + r0 + r] = a;
        a_lds[t * 65 + r0 + r] = a;
      }
    }
  }
  __syncthreads();
  // ---- per token: logits, probs, top-k, gates
  if (tid < nt) {
    const long tok = (long)b * T + t0 + tid;
    float lg[EMAX];
#pragma unroll
    for (int e = 0; e < EMAX; ++e) lg[e] = 0.f;
    for (int r = 0; r < R; ++r) {
      const float a = a_lds[tid * 65 + r];
#pragma unroll
      for (int e = 0; e < EMAX; ++e)
        if (e < E) lg[e] = fmaf(a, wu_lds[e * 65 + r], lg[e]);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < EMAX; ++e)
      if (e < E) {
        logits[tok * E + e] = lg[e];
        mx = fmaxf(mx, lg[e]);
      }
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < EMAX; ++e)
      if (e < E) sum += expf(lg[e] - mx);
#pragma unroll
    for (int e = 0; e < EMAX; ++e)
      if (e < E) probs[tok * E + e] = expf(lg[e] - mx) / sum;
    // top-k of the (optionally perturbed) logits; ties -> lowest block id
    float nz[EMAX];
#pragma unroll
    for (int e = 0; e < EMAX; ++e) nz[e] = (e < E) ? (noise ? fmaf(noise_scale, noise[tok * E + e], lg[e]) : lg[e]) : -INFINITY;
    int sel[TK];
    float val[TK];
#pragma unroll
    for (int t = 0; t < TK; ++t) {
      sel[t] = 0;
      val[t] = 0.f;
      if (t < topk) {
        int best = -1;
        float bv = -INFINITY;
#pragma unroll
        for (int e = 0; e < EMAX; ++e) {
          bool taken = false;
#pragma unroll
          for (int u = 0; u < TK; ++u)
            if (u < t && sel[u] == e) taken = true;
          if (e < E && !taken && (best < 0 || nz[e] > bv)) {
            best = e;
            bv = nz[e];
          }
        }
        sel[t] = best;
        val[t] = bv;
      }
    }
    float gs = 0.f;
#pragma unroll
    for (int t = 0; t < TK; ++t)
      if (t < topk) gs += expf(val[t] - val[0]);
#pragma unroll
    for (int t = 0; t < TK; ++t)
      if (t < topk) {
        top_idx[tok * topk + t] = sel[t];
        top_gates[tok * topk + t] = expf(val[t] - val[0]) / gs;
      }
  }
}

// ---------------------------------------------------------------------------
// Backward (1): per token, d(gates) / d(probs) / d(logits) -> w = dz / (t+1);
// per-workgroup partial of dW_up = dlogits^T a.
template <int EMAX, int TK>
__global__ __launch_bounds__(64) void router_bwd_token_kernel(
    const float* __restrict__ act, const float* __restrict__ probs, const int32_t* __restrict__ top_idx,
    const float* __restrict__ top_gates, const float* __restrict__ d_gates, const float* __restrict__ d_probs,
    const float* __restrict__ d_logits, const float* __restrict__ w_up, float* __restrict__ w_out,
    float* __restrict__ dwup_part, int T, int R, int E, int topk, long ntok) {
  __shared__ float dl_lds[64 * (EMAX + 1)];
  __shared__ float a_lds[64 * 65];
  __shared__ float wu_lds[EMAX * 65];
  const long tok = (long)blockIdx.x * 64 + threadIdx.x;
  const bool ok = tok < ntok;
  for (int i = threadIdx.x; i < E * R; i += 64) wu_lds[(i / R) * 65 + i % R] = w_up[i];
  for (int i = threadIdx.x; i < 64 * R; i += 64) {
    const long tk = (long)blockIdx.x * 64 + i / R;
    a_lds[(i / R) * 65 + i % R] = tk < ntok ? act[tk * R + i % R] : 0.f;
  }
  __syncthreads();
  float dl[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; ++e) dl[e] = 0.f;
  if (ok) {
    if (d_logits) {
#pragma unroll
      for (int e = 0; e < EMAX; ++e)
        if (e < E) dl[e] = d_logits[tok * E + e];
    }
    if (d_probs) {
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < EMAX; ++e)
        if (e < E) dot = fmaf(probs[tok * E + e], d_probs[tok * E + e], dot);
#pragma unroll
      for (int e = 0; e < EMAX; ++e)
        if (e < E) dl[e] = fmaf(probs[tok * E + e], d_probs[tok * E + e] - dot, dl[e]);
    }
    if (d_gates) {
      float gdot = 0.f;
#pragma unroll
      for (int t = 0; t < TK; ++t)
        if (t < topk) gdot = fmaf(top_gates[tok * topk + t], d_gates[tok * topk + t], gdot);
#pragma unroll
      for (int t = 0; t < TK; ++t)
        if (t < topk) {
          const float dv = top_gates[tok * topk + t] * (d_gates[tok * topk + t] - gdot);
          const int e = top_idx[tok * topk + t];
#pragma unroll
          for (int u = 0; u < EMAX; ++u)
            if (u == e) dl[u] += dv;
        }
    }
  }
  const float denom = ok ? (float)((tok % T) + 1) : 1.f;
  for (int r = 0; r < R; ++r) {
    float da = 0.f;
#pragma unroll
    for (int e = 0; e < EMAX; ++e)
      if (e < E) da = fmaf(dl[e], wu_lds[e * 65 + r], da);
    const float a = a_lds[threadIdx.x * 65 + r];
    if (ok) w_out[tok * R + r] = da * (1.f - a * a) / denom;
  }
#pragma unroll
  for (int e = 0; e < EMAX; ++e) dl_lds[threadIdx.x * (EMAX + 1) + e] = ok ? dl[e] : 0.f;
  __syncthreads();
  // partial dW_up[e][r] over this block's 64 tokens
  for (int i = threadIdx.x; i < E * R; i += 64) {
    const int e = i / R, r = i % R;
    float s = 0.f;
    for (int j = 0; j < 64; ++j) s = fmaf(dl_lds[j * (EMAX + 1) + e], a_lds[j * 65 + r], s);
    dwup_part[(long)blockIdx.x * E * R + i] = s;
  }
}

// Backward (2): reverse inclusive scan over t of w (per b, r) with fp64
// accumulation, in two passes over 64-token chunks: (2a) chunk sums,
// (2b) suffix carry of the later chunks + in-chunk reverse scan.
constexpr int kScanChunk = 64;

__global__ __launch_bounds__(256) void router_bwd_chunk_sums_kernel(const float* __restrict__ w,
                                                                    double* __restrict__ csum, int T, int R,
                                                                    int n_chunks) {
  // 256 threads = 32 ranks x 8 token groups of 8
  __shared__ double part[8][33];
  const int b = blockIdx.y, c = blockIdx.x, r0 = blockIdx.z * 32;
  const int r = threadIdx.x & 31, grp = threadIdx.x >> 5;
  const int rr = r0 + r;
  double s = 0.0;
  if (rr < R)
    for (int i = 0; i < 8; ++i) {
      const int t = c * kScanChunk + grp * 8 + i;
      if (t < T) s += (double)w[((long)b * T + t) * R + rr];
    }
  part[grp][r] = s;
  __syncthreads();
  if (grp == 0 && rr < R) {
    double tot = 0.0;
    for (int j = 0; j < 8; ++j) tot += part[j][r];
    csum[((long)b * n_chunks + c) * R + rr] = tot;
  }
}

__global__ __launch_bounds__(256) void router_bwd_scan_kernel(const float* __restrict__ w,
                                                              const double* __restrict__ csum,
                                                              float* __restrict__ wt, int T, int R, int n_chunks) {
  // 256 threads = 32 ranks x 8 token groups of 8; groups scanned in reverse
  __shared__ double part[8][33];
  const int b = blockIdx.y, c = blockIdx.x, r0 = blockIdx.z * 32;
  const int r = threadIdx.x & 31, grp = threadIdx.x >> 5;
  const int rr = r0 + r;
  double s = 0.0;
  if (rr < R)
    for (int i = 0; i < 8; ++i) {
      const int t = c * kScanChunk + grp * 8 + i;
      if (t < T) s += (double)w[((long)b * T + t) * R + rr];
    }
  part[grp][r] = s;
  __syncthreads();
  if (rr >= R) return;
  double carry = 0.0;
  for (int cc = c + 1; cc < n_chunks; ++cc) carry += csum[((long)b * n_chunks + cc) * R + rr];
  for (int j = grp + 1; j < 8; ++j) carry += part[j][r];
  for (int i = 7; i >= 0; --i) {
    const int t = c * kScanChunk + grp * 8 + i;
    if (t < T) {
      carry += (double)w[((long)b * T + t) * R + rr];
      wt[((long)b * T + t) * R + rr] = (float)carry;
    }
  }
}

// Backward (3): dx = W~ W_down and per-chunk partials of dW_down = W~^T x.
// One workgroup per (kDxChunk-token chunk, 256-feature slab); thread = feature,
// W_down column and the dW_down partial column live in registers.
constexpr int kDxChunk = 128;

template <typename XT, int RMAX>
__global__ __launch_bounds__(256) void router_bwd_dx_kernel(const XT* __restrict__ x, const float* __restrict__ wt,
                                                            const float* __restrict__ w_down, XT* __restrict__ dx,
                                                            float* __restrict__ dwd_part, int D, int R, long ntok) {
  constexpr int CT = kDxChunk;
  __shared__ float wt_lds[CT * RMAX];
  const long tok0 = (long)blockIdx.x * CT;
  const int d = blockIdx.y * 256 + threadIdx.x;
  const bool dok = d < D;
  for (int i = threadIdx.x; i < CT * RMAX; i += 256) {
    const int t = i / RMAX, r = i % RMAX;
    const long tk = tok0 + t;
    wt_lds[i] = (tk < ntok && r < R) ? wt[tk * R + r] : 0.f;
  }
  __syncthreads();
  float wd[RMAX], acc[RMAX];
#pragma unroll
  for (int r = 0; r < RMAX; ++r) {
    wd[r] = (dok && r < R) ? w_down[(long)r * D + d] : 0.f;
    acc[r] = 0.f;
  }
  const int nt = (int)(ntok - tok0 < CT ? ntok - tok0 : CT);
  for (int t8 = 0; t8 < nt; t8 += 8) {
    float xv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) xv[u] = (dok && t8 + u < nt) ? load_x32<XT>(x + (tok0 + t8 + u) * D + d) : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int t = t8 + u;
      if (t >= nt) break;
      const long tk = tok0 + t;
      float s = 0.f;
#pragma unroll
      for (int r = 0; r < RMAX; ++r) {
        const float w = wt_lds[t * RMAX + r];
        s = fmaf(w, wd[r], s);
        acc[r] = fmaf(w, xv[u], acc[r]);
      }
      if (dok) {
        if constexpr (sizeof(XT) == 2)
          dx[tk * D + d] = f32_to_bf16(s);
        else
          dx[tk * D + d] = s;
      }
    }
  }
  if (dok)
    for (int r = 0; r < R; ++r) dwd_part[((long)blockIdx.x * R + r) * D + d] = acc[r];
}

// Fixed-order reduction of per-chunk partials: out[i] = sum_c part[c][i].
// Block = 64 outputs x 4 interleaved partial groups; each group sums its
// partials in order, then the 4 group sums are added in a fixed order.
__global__ __launch_bounds__(256) void router_reduce_kernel(const float* __restrict__ part, float* __restrict__ out,
                                                            long n, int n_parts) {
  __shared__ float grp_sum[4][64];
  const int o = threadIdx.x & 63, gq = threadIdx.x >> 6;
  const long i = (long)blockIdx.x * 64 + o;
  float s = 0.f;
  if (i < n)
    for (int c = gq; c < n_parts; c += 4) s += part[(long)c * n + i];
  grp_sum[gq][o] = s;
  __syncthreads();
  if (gq == 0 && i < n) out[i] = ((grp_sum[0][o] + grp_sum[1][o]) + grp_sum[2][o]) + grp_sum[3][o];
}

// ---------------------------------------------------------------------------
RouterWs plan_router_ws(const RouterDims& d) {
  RouterWs w{};
  const long ntok = (long)d.B * d.T;
  const int n_chunks = (d.T + kRouterChunk - 1) / kRouterChunk;
  const long n_tok_blocks = (ntok + 63) / 64;
  auto a256 = [](size_t x) { return (x + 255) & ~(size_t)255; };
  size_t off = 0;
  w.carry = off;
  off += a256((size_t)d.B * n_chunks * d.D * 8);
  w.w = off;
  off += a256((size_t)ntok * d.R * 4);
  w.wt = off;
  off += a256((size_t)ntok * d.R * 4);
  w.scan_csum = off;
  off += a256((size_t)d.B * ((d.T + kScanChunk - 1) / kScanChunk) * d.R * 8);
  w.dwup_part = off;
  off += a256((size_t)n_tok_blocks * d.E * d.R * 4);
  w.dwd_part = off;
  off += a256((size_t)((ntok + kDxChunk - 1) / kDxChunk) * d.R * d.D * 4);
  w.total = off;
  w.fwd_total = w.w;
  return w;
}

template <typename XT, int EMAX, int TK>
static void fwd_launch(const void* x, const float* w_down, const float* w_up, const float* noise, float ns,
                       float* logits, float* probs, int32_t* idx, float* gates, float* act, float* h_out, char* ws,
                       const RouterWs& w, const RouterDims& d, hipStream_t st) {
  const int n_chunks = (d.T + kRouterChunk - 1) / kRouterChunk;
  double* carry = (double*)(ws + w.carry);
  const int dblk = (d.D + 2047) / 2048;
  NAYLIS_TIMED("router_chunk_sums", st, hipLaunchKernelGGL((router_chunk_sums_kernel<XT>), dim3(dblk, n_chunks, d.B), dim3(256), 0, st, (const XT*)x, carry,
                     d.T, d.D, n_chunks));

  NAYLIS_TIMED("router_chunk_carry", st,
               hipLaunchKernelGGL(router_chunk_carry_kernel, dim3((d.D + 255) / 256, d.B), dim3(256), 0, st, carry,
                                  d.D, n_chunks));
  NAYLIS_TIMED("router_fwd", st, hipLaunchKernelGGL((router_fwd_kernel<XT, EMAX, TK>), dim3(n_chunks, d.B), dim3(256), 0, st, (const XT*)x, carry,
                     w_down, w_up, noise, ns, logits, probs, idx, gates, act, h_out, d.T, d.D, d.R, d.E, d.topk,
                     n_chunks));
}

template <typename XT>
static void fwd_x(const void* x, const float* w_down, const float* w_up, const float* noise, float ns, float* logits,
                  float* probs, int32_t* idx, float* gates, float* act, float* h_out, char* ws, const RouterWs& w,
                  const RouterDims& d, hipStream_t st) {
  if (d.E <= 8 && d.topk <= 2)
    fwd_launch<XT, 8, 2>(x, w_down, w_up, noise, ns, logits, probs, idx, gates, act, h_out, ws, w, d, st);
  else if (d.E <= 8)
    fwd_launch<XT, 8, 8>(x, w_down, w_up, noise, ns, logits, probs, idx, gates, act, h_out, ws, w, d, st);
  else if (d.E <= 32)
    fwd_launch<XT, 32, 8>(x, w_down, w_up, noise, ns, logits, probs, idx, gates, act, h_out, ws, w, d, st);
  else
    fwd_launch<XT, 64, 8>(x, w_down, w_up, noise, ns, logits, probs, idx, gates, act, h_out, ws, w, d, st);
}

hipError_t launch_router_fwd(const void* x, bool x_bf16, const float* w_down, const float* w_up, const float* noise,
                             float noise_scale, float* logits, float* probs, int32_t* top_idx, float* top_gates,
                             float* act, float* h_out, void* ws, const RouterDims& d, hipStream_t st) {
  const RouterWs w = plan_router_ws(d);
  if (x_bf16)
    fwd_x<bf16_t>(x, w_down, w_up, noise, noise_scale, logits, probs, top_idx, top_gates, act, h_out, (char*)ws, w, d,
                  st);
  else
    fwd_x<float>(x, w_down, w_up, noise, noise_scale, logits, probs, top_idx, top_gates, act, h_out, (char*)ws, w, d,
                 st);
  return hipGetLastError();
}

template <int EMAX, int TK>
static void bwd_token(const float* act, const float* probs, const int32_t* idx, const float* gates, const float* dg,
                      const float* dp, const float* dl, const float* w_up, float* w_out, float* dwup_part,
                      const RouterDims& d, hipStream_t st) {
  const long ntok = (long)d.B * d.T;
  NAYLIS_TIMED("router_bwd_token", st, hipLaunchKernelGGL((router_bwd_token_kernel<EMAX, TK>), dim3((int)((ntok + 63) / 64)), dim3(64), 0, st, act, probs,
                     idx, gates, dg, dp, dl, w_up, w_out, dwup_part, d.T, d.R, d.E, d.topk, ntok));
}

template <typename XT>
static void bwd_dx(const void* x, const float* wt, const float* w_down, void* dx, float* dwd_part, const RouterDims& d,
                   hipStream_t st) {
  const long ntok = (long)d.B * d.T;
  const dim3 grid((int)((ntok + kDxChunk - 1) / kDxChunk), (d.D + 255) / 256);
  if (d.R <= 32)
    NAYLIS_TIMED("router_bwd_dx", st, hipLaunchKernelGGL((router_bwd_dx_kernel<XT, 32>), grid, dim3(256), 0, st, (const XT*)x, wt, w_down, (XT*)dx,
                       dwd_part, d.D, d.R, ntok));
  else
    NAYLIS_TIMED("router_bwd_dx", st, hipLaunchKernelGGL((router_bwd_dx_kernel<XT, 64>), grid, dim3(256), 0, st, (const XT*)x, wt, w_down, (XT*)dx,
                       dwd_part, d.D, d.R, ntok));
}

hipError_t launch_router_bwd(const void* x, bool x_bf16, const float* w_down, const float* w_up, const float* act,
                             const float* probs, const int32_t* top_idx, const float* top_gates, const float* d_gates,
                             const float* d_probs, const float* d_logits, void* dx, float* dw_down, float* dw_up,
                             void* ws, const RouterDims& d, hipStream_t st) {
  const RouterWs w = plan_router_ws(d);
  char* base = (char*)ws;
  float* wbuf = (float*)(base + w.w);
  float* wt = (float*)(base + w.wt);
  float* dwup_part = (float*)(base + w.dwup_part);
  float* dwd_part = (float*)(base + w.dwd_part);
  const long ntok = (long)d.B * d.T;
  const int n_tok_blocks = (int)((ntok + 63) / 64);
  const long nwd = (long)d.R * d.D;
  const long nwu = (long)d.E * d.R;
  if (ntok == 0) {  // no tokens: the weight gradients are zero
    NAYLIS_TIMED("router_reduce", st, hipLaunchKernelGGL(router_reduce_kernel, dim3((int)((nwd + 63) / 64)),
                       dim3(256), 0, st, dwd_part, dw_down, nwd, 0));
    NAYLIS_TIMED("router_reduce", st, hipLaunchKernelGGL(router_reduce_kernel, dim3((int)((nwu + 63) / 64)), dim3(256), 0, st, dwup_part, dw_up, nwu,
                       0));
    return hipGetLastError();
  }
  if (d.E <= 8 && d.topk <= 2)
    bwd_token<8, 2>(act, probs, top_idx, top_gates, d_gates, d_probs, d_logits, w_up, wbuf, dwup_part, d, st);
  else if (d.E <= 8)
    bwd_token<8, 8>(act, probs, top_idx, top_gates, d_gates, d_probs, d_logits, w_up, wbuf, dwup_part, d, st);
  else if (d.E <= 32)
    bwd_token<32, 8>(act, probs, top_idx, top_gates, d_gates, d_probs, d_logits, w_up, wbuf, dwup_part, d, st);
  else
    bwd_token<64, 8>(act, probs, top_idx, top_gates, d_gates, d_probs, d_logits, w_up, wbuf, dwup_part, d, st);
  {
    const int n_sc = (d.T + kScanChunk - 1) / kScanChunk;
    double* csum = (double*)(base + w.scan_csum);
    const dim3 grid(n_sc, d.B, (d.R + 31) / 32);
    NAYLIS_TIMED("router_bwd_scan", st,
                 hipLaunchKernelGGL(router_bwd_chunk_sums_kernel, grid, dim3(256), 0, st, wbuf, csum, d.T, d.R, n_sc));
    NAYLIS_TIMED("router_bwd_scan", st,
                 hipLaunchKernelGGL(router_bwd_scan_kernel, grid, dim3(256), 0, st, wbuf, csum, wt, d.T, d.R, n_sc));
  }
  if (x_bf16)
    bwd_dx<bf16_t>(x, wt, w_down, dx, dwd_part, d, st);
  else
    bwd_dx<float>(x, wt, w_down, dx, dwd_part, d, st);
  const int n_dx_chunks = (int)((ntok + kDxChunk - 1) / kDxChunk);
  NAYLIS_TIMED("router_reduce", st, hipLaunchKernelGGL(router_reduce_kernel, dim3((int)((nwd + 63) / 64)), dim3(256),
                     0, st, dwd_part, dw_down, nwd, n_dx_chunks));
  NAYLIS_TIMED("router_reduce", st, hipLaunchKernelGGL(router_reduce_kernel, dim3((int)((nwu + 63) / 64)), dim3(256), 0, st, dwup_part, dw_up, nwu,
                     n_tok_blocks));
  return hipGetLastError();
}

}  // namespace naylis
