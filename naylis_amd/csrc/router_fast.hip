// Router fast path for bf16 activations (gfx950): projection first, then the
// causal prefix over the R-wide projection.
//
// The reference forms the prefix mean h_t = cumsum(x)_t / (t+1) and projects
// it, z_t = h_t W_down^T (model.py:169-187).  The projection is linear, so
//   z_t = (sum_{s<=t} y_s) / (t+1),   y_s = x_s W_down^T,
// and the D-wide prefix never has to exist: x is read once, by one bf16 MFMA
// GEMM, and the scan runs over R = 32 columns.  bf16 x is exact in bf16;
// W_down (fp32) is split exactly into three bf16 planes w = w1 + w2 + w3
// (w1 = bf16(w), w2 = bf16(w - w1), w3 = bf16(w - w1 - w2); 3 x 8 significant
// bits cover fp32's 24), so every MFMA product is an exact fp32 product and y
// carries only the fp32 accumulation error of an fp32 GEMM (about 2^-24
// sqrt(D) relative), as the reference's own sgemm does.  The prefix sums run
// in fp64.  z therefore agrees with the reference to fp32 GEMM accuracy (not
// bitwise: the reference rounds h to fp32 before projecting); top-k indices
// agree outside near-ties, the same criterion as the exact-h path, which
// stays in router.hip for callers that ask for h itself or pass fp32 x.
//
// Backward: dx = W~ W_down (+ the caller's dx, accumulated in fp32 before the
// single bf16 rounding) and dW_down = W~^T x, W~ the reverse prefix of
// w_t = dz_t / (t+1) (router.hip).  W~ enters the MFMA as a bf16 hi/lo pair,
// W_down as a hi/lo pair; the three significant products give 2^-16 relative
// accuracy for the bf16 dx, and x is exact for dW_down.
#include <atomic>
#include <type_traits>

#include "common.h"
#include "launch.h"
#include "launch_router.h"
#include "timing.h"

namespace naylis {

constexpr int kFastChunk = 32;    // tokens per projection / head workgroup
constexpr int kFastDxRange = 256; // tokens per dx workgroup (one dW_down partial)
constexpr int kFastDxSlab = 128;  // features per dx workgroup

// Split 8 fp32 values into three bf16 planes whose sum is the input exactly.
__device__ __forceinline__ void split3(const f32x4& a, const f32x4& b, bf16x8& p1, bf16x8& p2, bf16x8& p3) {
  float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const __bf16 h1 = (__bf16)v[e];
    const float r1 = v[e] - (float)h1;
    const __bf16 h2 = (__bf16)r1;
    const float r2 = r1 - (float)h2;
    p1[e] = h1;
    p2[e] = h2;
    p3[e] = (__bf16)r2;
  }
}

// Split 8 fp32 values into a bf16 hi/lo pair (hi + lo within 2^-16 relative).
__device__ __forceinline__ void split2(const float (&v)[8], bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const __bf16 h = (__bf16)v[e];
    hi[e] = h;
    lo[e] = (__bf16)(v[e] - (float)h);
  }
}

// ---------------------------------------------------------------------------
// (F1) y[b][t][r] = x[b][t] . W_down[r] for NC consecutive 32-token chunks
// of one sequence per workgroup, and each chunk's fp64 column sums
// ycs[b][c][r].  Wave w of NW takes the features [w D/NW, (w+1) D/NW): its
// W_down rows are loaded and split into three bf16 planes once (B = W_down^T,
// d x r; every product of a bf16 x and a plane is exact in fp32), then the
// chunks stream through (A = x, tokens x d, 16-byte row loads straight from
// HBM, the next chunk's loads issued before this chunk's reduction); the NW
// partial 32 x R tiles of a chunk are added in wave order in LDS.  NC > 1
// amortises the W_down reads (and the plane split) over NC chunks.
template <int RT, int KSW, int NC>  // KSW: K-steps (16 features) per wave
__global__ __launch_bounds__(512) void router_proj_kernel(const bf16_t* __restrict__ x,
                                                          const float* __restrict__ w_down, float* __restrict__ y,
                                                          double* __restrict__ ycs, int T, int D, int R, int n_ch) {
  constexpr int CT = kFastChunk;
  constexpr int NW = 8;
  constexpr int P = 33;  // partial tile pitch
  __shared__ float part[NW][RT][CT * P];
  __shared__ float ysum[CT][RT * 32 + 1];
  const int cg = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int nks = D / (16 * NW);  // K-steps of this wave (<= KSW)
  const int d0 = wave * nks * 16;

  auto load_x = [&](bf16x8 (&xf)[KSW], int c) {
    const int t0 = c * CT, nt = min(CT, T - t0);
    const bf16_t* xrow = x + ((long)b * T + t0 + min(l32, nt - 1)) * D + d0 + 8 * g;
#pragma unroll
    for (int ks = 0; ks < KSW; ++ks) xf[ks] = *reinterpret_cast<const bf16x8*>(xrow + 16 * min(ks, nks - 1));
  };
  const int c_first = cg * NC;
  bf16x8 xf[KSW];
  load_x(xf, c_first);
  bf16x8 p1[KSW][RT], p2[KSW][RT], p3[KSW][RT];
  {
    f32x4 wf[KSW][RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const float* wrow = w_down + (long)min(rt * 32 + l32, R - 1) * D + d0 + 8 * g;
#pragma unroll
      for (int ks = 0; ks < KSW; ++ks) {
        const int kc = min(ks, nks - 1);
        wf[ks][rt][0] = *reinterpret_cast<const f32x4*>(wrow + 16 * kc);
        wf[ks][rt][1] = *reinterpret_cast<const f32x4*>(wrow + 16 * kc + 4);
      }
    }
#pragma unroll
    for (int ks = 0; ks < KSW; ++ks)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) split3(wf[ks][rt][0], wf[ks][rt][1], p1[ks][rt], p2[ks][rt], p3[ks][rt]);
  }
  const int RW = RT * 32;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = c_first + j;
    if (c >= n_ch) break;  // workgroup-uniform
    const int t0 = c * CT, nt = min(CT, T - t0);
    f32x16 acc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KSW; ++ks) {
      if (ks < nks) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          acc[rt] = mfma32(xf[ks], p3[ks][rt], acc[rt]);  // smallest terms first
          acc[rt] = mfma32(xf[ks], p2[ks][rt], acc[rt]);
          acc[rt] = mfma32(xf[ks], p1[ks][rt], acc[rt]);
        }
      }
    }
    if (j + 1 < NC && c + 1 < n_ch) load_x(xf, c + 1);  // in flight during the reduction below
    // partial tiles: D[row = token][col = rank]
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int v = 0; v < 16; ++v) part[wave][rt][acc_row(g, v) * P + l32] = acc[rt][v];
    lds_barrier();
    for (int i = tid; i < CT * RW; i += NW * 64) {
      const int t = i / RW, r = i % RW, rt = r >> 5, rl = r & 31;
      float sum = part[0][rt][t * P + rl];
#pragma unroll
      for (int w = 1; w < NW; ++w) sum += part[w][rt][t * P + rl];
      ysum[t][r] = sum;
      if (t < nt && r < R) y[((long)b * T + t0 + t) * R + r] = sum;
    }
    lds_barrier();
    if (tid < R) {
      double cs = 0.0;
      for (int t = 0; t < nt; ++t) cs += (double)ysum[t][tid];
      ycs[((long)b * n_ch + c) * R + tid] = cs;
    }
    // ysum / part are rewritten by the next chunk only after this barrier
    if (j + 1 < NC) lds_barrier();
  }
}

// run + p[0] + p[stride] + ... + p[(n-1) stride], added in that order (fp64);
// the LDS reads are issued 8 at a time so the chain waits on the adds only.
__device__ __forceinline__ double add_in_order(double run, const double* p, int stride, int n) {
  int k = 0;
  for (; k + 8 <= n; k += 8) {
    double v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = p[(k + u) * stride];
#pragma unroll
    for (int u = 0; u < 8; ++u) run += v[u];
  }
  for (; k < n; ++k) run += p[k * stride];
  return run;
}

// For threads tid < R: the fp64 sum of cs[c * R + tid] over the chunks
// c_lo <= c < c_hi, added in chunk order.  The chunk sums are staged through
// LDS (stage: 4096 doubles) 4096 / R chunks at a time, one coalesced load
// round per block, so the serial part is LDS reads and fp64 adds.  Called by
// the whole 256-thread workgroup (c_lo, c_hi uniform).
__device__ __forceinline__ double chunk_carry(const double* __restrict__ cs, int c_lo, int c_hi, int R,
                                              double* stage, int tid) {
  double run = 0.0;
  const int per = 4096 / R;
  for (int cb = c_lo; cb < c_hi; cb += per) {
    const int nc = min(per, c_hi - cb), n = nc * R;
    const double* src = cs + (long)cb * R;
    double v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = tid + 256 * u < n ? src[tid + 256 * u] : 0.0;
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (tid + 256 * u < n) stage[tid + 256 * u] = v[u];
    __syncthreads();
    if (tid < R) run = add_in_order(run, stage + tid, R, nc);
    __syncthreads();
  }
  return run;
}

// ---------------------------------------------------------------------------
// (F2) per (b, 32-token chunk): fp64 carry of the earlier chunks' sums, the
// in-chunk prefix, z = Z / (t+1), tanh, logits = a W_up^T, softmax probs,
// top-k (ties -> lowest id) and gates; the tail matches router_fwd_kernel.
// The prefix is one serial fp64 chain per rank (carry + y_0 + ... + y_t, in
// token order); everything else runs over (token, rank) pairs or over 8
// lanes per token (lane p of token t owns experts p, p + 8, ...).
// LDS of one chunk's head (router_head_body)
template <int EMAX>
struct HeadLds {
  float a[kFastChunk * 65];
  float lg[kFastChunk * (EMAX + 1)];
  float ex[kFastChunk * (EMAX + 1)];
  float sum[kFastChunk];
};

// The head of chunk c of sequence b from its projections y (y_lds, row pitch
// 65) and the fp64 carry of the earlier chunks (carry_lds[r]); run by 256
// threads (tid 0..255) with the W_up rows in wu_lds; zs_lds (32 x 65
// doubles) takes the in-chunk prefix.  Every thread of the workgroup must
// call it (it has barriers).
template <int EMAX, int TK>
__device__ __forceinline__ void router_head_body(
    int tid, int c, int b, const float* y_lds, const double* carry_lds, const float* wu_lds, double* zs_lds,
    HeadLds<EMAX>& L,
    const float* __restrict__ noise, float noise_scale, int noise_kind, float* __restrict__ logits,
    float* __restrict__ probs, int32_t* __restrict__ top_idx, float* __restrict__ top_gates,
    float* __restrict__ act, int T, int R, int E, int topk) {
  constexpr int CT = kFastChunk;
  constexpr int LP = EMAX + 1;
  constexpr int EPL = EMAX / 8;  // experts per lane
  constexpr int NONE = 0x7fffffff;
  const int t0 = c * CT, nt = min(CT, T - t0);
  float* a_lds = L.a;
  float* lg_lds = L.lg;
  float* ex_lds = L.ex;
  float* sum_lds = L.sum;
  // Z_t = carry + y_0 + ... + y_t in token order (fp64), one chain per rank
  if (tid < R) {
    double run = carry_lds[tid];
#pragma unroll
    for (int t = 0; t < CT; ++t)
      if (t < nt) {
        run += (double)y_lds[t * 65 + tid];
        zs_lds[t * 65 + tid] = run;
      }
  }
  __syncthreads();
  // z = fp32(Z_t * fp64(1 / (t+1))), a = tanh(z), (token, rank) pairs in parallel
  for (int i = tid; i < nt * R; i += 256) {
    const int t = i / R, r = i % R;
    const float z = (float)(zs_lds[t * 65 + r] * (1.0 / (double)(t0 + t + 1)));
    const float a = tanhf(z);
    a_lds[t * 65 + r] = a;
    act[((long)b * T + t0) * R + i] = a;
  }
  __syncthreads();
  const int tk = tid >> 3, part = tid & 7;
  const int tc = min(tk, nt - 1);
  const bool live = tk < nt;  // the 8 lanes of a token are all live or all idle
  const long tok = (long)b * T + t0 + tc;
  {
#pragma unroll
    for (int k = 0; k < EPL; ++k) {
      const int e = part + 8 * k;
      if (e < E) {
        float lg = 0.f;
        for (int r = 0; r < R; ++r) lg = fmaf(a_lds[tc * 65 + r], wu_lds[e * 65 + r], lg);
        if (live) {
          lg_lds[tc * LP + e] = lg;
          logits[tok * E + e] = lg;
        }
      }
    }
  }
  __syncthreads();
  float lg[EPL], nz[EPL];
#pragma unroll
  for (int k = 0; k < EPL; ++k) {
    const int e = part + 8 * k;
    lg[k] = e < E ? lg_lds[tc * LP + e] : 0.f;
    nz[k] = e < E ? (noise ? noisy_logit(lg[k], noise[tok * E + e], noise_scale, noise_kind) : lg[k]) : -INFINITY;
  }
  // softmax: the max over the token's lanes (exact in any order), the sum in
  // expert order by lane 0
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < EPL; ++k)
    if (part + 8 * k < E) mx = fmaxf(mx, lg[k]);
#pragma unroll
  for (int m = 1; m < 8; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 8));
  float ex[EPL];
#pragma unroll
  for (int k = 0; k < EPL; ++k) {
    const int e = part + 8 * k;
    ex[k] = e < E ? expf(lg[k] - mx) : 0.f;
    if (live && e < E) ex_lds[tc * LP + e] = ex[k];
  }
  __syncthreads();
  if (live && part == 0) {
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < EMAX; ++e)
      if (e < E) sum += ex_lds[tc * LP + e];
    sum_lds[tc] = sum;
  }
  __syncthreads();
  if (live) {
    const float sum = sum_lds[tc];
#pragma unroll
    for (int k = 0; k < EPL; ++k)
      if (part + 8 * k < E) probs[tok * E + part + 8 * k] = ex[k] / sum;
  }
  // top-k: per round each lane's best untaken expert (value, then lowest id),
  // combined over the token's 8 lanes and taken from lane 0 so that every
  // lane records the same choice
  int sel[TK];
  float val[TK];
  unsigned taken = 0;  // bit k: expert part + 8k of this lane
#pragma unroll
  for (int s = 0; s < TK; ++s) {
    sel[s] = 0;
    val[s] = 0.f;
    if (s < topk) {
      int best = NONE;
      float bv = -INFINITY;
#pragma unroll
      for (int k = 0; k < EPL; ++k) {
        const int e = part + 8 * k;
        if (e < E && !((taken >> k) & 1u) && (best == NONE || nz[k] > bv)) {
          best = e;
          bv = nz[k];
        }
      }
#pragma unroll
      for (int m = 1; m < 8; m <<= 1) {
        const int ob = __shfl_xor(best, m, 8);
        const float ov = __shfl_xor(bv, m, 8);
        if (ob != NONE && (best == NONE || ov > bv || (ov == bv && ob < best))) {
          best = ob;
          bv = ov;
        }
      }
      best = __shfl(best, 0, 8);
      bv = __shfl(bv, 0, 8);
      if (best != NONE && (best & 7) == part) taken |= 1u << (best >> 3);
      sel[s] = best == NONE ? -1 : best;
      val[s] = bv;
    }
  }
  if (live && part == 0) {
    float gs = 0.f;
#pragma unroll
    for (int s = 0; s < TK; ++s)
      if (s < topk) gs += expf(val[s] - val[0]);
#pragma unroll
    for (int s = 0; s < TK; ++s)
      if (s < topk) {
        top_idx[tok * topk + s] = sel[s];
        top_gates[tok * topk + s] = expf(val[s] - val[0]) / gs;
      }
  }
}

// ---------------------------------------------------------------------------
// (F) The forward in one launch: router_proj_kernel's projection of two
// chunks per workgroup, then router_head_body on both chunks (one per half of
// the workgroup), the carry of the earlier chunks' fp64 sums taken from the
// other workgroups of the sequence.  Each chunk's sums are published as word
// pairs (v, v ^ epoch), written and read with device-scope atomic 64-bit
// accesses: a pair is valid for this launch only when the words XOR to its
// epoch, so stale pairs (another launch) and torn ones (one word new, one
// old) are both rejected without a flag or a fence.  A workgroup waits only
// on the chunks before its own, i.e. on workgroups of lower dispatch order in
// the same sequence; the wait is bounded, and a chunk still missing after it
// is projected again from x here, the same operations in the same order, so
// the carry is bitwise that of the two launches whatever happens.  The bound
// (spin: polls, an s_sleep between them, per block of earlier chunks) is a
// launch argument; 0 skips the wait and re-projects every earlier chunk.

template <int RT, int KSW, int EMAX, int TK>
__global__ __launch_bounds__(512) void router_fwd_fused_kernel(
    const bf16_t* __restrict__ x, const float* __restrict__ w_down, const float* __restrict__ w_up,
    const float* __restrict__ noise, float noise_scale, int noise_kind, float* __restrict__ logits,
    float* __restrict__ probs, int32_t* __restrict__ top_idx, float* __restrict__ top_gates,
    float* __restrict__ act, unsigned long long* __restrict__ pub, unsigned long long epoch, int T, int D, int R,
    int E, int topk, int n_ch, int spin) {
  constexpr int CT = kFastChunk;
  constexpr int NW = 8, NC = 2;
  constexpr int P = 33;  // partial tile pitch
  __shared__ float part[NW][RT][CT * P];
  __shared__ float yk[NC][CT * 65];             // the two chunks' projections (head layout)
  __shared__ double stage[4160];                // earlier chunks' sums, then the two halves' prefixes
  __shared__ float wu_lds[EMAX * 65];
  __shared__ double carry_lds[NC][64];
  __shared__ HeadLds<EMAX> hl[NC];
  const int cg = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int nks = D / (16 * NW);
  const int d0 = wave * nks * 16;
  const int c_first = cg * NC;
  unsigned long long* pub_b = pub + (long)b * n_ch * R * 2;

  for (int i = tid; i < E * R; i += NW * 64) wu_lds[(i / R) * 65 + i % R] = w_up[i];
  auto load_x = [&](bf16x8 (&xf)[KSW], int c) {
    const int t0 = c * CT, nt = min(CT, T - t0);
    const bf16_t* xrow = x + ((long)b * T + t0 + min(l32, nt - 1)) * D + d0 + 8 * g;
#pragma unroll
    for (int ks = 0; ks < KSW; ++ks) xf[ks] = *reinterpret_cast<const bf16x8*>(xrow + 16 * min(ks, nks - 1));
  };
  bf16x8 xf[KSW];
  load_x(xf, c_first);
  bf16x8 p1[KSW][RT], p2[KSW][RT], p3[KSW][RT];
  {
    f32x4 wf[KSW][RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const float* wrow = w_down + (long)min(rt * 32 + l32, R - 1) * D + d0 + 8 * g;
#pragma unroll
      for (int ks = 0; ks < KSW; ++ks) {
        const int kc = min(ks, nks - 1);
        wf[ks][rt][0] = *reinterpret_cast<const f32x4*>(wrow + 16 * kc);
        wf[ks][rt][1] = *reinterpret_cast<const f32x4*>(wrow + 16 * kc + 4);
      }
    }
#pragma unroll
    for (int ks = 0; ks < KSW; ++ks)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) split3(wf[ks][rt][0], wf[ks][rt][1], p1[ks][rt], p2[ks][rt], p3[ks][rt]);
  }
  const int RW = RT * 32;
  // chunk c's projections into out (row pitch 65) and, for threads tid < R,
  // its fp64 column sum (the operations of router_proj_kernel, in its order)
  auto project = [&](const bf16x8 (&xc)[KSW], int c, float* out) -> double {
    const int t0 = c * CT, nt = min(CT, T - t0);
    f32x16 acc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KSW; ++ks) {
      if (ks < nks) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          acc[rt] = mfma32(xc[ks], p3[ks][rt], acc[rt]);  // smallest terms first
          acc[rt] = mfma32(xc[ks], p2[ks][rt], acc[rt]);
          acc[rt] = mfma32(xc[ks], p1[ks][rt], acc[rt]);
        }
      }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int v = 0; v < 16; ++v) part[wave][rt][acc_row(g, v) * P + l32] = acc[rt][v];
    __syncthreads();
    for (int i = tid; i < CT * RW; i += NW * 64) {
      const int t = i / RW, r = i % RW, rt = r >> 5, rl = r & 31;
      float sum = part[0][rt][t * P + rl];
#pragma unroll
      for (int w = 1; w < NW; ++w) sum += part[w][rt][t * P + rl];
      if (r < R) out[t * 65 + r] = sum;
    }
    __syncthreads();
    double cs = 0.0;
    if (tid < R)
      for (int t = 0; t < nt; ++t) cs += (double)out[t * 65 + tid];
    return cs;
  };
  // ---- the two chunks, each published as soon as its sums exist
  double cs_own[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = c_first + j;
    bf16x8 xn[KSW];
    if (j + 1 < NC) load_x(xn, c + 1);  // in flight during this chunk's reduction
    cs_own[j] = project(xf, c, yk[j]);
    if (tid < R) {
      const unsigned long long w1 = __double_as_longlong(cs_own[j]);
      unsigned long long* q = pub_b + ((long)c * R + tid) * 2;
      __hip_atomic_store(q, w1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(q + 1, w1 ^ epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (j + 1 < NC) {
#pragma unroll
      for (int ks = 0; ks < KSW; ++ks) xf[ks] = xn[ks];
    }
  }
  // ---- carry of chunk c_first: the published sums of chunks 0 .. c_first - 1
  // in chunk order (as chunk_carry), staged per block of 4096 / R chunks
  double run = 0.0;
  const int per = 4096 / R;
  for (int cb = 0; cb < c_first; cb += per) {
    const int nc = min(per, c_first - cb), n = nc * R;
    bool done = false;
    for (int it = 0; it < spin && !done; ++it) {
      int ok = 1;
      for (int i = tid; i < n; i += NW * 64) {
        const unsigned long long* q = pub_b + ((long)cb * R + i) * 2;
        const unsigned long long w1 = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned long long w2 = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((w1 ^ w2) == epoch) stage[i] = __longlong_as_double(w1);
        else ok = 0;
      }
      done = __syncthreads_and(ok) != 0;
      if (!done) __builtin_amdgcn_s_sleep(2);
    }
    if (!done) {
      // still missing after the bound: project the block's chunks here
      for (int k = 0; k < nc; ++k) {
        bf16x8 xc[KSW];
        load_x(xc, cb + k);
        const double cs = project(xc, cb + k, hl[0].a);  // (hl[0].a: scratch until the head)
        if (tid < R) stage[k * R + tid] = cs;
        __syncthreads();
      }
    }
    if (tid < R) run = add_in_order(run, stage + tid, R, nc);
    __syncthreads();
  }
  if (tid < R) {
    carry_lds[0][tid] = run;
    carry_lds[1][tid] = run + cs_own[0];  // the carry of chunk c_first + 1, extending the same chain
  }
  __syncthreads();
  // ---- the heads: chunk c_first + h by the threads of half h
  const int h = tid >> 8;
  router_head_body<EMAX, TK>(tid & 255, c_first + h, b, yk[h], carry_lds[h], wu_lds, stage + h * 2080, hl[h],
                             noise, noise_scale, noise_kind, logits, probs, top_idx, top_gates, act, T, R, E, topk);
}

template <int EMAX, int TK>
__global__ __launch_bounds__(256) void router_head_kernel(
    const float* __restrict__ y, const double* __restrict__ ycs, const float* __restrict__ w_up,
    const float* __restrict__ noise, float noise_scale, int noise_kind, float* __restrict__ logits,
    float* __restrict__ probs,
    int32_t* __restrict__ top_idx, float* __restrict__ top_gates, float* __restrict__ act, int T, int R, int E,
    int topk, int n_ch) {
  constexpr int CT = kFastChunk;
  __shared__ float y_lds[CT * 65];
  __shared__ double stage[4096];  // carry staging, then the in-chunk prefix
  __shared__ float wu_lds[EMAX * 65];
  __shared__ double carry_lds[64];
  __shared__ HeadLds<EMAX> hl;
  const int c = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x;
  const int t0 = c * CT, nt = min(CT, T - t0);
  for (int i = tid; i < E * R; i += 256) wu_lds[(i / R) * 65 + i % R] = w_up[i];
  for (int i = tid; i < nt * R; i += 256) y_lds[(i / R) * 65 + i % R] = y[((long)b * T + t0) * R + i];
  // carry = sum of the earlier chunks' fp64 sums, in chunk order
  const double carry = chunk_carry(ycs + (long)b * n_ch * R, 0, c, R, stage, tid);
  if (tid < R) carry_lds[tid] = carry;
  __syncthreads();
  router_head_body<EMAX, TK>(tid, c, b, y_lds, carry_lds, wu_lds, stage, hl, noise, noise_scale, noise_kind, logits,
                             probs, top_idx, top_gates, act, T, R, E, topk);
}

// ---------------------------------------------------------------------------
// (B3) dx and dW_down for one (256-token range, 128-feature slab); wave w
// owns features f0 = 128 slab + 32 w .. +31.  Per 32-token step the W~ rows
// (as a bf16 hi/lo pair) and the x rows are staged in LDS (double-buffered
// through registers):
//   dx^T (32 feat x 32 tok) = W_down^T W~^T: A = W_down^T from registers
//     (rows permuted by row_perm32 so a lane half holds 16 consecutive
//     features), B = W~ rows from LDS; + dx_in; one bf16 rounding.
//   dW_down^T (32 feat x R) += x^T W~: both operands K(token)-major, read
//     with transposing LDS reads from the natural-layout tiles.
// The range's dW_down partial goes to dwd_part[range][r][f] (summed over
// ranges in a fixed order by router_reduce_kernel).
//
// FUSED (R <= 32, T a multiple of the range): W~ is not read from wt but
// formed here from w and its chunk sums wcs, the range being 8 whole chunks
// of one sequence.  Thread (chunk j, rank r) adds the chunk sums after its
// chunk in chunk order (staged through LDS) and then runs the chunk's suffix
// in place over the range's w rows in LDS: the same fp64 operations in the
// same order as router_wtilde_kernel, so W~ is bitwise the same.
template <int RT, bool FUSED>
__global__ __launch_bounds__(256) void router_dx_fast_kernel(const bf16_t* __restrict__ x,
                                                             const float* __restrict__ wt,
                                                             const float* __restrict__ w_down,
                                                             const bf16_t* __restrict__ dx_in,
                                                             bf16_t* __restrict__ dx, float* __restrict__ dwd_part,
                                                             int D, int R, long ntok, const float* __restrict__ w,
                                                             const double* __restrict__ wcs, int T, int n_ch) {
  constexpr int ST = 32;                 // tokens per step
  constexpr int RW = RT * 32;            // staged ranks (zero padded)
  constexpr int WP = RW + 8;             // W~ plane pitch (bf16)
  constexpr int XP = kFastDxSlab + 8;    // x tile pitch (bf16)
  constexpr int KR = RW / 16;            // K-steps over ranks
  __shared__ __attribute__((aligned(16))) bf16_t wt_hi[2][ST * WP];
  __shared__ __attribute__((aligned(16))) bf16_t wt_lo[2][ST * WP];
  __shared__ __attribute__((aligned(16))) bf16_t x_lds[2][ST * XP];
  // FUSED: chunk-sum staging (4096 doubles), then the range's W~ rows
  // (kFastDxRange x 32 fp32, row pitch 32)
  __shared__ __attribute__((aligned(16))) double wt_s[FUSED ? 4096 : 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const long tok_beg = (long)blockIdx.x * kFastDxRange;
  const int slab = blockIdx.y * kFastDxSlab;
  const int f0 = slab + wave * 32;
  float* const wts = reinterpret_cast<float*>(wt_s);

  // A operand of dx^T: W_down[r = 16 ks + 8 g + e][f0 + row_perm32(l32)], hi/lo
  bf16x8 wa_hi[KR], wa_lo[KR];
  {
    const int f = f0 + row_perm32(l32);
#pragma unroll
    for (int ks = 0; ks < KR; ++ks) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int r = 16 * ks + 8 * g + e;
        v[e] = r < R ? w_down[(long)r * D + f] : 0.f;
      }
      split2(v, wa_hi[ks], wa_lo[ks]);
    }
  }
  f32x16 accw[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) accw[rt] = f32x16{};

  // staging registers: W~ (ST x RW fp32: RW / 8 values per thread) and x
  // (ST x 128 bf16: 16 per thread)
  constexpr int WV = ST * RW / 256;  // fp32 values of W~ per thread (4 or 8)
  float wreg[WV];
  uint4 xreg[2];
  // dx_in rows of this lane's token and 16 features, one step ahead (zeros
  // when there is no dx_in: bf16 0 adds +0.0f)
  uint4 dcur[2], dnext[2];
  auto fetch_dx_in = [&](uint4 (&dr)[2], long ts) {
    const long tok = ts + l32;
    if (dx_in != nullptr && tok < ntok) {
      const long o = tok * D + f0 + 16 * g;
      dr[0] = *reinterpret_cast<const uint4*>(dx_in + o);
      dr[1] = *reinterpret_cast<const uint4*>(dx_in + o + 8);
    } else {
      dr[0] = dr[1] = make_uint4(0, 0, 0, 0);
    }
  };
  auto fetch = [&](long ts) {
    if constexpr (!FUSED) {  // FUSED: stash reads W~ from wts
      const int t = tid / (RW / WV), r0 = (tid % (RW / WV)) * WV;
      const long tk = ts + t;
      if ((R & 3) == 0 && r0 + WV <= R && tk < ntok) {
#pragma unroll
        for (int e = 0; e < WV; e += 4) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(wt + tk * R + r0 + e);
          wreg[e] = v[0];
          wreg[e + 1] = v[1];
          wreg[e + 2] = v[2];
          wreg[e + 3] = v[3];
        }
      } else {
#pragma unroll
        for (int e = 0; e < WV; ++e) {
          const int r = r0 + e;
          wreg[e] = (tk < ntok && r < R) ? wt[tk * R + r] : 0.f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = tid + 256 * u, t = i >> 4, c8 = i & 15;
      const long tk = ts + t;
      xreg[u] = tk < ntok ? *reinterpret_cast<const uint4*>(x + tk * D + slab + 8 * c8) : make_uint4(0, 0, 0, 0);
    }
  };
  auto stash = [&](int buf, long ts) {
    {
      const int t = tid / (RW / WV), r0 = (tid % (RW / WV)) * WV;
      if constexpr (FUSED) {
#pragma unroll
        for (int e = 0; e < WV; ++e) wreg[e] = r0 + e < R ? wts[(ts - tok_beg + t) * 32 + r0 + e] : 0.f;
      }
#pragma unroll
      for (int e = 0; e < WV; ++e) {
        const __bf16 h = (__bf16)wreg[e];
        wt_hi[buf][t * WP + r0 + e] = __builtin_bit_cast(bf16_t, h);
        wt_lo[buf][t * WP + r0 + e] = f32_to_bf16(wreg[e] - (float)h);
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = tid + 256 * u, t = i >> 4, c8 = i & 15;
      *reinterpret_cast<uint4*>(&x_lds[buf][t * XP + 8 * c8]) = xreg[u];
    }
  };

  const int n_steps = (int)min((long)(kFastDxRange / ST), (ntok - tok_beg + ST - 1) / ST);
  fetch(tok_beg);
  fetch_dx_in(dcur, tok_beg);
  if constexpr (FUSED) {
    constexpr int CPR = kFastDxRange / kFastChunk;  // chunks per range (8)
    const int b = (int)(tok_beg / T), cf = (int)(tok_beg % T) / kFastChunk;
    const int j = tid >> 5, r = tid & 31;
    const double* cs = wcs + (long)b * n_ch * R;
    // the range's w rows (in flight during the carry below; wt_s holds the
    // staged chunk sums until then)
    float wv[32];
#pragma unroll
    for (int u = 0; u < 32; ++u) {
      const int i = tid + 256 * u;
      wv[u] = i < kFastDxRange * R ? w[tok_beg * R + i] : 0.f;
    }
    // carry of chunk cf + j: chunk sums c = cf + j + 1 .. n_ch - 1 in order
    double run = 0.0;
    for (int cb = cf + 1; cb < n_ch; cb += 4096 / R) {
      const int nc = min(4096 / R, n_ch - cb), n = nc * R;
      double v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = tid + 256 * u < n ? cs[(long)cb * R + tid + 256 * u] : 0.0;
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (tid + 256 * u < n) wt_s[tid + 256 * u] = v[u];
      __syncthreads();
      const int k0 = max(0, cf + j + 1 - cb);
      if (r < R) run = add_in_order(run, wt_s + k0 * R + r, R, nc - k0);
      __syncthreads();
    }
    // the w rows to LDS, then the in-chunk suffix in place
#pragma unroll
    for (int u = 0; u < 32; ++u) {
      const int i = tid + 256 * u;
      if (i < kFastDxRange * R) wts[R == 32 ? i : (i / R) * 32 + i % R] = wv[u];
    }
    __syncthreads();
    if (r < R) {
#pragma unroll
      for (int t = kFastChunk - 1; t >= 0; --t) {
        float* e = &wts[(j * kFastChunk + t) * 32 + r];
        run += (double)*e;
        *e = (float)run;
      }
    }
    static_assert(CPR * 32 == 256, "one thread per (chunk, rank)");
    __syncthreads();
  }
  stash(0, tok_beg);
  __syncthreads();
  for (int st = 0; st < n_steps; ++st) {
    const int buf = st & 1;
    const long ts = tok_beg + (long)st * ST;
    if (st + 1 < n_steps) {
      fetch(ts + ST);
      fetch_dx_in(dnext, ts + ST);
    }
    // ---- dx^T = W_down^T W~^T for this wave's 32 features x 32 tokens
    {
      f32x16 acc = f32x16{};
#pragma unroll
      for (int ks = 0; ks < KR; ++ks) {
        const int off = l32 * WP + 16 * ks + 8 * g;
        const bf16x8 bh = *reinterpret_cast<const bf16x8*>(&wt_hi[buf][off]);
        const bf16x8 bl = *reinterpret_cast<const bf16x8*>(&wt_lo[buf][off]);
        acc = mfma32(wa_lo[ks], bh, acc);
        acc = mfma32(wa_hi[ks], bl, acc);
        acc = mfma32(wa_hi[ks], bh, acc);
      }
      const long tok = ts + l32;
      if (tok < ntok) {
        const long o = tok * D + f0 + 16 * g;  // this lane half's 16 consecutive features
        float add[16];
        {
          const uint32_t w8[8] = {dcur[0].x, dcur[0].y, dcur[0].z, dcur[0].w,
                                  dcur[1].x, dcur[1].y, dcur[1].z, dcur[1].w};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            add[2 * e] = __uint_as_float(w8[e] << 16);
            add[2 * e + 1] = __uint_as_float(w8[e] & 0xffff0000u);
          }
        }
        bf16x8 lo, hi;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          lo[e] = (__bf16)(acc[e] + add[e]);
          hi[e] = (__bf16)(acc[8 + e] + add[8 + e]);
        }
        *reinterpret_cast<bf16x8*>(dx + o) = lo;
        *reinterpret_cast<bf16x8*>(dx + o + 8) = hi;
      }
    }
    // ---- dW_down^T (32 features x R) += x^T W~ over the step's 32 tokens
#pragma unroll
    for (int kk = 0; kk < ST / 16; ++kk) {
      const bf16x8 ax = lds_frag_T<false, false>(x_lds[buf], XP, 16 * kk, wave * 32);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const bf16x8 bh = lds_frag_T<false, false>(wt_hi[buf], WP, 16 * kk, 32 * rt);
        const bf16x8 bl = lds_frag_T<false, false>(wt_lo[buf], WP, 16 * kk, 32 * rt);
        accw[rt] = mfma32(ax, bl, accw[rt]);
        accw[rt] = mfma32(ax, bh, accw[rt]);
      }
    }
    if (st + 1 < n_steps) {
      stash(buf ^ 1, ts + ST);  // last read before the previous barrier
      dcur[0] = dnext[0];
      dcur[1] = dnext[1];
    }
    __syncthreads();
  }
  // dW_down partial of this range: accw[rt] row = feature f0 + acc_row(g, v), column = rank
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int r = rt * 32 + l32;
    if (r < R) {
#pragma unroll
      for (int v = 0; v < 16; ++v)
        dwd_part[((long)blockIdx.x * R + r) * D + f0 + acc_row(g, v)] = accw[rt][v];
    }
  }
}

// ---------------------------------------------------------------------------
// (B1) per (b, 32-token chunk): d(logits) of each token from d(gates),
// d(probs) and d(logits) (softmax and softmax-of-top-k chains, model.py:215-
// 220), then w_t = (dl_t W_up)(1 - a_t^2) / (t+1) for every (token, rank)
// pair in parallel, the chunk's fp64 column sums of w, and the chunk's
// partial dW_up = dl^T a (summed over chunks by router_reduce_kernel).
template <int EMAX, int TK>
__global__ __launch_bounds__(256) void router_bwd_token_fast_kernel(
    const float* __restrict__ act, const float* __restrict__ probs, const int32_t* __restrict__ top_idx,
    const float* __restrict__ top_gates, const float* __restrict__ d_gates, const float* __restrict__ d_probs,
    const float* __restrict__ d_logits, const float* __restrict__ w_up, float* __restrict__ w_out,
    double* __restrict__ wcs, float* __restrict__ dwup_part, int T, int R, int E, int topk, int n_ch, long dps) {
  constexpr int CT = kFastChunk;
  __shared__ float dl_lds[CT * (EMAX + 1)];
  __shared__ float a_lds[CT * 65];
  __shared__ float wu_lds[EMAX * 65];
  __shared__ float w_lds[CT * 65];
  const int c = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x;
  const int t0 = c * CT, nt = min(CT, T - t0);
  const long tok0 = (long)b * T + t0;
  for (int i = tid; i < E * R; i += 256) wu_lds[(i / R) * 65 + i % R] = w_up[i];
  for (int i = tid; i < CT * R; i += 256) a_lds[(i / R) * 65 + i % R] = i < nt * R ? act[tok0 * R + i] : 0.f;
  if (tid < CT) {
    float dl[EMAX];
#pragma unroll
    for (int e = 0; e < EMAX; ++e) dl[e] = 0.f;
    if (tid < nt) {
      const long tok = tok0 + tid;
      if (d_logits) {
#pragma unroll
        for (int e = 0; e < EMAX; ++e)
          if (e < E) dl[e] = d_logits[tok * E + e];
      }
      if (d_probs) {
        float pv[EMAX], dp[EMAX];
        float dot = 0.f;
#pragma unroll
        for (int e = 0; e < EMAX; ++e) {
          pv[e] = e < E ? probs[tok * E + e] : 0.f;
          dp[e] = e < E ? d_probs[tok * dps + e] : 0.f;
        }
#pragma unroll
        for (int e = 0; e < EMAX; ++e) dot = fmaf(pv[e], dp[e], dot);
#pragma unroll
        for (int e = 0; e < EMAX; ++e)
          if (e < E) dl[e] = fmaf(pv[e], dp[e] - dot, dl[e]);
      }
      if (d_gates) {
        float gv[TK], dg[TK];
        int gi[TK];
        float gdot = 0.f;
#pragma unroll
        for (int t = 0; t < TK; ++t) {
          gv[t] = t < topk ? top_gates[tok * topk + t] : 0.f;
          dg[t] = t < topk ? d_gates[tok * topk + t] : 0.f;
          gi[t] = t < topk ? top_idx[tok * topk + t] : -1;
        }
#pragma unroll
        for (int t = 0; t < TK; ++t) gdot = fmaf(gv[t], dg[t], gdot);
#pragma unroll
        for (int t = 0; t < TK; ++t)
          if (t < topk) {
            const float dv = gv[t] * (dg[t] - gdot);
#pragma unroll
            for (int u = 0; u < EMAX; ++u)
              if (u == gi[t]) dl[u] += dv;
          }
      }
    }
#pragma unroll
    for (int e = 0; e < EMAX; ++e) dl_lds[tid * (EMAX + 1) + e] = dl[e];
  }
  __syncthreads();
  for (int i = tid; i < nt * R; i += 256) {
    const int j = i / R, r = i % R;
    float da = 0.f;
#pragma unroll
    for (int e = 0; e < EMAX; ++e)
      if (e < E) da = fmaf(dl_lds[j * (EMAX + 1) + e], wu_lds[e * 65 + r], da);
    const float a = a_lds[j * 65 + r];
    const float wv = da * (1.f - a * a) / (float)(t0 + j + 1);
    w_lds[j * 65 + r] = wv;
    w_out[tok0 * R + i] = wv;
  }
  __syncthreads();
  if (tid < R) {
    double cs = 0.0;
    for (int t = 0; t < nt; ++t) cs += (double)w_lds[t * 65 + tid];
    wcs[((long)b * n_ch + c) * R + tid] = cs;
  }
  const long part = (long)b * n_ch + c;
  for (int i = tid; i < E * R; i += 256) {
    const int e = i / R, r = i % R;
    float acc = 0.f;
    for (int j = 0; j < nt; ++j) acc = fmaf(dl_lds[j * (EMAX + 1) + e], a_lds[j * 65 + r], acc);
    dwup_part[part * E * R + i] = acc;
  }
}

// (B2) W~_t = sum_{s >= t} w_s within the sequence: per (b, 32-token chunk),
// the fp64 carry of the later chunks' sums (chunk order) plus the in-chunk
// suffix (token order, descending), one serial chain per rank.
__global__ __launch_bounds__(256) void router_wtilde_kernel(const float* __restrict__ w,
                                                            const double* __restrict__ wcs,
                                                            float* __restrict__ wt, int T, int R, int n_ch) {
  constexpr int CT = kFastChunk;
  __shared__ float w_lds[CT * 65];
  __shared__ double stage[4096];
  const int c = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x;
  const int t0 = c * CT, nt = min(CT, T - t0);
  const long tok0 = (long)b * T + t0;
  for (int i = tid; i < nt * R; i += 256) w_lds[(i / R) * 65 + i % R] = w[tok0 * R + i];
  const double carry = chunk_carry(wcs + (long)b * n_ch * R, c + 1, n_ch, R, stage, tid);
  __syncthreads();
  // W~_t = carry + w_{nt-1} + ... + w_t (token order descending), one fp64
  // chain per rank
  if (tid < R) {
    double run = carry;
#pragma unroll
    for (int t = CT - 1; t >= 0; --t)
      if (t < nt) {
        run += (double)w_lds[t * 65 + tid];
        wt[(tok0 + t) * R + tid] = (float)run;
      }
  }
}

// ---------------------------------------------------------------------------
bool router_fast_fwd_ok(const void* x, bool x_bf16, const float* w_down, const float* h_out, const RouterDims& d) {
  // the projection holds a wave's D / 128 K-steps of x and W_down in registers:
  // at most 16 (R <= 32) or 8 (R <= 64) of them
  const int nks = d.D / 128;
  return x_bf16 && h_out == nullptr && d.D % 128 == 0 && d.R <= 64 && nks <= (d.R <= 32 ? 16 : 8) &&
         (((uintptr_t)x | (uintptr_t)w_down) & 15) == 0;
}

bool router_fast_bwd_ok(const void* x, bool x_bf16, const void* dx, const RouterDims& d) {
  return x_bf16 && d.D % kFastDxSlab == 0 && d.R <= 64 && (((uintptr_t)x | (uintptr_t)dx) & 15) == 0;
}

template <int RT, int EMAX, int TK>
static void fast_fwd_inst(const void* x, const float* w_down, const float* w_up, const float* noise, float ns,
                          float* logits, float* probs, int32_t* idx, float* gates, float* act, float* y, double* ycs,
                          unsigned long long* pub, const RouterDims& d, hipStream_t st) {
  const int n_ch = (d.T + kFastChunk - 1) / kFastChunk;
  // One launch (router_fwd_fused_kernel) where its two-chunk workgroups
  // apply: R <= 32, an even chunk count, and a stream that is not being
  // captured (a captured launch would replay one epoch)
  const bool fused = RT == 1 && pub != nullptr && n_ch % 2 == 0 && !stream_capturing(st);
  // 8 waves split D; a wave takes D / 128 K-steps, held in registers at once
  const int nks = d.D / 128;
  auto go = [&](auto ksw) {
    constexpr int KSW = decltype(ksw)::value;
    // chunks per workgroup: two when the W_down planes leave room in registers
    // (up to 12 K-steps: 226 VGPRs, one 8-wave workgroup per CU) and the grid
    // still has a workgroup per CU, so the grid runs in one round
    constexpr int NCW = KSW * RT <= 12 ? 2 : 1;
    const int nc = (NCW > 1 && (long)((n_ch + 1) / 2) * d.B >= 256) ? 2 : 1;
    if constexpr (NCW == 2 && RT == 1) {
      if (fused) {
        NAYLIS_TIMED("router_fwd", st,
                     hipLaunchKernelGGL((router_fwd_fused_kernel<RT, KSW, EMAX, TK>), dim3(n_ch / 2, d.B), dim3(512),
                                        0, st, (const bf16_t*)x, w_down, w_up, noise, ns, d.noise_kind, logits, probs,
                                        idx, gates, act, pub, next_launch_epoch(), d.T, d.D, d.R, d.E, d.topk,
                                        n_ch, one_launch_spin_limit(-1)));
        return true;
      }
    }
    if (nc == 2)
      NAYLIS_TIMED("router_proj", st,
                   hipLaunchKernelGGL((router_proj_kernel<RT, KSW, NCW>), dim3((n_ch + NCW - 1) / NCW, d.B),
                                      dim3(512), 0, st, (const bf16_t*)x, w_down, y, ycs, d.T, d.D, d.R, n_ch));
    else
      NAYLIS_TIMED("router_proj", st,
                   hipLaunchKernelGGL((router_proj_kernel<RT, KSW, 1>), dim3(n_ch, d.B), dim3(512), 0, st,
                                      (const bf16_t*)x, w_down, y, ycs, d.T, d.D, d.R, n_ch));
    return false;
  };
  bool one_launch;
  if (nks <= 2)
    one_launch = go(std::integral_constant<int, 2>{});
  else if (nks <= 4)
    one_launch = go(std::integral_constant<int, 4>{});
  else if (nks <= 8)
    one_launch = go(std::integral_constant<int, 8>{});
  else if constexpr (RT == 1) {
    if (nks <= 12)
      one_launch = go(std::integral_constant<int, 12>{});
    else
      one_launch = go(std::integral_constant<int, 16>{});
  } else {
    one_launch = go(std::integral_constant<int, 16 / RT>{});  // router_fast_fwd_ok bounds nks by 16 / RT
  }
  if (one_launch) return;
  NAYLIS_TIMED("router_head", st,
               hipLaunchKernelGGL((router_head_kernel<EMAX, TK>), dim3(n_ch, d.B), dim3(256), 0, st, y, ycs, w_up,
                                  noise, ns, d.noise_kind, logits, probs, idx, gates, act, d.T, d.R, d.E, d.topk,
                                  n_ch));
}

template <int RT>
static void fast_fwd_rt(const void* x, const float* w_down, const float* w_up, const float* noise, float ns,
                        float* logits, float* probs, int32_t* idx, float* gates, float* act, float* y, double* ycs,
                        unsigned long long* pub, const RouterDims& d, hipStream_t st) {
  if (d.E <= 8 && d.topk <= 2)
    fast_fwd_inst<RT, 8, 2>(x, w_down, w_up, noise, ns, logits, probs, idx, gates, act, y, ycs, pub, d, st);
  else if (d.E <= 8)
    fast_fwd_inst<RT, 8, 8>(x, w_down, w_up, noise, ns, logits, probs, idx, gates, act, y, ycs, pub, d, st);
  else if (d.E <= 32)
    fast_fwd_inst<RT, 32, 8>(x, w_down, w_up, noise, ns, logits, probs, idx, gates, act, y, ycs, pub, d, st);
  else
    fast_fwd_inst<RT, 64, 8>(x, w_down, w_up, noise, ns, logits, probs, idx, gates, act, y, ycs, pub, d, st);
}

void launch_router_fast_fwd(const void* x, const float* w_down, const float* w_up, const float* noise,
                            float noise_scale, float* logits, float* probs, int32_t* top_idx, float* top_gates,
                            float* act, float* y, double* ycs, unsigned long long* pub, const RouterDims& d,
                            hipStream_t st) {
  if (d.R <= 32)
    fast_fwd_rt<1>(x, w_down, w_up, noise, noise_scale, logits, probs, top_idx, top_gates, act, y, ycs, pub, d, st);
  else
    fast_fwd_rt<2>(x, w_down, w_up, noise, noise_scale, logits, probs, top_idx, top_gates, act, y, ycs, pub, d, st);
}

// The fused prologue (two memory rounds and the carry chains) is paid once
// per workgroup round: fuse only while the grid fits two workgroups per CU
// (LDS: 59 KB per workgroup), where it replaces a whole launch.
static int device_cus() {
  static std::atomic<int> cached[64] = {};  // per device; a racing first call stores the same value
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64 && n > 0) cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

bool router_fast_dx_fuses_scan(const RouterDims& d) {
  const long ranges = ((long)d.B * d.T + kFastDxRange - 1) / kFastDxRange;
  return d.R <= 32 && d.T % kFastDxRange == 0 && ranges * (d.D / kFastDxSlab) <= 2L * device_cus();
}

void launch_router_fast_dx(const void* x, const float* wt, const float* w, const double* wcs, const float* w_down,
                           const void* dx_in, void* dx, float* dwd_part, bool fuse_scan, const RouterDims& d,
                           hipStream_t st) {
  const long ntok = (long)d.B * d.T;
  const int n_ch = (d.T + kFastChunk - 1) / kFastChunk;
  const dim3 grid((unsigned)((ntok + kFastDxRange - 1) / kFastDxRange), d.D / kFastDxSlab);
  if (fuse_scan)
    NAYLIS_TIMED("router_bwd_dx", st,
                 hipLaunchKernelGGL((router_dx_fast_kernel<1, true>), grid, dim3(256), 0, st, (const bf16_t*)x, wt,
                                    w_down, (const bf16_t*)dx_in, (bf16_t*)dx, dwd_part, d.D, d.R, ntok, w, wcs, d.T,
                                    n_ch));
  else if (d.R <= 32)
    NAYLIS_TIMED("router_bwd_dx", st,
                 hipLaunchKernelGGL((router_dx_fast_kernel<1, false>), grid, dim3(256), 0, st, (const bf16_t*)x, wt,
                                    w_down, (const bf16_t*)dx_in, (bf16_t*)dx, dwd_part, d.D, d.R, ntok, w, wcs, d.T,
                                    n_ch));
  else
    NAYLIS_TIMED("router_bwd_dx", st,
                 hipLaunchKernelGGL((router_dx_fast_kernel<2, false>), grid, dim3(256), 0, st, (const bf16_t*)x, wt,
                                    w_down, (const bf16_t*)dx_in, (bf16_t*)dx, dwd_part, d.D, d.R, ntok, w, wcs, d.T,
                                    n_ch));
}

}  // namespace naylis

namespace naylis {

template <int EMAX, int TK>
static void fast_token(const float* act, const float* probs, const int32_t* idx, const float* gates, const float* dg,
                       const float* dp, const float* dl, const float* w_up, float* w, double* wcs, float* dwup_part,
                       const RouterDims& d, hipStream_t st) {
  const int n_ch = (d.T + kFastChunk - 1) / kFastChunk;
  NAYLIS_TIMED("router_bwd_token", st,
               hipLaunchKernelGGL((router_bwd_token_fast_kernel<EMAX, TK>), dim3(n_ch, d.B), dim3(256), 0, st, act,
                                  probs, idx, gates, dg, dp, dl, w_up, w, wcs, dwup_part, d.T, d.R, d.E, d.topk,
                                  n_ch, d.dp_stride));
}

int launch_router_fast_scan(const float* act, const float* probs, const int32_t* idx, const float* gates,
                            const float* dg, const float* dp, const float* dl, const float* w_up, float* w,
                            double* wcs, float* wt, float* dwup_part, bool fuse_scan, const RouterDims& d,
                            hipStream_t st) {
  if (d.E <= 8 && d.topk <= 2)
    fast_token<8, 2>(act, probs, idx, gates, dg, dp, dl, w_up, w, wcs, dwup_part, d, st);
  else if (d.E <= 8)
    fast_token<8, 8>(act, probs, idx, gates, dg, dp, dl, w_up, w, wcs, dwup_part, d, st);
  else if (d.E <= 32)
    fast_token<32, 8>(act, probs, idx, gates, dg, dp, dl, w_up, w, wcs, dwup_part, d, st);
  else
    fast_token<64, 8>(act, probs, idx, gates, dg, dp, dl, w_up, w, wcs, dwup_part, d, st);
  const int n_ch = (d.T + kFastChunk - 1) / kFastChunk;
  if (!fuse_scan)  // else the dx kernel forms W~ itself
    NAYLIS_TIMED("router_bwd_scan", st,
                 hipLaunchKernelGGL(router_wtilde_kernel, dim3(n_ch, d.B), dim3(256), 0, st, w, wcs, wt, d.T, d.R,
                                    n_ch));
  return d.B * n_ch;  // dW_up partials written
}

}  // namespace naylis
