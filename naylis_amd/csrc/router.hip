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
#include <algorithm>

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

// One element of x, raw bits, through a buffer resource (byte offsets), and
// its fp32 value.  Loads and conversions are kept apart so that a run of
// loads is not broken up by waits for each conversion's operand.
template <typename XT>
__device__ __forceinline__ uint32_t bload_raw(__amdgpu_buffer_rsrc_t r, int voff, int soff);
template <>
__device__ __forceinline__ uint32_t bload_raw<float>(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
template <>
__device__ __forceinline__ uint32_t bload_raw<bf16_t>(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}
template <typename XT>
__device__ __forceinline__ float raw_to_f32(uint32_t u) {
  return sizeof(XT) == 2 ? __uint_as_float(u << 16) : __uint_as_float(u);
}

template <typename XT>
__device__ __forceinline__ float load_x32(const XT* p);
template <>
__device__ __forceinline__ float load_x32<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_x32<bf16_t>(const bf16_t* p) { return bf16_to_f32(*p); }

// Eight consecutive elements of x as fp32 (16-byte aligned vector loads).
__device__ __forceinline__ void load8(const bf16_t* p, float (&v)[8]) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[2 * e] = __uint_as_float(w[e] << 16);
    v[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
  }
}
__device__ __forceinline__ void load8(const float* p, float (&v)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = a[e];
    v[4 + e] = b[e];
  }
}

// (1) chunk column sums, fp64: csum[b][c][d] (exact for bf16 input).
// One wave per (512 features, chunk, b); thread = 8 consecutive features.
// Rows are loaded in batches whose addresses are clamped to the chunk's last
// row, so a batch's loads are all in flight together.  vec: rows are 16-byte
// aligned (D % 8 == 0 and an aligned base).
template <typename XT>
__global__ __launch_bounds__(64) void router_chunk_sums_kernel(const XT* __restrict__ x, double* __restrict__ csum,
                                                               int T, int D, int n_chunks, int vec) {
  constexpr int TB = sizeof(XT) == 2 ? 16 : 8;  // rows per load batch
  const int d = (blockIdx.x * 64 + threadIdx.x) * 8;
  const int c = blockIdx.y;
  const int b = blockIdx.z;
  if (d >= D) return;
  const int t0 = c * kRouterChunk, nt = min(T - t0, kRouterChunk);
  const XT* base = x + ((long)b * T + t0) * D + d;
  double s[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) s[e] = 0.0;
  if (vec) {
#pragma unroll
    for (int tb = 0; tb < kRouterChunk; tb += TB) {
      float v[TB][8];
#pragma unroll
      for (int t = 0; t < TB; ++t) load8(base + (long)min(tb + t, nt - 1) * D, v[t]);
#pragma unroll
      for (int t = 0; t < TB; ++t)
        if (tb + t < nt) {
#pragma unroll
          for (int e = 0; e < 8; ++e) s[e] += (double)v[t][e];
        }
    }
  } else {
    for (int t = 0; t < nt; ++t)
      for (int e = 0; e < 8; ++e)
        if (d + e < D) s[e] += load_x64<XT>(base + (long)t * D + e);
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
// Wave w owns a quarter of the features (FW of them, a multiple of 64) and
// walks it in 64-feature passes, independently of the other waves: lane j
// scans feature f = w*FW + 64p + j over the chunk from the fp64 carry into a
// wave-private LDS tile h[t][j], then the wave accumulates z = h W_down^T
// over those 64 features with fp32 MFMA (v_mfma_f32_32x32x2f32: lane l
// holds A[l%32][l/32] and B[l/32][l%32]).  The product's K order is chosen
// so that K step kk of lane half hl is feature 32hl + kk of the pass: each
// lane's W_down operand is 32 consecutive floats of one row, loaded straight
// into registers.  Two register sets alternate, so a pass's loads are in
// flight during the previous pass.  The 4 per-wave partial z tiles are
// summed in LDS in a fixed order at the end.
//
// h = fp32(S) / fp32(t+1) is evaluated as fp32( fp64(fp32(S)) * fp64(1/(t+1)) ).
// For an fp32 numerator a and an integer denominator b <= 2^24 whose quotient
// is a normal fp32 number this is the correctly rounded quotient: a/b is then
// never an fp32 rounding midpoint and lies at least 2^-50 (relative) away from
// every midpoint, while the fp64 product is within 2^-52 (relative) of a/b,
// so both round alike.  Nonzero subnormal results (where exact ties occur)
// are recomputed with the IEEE fp32 division.
template <typename XT, int EMAX, int TK, bool VECW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void router_fwd_kernel(
    const XT* __restrict__ x, const double* __restrict__ carry, const float* __restrict__ w_down,
    const float* __restrict__ w_up, const float* __restrict__ noise, float noise_scale, int noise_kind,
    float* __restrict__ logits, float* __restrict__ probs, int32_t* __restrict__ top_idx,
    float* __restrict__ top_gates, float* __restrict__ act, float* __restrict__ h_out, int T, int D, int R, int E,
    int topk, int n_chunks) {
  constexpr int CT = kRouterChunk;   // 32 tokens: one MFMA row tile
  constexpr int WP = 65;             // wave tile pitch (floats)
  constexpr int LP = EMAX + 1;
  __shared__ float hw_lds[4][CT * WP];             // per wave: h[token][64 features]; then its z partial
  __shared__ float a_lds[CT * 65];                 // tanh activations [token][rank], R <= 64
  __shared__ float wu_lds[EMAX * 65];              // W_up [block][rank]
  __shared__ float lg_lds[CT * LP];                // logits [token][block]
  __shared__ double rinv_lds[CT];                  // 1 / (t+1) in fp64

  const int c = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const int t0 = c * CT;
  const int nt = min(CT, T - t0);
  const int FW = (((D + 3) / 4 + 63) / 64) * 64;  // features per wave
  const int fw0 = wave * FW;
  float* hw = hw_lds[wave];
  for (int i = tid; i < E * R; i += 256) wu_lds[(i / R) * 65 + i % R] = w_up[i];
  if (tid < CT) rinv_lds[tid] = 1.0 / (double)(t0 + tid + 1);
  __syncthreads();

  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x + ((long)b * T + t0) * D, (uint32_t)(nt * D * sizeof(XT)));
  for (int r0 = 0; r0 < R; r0 += 32) {
    f32x16 acc = f32x16{};
    const float* wrow = w_down + (long)min(r0 + l32, R - 1) * D;
    // one pass's registers: the lane's feature over the chunk (raw x bits),
    // its fp64 carry, and the lane's W_down operand (32 floats)
    auto load_pass = [&](int f0, uint32_t (&xv)[CT], float (&wv)[32], double& run) {
      const int dc = min(f0 + lane, D - 1);
#pragma unroll
      for (int t = 0; t < CT; ++t)
        xv[t] = bload_raw<XT>(xr, dc * (int)sizeof(XT), min(t, nt - 1) * D * (int)sizeof(XT));
      run = carry[((long)b * n_chunks + c) * D + dc];
      const int fb = f0 + 32 * hl;
      if constexpr (VECW) {  // D % 64 == 0 and W_down 16-byte aligned: a lane's 32 are all in or all out
        const float* wp = wrow + (fb < D ? fb : 0);  // past D the h operand is 0
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(wp + 4 * q);
          wv[4 * q] = v[0];
          wv[4 * q + 1] = v[1];
          wv[4 * q + 2] = v[2];
          wv[4 * q + 3] = v[3];
        }
      } else {
#pragma unroll
        for (int kk = 0; kk < 32; ++kk) wv[kk] = wrow[min(fb + kk, D - 1)];  // h is 0 past D
      }
    };
    auto pass = [&](int f0, const uint32_t (&xv)[CT], const float (&wv)[32], double run, uint32_t (&xn)[CT],
                    float (&wn)[32], double& rn, bool more) {
      const int d = f0 + lane;
      const bool dok = d < D;
      __builtin_amdgcn_wave_barrier();  // this wave's previous MFMA reads of hw come first (LDS is in order)
      // ---- scan this lane's feature over the chunk (fp64, rounded once);
      // rows past the chunk's end repeat its last row and are masked
      uint32_t need = 0;  // tokens whose quotient is a nonzero subnormal
#pragma unroll
      for (int t = 0; t < CT; ++t) {
        run += (double)raw_to_f32<XT>(xv[t]);
        const float cs = (float)run;
        const float hv = (float)((double)cs * rinv_lds[t]);
        const bool live = dok && t < nt;
        const bool sub = live && hv != 0.f && fabsf(hv) < 1.17549435e-38f;
        need |= (uint32_t)sub << t;
        hw[t * WP + lane] = sub ? cs : (live ? hv : 0.f);  // sub: numerator, divided below
      }
      // rare path (a loop, so it stays a branch): IEEE division where ties can occur
      while (need) {
        const int t = __builtin_ctz(need);
        need &= need - 1;
        hw[t * WP + lane] = hw[t * WP + lane] / (float)(t0 + t + 1);
      }
      if (h_out != nullptr && r0 == 0 && dok) {
        float* hp = h_out + ((long)b * T + t0) * D + d;
#pragma unroll 1
        for (int t = 0; t < nt; ++t) hp[(long)t * D] = hw[t * WP + lane];
      }
      __builtin_amdgcn_wave_barrier();  // the tile is written before any lane reads it
      if (more) load_pass(f0 + 64, xn, wn, rn);
      // ---- z[t][r] += sum_f h[t][f] Wd[r][f] over the pass's 64 features
      const float* hrow = hw + l32 * WP + 32 * hl;
#pragma unroll
      for (int kk = 0; kk < 32; ++kk) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(hrow[kk], wv[kk], acc, 0, 0, 0);
    };
    uint32_t xa[CT], xb[CT];
    float wa[32], wb[32];
    double ra = 0.0, rb = 0.0;
    load_pass(fw0, xa, wa, ra);
    for (int p = 0; p < FW; p += 128) {
      pass(fw0 + p, xa, wa, ra, xb, wb, rb, p + 64 < FW);
      if (p + 64 >= FW) break;
      pass(fw0 + p + 64, xb, wb, rb, xa, wa, ra, p + 128 < FW);
    }
    // ---- sum the 4 wave partials in a fixed order, tanh, stash
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int v = 0; v < 16; ++v) hw[acc_row(hl, v) * 33 + l32] = acc[v];
    __syncthreads();
    for (int i = tid; i < CT * 32; i += 256) {
      const int t = i >> 5, r = i & 31;
      const float z = ((hw_lds[0][t * 33 + r] + hw_lds[1][t * 33 + r]) + hw_lds[2][t * 33 + r]) + hw_lds[3][t * 33 + r];
      if (t < nt && r0 + r < R) {
        const float a = tanhf(z);
        act[((long)b * T + t0 + t) * R + r0 + r] = a;
        a_lds[t * 65 + r0 + r] = a;
      }
    }
    __syncthreads();  // the z partials are read before the next rank tile's scans overwrite the tiles
  }
  // ---- logits: 8 threads per token, block e handled by thread e % 8
  {
    const int t = tid >> 3, part = tid & 7;
    if (t < nt) {
      const long tok = (long)b * T + t0 + t;
#pragma unroll
      for (int e0 = 0; e0 < EMAX; e0 += 8) {
        const int e = e0 + part;
        if (e < E) {
          float lg = 0.f;
          for (int r = 0; r < R; ++r) lg = fmaf(a_lds[t * 65 + r], wu_lds[e * 65 + r], lg);
          lg_lds[t * LP + e] = lg;
          logits[tok * E + e] = lg;
        }
      }
    }
  }
  __syncthreads();
  // ---- per token: probs, top-k, gates
  if (tid < nt) {
    const long tok = (long)b * T + t0 + tid;
    float lg[EMAX];
#pragma unroll
    for (int e = 0; e < EMAX; ++e) lg[e] = e < E ? lg_lds[tid * LP + e] : 0.f;
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < EMAX; ++e)
      if (e < E) mx = fmaxf(mx, lg[e]);
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
    for (int e = 0; e < EMAX; ++e)
      nz[e] = (e < E) ? (noise ? noisy_logit(lg[e], noise[tok * E + e], noise_scale, noise_kind) : lg[e]) : -INFINITY;
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
// per-workgroup partial of dW_up = dlogits^T a.  A workgroup takes 64 tokens:
// thread j < 64 forms token j's d(logits); then all 256 threads compute the
// 64 x R values of w in token-major order (contiguous stores) and the E x R
// partial of dW_up.
template <int EMAX, int TK>
__global__ __launch_bounds__(256) void router_bwd_token_kernel(
    const float* __restrict__ act, const float* __restrict__ probs, const int32_t* __restrict__ top_idx,
    const float* __restrict__ top_gates, const float* __restrict__ d_gates, const float* __restrict__ d_probs,
    const float* __restrict__ d_logits, const float* __restrict__ w_up, float* __restrict__ w_out,
    float* __restrict__ dwup_part, int T, int R, int E, int topk, long ntok, long dps) {
  constexpr int TT = 64;
  constexpr int NW = (EMAX * 64 + 255) / 256;  // W_up elements per thread
  constexpr int NA = TT * 64 / 256;            // activation elements per thread
  __shared__ float dl_lds[TT * (EMAX + 1)];
  __shared__ float a_lds[TT * 65];
  __shared__ float wu_lds[EMAX * 65];
  const int tid = threadIdx.x;
  const long tok0 = (long)blockIdx.x * TT;
  const int nt = (int)(ntok - tok0 < TT ? ntok - tok0 : TT);
  {
    // all loads first (addresses clamped into range), then the LDS writes
    const int ner = E * R, nar = nt * R;
    float wv[NW], av[NA];
#pragma unroll
    for (int u = 0; u < NW; ++u) wv[u] = w_up[min(tid + u * 256, ner - 1)];
#pragma unroll
    for (int u = 0; u < NA; ++u) av[u] = act[tok0 * R + min(tid + u * 256, nar - 1)];
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      const int i = tid + u * 256;
      if (i < ner) wu_lds[(i / R) * 65 + i % R] = wv[u];
    }
#pragma unroll
    for (int u = 0; u < NA; ++u) {
      const int i = tid + u * 256;
      if (i < TT * R) a_lds[(i / R) * 65 + i % R] = i < nar ? av[u] : 0.f;
    }
  }
  if (tid < TT) {
    const long tok = tok0 + tid;
    float dl[EMAX];
#pragma unroll
    for (int e = 0; e < EMAX; ++e) dl[e] = 0.f;
    if (tid < nt) {
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
  // w[t][r] = (sum_e dl[t][e] W_up[e][r]) (1 - a^2) / (t+1), token-major
  for (int i = tid; i < nt * R; i += 256) {
    const int j = i / R, r = i % R;
    float da = 0.f;
#pragma unroll
    for (int e = 0; e < EMAX; ++e)
      if (e < E) da = fmaf(dl_lds[j * (EMAX + 1) + e], wu_lds[e * 65 + r], da);
    const float a = a_lds[j * 65 + r];
    const float denom = (float)(((tok0 + j) % T) + 1);
    w_out[tok0 * R + i] = da * (1.f - a * a) / denom;
  }
  // partial dW_up[e][r] over this block's tokens (rows past nt are zero)
  for (int i = tid; i < E * R; i += 256) {
    const int e = i / R, r = i % R;
    float acc = 0.f;
#pragma unroll 8
    for (int j = 0; j < TT; ++j) acc = fmaf(dl_lds[j * (EMAX + 1) + e], a_lds[j * 65 + r], acc);
    dwup_part[(long)blockIdx.x * E * R + i] = acc;
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

// Backward (3): dx = W~ W_down and partials of dW_down = W~^T x on fp32 MFMA
// (v_mfma_f32_32x32x2f32: lane l holds A[l%32][l/32] and B[l/32][l%32]).
// Workgroup = (kDxRange tokens, kDxSlab features); wave w owns the 32
// features f0 = slab + 32w.  The range is walked in kDxStep-token steps: x
// and W~ of a step are staged in LDS and the next step's loads are issued
// before the current step's MFMAs.
//   dx^T[f][t] = sum_r W_down[r][f] W~[t][r]   A = W_down^T (registers), with
//       rows permuted (row_perm32) so that each lane ends up holding 16
//       consecutive features of one token; B = W~^T (LDS)
//   dWd[r][f] += sum_t W~[t][r] x[t][f]        A = W~^T (LDS), B = x (LDS)
// The dW_down partial of the range is written once, in fixed order, for a
// deterministic reduction.
constexpr int kDxStep = 64, kDxRange = 256, kDxSlab = 128;

template <typename XT, int RT>  // RT = 32-rank tiles (R <= 32 * RT)
__global__ __launch_bounds__(256) void router_bwd_dx_kernel(const XT* __restrict__ x, const float* __restrict__ wt,
                                                            const float* __restrict__ w_down, XT* __restrict__ dx,
                                                            float* __restrict__ dwd_part, int D, int R, long ntok,
                                                            int vec) {
  constexpr int RW = 32 * RT;                         // staged ranks (zero padded)
  constexpr int RP = RW + 1;                          // W~ tile pitch (floats)
  constexpr int XP = sizeof(XT) == 2 ? 160 : 144;     // x tile pitch (elements)
  constexpr int NWT = kDxStep * RW / 256;             // W~ elements per thread
  constexpr int NXV = kDxStep * kDxSlab / 8 / 256;    // 8-element x vectors per thread
  __shared__ float wt_lds[kDxStep * RP];
  __shared__ __align__(16) XT x_lds[kDxStep * XP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const long tok_beg = (long)blockIdx.x * kDxRange;
  const int slab = blockIdx.y * kDxSlab;
  const int f0 = slab + wave * 32;

  float wa[16 * RT];  // A operand of dx: W_down[2kk + hl][f0 + row_perm32(l32)]
  {
    const int f = min(f0 + row_perm32(l32), D - 1);
#pragma unroll
    for (int kk = 0; kk < 16 * RT; ++kk) {
      const int r = 2 * kk + hl;
      const float w = w_down[(long)min(r, R - 1) * D + f];
      wa[kk] = r < R ? w : 0.f;
    }
  }
  f32x16 accw[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) accw[rt] = f32x16{};

  float wreg[NWT];
  float xreg[NXV][8];
  auto prefetch = [&](long ts) {
    const long lim = ntok * R - 1;
#pragma unroll
    for (int u = 0; u < NWT; ++u) {
      const int i = tid + u * 256, t = i / RW, r = i % RW;
      const long src = (ts + t) * R + min(r, R - 1);
      const float v = wt[src < lim ? src : lim];
      wreg[u] = (r < R && ts + t < ntok) ? v : 0.f;
    }
#pragma unroll
    for (int u = 0; u < NXV; ++u) {
      const int i = tid + u * 256, t = i / (kDxSlab / 8), g = i % (kDxSlab / 8);
      const long tk = min(ts + t, ntok - 1);
      const int f = slab + 8 * g;
      const bool ok = ts + t < ntok;
      if (vec && f + 8 <= D) {
        load8(x + tk * D + f, xreg[u]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) xreg[u][e] = load_x32<XT>(x + tk * D + min(f + e, D - 1));
      }
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (!ok || f + e >= D) xreg[u][e] = 0.f;
    }
  };

  prefetch(tok_beg);
  for (int st = 0; st < kDxRange / kDxStep; ++st) {
    const long ts = tok_beg + st * kDxStep;
    if (ts >= ntok) break;
    __syncthreads();  // the previous step's MFMAs are done with the tiles
#pragma unroll
    for (int u = 0; u < NWT; ++u) {
      const int i = tid + u * 256;
      wt_lds[(i / RW) * RP + i % RW] = wreg[u];
    }
#pragma unroll
    for (int u = 0; u < NXV; ++u) {
      const int i = tid + u * 256, t = i / (kDxSlab / 8), g = i % (kDxSlab / 8);
      XT* dst = x_lds + t * XP + 8 * g;
      if constexpr (sizeof(XT) == 2) {
        uint4 pk;
        uint32_t* w = reinterpret_cast<uint32_t*>(&pk);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[e] = (uint32_t)f32_to_bf16(xreg[u][2 * e]) | ((uint32_t)f32_to_bf16(xreg[u][2 * e + 1]) << 16);
        *reinterpret_cast<uint4*>(dst) = pk;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) dst[e] = xreg[u][e];
      }
    }
    __syncthreads();
    if (st + 1 < kDxRange / kDxStep && ts + kDxStep < ntok) prefetch(ts + kDxStep);

    // ---- dx for the step's two 32-token tiles
#pragma unroll
    for (int tt = 0; tt < kDxStep / 32; ++tt) {
      f32x16 acc = f32x16{};
#pragma unroll
      for (int kk = 0; kk < 16 * RT; ++kk)
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(wa[kk], wt_lds[(tt * 32 + l32) * RP + 2 * kk + hl], acc, 0, 0, 0);
      const long tok = ts + tt * 32 + l32;
      const int fb = f0 + 16 * hl;  // acc[v] = dx[tok][fb + v]
      if (tok < ntok) {
        XT* out = dx + tok * D + fb;
        if (vec && fb + 16 <= D) {
          if constexpr (sizeof(XT) == 2) {
            uint4 pk[2];
            uint32_t* w = reinterpret_cast<uint32_t*>(pk);
#pragma unroll
            for (int e = 0; e < 8; ++e)
              w[e] = (uint32_t)f32_to_bf16(acc[2 * e]) | ((uint32_t)f32_to_bf16(acc[2 * e + 1]) << 16);
            reinterpret_cast<uint4*>(out)[0] = pk[0];
            reinterpret_cast<uint4*>(out)[1] = pk[1];
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
              reinterpret_cast<f32x4*>(out)[q] = f32x4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
          }
        } else {
#pragma unroll
          for (int v = 0; v < 16; ++v)
            if (fb + v < D) {
              if constexpr (sizeof(XT) == 2)
                out[v] = f32_to_bf16(acc[v]);
              else
                out[v] = acc[v];
            }
        }
      }
    }
    // ---- dW_down partial over the step's tokens
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll 8
      for (int kk = 0; kk < kDxStep / 2; ++kk) {
        const int t = 2 * kk + hl;
        const float av = wt_lds[t * RP + rt * 32 + l32];
        float bv;
        if constexpr (sizeof(XT) == 2)
          bv = bf16_to_f32(x_lds[t * XP + wave * 32 + l32]);
        else
          bv = x_lds[t * XP + wave * 32 + l32];
        accw[rt] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, accw[rt], 0, 0, 0);
      }
    }
  }
  // partial[range][r][f], r = rt*32 + acc_row(hl, v), f = f0 + l32
  const int f = f0 + l32;
  if (f < D) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = rt * 32 + acc_row(hl, v);
        if (r < R) dwd_part[((long)blockIdx.x * R + r) * D + f] = accw[rt][v];
      }
  }
}

// The router backward's weight gradients from their fp32 partials, both in one
// launch: workgroups [0, blocks_a) reduce job a (dW_down), the rest job b
// (dW_up).  out[i] = sum over parts of part[p][i]: four lane groups take every
// fourth part in order, then their sums are added in group order, so the
// result does not depend on scheduling.
__global__ __launch_bounds__(256) void router_reduce_kernel(const float* __restrict__ part_a, float* __restrict__ out_a,
                                                             long n_a, int parts_a, int blocks_a,
                                                             const float* __restrict__ part_b, float* __restrict__ out_b,
                                                             long n_b, int parts_b) {
  __shared__ float grp_sum[4][64];
  const bool a = (int)blockIdx.x < blocks_a;
  const float* part = a ? part_a : part_b;
  float* out = a ? out_a : out_b;
  const long n = a ? n_a : n_b;
  const int n_parts = a ? parts_a : parts_b;
  const int o = threadIdx.x & 63, gq = threadIdx.x >> 6;
  const long i = (long)(a ? blockIdx.x : blockIdx.x - blocks_a) * 64 + o;
  float s = 0.f;
  if (i < n) {
    int c = gq;
    for (; c + 60 < n_parts; c += 64) {
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = part[(long)(c + 4 * u) * n + i];
#pragma unroll
      for (int u = 0; u < 16; ++u) s += v[u];
    }
    for (; c + 28 < n_parts; c += 32) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = part[(long)(c + 4 * u) * n + i];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; c < n_parts; c += 4) s += part[(long)c * n + i];
  }
  grp_sum[gq][o] = s;
  __syncthreads();
  if (gq == 0 && i < n) out[i] = ((grp_sum[0][o] + grp_sum[1][o]) + grp_sum[2][o]) + grp_sum[3][o];
}

static void launch_router_reduce2(const float* dwd_part, float* dw_down, long nwd, int parts_d, const float* dwup_part,
                                  float* dw_up, long nwu, int parts_u, hipStream_t st) {
  const int bd = (int)((nwd + 63) / 64), bu = (int)((nwu + 63) / 64);
  NAYLIS_TIMED("router_reduce", st,
               hipLaunchKernelGGL(router_reduce_kernel, dim3(bd + bu), dim3(256), 0, st, dwd_part, dw_down, nwd,
                                  parts_d, bd, dwup_part, dw_up, nwu, parts_u));
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
  w.y = off;  // fast path: y = x W_down^T and its per-chunk fp64 sums
  off += a256((size_t)ntok * d.R * 4);
  w.ycs = off;
  off += a256((size_t)d.B * n_chunks * d.R * 8);
  w.pub = off;  // one-launch fast forward: each 32-token chunk's sums as (v, v ^ epoch) word pairs
  off += a256((size_t)d.B * ((d.T + 31) / 32) * d.R * 16);
  w.fwd_total = off;
  w.w = off;
  off += a256((size_t)ntok * d.R * 4);
  w.wt = off;
  off += a256((size_t)ntok * d.R * 4);
  // sized for the larger of the two paths: 32-token chunks (fast) vs 64 (exact-h)
  w.scan_csum = off;
  off += a256((size_t)d.B * n_chunks * d.R * 8);
  w.dwup_part = off;
  off += a256((size_t)std::max<long>(n_tok_blocks, (long)d.B * n_chunks) * d.E * d.R * 4);
  w.dwd_part = off;
  off += a256((size_t)((ntok + kDxRange - 1) / kDxRange) * d.R * d.D * 4);
  w.total = off;
  return w;
}

template <typename XT, int EMAX, int TK>
static void fwd_launch(const void* x, const float* w_down, const float* w_up, const float* noise, float ns,
                       float* logits, float* probs, int32_t* idx, float* gates, float* act, float* h_out, char* ws,
                       const RouterWs& w, const RouterDims& d, hipStream_t st) {
  const int n_chunks = (d.T + kRouterChunk - 1) / kRouterChunk;
  double* carry = (double*)(ws + w.carry);
  const int dblk = (d.D + 511) / 512;
  const int vec = (d.D % 8 == 0 && ((uintptr_t)x & 15) == 0) ? 1 : 0;
  NAYLIS_TIMED("router_chunk_sums", st,
               hipLaunchKernelGGL((router_chunk_sums_kernel<XT>), dim3(dblk, n_chunks, d.B), dim3(64), 0, st,
                                  (const XT*)x, carry, d.T, d.D, n_chunks, vec));

  const int vecw = (d.D % 64 == 0 && ((uintptr_t)w_down & 15) == 0) ? 1 : 0;
  NAYLIS_TIMED("router_chunk_carry", st,
               hipLaunchKernelGGL(router_chunk_carry_kernel, dim3((d.D + 255) / 256, d.B), dim3(256), 0, st, carry,
                                  d.D, n_chunks));
  if (vecw)
    NAYLIS_TIMED("router_fwd", st,
                 hipLaunchKernelGGL((router_fwd_kernel<XT, EMAX, TK, true>), dim3(n_chunks, d.B), dim3(256), 0, st,
                                    (const XT*)x, carry, w_down, w_up, noise, ns, d.noise_kind, logits, probs, idx,
                                    gates, act, h_out,
                                    d.T, d.D, d.R, d.E, d.topk, n_chunks));
  else
    NAYLIS_TIMED("router_fwd", st,
                 hipLaunchKernelGGL((router_fwd_kernel<XT, EMAX, TK, false>), dim3(n_chunks, d.B), dim3(256), 0, st,
                                    (const XT*)x, carry, w_down, w_up, noise, ns, d.noise_kind, logits, probs, idx,
                                    gates, act, h_out,
                                    d.T, d.D, d.R, d.E, d.topk, n_chunks));
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
  if (router_fast_fwd_ok(x, x_bf16, w_down, h_out, d)) {
    const RouterWs w = plan_router_ws(d);
    launch_router_fast_fwd(x, w_down, w_up, noise, noise_scale, logits, probs, top_idx, top_gates, act,
                           (float*)((char*)ws + w.y), (double*)((char*)ws + w.ycs),
                           (unsigned long long*)((char*)ws + w.pub), d, st);
    return hipGetLastError();
  }
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
  NAYLIS_TIMED("router_bwd_token", st, hipLaunchKernelGGL((router_bwd_token_kernel<EMAX, TK>), dim3((int)((ntok + 63) / 64)), dim3(256), 0, st, act, probs,
                     idx, gates, dg, dp, dl, w_up, w_out, dwup_part, d.T, d.R, d.E, d.topk, ntok, d.dp_stride));
}

template <typename XT>
static void bwd_dx(const void* x, const float* wt, const float* w_down, void* dx, float* dwd_part, const RouterDims& d,
                   hipStream_t st) {
  const long ntok = (long)d.B * d.T;
  const dim3 grid((int)((ntok + kDxRange - 1) / kDxRange), (d.D + kDxSlab - 1) / kDxSlab);
  const int vec = (d.D % 8 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)dx & 15) == 0) ? 1 : 0;
  if (d.R <= 32)
    NAYLIS_TIMED("router_bwd_dx", st,
                 hipLaunchKernelGGL((router_bwd_dx_kernel<XT, 1>), grid, dim3(256), 0, st, (const XT*)x, wt, w_down,
                                    (XT*)dx, dwd_part, d.D, d.R, ntok, vec));
  else
    NAYLIS_TIMED("router_bwd_dx", st,
                 hipLaunchKernelGGL((router_bwd_dx_kernel<XT, 2>), grid, dim3(256), 0, st, (const XT*)x, wt, w_down,
                                    (XT*)dx, dwd_part, d.D, d.R, ntok, vec));
}

hipError_t launch_router_bwd(const void* x, bool x_bf16, const float* w_down, const float* w_up, const float* act,
                             const float* probs, const int32_t* top_idx, const float* top_gates, const float* d_gates,
                             const float* d_probs, const float* d_logits, void* dx, bool dx_accumulate,
                             float* dw_down, float* dw_up, void* ws, const RouterDims& d, hipStream_t st) {
  // accumulation into dx exists on the fast path only (bf16 x, D % 128 == 0);
  // the C ABI rejects other requests before this point
  if (dx_accumulate && !router_fast_bwd_ok(x, x_bf16, dx, d)) return hipErrorInvalidValue;
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
    launch_router_reduce2(dwd_part, dw_down, nwd, 0, dwup_part, dw_up, nwu, 0, st);
    return hipGetLastError();
  }
  const bool fast = router_fast_bwd_ok(x, x_bf16, dx, d);
  if (fast) {
    const bool fuse_scan = router_fast_dx_fuses_scan(d);  // decided once: both launches must agree
    const int n_up = launch_router_fast_scan(act, probs, top_idx, top_gates, d_gates, d_probs, d_logits, w_up, wbuf,
                                             (double*)(base + w.scan_csum), wt, dwup_part, fuse_scan, d, st);
    launch_router_fast_dx(x, wt, wbuf, (const double*)(base + w.scan_csum), w_down, dx_accumulate ? dx : nullptr, dx,
                          dwd_part, fuse_scan, d, st);
    launch_router_reduce2(dwd_part, dw_down, nwd, (int)((ntok + kDxRange - 1) / kDxRange), dwup_part, dw_up, nwu,
                          n_up, st);
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
  const int n_dx_chunks = (int)((ntok + kDxRange - 1) / kDxRange);  // both paths: 256-token ranges
  launch_router_reduce2(dwd_part, dw_down, nwd, n_dx_chunks, dwup_part, dw_up, nwu, n_tok_blocks, st);
  return hipGetLastError();
}

}  // namespace naylis
