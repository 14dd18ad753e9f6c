// Decode step of the MoM read (gfx950): one new token per sequence against a
// running prefix-sum state and an fp8 bank.
//
// The reference forms the prefix mean over the whole sequence on every
// forward (model.py:169-176) and describes the O(1) running-sum form only in
// a docstring (model.py:172-173).  Here the state S_b = sum_{s<t} x_s is kept
// in fp64, so fp32(S + x_t) is exactly the fp32 cumsum the reference's CPU
// forward computes, for any prior length, and one launch does
//   S' = S + x_t;  h = fp32(S') / fp32(t+1);  a = tanh(W_down h);
//   logits = W_up a;  (idx, gates) = top-k + softmax of the top-k logits;
//   o[h] = softmax_n(q_h . k_n / sqrt(hd) + log gate(n)) v_n over the slots
//   of the selected blocks,
// with K / V stored as OCP fp8 e4m3 (e4m3fn: bias 7, max 448, no infinities)
// and one fp32 scale per slot row: k_n = k_scale[n] * e4m3(k8[n]).
//
// Grid (head groups, sequences), four waves per workgroup.  Every workgroup
// of a sequence updates the state and runs the router (each wave a quarter of
// the ranks, lanes stride D, a fixed-order reduction per rank; W_down is read
// from L2 by every workgroup), so no workgroup waits on another; the one with
// head group 0 writes the new state and the selection.  Then wave w reads head
// 4 g + w: lanes own slots for q . k (every lane holds the q row, a k row is
// four 16-byte loads), max / sum are cross-lane, and for p . v lanes own
// (an eighth of the slots) x (an eighth of the features).  fp8 codes are
// widened with the gfx950 packed conversion v_cvt_pk_f32_fp8 (OCP e4m3 on
// this target; the tests compare the result with torch's float8_e4m3fn).
#include <stdint.h>

#include <type_traits>

#include "common.h"
#include "launch.h"
#include "timing.h"

namespace naylis {

// round-to-nearest-even fp32 -> e4m3fn code, from the format's bit layout:
// normal values 2^(e-7) (1 + m/8) for e in 1..15 (e = 15, m = 7 is NaN),
// subnormals m 2^-9.  Finite values beyond the rounding boundary of 448
// saturate to 448 (the quantizer never produces them).
__device__ __forceinline__ uint32_t e4m3fn_encode(float x) {
  const uint32_t sign = (__float_as_uint(x) >> 31) << 7;
  const float a = fabsf(x);
  if (!(a == a)) return 0x7f;
  if (a >= 464.f) return sign | 0x7e;
  int e = (int)((__float_as_uint(a) >> 23) & 255) - 127;
  if (e < -6) e = -6;                                              // subnormal quantum 2^-9
  const float q = __uint_as_float((uint32_t)(e - 3 + 127) << 23);  // quantum of the binade: 2^(e-3)
  const float r = __builtin_rintf(a / q) * q;                      // a / q is exact; rint rounds ties to even
  if (r == 0.f) return sign;
  const int er = (int)((__float_as_uint(r) >> 23) & 255) - 127;
  uint32_t code;
  if (er < -6)
    code = (uint32_t)(r * 512.f);  // subnormal: m = r / 2^-9
  else
    code = ((uint32_t)(er + 7) << 3) | ((__float_as_uint(r) >> 20) & 7);
  return sign | (code > 0x7e ? 0x7e : code);
}

// per slot row: scale = amax / 448 (1 for an all-zero row), code = e4m3fn(x / scale)
__global__ __launch_bounds__(256) void bank_quant_fp8_kernel(const bf16_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                             float* __restrict__ scale, int D) {
  __shared__ float red[4];
  const long row = blockIdx.x;
  const bf16_t* p = src + row * D;
  float amax = 0.f;
  for (int i = threadIdx.x; i < D; i += 256) amax = fmaxf(amax, fabsf(bf16_to_f32(p[i])));
  for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = amax > 0.f ? amax / 448.f : 1.f;
  if (threadIdx.x == 0) scale[row] = s;
  for (int i = threadIdx.x; i < D; i += 256) dst[row * D + i] = (uint8_t)e4m3fn_encode(bf16_to_f32(p[i]) / s);
}

// four e4m3 codes (bytes of c, low first) -> fp32
__device__ __forceinline__ void fp8x4_to_f32(uint32_t c, float* f) {
  const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)c, false);
  const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)c, true);
  f[0] = lo[0];
  f[1] = lo[1];
  f[2] = hi[0];
  f[3] = hi[1];
}

template <typename XT>
__device__ __forceinline__ double load_x(const XT* p) {
  if constexpr (std::is_same<XT, float>::value)
    return (double)*p;
  else
    return (double)bf16_to_f32(*p);
}

template <int HD, int TK, typename XT>
__global__ __launch_bounds__(256) void decode_step_kernel(
    const double* __restrict__ state_in, double* __restrict__ state_out, const int32_t* __restrict__ t_prev,
    const XT* __restrict__ x_new, const float* __restrict__ w_down, const float* __restrict__ w_up,
    const bf16_t* __restrict__ q_new, const uint8_t* __restrict__ k8, const uint8_t* __restrict__ v8,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale, bf16_t* __restrict__ out,
    int32_t* __restrict__ top_idx, float* __restrict__ top_gates, int D, int H, int R, int E, int block_size,
    int topk, float alpha) {
  static_assert(HD == 32 || HD == 64 || HD == 128, "head dim");
  constexpr int FPL = HD / 8;  // features per lane in p . v
  __shared__ float h_lds[kDecodeMaxD];
  __shared__ float a_lds[kDecodeMaxRank];
  __shared__ int sel_lds[TK];
  __shared__ float lgate_lds[TK];
  __shared__ float p_lds[4][kDecodeMaxSlots];  // per wave: p (then p v_scale) of its head's slots
  const int g = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // ---- running sum and prefix mean: one fp64 add, one rounding to fp32, IEEE division
  const float den = (float)(t_prev[b] + 1);
  for (int d = tid; d < D; d += 256) {
    const double sv = state_in[(long)b * D + d] + load_x(x_new + (long)b * D + d);
    if (g == 0) state_out[(long)b * D + d] = sv;
    h_lds[d] = (float)sv / den;
  }
  __syncthreads();
  // ---- a = tanh(W_down h): wave w takes ranks w, w + 4, ...; lane sums d = 4 lane + 256 j, then a fixed tree
  for (int r = wave; r < R; r += 4) {
    const float* wr = w_down + (long)r * D;
    float acc = 0.f;
#pragma unroll 4
    for (int d = 4 * lane; d < D; d += 256) {
      const float4 w4 = *reinterpret_cast<const float4*>(wr + d);
      acc = fmaf(w4.x, h_lds[d], acc);
      acc = fmaf(w4.y, h_lds[d + 1], acc);
      acc = fmaf(w4.z, h_lds[d + 2], acc);
      acc = fmaf(w4.w, h_lds[d + 3], acc);
    }
    for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (lane == 0) a_lds[r] = tanhf(acc);
  }
  __syncthreads();
  // ---- logits (lane = expert), top-k (ties to the lower id), gates: wave 0
  if (wave == 0) {
    float lg = -INFINITY;
    if (lane < E) {
      lg = 0.f;
      const float* wu = w_up + (long)lane * R;
      for (int r = 0; r < R; ++r) lg = fmaf(wu[r], a_lds[r], lg);
    }
    bool taken = lane >= E;
    float val[TK];
    int sel[TK];
#pragma unroll
    for (int k = 0; k < TK; ++k) {
      if (k < topk) {
        float bv = taken ? -INFINITY : lg;
        int bi = taken ? 0x7fffffff : lane;
        for (int o = 32; o >= 1; o >>= 1) {
          const float ov = __shfl_xor(bv, o, 64);
          const int oi = __shfl_xor(bi, o, 64);
          if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
          }
        }
        val[k] = bv;
        sel[k] = bi;
        taken |= lane == bi;
      }
    }
    if (lane == 0) {
      float gs = 0.f;
#pragma unroll
      for (int k = 0; k < TK; ++k)
        if (k < topk) gs += expf(val[k] - val[0]);
#pragma unroll
      for (int k = 0; k < TK; ++k) {
        if (k < topk) {
          const float gv = expf(val[k] - val[0]) / gs;
          sel_lds[k] = sel[k];
          lgate_lds[k] = log2f(fmaxf(gv, 1e-9f));
          if (g == 0) {
            top_idx[(long)b * topk + k] = sel[k];
            top_gates[(long)b * topk + k] = gv;
          }
        }
      }
    }
  }
  __syncthreads();

  // ---- read of head 4 g + wave over the top-k blocks (distinct ids: top-k of distinct experts)
  const int h = 4 * g + wave;
  if (h >= H) return;
  const long Dk = (long)H * HD;
  float qv[HD];
  {
    const bf16_t* qp = q_new + ((long)b * H + h) * HD;
#pragma unroll
    for (int i = 0; i < HD; i += 8) {
      const uint4 u = *reinterpret_cast<const uint4*>(qp + i);
      const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qv[i + 2 * e] = __uint_as_float(w4[e] << 16);
        qv[i + 2 * e + 1] = __uint_as_float(w4[e] & 0xffff0000u);
      }
    }
  }
  const int nslots = topk * block_size;
  float* pw = p_lds[wave];
  float m = -INFINITY;
#pragma unroll 2
  for (int u0 = 0; u0 < nslots; u0 += 64) {
    const int u = u0 + lane;
    if (u < nslots) {
      const int k = u / block_size;
      const long n = (long)sel_lds[k] * block_size + (u - k * block_size);
      const uint8_t* kr = k8 + n * Dk + (long)h * HD;
      float dot = 0.f;
#pragma unroll
      for (int i = 0; i < HD; i += 16) {
        const uint4 c = *reinterpret_cast<const uint4*>(kr + i);
        const uint32_t w4[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float f[4];
          fp8x4_to_f32(w4[e], f);
#pragma unroll
          for (int j = 0; j < 4; ++j) dot = fmaf(qv[i + 4 * e + j], f[j], dot);
        }
      }
      const float s = fmaf(dot * k_scale[n], alpha, lgate_lds[k]);
      pw[u] = s;
      m = fmaxf(m, s);
    }
  }
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  float l = 0.f;
  for (int u = lane; u < nslots; u += 64) {
    const int k = u / block_size;
    const long n = (long)sel_lds[k] * block_size + (u - k * block_size);
    const float p = __builtin_amdgcn_exp2f(pw[u] - m);
    l += p;
    pw[u] = p * v_scale[n];
  }
  for (int o = 32; o >= 1; o >>= 1) l += __shfl_xor(l, o, 64);
  // the p . v phase reads entries other lanes of this wave wrote
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // p . v: lane = (slot phase sp, feature group fo); slots sp, sp + 8, ...
  const int sp = lane >> 3, fo = (lane & 7) * FPL;
  float acc[FPL];
#pragma unroll
  for (int j = 0; j < FPL; ++j) acc[j] = 0.f;
#pragma unroll 4
  for (int u = sp; u < nslots; u += 8) {
    const int k = u / block_size;
    const long n = (long)sel_lds[k] * block_size + (u - k * block_size);
    const float pv = pw[u];
    const uint8_t* vr = v8 + n * Dk + (long)h * HD + fo;
    uint32_t c[FPL / 4];
    if constexpr (FPL == 4) {
      c[0] = *reinterpret_cast<const uint32_t*>(vr);
    } else if constexpr (FPL == 8) {
      const uint2 c2 = *reinterpret_cast<const uint2*>(vr);
      c[0] = c2.x;
      c[1] = c2.y;
    } else {
      const uint4 c4 = *reinterpret_cast<const uint4*>(vr);
      c[0] = c4.x;
      c[1] = c4.y;
      c[2] = c4.z;
      c[3] = c4.w;
    }
#pragma unroll
    for (int e = 0; e < FPL / 4; ++e) {
      float f[4];
      fp8x4_to_f32(c[e], f);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[4 * e + j] = fmaf(pv, f[j], acc[4 * e + j]);
    }
  }
  // sum the eight slot phases (lanes differing in bits 3..5), fixed order
#pragma unroll
  for (int j = 0; j < FPL; ++j) {
    acc[j] += __shfl_xor(acc[j], 8, 64);
    acc[j] += __shfl_xor(acc[j], 16, 64);
    acc[j] += __shfl_xor(acc[j], 32, 64);
  }
  if (sp == 0) {
    const float inv = 1.f / l;
    bf16_t* op = out + ((long)b * H + h) * HD + fo;
#pragma unroll
    for (int j = 0; j < FPL; ++j) op[j] = f32_to_bf16(acc[j] * inv);
  }
}

hipError_t launch_bank_quant_fp8(const void* k, const void* v, uint8_t* k8, uint8_t* v8, float* k_scale,
                                 float* v_scale, int L, int D, hipStream_t st) {
  NAYLIS_TIMED("bank_quant_fp8", st,
               hipLaunchKernelGGL(bank_quant_fp8_kernel, dim3(L), dim3(256), 0, st, (const bf16_t*)k, k8, k_scale, D));
  NAYLIS_TIMED("bank_quant_fp8", st,
               hipLaunchKernelGGL(bank_quant_fp8_kernel, dim3(L), dim3(256), 0, st, (const bf16_t*)v, v8, v_scale, D));
  return hipGetLastError();
}

hipError_t launch_decode_step(const double* state_in, double* state_out, const int32_t* t_prev, const void* x_new,
                              bool x_f32, const float* w_down, const float* w_up, const void* q_new,
                              const uint8_t* k8, const uint8_t* v8, const float* k_scale, const float* v_scale,
                              void* out, int32_t* top_idx, float* top_gates, const DecodeDims& d, hipStream_t st) {
  const float alpha = (float)(1.0 / __builtin_sqrt((double)d.HD)) * kLog2e;
  const dim3 grid((d.H + 3) / 4, d.B);
  hipError_t err = hipErrorInvalidValue;
  auto go = [&](auto hd, auto tk, auto xt) {
    constexpr int HD = decltype(hd)::value;
    constexpr int TK = decltype(tk)::value;
    using XT = decltype(xt);
    NAYLIS_TIMED("decode_step", st,
                 hipLaunchKernelGGL((decode_step_kernel<HD, TK, XT>), grid, dim3(256), 0, st, state_in, state_out,
                                    t_prev, (const XT*)x_new, w_down, w_up, (const bf16_t*)q_new, k8, v8, k_scale,
                                    v_scale, (bf16_t*)out, top_idx, top_gates, d.D, d.H, d.R, d.E, d.block_size,
                                    d.topk, alpha));
    err = hipGetLastError();
  };
  auto by_x = [&](auto hd, auto tk) {
    if (x_f32)
      go(hd, tk, float{});
    else
      go(hd, tk, bf16_t{});
  };
  auto by_k = [&](auto hd) {
    if (d.topk <= 2)
      by_x(hd, std::integral_constant<int, 2>{});
    else
      by_x(hd, std::integral_constant<int, 8>{});
  };
  if (d.HD == 32)
    by_k(std::integral_constant<int, 32>{});
  else if (d.HD == 64)
    by_k(std::integral_constant<int, 64>{});
  else if (d.HD == 128)
    by_k(std::integral_constant<int, 128>{});
  return err;
}

}  // namespace naylis
