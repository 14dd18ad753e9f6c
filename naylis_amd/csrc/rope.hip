// Rotary position embedding of the decoder's attention, fused: transformers'
// apply_rotary_pos_emb, called by the Llama attention of every Naylis decoder
// layer (model.py:279-345), computes in the activation dtype
//     q' = q * cos + rotate_half(q) * sin,   rotate_half(a | b) = (-b | a)
// as five elementwise launches per tensor forward (two products, a negation,
// a concatenation, a sum) and more backward.  Here one pass covers q and k,
// rounding like the reference's ops (each product rounded to the dtype, then
// the sum).
//
// Backward (the transposed rotation): dq = dy * cos + rotate_half^T(dy * sin),
// rotate_half^T(a | b) = (b | -a), again with the products rounded first.
#include "common.h"
#include "timing.h"

namespace naylis {

namespace {

template <typename T>
__device__ __forceinline__ float rnd(float v) {
  if constexpr (sizeof(T) == 2)
    return bf16_to_f32(f32_to_bf16(v));
  else
    return v;
}

}  // namespace

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

// One thread per 8 consecutive features of a (token, head) row: chunks
// 2 * B * S * H * HD / 8 (q's, then k's), consecutive threads on consecutive
// 16-byte pieces.  x (B, S, H, HD); cos / sin (CB, S, HD) with CB = B or 1.
// A thread also reads the partner piece HD / 2 features away (the other half
// of rotate_half).  BWD: x holds dy and the transposed rotation is applied.
template <typename T, int HD, bool BWD>
__global__ __launch_bounds__(256) void rope_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                   const T* __restrict__ cs, const T* __restrict__ sn,
                                                   T* __restrict__ qo, T* __restrict__ ko, long rows_per, int S,
                                                   int H, int cos_batch) {
  constexpr int CPR = HD / 8;   // pieces per row
  constexpr int HALF = HD / 2;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= 2 * rows_per * CPR) return;
  const long row = i / CPR;
  const int c = (int)(i - row * CPR);
  const bool is_k = row >= rows_per;
  const long rr = is_k ? row - rows_per : row;  // (b, s, h) row
  const T* x = (is_k ? k : q) + rr * HD;
  T* y = (is_k ? ko : qo) + rr * HD;
  const long bs = rr / H;                       // b * S + s
  const long b = bs / S, s = bs - b * S;
  const T* crow = cs + ((cos_batch > 1 ? b : 0) * S + s) * HD;
  const T* srow = sn + ((cos_batch > 1 ? b : 0) * S + s) * HD;
  const int e0 = 8 * c;
  const bool lo = e0 < HALF;
  const int p0 = lo ? e0 + HALF : e0 - HALF;   // partner piece
  float xv[8], xp[8], cv[8], sv[8];
  load8(x + e0, xv);
  load8(x + p0, xp);
  load8(crow + e0, cv);
  load8(srow + (BWD ? p0 : e0), sv);
  float out[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    // separate roundings (no fused multiply-add), as the reference's ops
    const float a = rnd<T>(mul_rn(xv[e], cv[e]));
    float t;
    if constexpr (!BWD)
      t = rnd<T>(mul_rn(lo ? -xp[e] : xp[e], sv[e]));  // rotate_half(x)[e] * sin[e]
    else
      t = lo ? rnd<T>(mul_rn(xp[e], sv[e])) : -rnd<T>(mul_rn(xp[e], sv[e]));  // rotate_half^T(dy * sin)[e]
    out[e] = add_rn(a, t);
  }
  store8(y + e0, out);
}

template <typename T, bool BWD>
static hipError_t rope_t(const void* q, const void* k, const void* cs, const void* sn, void* qo, void* ko, long B,
                         int S, int H, int HD, int cos_batch, hipStream_t st) {
  const long rows_per = B * S * H;
  const dim3 grid((unsigned)((2 * rows_per * (HD / 8) + 255) / 256));
#define NAYLIS_ROPE(HDV)                                                                                       \
  case HDV:                                                                                                    \
    NAYLIS_TIMED(BWD ? "rope_bwd" : "rope_fwd", st,                                                           \
                 hipLaunchKernelGGL((rope_kernel<T, HDV, BWD>), grid, dim3(256), 0, st, (const T*)q, (const T*)k, \
                                    (const T*)cs, (const T*)sn, (T*)qo, (T*)ko, rows_per, S, H, cos_batch));   \
    break;
  switch (HD) {
    NAYLIS_ROPE(32)
    NAYLIS_ROPE(64)
    NAYLIS_ROPE(128)
    default:
      return hipErrorInvalidValue;
  }
#undef NAYLIS_ROPE
  return hipGetLastError();
}

hipError_t launch_rope(const void* q, const void* k, const void* cs, const void* sn, void* qo, void* ko, bool bf16,
                       bool bwd, long B, int S, int H, int HD, int cos_batch, hipStream_t st) {
  if (B * S * H == 0) return hipSuccess;
  if (bf16)
    return bwd ? rope_t<bf16_t, true>(q, k, cs, sn, qo, ko, B, S, H, HD, cos_batch, st)
               : rope_t<bf16_t, false>(q, k, cs, sn, qo, ko, B, S, H, HD, cos_batch, st);
  return bwd ? rope_t<float, true>(q, k, cs, sn, qo, ko, B, S, H, HD, cos_batch, st)
             : rope_t<float, false>(q, k, cs, sn, qo, ko, B, S, H, HD, cos_batch, st);
}

}  // namespace naylis
