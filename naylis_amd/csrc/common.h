// Shared device helpers for the gfx950 (CDNA4) MoM kernels.
//
// MFMA conventions used everywhere (v_mfma_f32_32x32x16_bf16, wave64),
// checked on MI355X hardware:
//   A operand (32 x 16, bf16x8 per lane):  lane l holds A[l%32][8*(l/32) + e]
//   B operand (16 x 32, bf16x8 per lane):  lane l holds B[8*(l/32) + e][l%32]
//   D (32 x 32, f32x16 per lane):          lane l, reg v holds
//                                           D[8*(v/4) + 4*(l/32) + v%4][l%32]
// So the accumulator of one product has "column = lane" and "rows spread
// over registers"; the K index of the next product can be any fixed
// permutation as long as both operands use it.  Two permutations follow:
//
//  * slot_perm16(p): position p of a 16-wide K group holds element
//    8*((p%8)/4) + 4*(p/8) + p%4, i.e. bits 2 and 3 of p swapped.  With it,
//    registers 8*h .. 8*h+7 of an accumulator tile are exactly the bf16x8
//    B fragment for K-step h of the next product (no cross-lane moves).
//  * row_perm32(r): A-operand row r of a 32-row tile computes output
//    feature row_perm32(r) = 16*bit2(r) + 4*(r>>3) + (r&3); with it lane
//    group g (= l/32) of the product holds features 16*g .. 16*g+15 in
//    registers 0..15, so each lane stores 64 contiguous bytes.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace naylis {

// fp32 product / sum rounded on their own: HIP compiles with fp contraction
// on, and __fmul_rn / __fadd_rn are plain operators there, so a product
// followed by a sum may become one fused multiply-add.  These carry no
// contraction flag, which keeps the two roundings of a torch expression.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

// Routing logit perturbed as model.py:209-213 does it: logit + scale * g with
// the product and the sum rounded separately (two torch ops).  kind 0: g is
// the given noise; kind 1: the buffer holds the uniform draw u (torch.rand)
// and g = -log(-log(u + 1e-9) + 1e-9), the Gumbel transform, each step an
// fp32 operation like the reference's elementwise ops.
__device__ __forceinline__ float noisy_logit(float lg, float nz, float scale, int kind) {
  if (kind == 1) nz = -logf(add_rn(-logf(add_rn(nz, 1e-9f)), 1e-9f));
  return add_rn(lg, mul_rn(scale, nz));
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t bf16_t;  // bf16 storage in global memory
typedef short v4i16 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__host__ __device__ constexpr int slot_perm16(int p) {
  return (p & ~12) | ((p & 4) << 1) | ((p & 8) >> 1);
}

__host__ __device__ constexpr int row_perm32(int r) {
  return (((r >> 2) & 1) << 4) | ((r >> 3) << 2) | (r & 3);
}

// Inverse of row_perm32: the A-operand row that computes feature f.
__host__ __device__ constexpr int row_unperm32(int f) {
  return (((f >> 2) & 3) << 3) | ((f >> 4) << 2) | (f & 3);
}

// Row of the 32x32 accumulator held by (lane group g, register v).
__device__ __forceinline__ int acc_row(int g, int v) { return 8 * (v >> 2) + 4 * g + (v & 3); }

// Raw buffer resource over [base, base + bytes): buffer loads take a per-lane
// VGPR byte offset plus a wave-uniform SGPR byte offset, so a run of loads at
// uniform strides needs no per-load 64-bit address registers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ float bf16_to_f32(bf16_t u) {
  return __uint_as_float(((uint32_t)u) << 16);
}

__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  __bf16 b = (__bf16)f;  // round to nearest even
  return __builtin_bit_cast(bf16_t, b);
}

// Pack 8 fp32 values (registers lo..lo+7 of an accumulator) to a bf16x8 fragment.
__device__ __forceinline__ bf16x8 pack8(const f32x16& acc, int lo) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (__bf16)acc[lo + e];
  return r;
}

// hi = pack8(acc, lo) and the bf16 remainder lo_out = bf16(acc - float(hi)):
// hi + lo_out carries acc to ~2^-16 relative.  float(hi) is read back from the
// packed bits (low half << 16, high half masked), so each value costs one
// subtraction and half a conversion beyond hi.
__device__ __forceinline__ void pack8_hilo(const f32x16& acc, int lo, bf16x8& hi, bf16x8& lo_out) {
  hi = pack8(acc, lo);
  const uint4 hb = __builtin_bit_cast(uint4, hi);
  const uint32_t w[4] = {hb.x, hb.y, hb.z, hb.w};
  bf16x8 r;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    r[2 * p] = (__bf16)(acc[lo + 2 * p] - __uint_as_float(w[p] << 16));
    r[2 * p + 1] = (__bf16)(acc[lo + 2 * p + 1] - __uint_as_float(w[p] & 0xffff0000u));
  }
  lo_out = r;
}

// ds_read_b64_tr_b16 (gfx950 transposing LDS read), checked on MI355X: within
// each 16-lane group the 16 lanes x 4 halfwords read form a 16x4 matrix;
// output lane i, element e is input lane (4e + i/4)'s halfword (i % 4).
__device__ __forceinline__ v4i16 lds_read_tr16(const bf16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)p);
}

// MFMA A (or B) fragment of X^T from a natural-layout LDS tile X[k][m]
// (rows = the product's K index, contiguous along M), pitch in elements.
// Returns, for lane l, X[k0 + kpos(8*(l/32) + e)][m0 + mrow(l % 32)], e = 0..7,
// where kpos is the identity, or slot_perm16 when PERMK (matching P / dS taken
// from accumulator registers), and mrow is the identity, or row_perm32 when
// PERMM (so the product's lane group g holds rows 16g .. 16g+15).
template <bool PERMK, bool PERMM>
__device__ __forceinline__ bf16x8 lds_frag_T(const bf16_t* tile, int pitch, int k0, int m0) {
  const int lane = threadIdx.x & 63;
  const int q = (lane >> 4) & 3, j = lane & 15;
  const int g = q >> 1, mq = q & 1, c = j & 3;
  const int col = PERMM ? (16 * (c & 1) + 8 * mq + 4 * (c >> 1)) : (16 * mq + 4 * c);
  const int r0 = PERMK ? 4 * g : 8 * g;
  const int r1 = PERMK ? 8 + 4 * g : 8 * g + 4;
  const bf16_t* base = tile + (long)(k0 + (j >> 2)) * pitch + m0 + col;
  const v4i16 lo = lds_read_tr16(base + (long)r0 * pitch);
  const v4i16 hi = lds_read_tr16(base + (long)r1 * pitch);
  typedef short v8i16 __attribute__((ext_vector_type(8)));
  const v8i16 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, v);
}

// Contiguous logical work ranges land on one XCD: the hardware deals
// workgroup i to XCD i % 8, so logical id (i % 8) * (G / 8) + i / 8 keeps
// neighbouring logical ids (the same operand working set) in one L2.
__device__ __forceinline__ int xcd_remap(int i, int G) {
  if (G & 7) return i;
  return (i & 7) * (G >> 3) + (i >> 3);
}

__device__ __forceinline__ float wave_max_pair(float x) {
  // Combine lane l with lane l^32 (the two lane groups that share a column).
  return fmaxf(x, __shfl_xor(x, 32, 64));
}
__device__ __forceinline__ float wave_sum_pair(float x) { return x + __shfl_xor(x, 32, 64); }

// Cross-lane exchanges that stay in the VALU (DPP and the gfx950 permlane
// swaps) instead of going through the LDS crossbar as __shfl_xor does.
// DPP controls: quad_perm [1,0,3,2] = 0xb1 (lane ^ 1), [2,3,0,1] = 0x4e
// (lane ^ 2), row_half_mirror = 0x141 (i <-> 7 - i in eight lanes),
// row_mirror = 0x140 (i <-> 15 - i in a row of sixteen), row_ror:n = 0x120 + n.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xf, 0xf, false);
}
// lane l combined with lane l ^ 16 (row pairs) and with lane l ^ 32 (wave halves)
template <typename F>
__device__ __forceinline__ float xor16_f32(float x, F op) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
template <typename F>
__device__ __forceinline__ float xor32_f32(float x, F op) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Butterfly all-reduce over the 64 lanes: every lane gets the same result
// (each step combines two equal-shaped partials with a commutative op).
template <typename F>
__device__ __forceinline__ float wave_allreduce_f32(float x, F op) {
  x = op(x, dpp_f32<0xb1>(x));
  x = op(x, dpp_f32<0x4e>(x));
  x = op(x, dpp_f32<0x141>(x));
  x = op(x, dpp_f32<0x140>(x));
  x = xor16_f32(x, op);
  return xor32_f32(x, op);
}
__device__ __forceinline__ float wave_allsum(float x) {
  return wave_allreduce_f32(x, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ float wave_allmax(float x) {
  return wave_allreduce_f32(x, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ int wave_allmin_i32(int x) {
  x = min(x, dpp_i32<0xb1>(x));
  x = min(x, dpp_i32<0x4e>(x));
  x = min(x, dpp_i32<0x141>(x));
  x = min(x, dpp_i32<0x140>(x));
  auto r = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
  x = min((int)r[0], (int)r[1]);
  r = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
  return min((int)r[0], (int)r[1]);
}

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS
// operations, not for its outstanding global loads (a __syncthreads() fence
// would also drain those, serialising prefetches that are meant to stay in
// flight across the barrier).  The "memory" clobber keeps the compiler from
// moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1.0e30f;  // finite "minus infinity" for running maxima

}  // namespace naylis
