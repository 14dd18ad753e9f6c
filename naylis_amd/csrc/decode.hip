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
// the ranks, its W_down rows loaded up front, lane partial sums combined by a
// DPP / permlane butterfly; W_down is read from L2 by every workgroup), so no
// workgroup waits on another; the one with head group 0 writes the new state
// and the selection.  Each wave then ranks the experts itself (lane = expert)
// and reads head 4 g + wave: a slot's head row (HD fp8 bytes) is split into
// 16-byte pieces over HD / 16 consecutive lanes, so K and V loads are
// contiguous per slot, q . k is a partial dot per lane summed over the
// slot's lanes, and p stays in the registers of the lanes that multiply it
// into v; chunks of 16 slots per lane are combined by an online softmax.
// fp8 codes are widened with the gfx950 packed conversion v_cvt_pk_f32_fp8
// (OCP e4m3 on this target; the tests compare the result with torch's
// float8_e4m3fn).
//
// With one wave per SIMD nothing hides latency, so the step is a chain of
// two memory round trips (state / W_down / q up front, then K / V once the
// blocks are known) plus VALU issue: every load of a phase is issued back to
// back (indices clamped instead of branched around, 32-bit buffer offsets),
// cross-lane sums stay in DPP / permlane, and the per-slot row walk needs
// no integer division when block_size is a multiple of the slot phases.
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

// p . v partial sums: add the lanes that hold the same 16-byte piece of a slot
// row (lanes equal modulo KV16), i.e. the slot phases; every lane gets the sum
// of its class (within a row in lane-dependent order, then the row pairs).
template <int KV16>
__device__ __forceinline__ float phase_sum(float x) {
  const auto add = [](float a, float b) { return a + b; };
  if constexpr (KV16 == 2) x += dpp_f32<0x4e>(x);
  if constexpr (KV16 <= 4) x += dpp_f32<0x124>(x);
  x += dpp_f32<0x128>(x);
  x = xor16_f32(x, add);
  return xor32_f32(x, add);
}

// q . k partial dots: add the KV16 consecutive lanes that hold one slot's row
// (xor 1, xor 2, then the mirrored half of eight lanes); all of them get the sum.
template <int KV16>
__device__ __forceinline__ float slot_sum(float x) {
  x += dpp_f32<0xb1>(x);
  if constexpr (KV16 >= 4) x += dpp_f32<0x4e>(x);
  if constexpr (KV16 >= 8) x += dpp_f32<0x141>(x);
  return x;
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
  constexpr int CH = 16384 / HD;  // slots per chunk (16 per lane)
  constexpr int KV16 = HD / 16;   // 16-byte pieces of a slot's head row = lanes per slot in p . v
  constexpr int NPH = 64 / KV16;  // p . v: slot phases
  constexpr int VSPL = CH / NPH;  // p . v: slots per lane per chunk (16)
  constexpr int SPF = 4;          // state elements per thread loaded up front (D <= 1024)
  constexpr int RPF = 8;          // router ranks per wave whose W_down loads are issued up front ...
  constexpr int JPF = 4;          // ... and their float4 columns per lane (d < 1024)
  constexpr int UPF = 8;          // float4 of a w_up row loaded up front (R <= 32)
  __shared__ __align__(16) float h_lds[kDecodeMaxD];
  __shared__ float a_lds[kDecodeMaxRank];
  __shared__ int sel_lds[4][TK];
  __shared__ float lgate_lds[4][TK];
  const int g = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = 4 * g + wave;
  const bool reader = h < H;

  // ---- loads that depend on nothing, in the order they are needed (loads retire in issue order):
  // the state and token, this wave's W_down rows, its lane's w_up row, the q row
  // (all offsets fit 32 bits: B * D < 2^28, L * D <= 2^26, R * D <= 2^18)
  const uint32_t srow = (uint32_t)b * D;
  // (indices are clamped into range instead of branching around the loads, so that they are all
  // issued back to back; values past the end are dropped afterwards)
  double sv[SPF];
#pragma unroll
  for (int i = 0; i < SPF; ++i) {
    const int d = min(tid + 256 * i, D - 1);
    sv[i] = state_in[srow + d] + load_x(x_new + srow + d);
  }
  const float den = (float)(t_prev[b] + 1);
  // workgroups start on different rows so that their simultaneous requests spread over the L2 channels
  const int rot = (b + g) & (RPF - 1);
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc(w_down, (uint32_t)R * D * 4);
  float4 wpf[RPF][JPF];
#pragma unroll
  for (int i = 0; i < RPF; ++i)
#pragma unroll
    for (int j = 0; j < JPF; ++j) {
      const int r = min(wave + 4 * ((i + rot) & (RPF - 1)), R - 1), d = min(4 * lane + 256 * j, D - 4);
      const float4 w = __builtin_bit_cast(
          float4, __builtin_amdgcn_raw_buffer_load_b128(wrs, ((uint32_t)r * D + d) * 4, 0, 0));
      const bool in = 4 * lane + 256 * j < D;  // columns past D weigh nothing
      wpf[i][j] = make_float4(in ? w.x : 0.f, in ? w.y : 0.f, in ? w.z : 0.f, in ? w.w : 0.f);
    }
  const bool up_vec = (R & 3) == 0 && R <= 4 * UPF;
  float4 wu4[UPF];
#pragma unroll
  for (int i = 0; i < UPF; ++i)
    wu4[i] = up_vec ? *reinterpret_cast<const float4*>(w_up + ((uint32_t)min(lane, E - 1) * R + min(4 * i, R - 4)))
                    : make_float4(0.f, 0.f, 0.f, 0.f);
  const int vph = lane / KV16, vpc = lane % KV16;  // read: slot phase, 16-byte piece of the slot's head row
  uint4 qraw[2];                                   // q features 16 vpc .. 16 vpc + 15
  {
    const bf16_t* qp = q_new + (((uint32_t)b * H + (reader ? h : 0)) * HD + 16 * vpc);
    qraw[0] = *reinterpret_cast<const uint4*>(qp);
    qraw[1] = *reinterpret_cast<const uint4*>(qp + 8);
  }

  // ---- running sum and prefix mean: one fp64 add, one rounding to fp32, IEEE division
#pragma unroll
  for (int i = 0; i < SPF; ++i) {
    const int d = tid + 256 * i;
    if (d < D) {
      if (g == 0) state_out[srow + d] = sv[i];
      h_lds[d] = (float)sv[i] / den;
    }
  }
  for (int d = tid + 256 * SPF; d < D; d += 256) {
    const double v = state_in[srow + d] + load_x(x_new + srow + d);
    if (g == 0) state_out[srow + d] = v;
    h_lds[d] = (float)v / den;
  }
  lds_barrier();  // the W_down / q loads stay in flight
  // ---- a = tanh(W_down h): wave w takes ranks w, w + 4, ...; lane sums d = 4 lane + 256 j, then a butterfly
  {
    float acc[RPF];
#pragma unroll
    for (int i = 0; i < RPF; ++i) {
      acc[i] = 0.f;
#pragma unroll
      for (int j = 0; j < JPF; ++j) {
        const float4 hv = *reinterpret_cast<const float4*>(h_lds + min(4 * lane + 256 * j, D - 4));
        acc[i] = fmaf(wpf[i][j].x, hv.x, acc[i]);
        acc[i] = fmaf(wpf[i][j].y, hv.y, acc[i]);
        acc[i] = fmaf(wpf[i][j].z, hv.z, acc[i]);
        acc[i] = fmaf(wpf[i][j].w, hv.w, acc[i]);
      }
    }
    if (D > 256 * JPF) {  // columns beyond the prefetch
#pragma unroll
      for (int i = 0; i < RPF; ++i) {
        const int r = wave + 4 * ((i + rot) & (RPF - 1));
        if (r < R) {
          for (int d = 4 * lane + 256 * JPF; d < D; d += 256) {
            const float4 w4 = *reinterpret_cast<const float4*>(w_down + (long)r * D + d);
            const float4 hv = *reinterpret_cast<const float4*>(h_lds + d);
            acc[i] = fmaf(w4.x, hv.x, acc[i]);
            acc[i] = fmaf(w4.y, hv.y, acc[i]);
            acc[i] = fmaf(w4.z, hv.z, acc[i]);
            acc[i] = fmaf(w4.w, hv.w, acc[i]);
          }
        }
      }
    }
    // every lane gets all RPF sums; lane i < RPF takes the tanh of the i-th
    float mine = 0.f;
#pragma unroll
    for (int i = 0; i < RPF; ++i) {
      const float v = wave_allsum(acc[i]);
      mine = lane == i ? v : mine;
    }
    if (lane < RPF) {
      const int r = wave + 4 * ((lane + rot) & (RPF - 1));
      if (r < R) a_lds[r] = tanhf(mine);
    }
    for (int r = wave + 4 * RPF; r < R; r += 4) {  // ranks beyond the prefetch
      float v = 0.f;
      for (int d = 4 * lane; d < D; d += 256) {
        const float4 w4 = *reinterpret_cast<const float4*>(w_down + (long)r * D + d);
        const float4 hv = *reinterpret_cast<const float4*>(h_lds + d);
        v = fmaf(w4.x, hv.x, v);
        v = fmaf(w4.y, hv.y, v);
        v = fmaf(w4.z, hv.z, v);
        v = fmaf(w4.w, hv.w, v);
      }
      v = wave_allsum(v);
      if (lane == 0) a_lds[r] = tanhf(v);
    }
  }
  lds_barrier();
  // ---- logits (lane = expert), top-k (ties to the lower id), gates: every wave for itself
  float lg = -INFINITY;
  if (lane < E) {
    lg = 0.f;
    if (up_vec) {
#pragma unroll
      for (int i = 0; i < UPF; ++i) {
        if (4 * i < R) {
          lg = fmaf(wu4[i].x, a_lds[4 * i], lg);
          lg = fmaf(wu4[i].y, a_lds[4 * i + 1], lg);
          lg = fmaf(wu4[i].z, a_lds[4 * i + 2], lg);
          lg = fmaf(wu4[i].w, a_lds[4 * i + 3], lg);
        }
      }
    } else {
      const float* wu = w_up + (long)lane * R;
      for (int r = 0; r < R; ++r) lg = fmaf(wu[r], a_lds[r], lg);
    }
  }
  {
    bool taken = lane >= E;
    float val[TK];
    int sel[TK];
#pragma unroll
    for (int k = 0; k < TK; ++k) {
      if (k < topk) {
        const float bv = wave_allmax(taken ? -INFINITY : lg);
        const int bi = wave_allmin_i32(!taken && lg == bv ? lane : 0x7fffffff);
        val[k] = bv;
        sel[k] = bi;
        taken |= lane == bi;
      }
    }
    float gs = 0.f;
#pragma unroll
    for (int k = 0; k < TK; ++k)
      if (k < topk) gs += expf(val[k] - val[0]);
    if (lane == 0) {
#pragma unroll
      for (int k = 0; k < TK; ++k) {
        if (k < topk) {
          const float gv = expf(val[k] - val[0]) / gs;
          sel_lds[wave][k] = sel[k];
          lgate_lds[wave][k] = log2f(fmaxf(gv, 1e-9f));
          if (g == 0 && wave == 0) {
            top_idx[(long)b * topk + k] = sel[k];
            top_gates[(long)b * topk + k] = gv;
          }
        }
      }
    }
  }
  // lane 0's selection is read by the whole wave
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- read of head 4 g + wave over the top-k blocks (distinct ids: top-k of distinct experts).
  // Lane (vph, vpc) holds piece vpc (16 features) of slots vph, vph + NPH, ... of each chunk for both
  // K and V (a slot's KV16 lanes read its 16 * KV16 contiguous bytes), so q . k is a partial dot per lane
  // summed over the slot's lanes, and p stays in the registers of the lanes that multiply it into v.
  if (!reader) return;
  const int* selw = sel_lds[wave];
  const float* lgw = lgate_lds[wave];
  const uint32_t Dk = (uint32_t)H * HD;
  const uint32_t col = (uint32_t)h * HD + 16 * vpc;
  // buffer resources: 32-bit lane offsets, no 64-bit address arithmetic
  const uint32_t L = (uint32_t)E * block_size;
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(k8, L * Dk), vrs = make_rsrc(v8, L * Dk);
  const __amdgpu_buffer_rsrc_t ksrs = make_rsrc(k_scale, L * 4), vsrs = make_rsrc(v_scale, L * 4);
  const int nslots = topk * block_size;
  float qv[16];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t w4[4] = {qraw[i].x, qraw[i].y, qraw[i].z, qraw[i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      qv[8 * i + 2 * e] = __uint_as_float(w4[e] << 16);
      qv[8 * i + 2 * e + 1] = __uint_as_float(w4[e] & 0xffff0000u);
    }
  }
  float m = -INFINITY, l = 0.f;
  float acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.f;
  for (int c0 = 0; c0 < nslots; c0 += CH) {
    uint4 kreg[VSPL], vreg[VSPL];
    float ksc[VSPL], vsc[VSPL], kb[VSPL];
    uint32_t row[VSPL];
    if (block_size % NPH == 0) {
      // the NPH slots of step i lie in one block: walk (block, offset) with wave-uniform counters
      int k = c0 / block_size, off = c0 - k * block_size;
#pragma unroll
      for (int i = 0; i < VSPL; ++i) {
        const bool in = c0 + NPH * i < nslots;
        const int kk = in ? k : topk - 1, oo = in ? off : block_size - NPH;  // past the end: re-read the last slots
        row[i] = (uint32_t)(selw[kk] * block_size + oo + vph);
        kb[i] = in ? lgw[kk] : -INFINITY;
        off += NPH;
        if (off == block_size) {
          off = 0;
          ++k;
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < VSPL; ++i) {
        const int u = min(c0 + vph + NPH * i, nslots - 1);  // slots past the end re-read the last one
        const int k = u / block_size;
        row[i] = (uint32_t)(selw[k] * block_size + (u - k * block_size));
        kb[i] = c0 + vph + NPH * i < nslots ? lgw[k] : -INFINITY;
      }
    }
#pragma unroll
    for (int i = 0; i < VSPL; ++i)
      kreg[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(krs, row[i] * Dk + col, 0, 0));
#pragma unroll
    for (int i = 0; i < VSPL; ++i)
      ksc[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ksrs, row[i] * 4, 0, 0));
#pragma unroll
    for (int i = 0; i < VSPL; ++i)
      vreg[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vrs, row[i] * Dk + col, 0, 0));
#pragma unroll
    for (int i = 0; i < VSPL; ++i)
      vsc[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(vsrs, row[i] * 4, 0, 0));
    float sc[VSPL];
    float cmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < VSPL; ++i) {
      const uint32_t w4[4] = {kreg[i].x, kreg[i].y, kreg[i].z, kreg[i].w};
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float f[4];
        fp8x4_to_f32(w4[e], f);
#pragma unroll
        for (int j = 0; j < 4; ++j) dot = fmaf(qv[4 * e + j], f[j], dot);
      }
      dot = slot_sum<KV16>(dot);
      sc[i] = fmaf(dot * ksc[i], alpha, kb[i]);  // -inf past the last slot
      cmax = fmaxf(cmax, sc[i]);
    }
    const float m_new = fmaxf(m, wave_allmax(cmax));
    const float corr = __builtin_amdgcn_exp2f(m - m_new);  // 0 on the first chunk
    l *= corr;
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] *= corr;
#pragma unroll
    for (int i = 0; i < VSPL; ++i) {
      const float p = __builtin_amdgcn_exp2f(sc[i] - m_new);
      l += p;
      const float pv = p * vsc[i];
      const uint32_t w4[4] = {vreg[i].x, vreg[i].y, vreg[i].z, vreg[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float f[4];
        fp8x4_to_f32(w4[e], f);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[4 * e + j] = fmaf(pv, f[j], acc[4 * e + j]);
      }
    }
    m = m_new;
  }
  // every slot's p sits in its KV16 lanes: count it once (piece 0)
  l = wave_allsum(vpc == 0 ? l : 0.f);
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = phase_sum<KV16>(acc[j]);
  if (vph == 0) {
    const float inv = 1.f / l;
    uint32_t pk[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      pk[j] = (uint32_t)f32_to_bf16(acc[2 * j] * inv) | ((uint32_t)f32_to_bf16(acc[2 * j + 1] * inv) << 16);
    uint4* op = reinterpret_cast<uint4*>(out + (((uint32_t)b * H + h) * HD + 16 * vpc));
    op[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    op[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
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
