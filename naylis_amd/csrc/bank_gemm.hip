// Bank K/V projection of the MoM layer (gfx950, bf16 MFMA, fp32 accumulate).
//
// Forward (model.py:253-256, reference.py:86-89), once per layer and shared by
// the whole batch:   K = slots W_k^T,  V = slots W_v^T,  slots = M_blocks.view(L, D)
// Backward:           d_slots = dK W_k + dV W_v      (one GEMM, K-dim concatenated)
//                     dW_k = dK^T slots,  dW_v = dV^T slots
//
// One generic tile kernel C(MxN) = sum_k A(m,k) B(k,n) covers the three layouts;
// A and B are staged into LDS K-contiguous ([row][k]) whatever their global
// layout, so the MFMA fragments are single 16-byte LDS reads.  Tile 64x64x32,
// 4 waves in 2x2, one 32x32 accumulator per wave.  Each operand may be split
// along K at K1 into two tensors (A1|A2, B1;B2), which is how the two terms of
// d_slots become one product.
#include "common.h"
#include "timing.h"
#include "launch_bank.h"
#include "launch_gemm.h"

namespace naylis {

struct GemmOperand {
  const bf16_t* p1;  // k < K1
  const bf16_t* p2;  // k >= K1 (may equal p1 when K1 >= K)
  long ld;           // leading dimension (elements)
};

struct GemmProblem {
  GemmOperand a, b;
  void* c;
  long ldc;
};

struct GemmBatch {
  GemmProblem prob[2];
};

constexpr int GBM = 64, GBN = 64, GBK = 32, GPAD = GBK + 8;

// Element (row, k) of an operand: K-major -> p[row*ld + k]; else p[k*ld + row].
template <bool KMAJOR>
__device__ __forceinline__ void stage_operand(const GemmOperand& op, int K1, int rows, int K, int row0, int k0,
                                              bf16_t* lds, int tid) {
  if constexpr (KMAJOR) {
    // thread -> (row = tid/4, 8 consecutive k)
    const int r = tid >> 2, k8 = (tid & 3) * 8;
    const int gr = row0 + r, gk = k0 + k8;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (gr < rows) {
      const bf16_t* p = gk < K1 ? op.p1 + (long)gr * op.ld + gk : op.p2 + (long)gr * op.ld + (gk - K1);
      if (gk + 8 <= K && (gk >= K1 || gk + 8 <= K1)) {
        v = *reinterpret_cast<const uint4*>(p);
      } else {
        bf16_t* ve = reinterpret_cast<bf16_t*>(&v);
        for (int e = 0; e < 8; ++e) {
          const int kk = gk + e;
          if (kk < K) ve[e] = kk < K1 ? op.p1[(long)gr * op.ld + kk] : op.p2[(long)gr * op.ld + (kk - K1)];
        }
      }
    }
    *reinterpret_cast<uint4*>(&lds[r * GPAD + k8]) = v;
  } else {
    // thread -> (k = tid/8, 8 consecutive rows), transposed into [row][k]
    const int kk = tid >> 3, r8 = (tid & 7) * 8;
    const int gk = k0 + kk, gr = row0 + r8;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (gk < K) {
      const bf16_t* base = gk < K1 ? op.p1 + (long)gk * op.ld : op.p2 + (long)(gk - K1) * op.ld;
      if (gr + 8 <= rows && ((((uintptr_t)(base + gr)) & 15) == 0)) {
        v = *reinterpret_cast<const uint4*>(base + gr);
      } else {
        bf16_t* ve = reinterpret_cast<bf16_t*>(&v);
        for (int e = 0; e < 8; ++e)
          if (gr + e < rows) ve[e] = base[gr + e];
      }
    }
    const bf16_t* ve = reinterpret_cast<const bf16_t*>(&v);
#pragma unroll
    for (int e = 0; e < 8; ++e) lds[(r8 + e) * GPAD + kk] = ve[e];
  }
}

template <bool A_KMAJOR, bool B_KMAJOR, bool OUT_F32>
__global__ __launch_bounds__(256) void bank_gemm_kernel(GemmBatch batch, int M, int N, int K, int K1) {
  __shared__ __attribute__((aligned(16))) bf16_t a_lds[GBM * GPAD];
  __shared__ __attribute__((aligned(16))) bf16_t b_lds[GBN * GPAD];
  const GemmProblem& P = batch.prob[blockIdx.z];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, col = lane & 31;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * GBM, n0 = blockIdx.x * GBN;
  f32x16 acc = f32x16{};
  for (int k0 = 0; k0 < K; k0 += GBK) {
    __syncthreads();
    stage_operand<A_KMAJOR>(P.a, K1, M, K, m0, k0, a_lds, tid);
    stage_operand<B_KMAJOR>(P.b, K1, N, K, n0, k0, b_lds, tid);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < GBK / 16; ++ks) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(&a_lds[(wm * 32 + col) * GPAD + 16 * ks + 8 * g]);
      const bf16x8 b = *reinterpret_cast<const bf16x8*>(&b_lds[(wn * 32 + col) * GPAD + 16 * ks + 8 * g]);
      acc = mfma32(a, b, acc);
    }
  }
  const int n = n0 + wn * 32 + col;
  if (n < N) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = m0 + wm * 32 + acc_row(g, v);
      if (m < M) {
        if constexpr (OUT_F32)
          reinterpret_cast<float*>(P.c)[(long)m * P.ldc + n] = acc[v];
        else
          reinterpret_cast<bf16_t*>(P.c)[(long)m * P.ldc + n] = f32_to_bf16(acc[v]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
hipError_t launch_bank_kv_fwd(const void* slots, const void* w_k, const void* w_v, void* k_out, void* v_out, int L,
                              int D_in, int D_out, hipStream_t st) {
  GemmLaunch g{};
  g.njobs = 2;
  g.M = L;
  g.N = D_out;
  g.K = g.K1 = D_in;
  g.out = kGemmOutBF16;
  g.splits = 1;
  for (int z = 0; z < 2; ++z) {
    g.job[z].a = GemmOp{slots, nullptr, D_in, true};                   // A(l, i) = slots[l][i]
    g.job[z].b = GemmOp{z == 0 ? w_k : w_v, nullptr, D_in, true};      // B(i, o) = W[o][i]
    g.job[z].c = z == 0 ? k_out : v_out;
    g.job[z].ldc = D_out;
  }
  if (gemm_supported(g)) return launch_gemm(g, "bank_kv_fwd", st);
  // small or unaligned shapes: the simple 64 x 64 tile kernel
  GemmBatch bt{};
  for (int z = 0; z < 2; ++z) {
    GemmProblem& P = bt.prob[z];
    P.a = {(const bf16_t*)slots, (const bf16_t*)slots, D_in};
    const bf16_t* w = (const bf16_t*)(z == 0 ? w_k : w_v);
    P.b = {w, w, D_in};  // B(k, n) = W[n][k]: K-major
    P.c = z == 0 ? k_out : v_out;
    P.ldc = D_out;
  }
  const dim3 grid((D_out + GBN - 1) / GBN, (L + GBM - 1) / GBM, 2);
  NAYLIS_TIMED("bank_kv_fwd", st, hipLaunchKernelGGL((bank_gemm_kernel<true, true, false>), grid, dim3(256), 0, st, bt, L, D_out, D_in, D_in));
  return hipGetLastError();
}

hipError_t launch_bank_kv_bwd(const void* slots, const void* w_k, const void* w_v, const void* dk, const void* dv,
                              void* d_slots, bool slots_f32, void* dw_k, void* dw_v, bool w_f32, int L, int D_in,
                              int D_out, hipStream_t st) {
  // d_slots (L x D_in) = [dK | dV] (L x 2D_out) . [W_k ; W_v] (2D_out x D_in)
  GemmLaunch g1{};
  g1.njobs = 1;
  g1.M = L;
  g1.N = D_in;
  g1.K = 2 * D_out;
  g1.K1 = D_out;
  g1.out = slots_f32 ? kGemmOutF32 : kGemmOutBF16;
  g1.splits = 1;
  g1.job[0].a = GemmOp{dk, dv, D_out, true};      // A(l, o) = [dK | dV][l][o]
  g1.job[0].b = GemmOp{w_k, w_v, D_in, false};    // B(o, i) = [W_k ; W_v][o][i]
  g1.job[0].c = d_slots;
  g1.job[0].ldc = D_in;
  // config 4 (L 4096, D_in 1536): 384 workgroups of 128 x 128 against 768 of
  // 64 x 128 (three whole rounds), 76 -> 66 us; the dW product below keeps
  // the larger tile, where the same choice measured slower
  g1.whole_rounds = true;
  // dW (D_out x D_in) = dK^T (D_out x L) . slots (L x D_in)
  GemmLaunch g2{};
  g2.njobs = 2;
  g2.M = D_out;
  g2.N = D_in;
  g2.K = g2.K1 = L;
  g2.out = w_f32 ? kGemmOutF32 : kGemmOutBF16;
  g2.splits = 1;
  for (int z = 0; z < 2; ++z) {
    g2.job[z].a = GemmOp{z == 0 ? dk : dv, nullptr, D_out, false};   // A(o, l) = dK[l][o]
    g2.job[z].b = GemmOp{slots, nullptr, D_in, false};               // B(l, i) = slots[l][i]
    g2.job[z].c = z == 0 ? dw_k : dw_v;
    g2.job[z].ldc = D_in;
  }
  if (gemm_supported(g1) && gemm_supported(g2)) {
    hipError_t e = launch_gemm(g1, "bank_kv_bwd_dslots", st);
    if (e != hipSuccess) return e;
    return launch_gemm(g2, "bank_kv_bwd_dw", st);
  }
  GemmBatch b1{};
  b1.prob[0].a = {(const bf16_t*)dk, (const bf16_t*)dv, D_out};      // A(m=l, k=o): K-major
  b1.prob[0].b = {(const bf16_t*)w_k, (const bf16_t*)w_v, D_in};     // B(k=o, n=j) = W[o][j]: N-contiguous
  b1.prob[0].c = d_slots;
  b1.prob[0].ldc = D_in;
  const dim3 grid1((D_in + GBN - 1) / GBN, (L + GBM - 1) / GBM, 1);
  if (slots_f32)
    NAYLIS_TIMED("bank_kv_bwd_dslots", st, hipLaunchKernelGGL((bank_gemm_kernel<true, false, true>), grid1, dim3(256), 0, st, b1, L, D_in, 2 * D_out, D_out));
  else
    NAYLIS_TIMED("bank_kv_bwd_dslots", st, hipLaunchKernelGGL((bank_gemm_kernel<true, false, false>), grid1, dim3(256), 0, st, b1, L, D_in, 2 * D_out, D_out));
  // dW (D_out x D_in) = dK^T (D_out x L) . slots (L x D_in)
  GemmBatch b2{};
  for (int z = 0; z < 2; ++z) {
    GemmProblem& P = b2.prob[z];
    const bf16_t* g = (const bf16_t*)(z == 0 ? dk : dv);
    P.a = {g, g, D_out};                                              // A(m=o, k=l) = dK[l][o]: M-contiguous
    P.b = {(const bf16_t*)slots, (const bf16_t*)slots, D_in};         // B(k=l, n=j) = slots[l][j]: N-contiguous
    P.c = z == 0 ? dw_k : dw_v;
    P.ldc = D_in;
  }
  const dim3 grid2((D_in + GBN - 1) / GBN, (D_out + GBM - 1) / GBM, 2);
  if (w_f32)
    NAYLIS_TIMED("bank_kv_bwd_dw", st, hipLaunchKernelGGL((bank_gemm_kernel<false, false, true>), grid2, dim3(256), 0, st, b2, D_out, D_in, L, L));
  else
    NAYLIS_TIMED("bank_kv_bwd_dw", st, hipLaunchKernelGGL((bank_gemm_kernel<false, false, false>), grid2, dim3(256), 0, st, b2, D_out, D_in, L, L));
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// The projections of n layers that read one bank, one grouped launch each:
//   forward   K_i = slots W_k,i^T, V_i = slots W_v,i^T        (2n jobs)
//   backward  d_slots = sum_i dK_i W_k,i + dV_i W_v,i          (n jobs, summed in layer order)
//             dW_k,i = dK_i^T slots, dW_v,i = dV_i^T slots     (2n jobs)
// Each K_i, V_i, dW_k,i, dW_v,i is bitwise what the per-layer launch gives;
// d_slots is accumulated in fp32 over all layers and rounded once.
bool bank_grouped_ok(int n, int L, int D_in, int D_out) {
  // the backward's K splits at D_out between dK and dV: a whole number of 64-wide K steps
  return n >= 1 && 2 * n <= kGemmMaxGroupJobs && L > 0 && D_in % 8 == 0 && D_out % 64 == 0;
}

size_t bank_kv_bwd_grouped_ws_bytes(int n, int L, int D_in) { return gemm_grouped_ws_bytes(n, L, D_in, true); }

hipError_t launch_bank_kv_fwd_grouped(const void* slots, const void* const* w_k, const void* const* w_v,
                                      void* const* k_out, void* const* v_out, int n, int L, int D_in, int D_out,
                                      hipStream_t st) {
  GemmGroupedLaunch g{};
  g.njobs = 2 * n;
  g.M = L;
  g.N = D_out;
  g.K = g.K1 = D_in;
  g.out = kGemmOutBF16;
  for (int z = 0; z < 2 * n; ++z) {
    const int i = z / 2;
    g.job[z].a = GemmOp{slots, nullptr, D_in, true};
    g.job[z].b = GemmOp{z % 2 ? w_v[i] : w_k[i], nullptr, D_in, true};
    g.job[z].c = z % 2 ? v_out[i] : k_out[i];
    g.job[z].ldc = D_out;
  }
  if (!gemm_grouped_supported(g)) return hipErrorInvalidValue;
  return launch_gemm_grouped(g, "bank_kv_fwd", st);
}

hipError_t launch_bank_kv_bwd_grouped(const void* slots, const void* const* w_k, const void* const* w_v,
                                      const void* const* dk, const void* const* dv, void* d_slots, bool slots_f32,
                                      void* const* dw_k, void* const* dw_v, bool w_f32, void* ws, int n, int L,
                                      int D_in, int D_out, hipStream_t st) {
  GemmGroupedLaunch g1{};  // d_slots (L x D_in) = sum_i [dK_i | dV_i] . [W_k,i ; W_v,i]
  g1.njobs = n;
  g1.M = L;
  g1.N = D_in;
  g1.K = 2 * D_out;
  g1.K1 = D_out;
  g1.out = slots_f32 ? kGemmOutF32 : kGemmOutBF16;
  g1.sum_jobs = true;
  g1.ws = ws;
  for (int i = 0; i < n; ++i) {
    g1.job[i].a = GemmOp{dk[i], dv[i], D_out, true};
    g1.job[i].b = GemmOp{w_k[i], w_v[i], D_in, false};
    g1.job[i].c = d_slots;
    g1.job[i].ldc = D_in;
  }
  GemmGroupedLaunch g2{};  // dW_k,i, dW_v,i (D_out x D_in) = dK_i^T . slots
  g2.njobs = 2 * n;
  g2.M = D_out;
  g2.N = D_in;
  g2.K = g2.K1 = L;
  g2.out = w_f32 ? kGemmOutF32 : kGemmOutBF16;
  for (int z = 0; z < 2 * n; ++z) {
    const int i = z / 2;
    g2.job[z].a = GemmOp{z % 2 ? dv[i] : dk[i], nullptr, D_out, false};
    g2.job[z].b = GemmOp{slots, nullptr, D_in, false};
    g2.job[z].c = z % 2 ? dw_v[i] : dw_k[i];
    g2.job[z].ldc = D_in;
  }
  if (!gemm_grouped_supported(g1) || !gemm_grouped_supported(g2)) return hipErrorInvalidValue;
  hipError_t e = launch_gemm_grouped(g1, "bank_kv_bwd_dslots", st);
  if (e != hipSuccess) return e;
  return launch_gemm_grouped(g2, "bank_kv_bwd_dw", st);
}

}  // namespace naylis
