// General bf16 GEMM on MFMA (gemm.hip): C(m, n) = sum_k A(m, k) B(k, n).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace naylis {

// One operand.  K-contiguous: A(m, k) = p[m * ld + k] (B(k, n) = p[n * ld + k]);
// otherwise A(m, k) = p[k * ld + m] (B(k, n) = p[k * ld + n]).  The operand may
// be split along K into two tensors: p1 holds k < K1, p2 holds k >= K1 (then
// indexed from k - K1); K1 must be a multiple of 64 when it is inside [0, K).
struct GemmOp {
  const void* p1;
  const void* p2;
  long ld;
  bool kcontig;
};

enum GemmOut { kGemmOutF32 = 0, kGemmOutBF16 = 1 };

struct GemmJob {
  GemmOp a, b;
  void* c;
  long ldc;
};

// Up to two GEMMs of the same shape and layouts in one launch.  splits > 1
// splits K over workgroups: fp32 partials go to `ws` (gemm_ws_bytes) and a
// fixed-order reduction writes C, so results do not depend on the split.
struct GemmLaunch {
  GemmJob job[2];
  int njobs;
  int M, N, K, K1;
  GemmOut out;
  int splits;
  void* ws;
  // Gate epilogue (one job, splits > 1, C contiguous bf16): the partials sum
  // to dW', C = bf16(gate_s * dW') and gate_part[wg] = sum of dW' * gate_w
  // over the reduction workgroup's elements (gemm_gate_parts of them).
  const void* gate_w = nullptr;
  const float* gate_s = nullptr;
  float* gate_part = nullptr;
  // Take the 64 x 128 tile over 128 x 128 when that turns a grid of uneven
  // rounds (not a multiple of the CU count) into whole rounds.
  bool whole_rounds = false;
};
int gemm_gate_parts(int M, int N);

// true when the fast kernel supports the shapes and layouts (M, N, K, leading
// dimensions multiples of 8, 16-byte aligned pointers, K1 a multiple of 64)
bool gemm_supported(const GemmLaunch& g);
size_t gemm_ws_bytes(int njobs, int M, int N, int splits);
hipError_t launch_gemm(const GemmLaunch& g, const char* timer_name, hipStream_t st);

// Up to kGemmMaxGroupJobs GEMMs of one shape and layout in one launch (no K
// split; each job's C bitwise equal to launch_gemm of that job).  With
// sum_jobs, C = sum over jobs of A_j B_j, written to job[0].c through fp32
// partials in ws (gemm_grouped_ws_bytes) added in job order.
constexpr int kGemmMaxGroupJobs = 48;
struct GemmGroupedLaunch {
  GemmJob job[kGemmMaxGroupJobs];
  int njobs;
  int M, N, K, K1;
  GemmOut out;
  bool sum_jobs;
  void* ws;
};
bool gemm_grouped_supported(const GemmGroupedLaunch& g);
size_t gemm_grouped_ws_bytes(int njobs, int M, int N, bool sum_jobs);
hipError_t launch_gemm_grouped(const GemmGroupedLaunch& g, const char* timer_name, hipStream_t st);

// Zero `bytes` bytes at p with a kernel (safe inside captured HIP graphs).
hipError_t launch_zero(void* p, size_t bytes, hipStream_t st);

}  // namespace naylis
