// General bf16 GEMM for gfx950 on v_mfma_f32_32x32x16_bf16, fp32 accumulate:
//     C(m, n) = sum_k A(m, k) B(k, n)
// Used for the bank K/V projection and its gradients (model.py:253-256) and
// for the weight gradients of the layer's q/o projections (model.py:239,251),
// whose reduction runs over all tokens.
//
// Workgroup tile 128 x 128, K step 64; 4 waves in 2 x 2, each wave 64 x 64 =
// 2 x 2 MFMA tiles (256 x 128 with 8 waves, or 64 x 128 / 64 x 64 for small
// grids: see the GemmCfg list).  Each operand is staged into LDS in its global
// layout by plain 16-byte copies: a K-contiguous operand as [row][k] (an MFMA
// fragment is one 16-byte LDS read), an M- or N-contiguous one as [k][row] (a
// fragment is two gfx950 transposing reads, ds_read_b64_tr_b16).  LDS is
// double buffered with one barrier per K step; the next steps' global loads
// are in flight during the current step's MFMAs.  With splits > 1 the K range
// is divided over workgroups, fp32 partials go to a workspace and a
// fixed-order reduction writes C (deterministic, independent of scheduling).
// A grouped launch runs up to 48 GEMMs of one shape in one grid (the bank
// projection of all decoder layers), optionally adding their products into
// one output in job order.
#include "common.h"
#include "launch_gemm.h"
#include "timing.h"

namespace naylis {

constexpr int kGK = 64;  // K step

struct DevOp {
  const bf16_t* p1;
  const bf16_t* p2;
  long ld;
};
struct DevJob {
  DevOp a, b;
  void* c;
  long ldc;
};
struct DevJobs {
  DevJob j[2];
};
// the job table of a grouped launch (every job of one shape and layout)
struct DevJobsGrouped {
  DevJob j[kGemmMaxGroupJobs];
};

// Tile configuration: WAVES_M x WAVES_N waves, each owning TM x TN MFMA tiles
// of 32 x 32 (a (32 TM) x (32 TN) block of C).
template <int WAVES_M_, int WAVES_N_, int TM_, int TN_>
struct GemmCfg {
  static constexpr int WAVES_M = WAVES_M_, WAVES_N = WAVES_N_, TM = TM_, TN = TN_;
  static constexpr int NT = 64 * WAVES_M * WAVES_N;   // threads
  static constexpr int BM = 32 * TM * WAVES_M;        // workgroup tile rows
  static constexpr int BN = 32 * TN * WAVES_N;        // workgroup tile columns
  // K stages in flight in registers: the K loop of these tiles waits on
  // global-load latency (one stage of MFMA is 0.1 - 0.4 us), so a stage is
  // loaded DEPTH steps before it is copied to LDS
  static constexpr int DEPTH = TM * TN >= 4 ? 3 : 4;
};
// 128 x 128, 4 waves of 64 x 64.  (256 x 256 tiles with 8 waves of 128 x 64
// or 4 of 128 x 128 measured no faster on MI355X for these shapes: with one
// stage of prefetch the K loop waits on load latency, not on MFMA or LDS.)
using CfgSmall = GemmCfg<2, 2, 2, 2>;
// 256 x 128 with 8 waves of 64 x 64: the same waves, 3/4 of the staging
// traffic per MFMA.  Used when its grid is a whole number of waves of
// workgroups over the CUs: the q/o weight gradients at d = 1024 (8 K splits,
// 256 workgroups) run in 53 us instead of 57 us; the 2816 x 1024 MLP shapes
// (352 workgroups, a partial second wave) measured 7 % slower than with
// 128 x 128 tiles.
using CfgWide = GemmCfg<4, 2, 2, 2>;
// Narrower tiles for GEMMs too small to give every CU a 128 x 128 tile (the
// 1024 x 1024 bank projections): 64 x 128 and 64 x 64.  The 64 x 128 tile
// runs 8 waves of 32 x 32 (two per SIMD, so one wave's LDS and load waits
// overlap the other's products): bank K/V forward 12.7-13.5 -> 11.3-11.8 us
// and dW 13.3-14.0 -> 11.8-12.7 us at config 2 against 4 waves of 32 x 64,
// with every element summed in the same K order (bitwise the same C).
using CfgMid = GemmCfg<2, 4, 1, 1>;
using CfgTiny = GemmCfg<2, 2, 1, 1>;

// LDS pitches: a [row][k] tile row is 64 + 8 elements (36 dwords: eight
// consecutive rows' 16-byte reads hit distinct banks); a [k][row] tile row
// is ROWS + 32 elements (16 dwords mod 32).  Measured on MI355X for the
// transposed fragment reads below (two ds_read_b64_tr_b16 each, 16 waves per
// CU): 128-row tiles 173 B/clk/CU at pitch 160 against 111 at 144 and
// 113 - 117 at 152, 176, 192; 64-row tiles 182 at 96 against 118 - 121 at
// 72, 80, 88, 104, 112.
template <bool KC, int ROWS>
struct TileShape {
  static constexpr int PITCH = KC ? kGK + 8 : ROWS + 32;
  static constexpr int ELEMS = KC ? ROWS * PITCH : kGK * PITCH;
};

// One operand's share of a ROWS x 64 stage, loaded through a buffer
// resource: the per-chunk byte offsets are fixed per thread, a K step only
// moves the wave-uniform SGPR offset.  KC: [row][k], 8 chunks of 8 per row;
// else [k][row], ROWS/8 chunks per k.  Rows past the operand's end read a
// clamped (valid) row; they only feed C rows/columns that are not stored.
template <bool KC, int ROWS, int NT>
struct Stage {
  static constexpr int CPR = KC ? kGK / 8 : ROWS / 8;   // chunks per LDS row
  static constexpr int N = ROWS * kGK / 8 / NT;         // chunks per thread
  using Shape = TileShape<KC, ROWS>;
  int voff[N];   // byte offset of the chunk within a stage (k relative to the stage start)
  int lds[N];    // element offset in the LDS tile
  int kk[N];     // k of the chunk within the stage

  __device__ __forceinline__ void init(long ld, int nrows, int row0, int tid) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int i = tid + NT * j;
      const int r = KC ? i / CPR : (i % CPR) * 8;
      const int k = KC ? (i % CPR) * 8 : i / CPR;
      const int rr = min(row0 + r, nrows - (KC ? 1 : 8)) - row0;  // clamped row (relative)
      voff[j] = (int)(KC ? ((long)rr * ld + k) * 2 : ((long)k * ld + rr) * 2);
      lds[j] = KC ? r * Shape::PITCH + k : k * Shape::PITCH + r;
      kk[j] = k;
    }
  }
  // soff: byte offset of the stage start.  Loads only issue (no use of the
  // data here), so several stages can be in flight.
  __device__ __forceinline__ void load(uint4 (&r)[N], __amdgpu_buffer_rsrc_t rs, int soff) const {
#pragma unroll
    for (int j = 0; j < N; ++j)
      r[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff[j], soff, 0));
  }
  // klim: valid k within the stage (wave-uniform; only a split's last stage
  // is partial); chunks past it are written as zeros
  __device__ __forceinline__ void store(const uint4 (&r)[N], bf16_t* tile, int klim) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const uint32_t m = kk[j] < klim ? 0xffffffffu : 0u;
      *reinterpret_cast<uint4*>(&tile[lds[j]]) = make_uint4(r[j].x & m, r[j].y & m, r[j].z & m, r[j].w & m);
    }
  }
};

// MFMA fragment of rows row0 .. row0+31, K sub-step ks (16 k): lane l gets
// X(row0 + l%32, 16 ks + 8 (l/32) + e), e = 0..7 (the A layout; the B layout
// is the same with rows = n).
template <bool KC, int ROWS>
__device__ __forceinline__ bf16x8 gemm_frag(const bf16_t* tile, int row0, int ks) {
  constexpr int P = TileShape<KC, ROWS>::PITCH;
  const int lane = threadIdx.x & 63;
  if constexpr (KC) {
    return *reinterpret_cast<const bf16x8*>(&tile[(row0 + (lane & 31)) * P + ks * 16 + 8 * (lane >> 5)]);
  } else {
    return lds_frag_T<false, false>(tile, P, ks * 16, row0);
  }
}

// OUT: 0 = fp32 C, 1 = bf16 C, 2 = fp32 partial into ws[job][split][M][N]
template <class C, bool AKC, bool BKC, int OUT, class JOBS = DevJobs>
__global__ __launch_bounds__(C::NT) void gemm_kernel(JOBS jobs, int M, int N, int K1, int kper, int tiles_m,
                                                     int tiles_n, int splits, int njobs, int K,
                                                     float* __restrict__ ws) {
  using SA = Stage<AKC, C::BM, C::NT>;
  using SB = Stage<BKC, C::BN, C::NT>;
  __shared__ __align__(16) bf16_t a_lds[2][SA::Shape::ELEMS];
  __shared__ __align__(16) bf16_t b_lds[2][SB::Shape::ELEMS];
  const int tiles = tiles_m * tiles_n;
  const int G = tiles * splits * njobs;
  const int lid = xcd_remap(blockIdx.x, G);
  const int tile = lid % tiles;
  const int split = (lid / tiles) % splits;
  const int jb = lid / (tiles * splits);
  const int m0 = (tile / tiles_n) * C::BM, n0 = (tile % tiles_n) * C::BN;
  const int kbeg = split * kper;
  const int kend = min(K, kbeg + kper);
  const int nk = kend > kbeg ? (kend - kbeg + kGK - 1) / kGK : 0;
  const DevJob& job = jobs.j[jb];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, held in an SGPR
  const int wm = (wave % C::WAVES_M) * 32 * C::TM, wn = (wave / C::WAVES_M) * 32 * C::TN;

  // buffer resources over each operand segment, based at this tile's first
  // row (or column) and the segment's first k, sized to the segment's last
  // element: a stage's rows past the segment's k (a K that is not a multiple
  // of kGK) load zeros instead of reading past the operand
  auto rsrc = [&](const bf16_t* p, long ld, bool kc, int row0, int nrows, int kseg) {
    const long ext = kc ? (long)(nrows - row0 - 1) * ld + kseg : (long)(kseg - 1) * ld + (nrows - row0);
    return make_rsrc(kc ? p + (long)row0 * ld : p + row0, (uint32_t)(kseg > 0 && ext > 0 ? ext * 2 : 0));
  };
  const __amdgpu_buffer_rsrc_t ra1 = rsrc(job.a.p1, job.a.ld, AKC, m0, M, K1),
                               ra2 = rsrc(job.a.p2, job.a.ld, AKC, m0, M, K - K1);
  const __amdgpu_buffer_rsrc_t rb1 = rsrc(job.b.p1, job.b.ld, BKC, n0, N, K1),
                               rb2 = rsrc(job.b.p2, job.b.ld, BKC, n0, N, K - K1);
  // byte offset of k inside its segment
  auto koff = [&](int k, long ld, bool kc) { return (int)(kc ? (long)k * 2 : (long)k * ld * 2); };

  SA sa;
  SB sb;
  sa.init(job.a.ld, M, m0, tid);
  sb.init(job.b.ld, N, n0, tid);
  f32x16 acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j) acc[i][j] = f32x16{};

  // register slots of the stages in flight: slot p holds stages p, p + P, ...
  constexpr int P = C::DEPTH;
  uint4 ra[P][SA::N], rb[P][SB::N];
  // stage indices are clamped to the last stage, so loads are issued
  // unconditionally (a surplus load near the end is never stored) and the
  // compiler can count the loads in flight without merging paths
  auto load_stage = [&](uint4 (&xa)[SA::N], uint4 (&xb)[SB::N], int s) {
    const int k0 = kbeg + min(s, nk - 1) * kGK;
    const bool seg2 = k0 >= K1;
    const int kseg = seg2 ? k0 - K1 : k0;
    sa.load(xa, seg2 ? ra2 : ra1, koff(kseg, job.a.ld, AKC));
    sb.load(xb, seg2 ? rb2 : rb1, koff(kseg, job.b.ld, BKC));
  };
  auto store_stage = [&](const uint4 (&xa)[SA::N], const uint4 (&xb)[SB::N], int buf, int s) {
    const int klim = kend - (kbeg + s * kGK);
    sa.store(xa, a_lds[buf], klim);
    sb.store(xb, b_lds[buf], klim);
  };
  auto compute = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < kGK / 16; ++ks) {
      bf16x8 af[C::TM], bfr[C::TN];
#pragma unroll
      for (int i = 0; i < C::TM; ++i) af[i] = gemm_frag<AKC, C::BM>(a_lds[buf], wm + 32 * i, ks);
#pragma unroll
      for (int j = 0; j < C::TN; ++j) bfr[j] = gemm_frag<BKC, C::BN>(b_lds[buf], wn + 32 * j, ks);
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j) acc[i][j] = mfma32(af[i], bfr[j], acc[i][j]);
    }
  };

  if (nk > 0) {
    // stages 0 .. P-1 in flight, stage 0 to LDS, then its slot takes stage P
#pragma unroll
    for (int p = 0; p < P; ++p) load_stage(ra[p], rb[p], p);
    store_stage(ra[0], rb[0], 0, 0);
    load_stage(ra[0], rb[0], P);
  }
  // LDS-only barriers: the stages in flight stay in flight across them
  lds_barrier();
  // iteration s: compute stage s from LDS buffer s & 1; store stage s + 1
  // (slot (s + 1) % P) into the other buffer, which every wave finished
  // reading before the previous barrier; the slot then takes stage s + 1 + P
  int s0 = 0;
  for (; s0 + P < nk; s0 += P) {  // whole groups of P with a next stage each: no branches
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int s = s0 + p;
      const int q = (p + 1) % P;
      compute(s & 1);
      store_stage(ra[q], rb[q], (s + 1) & 1, s + 1);
      load_stage(ra[q], rb[q], s + 1 + P);
      lds_barrier();
    }
  }
#pragma unroll
  for (int p = 0; p < P; ++p) {  // the last group
    const int s = s0 + p;
    if (s < nk) {
      const int q = (p + 1) % P;
      compute(s & 1);
      if (s + 1 < nk) store_stage(ra[q], rb[q], (s + 1) & 1, s + 1);
      lds_barrier();
    }
  }

  // epilogue: acc[i][j][v] = C(m0 + wm + 32i + acc_row(l/32, v), n0 + wn + 32j + l%32)
  const int g = lane >> 5, col = lane & 31;
  const long ldo = OUT == 2 ? (long)N : job.ldc;
  auto put = [&](int m, int n, float x) {
    if constexpr (OUT == 0) {
      reinterpret_cast<float*>(job.c)[(long)m * ldo + n] = x;
    } else if constexpr (OUT == 1) {
      reinterpret_cast<bf16_t*>(job.c)[(long)m * ldo + n] = f32_to_bf16(x);
    } else {
      ws[((long)jb * splits + split) * M * (long)N + (long)m * ldo + n] = x;
    }
  };
  const bool full = m0 + wm + 32 * C::TM <= M && n0 + wn + 32 * C::TN <= N;  // wave-uniform
  if (full) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) put(m0 + wm + 32 * i + acc_row(g, v), n0 + wn + 32 * j + col, acc[i][j][v]);
  } else {
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j) {
        const int n = n0 + wn + 32 * j + col;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int m = m0 + wm + 32 * i + acc_row(g, v);
          if (m < M && n < N) put(m, n, acc[i][j][v]);
        }
      }
  }
}

// C = sum over splits (ascending) of the partials; 4 consecutive n per thread.
template <int OUT>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(DevJobs jobs, const float* __restrict__ ws, int M, int N,
                                                          int splits) {
  const int jb = blockIdx.y;
  const long i = ((long)blockIdx.x * 256 + threadIdx.x) * 4;
  const long mn = (long)M * N;
  if (i >= mn) return;
  const float* p = ws + (long)jb * splits * mn + i;
  f32x4 s = *reinterpret_cast<const f32x4*>(p);
  for (int sp = 1; sp < splits; ++sp) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p + sp * mn);
    s[0] += v[0];
    s[1] += v[1];
    s[2] += v[2];
    s[3] += v[3];
  }
  const long m = i / N, n = i % N;
  const DevJob& job = jobs.j[jb];
  if constexpr (OUT == 0) {
    float* c = reinterpret_cast<float*>(job.c) + m * job.ldc + n;
    c[0] = s[0];
    c[1] = s[1];
    c[2] = s[2];
    c[3] = s[3];
  } else {
    bf16_t* c = reinterpret_cast<bf16_t*>(job.c) + m * job.ldc + n;
    c[0] = f32_to_bf16(s[0]);
    c[1] = f32_to_bf16(s[1]);
    c[2] = f32_to_bf16(s[2]);
    c[3] = f32_to_bf16(s[3]);
  }
}

// C = sum over jobs (ascending) of the fp32 partials ws[job][M][N] (a grouped
// launch whose jobs add into one output); 4 consecutive elements per thread.
template <int OUT>
__global__ __launch_bounds__(256) void gemm_sum_jobs_kernel(const float* __restrict__ ws, void* __restrict__ c,
                                                            long ldc, int M, int N, int njobs) {
  const long i = ((long)blockIdx.x * 256 + threadIdx.x) * 4;
  const long mn = (long)M * N;
  if (i >= mn) return;
  f32x4 s = *reinterpret_cast<const f32x4*>(ws + i);
  for (int j = 1; j < njobs; ++j) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(ws + j * mn + i);
    s[0] += v[0];
    s[1] += v[1];
    s[2] += v[2];
    s[3] += v[3];
  }
  const long m = i / N, n = i % N;
  if constexpr (OUT == 0) {
    float* o = reinterpret_cast<float*>(c) + m * ldc + n;
    o[0] = s[0];
    o[1] = s[1];
    o[2] = s[2];
    o[3] = s[3];
  } else {
    bf16_t* o = reinterpret_cast<bf16_t*>(c) + m * ldc + n;
    o[0] = f32_to_bf16(s[0]);
    o[1] = f32_to_bf16(s[1]);
    o[2] = f32_to_bf16(s[2]);
    o[3] = f32_to_bf16(s[3]);
  }
}

// Zero-fill through a kernel (a memset node is not safe inside captured HIP graphs).
__global__ __launch_bounds__(256) void zero_fill_kernel(uint8_t* __restrict__ p, size_t bytes) {
  const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 16;
  if (i + 16 <= bytes && ((uintptr_t)(p + i) & 15) == 0) {
    *reinterpret_cast<uint4*>(p + i) = make_uint4(0, 0, 0, 0);
  } else {
    for (size_t j = i; j < i + 16 && j < bytes; ++j) p[j] = 0;
  }
}

hipError_t launch_zero(void* p, size_t bytes, hipStream_t st) {
  if (bytes == 0) return hipSuccess;
  hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)((bytes + 4095) / 4096)), dim3(256), 0, st, (uint8_t*)p, bytes);
  return hipGetLastError();
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

bool gemm_supported(const GemmLaunch& g) {
  if (g.njobs < 1 || g.njobs > 2 || g.M <= 0 || g.N <= 0 || g.K <= 0) return false;
  if (g.M % 8 || g.N % 8 || g.K % 8) return false;
  if (g.K1 < g.K && g.K1 % kGK) return false;
  for (int j = 0; j < g.njobs; ++j) {
    const GemmOp* ops[2] = {&g.job[j].a, &g.job[j].b};
    for (const GemmOp* o : ops) {
      if (o->ld % 8 || !aligned16(o->p1)) return false;
      if (g.K1 < g.K && !aligned16(o->p2)) return false;
      // buffer byte offsets (from a tile's first row and the segment's first k) fit in 31 bits
      const long span = o->kcontig ? (256L * o->ld + g.K) * 2 : ((long)g.K * o->ld + 256) * 2;
      if (span >= 0x7fffffffL) return false;
    }
  }
  return true;
}

// Split-K reduction with the gate epilogue (GemmLaunch::gate_w): the
// ascending sum of the partials is dW'; C = bf16(s dW') and one partial of
// sum dW' * W per workgroup (4 elements per thread, added in a fixed tree).
__global__ __launch_bounds__(256) void gemm_reduce_gate_kernel(const float* __restrict__ ws, long mn, int splits,
                                                               const bf16_t* __restrict__ w,
                                                               const float* __restrict__ s, bf16_t* __restrict__ c,
                                                               float* __restrict__ part) {
  __shared__ float red[256];
  const int tid = threadIdx.x;
  const long i = ((long)blockIdx.x * 256 + tid) * 4;
  float acc = 0.f;
  if (i < mn) {
    const float* p = ws + i;
    f32x4 v = *reinterpret_cast<const f32x4*>(p);
    for (int sp = 1; sp < splits; ++sp) {
      const f32x4 u = *reinterpret_cast<const f32x4*>(p + sp * mn);
      v[0] += u[0];
      v[1] += u[1];
      v[2] += u[2];
      v[3] += u[3];
    }
    const float sc = *s;
    const uint2 wb = *reinterpret_cast<const uint2*>(w + i);
    const float wf[4] = {__uint_as_float(wb.x << 16), __uint_as_float(wb.x & 0xffff0000u),
                         __uint_as_float(wb.y << 16), __uint_as_float(wb.y & 0xffff0000u)};
    uint2 o;
    o.x = (uint32_t)f32_to_bf16(sc * v[0]) | ((uint32_t)f32_to_bf16(sc * v[1]) << 16);
    o.y = (uint32_t)f32_to_bf16(sc * v[2]) | ((uint32_t)f32_to_bf16(sc * v[3]) << 16);
    *reinterpret_cast<uint2*>(c + i) = o;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = fmaf(v[e], wf[e], acc);
  }
  red[tid] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o) red[tid] += red[tid + o];
    __syncthreads();
  }
  if (tid == 0) part[blockIdx.x] = red[0];
}

int gemm_gate_parts(int M, int N) { return (int)(((long)M * N / 4 + 255) / 256); }

size_t gemm_ws_bytes(int njobs, int M, int N, int splits) {
  return splits > 1 ? (size_t)njobs * splits * M * N * sizeof(float) : 0;
}

template <class C, bool AKC, bool BKC>
static void gemm_dispatch(const DevJobs& dj, const GemmLaunch& g, int kper, int splits, const char* name,
                          hipStream_t st) {
  const int tiles_m = (g.M + C::BM - 1) / C::BM, tiles_n = (g.N + C::BN - 1) / C::BN;
  const dim3 grid(tiles_m * tiles_n * splits * g.njobs);
  float* ws = (float*)g.ws;
  // The gate epilogue lives in the split-K reduction, so a gated launch takes
  // the fp32-partial path even when K fits one split (K <= 64 tokens).
  if (splits > 1 || g.gate_w != nullptr) {
    NAYLIS_TIMED(name, st,
                 hipLaunchKernelGGL((gemm_kernel<C, AKC, BKC, 2>), grid, dim3(C::NT), 0, st, dj, g.M, g.N, g.K1, kper,
                                    tiles_m, tiles_n, splits, g.njobs, g.K, ws));
    const dim3 rg((unsigned)(((long)g.M * g.N / 4 + 255) / 256), g.njobs);
    if (g.gate_w != nullptr)
      NAYLIS_TIMED("gemm_reduce", st,
                   hipLaunchKernelGGL(gemm_reduce_gate_kernel, dim3(gemm_gate_parts(g.M, g.N)), dim3(256), 0, st, ws,
                                      (long)g.M * g.N, splits, (const bf16_t*)g.gate_w, g.gate_s,
                                      (bf16_t*)g.job[0].c, g.gate_part));
    else if (g.out == kGemmOutF32)
      NAYLIS_TIMED("gemm_reduce", st,
                   hipLaunchKernelGGL((gemm_reduce_kernel<0>), rg, dim3(256), 0, st, dj, ws, g.M, g.N, splits));
    else
      NAYLIS_TIMED("gemm_reduce", st,
                   hipLaunchKernelGGL((gemm_reduce_kernel<1>), rg, dim3(256), 0, st, dj, ws, g.M, g.N, splits));
  } else if (g.out == kGemmOutF32) {
    NAYLIS_TIMED(name, st,
                 hipLaunchKernelGGL((gemm_kernel<C, AKC, BKC, 0>), grid, dim3(C::NT), 0, st, dj, g.M, g.N, g.K1, kper,
                                    tiles_m, tiles_n, 1, g.njobs, g.K, ws));
  } else {
    NAYLIS_TIMED(name, st,
                 hipLaunchKernelGGL((gemm_kernel<C, AKC, BKC, 1>), grid, dim3(C::NT), 0, st, dj, g.M, g.N, g.K1, kper,
                                    tiles_m, tiles_n, 1, g.njobs, g.K, ws));
  }
}

template <class C>
static void gemm_layouts(const DevJobs& dj, const GemmLaunch& g, int kper, int splits, const char* name,
                         hipStream_t st) {
  const bool ak = g.job[0].a.kcontig, bk = g.job[0].b.kcontig;
  if (ak && bk)
    gemm_dispatch<C, true, true>(dj, g, kper, splits, name, st);
  else if (ak)
    gemm_dispatch<C, true, false>(dj, g, kper, splits, name, st);
  else if (bk)
    gemm_dispatch<C, false, true>(dj, g, kper, splits, name, st);
  else
    gemm_dispatch<C, false, false>(dj, g, kper, splits, name, st);
}

hipError_t launch_gemm(const GemmLaunch& g, const char* name, hipStream_t st) {
  DevJobs dj{};
  for (int j = 0; j < g.njobs; ++j) {
    const GemmJob& s = g.job[j];
    dj.j[j].a = DevOp{(const bf16_t*)s.a.p1, (const bf16_t*)(s.a.p2 ? s.a.p2 : s.a.p1), s.a.ld};
    dj.j[j].b = DevOp{(const bf16_t*)s.b.p1, (const bf16_t*)(s.b.p2 ? s.b.p2 : s.b.p1), s.b.ld};
    dj.j[j].c = s.c;
    dj.j[j].ldc = s.ldc;
  }
  int splits = g.splits < 1 ? 1 : g.splits;
  const int kper = ((g.K + splits - 1) / splits + kGK - 1) / kGK * kGK;
  splits = (g.K + kper - 1) / kper;
  GemmLaunch gl = g;
  gl.K1 = g.K1 < g.K ? g.K1 : g.K;
  // the largest tile that still gives at least one workgroup per CU
  auto wgs = [&](int bm, int bn) {
    return (long)((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn) * splits * g.njobs;
  };
  const long cus = 256;
  const long wide = wgs(CfgWide::BM, CfgWide::BN);
  if (wide >= cus && wide % cus == 0)
    gemm_layouts<CfgWide>(dj, gl, kper, splits, name, st);
  else if (wgs(CfgSmall::BM, CfgSmall::BN) >= cus &&
           !(g.whole_rounds && wgs(CfgSmall::BM, CfgSmall::BN) % cus != 0 && wgs(CfgMid::BM, CfgMid::BN) % cus == 0))
    gemm_layouts<CfgSmall>(dj, gl, kper, splits, name, st);
  else if (wgs(CfgMid::BM, CfgMid::BN) >= cus)
    gemm_layouts<CfgMid>(dj, gl, kper, splits, name, st);
  else
    gemm_layouts<CfgTiny>(dj, gl, kper, splits, name, st);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Grouped launch: njobs GEMMs of one shape and layout in one grid (no K split),
// on the tile launch_gemm would pick for the whole grid.  Every output element
// accumulates over K in the same order as a single launch_gemm of its job, so
// each job's C is bitwise what launch_gemm gives.  With sum_jobs the jobs' fp32
// products go to ws[job][M][N] and one more launch adds them in job order into
// job[0].c.
size_t gemm_grouped_ws_bytes(int njobs, int M, int N, bool sum_jobs) {
  return sum_jobs ? (size_t)njobs * M * N * sizeof(float) : 0;
}

bool gemm_grouped_supported(const GemmGroupedLaunch& g) {
  if (g.njobs < 1 || g.njobs > kGemmMaxGroupJobs) return false;
  if (g.sum_jobs && ((long)g.M * g.N) % 4) return false;
  for (int j = 0; j < g.njobs; ++j) {
    GemmLaunch one{};
    one.job[0] = g.job[j];
    one.njobs = 1;
    one.M = g.M;
    one.N = g.N;
    one.K = g.K;
    one.K1 = g.K1;
    one.out = g.out;
    one.splits = 1;
    if (!gemm_supported(one)) return false;
    if (g.job[j].a.kcontig != g.job[0].a.kcontig || g.job[j].b.kcontig != g.job[0].b.kcontig) return false;
  }
  return true;
}

template <class C, bool AKC, bool BKC>
static void grouped_dispatch(const DevJobsGrouped& dj, const GemmGroupedLaunch& g, int kper, const char* name,
                             hipStream_t st) {
  const int tiles_m = (g.M + C::BM - 1) / C::BM, tiles_n = (g.N + C::BN - 1) / C::BN;
  const dim3 grid(tiles_m * tiles_n * g.njobs);
  const int K1 = g.K1 < g.K ? g.K1 : g.K;
  if (g.sum_jobs)
    NAYLIS_TIMED(name, st,
                 hipLaunchKernelGGL((gemm_kernel<C, AKC, BKC, 2, DevJobsGrouped>), grid, dim3(C::NT), 0, st, dj, g.M,
                                    g.N, K1, kper, tiles_m, tiles_n, 1, g.njobs, g.K, (float*)g.ws));
  else if (g.out == kGemmOutF32)
    NAYLIS_TIMED(name, st,
                 hipLaunchKernelGGL((gemm_kernel<C, AKC, BKC, 0, DevJobsGrouped>), grid, dim3(C::NT), 0, st, dj, g.M,
                                    g.N, K1, kper, tiles_m, tiles_n, 1, g.njobs, g.K, (float*)nullptr));
  else
    NAYLIS_TIMED(name, st,
                 hipLaunchKernelGGL((gemm_kernel<C, AKC, BKC, 1, DevJobsGrouped>), grid, dim3(C::NT), 0, st, dj, g.M,
                                    g.N, K1, kper, tiles_m, tiles_n, 1, g.njobs, g.K, (float*)nullptr));
}

template <class C>
static void grouped_layouts(const DevJobsGrouped& dj, const GemmGroupedLaunch& g, int kper, const char* name,
                            hipStream_t st) {
  const bool ak = g.job[0].a.kcontig, bk = g.job[0].b.kcontig;
  if (ak && bk)
    grouped_dispatch<C, true, true>(dj, g, kper, name, st);
  else if (ak)
    grouped_dispatch<C, true, false>(dj, g, kper, name, st);
  else if (bk)
    grouped_dispatch<C, false, true>(dj, g, kper, name, st);
  else
    grouped_dispatch<C, false, false>(dj, g, kper, name, st);
}

hipError_t launch_gemm_grouped(const GemmGroupedLaunch& g, const char* name, hipStream_t st) {
  DevJobsGrouped dj{};
  for (int j = 0; j < g.njobs; ++j) {
    const GemmJob& s = g.job[j];
    dj.j[j].a = DevOp{(const bf16_t*)s.a.p1, (const bf16_t*)(s.a.p2 ? s.a.p2 : s.a.p1), s.a.ld};
    dj.j[j].b = DevOp{(const bf16_t*)s.b.p1, (const bf16_t*)(s.b.p2 ? s.b.p2 : s.b.p1), s.b.ld};
    dj.j[j].c = s.c;
    dj.j[j].ldc = s.ldc;
  }
  const int kper = (g.K + kGK - 1) / kGK * kGK;
  auto wgs = [&](int bm, int bn) { return (long)((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn) * g.njobs; };
  const long cus = 256;
  const long wide = wgs(CfgWide::BM, CfgWide::BN);
  if (wide >= cus && wide % cus == 0)
    grouped_layouts<CfgWide>(dj, g, kper, name, st);
  else if (wgs(CfgSmall::BM, CfgSmall::BN) >= cus)
    grouped_layouts<CfgSmall>(dj, g, kper, name, st);
  else if (wgs(CfgMid::BM, CfgMid::BN) >= cus)
    grouped_layouts<CfgMid>(dj, g, kper, name, st);
  else
    grouped_layouts<CfgTiny>(dj, g, kper, name, st);
  if (g.sum_jobs) {
    const long mn = (long)g.M * g.N;
    const dim3 rg((unsigned)((mn / 4 + 255) / 256));
    if (g.out == kGemmOutF32)
      NAYLIS_TIMED("gemm_sum_jobs", st,
                   hipLaunchKernelGGL((gemm_sum_jobs_kernel<0>), rg, dim3(256), 0, st, (const float*)g.ws,
                                      g.job[0].c, g.job[0].ldc, g.M, g.N, g.njobs));
    else
      NAYLIS_TIMED("gemm_sum_jobs", st,
                   hipLaunchKernelGGL((gemm_sum_jobs_kernel<1>), rg, dim3(256), 0, st, (const float*)g.ws,
                                      g.job[0].c, g.job[0].ldc, g.M, g.N, g.njobs));
  }
  return hipGetLastError();
}

}  // namespace naylis
