// Pair-tiled read of the shared MoM bank (gfx950): forward, single-pass
// backward and the backward's reduction, for head_dim 64, 128-slot blocks and
// top-2 routing (the Naylis configuration; mom_kernels/triton_gpu.py:64-320
// computes the same read with BLOCK_M = 128 sequence-order tiles).
//
// The order pass (read_order.hip) groups the batch's tokens by their sorted
// block pair (a, b) and cuts each pair's run into tiles of 32 positions, so
// every token of a tile reads exactly the 256 slots of blocks a and b (128
// when a == b).  A work item therefore holds the K / V rows of one pair
// resident for all of its tiles, with no per-tile block lists and no
// per-chunk selection tests:
//
//  * forward: persistent workgroups over the (head, up to 8 tiles of one
//    pair) items, 4 waves;
//    K and V of the pair staged in LDS once, each wave walks its tiles
//    (S^T = K Q^T per 32-slot chunk, online softmax per token column, O^T +=
//    V^T P^T), as the sequence-order kernel of read_fwd.hip does per chunk.
//    It also writes, into a side buffer for the backward, each row's share of
//    its weight on block a (the backward's gate gradients use it).
//  * backward: one workgroup per (head, equal range of the head's tiles), 8
//    waves each owning 32 of the pair's 256 slots.  Per tile S = Q K^T,
//    dP - delta = dO V^T - delta, P and dS once, then dV^T += dO^T P and dK^T
//    += Q^T dS into the waves' register accumulators, dS^T through LDS into
//    dQ^T = K^T dS^T (16 x 16 x 32 products, each wave one 16 x 16 tile over
//    all 256 slots, so dQ is complete in the workgroup and written once) and
//    the per-head gate gradients sum_{n in block} dS (from dS as bf16 plus
//    its bf16 remainder; the products themselves take bf16 operands, whose
//    exponent range holds gradients of any scale).  A range that crosses
//    from one pair to the next writes the pair's dK / dV sums as a partial
//    (segment = range + pair index: unique per (range, pair)) and loads the
//    next pair's rows.
//  * reduce: dK / dV of each block = its partials summed in (pair, range)
//    order, dK scaled; d(gates) = per-head partials summed in head order.
// No floating-point atomics: results are bitwise reproducible.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "launch.h"
#include "read_common.h"
#include "timing.h"

namespace naylis {

namespace {

constexpr int kPHD = 64;              // head_dim of the pair kernels
constexpr int kPBS = 128;             // block size of the pair kernels
constexpr int kPPitch = kPHD + 8;     // LDS row pitch (bf16) of K / V / Q / dO rows
constexpr int kPSlots = 2 * kPBS;     // slots of a pair
constexpr int kPDsPitch = kPairTile + 4;  // LDS row pitch of dS^T (slot rows, token columns; 72 B)

typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Buffer accesses of the tile pipelines.  A lane with nothing to load or
// store passes an offset past every buffer's end: the load returns 0 and the
// store is dropped, so every lane issues the same memory instructions and
// the compiler's in-order counter waits only for what each use needs (a load
// or store skipped on some path makes it wait for everything outstanding).
constexpr uint32_t kOob = 0x80000000u;
__device__ __forceinline__ uint32_t bld32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint4 bld128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ void bst32(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, 0);
}
__device__ __forceinline__ void bst64(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t a, uint32_t b) {
  __builtin_amdgcn_raw_buffer_store_b64(u32x2{a, b}, r, off, 0, 0);
}
__device__ __forceinline__ void bst128(__amdgpu_buffer_rsrc_t r, uint32_t off, const uint4& v) {
  __builtin_amdgcn_raw_buffer_store_b128(u32x4{v.x, v.y, v.z, v.w}, r, off, 0, 0);
}

// 16 x 16 x 32 bf16 product (the backward's dQ^T tiles)
__device__ __forceinline__ f32x4v mfma16(const bf16x8& a, const bf16x8& b, const f32x4v& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Bias (log2 domain) of a token on block e and whether any selection hits it;
// invalid ids select nothing (the key of such a token was formed from clamped
// ids, so it may sit in a tile of a pair it does not read).
__device__ __forceinline__ float pair_bias(int i0, int i1, float l0, float l1, int e, bool& sel) {
  float c = 0.f;
  sel = false;
  if (i0 == e) {
    c += l0;
    sel = true;
  }
  if (i1 == e) {
    c += l1;
    sel = true;
  }
  return c;
}

}  // namespace

// ------------------------------------------------------------------ forward
// Persistent workgroups of 4 waves over ranges of the head-major list of
// (head, work item), an item being up to 4 consecutive tiles of one pair
// (tile w for wave w): the 8 XCDs take one contiguous share each (the
// hardware deals workgroup i to XCD i % 8, so an L2 holds the K / V and q
// columns of about H / 8 heads), cut into equal pieces per CU of the XCD and
// each piece into the contiguous ranges of that CU's two workgroups.  The pair's K / V rows are staged in LDS when the (head,
// pair) changes from one item to the next; the waves then run through the
// pair's items without synchronising.  Per tile (32 tokens; lane column =
// token) a wave forms S^T = K Q^T for all of the pair's slots (eight 32-slot
// chunks held in registers), takes each token's exact maximum m of alpha s +
// c over its selected blocks, then P = exp2(alpha s + c - m) (<= 1: no
// rescaling) with its bf16 row sums, and O^T += V^T P^T.  The wave's next
// tile has its order entry in flight during the scores, its routing and q
// during the weights.  The side table gets each row's backward constants
// (c_a - lse, c_b - lse, block a's share of the row weight, which selections
// hit a / b).
__global__ __launch_bounds__(256, 2) void read_fwd_pair_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const int32_t* __restrict__ top_idx, const float* __restrict__ top_gates, bf16_t* __restrict__ out,
    float* __restrict__ rowtab, float* __restrict__ lse, const int32_t* __restrict__ plan, long N, int H, int L,
    int E, float alpha) {
  constexpr int HD = kPHD, KS = HD / 16, NO = HD / 32, PITCH = kPPitch, NT = 256;
  constexpr int NC = kPSlots / 32;            // 32-slot chunks of a pair
  constexpr int PER = kPSlots * HD / 8 / NT;  // 16-byte pieces per thread per staged tensor
  static_assert(NT / 64 == kPairFwdItem, "one wave per tile of an item");
  __shared__ __attribute__((aligned(16))) bf16_t k_lds[kPSlots * PITCH];
  __shared__ __attribute__((aligned(16))) bf16_t v_lds[kPSlots * PITCH];
  __shared__ int2 tl_lds[kPairFwdMaxRange];  // the range's item words (first position, tokens | blocks)

  const PairPlanLayout pl = pair_plan_layout(N, E);
  const int32_t* ord = plan + 1;
  const int32_t* fitems = plan + pl.fitems;
  const int n_fit = plan[pl.hdr + 2];
  const long T = (long)H * n_fit;
  const int G = gridDim.x, xcd = blockIdx.x & 7, gw = G >> 3, lw = blockIdx.x >> 3;
  // Two workgroups share a CU (workgroups j and j + gw / 2 of an XCD), and
  // the older one wins the issue arbitration, so a CU's time is that of its
  // two ranges together: the XCD share is cut into equal shares per CU, each
  // split between its two workgroups (the first taking the odd item).
  const long s0 = T * xcd / 8, sn = T * (xcd + 1) / 8 - s0;
  long c0, c1;
  if (gw >= 2 && (gw & 1) == 0) {
    const int half = gw >> 1, cu = lw % half;
    const long a0 = s0 + sn * cu / half, a1 = s0 + sn * (cu + 1) / half, am = a0 + (a1 - a0 + 1) / 2;
    c0 = lw < half ? a0 : am;
    c1 = lw < half ? am : a1;
  } else {
    c0 = s0 + sn * lw / gw;
    c1 = s0 + sn * (lw + 1) / gw;
  }
  const int u0 = (int)c0;
  // (the host sizes the grid so a range fits kPairFwdMaxRange: a CU's share
  // is at most 2 kPairFwdMaxRange items)
  const int u1 = (int)std::min<long>(c1, (long)u0 + kPairFwdMaxRange);
  if (u0 >= u1) return;  // uniform over the workgroup
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, col = lane & 31;
  const int D = H * HD;
  for (int i = tid; i < u1 - u0; i += NT) {
    const int it = (u0 + i) % n_fit;
    tl_lds[i] = make_int2(fitems[2 * it], fitems[2 * it + 1]);
  }
  __syncthreads();

  const uint32_t nd_bytes = (uint32_t)(N * D * 2);
  const __amdgpu_buffer_rsrc_t ord_rs = make_rsrc(ord, (uint32_t)N * 4u);
  const __amdgpu_buffer_rsrc_t q_rs = make_rsrc(q, nd_bytes);
  const __amdgpu_buffer_rsrc_t idx_rs = make_rsrc(top_idx, (uint32_t)N * 8u);
  const __amdgpu_buffer_rsrc_t gate_rs = make_rsrc(top_gates, (uint32_t)N * 8u);
  const __amdgpu_buffer_rsrc_t out_rs = make_rsrc(out, nd_bytes);
  const __amdgpu_buffer_rsrc_t lse_rs = make_rsrc(lse, (uint32_t)(N * H) * 4u);
  const __amdgpu_buffer_rsrc_t row_rs = make_rsrc(rowtab, rowtab != nullptr ? (uint32_t)(N * H) * 16u : 0u);
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(k, (uint32_t)L * (uint32_t)D * 2u);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(v, (uint32_t)L * (uint32_t)D * 2u);

  // A tile's token state for this lane (column col): its order entry (first
  // stage), then the token's routing and q fragments (B operand:
  // q[token][16 ks + 8 g ..]).  u = -1 / past the range: nothing.
  struct TileIn {
    int u;
    bool ok;
    int pos, raw;
    long tok;
    int i0, i1;
    float g0, g1;
    bf16x8 qf[KS];
  };
  auto stage_order = [&](TileIn& x, int u) {
    x.u = u;
    int pos0 = 0, cnt = 0;
    if (u < u1) {
      const int2 w = tl_lds[u - u0];
      pos0 = w.x + kPairTile * wave;
      cnt = pair_item_tokens(w.y) - kPairTile * wave;
    }
    x.ok = col < cnt;
    x.pos = pos0 + col;
    x.raw = (int)bld32(ord_rs, x.ok ? (uint32_t)x.pos * 4u : kOob);
  };
  auto stage_data = [&](TileIn& x) {
    const int h = x.u < u1 ? x.u / n_fit : 0;
    // a malformed order entry falls back to its position (wrong results, never
    // an access out of bounds)
    x.tok = x.ok ? ((x.raw >= 0 && x.raw < N) ? (long)x.raw : (long)x.pos) : 0;
    const uint32_t ro = x.ok ? (uint32_t)x.tok * 8u : kOob;
    const int i0v = (int)bld32(idx_rs, ro), i1v = (int)bld32(idx_rs, ro + 4u);
    const float g0v = __uint_as_float(bld32(gate_rs, ro)), g1v = __uint_as_float(bld32(gate_rs, ro + 4u));
    const uint32_t qo = x.ok ? (uint32_t)((x.tok * D + (long)h * HD + 8 * g) * 2) : kOob;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) x.qf[ks] = __builtin_bit_cast(bf16x8, bld128(q_rs, qo + 32u * ks));
    x.i0 = x.ok ? i0v : -1;
    x.i1 = x.ok ? i1v : -1;
    x.g0 = x.ok ? g0v : 1.f;
    x.g1 = x.ok ? g1v : 1.f;
  };

  // this wave's tile of item u (cur), the order entry of its tile of item u
  // + 1 (nxt: fetched a tile ahead), then its data (during item u)
  TileIn cur, nxt;
  stage_order(cur, u0);
  stage_data(cur);
  stage_order(nxt, u0 + 1);
  int kv_h = -1, kv_a = -1, kv_b = -1;  // the (head, pair) whose rows are in LDS
  for (int u = u0; u < u1; ++u) {
    const int2 iw = tl_lds[u - u0];
    const int h = u / n_fit, ba = pair_item_a(iw.y), bb = pair_item_b(iw.y);
    const int nblk = ba == bb ? 1 : 2;
    if (h != kv_h || ba != kv_a || bb != kv_b) {
      // ---- K and V rows of the pair: slots 0..127 block a, 128..255 block
      // b (every wave is done with the previous pair's rows)
      if (u != u0) lds_barrier();
      uint4 kr[PER], vr[PER];
#pragma unroll
      for (int r = 0; r < PER; ++r) {
        const int p = tid + NT * r;
        const int row = p >> 3, c8 = p & 7;
        const uint32_t slot = (uint32_t)((row < kPBS ? ba : bb) * kPBS + (row & (kPBS - 1)));
        const uint32_t off = (slot * (uint32_t)D + (uint32_t)(h * HD + 8 * c8)) * 2u;
        kr[r] = bld128(krs, off);
        vr[r] = bld128(vrs, off);
      }
#pragma unroll
      for (int r = 0; r < PER; ++r) {
        const int p = tid + NT * r;
        const int row = p >> 3, c8 = p & 7;
        *reinterpret_cast<uint4*>(&k_lds[row * PITCH + 8 * c8]) = kr[r];
        *reinterpret_cast<uint4*>(&v_lds[row * PITCH + 8 * c8]) = vr[r];
      }
      lds_barrier();
      kv_h = h;
      kv_a = ba;
      kv_b = bb;
    }
    if (kPairTile * wave < pair_item_tokens(iw.y)) {
      // (keeps the K fragment reads in the loop: hoisted, the 32 fragments
      // would take 128 registers for the whole range)
      asm volatile("" ::: "memory");
      TileIn n2;  // the order entry of the tile of item u + 2
      stage_order(n2, u + 2);

      bool sa, sb;
      const float l0 = log2f(fmaxf(cur.g0, 1e-9f)), l1 = log2f(fmaxf(cur.g1, 1e-9f));
      const float ca = pair_bias(cur.i0, cur.i1, l0, l1, ba, sa);
      const float cbv = pair_bias(cur.i0, cur.i1, l0, l1, bb, sb);
      sb = sb && nblk == 2;

      // ---- S^T chunks (slots 32 c .., tokens): registers 4 j4 .. 4 j4 + 3
      // are slots 8 j4 + 4 g + 0..3 of the chunk.  Chunk c's products are
      // issued beside chunk c - 1's maximum (VALU next to MFMA).
      f32x16 x[NC];
      float mxa = -INFINITY, mxb = -INFINITY;  // the lane's maxima over blocks a, b (alpha > 0)
#pragma unroll
      for (int c = 0; c <= NC; ++c) {
        if (c < NC) {
          x[c] = f32x16{};
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            const bf16x8 a = *reinterpret_cast<const bf16x8*>(&k_lds[(32 * c + col) * PITCH + 16 * ks + 8 * g]);
            x[c] = mfma32(a, cur.qf[ks], x[c]);
          }
        }
        if (c > 0) {
          const float mc = max16(x[c - 1]);
          if (c - 1 < NC / 2) mxa = fmaxf(mxa, mc);
          else mxb = fmaxf(mxb, mc);
        }
      }
      // the next tile's routing and q, in flight during the weights
      stage_data(nxt);

      // ---- the token's maximum over its selected blocks
      mxa = pair_max(mxa);
      mxb = pair_max(mxb);
      const float m = fmaxf(sa ? fmaf(mxa, alpha, ca) : -INFINITY, sb ? fmaf(mxb, alpha, cbv) : -INFINITY);
      const float ms = m == -INFINITY ? 0.f : m;  // no selected block: every weight is 0
      const float adda = sa ? ca - ms : -INFINITY, addb = sb ? cbv - ms : -INFINITY;

      // ---- P (bf16) and its row sums; O^T += V^T P^T, chunk c - 1's
      // products issued beside chunk c's weights
      f32x16 o[NO];
#pragma unroll
      for (int jj = 0; jj < NO; ++jj) o[jj] = f32x16{};
      float l_run = 0.f, la_run = 0.f;
      bf16x8 pk[2][2];
#pragma unroll
      for (int c = 0; c <= NC; ++c) {
        if (c < NC) {
          const float add = c < NC / 2 ? adda : addb;
          f32x16 p;
#pragma unroll
          for (int vv = 0; vv < 16; ++vv) p[vv] = __builtin_amdgcn_exp2f(fmaf(x[c][vv], alpha, add));
          pk[c & 1][0] = pack8(p, 0);
          pk[c & 1][1] = pack8(p, 8);
          l_run += add_bf16x8(pk[c & 1][1], add_bf16x8(pk[c & 1][0], 0.f));
          if (c == NC / 2 - 1) la_run = l_run;
        }
        if (c > 0) {
#pragma unroll
          for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int jj = 0; jj < NO; ++jj) {
              const bf16x8 a = lds_frag_T<true, true>(v_lds, PITCH, 32 * (c - 1) + 16 * kk, 32 * jj);
              o[jj] = mfma32(a, pk[(c - 1) & 1][kk], o[jj]);
            }
        }
      }

      // ---- epilogue: o, lse and the row's backward constants
      const float l = pair_sum(l_run);
      const float la = pair_sum(la_run);
      const long tok = cur.tok;
      const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
      for (int jj = 0; jj < NO; ++jj) {
        const int f0 = 32 * jj + 16 * g;
        f32x16 y;
#pragma unroll
        for (int e = 0; e < 16; ++e) y[e] = o[jj][e] * inv;
        const bf16x8 hi0 = pack8(y, 0), hi1 = pack8(y, 8);
        const uint32_t oo = cur.ok ? (uint32_t)((tok * D + (long)h * HD + f0) * 2) : kOob;
        bst128(out_rs, oo, __builtin_bit_cast(uint4, hi0));
        bst128(out_rs, oo + 16u, __builtin_bit_cast(uint4, hi1));
      }
      const float lse_v = ms + log2f(l);  // -inf for a row with no selected block
      const bool rw = cur.ok && g == 0;
      bst32(lse_rs, rw ? (uint32_t)((long)h * N + tok) * 4u : kOob, __float_as_uint(lse_v));
      if (rowtab != nullptr) {
        const float fa = nblk == 1 ? 1.f : (l > 0.f ? la / l : 0.f);
        const uint32_t sel = (cur.i0 == ba ? 1u : 0u) | (cur.i1 == ba ? 2u : 0u) | (cur.i0 == bb ? 4u : 0u) |
                             (cur.i1 == bb ? 8u : 0u);
        const uint4 row = make_uint4(__float_as_uint(sa ? ca - lse_v : -INFINITY),
                                     __float_as_uint(sb ? cbv - lse_v : -INFINITY), __float_as_uint(fa), sel);
        bst128(row_rs, rw ? (uint32_t)((long)h * N + tok) * 16u : kOob, row);
      }
      cur = nxt;
      nxt = n2;
    } else {
      // no tile of this wave in item u: move the pipeline on
      cur = nxt;
      stage_data(cur);
      stage_order(nxt, u + 2);
    }
  }
}

// ----------------------------------------------------------------- backward
// Workgroup (head h, range r of the head's tiles); wave w owns slots
// 32 w .. 32 w + 31 of the current pair (w < 4: block a, else block b).  The
// tiles run through a software pipeline with one barrier per tile: the step
// of tile t computes
//   S3(t - 1): dQ^T of tile t - 1 over all of the pair's slots and its
//              gate-gradient partials (from the dS^T that S2 left in LDS);
//   S2(t):     P and dS from tile t's S and dP - delta products, dV^T += dO^T P
//              and dK^T += Q^T dS, dS^T to LDS;
//   S1(t + 1): tile t + 1's S and dP - delta products (same pair);
//   S4(t - 2): tile t - 2's gate gradients from its partials;
// and stages tile t + 2's rows, so each barrier separates independent
// product, softmax and staging work of four tiles.  A pair change after
// tile t drains the pipeline: S3(t), S4(t - 1), the finished dK / dV sums as
// partials, the next pair's rows, S4(t), S1(t + 1).  Block b's half (waves 4..7)
// writes its sums per (range, pair), block a's half only when block a changes:
// pairs are sorted by (a, b), so consecutive pairs mostly share block a and a
// range writes one block-a partial per run of equal a.  One-block pairs run
// the same code: block b's bias is -inf, so its weights are zero.
__global__ __launch_bounds__(512, 1) void read_bwd_pair_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const bf16_t* __restrict__ o, const float* __restrict__ rowtab, const bf16_t* __restrict__ dout,
    const int32_t* __restrict__ plan, bf16_t* __restrict__ dq, float* __restrict__ dlg_part,
    float* __restrict__ dk_part, float* __restrict__ dv_part, long N, int H, int L, int E, float alpha,
    float dq_scale, int R, int n_seg_a, int n_seg_b) {
  constexpr int HD = kPHD, KS = HD / 16, NO = HD / 32, PITCH = kPPitch, TQ = kPairTile, NT = 512;
  constexpr int DSP = kPDsPitch;

  // tile t's rows in buffer (t - i0) % 3, its row constants in (t - i0) & 7,
  // its dS^T and gate partials in (t - i0) & 1
  __shared__ __attribute__((aligned(16))) bf16_t q_lds[3][TQ * PITCH];
  __shared__ __attribute__((aligned(16))) bf16_t do_lds[3][TQ * PITCH];
  __shared__ __attribute__((aligned(16))) float ctab[3][3][TQ];  // c_a - lse, c_b - lse, -delta
  __shared__ int32_t tok_lds[8][TQ];                              // token of each row (-1: none)
  __shared__ int32_t sel_lds[8][TQ];                              // which selections hit a (bit 0,1) / b (bit 2,3)
  __shared__ float fa_lds[8][TQ];                                 // the forward's weight share of block a
  __shared__ __attribute__((aligned(16))) bf16_t kt_lds[kPSlots * PITCH];    // the pair's K rows
  __shared__ __attribute__((aligned(16))) bf16_t ds_lds[2][kPSlots * DSP];   // dS^T (bf16)
  __shared__ __attribute__((aligned(16))) bf16_t dsl_lds[2][kPSlots * DSP];  // and its bf16 remainder
  __shared__ float dl_lds[2][4][TQ];  // gate-gradient partials: (block a | b) x (slot half)
  __shared__ int2 tl_lds[kPairBwdMaxRange];  // the range's tile words (first position, count | blocks | pair)

  const PairPlanLayout pl = pair_plan_layout(N, E);
  const int32_t* ord = plan + 1;
  const int32_t* tiles = plan + pl.tiles;
  const int wid = xcd_remap(blockIdx.x, H * R);
  const int h = wid / R, r = wid % R;
  const int n_tiles = plan[pl.hdr];
  const int per = (n_tiles + R - 1) / R;  // at most kPairBwdMaxRange (the host's choice of R)
  const int i0 = min(n_tiles, r * per), i1 = min(min(n_tiles, i0 + per), i0 + kPairBwdMaxRange);
  if (i0 >= i1) return;  // uniform over the workgroup

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, col = lane & 31;
  const int D = H * HD;
  // the range's tile words, so no step of the tile pipeline waits on a plan load
  for (int t = tid; t < i1 - i0; t += NT) tl_lds[t] = make_int2(tiles[2 * (i0 + t)], tiles[2 * (i0 + t) + 1]);
  __syncthreads();
  auto tile_w0 = [&](int t) { return tl_lds[t - i0].x; };
  auto tile_w1 = [&](int t) { return tl_lds[t - i0].y; };
  auto qbuf = [&](int t) { return (t - i0) % 3; };
  auto rbuf = [&](int t) { return (t - i0) & 7; };

  // ---- tile staging: waves 0..3 hold dO and o pieces (token row p >> 3,
  // features 8 (p & 7) ..), waves 4..7 a Q piece; every thread the row
  // constants of row tid % 32 (threads 0..31 keep them)
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int sp = tid & 255, srow = sp >> 3, sc8 = sp & 7, rrow = tid & 31;
  const bool s_do = wave_u < 4;  // wave-uniform
  const uint32_t nd_bytes = (uint32_t)(N * D * 2);
  const __amdgpu_buffer_rsrc_t ord_rs = make_rsrc(ord, (uint32_t)N * 4u);
  const __amdgpu_buffer_rsrc_t a_rs = make_rsrc(s_do ? dout : q, nd_bytes);
  const __amdgpu_buffer_rsrc_t o_rs = make_rsrc(o, nd_bytes);
  const __amdgpu_buffer_rsrc_t row_rs = make_rsrc(rowtab + (long)h * N * 4, (uint32_t)N * 16u);
  const __amdgpu_buffer_rsrc_t dq_rs = make_rsrc(dq, nd_bytes);
  const __amdgpu_buffer_rsrc_t dlg_rs = make_rsrc(dlg_part + (long)h * N * 2, (uint32_t)N * 8u);
  // Staging of one tile: order entries (of the staged piece's row and of row
  // tid % 32), then its data: the dO (or Q) / o piece and the row constants
  // of row tid % 32.  Two sets of each rotate: a tile's order entries are
  // fetched four steps and its data two steps before it is stored to LDS,
  // two steps before its S2.
  struct TokSet {
    int nx_pos, nx_raw, nr_pos, nr_raw;
  };
  struct DataSet {
    uint4 a, o, row;
    int tok;
  };
  auto fetch_tokens = [&](TokSet& ts, int t) {
    const int pos0 = t < i1 ? tile_w0(t) : 0, cnt = t < i1 ? pair_tile_count(tile_w1(t)) : 0;
    ts.nx_pos = srow < cnt ? pos0 + srow : -1;
    ts.nr_pos = rrow < cnt ? pos0 + rrow : -1;
    ts.nx_raw = (int)bld32(ord_rs, ts.nx_pos >= 0 ? (uint32_t)ts.nx_pos * 4u : kOob);
    ts.nr_raw = (int)bld32(ord_rs, ts.nr_pos >= 0 ? (uint32_t)ts.nr_pos * 4u : kOob);
  };
  // a malformed order entry falls back to its position (wrong results, never
  // an access out of bounds)
  auto token_of = [&](int pos, int raw) -> long {
    if (pos < 0) return -1;
    return (raw >= 0 && raw < N) ? (long)raw : (long)pos;
  };
  auto load_tile = [&](DataSet& ds, const TokSet& ts) {
    const long tk = token_of(ts.nx_pos, ts.nx_raw);
    const uint32_t off = tk >= 0 ? (uint32_t)((tk * D + (long)h * HD + 8 * sc8) * 2) : kOob;
    ds.a = bld128(a_rs, off);
    ds.o = bld128(o_rs, s_do ? off : kOob);
    const long tr = token_of(ts.nr_pos, ts.nr_raw);
    ds.tok = (int)tr;
    ds.row = bld128(row_rs, tr >= 0 ? (uint32_t)tr * 16u : kOob);
  };
  // tile t's Q / dO rows, the per-row bias and delta tables (the forward's
  // row constants), tokens and selections
  auto store_tile = [&](int t, const DataSet& ds) {
    const int qb = qbuf(t), rb = rbuf(t);
    if (s_do) {
      *reinterpret_cast<uint4*>(&do_lds[qb][srow * PITCH + 8 * sc8]) = ds.a;
      // delta = sum_f dO_f o_f over the 8 features of the piece, then over the
      // row's 8 threads (o is the forward's bf16 output; its rounding moves
      // the block sums of dS by (delta' - delta) M_x, which S4 removes, and
      // dQ, dK by far less than their tolerance)
      const uint32_t dw[4] = {ds.a.x, ds.a.y, ds.a.z, ds.a.w};
      const uint32_t ow[4] = {ds.o.x, ds.o.y, ds.o.z, ds.o.w};
      float dsum = 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float d0 = __uint_as_float(dw[u] << 16), d1 = __uint_as_float(dw[u] & 0xffff0000u);
        const float o0 = __uint_as_float(ow[u] << 16), o1 = __uint_as_float(ow[u] & 0xffff0000u);
        dsum = fmaf(d0, o0, dsum);
        dsum = fmaf(d1, o1, dsum);
      }
      dsum += dpp_f32<0xb1>(dsum);
      dsum += dpp_f32<0x4e>(dsum);
      dsum += dpp_f32<0x141>(dsum);
      if (sc8 == 0) ctab[qb][2][srow] = -dsum;
    } else {
      *reinterpret_cast<uint4*>(&q_lds[qb][srow * PITCH + 8 * sc8]) = ds.a;
    }
    if (tid < TQ) {
      const bool ok = ds.tok >= 0;
      ctab[qb][0][tid] = ok ? __uint_as_float(ds.row.x) : -INFINITY;
      ctab[qb][1][tid] = ok ? __uint_as_float(ds.row.y) : -INFINITY;
      tok_lds[rb][tid] = ds.tok;
      fa_lds[rb][tid] = ok ? __uint_as_float(ds.row.z) : 1.f;
      sel_lds[rb][tid] = ok ? (int)ds.row.w : 0;
    }
  };

  // ---- the current pair: its K rows in LDS (B operand of S, K^T fragments
  // of dQ), this lane's V slot row in registers (B operand of dP: lane =
  // slot), the dK / dV accumulators
  int key = -1, pa = -1, pb = -1;
  f32x16 acc_dk[NO], acc_dv[NO];
  bf16x8 vf[KS];
  const int w_slot = 32 * wave + col;  // this lane's slot in the pair (0..255)
  auto enter_pair = [&](int t) {
    const int w1 = __builtin_amdgcn_readfirstlane(tile_w1(t));
    key = pair_tile_key(w1);
    const int na = pair_tile_a(w1);
    // block a's half keeps its sums while block a stays (the previous pair's
    // were written by flush otherwise); block b's half starts over
    const bool zero = wave >= 4 || na != pa;
    pa = na;
    pb = pair_tile_b(w1);
    constexpr int PR = kPSlots * HD / 8 / NT;
#pragma unroll
    for (int rr = 0; rr < PR; ++rr) {
      const int p = tid + NT * rr;
      const int row = p >> 3, c8 = p & 7;
      const long off = ((long)(row < kPBS ? pa : pb) * kPBS + (row & (kPBS - 1))) * D + (long)h * HD + 8 * c8;
      *reinterpret_cast<uint4*>(&kt_lds[row * PITCH + 8 * c8]) = *reinterpret_cast<const uint4*>(k + off);
    }
    {
      const long srow_g = (long)(w_slot < kPBS ? pa : pb) * kPBS + (w_slot & (kPBS - 1));
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const long off = srow_g * D + (long)h * HD + 16 * ks + 8 * g;
        vf[ks] = *reinterpret_cast<const bf16x8*>(v + off);
      }
    }
    if (zero) {
#pragma unroll
      for (int j = 0; j < NO; ++j) {
        acc_dk[j] = f32x16{};
        acc_dv[j] = f32x16{};
      }
    }
  };
  // Transposed 16x16x32 operand from natural LDS rows: lane l gets
  // X[s0 + 8 (l/16) + e][c0 + l % 16], e = 0..7, for a tile X with slot rows
  // (pitch `pitch`) -- two transposing reads; within each 16-lane group,
  // input lane 4e + c reads columns c0 + 4c .. c0 + 4c + 3 of row s0' + e.
  auto frag16_T = [&](const bf16_t* tile, int pitch, int s0, int c0) {
    const int q4 = (lane >> 4) & 3, j = lane & 15;
    const bf16_t* base = &tile[(s0 + 8 * q4 + (j >> 2)) * pitch + c0 + 4 * (j & 3)];
    const v4i16 lo = lds_read_tr16(base);
    const v4i16 hi = lds_read_tr16(base + 4 * pitch);
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };
  // the finished sums before the pair `next` (-1: the range's end): block b's
  // half as the (range, pair) partial, segment r + key of the B partials;
  // block a's half, when block a changes, as the (range, block-a run)
  // partial, segment r + a of the A partials (both unique: ranges and pairs
  // are contiguous and sorted).  Rows: the block's 128 slots.
  auto flush = [&](int next_a) {
    long base;
    if (wave < 4) {
      if (next_a == pa) return;
      base = (((long)h * n_seg_a + (r + pa)) * kPBS + w_slot) * HD;
    } else {
      if (pa == pb) return;  // a one-block pair: block b's half is zeros
      base = ((long)H * n_seg_a * kPBS + ((long)h * n_seg_b + (r + key)) * kPBS + (w_slot - kPBS)) * HD;
    }
#pragma unroll
    for (int j = 0; j < NO; ++j) {
      const int f0 = 32 * j + 16 * g;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        *reinterpret_cast<f32x4*>(dk_part + base + f0 + 4 * u) =
            f32x4{acc_dk[j][4 * u], acc_dk[j][4 * u + 1], acc_dk[j][4 * u + 2], acc_dk[j][4 * u + 3]};
        *reinterpret_cast<f32x4*>(dv_part + base + f0 + 4 * u) =
            f32x4{acc_dv[j][4 * u], acc_dv[j][4 * u + 1], acc_dv[j][4 * u + 2], acc_dv[j][4 * u + 3]};
      }
    }
  };

  // ---- S1(t): S = Q K^T and dP - delta = dO V^T - delta for this wave's 32
  // slots x the tile's 32 tokens (registers 4 j4 .. 4 j4 + 3 are tokens
  // 8 j4 + 4 g + 0..3)
  f32x16 acc_s, acc_p;
  auto s1 = [&](int t) {
    const int qb = qbuf(t);
#pragma unroll
    for (int j4 = 0; j4 < 4; ++j4) {
      const f32x4 nd = *reinterpret_cast<const f32x4*>(&ctab[qb][2][8 * j4 + 4 * g]);
#pragma unroll
      for (int u = 0; u < 4; ++u) acc_p[4 * j4 + u] = nd[u];
    }
    acc_s = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int off = col * PITCH + 16 * ks + 8 * g;
      const bf16x8 aq = *reinterpret_cast<const bf16x8*>(&q_lds[qb][off]);
      const bf16x8 ad = *reinterpret_cast<const bf16x8*>(&do_lds[qb][off]);
      const bf16x8 bk = *reinterpret_cast<const bf16x8*>(&kt_lds[w_slot * PITCH + 16 * ks + 8 * g]);
      acc_s = mfma32(aq, bk, acc_s);
      acc_p = mfma32(ad, vf[ks], acc_p);
    }
  };
  // ---- S2(t): P, dS; dV^T += dO^T P with P as bf16 plus its bf16 remainder
  // (two products: ~2^-16 relative; bf16 P alone, all terms of one sign,
  // leaves 2^-9 per term in sums over thousands of tokens), dK^T += Q^T dS
  // with bf16 dS (terms of both signs); dS^T and its remainder to LDS for S3
  // (dQ takes the bf16 part, the gate sums both)
  auto s2 = [&](int t, auto par) {
    constexpr int B2 = decltype(par)::value;
    const int qb = qbuf(t);
    const int bsel = wave >> 2;  // 0: block a, 1: block b
#pragma unroll
    for (int j4 = 0; j4 < 4; ++j4) {
      const f32x4 c4 = *reinterpret_cast<const f32x4*>(&ctab[qb][bsel][8 * j4 + 4 * g]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int vv = 4 * j4 + u;
        const float p = __builtin_amdgcn_exp2f(fmaf(acc_s[vv], alpha, c4[u]));
        acc_s[vv] = p;
        acc_p[vv] = p * acc_p[vv];
      }
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      bf16x8 bp, bpl, bd, bdl;
      pack8_hilo(acc_s, 8 * kk, bp, bpl);
      pack8_hilo(acc_p, 8 * kk, bd, bdl);
#pragma unroll
      for (int j = 0; j < NO; ++j) {
        const bf16x8 a_do = lds_frag_T<true, true>(do_lds[qb], PITCH, 16 * kk, 32 * j);
        const bf16x8 a_q = lds_frag_T<true, true>(q_lds[qb], PITCH, 16 * kk, 32 * j);
        acc_dv[j] = mfma32(a_do, bpl, mfma32(a_do, bp, acc_dv[j]));
        acc_dk[j] = mfma32(a_q, bd, acc_dk[j]);
      }
      // registers 8 kk .. 8 kk + 7 are tokens 16 kk + 4 g + 0..3 and 16 kk + 8 + 4 g + 0..3
      const uint4 u = __builtin_bit_cast(uint4, bd), ul = __builtin_bit_cast(uint4, bdl);
      const int dso = w_slot * DSP + 16 * kk + 4 * g;
      *reinterpret_cast<uint2*>(&ds_lds[B2][dso]) = make_uint2(u.x, u.y);
      *reinterpret_cast<uint2*>(&ds_lds[B2][dso + 8]) = make_uint2(u.z, u.w);
      *reinterpret_cast<uint2*>(&dsl_lds[B2][dso]) = make_uint2(ul.x, ul.y);
      *reinterpret_cast<uint2*>(&dsl_lds[B2][dso + 8]) = make_uint2(ul.z, ul.w);
    }
  };
  // ---- S3(t): dQ^T tile (features 16 (w & 3) .., tokens 16 (w >> 2) ..)
  // over the pair's slots, and the gate-gradient partials: wave with
  // w & 3 == c sums dS over K-steps 2c, 2c + 1 (block a for c < 2, b
  // otherwise)
  auto s3 = [&](int t, auto par) {
    constexpr int B3 = decltype(par)::value;
    const int tq = wave >> 2, fq = wave & 3;
    const int q4 = (lane >> 4) & 3, j = lane & 15;
    f32x4v accq0 = f32x4v{0.f, 0.f, 0.f, 0.f}, accq1 = accq0;
#pragma unroll
    for (int kk = 0; kk < 8; kk += 2) {
      // A: K^T (features 16 fq .., slots 32 kk ..); B: dS^T (slots, tokens 16 tq ..)
      accq0 = mfma16(frag16_T(kt_lds, PITCH, 32 * kk, 16 * fq), frag16_T(ds_lds[B3], DSP, 32 * kk, 16 * tq), accq0);
      accq1 = mfma16(frag16_T(kt_lds, PITCH, 32 * kk + 32, 16 * fq),
                     frag16_T(ds_lds[B3], DSP, 32 * kk + 32, 16 * tq), accq1);
    }
    float gsum = 0.f;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int kk = 2 * fq + jj;
      gsum = add_bf16x8(frag16_T(ds_lds[B3], DSP, 32 * kk, 16 * tq), gsum);
      gsum = add_bf16x8(frag16_T(dsl_lds[B3], DSP, 32 * kk, 16 * tq), gsum);
    }
    // the four 16-lane groups hold different slots of the same token
    gsum = xor16_f32(gsum, [](float a, float b) { return a + b; });
    gsum = xor32_f32(gsum, [](float a, float b) { return a + b; });
    if (lane < 16) dl_lds[B3][fq][16 * tq + lane] = gsum;
    // dQ rows: lane holds features 16 fq + 4 (l / 16) + 0..3 of token row 16 tq + l % 16
    const f32x4v accq = accq0 + accq1;
    const int tk = tok_lds[rbuf(t)][16 * tq + j];
    const uint32_t px = (uint32_t)f32_to_bf16(accq[0] * dq_scale) | ((uint32_t)f32_to_bf16(accq[1] * dq_scale) << 16);
    const uint32_t py = (uint32_t)f32_to_bf16(accq[2] * dq_scale) | ((uint32_t)f32_to_bf16(accq[3] * dq_scale) << 16);
    bst64(dq_rs, tk >= 0 ? (uint32_t)(((long)tk * D + (long)h * HD + 16 * fq + 4 * q4) * 2) : kOob, px, py);
  };
  // ---- S4(t): gate gradients of tile t (partials of S3(t)): every thread
  // computes row tid % 32, threads 0..31 store it.  With P recomputed from
  // lse (fp32 weights over the bf16 row sum) and delta from o (the bf16
  // weights), sum_n dS_n over both blocks, which is 0 for the exact softmax,
  // keeps a residue (delta' - delta) S; the block sums are G_x = A_x - delta'
  // M_x, so G_a - (M_a / S)(G_a + G_b) is the exact A_a - delta M_a.  M_a / S
  // is the forward's share of the row weight on block a (its error only
  // scales that small residue).
  auto s4 = [&](int t, auto par) {
    constexpr int B4 = decltype(par)::value;
    const int rb = rbuf(t);
    const int tk = tok_lds[rb][rrow];
    const int sm = sel_lds[rb][rrow];
    const float fa = fa_lds[rb][rrow];
    const float g0 = dl_lds[B4][0][rrow] + dl_lds[B4][1][rrow];
    const float g1 = dl_lds[B4][2][rrow] + dl_lds[B4][3][rrow];
    const float tot = g0 + g1;
    const float ga = g0 - fa * tot;
    const float gb = g1 - (1.f - fa) * tot;
    const float d0 = (sm & 1) ? ga : ((sm & 4) ? gb : 0.f);
    const float d1 = (sm & 2) ? ga : ((sm & 8) ? gb : 0.f);
    bst64(dlg_rs, (tid < TQ && tk >= 0) ? (uint32_t)tk * 8u : kOob, __float_as_uint(d0), __float_as_uint(d1));
  };

  // ---- prologue: the first pair entered; tiles i0, i0 + 1 staged, the data
  // of i0 + 2, i0 + 3 and the order entries of i0 + 4, i0 + 5 in flight;
  // S1(i0).  Staging sets of parity (t - i0) & 1 serve tile t.
  TokSet tks[2];
  DataSet dts[2];
  enter_pair(i0);
  fetch_tokens(tks[0], i0);
  fetch_tokens(tks[1], i0 + 1);
  load_tile(dts[0], tks[0]);
  load_tile(dts[1], tks[1]);
  fetch_tokens(tks[0], i0 + 2);
  fetch_tokens(tks[1], i0 + 3);
  store_tile(i0, dts[0]);
  store_tile(i0 + 1, dts[1]);
  load_tile(dts[0], tks[0]);
  load_tile(dts[1], tks[1]);
  fetch_tokens(tks[0], i0 + 4);
  fetch_tokens(tks[1], i0 + 5);
  lds_barrier();
  s1(i0);
  int s3_done = i0 - 1, s4_done = i0 - 1;  // the last tiles whose S3 / S4 ran (uniform)

  // one step of the pipeline; P = (t - i0) & 1 as a compile-time constant
  // (the loop below is unrolled by two), so the staging sets stay in registers
  auto step = [&](auto par, int t) {
    constexpr int P = decltype(par)::value;
    using Pc = std::integral_constant<int, P>;
    using Qc = std::integral_constant<int, P ^ 1>;
    const int nkey = t + 1 < i1 ? (int)__builtin_amdgcn_readfirstlane(pair_tile_key(tile_w1(t + 1))) : -1;
    const bool cont = nkey == key;  // tile t + 1 in the current pair
    if (t - 1 > s3_done) s3(t - 1, Qc{});
    s2(t, Pc{});
    if (cont) s1(t + 1);
    if (t - 2 > s4_done) s4(t - 2, Pc{});
    store_tile(t + 2, dts[P]);
    load_tile(dts[P], tks[P]);     // tile t + 4
    fetch_tokens(tks[P], t + 6);
    lds_barrier();
    s3_done = max(s3_done, t - 1);
    s4_done = max(s4_done, t - 2);
    if (!cont) {
      // drain: tile t's dQ and gates (S4(t - 1) beside S3(t): other
      // partial buffers), the pair's sums, then the next pair
      s3(t, Pc{});
      if (t - 1 > s4_done) s4(t - 1, Qc{});
      flush(t + 1 < i1 ? (int)__builtin_amdgcn_readfirstlane(pair_tile_a(tile_w1(t + 1))) : -1);
      lds_barrier();  // S3(t) is done with kt_lds and has written tile t's partials
      s4(t, Pc{});
      if (t + 1 < i1) {
        enter_pair(t + 1);
        lds_barrier();  // the next pair's K rows complete (S1 reads other waves' rows)
        s1(t + 1);
      }
      s3_done = t;
      s4_done = t;
    }
  };
  for (int t = i0; t < i1; t += 2) {
    step(std::integral_constant<int, 0>{}, t);
    if (t + 1 < i1) step(std::integral_constant<int, 1>{}, t + 1);
  }
}

// ------------------------------------------------------------------- reduce
// dK / dV of block e (rows e * 128 ..), head h, an eighth of its slots: the
// A partials of the run of pairs (e, *) over its ranges (ascending), then
// for each pair (a, e) with a != e (ascending) the B partials over its
// ranges (ascending); dK scaled.  A thread holds one float4 of each tensor,
// so a batch of 16 partials' loads is in flight at once.
// Workgroups past the dK / dV ones sum the per-head gate-gradient partials
// (head order) into d(top_gates) through log(max(g, 1e-9)).
constexpr int kPairReduceParts = 8;  // workgroups per (head, block)
__global__ __launch_bounds__(256) void read_pair_reduce_kernel(
    const float* __restrict__ dk_part, const float* __restrict__ dv_part, const int32_t* __restrict__ plan,
    bf16_t* __restrict__ dk, bf16_t* __restrict__ dv, long N, int H, int E, int R, int n_seg_a, int n_seg_b,
    float dk_scale,
    int kv_blocks, const float* __restrict__ dlg_part, const float* __restrict__ top_gates,
    float* __restrict__ dgates) {
  constexpr int HD = kPHD, QS = kPBS / kPairReduceParts;  // slots per workgroup
  constexpr int MK = kPairBwdMaxE * (kPairBwdMaxE + 1) / 2;
  __shared__ long seg_off[1024];  // first float of each partial's block rows
  __shared__ int4 key_lds[MK];    // the pair table (block a, block b, first tile, tiles)
  __shared__ int n_s;
  if ((int)blockIdx.x >= kv_blocks) {
    const long n = N * 2;
    const long nb = gridDim.x - kv_blocks;
    for (long i = (blockIdx.x - kv_blocks) * (long)blockDim.x + threadIdx.x; i < n; i += nb * blockDim.x) {
      float s = 0.f;
      int hh = 0;
      for (; hh + 8 <= H; hh += 8) {
        float t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) t[u] = dlg_part[(long)(hh + u) * n + i];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += t[u];
      }
      for (; hh < H; ++hh) s += dlg_part[(long)hh * n + i];
      const float gt = top_gates[i];
      dgates[i] = gt >= 1e-9f ? s / gt : 0.f;
    }
    return;
  }
  const PairPlanLayout pl = pair_plan_layout(N, E);
  const int b = blockIdx.x;
  const int part = b % kPairReduceParts, e = (b / kPairReduceParts) % E, h = (b / kPairReduceParts) / E;
  const int n_tiles = plan[pl.hdr], n_keys = plan[pl.hdr + 1];
  const int per = (n_tiles + R - 1) / R;
  const int nk = min(n_keys, MK);  // (the backward's pair path takes E <= kPairBwdMaxE)
  for (int i = threadIdx.x; i < nk; i += blockDim.x)
    key_lds[i] = make_int4(plan[pl.keys + 4 * i], plan[pl.keys + 4 * i + 1], plan[pl.keys + 4 * i + 2],
                           plan[pl.keys + 4 * i + 3]);
  __syncthreads();
  static_assert(MK <= 64, "one pair per lane of wave 0");
  if (threadIdx.x < 64) {
    // wave 0, lane k = pair k: the run (e, *)'s tile span (its A partials),
    // then pair k's B partials when it is (a, e) with a != e, placed by a
    // prefix count over the lanes
    const int k = threadIdx.x;
    const long rows = (long)kPBS * HD;
    const int4 kr = k < nk ? key_lds[k] : make_int4(-1, -1, 0, 0);
    const bool in_run = kr.x == e && kr.w > 0;
    int t_first = in_run ? kr.z : 0x7fffffff, t_last = in_run ? kr.z + kr.w - 1 : -1;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      t_first = min(t_first, __shfl_xor(t_first, o));
      t_last = max(t_last, __shfl_xor(t_last, o));
    }
    const int na = t_last >= 0 ? t_last / per - t_first / per + 1 : 0;
    const bool is_b = kr.y == e && kr.x != e && kr.w > 0;
    const int nb = is_b ? (kr.z + kr.w - 1) / per - kr.z / per + 1 : 0;
    int incl = nb;  // inclusive prefix of nb over the lanes
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o);
      if (k >= o) incl += y;
    }
    const int total = na + __shfl(incl, 63);
    for (int i = k; i < na; i += 64)
      if (i < 1024) seg_off[i] = ((long)h * n_seg_a + t_first / per + i + e) * rows;
    for (int i = 0, at = na + incl - nb; i < nb; ++i)
      if (at + i < 1024) seg_off[at + i] = (long)H * n_seg_a * rows + ((long)h * n_seg_b + kr.z / per + i + k) * rows;
    if (k == 0) n_s = min(total, 1024);
  }
  __syncthreads();
  const int ns = n_s;
  const int D = H * HD;
  // 16 slots x 64 features = 256 float4 per tensor: one per thread, all of a
  // batch of 16 partials' loads in flight before the (ascending) sums
  constexpr int NB = 16;
  static_assert(QS * HD / 4 == 256, "one float4 per thread and tensor");
  const int s_in = part * QS + (int)threadIdx.x / (HD / 4);  // slot within the block
  const int f4 = (int)threadIdx.x % (HD / 4);
  f32x4 sk = f32x4{0.f, 0.f, 0.f, 0.f}, sv = sk;
  for (int i = 0; i < ns; i += NB) {
    f32x4 pk[NB], pv[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u)
      if (i + u < ns) {
        const long off = seg_off[i + u] + (long)s_in * HD + 4 * f4;
        pk[u] = *reinterpret_cast<const f32x4*>(dk_part + off);
        pv[u] = *reinterpret_cast<const f32x4*>(dv_part + off);
      }
#pragma unroll
    for (int u = 0; u < NB; ++u)
      if (i + u < ns) {
        sk += pk[u];
        sv += pv[u];
      }
  }
  bf16x4 ok, ov;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    ok[u] = (__bf16)(sk[u] * dk_scale);
    ov[u] = (__bf16)sv[u];
  }
  const long dst = ((long)e * kPBS + s_in) * D + (long)h * HD + 4 * f4;
  *reinterpret_cast<bf16x4*>(dk + dst) = ok;
  *reinterpret_cast<bf16x4*>(dv + dst) = ov;
}

// ------------------------------------------------------------------ host side
bool read_pair_fwd_shapes(const ReadDims& d, long N) {
  // (byte offsets of the token-indexed buffers and of K / V fit 31 bits)
  return d.HD == kPHD && d.block_size == kPBS && d.topk == 2 && d.E <= kPairMaxE &&
         read_has_pair_plan(N, d.E, d.topk) && (long)d.L * d.H * d.HD * 2 < (1L << 31) &&
         N * d.H * d.HD * 2 < (1L << 31);
}
bool read_pair_bwd_shapes(const ReadDims& d, long N) { return read_pair_fwd_shapes(d, N) && d.E <= kPairBwdMaxE; }
bool read_pair_fwd_ok(const ReadDims& d, long N) { return d.order != nullptr && read_pair_fwd_shapes(d, N); }
bool read_pair_bwd_ok(const ReadDims& d, long N) { return d.order != nullptr && read_pair_bwd_shapes(d, N); }

int read_pair_ranges(const ReadDims& d) {
  const long N = (long)d.B * d.S;
  const int want = d.H >= 256 ? 1 : 256 / d.H;  // one round of workgroups
  const int tiles = pair_plan_layout(N, d.E).max_tiles;
  // at least 4 tiles a range, at most kPairBwdMaxRange (the range's tile words sit in LDS)
  const int r = std::max(1, std::min(want, (tiles + 3) / 4));
  return std::max(r, (tiles + kPairBwdMaxRange - 1) / kPairBwdMaxRange);
}

// partial segments: A (per range and block-a run: r + a) and B (per range
// and pair: r + pair index)
int read_pair_segments_a(const ReadDims& d) { return read_pair_ranges(d) + d.E - 1; }
int read_pair_segments(const ReadDims& d) {
  const long N = (long)d.B * d.S;
  return read_pair_ranges(d) + pair_plan_layout(N, d.E).max_keys - 1;
}

size_t read_pair_part_bytes(const ReadDims& d) {
  return (size_t)d.H * (read_pair_segments_a(d) + read_pair_segments(d)) * kPBS * kPHD * sizeof(float);
}

// the side buffer: each row's backward constants, (H, N, 4) 32-bit words
// (c_a - lse, c_b - lse, block a's share of the row weight, selection bits)
size_t read_pair_side_bytes(const ReadDims& d) { return (size_t)d.B * d.S * d.H * 16; }

// Compute units of the current device (cached per device; 256 on MI355X).
static int pair_device_cus() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int c = cached[dev].load(std::memory_order_relaxed);
  if (c > 0) return c;
  if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
  cached[dev].store(c, std::memory_order_relaxed);
  return c;
}

hipError_t launch_read_fwd_pair(const void* q, const void* k, const void* v, const int32_t* top_idx,
                                const float* top_gates, void* out, void* side, float* lse, const ReadDims& d,
                                hipStream_t st) {
  const long N = (long)d.B * d.S;
  // two workgroups per CU (LDS: 74 KiB each) in 8 equal XCD groups, no more
  // than the work items can use (at most one per tile), and enough that a
  // range fits kPairFwdMaxRange
  const long items = (long)d.H * pair_plan_layout(N, d.E).max_tiles;
  const long per_xcd = (items + 7) / 8;
  const long gw = std::max<long>(std::max<long>(1, std::min<long>(2L * pair_device_cus() / 8, per_xcd)),
                                 (per_xcd + kPairFwdMaxRange - 1) / kPairFwdMaxRange);
  const float alpha = (float)(1.0 / __builtin_sqrt(64.0)) * kLog2e;  // > 0, as the kernel's maximum assumes
  NAYLIS_TIMED("read_fwd", st,
               hipLaunchKernelGGL(read_fwd_pair_kernel, dim3((unsigned)(8 * gw)), dim3(256), 0, st,
                                  (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, top_idx, top_gates,
                                  (bf16_t*)out, (float*)side, lse, d.order, N, d.H, d.L, d.E, alpha));
  return hipGetLastError();
}

hipError_t launch_read_bwd_pair(const void* q, const void* k, const void* v, const int32_t* top_idx,
                                const float* top_gates, const void* o, const void* side, const void* dout,
                                const float* lse, void* dq, void* dk, void* dv, float* dgates, float* dlg_part,
                                float* dk_part, float* dv_part, const ReadDims& d, hipStream_t st) {
  const long N = (long)d.B * d.S;
  const int R = read_pair_ranges(d);
  const int nsa = read_pair_segments_a(d), ns = read_pair_segments(d);
  const float alpha = (float)(1.0 / __builtin_sqrt(64.0)) * kLog2e;
  const float scale = (float)(1.0 / __builtin_sqrt(64.0));
  NAYLIS_TIMED("read_bwd_pair", st,
               hipLaunchKernelGGL(read_bwd_pair_kernel, dim3(d.H * R), dim3(512), 0, st, (const bf16_t*)q,
                                  (const bf16_t*)k, (const bf16_t*)v, (const bf16_t*)o, (const float*)side,
                                  (const bf16_t*)dout, d.order, (bf16_t*)dq, dlg_part,
                                  dk_part, dv_part, N, d.H, d.L, d.E, alpha, scale, R, nsa, ns));
  const int kv_blocks = d.H * d.E * kPairReduceParts;
  const int g_blocks = (int)std::min<long>(1024, (N * 2 + 255) / 256);
  NAYLIS_TIMED("read_bwd_reduce", st,
               hipLaunchKernelGGL(read_pair_reduce_kernel, dim3(kv_blocks + g_blocks), dim3(256), 0, st, dk_part,
                                  dv_part, d.order, (bf16_t*)dk, (bf16_t*)dv, N, d.H, d.E, R, nsa, ns, scale,
                                  kv_blocks,
                                  dlg_part, top_gates, dgates));
  return hipGetLastError();
}

}  // namespace naylis
