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
//  * forward: one workgroup per (head, up to 8 tiles of one pair), 4 waves;
//    K and V of the pair staged in LDS once, each wave walks its tiles
//    (S^T = K Q^T per 32-slot chunk, online softmax per token column, O^T +=
//    V^T P^T), as the sequence-order kernel of read_fwd.hip does per chunk.
//    It also writes, into a side buffer for the backward, o's bf16 remainder
//    (o - bf16(o)), from which the backward forms delta = rowsum(o * dO) to
//    fp32 accuracy, and each row's share of its weight on block a.
//  * backward: one workgroup per (head, equal range of the head's tiles), 8
//    waves each owning 32 of the pair's 256 slots.  Per tile S = Q K^T,
//    dP - delta = dO V^T - delta, P and dS once, then dV^T += dO^T P and dK^T
//    += Q^T dS into the waves' register accumulators, dS^T through LDS into
//    dQ^T = K^T dS^T (16 x 16 x 32 products, each wave one 16 x 16 tile over
//    all 256 slots, so dQ is complete in the workgroup and written once) and
//    the per-head gate gradients sum_{n in block} dS.  A range that crosses
//    from one pair to the next writes the pair's dK / dV sums as a partial
//    (segment = range + pair index: unique per (range, pair)) and loads the
//    next pair's rows.
//  * reduce: dK / dV of each block = its partials summed in (pair, range)
//    order, dK scaled; d(gates) = per-head partials summed in head order.
// No floating-point atomics: results are bitwise reproducible.
#include <algorithm>

#include "launch.h"
#include "read_common.h"
#include "timing.h"

namespace naylis {

namespace {

constexpr int kPHD = 64;              // head_dim of the pair kernels
constexpr int kPBS = 128;             // block size of the pair kernels
constexpr int kPPitch = kPHD + 8;     // LDS row pitch (bf16) of K / V / Q / dO rows
constexpr int kPSlots = 2 * kPBS;     // slots of a pair
constexpr int kPDsPitch = kPairTile + 8;  // LDS row pitch of dS^T (slot rows, token columns)

typedef float f32x4v __attribute__((ext_vector_type(4)));

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
// Workgroup (head h, forward item): the item's tiles are 32-position slices
// of one pair's run of the order, wave w takes slices w, w + 4, ...  Each
// wave fetches the next slice's tokens while it computes the current one
// (order entry at the slice's start, routing and q after block a), so the
// dependent loads of a slice overlap the previous slice's products.
__global__ __launch_bounds__(256, 2) void read_fwd_pair_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const int32_t* __restrict__ top_idx, const float* __restrict__ top_gates, bf16_t* __restrict__ out,
    bf16_t* __restrict__ out_lo, float* __restrict__ frac_a, float* __restrict__ lse,
    const int32_t* __restrict__ plan, long N, int H, int L, int E, float alpha, int max_items) {
  constexpr int HD = kPHD, KS = HD / 16, NO = HD / 32, PITCH = kPPitch, NT = 256, NW = NT / 64;
  constexpr int PER = kPSlots * HD / 8 / NT;  // 16-byte pieces per thread per staged tensor
  __shared__ __attribute__((aligned(16))) bf16_t k_lds[kPSlots * PITCH];
  __shared__ __attribute__((aligned(16))) bf16_t v_lds[kPSlots * PITCH];

  const PairPlanLayout pl = pair_plan_layout(N, E);
  const int32_t* ord = plan + 1;
  const int wid = xcd_remap(blockIdx.x, H * max_items);  // head-major: a head's items share one L2
  const int h = wid / max_items, it = wid % max_items;
  // the item count and the item's words in one round trip (entries past the
  // count are unwritten, but inside the plan's storage)
  const int n_fit = plan[pl.hdr + 2];
  const int2 itw = *reinterpret_cast<const int2*>(plan + pl.fitems + 2 * it);
  if (it >= n_fit) return;  // uniform over the workgroup
  const int pos0 = itw.x, ntok = pair_item_tokens(itw.y);
  const int ba = pair_item_a(itw.y), bb = pair_item_b(itw.y);
  const int nblk = ba == bb ? 1 : 2;
  const int nsl = (ntok + kPairTile - 1) / kPairTile;  // 32-position slices of the item
  const int D = H * HD;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, col = lane & 31;

  // per-slice token state: this lane's token (column col of the slice), its
  // routing and q fragments (B operand: q[token][16 ks + 8 g ..])
  struct Slice {
    long tok;
    bool ok;
    int i0, i1;
    float g0, g1;
    bf16x8 qf[KS];
  };
  auto slice_pos = [&](int j, bool& ok) {
    const int p = j * kPairTile + col;
    ok = j < nsl && p < ntok;
    return (long)pos0 + p;
  };
  auto fetch_data = [&](Slice& sc, long raw, long pos) {
    sc.tok = sc.ok ? ((raw >= 0 && raw < N) ? raw : pos) : 0;  // a malformed entry falls back to its position
    sc.i0 = sc.i1 = -1;
    sc.g0 = sc.g1 = 1.f;
    if (sc.ok) {
      sc.i0 = top_idx[2 * sc.tok];
      sc.i1 = top_idx[2 * sc.tok + 1];
      sc.g0 = top_gates[2 * sc.tok];
      sc.g1 = top_gates[2 * sc.tok + 1];
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      sc.qf[ks] = sc.ok ? *reinterpret_cast<const bf16x8*>(q + sc.tok * D + (long)h * HD + 16 * ks + 8 * g)
                        : bf16x8{};
  };

  // ---- the wave's first slice: token and data issued ahead of the K / V staging
  Slice cur;
  {
    const long p = slice_pos(wave, cur.ok);
    const long raw = cur.ok ? (long)ord[p] : 0;
    fetch_data(cur, raw, p);
  }

  // ---- K and V rows of the pair: slots 0..127 block a, 128..255 block b
  {
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(k, (uint32_t)L * (uint32_t)D * 2u);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(v, (uint32_t)L * (uint32_t)D * 2u);
    uint4 kr[PER], vr[PER];
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int p = tid + NT * r;
      const int row = p >> 3, c8 = p & 7;
      const uint32_t slot = (uint32_t)((row < kPBS ? ba : bb) * kPBS + (row & (kPBS - 1)));
      const uint32_t off = (slot * (uint32_t)D + (uint32_t)(h * HD + 8 * c8)) * 2u;
      kr[r] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(krs, off, 0, 0));
      vr[r] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vrs, off, 0, 0));
    }
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int p = tid + NT * r;
      const int row = p >> 3, c8 = p & 7;
      *reinterpret_cast<uint4*>(&k_lds[row * PITCH + 8 * c8]) = kr[r];
      *reinterpret_cast<uint4*>(&v_lds[row * PITCH + 8 * c8]) = vr[r];
    }
  }
  lds_barrier();

  for (int j = wave; j < nsl; j += NW) {
    // the next slice's order entry, in flight during this slice's block a
    Slice nxt;
    const long pn = slice_pos(j + NW, nxt.ok);
    const long rawn = nxt.ok ? (long)ord[pn] : 0;

    bool sa, sb;
    const float l0 = log2f(fmaxf(cur.g0, 1e-9f)), l1 = log2f(fmaxf(cur.g1, 1e-9f));
    const float ca = pair_bias(cur.i0, cur.i1, l0, l1, ba, sa);
    const float cbb = pair_bias(cur.i0, cur.i1, l0, l1, bb, sb);

    f32x16 o[NO];
#pragma unroll
    for (int jj = 0; jj < NO; ++jj) o[jj] = f32x16{};
    float m_run = kNegBig, l_run = 0.f;
    float la_run = 0.f;  // the row sum over block a's chunks, rescaled with l_run

    auto qk = [&](int c, f32x16& x) {
      x = f32x16{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(&k_lds[(32 * c + col) * PITCH + 16 * ks + 8 * g]);
        x = mfma32(a, cur.qf[ks], x);
      }
    };
    // softmax of chunk c's scores (bias cb, selected sl) into bf16 weights,
    // with the lazy reference of read_fwd.hip: set from one score of the
    // token's first selected chunk, moved only when a chunk gives some
    // p > 2^64 (then the chunk is recomputed against its maximum)
    auto softmax = [&](int c, float cb, bool sl, f32x16& x, bf16x8 (&pk)[2]) {
      if (__any(sl && m_run == kNegBig)) {
        const float ref = fmaf(pair_max(x[0]), alpha, cb);
        if (sl && m_run == kNegBig) m_run = ref;
      }
      float add = sl ? cb - m_run : -INFINITY;
#pragma unroll
      for (int vv = 0; vv < 16; ++vv) x[vv] = __builtin_amdgcn_exp2f(fmaf(x[vv], alpha, add));
      pk[0] = pack8(x, 0);
      pk[1] = pack8(x, 8);
      float part = add_bf16x8(pk[1], add_bf16x8(pk[0], 0.f));
      const bool big = !(pair_max(part) <= 0x1p64f);
      if (__any(sl && big)) {
        qk(c, x);
        const float cand = fmaf(pair_max(max16(x)), alpha, cb);
        if (sl && big) {
          const float cr = __builtin_amdgcn_exp2f(m_run - cand);
#pragma unroll
          for (int jj = 0; jj < NO; ++jj)
#pragma unroll
            for (int vv = 0; vv < 16; ++vv) o[jj][vv] *= cr;
          l_run *= cr;
          la_run *= cr;
          m_run = cand;
        }
        add = sl ? cb - m_run : -INFINITY;
#pragma unroll
        for (int vv = 0; vv < 16; ++vv) x[vv] = __builtin_amdgcn_exp2f(fmaf(x[vv], alpha, add));
        pk[0] = pack8(x, 0);
        pk[1] = pack8(x, 8);
        part = add_bf16x8(pk[1], add_bf16x8(pk[0], 0.f));
      }
      l_run += part;
    };
    auto pv = [&](int c, const bf16x8 (&pk)[2]) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int jj = 0; jj < NO; ++jj) {
          const bf16x8 a = lds_frag_T<true, true>(v_lds, PITCH, 32 * c + 16 * kk, 32 * jj);
          o[jj] = mfma32(a, pk[kk], o[jj]);
        }
    };
    auto block = [&](int bi) {
      const float cb = bi ? cbb : ca;
      const bool sl = bi ? sb : sa;
#pragma unroll
      for (int cc = 0; cc < kPBS / 32; ++cc) {
        const int c = bi * (kPBS / 32) + cc;
        f32x16 x;
        bf16x8 pk[2];
        qk(c, x);
        softmax(c, cb, sl, x, pk);
        pv(c, pk);
      }
    };

    block(0);
    la_run = l_run;
    // the next slice's routing and q, in flight during block b and the epilogue
    fetch_data(nxt, rawn, pn);
    if (nblk == 2) block(1);

    // ---- epilogue: normalise; o, its bf16 remainder, lse and block a's share
    const float l = pair_sum(l_run);
    const float la_tot = pair_sum(la_run);
    if (cur.ok) {
      const long tok = cur.tok;
      const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
      for (int jj = 0; jj < NO; ++jj) {
        const int f0 = 32 * jj + 16 * g;
        f32x16 y;
#pragma unroll
        for (int e = 0; e < 16; ++e) y[e] = o[jj][e] * inv;
        bf16x8 hi0, hi1, lo0, lo1;
        pack8_hilo(y, 0, hi0, lo0);
        pack8_hilo(y, 8, hi1, lo1);
        bf16_t* dst = out + tok * D + (long)h * HD + f0;
        *reinterpret_cast<bf16x8*>(dst) = hi0;
        *reinterpret_cast<bf16x8*>(dst + 8) = hi1;
        if (out_lo != nullptr) {
          bf16_t* dl = out_lo + tok * D + (long)h * HD + f0;
          *reinterpret_cast<bf16x8*>(dl) = lo0;
          *reinterpret_cast<bf16x8*>(dl + 8) = lo1;
        }
      }
      if (g == 0) {
        lse[(long)h * N + tok] = m_run + log2f(l);
        // the share of the row's weight on block a (1 for a one-block pair)
        if (frac_a != nullptr) frac_a[(long)h * N + tok] = nblk == 1 ? 1.f : (l > 0.f ? la_tot / l : 0.f);
      }
    }
    cur = nxt;
  }
}

// ----------------------------------------------------------------- backward
// Workgroup (head h, range r of the head's tiles); wave w owns slots
// 32 w .. 32 w + 31 of the current pair (w < 4: block a, else block b).
__global__ __launch_bounds__(512, 1) void read_bwd_pair_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const int32_t* __restrict__ top_idx, const float* __restrict__ top_gates, const bf16_t* __restrict__ o,
    const bf16_t* __restrict__ o_lo, const float* __restrict__ frac_a, const bf16_t* __restrict__ dout,
    const float* __restrict__ lse,
    const int32_t* __restrict__ plan, bf16_t* __restrict__ dq, float* __restrict__ dlg_part,
    float* __restrict__ dk_part, float* __restrict__ dv_part, long N, int H, int L, int E, float alpha,
    float dq_scale, int R, int n_seg) {
  constexpr int HD = kPHD, KS = HD / 16, NO = HD / 32, PITCH = kPPitch, TQ = kPairTile, NT = 512;
  constexpr int DSP = kPDsPitch;

  __shared__ __attribute__((aligned(16))) bf16_t q_lds[2][TQ * PITCH];
  __shared__ __attribute__((aligned(16))) bf16_t do_lds[2][TQ * PITCH];
  __shared__ __attribute__((aligned(16))) float ctab[2][3][TQ];  // c_a - lse, c_b - lse, -delta
  __shared__ int32_t tok_lds[2][TQ];                              // token of each row (-1: none)
  __shared__ int32_t sel_lds[2][TQ];                              // which selections hit a (bit 0,1) / b (bit 2,3)
  __shared__ float fa_lds[2][TQ];                                 // the forward's weight share of block a
  __shared__ __attribute__((aligned(16))) bf16_t kt_lds[kPSlots * PITCH];  // the pair's K rows
  __shared__ __attribute__((aligned(16))) bf16_t vt_lds[kPSlots * PITCH];  // the pair's V rows
  __shared__ __attribute__((aligned(16))) bf16_t ds_lds[kPSlots * DSP];    // dS^T of the tile: bf16(dS)
  __shared__ __attribute__((aligned(16))) bf16_t dsl_lds[kPSlots * DSP];   // and bf16(dS - bf16(dS))
  __shared__ float dl_lds[4][TQ];  // gate-gradient partials: (block a | b) x (slot half)
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

  // ---- tile staging: threads 0..255 hold dO, o, o_lo pieces (token row p >> 3,
  // features 8 (p & 7) ..), threads 256..511 a Q piece; threads 0..31 the row's routing
  const int sp = tid & 255, srow = sp >> 3, sc8 = sp & 7;
  const bool s_do = tid < 256;
  uint4 r_a = make_uint4(0, 0, 0, 0), r_o = r_a, r_ol = r_a;  // dO (or Q) / o / o_lo piece
  int r_tok = -1, r_i0 = -1, r_i1 = -1;                         // threads 0..31: row tid
  float r_g0 = 1.f, r_g1 = 1.f, r_lse = 0.f, r_fa = 1.f;
  // order entries of the staged piece's row and (threads 0..31) of row tid,
  // fetched a tile ahead of the loads that use them
  int nx_raw = 0, nx_pos = -1, nr_raw = 0, nr_pos = -1;
  auto fetch_tokens = [&](int t) {
    const int pos0 = tile_w0(t), cnt = pair_tile_count(tile_w1(t));
    nx_pos = srow < cnt ? pos0 + srow : -1;
    if (nx_pos >= 0) nx_raw = ord[nx_pos];
    if (tid < TQ) {
      nr_pos = tid < cnt ? pos0 + tid : -1;
      if (nr_pos >= 0) nr_raw = ord[nr_pos];
    }
  };
  // a malformed order entry falls back to its position (wrong results, never
  // an access out of bounds)
  auto token_of = [&](int pos, int raw) -> long {
    if (pos < 0) return -1;
    return (raw >= 0 && raw < N) ? (long)raw : (long)pos;
  };
  auto load_tile = [&]() {
    const long tk = token_of(nx_pos, nx_raw);
    r_a = r_o = r_ol = make_uint4(0, 0, 0, 0);
    if (tk >= 0) {
      const long off = tk * D + (long)h * HD + 8 * sc8;
      if (s_do) {
        r_a = *reinterpret_cast<const uint4*>(dout + off);
        r_o = *reinterpret_cast<const uint4*>(o + off);
        r_ol = *reinterpret_cast<const uint4*>(o_lo + off);
      } else {
        r_a = *reinterpret_cast<const uint4*>(q + off);
      }
    }
    if (tid < TQ) {
      const long tr = token_of(nr_pos, nr_raw);
      r_tok = (int)tr;
      r_i0 = r_i1 = -1;
      r_g0 = r_g1 = 1.f;
      r_lse = 0.f;
      r_fa = 1.f;
      if (tr >= 0) {
        r_i0 = top_idx[2 * tr];
        r_i1 = top_idx[2 * tr + 1];
        r_g0 = top_gates[2 * tr];
        r_g1 = top_gates[2 * tr + 1];
        r_lse = lse[(long)h * N + tr];
        r_fa = frac_a[(long)h * N + tr];
      }
    }
  };
  // into buffer `buf`, for the pair (a, b): Q / dO rows, the per-row bias and
  // delta tables, tokens and selections
  auto store_tile = [&](int buf, int a, int b) {
    if (s_do) {
      *reinterpret_cast<uint4*>(&do_lds[buf][srow * PITCH + 8 * sc8]) = r_a;
      // delta = sum_f dO_f (o_f + o_lo_f) over the 8 features of the piece, then over the row's 8 threads
      const uint32_t dw[4] = {r_a.x, r_a.y, r_a.z, r_a.w};
      const uint32_t ow[4] = {r_o.x, r_o.y, r_o.z, r_o.w};
      const uint32_t lw[4] = {r_ol.x, r_ol.y, r_ol.z, r_ol.w};
      float dsum = 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float d0 = __uint_as_float(dw[u] << 16), d1 = __uint_as_float(dw[u] & 0xffff0000u);
        const float o0 = __uint_as_float(ow[u] << 16) + __uint_as_float(lw[u] << 16);
        const float o1 = __uint_as_float(ow[u] & 0xffff0000u) + __uint_as_float(lw[u] & 0xffff0000u);
        dsum = fmaf(d0, o0, dsum);
        dsum = fmaf(d1, o1, dsum);
      }
      dsum += dpp_f32<0xb1>(dsum);
      dsum += dpp_f32<0x4e>(dsum);
      dsum += dpp_f32<0x141>(dsum);
      if (sc8 == 0) ctab[buf][2][srow] = -dsum;
    } else {
      *reinterpret_cast<uint4*>(&q_lds[buf][srow * PITCH + 8 * sc8]) = r_a;
    }
    if (tid < TQ) {
      const float l0 = log2f(fmaxf(r_g0, 1e-9f)), l1 = log2f(fmaxf(r_g1, 1e-9f));
      bool sa, sb;
      const float ca = pair_bias(r_i0, r_i1, l0, l1, a, sa);
      const float cb = pair_bias(r_i0, r_i1, l0, l1, b, sb);
      ctab[buf][0][tid] = sa ? ca - r_lse : -INFINITY;
      ctab[buf][1][tid] = (sb && b != a) ? cb - r_lse : -INFINITY;
      tok_lds[buf][tid] = r_tok;
      fa_lds[buf][tid] = r_fa;
      sel_lds[buf][tid] = (r_i0 == a ? 1 : 0) | (r_i1 == a ? 2 : 0) | (r_i0 == b ? 4 : 0) | (r_i1 == b ? 8 : 0);
    }
  };

  // ---- the current pair: its K and V rows in LDS (B operands of S and dP:
  // lane = slot; and the dQ product's K^T fragments), the dK / dV accumulators
  int key = -1, pa = 0, pb = 0, nblk = 2;
  bool w_on = true;
  f32x16 acc_dk[NO], acc_dv[NO];
  const int w_slot = 32 * wave + col;  // this lane's slot in the pair (0..255)
  auto enter_pair = [&](int t) {
    const int w1 = tile_w1(t);
    key = pair_tile_key(w1);
    pa = pair_tile_a(w1);
    pb = pair_tile_b(w1);
    nblk = pa == pb ? 1 : 2;
    w_on = wave < 4 * nblk;
    constexpr int PR = kPSlots * HD / 8 / NT;
#pragma unroll
    for (int rr = 0; rr < PR; ++rr) {
      const int p = tid + NT * rr;
      const int row = p >> 3, c8 = p & 7;
      const long off = ((long)(row < kPBS ? pa : pb) * kPBS + (row & (kPBS - 1))) * D + (long)h * HD + 8 * c8;
      *reinterpret_cast<uint4*>(&kt_lds[row * PITCH + 8 * c8]) = *reinterpret_cast<const uint4*>(k + off);
      *reinterpret_cast<uint4*>(&vt_lds[row * PITCH + 8 * c8]) = *reinterpret_cast<const uint4*>(v + off);
    }
#pragma unroll
    for (int j = 0; j < NO; ++j) {
      acc_dk[j] = f32x16{};
      acc_dv[j] = f32x16{};
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
  // the pair's sums of this range into segment r + key (rows: the pair's 256 slots)
  auto flush = [&]() {
    if (!w_on) return;
    const long base = (((long)h * n_seg + (r + key)) * kPSlots + w_slot) * HD;
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
  // gate gradients of the tile in buffer `buf` (partials in dl_lds): threads
  // 0..31.  With P recomputed from lse (fp32 weights over the bf16 row sum)
  // and delta from o (the bf16 weights), sum_n dS_n over both blocks, which
  // is 0 for the exact softmax, keeps a residue (delta' - delta) S; the
  // block sums are G_x = A_x - delta' M_x, so G_a - (M_a / S)(G_a + G_b) is
  // the exact A_a - delta M_a.  M_a / S is the forward's share of the row
  // weight on block a (its error only scales that small residue).
  auto finish_gates = [&](int buf) {
    if (tid < TQ) {
      const int tk = tok_lds[buf][tid];
      if (tk >= 0) {
        const int sm = sel_lds[buf][tid];
        const float fa = fa_lds[buf][tid];
        const float g0 = dl_lds[0][tid] + dl_lds[1][tid];
        const float g1 = dl_lds[2][tid] + dl_lds[3][tid];
        const float tot = g0 + g1;
        const float ga = g0 - fa * tot;
        const float gb = g1 - (1.f - fa) * tot;
        float* dst = dlg_part + ((long)h * N + tk) * 2;
        dst[0] = (sm & 1) ? ga : ((sm & 4) ? gb : 0.f);
        dst[1] = (sm & 2) ? ga : ((sm & 8) ? gb : 0.f);
      }
    }
  };

  // ---- prologue: tile i0 staged, its pair entered, tile i0 + 1 in flight
  enter_pair(i0);
  fetch_tokens(i0);
  load_tile();
  store_tile(0, pa, pb);
  if (i0 + 1 < i1) {
    fetch_tokens(i0 + 1);
    load_tile();
  }
  lds_barrier();

  for (int i = i0; i < i1; ++i) {
    const int buf = (i - i0) & 1;
    if (i + 2 < i1) fetch_tokens(i + 2);
    if (i > i0) finish_gates(buf ^ 1);  // the previous tile's gate gradients (its partials are complete)

    // ---- S, dP - delta, P, dS for this wave's 32 slots x the tile's 32 tokens
    f32x16 acc_s = f32x16{}, acc_p;
    if (w_on) {
      const int bsel = wave >> 2;  // 0: block a, 1: block b
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        const f32x4 nd = *reinterpret_cast<const f32x4*>(&ctab[buf][2][8 * j4 + 4 * g]);
#pragma unroll
        for (int u = 0; u < 4; ++u) acc_p[4 * j4 + u] = nd[u];
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int off = col * PITCH + 16 * ks + 8 * g;
        const int offk = w_slot * PITCH + 16 * ks + 8 * g;
        const bf16x8 aq = *reinterpret_cast<const bf16x8*>(&q_lds[buf][off]);
        const bf16x8 ad = *reinterpret_cast<const bf16x8*>(&do_lds[buf][off]);
        const bf16x8 bk = *reinterpret_cast<const bf16x8*>(&kt_lds[offk]);
        const bf16x8 bv = *reinterpret_cast<const bf16x8*>(&vt_lds[offk]);
        acc_s = mfma32(aq, bk, acc_s);
        acc_p = mfma32(ad, bv, acc_p);
      }
      // registers 4 j4 .. 4 j4 + 3 are tokens 8 j4 + 4 g + 0..3
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        const f32x4 c4 = *reinterpret_cast<const f32x4*>(&ctab[buf][bsel][8 * j4 + 4 * g]);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int vv = 4 * j4 + u;
          const float p = __builtin_amdgcn_exp2f(fmaf(acc_s[vv], alpha, c4[u]));
          acc_s[vv] = p;
          acc_p[vv] = p * acc_p[vv];
        }
      }
      // ---- dV^T += dO^T P (P as a bf16 hi + lo pair: dV sums P over many
      // tokens), dK^T += Q^T dS; dS^T to LDS for dQ
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        bf16x8 bp, bp_lo, bd, bd_lo;
        pack8_hilo(acc_s, 8 * kk, bp, bp_lo);
        pack8_hilo(acc_p, 8 * kk, bd, bd_lo);
#pragma unroll
        for (int j = 0; j < NO; ++j) {
          const bf16x8 a_do = lds_frag_T<true, true>(do_lds[buf], PITCH, 16 * kk, 32 * j);
          const bf16x8 a_q = lds_frag_T<true, true>(q_lds[buf], PITCH, 16 * kk, 32 * j);
          acc_dv[j] = mfma32(a_do, bp, acc_dv[j]);
          acc_dv[j] = mfma32(a_do, bp_lo, acc_dv[j]);
          acc_dk[j] = mfma32(a_q, bd, acc_dk[j]);
        }
        // registers 8 kk .. 8 kk + 7 are tokens 16 kk + 4 g + 0..3 and 16 kk + 8 + 4 g + 0..3
        const uint4 u = __builtin_bit_cast(uint4, bd);
        const uint4 ul = __builtin_bit_cast(uint4, bd_lo);
        const int dso = w_slot * DSP + 16 * kk + 4 * g;
        *reinterpret_cast<uint2*>(&ds_lds[dso]) = make_uint2(u.x, u.y);
        *reinterpret_cast<uint2*>(&ds_lds[dso + 8]) = make_uint2(u.z, u.w);
        *reinterpret_cast<uint2*>(&dsl_lds[dso]) = make_uint2(ul.x, ul.y);
        *reinterpret_cast<uint2*>(&dsl_lds[dso + 8]) = make_uint2(ul.z, ul.w);
      }
    }
    lds_barrier();  // dS^T of the tile complete

    // ---- dQ^T tile (features 16 (w & 3) .., tokens 16 (w >> 2) ..) over the
    // pair's slots, and the gate-gradient partials: wave with w & 3 == c sums
    // dS (as its bf16 hi + lo pair: the block sums need fp32 accuracy) over
    // K-steps 2c, 2c + 1 (block a for c < 2, b otherwise)
    {
      const int tq = wave >> 2, fq = wave & 3;
      const int q4 = (lane >> 4) & 3, j = lane & 15;
      f32x4v accq = f32x4v{0.f, 0.f, 0.f, 0.f};
      float gsum = 0.f;
      const int nks = 4 * nblk;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        if (kk < nks) {
          // A: K^T (features 16 fq .., slots 32 kk ..); B: dS^T (slots, tokens 16 tq ..)
          const bf16x8 akt = frag16_T(kt_lds, PITCH, 32 * kk, 16 * fq);
          const bf16x8 bds = frag16_T(ds_lds, DSP, 32 * kk, 16 * tq);
          accq = mfma16(akt, bds, accq);
        }
      }
      if (2 * fq < nks) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const int kk = 2 * fq + jj;
          const bf16x8 bds = frag16_T(ds_lds, DSP, 32 * kk, 16 * tq);
          const bf16x8 bdl = frag16_T(dsl_lds, DSP, 32 * kk, 16 * tq);
          gsum = add_bf16x8(bdl, add_bf16x8(bds, gsum));
        }
      }
      // the four 16-lane groups hold different slots of the same token
      gsum = xor16_f32(gsum, [](float a, float b) { return a + b; });
      gsum = xor32_f32(gsum, [](float a, float b) { return a + b; });
      if (lane < 16) dl_lds[fq][16 * tq + lane] = gsum;
      // dQ rows: lane holds features 16 fq + 4 (l / 16) + 0..3 of token row 16 tq + l % 16
      const int tk = tok_lds[buf][16 * tq + j];
      if (tk >= 0) {
        uint2 pk;
        pk.x = (uint32_t)f32_to_bf16(accq[0] * dq_scale) | ((uint32_t)f32_to_bf16(accq[1] * dq_scale) << 16);
        pk.y = (uint32_t)f32_to_bf16(accq[2] * dq_scale) | ((uint32_t)f32_to_bf16(accq[3] * dq_scale) << 16);
        *reinterpret_cast<uint2*>(dq + (long)tk * D + (long)h * HD + 16 * fq + 4 * q4) = pk;
      }
    }

    // ---- next tile: its pair (flush and reload on a change), staging, barrier
    if (i + 1 < i1) {
      const int nkey = pair_tile_key(tile_w1(i + 1));
      if (nkey != key) {
        // other waves may still read kt_lds in their dQ products: wait for
        // them before the next pair's rows overwrite it
        flush();
        lds_barrier();
        enter_pair(i + 1);
        store_tile(buf ^ 1, pa, pb);
        if (i + 2 < i1) load_tile();
      } else {
        store_tile(buf ^ 1, pa, pb);
        if (i + 2 < i1) load_tile();
      }
    }
    lds_barrier();
  }
  finish_gates((i1 - 1 - i0) & 1);
  flush();
}

// ------------------------------------------------------------------- reduce
// dK / dV of block e (rows e * 128 ..), head h, a quarter of its slots: the
// sum over the pairs holding e (ascending pair index) and, within a pair,
// over its ranges (ascending), of the pair's partial half for e; dK scaled.
// Workgroups past the dK / dV ones sum the per-head gate-gradient partials
// (head order) into d(top_gates) through log(max(g, 1e-9)).
__global__ __launch_bounds__(256) void read_pair_reduce_kernel(
    const float* __restrict__ dk_part, const float* __restrict__ dv_part, const int32_t* __restrict__ plan,
    bf16_t* __restrict__ dk, bf16_t* __restrict__ dv, long N, int H, int E, int R, int n_seg, float dk_scale,
    int kv_blocks, const float* __restrict__ dlg_part, const float* __restrict__ top_gates,
    float* __restrict__ dgates) {
  constexpr int HD = kPHD, QS = kPBS / 4;  // slots per workgroup
  __shared__ int seg[1024];
  __shared__ int half[1024];
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
  const int qtr = b & 3, e = (b >> 2) % E, h = (b >> 2) / E;
  const int n_tiles = plan[pl.hdr], n_keys = plan[pl.hdr + 1];
  const int per = (n_tiles + R - 1) / R;
  if (threadIdx.x == 0) {
    int n = 0;
    for (int kk = 0; kk < n_keys; ++kk) {
      const int* kr = plan + pl.keys + 4 * kk;
      const int a = kr[0], bb = kr[1], ts = kr[2], nt = kr[3];
      if ((a != e && bb != e) || nt <= 0) continue;
      const int hf = a == e ? 0 : 1;
      for (int rr = ts / per; rr <= (ts + nt - 1) / per && n < 1024; ++rr) {
        seg[n] = rr + kk;
        half[n] = hf;
        ++n;
      }
    }
    n_s = n;
  }
  __syncthreads();
  const int ns = n_s;
  const int D = H * HD;
  // 32 slots x 64 features = 512 float4 per tensor: two per thread
  for (int c = threadIdx.x; c < QS * HD / 4; c += blockDim.x) {
    const int sl = c / (HD / 4), f4 = c % (HD / 4);
    const int s_in = qtr * QS + sl;  // slot within the block
    f32x4 sk = f32x4{0.f, 0.f, 0.f, 0.f}, sv = sk;
    int i = 0;
    for (; i + 4 <= ns; i += 4) {
      f32x4 pk[4], pv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const long off = (((long)h * n_seg + seg[i + u]) * kPSlots + half[i + u] * kPBS + s_in) * HD + 4 * f4;
        pk[u] = *reinterpret_cast<const f32x4*>(dk_part + off);
        pv[u] = *reinterpret_cast<const f32x4*>(dv_part + off);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        sk += pk[u];
        sv += pv[u];
      }
    }
    for (; i < ns; ++i) {
      const long off = (((long)h * n_seg + seg[i]) * kPSlots + half[i] * kPBS + s_in) * HD + 4 * f4;
      sk += *reinterpret_cast<const f32x4*>(dk_part + off);
      sv += *reinterpret_cast<const f32x4*>(dv_part + off);
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
}

// ------------------------------------------------------------------ host side
bool read_pair_fwd_shapes(const ReadDims& d, long N) {
  return d.HD == kPHD && d.block_size == kPBS && d.topk == 2 && d.E <= kPairMaxE &&
         read_has_pair_plan(N, d.E, d.topk) && (long)d.L * d.H * d.HD * 2 < (1L << 31);
}
bool read_pair_bwd_shapes(const ReadDims& d, long N) { return read_pair_fwd_shapes(d, N) && d.E <= kPairBwdMaxE; }
bool read_pair_fwd_ok(const ReadDims& d, long N) { return d.order != nullptr && read_pair_fwd_shapes(d, N); }
bool read_pair_bwd_ok(const ReadDims& d, long N) { return d.order != nullptr && read_pair_bwd_shapes(d, N); }

static int pair_fwd_max_items(long N, int E) { return pair_plan_layout(N, E).max_tiles; }

int read_pair_ranges(const ReadDims& d) {
  const long N = (long)d.B * d.S;
  const int want = d.H >= 256 ? 1 : 256 / d.H;  // one round of workgroups
  const int tiles = pair_plan_layout(N, d.E).max_tiles;
  // at least 4 tiles a range, at most kPairBwdMaxRange (the range's tile words sit in LDS)
  const int r = std::max(1, std::min(want, (tiles + 3) / 4));
  return std::max(r, (tiles + kPairBwdMaxRange - 1) / kPairBwdMaxRange);
}

int read_pair_segments(const ReadDims& d) {
  const long N = (long)d.B * d.S;
  return read_pair_ranges(d) + pair_plan_layout(N, d.E).max_keys - 1;
}

size_t read_pair_part_bytes(const ReadDims& d) {
  return (size_t)d.H * read_pair_segments(d) * kPSlots * kPHD * sizeof(float);
}

size_t read_pair_side_bytes(const ReadDims& d) {
  const size_t N = (size_t)d.B * d.S;
  return ((N * d.H * d.HD * 2 + 255) & ~(size_t)255) + N * d.H * 4;
}

// the side buffer: o's bf16 remainder (N, D), then block a's weight share (H, N)
static bf16_t* side_out_lo(void* side) { return (bf16_t*)side; }
static float* side_frac_a(void* side, const ReadDims& d) {
  const size_t N = (size_t)d.B * d.S;
  return (float*)((char*)side + ((N * d.H * d.HD * 2 + 255) & ~(size_t)255));
}

hipError_t launch_read_fwd_pair(const void* q, const void* k, const void* v, const int32_t* top_idx,
                                const float* top_gates, void* out, void* side, float* lse, const ReadDims& d,
                                hipStream_t st) {
  const long N = (long)d.B * d.S;
  const int mi = pair_fwd_max_items(N, d.E);
  const float alpha = (float)(1.0 / __builtin_sqrt(64.0)) * kLog2e;
  bf16_t* olo = side ? side_out_lo(side) : nullptr;
  float* fa = side ? side_frac_a(side, d) : nullptr;
  NAYLIS_TIMED("read_fwd", st,
               hipLaunchKernelGGL(read_fwd_pair_kernel, dim3(d.H * mi), dim3(256), 0, st, (const bf16_t*)q,
                                  (const bf16_t*)k, (const bf16_t*)v, top_idx, top_gates, (bf16_t*)out, olo, fa,
                                  lse, d.order, N, d.H, d.L, d.E, alpha, mi));
  return hipGetLastError();
}

hipError_t launch_read_bwd_pair(const void* q, const void* k, const void* v, const int32_t* top_idx,
                                const float* top_gates, const void* o, const void* side, const void* dout,
                                const float* lse, void* dq, void* dk, void* dv, float* dgates, float* dlg_part,
                                float* dk_part, float* dv_part, const ReadDims& d, hipStream_t st) {
  const long N = (long)d.B * d.S;
  const int R = read_pair_ranges(d);
  const int ns = read_pair_segments(d);
  const float alpha = (float)(1.0 / __builtin_sqrt(64.0)) * kLog2e;
  const float scale = (float)(1.0 / __builtin_sqrt(64.0));
  NAYLIS_TIMED("read_bwd_pair", st,
               hipLaunchKernelGGL(read_bwd_pair_kernel, dim3(d.H * R), dim3(512), 0, st, (const bf16_t*)q,
                                  (const bf16_t*)k, (const bf16_t*)v, top_idx, top_gates, (const bf16_t*)o,
                                  side_out_lo((void*)side), side_frac_a((void*)side, d), (const bf16_t*)dout, lse,
                                  d.order, (bf16_t*)dq, dlg_part,
                                  dk_part, dv_part, N, d.H, d.L, d.E, alpha, scale, R, ns));
  const int kv_blocks = d.H * d.E * 4;
  const int g_blocks = (int)std::min<long>(1024, (N * 2 + 255) / 256);
  NAYLIS_TIMED("read_bwd_reduce", st,
               hipLaunchKernelGGL(read_pair_reduce_kernel, dim3(kv_blocks + g_blocks), dim3(256), 0, st, dk_part,
                                  dv_part, d.order, (bf16_t*)dk, (bf16_t*)dv, N, d.H, d.E, R, ns, scale, kv_blocks,
                                  dlg_part, top_gates, dgates));
  return hipGetLastError();
}

}  // namespace naylis
