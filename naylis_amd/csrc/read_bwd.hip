// Gated flash read of the shared MoM bank, backward (gfx950).
//
// Gradients of o = softmax(q k^T * scale + bias) v, bias = routed log-gates
// (mom_kernels/reference.py:14-61), the set mom_kernels/triton_gpu.py:359-409
// returns: dq, dk and dv of the SHARED bank projections (reduced over every
// token of the batch), and d(top_gates).  P is recomputed from the forward's
// log2-domain lse; dS = P (dP - delta), delta = rowsum(o * do).
//
// Launches, all deterministic (no floating-point atomics):
//  1. read_bwd_dq_kernel   — one workgroup per (b, h, 128-token tile), walks
//     the tile's active slot groups: S^T, dP^T, dS^T, dQ^T += K^T dS^T; also
//     writes the exact delta (sum_n P dP) and the per-head partial of
//     dlog_gates (sum of dS over each selected block).  The staged variant
//     (read_bwd_dq_fast_kernel, head_dim 64) also writes which blocks each
//     64-token tile selects.
//  2. read_tile_flags / read_tile_lists — which 64-token tiles select any
//     block of each 128-slot group, as compact ascending lists (the flags
//     launch only when the dQ kernel did not write them).
//  3. read_bwd_dkdv_kernel — one workgroup per (h, equal range of the
//     (128-slot group, active tile) items), 4 waves of 32 slots; K/V rows of
//     the current group's slots stay in registers;
//     S, dP, dS per tile, dV^T += dO^T P and dK^T += Q^T dS with dO^T / Q^T
//     read transposed from the natural-layout tiles; an fp32 partial per
//     (range, group) segment.
//  4. read_bwd_reduce_kernel — one launch: each group's partials summed in
//     range order (dk scaled), per-head dlog partials summed over heads and
//     mapped to d(top_gates) through log(max(g, 1e-9)).
#include "launch.h"
#include "read_common.h"
#include "timing.h"

namespace naylis {

template <int HD, int SG, bool ALIGNED, int TK>
__global__ __launch_bounds__(256, 2) void read_bwd_dq_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const int32_t* __restrict__ top_idx, const float* __restrict__ top_gates, const bf16_t* __restrict__ o,
    const bf16_t* __restrict__ dout, const float* __restrict__ lse, bf16_t* __restrict__ dq,
    float* __restrict__ delta, float* __restrict__ dlg_part, const int32_t* __restrict__ order, long N, int H,
    int L, int E, int block_size, int topk, float alpha, float scale, int n_tiles) {
  constexpr int HDP = HD < 32 ? 32 : HD;
  constexpr int KS = HD / 16;
  constexpr int NS = SG / 32;
  constexpr int NO = HDP / 32;
  constexpr int PITCH = HDP + 8;

  __shared__ __attribute__((aligned(16))) bf16_t k_lds[SG * PITCH];
  __shared__ __attribute__((aligned(16))) bf16_t v_lds[SG * PITCH];
  __shared__ uint8_t flags[kMaxBlocks];
  __shared__ uint16_t groups[kMaxGroups];
  __shared__ int n_active;

  const int G = H * n_tiles;
  const int wid = xcd_remap(blockIdx.x, G);
  const int tile = wid % n_tiles;
  const int h = wid / n_tiles;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int col = lane & 31;
  const long pos = (long)tile * 128 + wave * 32 + col;  // position in the token order
  const bool tok_ok = pos < N;
  const int32_t* ord = order_table(order);
  const long tok = tok_ok ? order_token(ord, pos, N) : 0;  // flattened b*S + s
  const int D = H * HD;

  TokenRoute<TK> rt;
  load_route<TK>(rt, top_idx, top_gates, tok, tok_ok, topk);
  // Q^T, dO^T and o rows and the lse, issued right after the routing loads
  // (loads retire in issue order, so the routing can be used while these are
  // still in flight across the LDS barriers below)
  bf16x8 qf[KS], df[KS], of[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if (tok_ok) {
      const long off = tok * D + (long)h * HD + 16 * ks + 8 * g;
      qf[ks] = *reinterpret_cast<const bf16x8*>(q + off);
      df[ks] = *reinterpret_cast<const bf16x8*>(dout + off);
      of[ks] = *reinterpret_cast<const bf16x8*>(o + off);
    } else {
      qf[ks] = bf16x8{};
      df[ks] = bf16x8{};
      of[ks] = bf16x8{};
    }
  }
  const float lse_t = tok_ok ? lse[(long)h * N + tok] : 0.f;
  for (int e = tid; e < E; e += 256) flags[e] = 0;
  if constexpr (HD < 32) {
    for (int i = tid; i < SG * PITCH; i += 256) k_lds[i] = 0;  // K^T rows beyond HD stay zero
  }
  lds_barrier();
  if (g == 0 && tok_ok) {
#pragma unroll
    for (int t = 0; t < TK; ++t)
      if (t < topk && rt.idx[t] >= 0 && rt.idx[t] < E) flags[rt.idx[t]] = 1;
  }
  lds_barrier();
  const int n_groups = (L + SG - 1) / SG;
  if (wave == 0) build_group_list<SG>(flags, E, L, block_size, n_groups, groups, &n_active);

  // delta0 = rowsum(o * do) from the rows loaded above
  float dl = 0.f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
#pragma unroll
    for (int e = 0; e < 8; ++e) dl = fmaf((float)of[ks][e], (float)df[ks][e], dl);
  dl = wave_sum_pair(dl);

  f32x16 acc_dq[NO];
#pragma unroll
  for (int j = 0; j < NO; ++j) acc_dq[j] = f32x16{};
  // dlog_gates without the bf16 rounding of o inside delta: per selection t
  // accumulate A_t = sum_{n in block t} P dP and M_t = sum_{n in block t} P,
  // plus dx = sum_n P dP and S = sum_n P over every selected slot.  P is
  // recomputed from the forward's lse, so S = 1 only up to the rounding of
  // the forward's row sum; dividing by S makes the weights exactly
  // normalised: delta = dx / S and dlog_t = A_t / S - delta M_t / S.
  float accA[TK], accM[TK];
#pragma unroll
  for (int t = 0; t < TK; ++t) {
    accA[t] = 0.f;
    accM[t] = 0.f;
  }
  float dx = 0.f, sp = 0.f;

  lds_barrier();
  const int n_act = n_active;

  constexpr int VEC = SG * HD / 8;
  constexpr int PER = (VEC + 255) / 256;
  uint4 kreg[PER], vreg[PER];

  auto load_group = [&](int gi) {
    const int s0 = gi * SG;
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int vi = tid + 256 * r;
      uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
      if (vi < VEC) {
        const int srow = vi / (HD / 8), c8 = vi % (HD / 8);
        if (s0 + srow < L) {
          const long off = (long)(s0 + srow) * D + (long)h * HD + 8 * c8;
          kv = *reinterpret_cast<const uint4*>(k + off);
          vv = *reinterpret_cast<const uint4*>(v + off);
        }
      }
      kreg[r] = kv;
      vreg[r] = vv;
    }
  };
  auto store_group = [&]() {
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int vi = tid + 256 * r;
      if (vi < VEC) {
        const int srow = vi / (HD / 8), c8 = vi % (HD / 8);
        *reinterpret_cast<uint4*>(&k_lds[srow * PITCH + 8 * c8]) = kreg[r];
        *reinterpret_cast<uint4*>(&v_lds[srow * PITCH + 8 * c8]) = vreg[r];
      }
    }
  };

  if (n_act > 0) load_group(groups[0]);

  for (int it = 0; it < n_act; ++it) {
    const int gi = groups[it];
    lds_barrier();
    store_group();
    lds_barrier();
    if (it + 1 < n_act) load_group(groups[it + 1]);

    // a wave whose 32 tokens select no block of the group has P = 0 there:
    // nothing to add to dQ, the gate sums or delta
    bool mine = false;
    if constexpr (ALIGNED) {
      const int e = (gi * SG) / block_size;
#pragma unroll
      for (int t = 0; t < TK; ++t) mine |= (t < topk && rt.idx[t] == e);
    } else {
      const int b0 = (gi * SG) / block_size, b1 = (min(gi * SG + SG, L) - 1) / block_size;
#pragma unroll
      for (int t = 0; t < TK; ++t) mine |= (t < topk && rt.idx[t] >= b0 && rt.idx[t] <= b1);
    }
    if (!__any(mine)) continue;

    f32x16 acc_s[NS], acc_p[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      acc_s[i] = f32x16{};
      acc_p[i] = f32x16{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int off = (32 * i + col) * PITCH + 16 * ks + 8 * g;
        const bf16x8 ak = *reinterpret_cast<const bf16x8*>(&k_lds[off]);
        const bf16x8 av = *reinterpret_cast<const bf16x8*>(&v_lds[off]);
        acc_s[i] = mfma32(ak, qf[ks], acc_s[i]);
        acc_p[i] = mfma32(av, df[ks], acc_p[i]);
      }
    }

    if constexpr (ALIGNED) {
      const int e = (gi * SG) / block_size;
      bool sel;
      const float c2 = route_bias<TK>(rt, e, topk, sel);
      const float add = sel ? c2 - lse_t : -INFINITY;
      float rsA = 0.f, rsM = 0.f;
#pragma unroll
      for (int i = 0; i < NS; ++i)
#pragma unroll
        for (int vv = 0; vv < 16; ++vv) {
          const float p = __builtin_amdgcn_exp2f(fmaf(acc_s[i][vv], alpha, add));
          const float dp = acc_p[i][vv];
          acc_s[i][vv] = p * (dp - dl);
          rsA = fmaf(p, dp, rsA);
          rsM += p;
        }
      dx += rsA;
      sp += rsM;
#pragma unroll
      for (int t = 0; t < TK; ++t)
        if (t < topk && rt.idx[t] == e) {
          accA[t] += rsA;
          accM[t] += rsM;
        }
    } else {
#pragma unroll
      for (int i = 0; i < NS; ++i)
#pragma unroll
        for (int vv = 0; vv < 16; ++vv) {
          const int slot = gi * SG + 32 * i + acc_row(g, vv);
          bool sel = false;
          float c2 = 0.f;
          const int e = slot < L ? slot / block_size : -2;
          if (slot < L) c2 = route_bias<TK>(rt, e, topk, sel);
          const float p = sel ? __builtin_amdgcn_exp2f(fmaf(acc_s[i][vv], alpha, c2 - lse_t)) : 0.f;
          const float dp = acc_p[i][vv];
          acc_s[i][vv] = p * (dp - dl);
          const float pdp = p * dp;
          dx += pdp;
          sp += p;
#pragma unroll
          for (int t = 0; t < TK; ++t)
            if (t < topk && rt.idx[t] == e) {
              accA[t] += pdp;
              accM[t] += p;
            }
        }
    }

    // dQ^T += K^T . dS^T  (K^T read transposed from the natural K tile)
#pragma unroll
    for (int kk = 0; kk < SG / 16; ++kk) {
      const bf16x8 bs = pack8(acc_s[kk >> 1], 8 * (kk & 1));
#pragma unroll
      for (int j = 0; j < NO; ++j) {
        const bf16x8 a = lds_frag_T<true, true>(k_lds, PITCH, 16 * kk, 32 * j);
        acc_dq[j] = mfma32(a, bs, acc_dq[j]);
      }
    }
  }

  sp = wave_sum_pair(sp);
  const float inv_sp = sp > 0.f ? 1.f / sp : 0.f;
  dx = wave_sum_pair(dx) * inv_sp;  // delta of the normalised weights
  float dlg[TK];
#pragma unroll
  for (int t = 0; t < TK; ++t) dlg[t] = (wave_sum_pair(accA[t]) - dx * wave_sum_pair(accM[t])) * inv_sp;

  if (tok_ok) {
#pragma unroll
    for (int j = 0; j < NO; ++j) {
      const int f0 = 32 * j + 16 * g;
      if (f0 < HD) {
        bf16x8 lo, hi;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          lo[e] = (__bf16)(acc_dq[j][e] * scale);
          hi[e] = (__bf16)(acc_dq[j][8 + e] * scale);
        }
        bf16_t* dst = dq + tok * D + (long)h * HD + f0;
        *reinterpret_cast<bf16x8*>(dst) = lo;
        *reinterpret_cast<bf16x8*>(dst + 8) = hi;
      }
    }
    if (g == 0) {
      const long ntok = N;
      delta[(long)h * N + tok] = dx;
#pragma unroll
      for (int t = 0; t < TK; ++t)
        if (t < topk) dlg_part[((long)h * ntok + tok) * topk + t] = dlg[t];
    }
  }
}

// ---------------------------------------------------------------------------
// Fast dQ: head_dim 64, block sizes that are multiples of 32 (every Naylis
// configuration).  Same work and outputs as read_bwd_dq_kernel, organised as
// the fast forward: the tile's active 32-slot chunks (ascending) pass through
// LDS in stages of up to 4 chunks (K and V of 128 slots, 36 KiB), all of a
// stage's loads in flight at once and one barrier pair per stage; inside a
// stage each wave walks the chunks some token of its 32 selects with no
// barrier.  A chunk never spans two blocks, so its gate bias is one value per
// token.  At top-2 the kernel fits 168 VGPRs, so three workgroups share a CU
// (measured on MI355X: 8 % faster than 64-slot groups with one group of
// prefetch at config 2, 11 % at config 4; 8-chunk stages at two workgroups
// per CU were no faster than those groups).
template <int TK>
__global__ __launch_bounds__(256, TK <= 2 ? 3 : 2) void read_bwd_dq_fast_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const int32_t* __restrict__ top_idx, const float* __restrict__ top_gates, const bf16_t* __restrict__ o,
    const bf16_t* __restrict__ dout, const float* __restrict__ lse, bf16_t* __restrict__ dq,
    float* __restrict__ delta, float* __restrict__ dlg_part, uint8_t* __restrict__ tile_flags,
    const int32_t* __restrict__ order, long N, int H, int L, int E, int block_size, int topk, float alpha,
    float scale, int n_tiles) {
  constexpr int HD = 64, KS = HD / 16, NO = HD / 32, PITCH = HD + 8;
  constexpr int NT = 256;
  constexpr int SCH = 4;                       // 32-slot chunks per LDS stage
  constexpr int TILE = SCH * 32 * PITCH;       // bf16 elements of one staged tensor
  constexpr int PER = SCH * 32 * HD / 8 / NT;  // 16-byte pieces per thread per tensor
  static_assert(PER * NT * 8 == SCH * 32 * HD, "stage copy must tile the workgroup");

  __shared__ __attribute__((aligned(16))) bf16_t k_lds[TILE];
  __shared__ __attribute__((aligned(16))) bf16_t v_lds[TILE];
  __shared__ uint8_t flags[kMaxBlocks];
  __shared__ uint8_t tflags[2][kMaxBlocks];  // per 64-position half (the dK/dV kernel's tiles)
  __shared__ uint32_t chunks[kMaxGroups];  // (block << 16) | chunk index (slot / 32)
  __shared__ int n_chunks_s;

  const int G = H * n_tiles;
  const int wid = xcd_remap(blockIdx.x, G);
  const int tile = wid % n_tiles;
  const int h = wid / n_tiles;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int col = lane & 31;
  const long pos = (long)tile * 128 + wave * 32 + col;  // position in the token order
  const bool tok_ok = pos < N;
  const int32_t* ord = order_table(order);
  const long tok = tok_ok ? order_token(ord, pos, N) : 0;  // flattened b*S + s
  const int D = H * HD;
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(k, (uint32_t)L * (uint32_t)D * 2u);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(v, (uint32_t)L * (uint32_t)D * 2u);
  const int hoff = h * HD * 2;  // byte offset of head h in a row

  TokenRoute<TK> rt;
  load_route<TK>(rt, top_idx, top_gates, tok, tok_ok, topk);
  bf16x8 qf[KS], df[KS], of[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if (tok_ok) {
      const long off = tok * D + (long)h * HD + 16 * ks + 8 * g;
      qf[ks] = *reinterpret_cast<const bf16x8*>(q + off);
      df[ks] = *reinterpret_cast<const bf16x8*>(dout + off);
      of[ks] = *reinterpret_cast<const bf16x8*>(o + off);
    } else {
      qf[ks] = bf16x8{};
      df[ks] = bf16x8{};
      of[ks] = bf16x8{};
    }
  }
  const float lse_t = tok_ok ? lse[(long)h * N + tok] : 0.f;

  // ---- the tile's active chunks, ascending
  for (int e = tid; e < E; e += NT) {
    flags[e] = 0;
    tflags[0][e] = 0;
    tflags[1][e] = 0;
  }
  lds_barrier();
  if (g == 0 && tok_ok) {
#pragma unroll
    for (int t = 0; t < TK; ++t)
      if (t < topk && rt.idx[t] >= 0 && rt.idx[t] < E) {
        flags[rt.idx[t]] = 1;
        tflags[wave >> 1][rt.idx[t]] = 1;
      }
  }
  lds_barrier();
  if (tile_flags != nullptr && h == 0) {
    // the dK/dV kernel's 64-position tiles 2 tile and 2 tile + 1: which blocks their tokens select
    const long n_tt = (N + kDkdvTile - 1) / kDkdvTile;
    for (int i = tid; i < 2 * E; i += NT) {
      const long t64 = 2L * tile + i / E;
      if (t64 < n_tt) tile_flags[t64 * E + i % E] = tflags[i / E][i % E];
    }
  }
  if (wave == 0) {
    const int cpb = block_size >> 5;  // chunks per block
    int total = 0;
    for (int base = 0; base < E; base += 64) {
      const int e = base + lane;
      const bool act = e < E && flags[e] != 0;
      const unsigned long long m = __ballot(act);
      if (act) {
        const int p0 = (total + __popcll(m & ((1ull << lane) - 1ull))) * cpb;
        for (int j = 0; j < cpb; ++j) chunks[p0 + j] = ((uint32_t)e << 16) | (uint32_t)(e * cpb + j);
      }
      total += __popcll(m);
    }
    if (lane == 0) n_chunks_s = total * cpb;
  }

  // delta0 = rowsum(o * do) from the rows loaded above
  float dl = 0.f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
#pragma unroll
    for (int e = 0; e < 8; ++e) dl = fmaf((float)of[ks][e], (float)df[ks][e], dl);
  dl = wave_sum_pair(dl);

  f32x16 acc_dq[NO];
#pragma unroll
  for (int j = 0; j < NO; ++j) acc_dq[j] = f32x16{};
  // dlog_gates without the bf16 rounding of o inside delta: per selection t
  // accumulate A_t = sum_{n in block t} P dP and M_t = sum_{n in block t} P,
  // plus dx = sum_n P dP and S = sum_n P over every selected slot.  P is
  // recomputed from the forward's lse, so S = 1 only up to the rounding of
  // the forward's row sum; dividing by S makes the weights exactly
  // normalised: delta = dx / S and dlog_t = A_t / S - delta M_t / S.
  float accA[TK], accM[TK];
#pragma unroll
  for (int t = 0; t < TK; ++t) {
    accA[t] = 0.f;
    accM[t] = 0.f;
  }
  float dx = 0.f, sp = 0.f;
  lds_barrier();
  const int n_ch = n_chunks_s;

  for (int s0 = 0; s0 < n_ch; s0 += SCH) {
    const int nst = min(SCH, n_ch - s0);
    if (s0 > 0) lds_barrier();  // every wave is done with the previous stage
    {
      uint4 kr[PER], vr[PER];
#pragma unroll
      for (int r = 0; r < PER; ++r) {
        const int p = tid + NT * r;
        const int row = p >> 3, c8 = p & 7, ch = row >> 5;
        // rows of chunks beyond the stage read past the buffer's end, which
        // a buffer load returns as zeros
        const uint32_t slot = ch < nst ? (chunks[s0 + ch] & 0xffffu) * 32u + (uint32_t)(row & 31) : (uint32_t)L;
        const uint32_t off = (slot * (uint32_t)D + 8u * (uint32_t)c8) * 2u;
        kr[r] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(krs, off, hoff, 0));
        vr[r] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vrs, off, hoff, 0));
      }
#pragma unroll
      for (int r = 0; r < PER; ++r) {
        const int p = tid + NT * r;
        const int row = p >> 3, c8 = p & 7;
        *reinterpret_cast<uint4*>(&k_lds[row * PITCH + 8 * c8]) = kr[r];
        *reinterpret_cast<uint4*>(&v_lds[row * PITCH + 8 * c8]) = vr[r];
      }
    }
    // chunks of this stage that some token of the wave selects
    unsigned mine = 0;
    for (int c = 0; c < nst; ++c) {
      const int e = (int)(chunks[s0 + c] >> 16);
      bool sel = false;
#pragma unroll
      for (int t = 0; t < TK; ++t) sel |= t < topk && rt.idx[t] == e;
      if (__any(sel)) mine |= 1u << c;
    }
    lds_barrier();

    while (mine) {
      const int c = __builtin_ctz(mine);
      mine &= mine - 1;
      // S^T = K Q^T and dP^T = V dO^T for the chunk's 32 slots x the wave's 32 tokens
      f32x16 acc_s = f32x16{}, acc_p = f32x16{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int off = (32 * c + col) * PITCH + 16 * ks + 8 * g;
        const bf16x8 ak = *reinterpret_cast<const bf16x8*>(&k_lds[off]);
        const bf16x8 av = *reinterpret_cast<const bf16x8*>(&v_lds[off]);
        acc_s = mfma32(ak, qf[ks], acc_s);
        acc_p = mfma32(av, df[ks], acc_p);
      }
      const int e = (int)(chunks[s0 + c] >> 16);
      bool sel;
      const float c2 = route_bias<TK>(rt, e, topk, sel);
      const float add = sel ? c2 - lse_t : -INFINITY;
      float rsA = 0.f, rsM = 0.f;
#pragma unroll
      for (int vv = 0; vv < 16; ++vv) {
        const float p = __builtin_amdgcn_exp2f(fmaf(acc_s[vv], alpha, add));
        const float dp = acc_p[vv];
        acc_s[vv] = p * (dp - dl);
        rsA = fmaf(p, dp, rsA);
        rsM += p;
      }
      dx += rsA;
      sp += rsM;
#pragma unroll
      for (int t = 0; t < TK; ++t)
        if (t < topk && rt.idx[t] == e) {
          accA[t] += rsA;
          accM[t] += rsM;
        }
      // dQ^T += K^T . dS^T  (K^T read transposed from the natural K rows)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const bf16x8 bs = pack8(acc_s, 8 * kk);
#pragma unroll
        for (int j = 0; j < NO; ++j) {
          const bf16x8 a = lds_frag_T<true, true>(k_lds, PITCH, 32 * c + 16 * kk, 32 * j);
          acc_dq[j] = mfma32(a, bs, acc_dq[j]);
        }
      }
    }
  }

  sp = wave_sum_pair(sp);
  const float inv_sp = sp > 0.f ? 1.f / sp : 0.f;
  dx = wave_sum_pair(dx) * inv_sp;  // delta of the normalised weights
  float dlg[TK];
#pragma unroll
  for (int t = 0; t < TK; ++t) dlg[t] = (wave_sum_pair(accA[t]) - dx * wave_sum_pair(accM[t])) * inv_sp;

  if (tok_ok) {
#pragma unroll
    for (int j = 0; j < NO; ++j) {
      const int f0 = 32 * j + 16 * g;
      bf16x8 lo, hi;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        lo[e] = (__bf16)(acc_dq[j][e] * scale);
        hi[e] = (__bf16)(acc_dq[j][8 + e] * scale);
      }
      bf16_t* dst = dq + tok * D + (long)h * HD + f0;
      *reinterpret_cast<bf16x8*>(dst) = lo;
      *reinterpret_cast<bf16x8*>(dst + 8) = hi;
    }
    if (g == 0) {
      delta[(long)h * N + tok] = dx;
#pragma unroll
      for (int t = 0; t < TK; ++t)
        if (t < topk) dlg_part[((long)h * N + tok) * topk + t] = dlg[t];
    }
  }
}

// ---------------------------------------------------------------------------
// Active 64-token tiles per 128-slot group (kDkdvTile positions of the token order each).

// tile_flags[tile][e] = 1 when a token of the tile (64 positions of the token
// order) selects block e
__global__ __launch_bounds__(64) void read_tile_flags_kernel(const int32_t* __restrict__ top_idx,
                                                             const int32_t* __restrict__ order,
                                                             uint8_t* __restrict__ tile_flags, long ntok, int E,
                                                             int topk) {
  __shared__ uint8_t fl[kMaxBlocks];
  const long tile = blockIdx.x;
  for (int e = threadIdx.x; e < E; e += 64) fl[e] = 0;
  __syncthreads();
  const long pos = tile * kDkdvTile + threadIdx.x;
  const long tk = pos < ntok ? order_token(order_table(order), pos, ntok) : ntok;
  if (tk < ntok)
    for (int t = 0; t < topk; ++t) {
      const int id = top_idx[tk * topk + t];
      if (id >= 0 && id < E) fl[id] = 1;
    }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 64) tile_flags[tile * E + e] = fl[e];
}

// list[sg][0 .. count[sg]) = ascending tiles with a token selecting a block
// that overlaps slots [128 sg, 128 sg + 128)
__global__ __launch_bounds__(256) void read_tile_lists_kernel(const uint8_t* __restrict__ tile_flags,
                                                              int32_t* __restrict__ list, int32_t* __restrict__ count,
                                                              int n_ttiles, int E, int L, int block_size) {
  __shared__ int scan[256];
  const int sg = blockIdx.x;
  const int blk_lo = (sg * 128) / block_size;
  const int blk_hi = min((min(sg * 128 + 128, L) - 1) / block_size, E - 1);
  int total = 0;
  for (int base = 0; base < n_ttiles; base += 256) {
    const int t = base + threadIdx.x;
    int act = 0;
    if (t < n_ttiles)
      for (int e = blk_lo; e <= blk_hi; ++e) act |= tile_flags[(long)t * E + e];
    scan[threadIdx.x] = act;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {  // inclusive Hillis-Steele scan
      const int vadd = threadIdx.x >= off ? scan[threadIdx.x - off] : 0;
      __syncthreads();
      scan[threadIdx.x] += vadd;
      __syncthreads();
    }
    if (act) list[(long)sg * n_ttiles + total + scan[threadIdx.x] - 1] = t;
    total += scan[255];
    __syncthreads();
  }
  if (threadIdx.x == 0) count[sg] = total;
}

// Work split of the dK / dV pass.  Its items are the (128-slot group, active
// 64-token tile) pairs, group-major: group sg owns items [pre[sg], pre[sg+1])
// with pre the exclusive prefix of the per-group tile counts.  Per head the
// items are cut into R equal contiguous ranges (the last ones may be short or
// empty), one workgroup each, so every workgroup does the same number of
// tiles however unevenly the groups are selected.  A range that crosses into
// another group writes the partial of the group it leaves and starts afresh:
// the segment (range r, group sg) writes partial r + sg, which is unique
// (a later group in the same or a later range has a larger sum), and group
// sg's partials are r + sg for r in [pre[sg] / per, (pre[sg+1] - 1) / per].
//
// Exclusive prefix of count[0 .. n_sg) into pre[0 .. n_sg], pre[n_sg] the
// total, by one wave (n_sg <= kMaxSlotGroups = 128: two groups per lane).
__device__ __forceinline__ void tile_count_prefix(const int32_t* __restrict__ count, int n_sg, int* pre) {
  const int lane = threadIdx.x & 63;
  const int c0 = 2 * lane < n_sg ? count[2 * lane] : 0;
  const int c1 = 2 * lane + 1 < n_sg ? count[2 * lane + 1] : 0;
  int incl = c0 + c1;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  const int excl = incl - c0 - c1;
  if (2 * lane < n_sg) pre[2 * lane] = excl;
  if (2 * lane + 1 < n_sg) pre[2 * lane + 1] = excl + c0;
  if (lane == 63) pre[n_sg] = incl;
}

// dK / dV over the shared bank.  One workgroup per (head, range of items);
// four waves, wave w owning slots 128 sg + 32 w + lane%32 of the current
// group, whose K / V rows it holds in registers.  Two workgroups share a CU,
// so the two waves on a SIMD belong to different workgroups: they drift apart
// and one's MFMA work overlaps the other's exp2 work (one 8-wave workgroup
// per CU, waves splitting each tile's tokens, measured 4-6 % slower).
// Lanes own slots (S = Q K^T orientation), so P and dS come out of the
// accumulators already in the B-operand layout of dV^T = dO^T P and
// dK^T = Q^T dS, whose A operands are read transposed from the tiles.
template <int HD, bool ALIGNED, int TK, bool SPLIT_V>
__global__ __launch_bounds__(256, 2) void read_bwd_dkdv_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const int32_t* __restrict__ top_idx, const float* __restrict__ top_gates, const bf16_t* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, const int32_t* __restrict__ tile_list,
    const int32_t* __restrict__ tile_count, float* __restrict__ dk_part, float* __restrict__ dv_part,
    bf16_t* __restrict__ dk_out, bf16_t* __restrict__ dv_out, float dk_scale, const int32_t* __restrict__ order,
    long ntok, int H, int L, int Lq, int E, int block_size, int topk, float alpha, int R, int n_ttiles) {
  constexpr int HDP = HD < 32 ? 32 : HD;
  constexpr int KS = HD / 16;
  constexpr int NO = HDP / 32;
  constexpr int TT = kDkdvTile;
  constexpr int PITCH = HDP + 8;
  constexpr int NT = 256;
  constexpr int VEC = TT * HD / 8;        // 16-byte vectors per staged tensor tile
  constexpr int PER = (VEC + NT - 1) / NT;

  // two buffers: tile it + 1 is stored while tile it is read, one barrier per tile
  __shared__ __attribute__((aligned(16))) bf16_t q_lds2[2][TT * PITCH];
  __shared__ __attribute__((aligned(16))) bf16_t do_lds2[2][TT * PITCH];
  __shared__ __attribute__((aligned(16))) float add_lds2[2][4][TT];  // per quarter: c2 - lse, or -inf
  __shared__ __attribute__((aligned(16))) float dl_lds2[2][TT];    // -delta per token
  __shared__ int32_t idx_lds2[2][TT * TK];
  __shared__ float lg_lds2[2][TT * TK];
  __shared__ float lse_lds2[2][TT];
  __shared__ int pre[kMaxSlotGroups + 1];

  const int n_sg = Lq / 128;
  const int wid = xcd_remap(blockIdx.x, H * R);
  const int r = wid % R;
  const int h = wid / R;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int col = lane & 31;
  const int D = H * HD;

  if (wave == 0) tile_count_prefix(tile_count, n_sg, pre);
  lds_barrier();
  const int total = pre[n_sg];
  const int per = (total + R - 1) / R;
  const int i_begin = min(total, r * per), i_end = min(total, i_begin + per);
  if (i_begin >= i_end) return;  // uniform over the workgroup
  // first group at or after `s` whose items reach past item j
  auto group_of = [&](int j, int s) {
    while (j >= pre[s + 1]) ++s;
    return s;
  };
  auto item_tile = [&](int j, int s) { return tile_list[(long)s * n_ttiles + (j - pre[s])]; };

  // the current group's slots and K / V rows
  int sgc = group_of(i_begin, 0);
  int slot = 0, lane_blk = 0;
  bool slot_ok = false;
  bf16x8 kf[KS], vf[KS];
  auto load_kv = [&]() {
    slot = sgc * 128 + wave * 32 + col;
    slot_ok = slot < L;
    lane_blk = slot / block_size;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (slot_ok) {
        const long off = (long)slot * D + (long)h * HD + 16 * ks + 8 * g;
        kf[ks] = *reinterpret_cast<const bf16x8*>(k + off);
        vf[ks] = *reinterpret_cast<const bf16x8*>(v + off);
      } else {
        kf[ks] = bf16x8{};
        vf[ks] = bf16x8{};
      }
    }
  };
  load_kv();
  f32x16 acc_dk[NO], acc_dv[NO];
#pragma unroll
  for (int j = 0; j < NO; ++j) {
    acc_dk[j] = f32x16{};
    acc_dv[j] = f32x16{};
  }
  if constexpr (HD < 32) {
    for (int i = tid; i < 2 * TT * PITCH; i += NT) {
      q_lds2[i / (TT * PITCH)][i % (TT * PITCH)] = 0;
      do_lds2[i / (TT * PITCH)][i % (TT * PITCH)] = 0;
    }
  }

  // prefetch registers: Q / dO vectors, per-token routing, lse, delta
  uint4 qreg[PER], dreg[PER];
  int pidx[TK];
  float pg[TK], plse = 0.f, pdl = 0.f;
  // per-thread constant part of the tile copy: row (token in tile) and column
  int cp_row[PER], cp_col[PER];
#pragma unroll
  for (int rr = 0; rr < PER; ++rr) {
    const int vi = tid + NT * rr;
    cp_row[rr] = vi < VEC ? vi / (HD / 8) : TT;
    cp_col[rr] = h * HD + 8 * (vi % (HD / 8));
  }
  // Tokens of a tile (rows of this thread's copies, and row tid < TT for the
  // routing / statistics), fetched from the token order one tile ahead of the
  // data loads that use them.  The raw order entries are only checked when
  // those loads are issued (next iteration, after the loop's wait for the
  // previous tile), so fetching them never makes the wave wait for the tile
  // loads just issued.
  const int32_t* ord = order_table(order);
  long rpos[PER], tpos = -1;  // position in the order, -1: no token
  int rraw[PER], traw = 0;    // the order's entry at that position
  auto fetch_tokens = [&](int tt) {
    const long pos0 = (long)tt * TT;
    const int rows = (int)min((long)TT, ntok - pos0);
#pragma unroll
    for (int rr = 0; rr < PER; ++rr) {
      rpos[rr] = cp_row[rr] < rows ? pos0 + cp_row[rr] : -1;
      if (ord != nullptr && rpos[rr] >= 0) rraw[rr] = ord[rpos[rr]];
    }
    tpos = (tid < TT && tid < rows) ? pos0 + tid : -1;
    if (ord != nullptr && tpos >= 0) traw = ord[tpos];
  };
  auto token_at = [&](long pos, int raw) -> long {
    if (pos < 0 || ord == nullptr) return pos;
    return (raw >= 0 && raw < ntok) ? (long)raw : pos;  // a malformed entry falls back to the position
  };
  auto load_tile = [&]() {
    long rtok[PER];
#pragma unroll
    for (int rr = 0; rr < PER; ++rr) rtok[rr] = token_at(rpos[rr], rraw[rr]);
    const long ttok = token_at(tpos, traw);
#pragma unroll
    for (int rr = 0; rr < PER; ++rr) {
      uint4 qv = make_uint4(0, 0, 0, 0), dv4 = make_uint4(0, 0, 0, 0);
      if (rtok[rr] >= 0) {
        const long off = rtok[rr] * D + cp_col[rr];
        qv = *reinterpret_cast<const uint4*>(q + off);
        dv4 = *reinterpret_cast<const uint4*>(dout + off);
      }
      qreg[rr] = qv;
      dreg[rr] = dv4;
    }
    if (tid < TT) {
      const bool ok = ttok >= 0;
      const long tk = ok ? ttok : 0;
#pragma unroll
      for (int t = 0; t < TK; ++t) {
        pidx[t] = (ok && t < topk) ? top_idx[tk * topk + t] : -1;
        pg[t] = (ok && t < topk) ? top_gates[tk * topk + t] : 1.f;
      }
      plse = ok ? lse[(long)h * ntok + tk] : 0.f;
      pdl = ok ? delta[(long)h * ntok + tk] : 0.f;
    }
  };
  // stores the prefetched tile; sg: the group the tile is read against
  auto store_tile = [&](int buf, int sg) {
    bf16_t* q_lds = q_lds2[buf];
    bf16_t* do_lds = do_lds2[buf];
    float(*add_lds)[TT] = add_lds2[buf];
    float* dl_lds = dl_lds2[buf];
    int32_t* idx_lds = idx_lds2[buf];
    float* lg_lds = lg_lds2[buf];
    float* lse_lds = lse_lds2[buf];
#pragma unroll
    for (int rr = 0; rr < PER; ++rr) {
      const int vi = tid + NT * rr;
      if (vi < VEC) {
        const int row = vi / (HD / 8), c8 = vi % (HD / 8);
        *reinterpret_cast<uint4*>(&q_lds[row * PITCH + 8 * c8]) = qreg[rr];
        *reinterpret_cast<uint4*>(&do_lds[row * PITCH + 8 * c8]) = dreg[rr];
      }
    }
    if (tid < TT) {
      float lg2[TK];
#pragma unroll
      for (int t = 0; t < TK; ++t) {
        lg2[t] = log2f(fmaxf(pg[t], 1e-9f));
        idx_lds[tid * TK + t] = pidx[t];
        lg_lds[tid * TK + t] = lg2[t];
      }
      lse_lds[tid] = plse;
      dl_lds[tid] = -pdl;
      if constexpr (ALIGNED) {
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int e = (sg * 128 + qq * 32) / block_size;
          float c = 0.f;
          bool sel = false;
#pragma unroll
          for (int t = 0; t < TK; ++t)
            if (t < topk && pidx[t] == e) {
              c += lg2[t];
              sel = true;
            }
          add_lds[qq][tid] = sel ? c - plse : -INFINITY;
        }
      }
    }
  };
  // this segment's sums into partial r + sgc (rows of the group's slots); a
  // segment holding all of the group's items is the group's whole sum and
  // goes straight to dk / dv as the reduce would write it (the reduce skips
  // groups with one segment)
  auto flush = [&]() {
    if (!slot_ok) return;
    if (pre[sgc] >= i_begin && pre[sgc + 1] <= i_end) {
#pragma unroll
      for (int j = 0; j < NO; ++j) {
        const int f0 = 32 * j + 16 * g;
        if (f0 < HD) {
          const long o = (long)slot * D + (long)h * HD + f0;
          bf16x8 k0, k1, v0, v1;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            k0[e] = (__bf16)(acc_dk[j][e] * dk_scale);
            k1[e] = (__bf16)(acc_dk[j][8 + e] * dk_scale);
            v0[e] = (__bf16)acc_dv[j][e];
            v1[e] = (__bf16)acc_dv[j][8 + e];
          }
          *reinterpret_cast<bf16x8*>(dk_out + o) = k0;
          *reinterpret_cast<bf16x8*>(dk_out + o + 8) = k1;
          *reinterpret_cast<bf16x8*>(dv_out + o) = v0;
          *reinterpret_cast<bf16x8*>(dv_out + o + 8) = v1;
        }
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < NO; ++j) {
      const int f0 = 32 * j + 16 * g;
      if (f0 < HD) {
        const long base = ((long)(r + sgc) * 128 + wave * 32 + col) * D + (long)h * HD + f0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          *reinterpret_cast<f32x4*>(dk_part + base + 4 * u) =
              f32x4{acc_dk[j][4 * u], acc_dk[j][4 * u + 1], acc_dk[j][4 * u + 2], acc_dk[j][4 * u + 3]};
          *reinterpret_cast<f32x4*>(dv_part + base + 4 * u) =
              f32x4{acc_dv[j][4 * u], acc_dv[j][4 * u + 1], acc_dv[j][4 * u + 2], acc_dv[j][4 * u + 3]};
        }
      }
    }
  };

  // groups of items it + 1 .. it + 3 (the pipeline's stages), walked forward
  int sg1 = sgc, sg2 = sgc, sg3 = sgc;
  fetch_tokens(item_tile(i_begin, sgc));
  load_tile();
  if (i_begin + 1 < i_end) {
    sg1 = group_of(i_begin + 1, sgc);
    fetch_tokens(item_tile(i_begin + 1, sg1));
  }
  store_tile(0, sgc);
  if (i_begin + 1 < i_end) load_tile();                  // tile i_begin + 1 in flight
  if (i_begin + 2 < i_end) {
    sg2 = group_of(i_begin + 2, sg1);
    fetch_tokens(item_tile(i_begin + 2, sg2));
  }
  lds_barrier();
  for (int it = i_begin; it < i_end; ++it) {
    const int buf = (it - i_begin) & 1;
    // tile it + 1 into the other buffer (last read before the previous barrier)
    if (it + 1 < i_end) store_tile(buf ^ 1, sg1);
    if (it + 2 < i_end) load_tile();                       // in flight during the math below
    if (it + 3 < i_end) {                                  // the tokens of the tile after
      sg3 = group_of(it + 3, sg2);
      fetch_tokens(item_tile(it + 3, sg3));
    }
    const bf16_t* q_lds = q_lds2[buf];
    const bf16_t* do_lds = do_lds2[buf];
    const float(*add_lds)[TT] = add_lds2[buf];
    const float* dl_lds = dl_lds2[buf];
    const int32_t* idx_lds = idx_lds2[buf];
    const float* lg_lds = lg_lds2[buf];
    const float* lse_lds = lse_lds2[buf];

#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {  // the tile's two 32-token halves
      // ---- S = Q K^T and dP - delta = dO V^T - delta for this wave's 32 tokens x
      // 32 slots (the dP accumulator starts at -delta of each register's token)
      f32x16 acc_s = f32x16{}, acc_p;
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        const f32x4 nd4 = *reinterpret_cast<const f32x4*>(&dl_lds[32 * hh + 8 * j4 + 4 * g]);
#pragma unroll
        for (int u = 0; u < 4; ++u) acc_p[4 * j4 + u] = nd4[u];
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int off = (32 * hh + col) * PITCH + 16 * ks + 8 * g;
        const bf16x8 aq = *reinterpret_cast<const bf16x8*>(&q_lds[off]);
        const bf16x8 ad = *reinterpret_cast<const bf16x8*>(&do_lds[off]);
        acc_s = mfma32(aq, kf[ks], acc_s);
        acc_p = mfma32(ad, vf[ks], acc_p);
      }
      // ---- P and dS, registers indexed by token
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        const int r0 = 32 * hh + 8 * j4 + 4 * g;  // tokens r0 .. r0+3 in registers 4*j4 .. 4*j4+3
        f32x4 ad4;
        if constexpr (ALIGNED) {
          ad4 = *reinterpret_cast<const f32x4*>(&add_lds[wave][r0]);
        } else {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            float c = 0.f;
            bool sel = false;
#pragma unroll
            for (int t = 0; t < TK; ++t)
              if (t < topk && idx_lds[(r0 + u) * TK + t] == lane_blk) {
                c += lg_lds[(r0 + u) * TK + t];
                sel = true;
              }
            ad4[u] = (sel && slot_ok) ? c - lse_lds[r0 + u] : -INFINITY;
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int vv = 4 * j4 + u;
          const float p = __builtin_amdgcn_exp2f(fmaf(acc_s[vv], alpha, ad4[u]));
          acc_s[vv] = p;
          acc_p[vv] = p * acc_p[vv];
        }
      }
      // ---- dV^T += dO^T P ; dK^T += Q^T dS   (K = this wave's 32 tokens)
      // dV sums P over thousands of tokens, so P enters as hi + lo bf16 parts
      // (hi = bf16(P), lo = bf16(P - hi)); bf16 rounding of P would otherwise
      // dominate the error of small dV entries.
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        bf16x8 bp, bp_lo;
        if constexpr (SPLIT_V)
          pack8_hilo(acc_s, 8 * kk, bp, bp_lo);
        else
          bp = pack8(acc_s, 8 * kk);
        const bf16x8 bd = pack8(acc_p, 8 * kk);
#pragma unroll
        for (int j = 0; j < NO; ++j) {
          const bf16x8 a_do = lds_frag_T<true, true>(do_lds, PITCH, 32 * hh + 16 * kk, 32 * j);
          const bf16x8 a_q = lds_frag_T<true, true>(q_lds, PITCH, 32 * hh + 16 * kk, 32 * j);
          acc_dv[j] = mfma32(a_do, bp, acc_dv[j]);
          if constexpr (SPLIT_V) acc_dv[j] = mfma32(a_do, bp_lo, acc_dv[j]);
          acc_dk[j] = mfma32(a_q, bd, acc_dk[j]);
        }
      }
    }
    lds_barrier();  // every wave is done with buffer buf before it is refilled
    if (it + 1 == i_end || sg1 != sgc) {  // the segment of group sgc ends with this tile
      flush();
      if (it + 1 < i_end) {
        sgc = sg1;
        load_kv();
#pragma unroll
        for (int j = 0; j < NO; ++j) {
          acc_dk[j] = f32x16{};
          acc_dv[j] = f32x16{};
        }
      }
    }
    sg1 = sg2;
    sg2 = sg3;
  }
}

// One launch for both reductions of the backward: workgroups [0, kv_blocks)
// sum the dK/dV partials, the rest the per-head dlog partials.
//
// dk / dv of a slot = the sum of its group's partials in ascending range order
// (a fixed order; the work split above), dk scaled; groups with a single
// segment were written by the dK/dV kernel.  A workgroup takes whole slot
// rows; pre: LDS for the group prefix.
__device__ __forceinline__ void read_bwd_reduce_kv(const float* __restrict__ dk_part,
                                                   const float* __restrict__ dv_part,
                                                   const int32_t* __restrict__ tile_count, bf16_t* __restrict__ dk,
                                                   bf16_t* __restrict__ dv, int L, int n_sg, int D, int R,
                                                   float scale, long blk, long nblk, int* pre) {
  if (threadIdx.x < 64) tile_count_prefix(tile_count, n_sg, pre);
  __syncthreads();
  const int total = pre[n_sg];
  const int per = max(1, (total + R - 1) / R);
  const long stride = 128L * D;  // one partial
  for (long slot = blk; slot < L; slot += nblk) {
    const int sg = (int)(slot >> 7);
    const int lo = pre[sg], hi = pre[sg + 1];
    const int r0 = lo / per, n = hi > lo ? (hi - 1) / per - r0 + 1 : 0;
    if (n == 1) continue;  // the dK/dV kernel wrote the group's rows
    const long base = ((long)(r0 + sg) * 128 + (slot & 127)) * D;
    for (int c4 = threadIdx.x; c4 < D / 4; c4 += blockDim.x) {
      f32x4 sk = f32x4{0.f, 0.f, 0.f, 0.f}, sv = f32x4{0.f, 0.f, 0.f, 0.f};
      // partials in order, their loads issued four at a time
      int i = 0;
      for (; i + 4 <= n; i += 4) {
        f32x4 pk[4], pv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          pk[u] = *reinterpret_cast<const f32x4*>(dk_part + base + (i + u) * stride + 4 * c4);
          pv[u] = *reinterpret_cast<const f32x4*>(dv_part + base + (i + u) * stride + 4 * c4);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          sk += pk[u];
          sv += pv[u];
        }
      }
      for (; i < n; ++i) {
        sk += *reinterpret_cast<const f32x4*>(dk_part + base + i * stride + 4 * c4);
        sv += *reinterpret_cast<const f32x4*>(dv_part + base + i * stride + 4 * c4);
      }
      bf16x4 ok, ov;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        ok[u] = (__bf16)(sk[u] * scale);
        ov[u] = (__bf16)sv[u];
      }
      *reinterpret_cast<bf16x4*>(dk + slot * D + 4 * c4) = ok;
      *reinterpret_cast<bf16x4*>(dv + slot * D + 4 * c4) = ov;
    }
  }
}

// d(top_gates) = (sum_h dlog partial) / g  where g >= 1e-9, else 0
// (the gradient of log(clamp_min(g, 1e-9)), triton_gpu.py:435).
__device__ __forceinline__ void read_bwd_reduce_gates(const float* __restrict__ dlg_part,
                                                      const float* __restrict__ top_gates,
                                                      float* __restrict__ dgates, long n, int H, long blk, long nblk) {
  for (long i = blk * (long)blockDim.x + threadIdx.x; i < n; i += nblk * blockDim.x) {
    float s = 0.f;
    int h = 0;
    for (; h + 8 <= H; h += 8) {  // head partials in order, loads issued eight at a time
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = dlg_part[(long)(h + u) * n + i];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; h < H; ++h) s += dlg_part[(long)h * n + i];
    const float gt = top_gates[i];
    dgates[i] = gt >= 1e-9f ? s / gt : 0.f;
  }
}

__global__ __launch_bounds__(256) void read_bwd_reduce_kernel(
    const float* __restrict__ dk_part, const float* __restrict__ dv_part, const int32_t* __restrict__ tile_count,
    bf16_t* __restrict__ dk, bf16_t* __restrict__ dv, int L, int n_sg, int D, int R, float scale, int kv_blocks,
    const float* __restrict__ dlg_part, const float* __restrict__ top_gates, float* __restrict__ dgates, long ng,
    int H) {
  __shared__ int pre[kMaxSlotGroups + 1];
  if ((int)blockIdx.x < kv_blocks)
    read_bwd_reduce_kv(dk_part, dv_part, tile_count, dk, dv, L, n_sg, D, R, scale, blockIdx.x, kv_blocks, pre);
  else
    read_bwd_reduce_gates(dlg_part, top_gates, dgates, ng, H, blockIdx.x - kv_blocks, gridDim.x - kv_blocks);
}

// ---------------------------------------------------------------------------
static float read_scale(int HD) { return (float)(1.0 / __builtin_sqrt((double)HD)); }

template <int HD, int SG, bool AL, int TK>
static void dq_inst(const void* q, const void* k, const void* v, const int32_t* ti, const float* tg, const void* o,
                    const void* dout, const float* lse, void* dq, float* delta, float* dlg, const ReadDims& d,
                    hipStream_t st) {
  const long N = (long)d.B * d.S;
  const int n_tiles = (int)((N + 127) / 128);
  const float scale = read_scale(HD);
  NAYLIS_TIMED("read_bwd_dq", st,
               hipLaunchKernelGGL((read_bwd_dq_kernel<HD, SG, AL, TK>), dim3(d.H * n_tiles), dim3(256), 0, st,
                                  (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, ti, tg, (const bf16_t*)o,
                                  (const bf16_t*)dout, lse, (bf16_t*)dq, delta, dlg, d.order, N, d.H, d.L, d.E,
                                  d.block_size, d.topk, scale * kLog2e, scale, n_tiles));
}

template <int HD, int TK>
static void dq_hdk(const void* q, const void* k, const void* v, const int32_t* ti, const float* tg, const void* o,
                   const void* dout, const float* lse, void* dq, float* delta, float* dlg, uint8_t* tflags,
                   const ReadDims& d, hipStream_t st) {
  if constexpr (HD == 64) {
    if (read_dq_writes_tile_flags(d)) {  // the staged kernel (every Naylis configuration)
      const long N = (long)d.B * d.S;
      const int n_tiles = (int)((N + 127) / 128);
      const float scale = read_scale(HD);
      NAYLIS_TIMED("read_bwd_dq", st,
                   hipLaunchKernelGGL((read_bwd_dq_fast_kernel<TK>), dim3(d.H * n_tiles), dim3(256), 0, st,
                                      (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, ti, tg,
                                      (const bf16_t*)o, (const bf16_t*)dout, lse, (bf16_t*)dq, delta, dlg, tflags,
                                      d.order, N, d.H, d.L, d.E, d.block_size, d.topk, scale * kLog2e, scale,
                                      n_tiles));
      return;
    }
  }
  constexpr int SGMAX = HD <= 64 ? 64 : 32;
  if (d.block_size % SGMAX == 0)
    dq_inst<HD, SGMAX, true, TK>(q, k, v, ti, tg, o, dout, lse, dq, delta, dlg, d, st);
  else if (d.block_size % 32 == 0)
    dq_inst<HD, 32, true, TK>(q, k, v, ti, tg, o, dout, lse, dq, delta, dlg, d, st);
  else
    dq_inst<HD, 32, false, TK>(q, k, v, ti, tg, o, dout, lse, dq, delta, dlg, d, st);
}

template <int HD>
static void dq_hd(const void* q, const void* k, const void* v, const int32_t* ti, const float* tg, const void* o,
                  const void* dout, const float* lse, void* dq, float* delta, float* dlg, uint8_t* tflags,
                  const ReadDims& d, hipStream_t st) {
  if (d.topk <= 2)
    dq_hdk<HD, 2>(q, k, v, ti, tg, o, dout, lse, dq, delta, dlg, tflags, d, st);
  else
    dq_hdk<HD, kMaxTopK>(q, k, v, ti, tg, o, dout, lse, dq, delta, dlg, tflags, d, st);
}

bool read_dq_writes_tile_flags(const ReadDims& d) { return d.HD == 64 && d.block_size % 32 == 0; }

hipError_t launch_read_bwd_dq(const void* q, const void* k, const void* v, const int32_t* top_idx,
                              const float* top_gates, const void* o, const void* dout, const float* lse, void* dq,
                              float* delta, float* dlg_part, uint8_t* tile_flags, const ReadDims& d,
                              hipStream_t st) {
  switch (d.HD) {
    case 16: dq_hd<16>(q, k, v, top_idx, top_gates, o, dout, lse, dq, delta, dlg_part, tile_flags, d, st); break;
    case 32: dq_hd<32>(q, k, v, top_idx, top_gates, o, dout, lse, dq, delta, dlg_part, tile_flags, d, st); break;
    case 64: dq_hd<64>(q, k, v, top_idx, top_gates, o, dout, lse, dq, delta, dlg_part, tile_flags, d, st); break;
    case 128: dq_hd<128>(q, k, v, top_idx, top_gates, o, dout, lse, dq, delta, dlg_part, tile_flags, d, st); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

int read_bwd_n_ttiles(const ReadDims& d) { return (int)(((long)d.B * d.S + kDkdvTile - 1) / kDkdvTile); }

// ranges of the dK/dV work split per head: the heads' ranges together fill
// the chip's 256 CUs with two workgroups each
int read_bwd_ranges(const ReadDims& d) { return d.H >= 512 ? 1 : 512 / d.H; }
int read_bwd_parts(const ReadDims& d) { return read_bwd_ranges(d) + read_lq(d.L) / 128 - 1; }

hipError_t launch_read_tile_lists(const int32_t* top_idx, uint8_t* tile_flags, int32_t* list, int32_t* count,
                                  const ReadDims& d, hipStream_t st) {
  const long ntok = (long)d.B * d.S;
  const int n_tt = read_bwd_n_ttiles(d);
  // the staged dQ kernel already wrote the flags (launch_read_bwd_dq runs first)
  if (n_tt > 0 && !read_dq_writes_tile_flags(d))
    NAYLIS_TIMED("read_tile_lists", st,
                 hipLaunchKernelGGL(read_tile_flags_kernel, dim3(n_tt), dim3(64), 0, st, top_idx, d.order, tile_flags,
                                    ntok, d.E, d.topk));
  NAYLIS_TIMED("read_tile_lists", st,
               hipLaunchKernelGGL(read_tile_lists_kernel, dim3(read_lq(d.L) / 128), dim3(256), 0, st, tile_flags, list,
                                  count, n_tt, d.E, d.L, d.block_size));
  return hipGetLastError();
}

template <int HD, bool AL, int TK>
static void dkdv_inst(const void* q, const void* k, const void* v, const int32_t* ti, const float* tg,
                      const void* dout, const float* lse, const float* delta, const int32_t* list,
                      const int32_t* count, float* dkp, float* dvp, void* dk, void* dv, const ReadDims& d,
                      hipStream_t st) {
  const int Lq = read_lq(d.L);
  const int R = read_bwd_ranges(d);
  const float alpha = read_scale(HD) * kLog2e;
  NAYLIS_TIMED("read_bwd_dkdv", st,
               hipLaunchKernelGGL((read_bwd_dkdv_kernel<HD, AL, TK, true>), dim3(d.H * R), dim3(256), 0, st,
                                  (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, ti, tg, (const bf16_t*)dout,
                                  lse, delta, list, count, dkp, dvp, (bf16_t*)dk, (bf16_t*)dv, read_scale(HD),
                                  d.order, (long)d.B * d.S, d.H, d.L, Lq, d.E,
                                  d.block_size, d.topk, alpha, R, read_bwd_n_ttiles(d)));
}

hipError_t launch_read_bwd_dkdv(const void* q, const void* k, const void* v, const int32_t* top_idx,
                                const float* top_gates, const void* dout, const float* lse, const float* delta,
                                const int32_t* list, const int32_t* count, float* dk_part, float* dv_part, void* dk,
                                void* dv, const ReadDims& d, hipStream_t st) {
  const bool al = d.block_size % 32 == 0;
#define NAYLIS_DKDV2(HDV, TKV)                                                                                 \
  if (al)                                                                                                      \
    dkdv_inst<HDV, true, TKV>(q, k, v, top_idx, top_gates, dout, lse, delta, list, count, dk_part, dv_part, dk, \
                              dv, d, st);                                                                      \
  else                                                                                                         \
    dkdv_inst<HDV, false, TKV>(q, k, v, top_idx, top_gates, dout, lse, delta, list, count, dk_part, dv_part,   \
                               dk, dv, d, st);
#define NAYLIS_DKDV(HDV)        \
  if (d.topk <= 2) {            \
    NAYLIS_DKDV2(HDV, 2)        \
  } else {                      \
    NAYLIS_DKDV2(HDV, kMaxTopK) \
  }
  switch (d.HD) {
    case 16: NAYLIS_DKDV(16) break;
    case 32: NAYLIS_DKDV(32) break;
    case 64: NAYLIS_DKDV(64) break;
    case 128: NAYLIS_DKDV(128) break;
    default: return hipErrorInvalidValue;
  }
#undef NAYLIS_DKDV
#undef NAYLIS_DKDV2
  return hipGetLastError();
}

hipError_t launch_read_bwd_reduce(const float* dk_part, const float* dv_part, const int32_t* count,
                                  const float* dlg_part, const float* top_gates, void* dk, void* dv, float* dgates,
                                  const ReadDims& d, hipStream_t st) {
  const int D = d.H * d.HD;
  const int blocks = d.L < 8192 ? d.L : 8192;  // slot rows
  const long ng = (long)d.B * d.S * d.topk;
  long gb = (ng + 255) / 256;
  if (gb > 8192) gb = 8192;
  NAYLIS_TIMED("read_bwd_reduce", st,
               hipLaunchKernelGGL(read_bwd_reduce_kernel, dim3((int)(blocks + gb)), dim3(256), 0, st, dk_part, dv_part,
                                  count, (bf16_t*)dk, (bf16_t*)dv, d.L, read_lq(d.L) / 128, D, read_bwd_ranges(d),
                                  read_scale(d.HD), blocks, dlg_part, top_gates, dgates, ng, d.H));
  return hipGetLastError();
}

}  // namespace naylis
