// Gated flash read of the shared MoM bank, forward (gfx950).
//
// Computes, per (b, s, h):  o = softmax_n(q.k_n / sqrt(hd) + bias[b,s,n]) v_n
// with bias = log(gate) summed over the token's selections that hit the
// block of slot n and a hard mask elsewhere (mom_kernels/reference.py:14-61,
// the structured form of mom_kernels/triton_gpu.py:64-141).  The bias is
// never materialised: it is one scalar per (token, bank block), folded into
// the exp2 argument together with the running max.
//
// Work decomposition: one workgroup = (h, 256 consecutive positions of the
// token order), 8 waves, each wave owns 32 tokens (one MFMA column each).
// The order (read_order.hip) groups tokens of the whole batch by the blocks
// they select, so a workgroup's tokens share few blocks.  The workgroup walks the slot groups
// (SG slots) of the bank blocks any of its tokens selects, streaming K and V
// rows through double-buffered LDS (one barrier per group, the next group's
// copy in flight during the math); a wave computes a group only when one of
// its own 32 tokens selects it.  Per group: S^T = K_g Q^T (slots x tokens, K
// from LDS, Q^T resident in registers), online softmax per token column,
// O^T += V_g^T P^T with P^T taken straight from the accumulator registers and
// V^T read from the natural-layout V tile with the transposing LDS read.
#include "launch.h"
#include "read_common.h"
#include "timing.h"

namespace naylis {

template <int HD, int SG, bool ALIGNED, int TK>
__global__ __launch_bounds__(512) void read_fwd_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const int32_t* __restrict__ top_idx, const float* __restrict__ top_gates, bf16_t* __restrict__ out,
    float* __restrict__ lse, const int32_t* __restrict__ order, long N, int H, int L, int E, int block_size,
    int topk, float alpha, int n_tiles) {
  constexpr int NW = kReadWaves;
  constexpr int NT = 64 * NW;
  constexpr int TM = 32 * NW;       // tokens per workgroup
  constexpr int HDP = HD < 32 ? 32 : HD;
  constexpr int KS = HD / 16;       // K-steps over features for Q.K^T
  constexpr int NS = SG / 32;       // 32-slot accumulator tiles per group
  constexpr int NO = HDP / 32;      // 32-feature output tiles
  constexpr int PITCH = HDP + 8;    // LDS row pitch (bf16) of the K and V tiles
  constexpr int TILE = SG * PITCH;

  __shared__ __attribute__((aligned(16))) bf16_t k_lds[2 * TILE];
  __shared__ __attribute__((aligned(16))) bf16_t v_lds[2 * TILE];
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
  const long pos = (long)tile * TM + wave * 32 + col;  // position in the token order
  const bool tok_ok = pos < N;
  const int32_t* ord = order_table(order);
  const long tok = tok_ok ? order_token(ord, pos, N) : 0;  // flattened b*S + s
  const int D = H * HD;

  // ---- routing of this lane's token; active-block flags of the workgroup
  TokenRoute<TK> rt;
  load_route<TK>(rt, top_idx, top_gates, tok, tok_ok, topk);
  // Q^T fragments (B operand): lane holds q[token][16*ks + 8*g .. +8]; issued
  // right after the routing loads (loads retire in issue order, so the
  // routing can be used while these are in flight across the LDS barriers)
  bf16x8 qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if (tok_ok)
      qf[ks] = *reinterpret_cast<const bf16x8*>(q + tok * D + (long)h * HD + 16 * ks + 8 * g);
    else
      qf[ks] = bf16x8{};
  }
  for (int e = tid; e < E; e += NT) flags[e] = 0;
  if constexpr (HD < 32) {
    // feature columns HD..31 of the V tiles stay zero (V^T rows beyond HD)
    for (int i = tid; i < 2 * TILE; i += NT) v_lds[i] = 0;
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

  f32x16 acc_o[NO];
#pragma unroll
  for (int j = 0; j < NO; ++j) acc_o[j] = f32x16{};
  float m_run = kNegBig, l_run = 0.f;

  lds_barrier();
  const int n_act = n_active;

  // staging: K and V rows of a group (SG x HD) as 16-byte vectors
  constexpr int VEC = SG * HD / 8;
  constexpr int PER = (VEC + NT - 1) / NT;
  uint4 kreg[PER], vreg[PER];
  auto load_group = [&](int gi) {
    const int s0 = gi * SG;
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int vi = tid + NT * r;
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
  auto store_group = [&](int buf) {
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int vi = tid + NT * r;
      if (vi < VEC) {
        const int srow = vi / (HD / 8), c8 = vi % (HD / 8);
        *reinterpret_cast<uint4*>(&k_lds[buf * TILE + srow * PITCH + 8 * c8]) = kreg[r];
        *reinterpret_cast<uint4*>(&v_lds[buf * TILE + srow * PITCH + 8 * c8]) = vreg[r];
      }
    }
  };

  if (n_act > 0) {
    load_group(groups[0]);
    store_group(0);
  }
  lds_barrier();

  for (int it = 0; it < n_act; ++it) {
    const int gi = groups[it];
    const int buf = it & 1;
    if (it + 1 < n_act) load_group(groups[it + 1]);  // in flight during the math below
    const bf16_t* kt = k_lds + buf * TILE;
    const bf16_t* vt = v_lds + buf * TILE;

    // does any token of this wave select a block of the group?
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
    if (__any(mine)) {
      // ---- S^T = K_g . Q^T  (SG slots x 32 tokens per wave)
      f32x16 acc_s[NS];
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        acc_s[i] = f32x16{};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(&kt[(32 * i + col) * PITCH + 16 * ks + 8 * g]);
          acc_s[i] = mfma32(a, qf[ks], acc_s[i]);
        }
      }

      // ---- online softmax over this group, per token column
      float m_new = m_run;
      if constexpr (ALIGNED) {
        bool sel;
        const float c2 = route_bias<TK>(rt, (gi * SG) / block_size, topk, sel);
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < NS; ++i)
#pragma unroll
          for (int vv = 0; vv < 16; ++vv) mx = fmaxf(mx, acc_s[i][vv]);
        mx = wave_max_pair(mx);
        // Lazy rescaling: the running max only moves when the group's max
        // exceeds it by more than 8 (log2 units) — p stays <= 2^8, exact in
        // fp32 and in range for bf16 — or on the token's first selected group
        // (its accumulators are still zero then), so O is rarely rescaled.
        if (sel) {
          const float cand = fmaf(mx, alpha, c2);
          if (cand > m_run + 8.f) m_new = cand;
        }
        const float add = sel ? c2 - m_new : -INFINITY;
        float rs = 0.f;
#pragma unroll
        for (int i = 0; i < NS; ++i)
#pragma unroll
          for (int vv = 0; vv < 16; ++vv) {
            const float p = __builtin_amdgcn_exp2f(fmaf(acc_s[i][vv], alpha, add));
            acc_s[i][vv] = p;
            rs += p;
          }
        rs = wave_sum_pair(rs);
        const bool moved = m_new != m_run;
        const float corr = moved ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.f;
        l_run = fmaf(l_run, corr, rs);
        if (__any(moved && m_run != kNegBig)) {
#pragma unroll
          for (int j = 0; j < NO; ++j)
#pragma unroll
            for (int vv = 0; vv < 16; ++vv) acc_o[j][vv] *= corr;
        }
      } else {
        // generic slot->block lookup per element (block_size not a multiple of SG)
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < NS; ++i)
#pragma unroll
          for (int vv = 0; vv < 16; ++vv) {
            const int slot = gi * SG + 32 * i + acc_row(g, vv);
            bool sel = false;
            float c2 = 0.f;
            if (slot < L) c2 = route_bias<TK>(rt, slot / block_size, topk, sel);
            const float t = sel ? fmaf(acc_s[i][vv], alpha, c2) : -INFINITY;
            acc_s[i][vv] = t;
            mx = fmaxf(mx, t);
          }
        mx = wave_max_pair(mx);
        m_new = fmaxf(m_run, mx);
        float rs = 0.f;
#pragma unroll
        for (int i = 0; i < NS; ++i)
#pragma unroll
          for (int vv = 0; vv < 16; ++vv) {
            const float p = __builtin_amdgcn_exp2f(acc_s[i][vv] - m_new);
            acc_s[i][vv] = p;
            rs += p;
          }
        rs = wave_sum_pair(rs);
        const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
        l_run = fmaf(l_run, corr, rs);
#pragma unroll
        for (int j = 0; j < NO; ++j)
#pragma unroll
          for (int vv = 0; vv < 16; ++vv) acc_o[j][vv] *= corr;
      }
      m_run = m_new;

      // ---- O^T += V_g^T . P^T   (P^T fragments come straight from acc_s)
#pragma unroll
      for (int kk = 0; kk < SG / 16; ++kk) {
        const bf16x8 bp = pack8(acc_s[kk >> 1], 8 * (kk & 1));
#pragma unroll
        for (int j = 0; j < NO; ++j) {
          const bf16x8 a = lds_frag_T<true, true>(vt, PITCH, 16 * kk, 32 * j);
          acc_o[j] = mfma32(a, bp, acc_o[j]);
        }
      }
    }
    if (it + 1 < n_act) store_group(buf ^ 1);  // that buffer was last read before the previous barrier
    lds_barrier();
  }

  // ---- epilogue: normalise, store o (bf16) and the log2-domain lse
  if (tok_ok) {
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
#pragma unroll
    for (int j = 0; j < NO; ++j) {
      const int f0 = 32 * j + 16 * g;  // features held by this lane group
      if (f0 < HD) {
        bf16x8 lo, hi;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          lo[e] = (__bf16)(acc_o[j][e] * inv);
          hi[e] = (__bf16)(acc_o[j][8 + e] * inv);
        }
        bf16_t* dst = out + tok * D + (long)h * HD + f0;
        *reinterpret_cast<bf16x8*>(dst) = lo;
        *reinterpret_cast<bf16x8*>(dst + 8) = hi;
      }
    }
    if (g == 0) lse[(long)h * N + tok] = m_run + log2f(l_run);
  }
}

// ---------------------------------------------------------------------------
// Fast forward: head_dim 64, block sizes that are multiples of 32 (every
// Naylis configuration).  One workgroup = (h, 128 consecutive positions of the
// token order), 4 waves x 32 tokens (one MFMA column tile each).
//
// The workgroup's active 32-slot chunks (every chunk of every block one of its
// tokens selects, ascending) pass through LDS in stages of up to 4 chunks (K
// and V of 128 slots: 36 KiB, four workgroups per CU), so a stage costs one
// barrier pair instead of a barrier per slot group; inside a stage each wave
// walks the chunks some token of its 32 selects with no barrier.  (Measured on
// MI355X against 8 waves x 32 tokens with 8-chunk stages: equal at config 2,
// 17 % faster at config 4, whose sequence-order tiles touch fewer blocks at
// 128 tokens than at 256.)
//
// Softmax: a token's reference m is one score of the first chunk it selects
// and afterwards moves only when a chunk gives it some p > 2^64 (p <= 2^64 is
// exact in fp32 and in range for bf16; O and l carry the same scale), so the
// common chunk needs one fma and one exp2 per score, no maximum and no
// rescale of O.  The row sum l adds the bf16 weights that multiply V
// (v_dot2c_f32_bf16), so O / l is a convex combination of V rows exactly as
// the MFMA sees them.
template <int TK>
__global__ __launch_bounds__(256, 4) void read_fwd_fast_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const int32_t* __restrict__ top_idx, const float* __restrict__ top_gates, bf16_t* __restrict__ out,
    float* __restrict__ lse, const int32_t* __restrict__ order, long N, int H, int L, int E, int block_size,
    int topk, float alpha, int n_tiles) {
  constexpr int HD = 64, KS = HD / 16, NO = HD / 32, PITCH = HD + 8;
  constexpr int NW = 4, NT = 64 * NW, TM = 32 * NW;  // 4 waves x 32 tokens
  constexpr int SCH = 4;                     // 32-slot chunks per LDS stage
  constexpr int TILE = SCH * 32 * PITCH;     // bf16 elements of one staged tensor
  constexpr int PER = SCH * 32 * HD / 8 / NT;  // 16-byte pieces per thread per tensor
  static_assert(PER * NT * 8 == SCH * 32 * HD, "stage copy must tile the workgroup");

  __shared__ __attribute__((aligned(16))) bf16_t k_lds[TILE];
  __shared__ __attribute__((aligned(16))) bf16_t v_lds[TILE];
  __shared__ uint8_t flags[kMaxBlocks];
  __shared__ uint32_t chunks[kMaxGroups];  // (block << 16) | chunk index (slot / 32)
  __shared__ int n_chunks_s;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int col = lane & 31;
  const int32_t* ord = order_table(order);
  const int D = H * HD;
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(k, (uint32_t)L * (uint32_t)D * 2u);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(v, (uint32_t)L * (uint32_t)D * 2u);
  {
    const int wid = xcd_remap(blockIdx.x, H * n_tiles);
    const int h = wid / n_tiles;
    const int tile = wid % n_tiles;
    const int hoff = h * HD * 2;  // byte offset of head h in a row

    // ---- this lane's token, routing and q
    const long pos = (long)tile * TM + wave * 32 + col;
    const bool ok = pos < N;
    const long tok = ok ? order_token(ord, pos, N) : 0;
    TokenRoute<TK> rt;
    load_route<TK>(rt, top_idx, top_gates, tok, ok, topk);
    bf16x8 qf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[ks] = ok ? *reinterpret_cast<const bf16x8*>(q + tok * D + (long)h * HD + 16 * ks + 8 * g) : bf16x8{};

    // ---- the item's active chunks, ascending
    for (int e = tid; e < E; e += NT) flags[e] = 0;
    lds_barrier();
    if (g == 0 && ok) {
#pragma unroll
      for (int s = 0; s < TK; ++s)
        if (s < topk && rt.idx[s] >= 0 && rt.idx[s] < E) flags[rt.idx[s]] = 1;
    }
    lds_barrier();
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
    f32x16 o[NO];
#pragma unroll
    for (int j = 0; j < NO; ++j) o[j] = f32x16{};
    float m_run = kNegBig, l_run = 0.f;  // l_run: this lane's share of the row sum
    lds_barrier();
    const int n_ch = n_chunks_s;

    auto qk = [&](int c, f32x16& x) {
      x = f32x16{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(&k_lds[(32 * c + col) * PITCH + 16 * ks + 8 * g]);
        x = mfma32(a, qf[ks], x);
      }
    };
    // VALU phase: softmax of the scores in x into bf16 weights pk.  The
    // reference m_run of a token is set on its first selected chunk from one
    // of the chunk's scores (the larger of the lane pair's first), not from
    // the chunk maximum, which would cost 13 VALU instructions a chunk; it
    // moves only when a chunk gives some p > 2^64, which the chunk's sum of
    // p shows (inf included).  Then the chunk's scores are recomputed from
    // the stage, the reference moves to their maximum (every p <= 1) and o
    // and l_run are rescaled.  Any reference gives the same o and lse up to
    // the bf16 rounding of p.
    auto softmax = [&](int s0, int c, f32x16& x, bf16x8 (&pk)[2]) {
      const int e = (int)(chunks[s0 + c] >> 16);
      bool sl;
      const float cb = route_bias<TK>(rt, e, topk, sl);
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
      // the lane pair holds one token: both move together
      const bool big = !(pair_max(part) <= 0x1p64f);
      if (__any(sl && big)) {
        qk(c, x);
        const float cand = fmaf(pair_max(max16(x)), alpha, cb);
        if (sl && big) {
          const float cr = __builtin_amdgcn_exp2f(m_run - cand);
#pragma unroll
          for (int j = 0; j < NO; ++j)
#pragma unroll
            for (int vv = 0; vv < 16; ++vv) o[j][vv] *= cr;
          l_run *= cr;
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
    // MFMA phase part: O^T += V^T P^T with V^T read transposed from the stage
    auto pv = [&](int c, const bf16x8 (&pk)[2]) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int j = 0; j < NO; ++j) {
          const bf16x8 a = lds_frag_T<true, true>(v_lds, PITCH, 32 * c + 16 * kk, 32 * j);
          o[j] = mfma32(a, pk[kk], o[j]);
        }
    };

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
        for (int s = 0; s < TK; ++s) sel |= s < topk && rt.idx[s] == e;
        if (__any(sel)) mine |= 1u << c;
      }
      lds_barrier();

      // the wave's chunks of the stage, with no barrier in between
      while (mine) {
        const int c = __builtin_ctz(mine);
        mine &= mine - 1;
        f32x16 x;
        bf16x8 pk[2];
        qk(c, x);
        softmax(s0, c, x, pk);
        pv(c, pk);
      }
    }

    // ---- epilogue: row sum over both lane halves, normalise, store o and lse
    const float l = pair_sum(l_run);
    if (ok) {
      const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
      for (int j = 0; j < NO; ++j) {
        const int f0 = 32 * j + 16 * g;
        bf16x8 lo, hi;
#pragma unroll
        for (int e2 = 0; e2 < 8; ++e2) {
          lo[e2] = (__bf16)(o[j][e2] * inv);
          hi[e2] = (__bf16)(o[j][8 + e2] * inv);
        }
        bf16_t* dst = out + tok * D + (long)h * HD + f0;
        *reinterpret_cast<bf16x8*>(dst) = lo;
        *reinterpret_cast<bf16x8*>(dst + 8) = hi;
      }
      if (g == 0) lse[(long)h * N + tok] = m_run + log2f(l);
    }
  }
}

// The fast kernel covers head_dim 64 with block sizes that are multiples of 32.
static bool fwd_fast_fits(const ReadDims& d) { return d.HD == 64 && d.block_size % 32 == 0; }

template <int TK>
static void fwd_fast_inst(const void* q, const void* k, const void* v, const int32_t* ti, const float* tg, void* out,
                          float* lse, const ReadDims& d, hipStream_t st) {
  const long N = (long)d.B * d.S;
  const int n_tiles = (int)((N + 127) / 128);
  const float alpha = (float)(1.0 / __builtin_sqrt(64.0)) * kLog2e;
  NAYLIS_TIMED("read_fwd", st,
               hipLaunchKernelGGL((read_fwd_fast_kernel<TK>), dim3(d.H * n_tiles), dim3(256), 0, st,
                                  (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, ti, tg, (bf16_t*)out, lse,
                                  d.order, N, d.H, d.L, d.E, d.block_size, d.topk, alpha, n_tiles));
}

template <int HD, int SG, bool AL, int TK>
static void fwd_inst(const void* q, const void* k, const void* v, const int32_t* ti, const float* tg, void* out,
                     float* lse, const ReadDims& d, hipStream_t st) {
  const long N = (long)d.B * d.S;
  const int n_tiles = (int)((N + 32 * kReadWaves - 1) / (32 * kReadWaves));
  const float alpha = (float)(1.0 / __builtin_sqrt((double)HD)) * kLog2e;
  NAYLIS_TIMED("read_fwd", st,
               hipLaunchKernelGGL((read_fwd_kernel<HD, SG, AL, TK>), dim3(d.H * n_tiles), dim3(64 * kReadWaves), 0, st,
                                  (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, ti, tg, (bf16_t*)out, lse,
                                  d.order, N, d.H, d.L, d.E, d.block_size, d.topk, alpha, n_tiles));
}

template <int HD, int TK>
static void fwd_hdk(const void* q, const void* k, const void* v, const int32_t* ti, const float* tg, void* out,
                    float* lse, const ReadDims& d, hipStream_t st) {
  constexpr int SGMAX = 64;  // measured faster than 128 on MI355X (fewer registers, 2 workgroups per CU)
  if (d.block_size % SGMAX == 0)
    fwd_inst<HD, SGMAX, true, TK>(q, k, v, ti, tg, out, lse, d, st);
  else if (d.block_size % 64 == 0)
    fwd_inst<HD, 64, true, TK>(q, k, v, ti, tg, out, lse, d, st);
  else if (d.block_size % 32 == 0)
    fwd_inst<HD, 32, true, TK>(q, k, v, ti, tg, out, lse, d, st);
  else
    fwd_inst<HD, 32, false, TK>(q, k, v, ti, tg, out, lse, d, st);
}

template <int HD>
static void fwd_hd(const void* q, const void* k, const void* v, const int32_t* ti, const float* tg, void* out,
                   float* lse, const ReadDims& d, hipStream_t st) {
  if constexpr (HD == 64) {
    if (fwd_fast_fits(d)) {
      if (d.topk <= 2)
        fwd_fast_inst<2>(q, k, v, ti, tg, out, lse, d, st);
      else
        fwd_fast_inst<kMaxTopK>(q, k, v, ti, tg, out, lse, d, st);
      return;
    }
  }
  if (d.topk <= 2)
    fwd_hdk<HD, 2>(q, k, v, ti, tg, out, lse, d, st);
  else
    fwd_hdk<HD, kMaxTopK>(q, k, v, ti, tg, out, lse, d, st);
}

hipError_t launch_read_fwd(const void* q, const void* k, const void* v, const int32_t* top_idx,
                           const float* top_gates, void* out, float* lse, const ReadDims& d, hipStream_t st) {
  switch (d.HD) {
    case 16: fwd_hd<16>(q, k, v, top_idx, top_gates, out, lse, d, st); break;
    case 32: fwd_hd<32>(q, k, v, top_idx, top_gates, out, lse, d, st); break;
    case 64: fwd_hd<64>(q, k, v, top_idx, top_gates, out, lse, d, st); break;
    case 128: fwd_hd<128>(q, k, v, top_idx, top_gates, out, lse, d, st); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace naylis
