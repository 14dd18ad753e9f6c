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
#include <stdlib.h>

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
// Wide forward: 4 waves x 64 tokens per workgroup (256 positions of the token
// order), for block sizes that are multiples of 32 and head_dim 32/64/128.
// Each wave owns two 32-token MFMA column tiles (a: tokens 0..31, b: 32..63 of
// its 64), so every K fragment and every V^T fragment read from LDS feeds two
// MFMAs; the bank is streamed through LDS one SG-slot stage (a slice of one
// block) at a time, double-buffered, with one barrier per stage.  Inside a
// stage the wave walks 32-slot chunks and computes S^T of chunk c+1 before
// the softmax of chunk c, so the MFMA pipe has independent work while the
// exp2 / max / convert instructions of the previous chunk issue.  The running
// max follows the same lazy rule as the narrow kernel (moves only by more
// than 8 in log2 units); the per-lane row sums stay lane-local until the
// epilogue, and the one cross-lane step per chunk (max over the two lane
// halves that hold one token column) is a v_permlane32_swap.
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int HD>
struct WideFwdCfg {
  static constexpr int SG = HD >= 128 ? 64 : 128;  // slots per LDS stage
  static constexpr int MINB = HD >= 128 ? 1 : 2;   // workgroups per CU the registers allow
};

template <int HD, int TK>
__global__ __launch_bounds__(256, WideFwdCfg<HD>::MINB) void read_fwd_wide_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const int32_t* __restrict__ top_idx, const float* __restrict__ top_gates, bf16_t* __restrict__ out,
    float* __restrict__ lse, const int32_t* __restrict__ order, long N, int H, int L, int E, int block_size,
    int topk, float alpha, int n_tiles) {
  constexpr int SG = WideFwdCfg<HD>::SG;
  constexpr int NT = 256;
  constexpr int TM = 256;           // positions per workgroup
  constexpr int KS = HD / 16;       // K-steps of Q.K^T
  constexpr int NC = SG / 32;       // 32-slot chunks per stage
  constexpr int NO = HD / 32;       // 32-feature output tiles
  constexpr int PITCH = HD + 8;     // LDS row pitch (bf16): conflict-free 16-byte row reads
  constexpr int TILE = SG * PITCH;
  constexpr int VEC = SG * HD / 8;  // 16-byte vectors per K (or V) stage
  constexpr int PER = VEC / NT;
  static_assert(VEC % NT == 0, "stage copy must tile the workgroup");

  __shared__ __attribute__((aligned(16))) bf16_t k_lds[2 * TILE];
  __shared__ __attribute__((aligned(16))) bf16_t v_lds[2 * TILE];
  __shared__ uint8_t flags[kMaxBlocks];
  __shared__ uint16_t blist[kMaxBlocks];
  __shared__ int n_blk;

  const int G = H * n_tiles;
  const int wid = xcd_remap(blockIdx.x, G);
  const int tile = wid % n_tiles;
  const int h = wid / n_tiles;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int col = lane & 31;
  const long pos_a = (long)tile * TM + wave * 64 + col;
  const long pos_b = pos_a + 32;
  const bool ok_a = pos_a < N, ok_b = pos_b < N;
  const int32_t* ord = order_table(order);
  const long tok_a = ok_a ? order_token(ord, pos_a, N) : 0;
  const long tok_b = ok_b ? order_token(ord, pos_b, N) : 0;
  const int D = H * HD;

  TokenRoute<TK> ra, rb;
  load_route<TK>(ra, top_idx, top_gates, tok_a, ok_a, topk);
  load_route<TK>(rb, top_idx, top_gates, tok_b, ok_b, topk);
  // Q^T fragments (B operand) of both token tiles, issued right after the
  // routing loads (loads retire in issue order, so the routing can be used
  // while these are still in flight across the LDS barriers below)
  bf16x8 qa[KS], qb[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const long col_off = (long)h * HD + 16 * ks + 8 * g;
    qa[ks] = ok_a ? *reinterpret_cast<const bf16x8*>(q + tok_a * D + col_off) : bf16x8{};
    qb[ks] = ok_b ? *reinterpret_cast<const bf16x8*>(q + tok_b * D + col_off) : bf16x8{};
  }

  for (int e = tid; e < E; e += NT) flags[e] = 0;
  lds_barrier();
  {
    const TokenRoute<TK>& r = g == 0 ? ra : rb;
    const bool ok = g == 0 ? ok_a : ok_b;
    if (ok) {
#pragma unroll
      for (int t = 0; t < TK; ++t)
        if (t < topk && r.idx[t] >= 0 && r.idx[t] < E) flags[r.idx[t]] = 1;
    }
  }
  lds_barrier();
  if (wave == 0) {
    int total = 0;
    for (int base = 0; base < E; base += 64) {
      const int e = base + lane;
      const bool act = e < E && flags[e] != 0;
      const unsigned long long m = __ballot(act);
      if (act) blist[total + __popcll(m & ((1ull << lane) - 1ull))] = (uint16_t)e;
      total += __popcll(m);
    }
    if (lane == 0) n_blk = total;
  }


  f32x16 oa[NO], ob[NO];
#pragma unroll
  for (int j = 0; j < NO; ++j) {
    oa[j] = f32x16{};
    ob[j] = f32x16{};
  }
  float ma = kNegBig, mb = kNegBig, la = 0.f, lb = 0.f;  // la/lb: this lane's share of the row sums

  lds_barrier();
  const int spb = block_size / SG > 0 ? block_size / SG : 1;  // stages per block (block_size % SG == 0)
  const int sg_eff = block_size < SG ? block_size : SG;       // slots a stage covers
  const int n_stage = n_blk * spb;

  uint4 kreg[PER], vreg[PER];
  auto load_stage = [&](int s) {
    const int e = blist[s / spb];
    const int s0 = e * block_size + (s % spb) * sg_eff;
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int vi = tid + NT * r;
      const int row = vi / (HD / 8), c8 = vi % (HD / 8);
      uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
      if (row < sg_eff) {
        const long off = (long)(s0 + row) * D + (long)h * HD + 8 * c8;
        kv = *reinterpret_cast<const uint4*>(k + off);
        vv = *reinterpret_cast<const uint4*>(v + off);
      }
      kreg[r] = kv;
      vreg[r] = vv;
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int vi = tid + NT * r;
      const int row = vi / (HD / 8), c8 = vi % (HD / 8);
      *reinterpret_cast<uint4*>(&k_lds[buf * TILE + row * PITCH + 8 * c8]) = kreg[r];
      *reinterpret_cast<uint4*>(&v_lds[buf * TILE + row * PITCH + 8 * c8]) = vreg[r];
    }
  };

  if (n_stage > 0) {
    load_stage(0);
    store_stage(0);
  }
  lds_barrier();

  for (int s = 0; s < n_stage; ++s) {
    const int buf = s & 1;
    if (s + 1 < n_stage) load_stage(s + 1);  // in flight during the math below
    const int e = blist[s / spb];
    bool sa_sel, sb_sel;
    const float ca = route_bias<TK>(ra, e, topk, sa_sel);
    const float cb = route_bias<TK>(rb, e, topk, sb_sel);
    if (__any(sa_sel || sb_sel)) {
      const bf16_t* kt = k_lds + buf * TILE;
      const bf16_t* vt = v_lds + buf * TILE;
      f32x16 sa[2], sb[2];
      auto qk = [&](int c, f32x16& xa, f32x16& xb) {
        xa = f32x16{};
        xb = f32x16{};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(&kt[(32 * c + col) * PITCH + 16 * ks + 8 * g]);
          xa = mfma32(a, qa[ks], xa);
          xb = mfma32(a, qb[ks], xb);
        }
      };
      qk(0, sa[0], sb[0]);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if (32 * c >= sg_eff) break;  // a 32- or 64-slot block fills part of a stage
        f32x16& xa = sa[c & 1];
        f32x16& xb = sb[c & 1];
        if (c + 1 < NC && 32 * (c + 1) < sg_eff) qk(c + 1, sa[(c + 1) & 1], sb[(c + 1) & 1]);

        // ---- online softmax (lazy running max), both token tiles
        float mxa = -INFINITY, mxb = -INFINITY;
#pragma unroll
        for (int vv = 0; vv < 16; ++vv) {
          mxa = fmaxf(mxa, xa[vv]);
          mxb = fmaxf(mxb, xb[vv]);
        }
        mxa = pair_max(mxa);
        mxb = pair_max(mxb);
        float na = ma, nb = mb;
        if (sa_sel) {
          const float cand = fmaf(mxa, alpha, ca);
          if (cand > ma + 8.f) na = cand;
        }
        if (sb_sel) {
          const float cand = fmaf(mxb, alpha, cb);
          if (cand > mb + 8.f) nb = cand;
        }
        const bool mva = na != ma, mvb = nb != mb;
        if (__any((mva && ma != kNegBig) || (mvb && mb != kNegBig))) {
          const float cra = mva ? __builtin_amdgcn_exp2f(ma - na) : 1.f;
          const float crb = mvb ? __builtin_amdgcn_exp2f(mb - nb) : 1.f;
#pragma unroll
          for (int j = 0; j < NO; ++j)
#pragma unroll
            for (int vv = 0; vv < 16; ++vv) {
              oa[j][vv] *= cra;
              ob[j][vv] *= crb;
            }
          la *= cra;
          lb *= crb;
        }
        ma = na;
        mb = nb;
        const float adda = sa_sel ? ca - ma : -INFINITY;
        const float addb = sb_sel ? cb - mb : -INFINITY;
#pragma unroll
        for (int vv = 0; vv < 16; ++vv) {
          const float pa = __builtin_amdgcn_exp2f(fmaf(xa[vv], alpha, adda));
          const float pb = __builtin_amdgcn_exp2f(fmaf(xb[vv], alpha, addb));
          xa[vv] = pa;
          xb[vv] = pb;
          la += pa;
          lb += pb;
        }

        // ---- O^T += V^T P^T for both tiles; each V^T fragment feeds two MFMAs
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const bf16x8 bpa = pack8(xa, 8 * kk);
          const bf16x8 bpb = pack8(xb, 8 * kk);
#pragma unroll
          for (int j = 0; j < NO; ++j) {
            const bf16x8 a = lds_frag_T<true, true>(vt, PITCH, 32 * c + 16 * kk, 32 * j);
            oa[j] = mfma32(a, bpa, oa[j]);
            ob[j] = mfma32(a, bpb, ob[j]);
          }
        }
      }
    }
    if (s + 1 < n_stage) store_stage(buf ^ 1);  // that buffer was last read before the previous barrier
    lds_barrier();
  }

  // ---- epilogue: row sums over both lane halves, normalise, store o and lse
  la = pair_sum(la);
  lb = pair_sum(lb);
  auto store_tok = [&](const f32x16* o, float l, float m, long tok, bool ok) {
    if (!ok) return;
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
    if (g == 0) lse[(long)h * N + tok] = m + log2f(l);
  };
  store_tok(oa, la, ma, tok_a, ok_a);
  store_tok(ob, lb, mb, tok_b, ok_b);
}

template <int HD, int TK>
static void fwd_wide_inst(const void* q, const void* k, const void* v, const int32_t* ti, const float* tg, void* out,
                          float* lse, const ReadDims& d, hipStream_t st) {
  const long N = (long)d.B * d.S;
  const int n_tiles = (int)((N + 255) / 256);
  const float alpha = (float)(1.0 / __builtin_sqrt((double)HD)) * kLog2e;
  NAYLIS_TIMED("read_fwd", st,
               hipLaunchKernelGGL((read_fwd_wide_kernel<HD, TK>), dim3(d.H * n_tiles), dim3(256), 0, st,
                                  (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, ti, tg, (bf16_t*)out, lse,
                                  d.order, N, d.H, d.L, d.E, d.block_size, d.topk, alpha, n_tiles));
}

// The wide kernel covers block sizes that are multiples of 32 whose stage
// slices tile the block (block_size % SG == 0, or block_size < SG dividing it)
// and head_dim 32/64/128.  It is opt-in (NAYLIS_READ_FWD_WIDE=1): on MI355X at
// config 2 the narrow kernel measured faster (47 vs 53 us), its per-workgroup
// latency (route -> Q -> first stage) being spread over more workgroups.
static bool fwd_wide_enabled() {
  static const bool v = [] {
    const char* e = getenv("NAYLIS_READ_FWD_WIDE");
    return e && e[0] == '1';
  }();
  return v;
}

template <int HD>
static bool fwd_wide_fits(const ReadDims& d) {
  constexpr int SG = WideFwdCfg<HD>::SG;
  if (d.block_size % 32 != 0) return false;
  return d.block_size % SG == 0 || SG % d.block_size == 0;
}

// ---------------------------------------------------------------------------
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

// Slot-group size of the forward: NAYLIS_READ_FWD_SG=128 selects 128-slot
// groups instead of the default 64 (read once per process; a tuning knob like
// the reference's NAYLIS_TRITON_BLOCK_N, mom_kernels/triton_gpu.py:48-55).
static int fwd_sg_override() {
  static const int v = [] {
    const char* e = getenv("NAYLIS_READ_FWD_SG");
    return e ? atoi(e) : 0;
  }();
  return v;
}

template <int HD, int TK>
static void fwd_hdk(const void* q, const void* k, const void* v, const int32_t* ti, const float* tg, void* out,
                    float* lse, const ReadDims& d, hipStream_t st) {
  constexpr int SGMAX = 64;  // measured faster than 128 on MI355X (fewer registers, 2 workgroups per CU)
  if (fwd_sg_override() == 128 && HD <= 64 && d.block_size % 128 == 0)
    fwd_inst<HD, (HD <= 64 ? 128 : 64), true, TK>(q, k, v, ti, tg, out, lse, d, st);
  else if (d.block_size % SGMAX == 0)
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
  // wide kernel: head_dim 32/64 and top-k <= 2 fit its registers without spills
  if constexpr (HD == 32 || HD == 64) {
    if (fwd_wide_enabled() && d.topk <= 2 && fwd_wide_fits<HD>(d)) {
      fwd_wide_inst<HD, 2>(q, k, v, ti, tg, out, lse, d, st);
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
