// Pieces shared by the read forward and backward kernels: routing decode,
// the per-tile active-group list, bank relayout, launch remap.
#pragma once
#include "common.h"

namespace naylis {

constexpr int kMaxTopK = 8;       // selections per token supported in registers
constexpr int kMaxBlocks = 1024;  // bank blocks (flags live in LDS)
constexpr int kMaxGroups = 512;   // slot groups of 32 over the whole bank (L <= 16384)
constexpr int kMaxSlotGroups = kMaxGroups / 4;  // 128-slot groups (dK/dV work split)
constexpr int kDkdvTile = 64;     // token-order positions per dK/dV tile (tile flags and lists)
constexpr int kReadWaves = 8;     // waves (x 32 tokens) per forward / dQ workgroup

// A token-order buffer (read_order.hip) is 1 + N int32: word 0 is 1 when
// words 1..N hold a grouped order, 0 for sequence order.  order_table()
// returns the table to follow, or nullptr for sequence order (read once per
// kernel: a uniform scalar load), so sequence order costs no loads.
__device__ __forceinline__ const int32_t* order_table(const int32_t* __restrict__ buf) {
  return (buf != nullptr && buf[0] != 0) ? buf + 1 : nullptr;
}

// Token at position `pos` of an order table (nullptr: sequence order).  An
// entry outside [0, N) falls back to `pos`, so a malformed order can produce
// wrong results but never an out-of-bounds access.
__device__ __forceinline__ long order_token(const int32_t* __restrict__ order, long pos, long N) {
  if (order == nullptr) return pos;
  const long t = order[pos];
  return (t >= 0 && t < N) ? t : pos;
}

// Per-token routing held in registers: block ids and log2 of the clamped
// gates, as mom_kernels/reference.py:23 builds them (log(max(g, 1e-9))).
// TK is the compiled maximum of selections per token (>= the runtime topk).
template <int TK>
struct TokenRoute {
  int idx[TK];
  float lg2[TK];
};

template <int TK>
__device__ __forceinline__ void load_route(TokenRoute<TK>& r, const int32_t* __restrict__ top_idx,
                                           const float* __restrict__ top_gates, long tok, bool valid,
                                           int topk) {
#pragma unroll
  for (int t = 0; t < TK; ++t) {
    r.idx[t] = -1;
    r.lg2[t] = 0.f;
    if (t < topk && valid) {
      r.idx[t] = top_idx[tok * topk + t];
      r.lg2[t] = log2f(fmaxf(top_gates[tok * topk + t], 1e-9f));
    }
  }
}

// Bias (log2 domain) a token puts on block e: sum of log-gates over the
// selections equal to e (duplicate ids add, reference.py:26-27); sel=false
// when no selection hits e (the reference's hard mask).
template <int TK>
__device__ __forceinline__ float route_bias(const TokenRoute<TK>& r, int e, int topk, bool& sel) {
  float c = 0.f;
  bool s = false;
#pragma unroll
  for (int t = 0; t < TK; ++t) {
    if (t < topk && r.idx[t] == e) {
      c += r.lg2[t];
      s = true;
    }
  }
  sel = s;
  return c;
}

// Build the compact list of active slot groups (size SG) for a token tile:
// flags[e] != 0 marks blocks some token of the tile selects.  A group is
// active when any block overlapping it is flagged.  Executed by wave 0.
template <int SG>
__device__ __forceinline__ void build_group_list(const uint8_t* flags, int E, int L, int block_size,
                                                 int n_groups, uint16_t* list, int* count) {
  const int lane = threadIdx.x & 63;
  int total = 0;
  for (int base = 0; base < n_groups; base += 64) {
    const int gi = base + lane;
    bool act = false;
    if (gi < n_groups) {
      const int s0 = gi * SG;
      const int s1 = min(s0 + SG, L) - 1;
      const int b0 = s0 / block_size, b1 = s1 / block_size;
      for (int b = b0; b <= b1 && b < E; ++b) act |= flags[b] != 0;
    }
    const unsigned long long m = __ballot(act);
    const int pos = total + __popcll(m & ((1ull << lane) - 1ull));
    if (act) list[pos] = (uint16_t)gi;
    total += __popcll(m);
  }
  if (lane == 0) *count = total;
}

}  // namespace naylis
