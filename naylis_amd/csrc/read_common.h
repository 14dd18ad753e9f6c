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

// ---------------------------------------------------------------------------
// Pair plan: for top-2 routing over at most 32 blocks the order buffer also
// carries, after the order table, the work list of the pair-tiled read
// kernels (read_pair.hip).  Tokens are grouped by their sorted block pair
// ("key"); each key's run of the order is cut into tiles of kPairTile
// consecutive positions, so every token of a tile selects the same one or
// two blocks.  The table is written whenever the plan is (whatever the mode
// word says), so the pair kernels always follow the grouped order.
//   hdr    [8]           n_tiles, n_keys, n_fitems, 0...
//   keys   [max_keys][4] block a, block b (a <= b), first tile, tiles
//   tiles  [max_tiles][2] first position, count | a << 6 | b << 11 | key << 16
//   fitems [max_tiles][2] forward work items (up to kPairFwdItem consecutive
//                         tiles of one key, one per forward wave): first
//                         position, tokens | a << 16 | b << 21
constexpr int kPairTile = 32;
constexpr int kPairFwdItem = 4;
constexpr int kPairMaxE = 32;      // pair plan and pair-tiled forward
constexpr int kPairBwdMaxE = 8;    // pair-tiled backward: its dK / dV partials grow with the pairs
constexpr int kPairBwdMaxRange = 256;  // tiles per backward range (their plan words sit in LDS)
constexpr int kPairFwdMaxRange = 256;  // work items per forward range (likewise)

struct PairPlanLayout {
  long hdr, keys, tiles, fitems, words;
  int max_keys, max_tiles;
};

__host__ __device__ inline PairPlanLayout pair_plan_layout(long N, int E) {
  PairPlanLayout p;
  const long all_keys = (long)E * (E + 1) / 2;
  const long mk = all_keys < N ? all_keys : N;
  p.max_keys = (int)mk;
  p.max_tiles = (int)((N + kPairTile - 1) / kPairTile + mk);
  long off = (1 + N + 3) & ~3L;
  p.hdr = off;
  off += 8;
  p.keys = off;
  off += 4 * mk;
  p.tiles = off;
  off += 2L * p.max_tiles;
  p.fitems = off;
  off += 2L * p.max_tiles;
  p.words = off;
  return p;
}

__device__ __forceinline__ int pair_tile_count(int w1) { return w1 & 63; }
__device__ __forceinline__ int pair_tile_a(int w1) { return (w1 >> 6) & 31; }
__device__ __forceinline__ int pair_tile_b(int w1) { return (w1 >> 11) & 31; }
__device__ __forceinline__ int pair_tile_key(int w1) { return (int)((unsigned)w1 >> 16); }
__device__ __forceinline__ int pair_item_tokens(int w1) { return w1 & 0xffff; }
__device__ __forceinline__ int pair_item_a(int w1) { return (w1 >> 16) & 31; }
__device__ __forceinline__ int pair_item_b(int w1) { return (w1 >> 21) & 31; }

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

// Lane-pair (l, l ^ 32) combinations, the 16-register maximum and the bf16
// row sum of the read kernels' softmax.
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max16(const f32x16& x) {
  float m = fmaxf(fmaxf(x[0], x[1]), x[2]);
#pragma unroll
  for (int v = 3; v < 15; v += 2) m = fmaxf(fmaxf(m, x[v]), x[v + 1]);
  return fmaxf(m, x[15]);
}
// Sum of 8 bf16 values into an fp32 accumulator (v_dot2c_f32_bf16 against 1.0).
__device__ __forceinline__ float add_bf16x8(const bf16x8& p, float acc) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  const uint4 u = __builtin_bit_cast(uint4, p);
  float s0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u.x), one, acc, false);
  float s1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u.y), one, 0.f, false);
  s0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u.z), one, s0, false);
  s1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u.w), one, s1, false);
  return s0 + s1;
}

}  // namespace naylis
