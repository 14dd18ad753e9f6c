// Token order for the read.  The bank's K/V rows are shared by every token of
// the batch, so the read may process tokens in any order: grouping tokens by
// the blocks they select makes a tile of consecutive positions touch fewer
// blocks, and the read's work is proportional to the (tile, block) pairs it
// touches.  The reference walks tokens in sequence order with BLOCK_M = 128
// (mom_kernels/triton_gpu.py:50, 98) and skips blocks no token of the tile
// selects; the same skipping applies here to the reordered tiles.
//
//   key(t) = the sorted pair of token t's two selected blocks (top-2 over at
//            most 32 blocks: at most 1024 keys; other routings keep sequence
//            order)
//   sorted = tokens in ascending key order, sequence order within a key
//            (a stable counting sort: the order is a function of top_idx only,
//            so the forward and the backward get the same one)
//   order  = sorted, if it lowers the number of (128-token tile, block) pairs
//            by at least 10 %; otherwise the identity (routing that is already
//            coherent within tiles, e.g. one logit bias per tile).  Calls with
//            more than 2^18 tokens keep the identity.  For block pairs the
//            grouped order's (tile, block) count follows exactly from the key
//            offsets, so the decision needs no pass over the grouped order.
//
// Kernels: (1) per 1024-token chunk, each token's rank among the chunk's
// earlier tokens of the same key, the chunk's key histogram and its tiles'
// sequence-order block counts; (2) per chunk, key offsets (a scan over the
// histograms), the decision, and the placement of the chunk's tokens.  The
// second launch also writes the pair plan (read_common.h): the grouped table
// (always, whatever the decision), the keys with tokens, their 32-token tiles
// and the forward's work items; one extra workgroup writes the lists.
#include "launch.h"
#include "read_common.h"
#include "timing.h"

namespace naylis {

constexpr int kOrdChunk = 1024;  // tokens per chunk of the local ranking (one thread each)
constexpr int kOrdTile = 128;    // tile of the decision (the reference's BLOCK_M)
constexpr int kOrdWaves = kOrdChunk / 64;
constexpr int kOrdMaxE = 32;     // grouping by block pair: E <= 32 (at most 1024 keys), top-2

// Above this many tokens the scatter's scan over all chunks grows too long;
// such calls keep the sequence order.
constexpr long kOrdMaxTokens = 1L << 18;

static bool ord_grouping(long N, int E, int topk) { return topk == 2 && E <= kOrdMaxE && N <= kOrdMaxTokens; }

struct OrderWs {
  size_t keys, rank, hist, seqcnt, total;
};

static OrderWs plan_order_ws(long N, int E) {
  auto a256 = [](size_t x) { return (x + 255) & ~(size_t)255; };
  const long nchunks = (N + kOrdChunk - 1) / kOrdChunk;
  const long ntiles = (N + kOrdTile - 1) / kOrdTile;
  OrderWs w{};
  size_t off = 0;
  w.keys = off;
  off += a256((size_t)N * 2);
  w.rank = off;
  off += a256((size_t)N * 4);
  w.hist = off;
  off += a256((size_t)nchunks * E * E * 4);
  w.seqcnt = off;
  off += a256((size_t)ntiles * 4);
  w.total = off;
  return w;
}

// Key of a top-2 selection (the sorted block pair of the clamped ids) and
// the mask of its valid ids.
__device__ __forceinline__ int pair_key(int a0, int b0, int E, uint32_t& mask) {
  const int a = min(max(a0, 0), E - 1), b = min(max(b0, 0), E - 1);
  mask = 0;
  if (a0 >= 0 && a0 < E) mask |= 1u << a0;
  if (b0 >= 0 && b0 < E) mask |= 1u << b0;
  return a < b ? a * E + b : b * E + a;
}

// Lanes of this wave with this lane's key, below and above this lane: the
// real lanes that agree with it on every key bit (one ballot per bit).
__device__ __forceinline__ void same_key_lanes(bool real, int key, int nkeys, int& before, int& after) {
  const int lane = threadIdx.x & 63;
  const uint64_t below = (1ull << lane) - 1;
  uint64_t m = __ballot(real);
  const int nb = 32 - __clz(max(nkeys - 1, 1));
  for (int bit = 0; bit < nb; ++bit) {
    const bool on = real && ((key >> bit) & 1);
    const uint64_t bm = __ballot(on);
    m &= on ? bm : ~bm;
  }
  before = real ? __popcll(m & below) : 0;
  after = real ? __popcll(m & ~below) - 1 : 0;
}

// (1) per chunk of 1024 tokens: key = sorted block pair, rank among the
// chunk's earlier tokens of the same key (inside a wave the lanes with the
// same key from one ballot per key bit, per-wave key counts across waves),
// the chunk's key histogram, and the distinct-block count of each 128-token
// tile in sequence order.
__global__ __launch_bounds__(kOrdChunk) void order_local_kernel(const int32_t* __restrict__ top_idx,
                                                                uint16_t* __restrict__ keys, int32_t* __restrict__ rank,
                                                                int32_t* __restrict__ hist,
                                                                int32_t* __restrict__ seqcnt, long N, int E) {
  __shared__ int32_t wcnt[kOrdWaves][kOrdMaxE * kOrdMaxE];
  __shared__ uint32_t wmask[kOrdWaves];
  const int nkeys = E * E;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long tok = (long)blockIdx.x * kOrdChunk + tid;
  const bool real = tok < N;
  int key = -1;
  uint32_t mask = 0;
  if (real) key = pair_key(top_idx[tok * 2], top_idx[tok * 2 + 1], E, mask);
  for (int i = tid; i < kOrdWaves * nkeys; i += kOrdChunk) wcnt[i / nkeys][i % nkeys] = 0;
  int before, after;
  same_key_lanes(real, key, nkeys, before, after);
  for (int o = 32; o > 0; o >>= 1) mask |= __shfl_xor(mask, o, 64);
  if (lane == 0) wmask[wave] = mask;
  __syncthreads();
  if (real && after == 0) wcnt[wave][key] = before + 1;  // the last lane of its key in this wave
  if (tid < kOrdChunk / kOrdTile) {                     // a 128-token tile = 2 waves
    const long t = (long)blockIdx.x * (kOrdChunk / kOrdTile) + tid;
    if (t * kOrdTile < N) seqcnt[t] = __popc(wmask[2 * tid] | wmask[2 * tid + 1]);
  }
  __syncthreads();
  if (tid < nkeys) {
    int run = 0;
    for (int w = 0; w < kOrdWaves; ++w) {
      const int c = wcnt[w][tid];
      wcnt[w][tid] = run;
      run += c;
    }
    hist[(long)blockIdx.x * nkeys + tid] = run;
  }
  __syncthreads();
  if (real) {
    keys[tok] = (uint16_t)key;
    rank[tok] = wcnt[wave][key] + before;
  }
}

// Inclusive scans of two values over threads 0..n-1 of the workgroup (n <=
// 1024; threads from n on add 0): a scan inside each wave, then the wave
// totals through LDS (two barriers).  Every thread of the workgroup must call
// it; `tot` gets the two totals.
__device__ __forceinline__ int2 block_scan2(int x, int y, int n, int2* wsum, int2& tot) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = (int)(blockDim.x >> 6);
  int a = tid < n ? x : 0, b = tid < n ? y : 0;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int ua = __shfl_up(a, o, 64), ub = __shfl_up(b, o, 64);
    if (lane >= o) {
      a += ua;
      b += ub;
    }
  }
  if (lane == 63) wsum[wave] = make_int2(a, b);
  __syncthreads();
  int2 add = make_int2(0, 0), t = make_int2(0, 0);
  for (int w = 0; w < nw; ++w) {
    const int2 s = wsum[w];
    if (w < wave) {
      add.x += s.x;
      add.y += s.y;
    }
    t.x += s.x;
    t.y += s.y;
  }
  __syncthreads();  // (wsum free for the next scan)
  tot = t;
  return make_int2(a + add.x, b + add.y);
}

// Largest i in [0, n) with a[i] <= x (a ascending, a[0] <= x).
__device__ __forceinline__ int last_le(const int32_t* a, int n, int x) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a[mid] <= x) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// The pair plan (layout in read_common.h), written by the scatter launch's
// last workgroup from the key totals: thread t holds key t's token count
// `all`, the inclusive scans `end` (of the counts) and `nz` (of "key has
// tokens") at key t, and nnz (keys with tokens).
__device__ void write_pair_plan(int32_t* __restrict__ order, long N, int E, int nkeys, int all, int end, int nz,
                                int nnz, int2* wsum, int32_t* ktile, int32_t* kfit, int32_t* kpos, int32_t* kcnt,
                                int32_t* kab) {
  const PairPlanLayout pl = pair_plan_layout(N, E);
  int32_t* hdr = order + pl.hdr;
  int32_t* kl = order + pl.keys;
  int32_t* tl = order + pl.tiles;
  int32_t* fl = order + pl.fitems;
  const int tid = threadIdx.x;
  const int nt = tid < nkeys ? (all + kPairTile - 1) / kPairTile : 0;
  const int nf = (nt + kPairFwdItem - 1) / kPairFwdItem;
  int2 tot;
  const int2 sc = block_scan2(nt, nf, nkeys, wsum, tot);  // tiles, forward items
  if (tid < nkeys && all > 0) {
    const int k = nz - 1;
    const int a = tid / E, b = tid % E;
    ktile[k] = sc.x - nt;
    kfit[k] = sc.y - nf;
    kpos[k] = end - all;
    kcnt[k] = all;
    kab[k] = a | (b << 5);
    kl[4 * k + 0] = a;
    kl[4 * k + 1] = b;
    kl[4 * k + 2] = sc.x - nt;
    kl[4 * k + 3] = nt;
  }
  __syncthreads();
  const int n_tiles = tot.x, n_fit = tot.y;
  if (tid == 0) {
    hdr[0] = n_tiles;
    hdr[1] = nnz;
    hdr[2] = n_fit;
    for (int i = 3; i < 8; ++i) hdr[i] = 0;
  }
  for (int t = tid; t < n_tiles; t += blockDim.x) {
    const int k = last_le(ktile, nnz, t);
    const int j = t - ktile[k];
    const int cnt = min(kPairTile, kcnt[k] - j * kPairTile);
    const int ab = kab[k];
    tl[2 * t] = kpos[k] + j * kPairTile;
    tl[2 * t + 1] = cnt | ((ab & 31) << 6) | (((ab >> 5) & 31) << 11) | (k << 16);
  }
  constexpr int item_tokens = kPairFwdItem * kPairTile;
  for (int i = tid; i < n_fit; i += blockDim.x) {
    const int k = last_le(kfit, nnz, i);
    const int c = i - kfit[k];
    const int ab = kab[k];
    fl[2 * i] = kpos[k] + c * item_tokens;
    fl[2 * i + 1] = min(item_tokens, kcnt[k] - c * item_tokens) | ((ab & 31) << 16) | (((ab >> 5) & 31) << 21);
  }
}

// (tile, block) pairs of this thread's 128-token tiles in the grouped order:
// the keys with tokens tile [0, N) in ascending order (segment ends cend,
// block pair masks cmask); a tile's blocks are those of the keys whose
// segments overlap it.
__device__ __forceinline__ long grouped_pairs(long N, int nnz, const int32_t* cend, const uint32_t* cmask) {
  const long ntiles = (N + kOrdTile - 1) / kOrdTile;
  long grp = 0;
  for (long t = threadIdx.x; t < ntiles; t += blockDim.x) {
    const long p0 = t * kOrdTile, p1 = min(N, p0 + kOrdTile);
    // from the first key whose segment ends after p0, those that start before p1
    int lo = 0, hi = nnz - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (cend[mid] > p0) hi = mid; else lo = mid + 1;
    }
    uint32_t mask = 0;
    for (int i = lo; i < nnz && (i == 0 ? 0 : cend[i - 1]) < p1; ++i) mask |= cmask[i];
    grp += __popc(mask);
  }
  return grp;
}

// The decision from every thread's sequence-order and grouped-order pair
// counts (summed over the workgroup): grouping is kept when it lowers the
// pairs by at least 10 %.  Every thread of the workgroup must call it.
__device__ __forceinline__ bool keep_grouping(long seq, long grp, long (*red)[kOrdWaves]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = (int)(blockDim.x >> 6);
  for (int o = 32; o > 0; o >>= 1) {
    seq += __shfl_xor(seq, o, 64);
    grp += __shfl_xor(grp, o, 64);
  }
  if (lane == 0) {
    red[0][wave] = seq;
    red[1][wave] = grp;
  }
  __syncthreads();
  long s_all = 0, g_all = 0;
  for (int w = 0; w < nw; ++w) {
    s_all += red[0][w];
    g_all += red[1][w];
  }
  return g_all * 10 <= s_all * 9;
}

// (2) per chunk: key offsets = (tokens of smaller keys) + (tokens of the same
// key in earlier chunks).  Every workgroup also evaluates the decision from
// the same data: in the grouped order a tile's blocks are the union of the
// block pairs of the keys whose segments overlap it, which the offsets give
// exactly.  Grouping is kept when it lowers the (tile, block) pairs by at
// least 10 %: then the mode word order[0] = 1, otherwise 0.  The table
// order[1 + offset + rank] = token is written either way (the pair plan
// indexes it).  One workgroup more than the chunks writes the pair plan, in
// parallel with them.
__global__ __launch_bounds__(kOrdChunk) void order_scatter_kernel(const uint16_t* __restrict__ keys,
                                                                  const int32_t* __restrict__ rank,
                                                                  const int32_t* __restrict__ hist,
                                                                  const int32_t* __restrict__ seqcnt,
                                                                  int32_t* __restrict__ order, long N, int E,
                                                                  int nchunks) {
  __shared__ int32_t off[kOrdMaxE * kOrdMaxE];
  __shared__ int32_t cend[kOrdMaxE * kOrdMaxE];  // the keys with tokens, ascending: segment end
  __shared__ uint32_t cmask[kOrdMaxE * kOrdMaxE];  // and block pair mask
  __shared__ int2 wsum[kOrdWaves];
  __shared__ long red[2][kOrdWaves];
  // pair plan (last workgroup): per key with tokens (ascending) its first
  // tile, first item, first position, token count and blocks
  __shared__ int32_t ktile[kOrdMaxE * kOrdMaxE], kfit[kOrdMaxE * kOrdMaxE], kpos[kOrdMaxE * kOrdMaxE];
  __shared__ int32_t kcnt[kOrdMaxE * kOrdMaxE], kab[kOrdMaxE * kOrdMaxE];
  const int nkeys = E * E;
  const int tid = threadIdx.x;
  const int c = blockIdx.x;
  // this thread's token and the first tile count of the decision, loaded
  // before the scans so their latency is hidden
  const long ntiles = (N + kOrdTile - 1) / kOrdTile;
  const long tok = (long)c * kOrdChunk + tid;
  const bool tok_ok = c < nchunks && tok < N;
  const int my_key = tok_ok ? (int)keys[tok] : 0;
  const int my_rank = tok_ok ? rank[tok] : 0;
  const int seq0 = (c < nchunks && tid < ntiles) ? seqcnt[tid] : 0;
  int before = 0, all = 0;
  if (tid < nkeys) {
    for (int c0 = 0; c0 < nchunks; c0 += 16) {  // 16 independent loads in flight
      int h[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) h[u] = c0 + u < nchunks ? hist[(long)(c0 + u) * nkeys + tid] : 0;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        all += h[u];
        before += (c0 + u < c) ? h[u] : 0;
      }
    }
  }
  // inclusive scans over keys of the totals and of "key has tokens"
  int2 tot;
  const int2 sc = block_scan2(all, all > 0 ? 1 : 0, nkeys, wsum, tot);
  const int nnz = tot.y;
  if (c == nchunks) {
    write_pair_plan(order, N, E, nkeys, all, sc.x, sc.y, nnz, wsum, ktile, kfit, kpos, kcnt, kab);
    return;
  }
  if (tid < nkeys) {
    off[tid] = sc.x - all + before;
    if (all > 0) {
      cend[sc.y - 1] = sc.x;
      cmask[sc.y - 1] = (1u << (tid / E)) | (1u << (tid % E));
    }
  }
  __syncthreads();
  // (tile, block) pairs of both orders
  long seq = 0;
  for (long t = tid; t < ntiles; t += kOrdChunk) seq += t == tid ? seq0 : seqcnt[t];
  const bool grouped = keep_grouping(seq, grouped_pairs(N, nnz, cend, cmask), red);
  if (c == 0 && tid == 0) order[0] = grouped ? 1 : 0;  // the mode word
  if (!tok_ok) return;
  const long dst = (long)off[my_key] + my_rank;
  if (dst >= 0 && dst < N) order[1 + dst] = (int32_t)tok;
}

// sequence order: only the mode word
__global__ __launch_bounds__(64) void order_sequence_kernel(int32_t* __restrict__ order) {
  if (threadIdx.x == 0) order[0] = 0;
}

size_t read_order_ws_bytes(long N, int E, int topk) {
  return ord_grouping(N, E, topk) ? plan_order_ws(N, E).total : 256;
}

bool read_has_pair_plan(long N, int E, int topk) { return N > 0 && ord_grouping(N, E, topk); }

long read_order_words(long N, int E, int topk) {
  return read_has_pair_plan(N, E, topk) ? pair_plan_layout(N, E).words : 1 + N;
}

hipError_t launch_read_order(const int32_t* top_idx, long N, int E, int topk, int32_t* order, void* ws,
                             hipStream_t st) {
  if (N == 0) return hipSuccess;
  if (!ord_grouping(N, E, topk)) {
    NAYLIS_TIMED("read_order", st, hipLaunchKernelGGL(order_sequence_kernel, dim3(1), dim3(64), 0, st, order));
    return hipGetLastError();
  }
  const OrderWs w = plan_order_ws(N, E);
  char* base = (char*)ws;
  uint16_t* keys = (uint16_t*)(base + w.keys);
  int32_t* rank = (int32_t*)(base + w.rank);
  int32_t* hist = (int32_t*)(base + w.hist);
  int32_t* seqcnt = (int32_t*)(base + w.seqcnt);
  const int nchunks = (int)((N + kOrdChunk - 1) / kOrdChunk);
  NAYLIS_TIMED("read_order", st,
               hipLaunchKernelGGL(order_local_kernel, dim3(nchunks), dim3(kOrdChunk), 0, st, top_idx, keys, rank, hist,
                                  seqcnt, N, E));
  NAYLIS_TIMED("read_order", st,
               hipLaunchKernelGGL(order_scatter_kernel, dim3(nchunks + 1), dim3(kOrdChunk), 0, st, keys, rank,
                                  hist, seqcnt, order, N, E, nchunks));
  return hipGetLastError();
}

}  // namespace naylis
