// Host-side launchers of the device kernels.  Each returns hipSuccess or the
// launch error; argument validation lives in the C ABI layer (capi.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace naylis {

struct ReadDims {
  int B, S, H, HD, L, E, block_size, topk;
  // Token order of the read's tiles, from launch_read_order: word 0 = 1 when
  // words 1..N map position -> flattened token b*S + s (grouped order), 0 for
  // sequence order, then the pair plan when read_has_pair_plan; nullptr is
  // sequence order.
  const int32_t* order = nullptr;
};

// One-launch kernels whose workgroups take other workgroups' results (the
// router forward) tag them with a per-device launch epoch (pseudo-random
// bits, never 0 in its upper 48) and wait for them at most a process-wide
// number of polls: one_launch_spin_limit(polls) sets it (polls >= 0) and
// returns the previous bound; polls < 0 only reads it.
unsigned long long next_launch_epoch();
int one_launch_spin_limit(int polls);
// true when st is capturing a graph (a replay would reuse the captured epoch,
// so the one-launch kernels are not taken then)
bool stream_capturing(hipStream_t st);

// The read's token order (read_order.hip): tokens grouped by selected blocks
// when that lowers the (tile, block) pairs, else the sequence-order mode word.
size_t read_order_ws_bytes(long N, int E, int topk);
// true when launch_read_order also writes the pair plan (top-2 over at most
// 32 blocks, 1 <= N <= 2^18); the order buffer then has read_order_words words
bool read_has_pair_plan(long N, int E, int topk);
long read_order_words(long N, int E, int topk);
hipError_t launch_read_order(const int32_t* top_idx, long N, int E, int topk, int32_t* order, void* ws,
                             hipStream_t st);

hipError_t launch_read_fwd(const void* q, const void* k, const void* v, const int32_t* top_idx,
                           const float* top_gates, void* out, float* lse, const ReadDims& d, hipStream_t st);

hipError_t launch_read_bwd_dq(const void* q, const void* k, const void* v, const int32_t* top_idx,
                              const float* top_gates, const void* o, const void* dout, const float* lse, void* dq,
                              float* delta, float* dlg_part, uint8_t* tile_flags, const ReadDims& d,
                              hipStream_t st);

hipError_t launch_read_tile_lists(const int32_t* top_idx, uint8_t* tile_flags, int32_t* list, int32_t* count,
                                  const ReadDims& d, hipStream_t st);

hipError_t launch_read_bwd_dkdv(const void* q, const void* k, const void* v, const int32_t* top_idx,
                                const float* top_gates, const void* dout, const float* lse, const float* delta,
                                const int32_t* list, const int32_t* count, float* dk_part, float* dv_part, void* dk,
                                void* dv, const ReadDims& d, hipStream_t st);

hipError_t launch_read_bwd_reduce(const float* dk_part, const float* dv_part, const int32_t* count,
                                  const float* dlg_part, const float* top_gates, void* dk, void* dv, float* dgates,
                                  const ReadDims& d, hipStream_t st);

// Pair-tiled read (read_pair.hip): head_dim 64, block size 128, top-2 over at
// most 32 blocks (backward: 8), with the pair plan in d.order.
bool read_pair_fwd_shapes(const ReadDims& d, long N);  // the shape conditions alone
bool read_pair_bwd_shapes(const ReadDims& d, long N);
bool read_pair_fwd_ok(const ReadDims& d, long N);  // shapes and an order buffer (with its plan)
bool read_pair_bwd_ok(const ReadDims& d, long N);
int read_pair_ranges(const ReadDims& d);
int read_pair_segments(const ReadDims& d);
size_t read_pair_part_bytes(const ReadDims& d);  // one of the dK / dV partial arrays
// bytes of the side buffer the pair forward writes for the pair backward
size_t read_pair_side_bytes(const ReadDims& d);
hipError_t launch_read_fwd_pair(const void* q, const void* k, const void* v, const int32_t* top_idx,
                                const float* top_gates, void* out, void* side, float* lse, const ReadDims& d,
                                hipStream_t st);
hipError_t launch_read_bwd_pair(const void* q, const void* k, const void* v, const int32_t* top_idx,
                                const float* top_gates, const void* o, const void* side, const void* dout,
                                const float* lse, void* dq, void* dk, void* dv, float* dgates, float* dlg_part,
                                float* dk_part, float* dv_part, const ReadDims& d, hipStream_t st);

// Decode step (decode.hip): B sequences, D = H * HD features, router rank R,
// E experts (= bank blocks) of block_size slots, top-k blocks per token.
struct DecodeDims {
  int B, D, H, HD, R, E, block_size, topk;
};
constexpr int kDecodeMaxD = 4096;      // prefix mean held in LDS
constexpr int kDecodeMaxRank = 64;     // router rank
constexpr int kDecodeMaxExperts = 64;  // one wave's lanes rank the experts

// fp8 e4m3 (OCP) bank with one fp32 scale per slot row, from bf16 K / V (L, D)
hipError_t launch_bank_quant_fp8(const void* k, const void* v, uint8_t* k8, uint8_t* v8, float* k_scale,
                                 float* v_scale, int L, int D, hipStream_t st);
hipError_t launch_decode_step(const double* state_in, double* state_out, const int32_t* t_prev, const void* x_new,
                              bool x_f32, const float* w_down, const float* w_up, const void* q_new,
                              const uint8_t* k8, const uint8_t* v8, const float* k_scale, const float* v_scale,
                              void* out, int32_t* top_idx, float* top_gates, const DecodeDims& d, hipStream_t st);

// Fused RMSNorm (rmsnorm.hip): rows of D features, D a multiple of 512 up to
// 4096; x, w, y, dy, dx in one dtype (bf16 or fp32); rstd fp32 per row.
int rmsnorm_bwd_parts(long N);
size_t rmsnorm_ws_bytes(long N, int D);
hipError_t launch_rmsnorm_fwd(const void* x, bool bf16, const void* w, void* y, float* rstd, long N, int D,
                              float eps, hipStream_t st);
// add variant: s = x + T(a) (a bf16 or fp32) written to s_out, then y = norm(s)
hipError_t launch_add_rmsnorm_fwd(const void* x, const void* a, bool a_f32, bool bf16, const void* w, void* s_out,
                                  void* y, float* rstd, long N, int D, float eps, hipStream_t st);
// dres (may be null) is added to dx
hipError_t launch_rmsnorm_bwd(const void* x, bool bf16, const void* w, const float* rstd, const void* dy,
                              const void* dres, void* dx, void* dw, void* ws, long N, int D, hipStream_t st);

// Rotary position embedding of q and k (rope.hip): x (B, S, H, HD) for HD in
// {32, 64, 128}, cos / sin (cos_batch, S, HD) with cos_batch 1 or B; bwd applies
// the transposed rotation to the incoming gradients.
hipError_t launch_rope(const void* q, const void* k, const void* cs, const void* sn, void* qo, void* ko, bool bf16,
                       bool bwd, long B, int S, int H, int HD, int cos_batch, hipStream_t st);

// SwiGLU of the decoder MLP (swiglu.hip): h = silu(g) * u forward; backward
// writes dg and du from dh; n elements, a multiple of 8.
hipError_t launch_swiglu(const void* g, const void* u, const void* dh, void* h_or_dg, void* du, bool bf16, bool bwd,
                         long n, hipStream_t st);

// Cross-entropy of the LM head (xent.hip): bf16 logits (N, V), V a multiple of
// 2048; forward writes per-row loss and log-sum-exp, backward the bf16
// gradient scaled by g[row * g_stride].
hipError_t launch_xent(const void* logits, const int64_t* labels, float* loss, float* lse, const float* g,
                       long g_stride, void* dlogits, bool bwd, long N, int V, long ignore_index, hipStream_t st);

// helpers shared by the workspace planner and the launchers
inline int round_up(int x, int m) { return (x + m - 1) / m * m; }
inline int read_lq(int L) { return round_up(L, 128); }
// the dK/dV pass's ranges per head and fp32 partials (128 slot rows each)
int read_bwd_ranges(const ReadDims& d);
int read_bwd_parts(const ReadDims& d);
int read_bwd_n_ttiles(const ReadDims& d);
// true when launch_read_bwd_dq also writes the dK/dV tile flags (launch_read_tile_lists then skips them)
bool read_dq_writes_tile_flags(const ReadDims& d);

}  // namespace naylis
