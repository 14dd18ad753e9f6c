// Host-side launchers of the router kernels (router.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace naylis {

struct RouterDims {
  int B, T, D, R, E, topk;
  int noise_kind = 0;   // 0: additive noise as given; 1: uniform draw, Gumbel-transformed in the kernel
  long dp_stride = 0;   // d_probs row stride: E (one row per token) or 0 (one row for all tokens)
};

// Byte offsets into the caller's workspace.  The forward uses [0, fwd_total).
struct RouterWs {
  size_t carry, y, ycs, pub, w, wt, scan_csum, dwup_part, dwd_part;
  size_t fwd_total, total;
};

RouterWs plan_router_ws(const RouterDims& d);

hipError_t launch_router_fwd(const void* x, bool x_bf16, const float* w_down, const float* w_up, const float* noise,
                             float noise_scale, float* logits, float* probs, int32_t* top_idx, float* top_gates,
                             float* act, float* h_out, void* ws, const RouterDims& d, hipStream_t st);

// dx_accumulate: dx += the router's input gradient (one rounding of the fp32
// sum) instead of dx = it.
hipError_t launch_router_bwd(const void* x, bool x_bf16, const float* w_down, const float* w_up, const float* act,
                             const float* probs, const int32_t* top_idx, const float* top_gates, const float* d_gates,
                             const float* d_probs, const float* d_logits, void* dx, bool dx_accumulate,
                             float* dw_down, float* dw_up, void* ws, const RouterDims& d, hipStream_t st);

// Fast path (router_fast.hip): bf16 x, projection before the prefix scan.
bool router_fast_fwd_ok(const void* x, bool x_bf16, const float* w_down, const float* h_out, const RouterDims& d);
bool router_fast_bwd_ok(const void* x, bool x_bf16, const void* dx, const RouterDims& d);
void launch_router_fast_fwd(const void* x, const float* w_down, const float* w_up, const float* noise,
                            float noise_scale, float* logits, float* probs, int32_t* top_idx, float* top_gates,
                            float* act, float* y, double* ycs, unsigned long long* pub, const RouterDims& d,
                            hipStream_t st);
// fast backward (B1 + B2): w, its 32-token chunk sums, W~ (skipped when
// fuse_scan: the dx kernel then forms it) and the dW_up partials; returns the
// number of dW_up partials
int launch_router_fast_scan(const float* act, const float* probs, const int32_t* idx, const float* gates,
                            const float* dg, const float* dp, const float* dl, const float* w_up, float* w,
                            double* wcs, float* wt, float* dwup_part, bool fuse_scan, const RouterDims& d,
                            hipStream_t st);
// Load-balance statistics of a routing (router_stats.hip): stats[2E + 3].
size_t router_stats_ws_bytes(long N, int E);
hipError_t launch_router_stats(const float* probs, const int32_t* top_idx, float* stats, void* ws, long N, int E,
                               int topk, hipStream_t st);
// true when the dx kernel can form W~ from w and its chunk sums itself (R <=
// 32, T a multiple of its 256-token range, one round of workgroups).  The
// caller decides once per backward and passes the same flag to
// launch_router_fast_scan (which then skips B2) and launch_router_fast_dx.
bool router_fast_dx_fuses_scan(const RouterDims& d);
void launch_router_fast_dx(const void* x, const float* wt, const float* w, const double* wcs, const float* w_down,
                           const void* dx_in, void* dx, float* dwd_part, bool fuse_scan, const RouterDims& d,
                           hipStream_t st);

}  // namespace naylis
