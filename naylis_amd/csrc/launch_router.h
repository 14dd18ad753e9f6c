// Host-side launchers of the router kernels (router.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace naylis {

struct RouterDims {
  int B, T, D, R, E, topk;
};

// Byte offsets into the caller's workspace.  The forward uses [0, fwd_total).
struct RouterWs {
  size_t carry, w, wt, scan_csum, dwup_part, dwd_part;
  size_t fwd_total, total;
};

RouterWs plan_router_ws(const RouterDims& d);

hipError_t launch_router_fwd(const void* x, bool x_bf16, const float* w_down, const float* w_up, const float* noise,
                             float noise_scale, float* logits, float* probs, int32_t* top_idx, float* top_gates,
                             float* act, float* h_out, void* ws, const RouterDims& d, hipStream_t st);

hipError_t launch_router_bwd(const void* x, bool x_bf16, const float* w_down, const float* w_up, const float* act,
                             const float* probs, const int32_t* top_idx, const float* top_gates, const float* d_gates,
                             const float* d_probs, const float* d_logits, void* dx, float* dw_down, float* dw_up,
                             void* ws, const RouterDims& d, hipStream_t st);

}  // namespace naylis
