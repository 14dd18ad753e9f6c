// Host-side launchers of the device kernels.  Each returns hipSuccess or the
// launch error; argument validation lives in the C ABI layer (capi.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace naylis {

struct ReadDims {
  int B, S, H, HD, L, E, block_size, topk;
};

hipError_t launch_read_fwd(const void* q, const void* k, const void* v, const int32_t* top_idx,
                           const float* top_gates, void* out, float* lse, const ReadDims& d, hipStream_t st);

hipError_t launch_read_bwd_dq(const void* q, const void* k, const void* v, const int32_t* top_idx,
                              const float* top_gates, const void* o, const void* dout, const float* lse, void* dq,
                              float* delta, float* dlg_part, const ReadDims& d, hipStream_t st);

hipError_t launch_read_tile_lists(const int32_t* top_idx, uint8_t* tile_flags, int32_t* list, int32_t* count,
                                  const ReadDims& d, hipStream_t st);

hipError_t launch_read_bwd_dkdv(const void* q, const void* k, const void* v, const int32_t* top_idx,
                                const float* top_gates, const void* dout, const float* lse, const float* delta,
                                const int32_t* list, const int32_t* count, float* dk_part, float* dv_part,
                                int n_chunks, const ReadDims& d, hipStream_t st);

hipError_t launch_read_bwd_reduce(const float* dk_part, const float* dv_part, const float* dlg_part,
                                  const float* top_gates, void* dk, void* dv, float* dgates, int n_chunks,
                                  const ReadDims& d, hipStream_t st);

// helpers shared by the workspace planner and the launchers
inline int round_up(int x, int m) { return (x + m - 1) / m * m; }
inline int read_lq(int L) { return round_up(L, 128); }
int read_bwd_chunks(const ReadDims& d);
int read_bwd_n_ttiles(const ReadDims& d);

}  // namespace naylis
