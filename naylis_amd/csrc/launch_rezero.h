// Host-side launchers of the ReZero output gate (rezero.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>

namespace naylis {

size_t rezero_ws_bytes(long n);
hipError_t launch_rezero_fwd(const void* z, bool z_bf16, const float* s, float* y, long n, hipStream_t st);
// y = s * z in y's dtype (bf16 or fp32)
hipError_t launch_rezero_scale(const void* z, bool z_bf16, const float* s, void* y, bool y_bf16, long n,
                               hipStream_t st);
// ds = the sum of nparts partials in index order (one workgroup)
hipError_t launch_rezero_reduce(const float* part, int nparts, float* ds, hipStream_t st);
hipError_t launch_rezero_bwd(const void* dy, bool dy_bf16, const void* z, bool z_bf16, const float* s, void* dz,
                             float* ds, void* ws, long n, hipStream_t st);

}  // namespace naylis
