// Host-side launchers of the bank K/V projection GEMMs (bank_gemm.hip).
#pragma once
#include <hip/hip_runtime.h>

namespace naylis {

hipError_t launch_bank_kv_fwd(const void* slots, const void* w_k, const void* w_v, void* k_out, void* v_out, int L,
                              int D_in, int D_out, hipStream_t st);

hipError_t launch_bank_kv_bwd(const void* slots, const void* w_k, const void* w_v, const void* dk, const void* dv,
                              void* d_slots, bool slots_f32, void* dw_k, void* dw_v, bool w_f32, int L, int D_in,
                              int D_out, hipStream_t st);

}  // namespace naylis
