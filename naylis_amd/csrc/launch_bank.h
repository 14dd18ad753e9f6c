// Host-side launchers of the bank K/V projection GEMMs (bank_gemm.hip).
#pragma once
#include <hip/hip_runtime.h>

namespace naylis {

hipError_t launch_bank_kv_fwd(const void* slots, const void* w_k, const void* w_v, void* k_out, void* v_out, int L,
                              int D_in, int D_out, hipStream_t st);

hipError_t launch_bank_kv_bwd(const void* slots, const void* w_k, const void* w_v, const void* dk, const void* dv,
                              void* d_slots, bool slots_f32, void* dw_k, void* dw_v, bool w_f32, int L, int D_in,
                              int D_out, hipStream_t st);

// n layers reading one bank (bank_gemm.hip): one grouped launch per product
bool bank_grouped_ok(int n, int L, int D_in, int D_out);
size_t bank_kv_bwd_grouped_ws_bytes(int n, int L, int D_in);
hipError_t launch_bank_kv_fwd_grouped(const void* slots, const void* const* w_k, const void* const* w_v,
                                      void* const* k_out, void* const* v_out, int n, int L, int D_in, int D_out,
                                      hipStream_t st);
hipError_t launch_bank_kv_bwd_grouped(const void* slots, const void* const* w_k, const void* const* w_v,
                                      const void* const* dk, const void* const* dv, void* d_slots, bool slots_f32,
                                      void* const* dw_k, void* const* dw_v, bool w_f32, void* ws, int n, int L,
                                      int D_in, int D_out, hipStream_t st);

}  // namespace naylis
