/* naylis_mom.h — C ABI of libnaylis_mom.so, the MI355X (gfx950) Mixture-of-
 * Memory read of OpenRootdev/Naylis.
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers (HIP), tensors are dense row-major with the
 *     shapes given below; bf16 tensors are passed as `const void*`.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream); launches
 *     are asynchronous, nothing synchronises the host.
 *   - Return value: NAYLIS_OK (0) or a NAYLIS_ERR_* code; the message of the
 *     calling thread's last failure is naylis_mom_last_error().
 *   - Scratch memory ("workspace") is owned by the caller; its size comes from
 *     the matching *_workspace_bytes() query.  Workspace contents do not carry
 *     over between calls.
 *   - Notation: N = B*S tokens, D = H*head_dim, L = num_blocks*block_size bank
 *     slots, E = num_blocks, k = top_k, R = router rank.
 */
#ifndef NAYLIS_MOM_H
#define NAYLIS_MOM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NAYLIS_MOM_ABI_VERSION 1

#define NAYLIS_OK 0
#define NAYLIS_ERR_ARG 1       /* invalid shape / argument (the reference raises RuntimeError) */
#define NAYLIS_ERR_WORKSPACE 2 /* workspace smaller than the query returned */
#define NAYLIS_ERR_HIP 3       /* a HIP launch failed */

#define NAYLIS_MAX_TOPK 8
#define NAYLIS_MAX_BLOCKS 1024
#define NAYLIS_MAX_SLOTS 16384

int naylis_mom_abi_version(void);
const char* naylis_mom_last_error(void);

/* ---------------------------------------------------------------- read ---
 * Replaces the Triton read of mom_kernels/triton_gpu.py:412-439
 * (`mom_read(q_sh, k, v, top_idx, top_gates, *, num_blocks, block_size)`),
 * i.e. _MomReadFunction.forward (triton_gpu.py:327-356) and .backward
 * (triton_gpu.py:359-409), with the log-gate transform of triton_gpu.py:435
 * folded in.
 *
 *   q        (B, S, H, head_dim) bf16      the shared query stream
 *   k, v     (L, D) bf16                   shared bank projections
 *   top_idx  (B, S, k) int32               selected bank blocks (ids outside
 *                                          [0, E) select nothing)
 *   top_gates(B, S, k) fp32                router gates; the read adds
 *                                          log(max(g, 1e-9)) on each selected
 *                                          block (duplicate ids add up)
 *   out      (B, S, H, head_dim) bf16
 *   lse      (B, H, S) fp32                log2-domain log-sum-exp per row,
 *                                          saved for the backward
 * Constraints: head_dim a power of two in [16, 128]; 1 <= k <= min(8, E);
 * E <= 1024; L <= 16384.
 */
size_t naylis_mom_read_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t head_dim, int64_t num_blocks,
                                       int64_t block_size, int64_t top_k);

int naylis_mom_read_fwd(const void* q, const void* k, const void* v, const int32_t* top_idx,
                        const float* top_gates, void* out, float* lse, void* workspace, size_t workspace_bytes,
                        int64_t B, int64_t S, int64_t H, int64_t head_dim, int64_t num_blocks, int64_t block_size,
                        int64_t top_k, void* stream);

/* Backward of the read: dq (B,S,H,head_dim) bf16; dk, dv (L, D) bf16 reduced
 * over all N tokens (deterministic, fixed-order); dgates (B,S,k) fp32 =
 * d loss / d top_gates.  `out` and `lse` are the forward's outputs. */
int naylis_mom_read_bwd(const void* q, const void* k, const void* v, const int32_t* top_idx,
                        const float* top_gates, const void* out, const float* lse, const void* dout, void* dq,
                        void* dk, void* dv, float* dgates, void* workspace, size_t workspace_bytes, int64_t B,
                        int64_t S, int64_t H, int64_t head_dim, int64_t num_blocks, int64_t block_size,
                        int64_t top_k, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NAYLIS_MOM_H */
