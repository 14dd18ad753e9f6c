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

#define NAYLIS_MOM_ABI_VERSION 17

#define NAYLIS_OK 0
#define NAYLIS_ERR_ARG 1       /* invalid shape / argument (the reference raises RuntimeError) */
#define NAYLIS_ERR_WORKSPACE 2 /* workspace smaller than the query returned */
#define NAYLIS_ERR_HIP 3       /* a HIP launch failed */

#define NAYLIS_DTYPE_F32 0
#define NAYLIS_DTYPE_BF16 1

/* noise_kind of naylis_mom_router_fwd */
#define NAYLIS_NOISE_ADDITIVE 0        /* noise holds the perturbation itself */
#define NAYLIS_NOISE_GUMBEL_UNIFORM 1  /* noise holds the uniform draw u; the kernel applies
                                          g = -log(-log(u + 1e-9) + 1e-9) (model.py:210) */

#define NAYLIS_MAX_TOPK 8
#define NAYLIS_MAX_BLOCKS 1024
#define NAYLIS_MAX_SLOTS 16384
#define NAYLIS_ROUTER_MAX_RANK 64
#define NAYLIS_ROUTER_MAX_BLOCKS 64

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
 *   side     naylis_mom_read_side_bytes() bytes, or NULL: what the
 *                                          pair-tiled forward leaves for the
 *                                          pair-tiled backward, (H, B, S, 4)
 *                                          32-bit words per row: its log2
 *                                          bias minus lse on the pair's first
 *                                          and second block (-inf: not
 *                                          selected), its share of the row
 *                                          weight on the first block, and
 *                                          which selections hit which block
 *                                          (bits 0-1: first, 2-3: second).  Used
 *                                          when side_bytes > 0 and a
 *                                          token_order is given; with NULL the
 *                                          backward takes the two-pass
 *                                          kernels.  Ignored otherwise.
 *   lse      (H, B, S) fp32                log2-domain log-sum-exp per row,
 *                                          saved for the backward
 *   token_order  int32 or NULL             the order in which the read walks
 *                                          the flattened tokens b*S + s, as
 *                                          written by naylis_mom_read_order
 *                                          into naylis_mom_read_order_words()
 *                                          words: word 0 = 1 when words
 *                                          1..B*S hold a grouped order, 0 for
 *                                          sequence order, then (top-2 over
 *                                          at most 32 blocks) the pair plan of
 *                                          the pair-tiled kernels; NULL is
 *                                          sequence order.  Results do not
 *                                          depend on it beyond fp32 rounding
 *                                          of the dK/dV sums; the backward
 *                                          must get the forward's order.
 * Constraints: head_dim a power of two in [16, 128]; 1 <= k <= min(8, E);
 * E <= 1024; L <= 16384.  The forward needs no workspace (pass NULL, 0); the
 * backward needs naylis_mom_read_workspace_bytes() bytes.
 */
size_t naylis_mom_read_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t head_dim, int64_t num_blocks,
                                       int64_t block_size, int64_t top_k);

/* Bytes of the side buffer when, given a token_order from
 * naylis_mom_read_order and that buffer, the read takes the pair-tiled path
 * both ways (head_dim 64, block size 128, top-2, num_blocks <= 8,
 * 1 <= B*S <= 2^18; the forward alone also for num_blocks <= 32); 0
 * otherwise (no side buffer needed). */
size_t naylis_mom_read_side_bytes(int64_t B, int64_t S, int64_t H, int64_t head_dim, int64_t num_blocks,
                                  int64_t block_size, int64_t top_k);

int naylis_mom_read_fwd(const void* q, const void* k, const void* v, const int32_t* top_idx,
                        const float* top_gates, const int32_t* token_order, void* out, void* side, float* lse,
                        void* workspace, size_t workspace_bytes, int64_t B, int64_t S, int64_t H, int64_t head_dim,
                        int64_t num_blocks, int64_t block_size, int64_t top_k, void* stream);

/* Backward of the read: dq (B,S,H,head_dim) bf16; dk, dv (L, D) bf16 reduced
 * over all N tokens (deterministic, fixed-order); dgates (B,S,k) fp32 =
 * d loss / d top_gates.  `out`, `side` and `lse` are the forward's
 * outputs (side may be NULL, see above). */
int naylis_mom_read_bwd(const void* q, const void* k, const void* v, const int32_t* top_idx,
                        const float* top_gates, const int32_t* token_order, const void* out, const void* side,
                        const float* lse, const void* dout, void* dq, void* dk, void* dv, float* dgates,
                        void* workspace, size_t workspace_bytes, int64_t B, int64_t S, int64_t H, int64_t head_dim,
                        int64_t num_blocks, int64_t block_size, int64_t top_k, void* stream);

/* The read backward with no workspace argument: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, tight training or serving loops, harnesses that forbid
 * hipMalloc); it allocates nothing.  Same arguments (less the workspace),
 * results (bitwise) and errors as naylis_mom_read_bwd.  Its workspace is a
 * scratch array of NAYLIS_READ_BWD_NOALLOC_MAX_BYTES (128 MiB) in the
 * library's code object: every device the library is loaded on reserves it
 * from the load until the process ends, whether or not this entry point is
 * ever called.  A read whose naylis_mom_read_workspace_bytes() exceeds it
 * returns NAYLIS_ERR_WORKSPACE.  `stream` must belong to the current device
 * (the array's address is looked up there); otherwise NAYLIS_ERR_ARG.  All
 * calls on one device share that array and its contents: calls that overlap
 * on one GPU (on other streams or threads) race, and the caller must order
 * them. */
#define NAYLIS_READ_BWD_NOALLOC_MAX_BYTES ((size_t)128 << 20)
int naylis_mom_read_bwd_noalloc(const void* q, const void* k, const void* v, const int32_t* top_idx,
                                const float* top_gates, const int32_t* token_order, const void* out,
                                const void* side, const float* lse, const void* dout, void* dq, void* dk, void* dv,
                                float* dgates, int64_t B, int64_t S, int64_t H, int64_t head_dim,
                                int64_t num_blocks, int64_t block_size, int64_t top_k, void* stream);

/* Token order for the read (no counterpart in the reference, which walks
 * tokens in sequence order with BLOCK_M = 128, triton_gpu.py:50,98): the
 * bank's K/V are shared by the whole batch, so tokens may be read in any
 * order.  order: naylis_mom_read_order_words() int32 (1 + B*S, plus the pair
 * plan when there is one).  For top-2 routing over at most 32 blocks and at
 * most 2^18 tokens, words 1..B*S receive the flattened tokens grouped by
 * their block pair (stable within a pair), and the words after them the pair
 * plan (the pair-tiled kernels' 32-token tiles and work items); word 0 = 1
 * when the grouping lowers the number of (128-token tile, block) pairs by at
 * least 10 % (the two-pass kernels then follow it), else 0.  Every other
 * routing: word 0 = 0 (sequence order) and nothing else.  A function of
 * top_idx only.  Workspace: naylis_mom_read_order_workspace_bytes(). */
int64_t naylis_mom_read_order_words(int64_t B, int64_t S, int64_t num_blocks, int64_t top_k);
size_t naylis_mom_read_order_workspace_bytes(int64_t B, int64_t S, int64_t num_blocks, int64_t top_k);
int naylis_mom_read_order(const int32_t* top_idx, int32_t* order, void* workspace, size_t workspace_bytes, int64_t B,
                          int64_t S, int64_t num_blocks, int64_t top_k, void* stream);

/* -------------------------------------------------------------- router ---
 * The causal prefix-mean router of MoMLayer, which the reference runs as
 * eager torch ops with no kernel boundary: model.py:169-187
 * (_prefix_mean, _router_logits) and model.py:209-220 (noise, softmax probs,
 * topk, gates); mirror in mom_kernels/reference.py:32-36,75-84.
 *
 *   x          (B, T, D) fp32 or bf16 (x_dtype: NAYLIS_DTYPE_*)
 *   w_down     (R, D) fp32          router_down.weight
 *   w_up       (E, R) fp32          router_up.weight
 *   noise      (B, T, E) fp32 or NULL; topk ranks logits + noise_scale*g with
 *              g = noise (noise_kind NAYLIS_NOISE_ADDITIVE: any logit bias) or
 *              g = -log(-log(noise + 1e-9) + 1e-9) (NAYLIS_NOISE_GUMBEL_UNIFORM:
 *              noise is the torch.rand draw of model.py:210, transformed in the
 *              kernel with the reference's fp32 steps); product and sum are
 *              rounded separately, as the reference's two ops
 *   logits     (B, T, E) fp32       clean router logits
 *   probs      (B, T, E) fp32       softmax(logits)
 *   top_idx    (B, T, k) int32      descending by perturbed logit; ties ->
 *                                   lowest block id
 *   top_gates  (B, T, k) fp32       softmax of the selected perturbed logits
 *   act        (B, T, R) fp32       tanh activations, saved for the backward
 *   h_out      (B, T, D) fp32 or NULL: the prefix mean h_t (bit-exact with
 *              the reference's fp32 cumsum / (t+1))
 * Constraints: R <= 64, E <= 64, 1 <= k <= min(8, E).
 */
size_t naylis_mom_router_workspace_bytes(int64_t B, int64_t T, int64_t D, int64_t R, int64_t E, int64_t top_k);

int naylis_mom_router_fwd(const void* x, int x_dtype, const float* w_down, const float* w_up, const float* noise,
                          int noise_kind, float noise_scale, float* logits, float* probs, int32_t* top_idx,
                          float* top_gates, float* act, float* h_out, void* workspace, size_t workspace_bytes,
                          int64_t B, int64_t T, int64_t D, int64_t R, int64_t E, int64_t top_k, void* stream);

/* No counterpart in the reference; for tests and for callers that want to
 * bound the cross-workgroup wait of the library's one-launch kernel: with
 * bf16 x, R <= 32 and an even number of 32-token chunks, naylis_mom_router_fwd
 * runs in one launch whose workgroups read the earlier chunks' projection
 * sums from the workgroups that made them, polling at most `polls` times per
 * block of chunks, and project the chunks still missing themselves (same
 * results, bitwise).  Not taken on a stream that is capturing a graph (the
 * two launches run there).  Sets the process-wide bound to polls (0: never
 * wait, always re-project) and returns the previous one; polls < 0 only
 * returns the current bound (default 20000).  Launches already enqueued keep
 * the bound they took. */
int naylis_mom_spin_limit(int polls);

/* Backward of the router: any of d_gates (B,T,k), d_probs, d_logits
 * (B,T,E) may be NULL (no gradient from that output).  d_probs_stride is the
 * distance between tokens' rows of d_probs: E for a (B,T,E) tensor, or 0 for
 * one row of E values shared by every token (the gradient the load-balance
 * aux term sends through mean_prob, without an (N, E) tensor).  Writes dx (same dtype
 * and shape as x), dw_down (R, D) and dw_up (E, R), both fp32, reduced over
 * all tokens in a fixed order.  dx_accumulate != 0 adds the router's input
 * gradient to the dx the caller passes (the sum of x's gradients from the
 * router and from the query projection that autograd would form, with one
 * bf16 rounding of the fp32 sum); it needs bf16 x, D a multiple of 128,
 * R <= 64 and 16-byte aligned x / dx (NAYLIS_ERR_ARG otherwise).
 *
 * For bf16 x with D % 128 == 0 (D <= 2048) and no h_out, the forward projects x first
 * (y = x W_down^T, W_down split exactly into three bf16 planes on the bf16
 * MFMA) and scans the R-wide y in fp64: the linear-algebra identity
 * cumsum(x) W^T = cumsum(x W^T) of model.py:169-187, with fp32-GEMM accuracy
 * and indices equal outside near-ties; with h_out (or fp32 x) it scans x
 * itself and h_out is bit-exact. */
int naylis_mom_router_bwd(const void* x, int x_dtype, const float* w_down, const float* w_up, const float* act,
                          const float* probs, const int32_t* top_idx, const float* top_gates, const float* d_gates,
                          const float* d_probs, int64_t d_probs_stride, const float* d_logits, void* dx,
                          int dx_accumulate, float* dw_down, float* dw_up, void* workspace, size_t workspace_bytes,
                          int64_t B, int64_t T, int64_t D, int64_t R, int64_t E, int64_t top_k, void* stream);

/* Load-balance statistics of one layer's routing, replacing the per-layer
 * torch ops of model.py:476-517 (_collect_mom_aux_loss) with one pass over
 * probs (N, E) fp32 and top_idx (N, k) int32:
 *   stats[0, E)   mean_prob_e = mean over tokens of probs[:, e]
 *   stats[E, 2E)  frac_e      = fraction of tokens whose top-k contains e
 *   stats[2E]     aux         = E * sum_e frac_e * mean_prob_e
 *   stats[2E+1]   entropy     = mean over tokens of -sum_e p log(max(p, 1e-9))
 *   stats[2E+2]   dead        = fraction of blocks no token selects
 * (2E+3 floats).  Sums run in fp64 in a fixed order (deterministic).  The aux
 * gradient with respect to probs is one row, d_aux * E * frac_e / N, for
 * naylis_mom_router_bwd with d_probs_stride = 0. */
size_t naylis_mom_router_stats_workspace_bytes(int64_t N, int64_t E);
int naylis_mom_router_stats(const float* probs, const int32_t* top_idx, float* stats, void* workspace,
                            size_t workspace_bytes, int64_t N, int64_t E, int64_t top_k, void* stream);

/* ------------------------------------------------------------- RMSNorm ---
 * The decoder's RMSNorm, fused: model.py:304-305 builds mom_norm (the MoM
 * layer's pre-norm) and the Llama block's norms as LlamaRMSNorm (or Liger's
 * fused RMSNorm with use_liger):
 *   h = fp32(x) * rsqrt(mean(fp32(x)^2) + eps);  y = weight * h.to(dtype)
 * x, weight, y, dy, dx share one dtype (NAYLIS_DTYPE_*); x (N, D) row-major,
 * weight (D,), rstd (N,) fp32 written by the forward for the backward.
 * D a multiple of 512 in [512, 4096]; x / weight / y / dy / dx 16-byte aligned.
 * The backward writes dx and dweight (summed over rows in a fixed order). */
int naylis_mom_rmsnorm_fwd(const void* x, int dtype, const void* weight, void* y, float* rstd, int64_t N, int64_t D,
                           float eps, void* stream);
size_t naylis_mom_rmsnorm_workspace_bytes(int64_t N, int64_t D);
int naylis_mom_rmsnorm_bwd(const void* x, int dtype, const void* weight, const float* rstd, const void* dy, void* dx,
                           void* dweight, void* workspace, size_t workspace_bytes, int64_t N, int64_t D,
                           void* stream);
/* The residual add that precedes every norm of the decoder block, fused:
 * s = x + dtype(a) (a in the stream's dtype or fp32 — the ReZero output is
 * fp32) is written to s_out and y = RMSNorm(s).  The backward takes the
 * gradient arriving at s from the residual stream (dres, may be NULL) and
 * writes ds = dres + the norm's input gradient (one rounding), which is the
 * gradient of both x and a. */
int naylis_mom_add_rmsnorm_fwd(const void* x, const void* a, int a_dtype, const void* weight, void* s_out, void* y,
                               float* rstd, int dtype, int64_t N, int64_t D, float eps, void* stream);
int naylis_mom_add_rmsnorm_bwd(const void* s, const void* weight, const float* rstd, const void* dy, const void* dres,
                               void* ds, void* dweight, void* workspace, size_t workspace_bytes, int dtype, int64_t N,
                               int64_t D, void* stream);

/* ---------------------------------------------------------------- RoPE ---
 * Rotary position embedding of the decoder attention's q and k
 * (transformers' apply_rotary_pos_emb inside the Llama attention of each
 * Naylis decoder layer, model.py:279-345):
 *   out = x * cos + rotate_half(x) * sin,  rotate_half(a | b) = (-b | a)
 * with each product rounded to the dtype before the sum, as the reference's
 * elementwise ops.  backward != 0 applies the transposed rotation to incoming
 * gradients: out = dy * cos + rotate_half^T(dy * sin), rotate_half^T(a | b) =
 * (b | -a).  q, k, q_out, k_out (B, S, H, head_dim) row-major, outputs not
 * overlapping the inputs, cos / sin (cos_batch, S, head_dim) with cos_batch 1 or B;
 * head_dim 32, 64 or 128; one dtype (NAYLIS_DTYPE_*) for all. */
int naylis_mom_rope(const void* q, const void* k, const void* cos, const void* sin, void* q_out, void* k_out,
                    int dtype, int backward, int64_t B, int64_t S, int64_t H, int64_t head_dim, int64_t cos_batch,
                    void* stream);

/* -------------------------------------------------------------- SwiGLU ---
 * The decoder MLP's activation (transformers' LlamaMLP inside each Naylis
 * decoder layer, model.py:279-345): h = silu(gate) * up, silu(g) =
 * g / (1 + exp(-g)), silu rounded to the dtype before the product.  The
 * backward writes dgate = silu'(gate) * T(dh * up) and dup = dh * T(silu(gate)).
 * n elements (a multiple of 8) of one dtype, 16-byte aligned. */
int naylis_mom_swiglu_fwd(const void* gate, const void* up, void* h, int dtype, int64_t n, void* stream);
int naylis_mom_swiglu_bwd(const void* gate, const void* up, const void* dh, void* dgate, void* dup, int dtype,
                          int64_t n, void* stream);

/* ------------------------------------------------------- cross-entropy ---
 * The LM head loss of the decoder (model.py:536-545: F.cross_entropy of the
 * fp32 logits, reduction "sum", ignore_index) from bf16 logits (N, V) in one
 * pass: the forward writes each row's loss (log-sum-exp minus the label's
 * logit; 0 for rows labelled ignore_index; NaN for a label outside [0, V),
 * where the reference raises) and its log-sum-exp; the backward writes
 * dlogits (N, V) bf16 = (softmax - one_hot(label)) * grad_rows[r *
 * grad_stride] (grad_stride 1: one gradient per row, 0: one for all rows;
 * zero rows for ignore_index, NaN rows for out-of-range labels).
 * V a multiple of 2048; labels int64; logits / dlogits 16-byte aligned. */
int naylis_mom_xent_fwd(const void* logits, const int64_t* labels, float* loss_rows, float* lse, int64_t N, int64_t V,
                        int64_t ignore_index, void* stream);
int naylis_mom_xent_bwd(const void* logits, const int64_t* labels, const float* lse, const float* grad_rows,
                        int64_t grad_stride, void* dlogits, int64_t N, int64_t V, int64_t ignore_index, void* stream);

/* ------------------------------------------------------------ bank K/V ---
 * Projection of the shared bank, once per layer and shared by the batch:
 * model.py:253-256 (`k_proj(M_blocks.view(L, D))`, `v_proj(...)`), mirror in
 * mom_kernels/reference.py:86-89.  The reference runs two nn.Linear calls.
 *
 *   slots  (L, D_in) bf16        M_blocks viewed as L slots
 *   w_k, w_v (D_out, D_in) bf16  k_proj.weight, v_proj.weight
 *   k_out, v_out (L, D_out) bf16
 * Constraint: D_in a multiple of 8.
 */
int naylis_mom_bank_kv_fwd(const void* slots, const void* w_k, const void* w_v, void* k_out, void* v_out, int64_t L,
                           int64_t D_in, int64_t D_out, void* stream);

/* Backward: d_slots = dk w_k + dv w_v  (L, D_in), dw_k = dk^T slots and
 * dw_v = dv^T slots (D_out, D_in); gradients are written in the requested
 * dtype (NAYLIS_DTYPE_F32 or _BF16), accumulation is fp32.  D_out a multiple
 * of 8. */
int naylis_mom_bank_kv_bwd(const void* slots, const void* w_k, const void* w_v, const void* dk, const void* dv,
                           void* d_slots, int slots_grad_dtype, void* dw_k, void* dw_v, int w_grad_dtype, int64_t L,
                           int64_t D_in, int64_t D_out, void* stream);

/* Grouped: the projections of n layers that read one bank (the decoder's 20
 * MoM layers share model.M_blocks, model.py:409-416, and each projects it,
 * model.py:253-256), one launch per product instead of n.  Arrays hold one
 * pointer per layer (host memory); shapes and dtypes as above, the same for
 * every layer.
 *   forward   k_out[i] = slots w_k[i]^T, v_out[i] = slots w_v[i]^T, each
 *             bitwise equal to naylis_mom_bank_kv_fwd of layer i;
 *   backward  d_slots = sum_i dk[i] w_k[i] + dv[i] w_v[i], accumulated in
 *             fp32 over every layer in layer order and rounded once (the
 *             reference sums the per-layer bank gradients in autograd);
 *             dw_k[i], dw_v[i] bitwise equal to naylis_mom_bank_kv_bwd's.
 * 1 <= n <= NAYLIS_BANK_GROUP_MAX_LAYERS; D_in a multiple of 8, D_out of 64;
 * pointers 16-byte aligned.  The backward keeps n fp32 (L, D_in) partials in
 * the caller's workspace (naylis_mom_bank_kv_bwd_grouped_workspace_bytes). */
#define NAYLIS_BANK_GROUP_MAX_LAYERS 24
int naylis_mom_bank_kv_fwd_grouped(const void* slots, const void* const* w_k, const void* const* w_v,
                                   void* const* k_out, void* const* v_out, int64_t n_layers, int64_t L, int64_t D_in,
                                   int64_t D_out, void* stream);
size_t naylis_mom_bank_kv_bwd_grouped_workspace_bytes(int64_t n_layers, int64_t L, int64_t D_in, int64_t D_out);
int naylis_mom_bank_kv_bwd_grouped(const void* slots, const void* const* w_k, const void* const* w_v,
                                   const void* const* dk, const void* const* dv, void* d_slots, int slots_grad_dtype,
                                   void* const* dw_k, void* const* dw_v, int w_grad_dtype, void* workspace,
                                   size_t workspace_bytes, int64_t n_layers, int64_t L, int64_t D_in, int64_t D_out,
                                   void* stream);

/* ------------------------------------------------- projection weight grad ---
 * Weight gradient of the layer's bias-free query / output projections
 * (model.py:239 `q_proj`, model.py:251 `o_proj`, both nn.Linear(d, d,
 * bias=False)), which the reference gets from autograd as dy^T x summed over
 * all B*T tokens:
 *   dw[o][i] = sum_t dy[t][o] * x[t][i]      (fp32 accumulation)
 *   x  (N, D_in) bf16, dy (N, D_out) bf16, dw (D_out, D_in) in dw_dtype.
 * The token reduction is split over workgroups; the fp32 partials live in the
 * caller's workspace (naylis_mom_linear_wgrad_workspace_bytes) and are summed
 * in a fixed order, so the result is deterministic.
 * Constraints: N, D_in, D_out multiples of 8; pointers 16-byte aligned;
 * N * max(D_in, D_out) below 2^30. */
size_t naylis_mom_linear_wgrad_workspace_bytes(int64_t N, int64_t D_in, int64_t D_out);
int naylis_mom_linear_wgrad(const void* x, const void* dy, void* dw, int dw_dtype, void* workspace,
                            size_t workspace_bytes, int64_t N, int64_t D_in, int64_t D_out, void* stream);

/* ------------------------------------------------------------- ReZero ---
 * The layer's output gate (model.py:151 `mom_scale`, applied at model.py:239
 * as `self.mom_scale * out`): y = s * z with s the (1,) fp32 parameter on the
 * device, z (n elements) in z_dtype, y fp32 (torch type promotion).
 * Backward: dz = s * dy in z_dtype (dz may be NULL when z needs no gradient)
 * and ds = sum(dy * z), one fp32 value reduced in a fixed order through the
 * caller's workspace (naylis_mom_rezero_workspace_bytes).  dy in dy_dtype.
 * No counterpart kernel in the reference (eager elementwise ops there). */
size_t naylis_mom_rezero_workspace_bytes(int64_t n);
int naylis_mom_rezero_fwd(const void* z, int z_dtype, const float* s, float* y, int64_t n, void* stream);
int naylis_mom_rezero_bwd(const void* dy, int dy_dtype, const void* z, int z_dtype, const float* s, void* dz, float* ds,
                          void* workspace, size_t workspace_bytes, int64_t n, void* stream);
/* y = s * x with y in y_dtype (bf16 or fp32): the gate folded into the o
 * projection's weight, W' = s * W_o, so that the layer's fp32 output is one
 * GEMM, o W'^T = s * (o W_o^T) (model.py:239, 251).  The gradients of W_o and
 * s then follow from dW' (the gradient of W') by naylis_mom_rezero_bwd over
 * the weight's elements: dW_o = s * dW', ds = sum(dW' * W_o). */
int naylis_mom_rezero_scale(const void* x, int x_dtype, const float* s, void* y, int y_dtype, int64_t n, void* stream);
/* The two steps above in one call for the layer's backward (the o projection's
 * weight gradient, model.py:251, with the gate of model.py:239 folded in):
 *   dW'[o][i] = sum_t dy[t][o] * x[t][i]   (fp32, as naylis_mom_linear_wgrad)
 *   dw = bf16(s * dW')                     (the gradient of W_o)
 *   ds = sum(dW' * w)                      (the gradient of s; w = W_o)
 * x (N, D_in), dy (N, D_out), w and dw (D_out, D_in), all bf16; s and ds one
 * fp32 value each on the device.  dW' never leaves the split-K reduction: its
 * epilogue scales it and forms ds's partials, summed in a fixed order, so
 * the results are deterministic.  dw equals bf16(s * dW') of the two-step
 * path's dW' only where both reduce the same K splits; the K range is always
 * split at least in two here.  Workspace: naylis_mom_gated_wgrad_workspace_bytes.
 * Constraints as naylis_mom_linear_wgrad, and w, dw, workspace 16-byte aligned. */
size_t naylis_mom_gated_wgrad_workspace_bytes(int64_t N, int64_t D_in, int64_t D_out);
int naylis_mom_gated_wgrad(const void* x, const void* dy, const void* w, const float* s, void* dw, float* ds,
                           void* workspace, size_t workspace_bytes, int64_t N, int64_t D_in, int64_t D_out,
                           void* stream);

/* --------------------------------------------------------- decode step ---
 * One new token per sequence: the O(1) running-sum form of the prefix-mean
 * router that model.py:172-173 describes (the reference itself recomputes
 * the cumsum over the whole sequence, model.py:169-176, and has no decode
 * path: no reference entry point is replaced), then the gated read of the
 * token's top-k blocks from an fp8 bank.
 *
 * naylis_mom_bank_quant_fp8: K / V (L, D) bf16 -> OCP fp8 e4m3 codes (L, D)
 * uint8 and one fp32 scale per slot row, scale = max|row| / 448 (1 for an
 * all-zero row), code = e4m3fn(x / scale) rounded to nearest even.  Run once
 * per bank (the bank is fixed at inference).
 *
 * naylis_mom_decode_step, per sequence b:
 *   S' = S + x_new             state_in / state_out (B, D) fp64 (sum of the
 *                              tokens so far; must not overlap)
 *   h = fp32(S') / fp32(t_prev[b] + 1)     t_prev (B,) int32 >= 0, the
 *                              number of earlier tokens
 *   logits = w_up tanh(w_down h)           w_down (R, D), w_up (E, R) fp32
 *   top_idx (B, top_k) int32 = top-k logits (ties to the lower id),
 *   top_gates (B, top_k) fp32 = softmax over them (model.py:209-220)
 *   out (B, H, D/H) bf16 = softmax_n(q . k_n / sqrt(D/H) + log gate) v_n over
 *   the slots n of the selected blocks (mom_kernels/reference.py:39-61 with the
 *   bias of reference.py:14-29), q = q_new (B, H, D/H) bf16 and
 *   k_n = k_scale[n] e4m3(k8[n]), v_n = v_scale[n] e4m3(v8[n]).
 * x_new in x_dtype.  E = number of bank blocks, L = E * block_size.
 * Constraints: D = H * head_dim with head_dim in {32, 64, 128}, D <= 4096,
 * R <= 64, E <= 64, top_k <= min(8, E), E * block_size <= 16384, pointers
 * 16-byte aligned. */
int naylis_mom_bank_quant_fp8(const void* k, const void* v, uint8_t* k8, uint8_t* v8, float* k_scale, float* v_scale,
                              int64_t L, int64_t D, void* stream);
int naylis_mom_decode_step(const double* state_in, double* state_out, const int32_t* t_prev, const void* x_new,
                           int x_dtype, const float* w_down, const float* w_up, const void* q_new, const uint8_t* k8,
                           const uint8_t* v8, const float* k_scale, const float* v_scale, void* out, int32_t* top_idx,
                           float* top_gates, int64_t B, int64_t D, int64_t H, int64_t R, int64_t E, int64_t block_size,
                           int64_t top_k, void* stream);

/* -------------------------------------------------------------- timing ---
 * Optional instrumentation (no counterpart in the reference; for benchmarks):
 * when enabled, each kernel launch of this library is bracketed by hipEvents
 * on its stream.  naylis_mom_timing_get() waits for the recorded events and
 * returns the summed duration (ms) and launch count of one kernel name
 * (names: naylis_mom_timing_names(), comma-separated).  Off by default;
 * enabling it adds two event records per launch. */
void naylis_mom_timing_enable(int on);
void naylis_mom_timing_reset(void);
int naylis_mom_timing_get(const char* name, double* total_ms, int64_t* count);
int naylis_mom_timing_names(char* buf, size_t buf_bytes);

#ifdef __cplusplus
}
#endif

#endif /* NAYLIS_MOM_H */
