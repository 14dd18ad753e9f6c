// C ABI of libnaylis_mom.so: plain pointers, sizes and a hipStream_t.
// Every entry point validates its arguments the way the reference's Python
// layer raises (mom_kernels/triton_gpu.py:420-429, mom_kernels/__init__.py:
// 69-79) and returns a status code; no C++ exception crosses the boundary.
// The library holds no tensors and no mutable global state; the last error
// message is per calling thread (like errno).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <string>

#include "../../include/naylis_mom.h"
#include "launch.h"

using namespace naylis;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return NAYLIS_OK;
  return fail(NAYLIS_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

bool pow2(long x) { return x > 0 && (x & (x - 1)) == 0; }

int check_read_dims(int64_t B, int64_t S, int64_t H, int64_t hd, int64_t num_blocks, int64_t block_size,
                    int64_t top_k, ReadDims* d) {
  if (B < 0 || S < 0 || H <= 0) return fail(NAYLIS_ERR_ARG, "mom_read: bad shape B=%lld S=%lld H=%lld",
                                            (long long)B, (long long)S, (long long)H);
  if (!pow2(hd) || hd > 128 || hd < 16)
    return fail(NAYLIS_ERR_ARG, "mom_read: head_dim %lld must be a power of two in [16, 128]", (long long)hd);
  if (num_blocks <= 0 || block_size <= 0)
    return fail(NAYLIS_ERR_ARG, "mom_read: num_blocks (%lld) and block_size (%lld) must be positive",
                (long long)num_blocks, (long long)block_size);
  if (num_blocks > NAYLIS_MAX_BLOCKS)
    return fail(NAYLIS_ERR_ARG, "mom_read: num_blocks %lld exceeds %d", (long long)num_blocks, NAYLIS_MAX_BLOCKS);
  const int64_t L = num_blocks * block_size;
  if (L > NAYLIS_MAX_SLOTS)
    return fail(NAYLIS_ERR_ARG, "mom_read: bank of %lld slots exceeds %d", (long long)L, NAYLIS_MAX_SLOTS);
  if (top_k < 1 || top_k > NAYLIS_MAX_TOPK || top_k > num_blocks)
    return fail(NAYLIS_ERR_ARG, "mom_read: top_k %lld must be in [1, min(%d, num_blocks=%lld)]", (long long)top_k,
                NAYLIS_MAX_TOPK, (long long)num_blocks);
  if (B * S > (int64_t)1 << 30 || H * hd > 65536)
    return fail(NAYLIS_ERR_ARG, "mom_read: problem too large (B*S=%lld, H*hd=%lld)", (long long)(B * S),
                (long long)(H * hd));
  d->B = (int)B;
  d->S = (int)S;
  d->H = (int)H;
  d->HD = (int)hd;
  d->L = (int)L;
  d->E = (int)num_blocks;
  d->block_size = (int)block_size;
  d->topk = (int)top_k;
  return NAYLIS_OK;
}

struct ReadWs {
  size_t relayout, delta, dlg, part;  // byte offsets
  size_t total;
  int n_chunks;
};

ReadWs plan_read_ws(const ReadDims& d) {
  ReadWs w{};
  const size_t relay = (size_t)d.H * read_hdp(d.HD) * read_lp(d.L) * 2;
  const size_t ntok = (size_t)d.B * d.S;
  w.n_chunks = read_bwd_chunks(d);
  size_t off = 0;
  w.relayout = off;
  off += align256(relay);
  w.delta = off;
  off += align256(ntok * d.H * 4);
  w.dlg = off;
  off += align256(ntok * d.H * d.topk * 4);
  w.part = off;
  off += 2 * align256((size_t)w.n_chunks * read_lq(d.L) * d.H * d.HD * 4);
  w.total = off;
  return w;
}

}  // namespace

extern "C" {

int naylis_mom_abi_version(void) { return NAYLIS_MOM_ABI_VERSION; }

const char* naylis_mom_last_error(void) { return g_last_error.c_str(); }

size_t naylis_mom_read_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t head_dim, int64_t num_blocks,
                                       int64_t block_size, int64_t top_k) {
  ReadDims d;
  if (check_read_dims(B, S, H, head_dim, num_blocks, block_size, top_k, &d) != NAYLIS_OK) return 0;
  return plan_read_ws(d).total;
}

int naylis_mom_read_fwd(const void* q, const void* k, const void* v, const int32_t* top_idx, const float* top_gates,
                        void* out, float* lse, void* workspace, size_t workspace_bytes, int64_t B, int64_t S,
                        int64_t H, int64_t head_dim, int64_t num_blocks, int64_t block_size, int64_t top_k,
                        void* stream) {
  ReadDims d;
  int rc = check_read_dims(B, S, H, head_dim, num_blocks, block_size, top_k, &d);
  if (rc) return rc;
  if (B * S == 0) return NAYLIS_OK;
  if (!q || !k || !v || !top_idx || !top_gates || !out || !lse || !workspace)
    return fail(NAYLIS_ERR_ARG, "mom_read_fwd: null pointer argument");
  const ReadWs w = plan_read_ws(d);
  if (workspace_bytes < w.relayout + align256((size_t)d.H * read_hdp(d.HD) * read_lp(d.L) * 2))
    return fail(NAYLIS_ERR_WORKSPACE, "mom_read_fwd: workspace of %zu bytes is too small", workspace_bytes);
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  rc = hip_status(launch_bank_relayout(v, ws + w.relayout, d, st), "mom_read_fwd relayout");
  if (rc) return rc;
  return hip_status(launch_read_fwd(q, k, ws + w.relayout, top_idx, top_gates, out, lse, d, st), "mom_read_fwd");
}

int naylis_mom_read_bwd(const void* q, const void* k, const void* v, const int32_t* top_idx, const float* top_gates,
                        const void* out, const float* lse, const void* dout, void* dq, void* dk, void* dv,
                        float* dgates, void* workspace, size_t workspace_bytes, int64_t B, int64_t S, int64_t H,
                        int64_t head_dim, int64_t num_blocks, int64_t block_size, int64_t top_k, void* stream) {
  ReadDims d;
  int rc = check_read_dims(B, S, H, head_dim, num_blocks, block_size, top_k, &d);
  if (rc) return rc;
  if (!k || !v || !dk || !dv || !workspace) return fail(NAYLIS_ERR_ARG, "mom_read_bwd: null pointer argument");
  if (B * S > 0 && (!q || !top_idx || !top_gates || !out || !lse || !dout || !dq || !dgates))
    return fail(NAYLIS_ERR_ARG, "mom_read_bwd: null pointer argument");
  const ReadWs w = plan_read_ws(d);
  if (workspace_bytes < w.total)
    return fail(NAYLIS_ERR_WORKSPACE, "mom_read_bwd: workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, w.total);
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  float* delta = (float*)(ws + w.delta);
  float* dlg = (float*)(ws + w.dlg);
  const size_t part_bytes = align256((size_t)w.n_chunks * read_lq(d.L) * d.H * d.HD * 4);
  float* dkp = (float*)(ws + w.part);
  float* dvp = (float*)(ws + w.part + part_bytes);
  if (B * S > 0) {
    rc = hip_status(launch_bank_relayout(k, ws + w.relayout, d, st), "mom_read_bwd relayout");
    if (rc) return rc;
    rc = hip_status(launch_read_bwd_dq(q, k, v, ws + w.relayout, top_idx, top_gates, out, dout, lse, dq, delta, dlg,
                                       d, st),
                    "mom_read_bwd dq");
    if (rc) return rc;
  }
  rc = hip_status(launch_read_bwd_dkdv(q, k, v, top_idx, top_gates, dout, lse, delta, dkp, dvp, w.n_chunks, d, st),
                  "mom_read_bwd dkdv");
  if (rc) return rc;
  return hip_status(launch_read_bwd_reduce(dkp, dvp, dlg, top_gates, dk, dv, dgates, w.n_chunks, d, st),
                    "mom_read_bwd reduce");
}

}  // extern "C"
