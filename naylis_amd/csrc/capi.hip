// C ABI of libnaylis_mom.so: plain pointers, sizes and a hipStream_t.
// Every entry point validates its arguments the way the reference's Python
// layer raises (mom_kernels/triton_gpu.py:420-429, mom_kernels/__init__.py:
// 69-79) and returns a status code; no C++ exception crosses the boundary.
// The library holds no tensors; its only mutable global state is the
// per-device scratch array of naylis_mom_read_bwd_noalloc (with the table of
// its device addresses) and the last error message, which is per calling
// thread (like errno).
#include <stdarg.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <initializer_list>
#include <mutex>
#include <string>

#include "../../include/naylis_mom.h"
#include "launch.h"
#include "launch_router.h"
#include "launch_bank.h"
#include <algorithm>

#include "launch_gemm.h"
#include "launch_rezero.h"

namespace naylis {

// The epoch is the per-device launch count passed through the SplitMix64
// finalizer (Steele, Lea and Flood, 2014), so its bits look random: a word
// left in a reused workspace by other data (small integers, zeros, floats)
// matches it only by a 2^-48 chance, where a plain counter would collide
// with small integers.
unsigned long long next_launch_epoch() {
  static std::atomic<unsigned long long> counts[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  unsigned long long z;
  do {
    z = counts[dev].fetch_add(1, std::memory_order_relaxed) + 1 + ((unsigned long long)dev << 56);
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
  } while ((z >> 16) == 0);
  return z;
}

static std::atomic<int> g_spin_limit{20000};

int one_launch_spin_limit(int polls) {
  return polls < 0 ? g_spin_limit.load(std::memory_order_relaxed)
                   : g_spin_limit.exchange(polls, std::memory_order_relaxed);
}

bool stream_capturing(hipStream_t st) {
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(st, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone;
}

}  // namespace naylis

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

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

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
  size_t delta, dlg, tile_flags, list, count, part;  // byte offsets
  size_t total;
  int n_parts;
};

// The forward needs no workspace; the backward's layout is below.
ReadWs plan_read_ws(const ReadDims& d) {
  ReadWs w{};
  const size_t ntok = (size_t)d.B * d.S;
  const size_t n_tt = (size_t)read_bwd_n_ttiles(d);
  const size_t n_sg = (size_t)read_lq(d.L) / 128;
  w.n_parts = read_bwd_parts(d);
  size_t off = 0;
  w.delta = off;
  off += align256(ntok * d.H * 4);
  w.dlg = off;
  off += align256(ntok * d.H * d.topk * 4);
  w.tile_flags = off;
  off += align256(n_tt * d.E);
  w.list = off;
  off += align256(n_sg * n_tt * 4);
  w.count = off;
  off += align256(n_sg * 4);
  w.part = off;
  off += 2 * align256((size_t)w.n_parts * 128 * d.H * d.HD * 4);
  w.total = off;
  return w;
}

// The pair-tiled backward's workspace: per-head gate-gradient partials and
// the dK / dV partials of its (range, pair) segments.
struct PairWs {
  size_t dlg, dk_part, dv_part, total;
};

PairWs plan_pair_ws(const ReadDims& d) {
  PairWs w{};
  const size_t ntok = (size_t)d.B * d.S;
  const size_t part = align256(read_pair_part_bytes(d));
  size_t off = 0;
  w.dlg = off;
  off += align256(ntok * d.H * 2 * 4);
  w.dk_part = off;
  off += part;
  w.dv_part = off;
  off += part;
  w.total = off;
  return w;
}

// Shapes for which a call with a token order and a side buffer takes the pair-tiled
// backward.
bool pair_bwd_shapes(const ReadDims& d) { return read_pair_bwd_shapes(d, (long)d.B * d.S); }

int check_router_dims(int64_t B, int64_t T, int64_t D, int64_t R, int64_t E, int64_t top_k, RouterDims* d) {
  if (B < 0 || T < 0 || D <= 0)
    return fail(NAYLIS_ERR_ARG, "mom_route: bad shape B=%lld T=%lld D=%lld", (long long)B, (long long)T,
                (long long)D);
  if (R < 1 || R > NAYLIS_ROUTER_MAX_RANK)
    return fail(NAYLIS_ERR_ARG, "mom_route: router rank %lld must be in [1, %d]", (long long)R,
                NAYLIS_ROUTER_MAX_RANK);
  if (E < 1 || E > NAYLIS_ROUTER_MAX_BLOCKS)
    return fail(NAYLIS_ERR_ARG, "mom_route: num_blocks %lld must be in [1, %d]", (long long)E,
                NAYLIS_ROUTER_MAX_BLOCKS);
  if (top_k < 1 || top_k > NAYLIS_MAX_TOPK || top_k > E)
    return fail(NAYLIS_ERR_ARG, "mom_route: top_k %lld must be in [1, min(%d, num_blocks=%lld)]", (long long)top_k,
                NAYLIS_MAX_TOPK, (long long)E);
  if (B * T > ((int64_t)1 << 30) || D > (1 << 20) || T > (1 << 24))
    return fail(NAYLIS_ERR_ARG, "mom_route: problem too large (B*T <= 2^30, D <= 2^20, T <= 2^24)");
  d->B = (int)B;
  d->T = (int)T;
  d->D = (int)D;
  d->R = (int)R;
  d->E = (int)E;
  d->topk = (int)top_k;
  return NAYLIS_OK;
}

int check_dtype(int dt, const char* what) {
  if (dt != NAYLIS_DTYPE_F32 && dt != NAYLIS_DTYPE_BF16)
    return fail(NAYLIS_ERR_ARG, "%s: unsupported dtype code %d (0 = fp32, 1 = bf16)", what, dt);
  return NAYLIS_OK;
}

}  // namespace

extern "C" {

int naylis_mom_abi_version(void) { return NAYLIS_MOM_ABI_VERSION; }

const char* naylis_mom_last_error(void) { return g_last_error.c_str(); }

size_t naylis_mom_read_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t head_dim, int64_t num_blocks,
                                       int64_t block_size, int64_t top_k) {
  ReadDims d;
  if (check_read_dims(B, S, H, head_dim, num_blocks, block_size, top_k, &d) != NAYLIS_OK) return 0;
  const size_t two_pass = plan_read_ws(d).total;
  return pair_bwd_shapes(d) ? std::max(two_pass, plan_pair_ws(d).total) : two_pass;
}

size_t naylis_mom_read_side_bytes(int64_t B, int64_t S, int64_t H, int64_t head_dim, int64_t num_blocks,
                                  int64_t block_size, int64_t top_k) {
  ReadDims d;
  if (check_read_dims(B, S, H, head_dim, num_blocks, block_size, top_k, &d) != NAYLIS_OK) return 0;
  return pair_bwd_shapes(d) ? read_pair_side_bytes(d) : 0;
}

int naylis_mom_read_fwd(const void* q, const void* k, const void* v, const int32_t* top_idx, const float* top_gates,
                        const int32_t* token_order, void* out, void* side, float* lse, void* workspace,
                        size_t workspace_bytes, int64_t B, int64_t S, int64_t H, int64_t head_dim,
                        int64_t num_blocks, int64_t block_size, int64_t top_k, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  ReadDims d;
  int rc = check_read_dims(B, S, H, head_dim, num_blocks, block_size, top_k, &d);
  if (rc) return rc;
  d.order = token_order;
  if (B * S == 0) return NAYLIS_OK;
  if (!q || !k || !v || !top_idx || !top_gates || !out || !lse)
    return fail(NAYLIS_ERR_ARG, "mom_read_fwd: null pointer argument");
  hipStream_t st = (hipStream_t)stream;
  if (read_pair_fwd_ok(d, (long)B * S))
    return hip_status(launch_read_fwd_pair(q, k, v, top_idx, top_gates, out, read_pair_bwd_ok(d, (long)B * S) ? side
                                                                                                : nullptr,
                                           lse, d, st),
                      "mom_read_fwd");
  return hip_status(launch_read_fwd(q, k, v, top_idx, top_gates, out, lse, d, st), "mom_read_fwd");
}

int naylis_mom_read_bwd(const void* q, const void* k, const void* v, const int32_t* top_idx, const float* top_gates,
                        const int32_t* token_order, const void* out, const void* side, const float* lse,
                        const void* dout, void* dq, void* dk, void* dv, float* dgates, void* workspace,
                        size_t workspace_bytes, int64_t B, int64_t S, int64_t H, int64_t head_dim,
                        int64_t num_blocks, int64_t block_size, int64_t top_k, void* stream) {
  ReadDims d;
  int rc = check_read_dims(B, S, H, head_dim, num_blocks, block_size, top_k, &d);
  if (rc) return rc;
  d.order = token_order;
  if (!k || !v || !dk || !dv || !workspace) return fail(NAYLIS_ERR_ARG, "mom_read_bwd: null pointer argument");
  if (B * S > 0 && (!q || !top_idx || !top_gates || !out || !lse || !dout || !dq || !dgates))
    return fail(NAYLIS_ERR_ARG, "mom_read_bwd: null pointer argument");
  hipStream_t st = (hipStream_t)stream;
  if (side != nullptr && read_pair_bwd_ok(d, (long)B * S)) {
    const PairWs pw = plan_pair_ws(d);
    if (workspace_bytes < pw.total)
      return fail(NAYLIS_ERR_WORKSPACE, "mom_read_bwd: workspace of %zu bytes is smaller than the %zu required",
                  workspace_bytes, pw.total);
    char* ws = (char*)workspace;
    return hip_status(launch_read_bwd_pair(q, k, v, top_idx, top_gates, out, side, dout, lse, dq, dk, dv, dgates,
                                           (float*)(ws + pw.dlg), (float*)(ws + pw.dk_part),
                                           (float*)(ws + pw.dv_part), d, st),
                      "mom_read_bwd");
  }
  const ReadWs w = plan_read_ws(d);
  if (workspace_bytes < w.total)
    return fail(NAYLIS_ERR_WORKSPACE, "mom_read_bwd: workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, w.total);
  char* ws = (char*)workspace;
  float* delta = (float*)(ws + w.delta);
  float* dlg = (float*)(ws + w.dlg);
  uint8_t* tflags = (uint8_t*)(ws + w.tile_flags);
  int32_t* list = (int32_t*)(ws + w.list);
  int32_t* count = (int32_t*)(ws + w.count);
  const size_t part_bytes = align256((size_t)w.n_parts * 128 * d.H * d.HD * 4);
  float* dkp = (float*)(ws + w.part);
  float* dvp = (float*)(ws + w.part + part_bytes);
  if (B * S > 0) {
    rc = hip_status(launch_read_bwd_dq(q, k, v, top_idx, top_gates, out, dout, lse, dq, delta, dlg, tflags, d, st),
                    "mom_read_bwd dq");
    if (rc) return rc;
  }
  rc = hip_status(launch_read_tile_lists(top_idx, tflags, list, count, d, st), "mom_read_bwd tile lists");
  if (rc) return rc;
  rc = hip_status(launch_read_bwd_dkdv(q, k, v, top_idx, top_gates, dout, lse, delta, list, count, dkp, dvp, dk,
                                       dv, d, st),
                  "mom_read_bwd dkdv");
  if (rc) return rc;
  return hip_status(launch_read_bwd_reduce(dkp, dvp, count, dlg, top_gates, dk, dv, dgates, d, st),
                    "mom_read_bwd reduce");
}

// ------------------------------------------- read backward, no allocation
// The workspace of naylis_mom_read_bwd_noalloc: a file-scope device array
// that each device the library runs on holds from the code object's load to
// the end of the process.  In host code its name is not a device address:
// every host use goes through the address hipGetSymbolAddress returns on the
// device in question (one per device, looked up once).  Nothing in the read
// backward's workspace has to start at zero (each word is written before it
// is read within one call), so calls do not clear it.
static __device__ __align__(256) unsigned char scratch[NAYLIS_READ_BWD_NOALLOC_MAX_BYTES];

namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_addr[kScratchDevices];

// The scratch array's address on the device the stream belongs to, which must
// be the current device: hipGetSymbolAddress answers for the current device,
// and the kernels run on the stream's.
int scratch_address(hipStream_t stream, void** out) {
  int dev = -1;
  int rc = hip_status(hipGetDevice(&dev), "mom_read_bwd_noalloc: hipGetDevice");
  if (rc) return rc;
  hipDevice_t sdev = -1;
  rc = hip_status(hipStreamGetDevice(stream, &sdev), "mom_read_bwd_noalloc: hipStreamGetDevice");
  if (rc) return rc;
  if ((int)sdev != dev)
    return fail(NAYLIS_ERR_ARG,
                "mom_read_bwd_noalloc: the stream belongs to device %d but device %d is current; make the stream's "
                "device current before the call",
                (int)sdev, dev);
  if (dev < 0 || dev >= kScratchDevices)
    return fail(NAYLIS_ERR_ARG, "mom_read_bwd_noalloc: device %d beyond the %d the library tracks", dev,
                kScratchDevices);
  void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (!p) {
      rc = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "mom_read_bwd_noalloc: hipGetSymbolAddress");
      if (rc) return rc;
      if (!p) return fail(NAYLIS_ERR_HIP, "mom_read_bwd_noalloc: no device address for the scratch array");
      g_scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return NAYLIS_OK;
}

}  // namespace

int naylis_mom_read_bwd_noalloc(const void* q, const void* k, const void* v, const int32_t* top_idx,
                                const float* top_gates, const int32_t* token_order, const void* out,
                                const void* side, const float* lse, const void* dout, void* dq, void* dk, void* dv,
                                float* dgates, int64_t B, int64_t S, int64_t H, int64_t head_dim,
                                int64_t num_blocks, int64_t block_size, int64_t top_k, void* stream) {
  ReadDims d;
  int rc = check_read_dims(B, S, H, head_dim, num_blocks, block_size, top_k, &d);
  if (rc) return rc;
  d.order = token_order;
  const size_t need = (side != nullptr && read_pair_bwd_ok(d, (long)B * S)) ? plan_pair_ws(d).total
                                                                               : plan_read_ws(d).total;
  if (need > NAYLIS_READ_BWD_NOALLOC_MAX_BYTES)
    return fail(NAYLIS_ERR_WORKSPACE,
                "mom_read_bwd_noalloc: this read needs %zu bytes of workspace, more than the %zu of the library's "
                "scratch array; call naylis_mom_read_bwd with a workspace",
                need, (size_t)NAYLIS_READ_BWD_NOALLOC_MAX_BYTES);
  void* ws = nullptr;
  if ((rc = scratch_address((hipStream_t)stream, &ws))) return rc;
  return naylis_mom_read_bwd(q, k, v, top_idx, top_gates, token_order, out, side, lse, dout, dq, dk, dv, dgates,
                             ws, NAYLIS_READ_BWD_NOALLOC_MAX_BYTES, B, S, H, head_dim, num_blocks, block_size, top_k,
                             stream);
}

static int check_order_dims(int64_t B, int64_t S, int64_t num_blocks, int64_t top_k) {
  if (B < 0 || S < 0 || B * S > ((int64_t)1 << 30))
    return fail(NAYLIS_ERR_ARG, "mom_read_order: bad token count B=%lld S=%lld", (long long)B, (long long)S);
  if (num_blocks < 1 || num_blocks > NAYLIS_MAX_BLOCKS)
    return fail(NAYLIS_ERR_ARG, "mom_read_order: num_blocks %lld must be in [1, %d]", (long long)num_blocks,
                NAYLIS_MAX_BLOCKS);
  if (top_k < 1 || top_k > NAYLIS_MAX_TOPK || top_k > num_blocks)
    return fail(NAYLIS_ERR_ARG, "mom_read_order: top_k %lld must be in [1, min(%d, num_blocks=%lld)]",
                (long long)top_k, NAYLIS_MAX_TOPK, (long long)num_blocks);
  return NAYLIS_OK;
}

int64_t naylis_mom_read_order_words(int64_t B, int64_t S, int64_t num_blocks, int64_t top_k) {
  if (check_order_dims(B, S, num_blocks, top_k) != NAYLIS_OK) return 0;
  return read_order_words((long)(B * S), (int)num_blocks, (int)top_k);
}

size_t naylis_mom_read_order_workspace_bytes(int64_t B, int64_t S, int64_t num_blocks, int64_t top_k) {
  if (check_order_dims(B, S, num_blocks, top_k) != NAYLIS_OK) return 0;
  return read_order_ws_bytes((long)(B * S), (int)num_blocks, (int)top_k);
}

int naylis_mom_read_order(const int32_t* top_idx, int32_t* order, void* workspace, size_t workspace_bytes, int64_t B,
                          int64_t S, int64_t num_blocks, int64_t top_k, void* stream) {
  int rc = check_order_dims(B, S, num_blocks, top_k);
  if (rc) return rc;
  if (B * S == 0) return NAYLIS_OK;
  if (!top_idx || !order || !workspace) return fail(NAYLIS_ERR_ARG, "mom_read_order: null pointer argument");
  const size_t need = read_order_ws_bytes((long)(B * S), (int)num_blocks, (int)top_k);
  if (workspace_bytes < need)
    return fail(NAYLIS_ERR_WORKSPACE, "mom_read_order: workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, need);
  return hip_status(launch_read_order(top_idx, (long)(B * S), (int)num_blocks, (int)top_k, order, workspace,
                                      (hipStream_t)stream),
                    "mom_read_order");
}

size_t naylis_mom_router_workspace_bytes(int64_t B, int64_t T, int64_t D, int64_t R, int64_t E, int64_t top_k) {
  RouterDims d;
  if (check_router_dims(B, T, D, R, E, top_k, &d) != NAYLIS_OK) return 0;
  return plan_router_ws(d).total;
}

int naylis_mom_router_fwd(const void* x, int x_dtype, const float* w_down, const float* w_up, const float* noise,
                          int noise_kind, float noise_scale, float* logits, float* probs, int32_t* top_idx,
                          float* top_gates, float* act, float* h_out, void* workspace, size_t workspace_bytes,
                          int64_t B, int64_t T, int64_t D, int64_t R, int64_t E, int64_t top_k, void* stream) {
  RouterDims d;
  int rc = check_router_dims(B, T, D, R, E, top_k, &d);
  if (rc) return rc;
  if ((rc = check_dtype(x_dtype, "mom_route"))) return rc;
  if (noise_kind != NAYLIS_NOISE_ADDITIVE && noise_kind != NAYLIS_NOISE_GUMBEL_UNIFORM)
    return fail(NAYLIS_ERR_ARG, "mom_route_fwd: noise_kind %d must be %d (additive) or %d (uniform draw, Gumbel)",
                noise_kind, NAYLIS_NOISE_ADDITIVE, NAYLIS_NOISE_GUMBEL_UNIFORM);
  d.noise_kind = noise_kind;
  if (B * T == 0) return NAYLIS_OK;
  if (!x || !w_down || !w_up || !logits || !probs || !top_idx || !top_gates || !act || !workspace)
    return fail(NAYLIS_ERR_ARG, "mom_route_fwd: null pointer argument");
  const RouterWs w = plan_router_ws(d);
  if (workspace_bytes < w.fwd_total)
    return fail(NAYLIS_ERR_WORKSPACE, "mom_route_fwd: workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, w.fwd_total);
  return hip_status(launch_router_fwd(x, x_dtype == NAYLIS_DTYPE_BF16, w_down, w_up, noise, noise_scale, logits, probs,
                                      top_idx, top_gates, act, h_out, workspace, d, (hipStream_t)stream),
                    "mom_route_fwd");
}

int naylis_mom_spin_limit(int polls) { return one_launch_spin_limit(polls); }

int naylis_mom_router_bwd(const void* x, int x_dtype, const float* w_down, const float* w_up, const float* act,
                          const float* probs, const int32_t* top_idx, const float* top_gates, const float* d_gates,
                          const float* d_probs, int64_t d_probs_stride, const float* d_logits, void* dx,
                          int dx_accumulate, float* dw_down, float* dw_up, void* workspace, size_t workspace_bytes,
                          int64_t B, int64_t T, int64_t D, int64_t R, int64_t E, int64_t top_k, void* stream) {
  RouterDims d;
  int rc = check_router_dims(B, T, D, R, E, top_k, &d);
  if (rc) return rc;
  if ((rc = check_dtype(x_dtype, "mom_route"))) return rc;
  if (d_probs && d_probs_stride != 0 && d_probs_stride != E)
    return fail(NAYLIS_ERR_ARG, "mom_route_bwd: d_probs_stride %lld must be num_blocks (%lld) or 0",
                (long long)d_probs_stride, (long long)E);
  d.dp_stride = (long)d_probs_stride;
  if (dx_accumulate && B * T > 0 && !router_fast_bwd_ok(x, x_dtype == NAYLIS_DTYPE_BF16, dx, d))
    return fail(NAYLIS_ERR_ARG,
                "mom_route_bwd: dx_accumulate needs bf16 x, D a multiple of 128, R <= 64 and 16-byte aligned x / dx");
  if (!w_down || !w_up || !dw_down || !dw_up || !workspace)
    return fail(NAYLIS_ERR_ARG, "mom_route_bwd: null pointer argument");
  if (B * T > 0 && (!x || !act || !probs || !top_idx || !top_gates || !dx))
    return fail(NAYLIS_ERR_ARG, "mom_route_bwd: null pointer argument");
  const RouterWs w = plan_router_ws(d);
  if (workspace_bytes < w.total)
    return fail(NAYLIS_ERR_WORKSPACE, "mom_route_bwd: workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, w.total);
  return hip_status(launch_router_bwd(x, x_dtype == NAYLIS_DTYPE_BF16, w_down, w_up, act, probs, top_idx, top_gates,
                                      d_gates, d_probs, d_logits, dx, dx_accumulate != 0, dw_down, dw_up, workspace, d,
                                      (hipStream_t)stream),
                    "mom_route_bwd");
}

static int check_norm(int dtype, int64_t N, int64_t D, const char* who) {
  int rc = check_dtype(dtype, who);
  if (rc) return rc;
  if (N < 0 || N > ((int64_t)1 << 31))
    return fail(NAYLIS_ERR_ARG, "%s: bad row count N=%lld", who, (long long)N);
  if (D < 512 || D > 4096 || D % 512 != 0)
    return fail(NAYLIS_ERR_ARG, "%s: D=%lld must be a multiple of 512 in [512, 4096]", who, (long long)D);
  return NAYLIS_OK;
}

int naylis_mom_rmsnorm_fwd(const void* x, int dtype, const void* weight, void* y, float* rstd, int64_t N, int64_t D,
                           float eps, void* stream) {
  int rc = check_norm(dtype, N, D, "mom_rmsnorm_fwd");
  if (rc) return rc;
  if (!(eps >= 0.f) || eps > 1.f) return fail(NAYLIS_ERR_ARG, "mom_rmsnorm_fwd: eps %g must be in [0, 1]", (double)eps);
  if (N == 0) return NAYLIS_OK;
  if (!x || !weight || !y || !rstd) return fail(NAYLIS_ERR_ARG, "mom_rmsnorm_fwd: null pointer argument");
  if (!aligned16(x) || !aligned16(weight) || !aligned16(y))
    return fail(NAYLIS_ERR_ARG, "mom_rmsnorm_fwd: x, weight and y must be 16-byte aligned");
  return hip_status(launch_rmsnorm_fwd(x, dtype == NAYLIS_DTYPE_BF16, weight, y, rstd, (long)N, (int)D, eps,
                                       (hipStream_t)stream),
                    "mom_rmsnorm_fwd");
}

size_t naylis_mom_rmsnorm_workspace_bytes(int64_t N, int64_t D) {
  if (N < 0 || N > ((int64_t)1 << 31) || D < 512 || D > 4096 || D % 512 != 0) return 0;
  return rmsnorm_ws_bytes((long)N, (int)D);
}

int naylis_mom_rmsnorm_bwd(const void* x, int dtype, const void* weight, const float* rstd, const void* dy, void* dx,
                           void* dweight, void* workspace, size_t workspace_bytes, int64_t N, int64_t D,
                           void* stream) {
  int rc = check_norm(dtype, N, D, "mom_rmsnorm_bwd");
  if (rc) return rc;
  if (!weight || !dweight || !workspace) return fail(NAYLIS_ERR_ARG, "mom_rmsnorm_bwd: null pointer argument");
  if (N > 0 && (!x || !rstd || !dy || !dx)) return fail(NAYLIS_ERR_ARG, "mom_rmsnorm_bwd: null pointer argument");
  if (N > 0 && (!aligned16(x) || !aligned16(weight) || !aligned16(dy) || !aligned16(dx)))
    return fail(NAYLIS_ERR_ARG, "mom_rmsnorm_bwd: x, weight, dy and dx must be 16-byte aligned");
  const size_t need = rmsnorm_ws_bytes((long)N, (int)D);
  if (workspace_bytes < need)
    return fail(NAYLIS_ERR_WORKSPACE, "mom_rmsnorm_bwd: workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, need);
  return hip_status(launch_rmsnorm_bwd(x, dtype == NAYLIS_DTYPE_BF16, weight, rstd, dy, nullptr, dx, dweight,
                                       workspace, (long)N, (int)D, (hipStream_t)stream),
                    "mom_rmsnorm_bwd");
}

int naylis_mom_add_rmsnorm_fwd(const void* x, const void* a, int a_dtype, const void* weight, void* s_out, void* y,
                               float* rstd, int dtype, int64_t N, int64_t D, float eps, void* stream) {
  int rc = check_norm(dtype, N, D, "mom_add_rmsnorm_fwd");
  if (rc) return rc;
  if ((rc = check_dtype(a_dtype, "mom_add_rmsnorm_fwd"))) return rc;
  if (dtype == NAYLIS_DTYPE_F32 && a_dtype != NAYLIS_DTYPE_F32)
    return fail(NAYLIS_ERR_ARG, "mom_add_rmsnorm_fwd: an fp32 stream takes an fp32 residual branch");
  if (!(eps >= 0.f) || eps > 1.f)
    return fail(NAYLIS_ERR_ARG, "mom_add_rmsnorm_fwd: eps %g must be in [0, 1]", (double)eps);
  if (N == 0) return NAYLIS_OK;
  if (!x || !a || !weight || !s_out || !y || !rstd)
    return fail(NAYLIS_ERR_ARG, "mom_add_rmsnorm_fwd: null pointer argument");
  if (!aligned16(x) || !aligned16(a) || !aligned16(weight) || !aligned16(s_out) || !aligned16(y))
    return fail(NAYLIS_ERR_ARG, "mom_add_rmsnorm_fwd: x, a, weight, s_out and y must be 16-byte aligned");
  return hip_status(launch_add_rmsnorm_fwd(x, a, a_dtype == NAYLIS_DTYPE_F32, dtype == NAYLIS_DTYPE_BF16, weight,
                                           s_out, y, rstd, (long)N, (int)D, eps, (hipStream_t)stream),
                    "mom_add_rmsnorm_fwd");
}

int naylis_mom_add_rmsnorm_bwd(const void* s, const void* weight, const float* rstd, const void* dy, const void* dres,
                               void* ds, void* dweight, void* workspace, size_t workspace_bytes, int dtype, int64_t N,
                               int64_t D, void* stream) {
  int rc = check_norm(dtype, N, D, "mom_add_rmsnorm_bwd");
  if (rc) return rc;
  if (!weight || !dweight || !workspace) return fail(NAYLIS_ERR_ARG, "mom_add_rmsnorm_bwd: null pointer argument");
  if (N > 0 && (!s || !rstd || !dy || !ds)) return fail(NAYLIS_ERR_ARG, "mom_add_rmsnorm_bwd: null pointer argument");
  if (N > 0 && (!aligned16(s) || !aligned16(weight) || !aligned16(dy) || !aligned16(ds) ||
                (dres && !aligned16(dres))))
    return fail(NAYLIS_ERR_ARG, "mom_add_rmsnorm_bwd: s, weight, dy, dres and ds must be 16-byte aligned");
  const size_t need = rmsnorm_ws_bytes((long)N, (int)D);
  if (workspace_bytes < need)
    return fail(NAYLIS_ERR_WORKSPACE, "mom_add_rmsnorm_bwd: workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, need);
  return hip_status(launch_rmsnorm_bwd(s, dtype == NAYLIS_DTYPE_BF16, weight, rstd, dy, dres, ds, dweight, workspace,
                                       (long)N, (int)D, (hipStream_t)stream),
                    "mom_add_rmsnorm_bwd");
}

int naylis_mom_rope(const void* q, const void* k, const void* cos, const void* sin, void* q_out, void* k_out,
                    int dtype, int backward, int64_t B, int64_t S, int64_t H, int64_t head_dim, int64_t cos_batch,
                    void* stream) {
  int rc = check_dtype(dtype, "mom_rope");
  if (rc) return rc;
  if (B < 0 || S < 0 || H < 0 || B * S * H > ((int64_t)1 << 30))
    return fail(NAYLIS_ERR_ARG, "mom_rope: bad shape B=%lld S=%lld H=%lld", (long long)B, (long long)S, (long long)H);
  if (head_dim != 32 && head_dim != 64 && head_dim != 128)
    return fail(NAYLIS_ERR_ARG, "mom_rope: head_dim %lld must be 32, 64 or 128", (long long)head_dim);
  if (cos_batch != 1 && cos_batch != B)
    return fail(NAYLIS_ERR_ARG, "mom_rope: cos / sin batch %lld must be 1 or B=%lld", (long long)cos_batch,
                (long long)B);
  if (B * S * H == 0) return NAYLIS_OK;
  if (!q || !k || !cos || !sin || !q_out || !k_out) return fail(NAYLIS_ERR_ARG, "mom_rope: null pointer argument");
  {
    const size_t bytes = (size_t)(B * S * H * head_dim) * (dtype == NAYLIS_DTYPE_BF16 ? 2 : 4);
    const void* ins[2] = {q, k};
    const void* outs[2] = {q_out, k_out};
    for (const void* o : outs)
      for (const void* in : ins) {
        const uintptr_t a = (uintptr_t)o, b = (uintptr_t)in;
        if (a < b + bytes && b < a + bytes)
          return fail(NAYLIS_ERR_ARG, "mom_rope: outputs must not overlap q or k");
      }
    if (!aligned16(q) || !aligned16(k) || !aligned16(cos) || !aligned16(sin) || !aligned16(q_out) ||
        !aligned16(k_out))
      return fail(NAYLIS_ERR_ARG, "mom_rope: all tensors must be 16-byte aligned");
  }
  return hip_status(launch_rope(q, k, cos, sin, q_out, k_out, dtype == NAYLIS_DTYPE_BF16, backward != 0, (long)B,
                                (int)S, (int)H, (int)head_dim, (int)cos_batch, (hipStream_t)stream),
                    "mom_rope");
}

static int check_swiglu(int dtype, int64_t n, std::initializer_list<const void*> ptrs, const char* who) {
  int rc = check_dtype(dtype, who);
  if (rc) return rc;
  if (n < 0 || n % 8 != 0 || n > ((int64_t)1 << 36))
    return fail(NAYLIS_ERR_ARG, "%s: element count %lld must be a non-negative multiple of 8", who, (long long)n);
  if (n == 0) return NAYLIS_OK;
  for (const void* p : ptrs) {
    if (!p) return fail(NAYLIS_ERR_ARG, "%s: null pointer argument", who);
    if (!aligned16(p)) return fail(NAYLIS_ERR_ARG, "%s: every tensor must be 16-byte aligned", who);
  }
  return NAYLIS_OK;
}

int naylis_mom_swiglu_fwd(const void* gate, const void* up, void* h, int dtype, int64_t n, void* stream) {
  int rc = check_swiglu(dtype, n, {gate, up, h}, "mom_swiglu_fwd");
  if (rc || n == 0) return rc;
  return hip_status(launch_swiglu(gate, up, nullptr, h, nullptr, dtype == NAYLIS_DTYPE_BF16, false, (long)n,
                                  (hipStream_t)stream),
                    "mom_swiglu_fwd");
}

int naylis_mom_swiglu_bwd(const void* gate, const void* up, const void* dh, void* dgate, void* dup, int dtype,
                          int64_t n, void* stream) {
  int rc = check_swiglu(dtype, n, {gate, up, dh, dgate, dup}, "mom_swiglu_bwd");
  if (rc || n == 0) return rc;
  return hip_status(launch_swiglu(gate, up, dh, dgate, dup, dtype == NAYLIS_DTYPE_BF16, true, (long)n,
                                  (hipStream_t)stream),
                    "mom_swiglu_bwd");
}

static int check_xent(int64_t N, int64_t V, const char* who) {
  if (N < 0 || N > ((int64_t)1 << 31)) return fail(NAYLIS_ERR_ARG, "%s: bad row count N=%lld", who, (long long)N);
  if (V < 2048 || V % 2048 != 0 || V > (1 << 24))
    return fail(NAYLIS_ERR_ARG, "%s: vocabulary %lld must be a multiple of 2048 up to 2^24", who, (long long)V);
  return NAYLIS_OK;
}

int naylis_mom_xent_fwd(const void* logits, const int64_t* labels, float* loss_rows, float* lse, int64_t N, int64_t V,
                        int64_t ignore_index, void* stream) {
  int rc = check_xent(N, V, "mom_xent_fwd");
  if (rc || N == 0) return rc;
  if (!logits || !labels || !loss_rows || !lse) return fail(NAYLIS_ERR_ARG, "mom_xent_fwd: null pointer argument");
  if (!aligned16(logits)) return fail(NAYLIS_ERR_ARG, "mom_xent_fwd: logits must be 16-byte aligned");
  return hip_status(launch_xent(logits, labels, loss_rows, lse, nullptr, 0, nullptr, false, (long)N, (int)V,
                                (long)ignore_index, (hipStream_t)stream),
                    "mom_xent_fwd");
}

int naylis_mom_xent_bwd(const void* logits, const int64_t* labels, const float* lse, const float* grad_rows,
                        int64_t grad_stride, void* dlogits, int64_t N, int64_t V, int64_t ignore_index, void* stream) {
  int rc = check_xent(N, V, "mom_xent_bwd");
  if (rc || N == 0) return rc;
  if (grad_stride != 0 && grad_stride != 1)
    return fail(NAYLIS_ERR_ARG, "mom_xent_bwd: grad_stride %lld must be 0 or 1", (long long)grad_stride);
  if (!logits || !labels || !lse || !grad_rows || !dlogits)
    return fail(NAYLIS_ERR_ARG, "mom_xent_bwd: null pointer argument");
  if (!aligned16(logits) || !aligned16(dlogits))
    return fail(NAYLIS_ERR_ARG, "mom_xent_bwd: logits and dlogits must be 16-byte aligned");
  return hip_status(launch_xent(logits, labels, nullptr, const_cast<float*>(lse), grad_rows, (long)grad_stride,
                                dlogits, true, (long)N, (int)V, (long)ignore_index, (hipStream_t)stream),
                    "mom_xent_bwd");
}

size_t naylis_mom_router_stats_workspace_bytes(int64_t N, int64_t E) {
  if (N < 0 || N > ((int64_t)1 << 30) || E < 1 || E > NAYLIS_ROUTER_MAX_BLOCKS) return 0;
  return router_stats_ws_bytes((long)N, (int)E);
}

int naylis_mom_router_stats(const float* probs, const int32_t* top_idx, float* stats, void* workspace,
                            size_t workspace_bytes, int64_t N, int64_t E, int64_t top_k, void* stream) {
  if (N < 0 || N > ((int64_t)1 << 30))
    return fail(NAYLIS_ERR_ARG, "mom_router_stats: bad token count N=%lld", (long long)N);
  if (E < 1 || E > NAYLIS_ROUTER_MAX_BLOCKS)
    return fail(NAYLIS_ERR_ARG, "mom_router_stats: num_blocks %lld must be in [1, %d]", (long long)E,
                NAYLIS_ROUTER_MAX_BLOCKS);
  if (top_k < 1 || top_k > NAYLIS_MAX_TOPK || top_k > E)
    return fail(NAYLIS_ERR_ARG, "mom_router_stats: top_k %lld must be in [1, min(%d, num_blocks=%lld)]",
                (long long)top_k, NAYLIS_MAX_TOPK, (long long)E);
  if (!stats || !workspace || (N > 0 && (!probs || !top_idx)))
    return fail(NAYLIS_ERR_ARG, "mom_router_stats: null pointer argument");
  const size_t need = router_stats_ws_bytes((long)N, (int)E);
  if (workspace_bytes < need)
    return fail(NAYLIS_ERR_WORKSPACE, "mom_router_stats: workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, need);
  return hip_status(launch_router_stats(probs, top_idx, stats, workspace, (long)N, (int)E, (int)top_k,
                                        (hipStream_t)stream),
                    "mom_router_stats");
}

int naylis_mom_bank_kv_fwd(const void* slots, const void* w_k, const void* w_v, void* k_out, void* v_out, int64_t L,
                           int64_t D_in, int64_t D_out, void* stream) {
  if (L < 0 || D_in <= 0 || D_out <= 0 || L > NAYLIS_MAX_SLOTS || D_in > 65536 || D_out > 65536)
    return fail(NAYLIS_ERR_ARG, "mom_bank_kv: bad shape L=%lld D_in=%lld D_out=%lld", (long long)L,
                (long long)D_in, (long long)D_out);
  if (D_in % 8 != 0) return fail(NAYLIS_ERR_ARG, "mom_bank_kv: D_in (%lld) must be a multiple of 8", (long long)D_in);
  if (L == 0) return NAYLIS_OK;
  if (!slots || !w_k || !w_v || !k_out || !v_out) return fail(NAYLIS_ERR_ARG, "mom_bank_kv_fwd: null pointer argument");
  return hip_status(launch_bank_kv_fwd(slots, w_k, w_v, k_out, v_out, (int)L, (int)D_in, (int)D_out,
                                       (hipStream_t)stream),
                    "mom_bank_kv_fwd");
}

int naylis_mom_bank_kv_bwd(const void* slots, const void* w_k, const void* w_v, const void* dk, const void* dv,
                           void* d_slots, int slots_grad_dtype, void* dw_k, void* dw_v, int w_grad_dtype, int64_t L,
                           int64_t D_in, int64_t D_out, void* stream) {
  if (L < 0 || D_in <= 0 || D_out <= 0 || L > NAYLIS_MAX_SLOTS || D_in > 65536 || D_out > 65536)
    return fail(NAYLIS_ERR_ARG, "mom_bank_kv: bad shape L=%lld D_in=%lld D_out=%lld", (long long)L,
                (long long)D_in, (long long)D_out);
  if (D_in % 8 != 0 || D_out % 8 != 0)
    return fail(NAYLIS_ERR_ARG, "mom_bank_kv_bwd: D_in (%lld) and D_out (%lld) must be multiples of 8",
                (long long)D_in, (long long)D_out);
  int rc;
  if ((rc = check_dtype(slots_grad_dtype, "mom_bank_kv_bwd"))) return rc;
  if ((rc = check_dtype(w_grad_dtype, "mom_bank_kv_bwd"))) return rc;
  if (!w_k || !w_v || !dw_k || !dw_v) return fail(NAYLIS_ERR_ARG, "mom_bank_kv_bwd: null pointer argument");
  if (L > 0 && (!slots || !dk || !dv || !d_slots))
    return fail(NAYLIS_ERR_ARG, "mom_bank_kv_bwd: null pointer argument");
  return hip_status(launch_bank_kv_bwd(slots, w_k, w_v, dk, dv, d_slots, slots_grad_dtype == NAYLIS_DTYPE_F32, dw_k,
                                       dw_v, w_grad_dtype == NAYLIS_DTYPE_F32, (int)L, (int)D_in, (int)D_out,
                                       (hipStream_t)stream),
                    "mom_bank_kv_bwd");
}

static int check_bank_grouped(int64_t n, int64_t L, int64_t D_in, int64_t D_out, const char* what) {
  if (n < 1 || n > NAYLIS_BANK_GROUP_MAX_LAYERS)
    return fail(NAYLIS_ERR_ARG, "%s: n_layers (%lld) outside [1, %d]", what, (long long)n,
                NAYLIS_BANK_GROUP_MAX_LAYERS);
  if (L <= 0 || D_in <= 0 || D_out <= 0 || L > NAYLIS_MAX_SLOTS || D_in > 65536 || D_out > 65536)
    return fail(NAYLIS_ERR_ARG, "%s: bad shape L=%lld D_in=%lld D_out=%lld", what, (long long)L, (long long)D_in,
                (long long)D_out);
  if (!bank_grouped_ok((int)n, (int)L, (int)D_in, (int)D_out))
    return fail(NAYLIS_ERR_ARG, "%s: D_in (%lld) must be a multiple of 8 and D_out (%lld) of 64", what,
                (long long)D_in, (long long)D_out);
  return NAYLIS_OK;
}

static bool all_set(const void* const* p, int64_t n) {
  if (!p) return false;
  for (int64_t i = 0; i < n; ++i)
    if (!p[i]) return false;
  return true;
}

int naylis_mom_bank_kv_fwd_grouped(const void* slots, const void* const* w_k, const void* const* w_v,
                                   void* const* k_out, void* const* v_out, int64_t n_layers, int64_t L, int64_t D_in,
                                   int64_t D_out, void* stream) {
  int rc = check_bank_grouped(n_layers, L, D_in, D_out, "mom_bank_kv_fwd_grouped");
  if (rc) return rc;
  if (!slots || !all_set(w_k, n_layers) || !all_set(w_v, n_layers) || !all_set((const void* const*)k_out, n_layers) ||
      !all_set((const void* const*)v_out, n_layers))
    return fail(NAYLIS_ERR_ARG, "mom_bank_kv_fwd_grouped: null pointer argument");
  const hipError_t e = launch_bank_kv_fwd_grouped(slots, w_k, w_v, k_out, v_out, (int)n_layers, (int)L, (int)D_in,
                                                  (int)D_out, (hipStream_t)stream);
  if (e == hipErrorInvalidValue)
    return fail(NAYLIS_ERR_ARG, "mom_bank_kv_fwd_grouped: pointers must be 16-byte aligned");
  return hip_status(e, "mom_bank_kv_fwd_grouped");
}

size_t naylis_mom_bank_kv_bwd_grouped_workspace_bytes(int64_t n_layers, int64_t L, int64_t D_in, int64_t D_out) {
  if (check_bank_grouped(n_layers, L, D_in, D_out, "mom_bank_kv_bwd_grouped_workspace_bytes") != NAYLIS_OK) return 0;
  return bank_kv_bwd_grouped_ws_bytes((int)n_layers, (int)L, (int)D_in);
}

int naylis_mom_bank_kv_bwd_grouped(const void* slots, const void* const* w_k, const void* const* w_v,
                                   const void* const* dk, const void* const* dv, void* d_slots, int slots_grad_dtype,
                                   void* const* dw_k, void* const* dw_v, int w_grad_dtype, void* workspace,
                                   size_t workspace_bytes, int64_t n_layers, int64_t L, int64_t D_in, int64_t D_out,
                                   void* stream) {
  int rc = check_bank_grouped(n_layers, L, D_in, D_out, "mom_bank_kv_bwd_grouped");
  if (rc) return rc;
  if ((rc = check_dtype(slots_grad_dtype, "mom_bank_kv_bwd_grouped"))) return rc;
  if ((rc = check_dtype(w_grad_dtype, "mom_bank_kv_bwd_grouped"))) return rc;
  if (!slots || !d_slots || !all_set(w_k, n_layers) || !all_set(w_v, n_layers) || !all_set(dk, n_layers) ||
      !all_set(dv, n_layers) || !all_set((const void* const*)dw_k, n_layers) ||
      !all_set((const void* const*)dw_v, n_layers))
    return fail(NAYLIS_ERR_ARG, "mom_bank_kv_bwd_grouped: null pointer argument");
  const size_t need = bank_kv_bwd_grouped_ws_bytes((int)n_layers, (int)L, (int)D_in);
  if (!workspace || workspace_bytes < need)
    return fail(NAYLIS_ERR_WORKSPACE, "mom_bank_kv_bwd_grouped: workspace of %zu bytes, %zu needed", workspace_bytes,
                need);
  const hipError_t e = launch_bank_kv_bwd_grouped(
      slots, w_k, w_v, dk, dv, d_slots, slots_grad_dtype == NAYLIS_DTYPE_F32, dw_k, dw_v,
      w_grad_dtype == NAYLIS_DTYPE_F32, workspace, (int)n_layers, (int)L, (int)D_in, (int)D_out, (hipStream_t)stream);
  if (e == hipErrorInvalidValue)
    return fail(NAYLIS_ERR_ARG, "mom_bank_kv_bwd_grouped: pointers must be 16-byte aligned");
  return hip_status(e, "mom_bank_kv_bwd_grouped");
}

// ---------------------------------------------------- projection weight grad
static int wgrad_splits(int64_t N, int64_t D_in, int64_t D_out) {
  // enough workgroups for two per CU, each reducing at least 1024 tokens, as a power of two: the
  // token range then splits into equal whole K tiles (3, 5 or 6 splits measure 10-25 % slower than
  // the neighbouring power of two at 16384 tokens)
  const int64_t tiles = ((D_out + 127) / 128) * ((D_in + 127) / 128);
  const int64_t want = (512 + tiles - 1) / tiles;
  int64_t s = 1;
  while (s < want && s < 64 && 2 * s * 1024 <= N) s *= 2;
  // ... unless its last round of workgroups would be less than a quarter full:
  // then the largest count that fits one round, if it still splits three ways
  // (1536 x 1536 at 16384 tokens: 4 splits, 576 workgroups, 126 us; 3 splits,
  // 432 workgroups, 110 us)
  const int64_t slots = 512;
  if (s > 1 && (tiles * s) % slots != 0 && (tiles * s) % slots < slots / 4) {
    const int64_t one = slots / tiles;
    if (one >= 3 && one < s && one * 1024 <= N) s = one;
  }
  return (int)s;
}

static int check_wgrad_dims(int64_t N, int64_t D_in, int64_t D_out) {
  if (N < 0 || D_in <= 0 || D_out <= 0 || N > ((int64_t)1 << 30) || D_in > 65536 || D_out > 65536)
    return fail(NAYLIS_ERR_ARG, "linear_wgrad: bad shape N=%lld D_in=%lld D_out=%lld", (long long)N, (long long)D_in,
                (long long)D_out);
  if (N % 8 || D_in % 8 || D_out % 8)
    return fail(NAYLIS_ERR_ARG, "linear_wgrad: N (%lld), D_in (%lld) and D_out (%lld) must be multiples of 8",
                (long long)N, (long long)D_in, (long long)D_out);
  return NAYLIS_OK;
}

size_t naylis_mom_linear_wgrad_workspace_bytes(int64_t N, int64_t D_in, int64_t D_out) {
  if (check_wgrad_dims(N, D_in, D_out) != NAYLIS_OK) return 0;
  const size_t b = gemm_ws_bytes(1, (int)D_out, (int)D_in, wgrad_splits(N, D_in, D_out));
  return b ? b : 256;
}

int naylis_mom_linear_wgrad(const void* x, const void* dy, void* dw, int dw_dtype, void* workspace,
                            size_t workspace_bytes, int64_t N, int64_t D_in, int64_t D_out, void* stream) {
  int rc = check_wgrad_dims(N, D_in, D_out);
  if (rc) return rc;
  if ((rc = check_dtype(dw_dtype, "linear_wgrad"))) return rc;
  if (!dw || (N > 0 && (!x || !dy))) return fail(NAYLIS_ERR_ARG, "linear_wgrad: null pointer argument");
  const int splits = wgrad_splits(N, D_in, D_out);
  const size_t need = gemm_ws_bytes(1, (int)D_out, (int)D_in, splits);
  if (need && (!workspace || workspace_bytes < need))
    return fail(NAYLIS_ERR_WORKSPACE, "linear_wgrad: workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, need);
  if (N == 0)  // no tokens: the gradient is zero
    return hip_status(launch_zero(dw, (size_t)D_out * D_in * (dw_dtype == NAYLIS_DTYPE_F32 ? 4 : 2),
                                  (hipStream_t)stream),
                      "linear_wgrad");
  GemmLaunch g{};
  g.njobs = 1;
  g.M = (int)D_out;
  g.N = (int)D_in;
  g.K = g.K1 = (int)N;
  g.out = dw_dtype == NAYLIS_DTYPE_F32 ? kGemmOutF32 : kGemmOutBF16;
  g.splits = splits;
  g.ws = workspace;
  g.job[0].a = GemmOp{dy, nullptr, D_out, false};  // A(o, t) = dy[t][o]
  g.job[0].b = GemmOp{x, nullptr, D_in, false};    // B(t, i) = x[t][i]
  g.job[0].c = dw;
  g.job[0].ldc = D_in;
  if (!gemm_supported(g))
    return fail(NAYLIS_ERR_ARG, "linear_wgrad: needs 16-byte aligned pointers and N * max(D_in, D_out) < 2^30");
  return hip_status(launch_gemm(g, "linear_wgrad", (hipStream_t)stream), "linear_wgrad");
}

// The gated weight gradient: at least two K splits, so the gate epilogue of
// the split-K reduction always runs.
static int gated_wgrad_splits(int64_t N, int64_t D_in, int64_t D_out) {
  return std::max(2, wgrad_splits(N, D_in, D_out));
}

static size_t gated_wgrad_part_off(int64_t N, int64_t D_in, int64_t D_out) {
  return (gemm_ws_bytes(1, (int)D_out, (int)D_in, gated_wgrad_splits(N, D_in, D_out)) + 255) & ~(size_t)255;
}

size_t naylis_mom_gated_wgrad_workspace_bytes(int64_t N, int64_t D_in, int64_t D_out) {
  if (check_wgrad_dims(N, D_in, D_out) != NAYLIS_OK) return 0;
  return gated_wgrad_part_off(N, D_in, D_out) + (size_t)std::max(1, gemm_gate_parts((int)D_out, (int)D_in)) * 4;
}

int naylis_mom_gated_wgrad(const void* x, const void* dy, const void* w, const float* s, void* dw, float* ds,
                           void* workspace, size_t workspace_bytes, int64_t N, int64_t D_in, int64_t D_out,
                           void* stream) {
  int rc = check_wgrad_dims(N, D_in, D_out);
  if (rc) return rc;
  if (!dw || !ds || !w || !s || (N > 0 && (!x || !dy)))
    return fail(NAYLIS_ERR_ARG, "gated_wgrad: null pointer argument");
  const size_t need = naylis_mom_gated_wgrad_workspace_bytes(N, D_in, D_out);
  if (!workspace || workspace_bytes < need)
    return fail(NAYLIS_ERR_WORKSPACE, "gated_wgrad: workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, need);
  if ((((uintptr_t)w | (uintptr_t)dw | (uintptr_t)workspace) & 15) != 0)
    return fail(NAYLIS_ERR_ARG, "gated_wgrad: w, dw and the workspace must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  if (N == 0) {  // no tokens: both gradients are zero
    hipError_t e = launch_zero(dw, (size_t)D_out * D_in * 2, st);
    if (e == hipSuccess) e = launch_zero(ds, sizeof(float), st);
    return hip_status(e, "gated_wgrad");
  }
  GemmLaunch g{};
  g.njobs = 1;
  g.M = (int)D_out;
  g.N = (int)D_in;
  g.K = g.K1 = (int)N;
  g.out = kGemmOutBF16;
  g.splits = gated_wgrad_splits(N, D_in, D_out);
  g.ws = workspace;
  g.job[0].a = GemmOp{dy, nullptr, D_out, false};  // A(o, t) = dy[t][o]
  g.job[0].b = GemmOp{x, nullptr, D_in, false};    // B(t, i) = x[t][i]
  g.job[0].c = dw;
  g.job[0].ldc = D_in;
  float* part = (float*)((char*)workspace + gated_wgrad_part_off(N, D_in, D_out));
  g.gate_w = w;
  g.gate_s = s;
  g.gate_part = part;
  if (!gemm_supported(g))
    return fail(NAYLIS_ERR_ARG, "gated_wgrad: needs 16-byte aligned pointers and N * max(D_in, D_out) < 2^30");
  hipError_t e = launch_gemm(g, "linear_wgrad", st);
  if (e == hipSuccess) e = launch_rezero_reduce(part, gemm_gate_parts((int)D_out, (int)D_in), ds, st);
  return hip_status(e, "gated_wgrad");
}

// -------------------------------------------------------------------- ReZero
size_t naylis_mom_rezero_workspace_bytes(int64_t n) {
  if (n < 0) return 0;
  return rezero_ws_bytes((long)n);
}

int naylis_mom_rezero_fwd(const void* z, int z_dtype, const float* s, float* y, int64_t n, void* stream) {
  int rc;
  if (n < 0) return fail(NAYLIS_ERR_ARG, "rezero_fwd: negative size %lld", (long long)n);
  if ((rc = check_dtype(z_dtype, "rezero_fwd"))) return rc;
  if (n == 0) return NAYLIS_OK;
  if (!z || !s || !y) return fail(NAYLIS_ERR_ARG, "rezero_fwd: null pointer argument");
  return hip_status(launch_rezero_fwd(z, z_dtype == NAYLIS_DTYPE_BF16, s, y, (long)n, (hipStream_t)stream),
                    "rezero_fwd");
}

int naylis_mom_rezero_scale(const void* x, int x_dtype, const float* s, void* y, int y_dtype, int64_t n, void* stream) {
  int rc;
  if (n < 0) return fail(NAYLIS_ERR_ARG, "rezero_scale: negative size %lld", (long long)n);
  if ((rc = check_dtype(x_dtype, "rezero_scale"))) return rc;
  if ((rc = check_dtype(y_dtype, "rezero_scale"))) return rc;
  if (n == 0) return NAYLIS_OK;
  if (!x || !s || !y) return fail(NAYLIS_ERR_ARG, "rezero_scale: null pointer argument");
  return hip_status(launch_rezero_scale(x, x_dtype == NAYLIS_DTYPE_BF16, s, y, y_dtype == NAYLIS_DTYPE_BF16, (long)n,
                                        (hipStream_t)stream),
                    "rezero_scale");
}

int naylis_mom_rezero_bwd(const void* dy, int dy_dtype, const void* z, int z_dtype, const float* s, void* dz, float* ds,
                          void* workspace, size_t workspace_bytes, int64_t n, void* stream) {
  int rc;
  if (n < 0) return fail(NAYLIS_ERR_ARG, "rezero_bwd: negative size %lld", (long long)n);
  if ((rc = check_dtype(dy_dtype, "rezero_bwd"))) return rc;
  if ((rc = check_dtype(z_dtype, "rezero_bwd"))) return rc;
  if (!s || !ds || (n > 0 && (!dy || !z))) return fail(NAYLIS_ERR_ARG, "rezero_bwd: null pointer argument");
  const size_t need = rezero_ws_bytes((long)n);
  if (!workspace || workspace_bytes < need)
    return fail(NAYLIS_ERR_WORKSPACE, "rezero_bwd: workspace of %zu bytes is smaller than the %zu required",
                workspace_bytes, need);
  return hip_status(launch_rezero_bwd(dy, dy_dtype == NAYLIS_DTYPE_BF16, z, z_dtype == NAYLIS_DTYPE_BF16, s, dz, ds,
                                      workspace, (long)n, (hipStream_t)stream),
                    "rezero_bwd");
}

}  // extern "C"

// ---------------------------------------------------------------- decode step
namespace {

bool overlap(const void* a, const void* b, size_t bytes) {
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + bytes && y < x + bytes;
}

}  // namespace

extern "C" {

int naylis_mom_bank_quant_fp8(const void* k, const void* v, uint8_t* k8, uint8_t* v8, float* k_scale, float* v_scale,
                              int64_t L, int64_t D, void* stream) {
  if (L < 0 || D <= 0 || L > NAYLIS_MAX_SLOTS || D > 65536)
    return fail(NAYLIS_ERR_ARG, "bank_quant_fp8: bad shape L=%lld D=%lld", (long long)L, (long long)D);
  if (L == 0) return NAYLIS_OK;
  if (!k || !v || !k8 || !v8 || !k_scale || !v_scale)
    return fail(NAYLIS_ERR_ARG, "bank_quant_fp8: null pointer argument");
  return hip_status(launch_bank_quant_fp8(k, v, k8, v8, k_scale, v_scale, (int)L, (int)D, (hipStream_t)stream),
                    "bank_quant_fp8");
}

int naylis_mom_decode_step(const double* state_in, double* state_out, const int32_t* t_prev, const void* x_new,
                           int x_dtype, const float* w_down, const float* w_up, const void* q_new, const uint8_t* k8,
                           const uint8_t* v8, const float* k_scale, const float* v_scale, void* out, int32_t* top_idx,
                           float* top_gates, int64_t B, int64_t D, int64_t H, int64_t R, int64_t E, int64_t block_size,
                           int64_t top_k, void* stream) {
  int rc;
  if ((rc = check_dtype(x_dtype, "decode_step"))) return rc;
  if (B < 0 || B > 65535 || H <= 0 || D <= 0 || D % H != 0)
    return fail(NAYLIS_ERR_ARG, "decode_step: bad shape B=%lld D=%lld H=%lld", (long long)B, (long long)D,
                (long long)H);
  const int64_t hd = D / H;
  if (hd != 32 && hd != 64 && hd != 128)
    return fail(NAYLIS_ERR_ARG, "decode_step: head_dim %lld must be 32, 64 or 128", (long long)hd);
  if (D > kDecodeMaxD) return fail(NAYLIS_ERR_ARG, "decode_step: D %lld exceeds %d", (long long)D, kDecodeMaxD);
  if (R <= 0 || R > kDecodeMaxRank)
    return fail(NAYLIS_ERR_ARG, "decode_step: router rank %lld must be in [1, %d]", (long long)R, kDecodeMaxRank);
  if (E <= 0 || E > kDecodeMaxExperts)
    return fail(NAYLIS_ERR_ARG, "decode_step: num_blocks %lld must be in [1, %d]", (long long)E, kDecodeMaxExperts);
  if (top_k < 1 || top_k > NAYLIS_MAX_TOPK || top_k > E)
    return fail(NAYLIS_ERR_ARG, "decode_step: top_k %lld must be in [1, min(%d, num_blocks)]", (long long)top_k,
                NAYLIS_MAX_TOPK);
  if (block_size <= 0 || E * block_size > NAYLIS_MAX_SLOTS)
    return fail(NAYLIS_ERR_ARG, "decode_step: num_blocks * block_size (%lld) must be in [1, %d]",
                (long long)(E * block_size), NAYLIS_MAX_SLOTS);
  if (B == 0) return NAYLIS_OK;
  if (!state_in || !state_out || !t_prev || !x_new || !w_down || !w_up || !q_new || !k8 || !v8 || !k_scale ||
      !v_scale || !out || !top_idx || !top_gates)
    return fail(NAYLIS_ERR_ARG, "decode_step: null pointer argument");
  if (!aligned16(w_down) || !aligned16(q_new) || !aligned16(k8) || !aligned16(v8))
    return fail(NAYLIS_ERR_ARG, "decode_step: w_down, q_new, k8 and v8 must be 16-byte aligned");
  if (overlap(state_in, state_out, (size_t)B * D * sizeof(double)))
    return fail(NAYLIS_ERR_ARG, "decode_step: state_in and state_out overlap");
  DecodeDims d{(int)B, (int)D, (int)H, (int)hd, (int)R, (int)E, (int)block_size, (int)top_k};
  return hip_status(launch_decode_step(state_in, state_out, t_prev, x_new, x_dtype == NAYLIS_DTYPE_F32, w_down, w_up,
                                       q_new, k8, v8, k_scale, v_scale, out, top_idx, top_gates, d,
                                       (hipStream_t)stream),
                    "decode_step");
}

}  // extern "C"
