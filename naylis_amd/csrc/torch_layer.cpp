// Host side of the fused MoM layer node (model.py:189-276) in C++: a torch
// extension over the C ABI of libnaylis_mom.so.  layer_fwd / layer_bwd run
// the forward and the backward of mom_kernels.hip_layer.MomLayerFunction --
// router, bank K/V, q projection, token order, gated read, o projection with
// the folded ReZero gate, and their gradients -- as one call each from
// Python instead of about fifteen ctypes and torch calls.  They make the same
// library calls in the same order, with the same allocations and torch GEMMs
// (hipBLASLt through at::mm / at::linear on torch's current stream), so their
// results are bitwise those of the Python node.
//
// MomLayerNode is the same node as a C++ autograd function: its forward
// calls layer_fwd and saves what the Python node saves, its backward calls
// layer_bwd, so the autograd engine runs the backward without Python.
//
// The library's symbols are not linked here: libnaylis_mom.so is loaded with
// global visibility before this module (naylis_amd/_lib.py), so these calls
// bind to that one instance (its timing state and scratch arrays included).
#include <torch/extension.h>

#include <algorithm>
#include <vector>

#include "../../include/naylis_mom.h"

namespace {

constexpr int kF32 = 0, kBF16 = 1;

void check(int rc, const char* what) {
  if (rc != NAYLIS_OK) {
    const char* msg = naylis_mom_last_error();
    TORCH_CHECK(false, "naylis_mom ", what, " failed (status ", rc, "): ", msg ? msg : "");
  }
}

at::Tensor workspace(size_t nbytes, const at::Tensor& like) {
  return at::empty({(int64_t)std::max<size_t>(nbytes, 1)}, like.options().dtype(at::kByte));
}

int dtype_code(const at::Tensor& t) { return t.scalar_type() == at::kBFloat16 ? kBF16 : kF32; }

void* opt_ptr(const c10::optional<at::Tensor>& t) { return t.has_value() && t->defined() ? t->data_ptr() : nullptr; }

// dW = dy^T xin over all rows: the library's split-K GEMM when N, D_in, D_out
// are multiples of 8, else torch's product (the hip_linear.library_wgrad rule)
at::Tensor library_wgrad(const at::Tensor& xin, const at::Tensor& dy, at::ScalarType dtype, void* st) {
  const int64_t N = xin.size(0), D_in = xin.size(1), D_out = dy.size(1);
  if (N % 8 || D_in % 8 || D_out % 8) {
    if (dtype == at::kFloat) return at::mm(dy.t(), xin, at::kFloat);
    return at::mm(dy.t(), xin).to(dtype);
  }
  at::Tensor ws = workspace(naylis_mom_linear_wgrad_workspace_bytes(N, D_in, D_out), xin);
  at::Tensor dw = at::empty({D_out, D_in}, xin.options().dtype(dtype));
  check(naylis_mom_linear_wgrad(xin.data_ptr(), dy.data_ptr(), dw.data_ptr(), dtype == at::kBFloat16 ? kBF16 : kF32,
                                ws.data_ptr(), ws.numel(), N, D_in, D_out, st),
        "linear_wgrad");
  return dw;
}

}  // namespace

// Returns [y, probs, top_idx, act, gates, slots, k, v, q, order, out, side,
// lse, w_os]; slots is undefined (None) with an external bank, side when the
// read keeps no side buffer.
std::vector<at::Tensor> layer_fwd(at::Tensor x, c10::optional<at::Tensor> m_blocks, at::Tensor w_down,
                                  at::Tensor w_up, at::Tensor w_q, at::Tensor w_k, at::Tensor w_v, at::Tensor w_o,
                                  at::Tensor scale, c10::optional<at::Tensor> noise, double noise_scale,
                                  int64_t n_heads, int64_t num_blocks, int64_t block_size, int64_t top_k,
                                  int64_t noise_kind, c10::optional<at::Tensor> k_ext,
                                  c10::optional<at::Tensor> v_ext, int64_t stream) {
  at::DeviceGuard guard(x.device());
  void* st = reinterpret_cast<void*>(stream);
  x = x.contiguous();
  const int64_t B = x.size(0), T = x.size(1), D = x.size(2);
  const int64_t R = w_down.size(0), E = w_up.size(0), H = n_heads, HD = D / n_heads;
  const auto f32 = x.options().dtype(at::kFloat);
  // ---- router (model.py:169-220)
  at::Tensor logits = at::empty({B, T, E}, f32), probs = at::empty({B, T, E}, f32);
  at::Tensor top_idx = at::empty({B, T, top_k}, x.options().dtype(at::kInt));
  at::Tensor gates = at::empty({B, T, top_k}, f32), act = at::empty({B, T, R}, f32);
  {
    at::Tensor rws = workspace(naylis_mom_router_workspace_bytes(B, T, D, R, E, top_k), x);
    check(naylis_mom_router_fwd(x.data_ptr(), kBF16, w_down.data_ptr<float>(), w_up.data_ptr<float>(),
                                static_cast<const float*>(opt_ptr(noise)), (int)noise_kind, (float)noise_scale,
                                logits.data_ptr<float>(), probs.data_ptr<float>(), top_idx.data_ptr<int32_t>(),
                                gates.data_ptr<float>(), act.data_ptr<float>(), nullptr, rws.data_ptr(), rws.numel(),
                                B, T, D, R, E, top_k, st),
          "router_fwd");
  }
  // ---- bank K/V (model.py:253-256), unless the caller projected the bank
  at::Tensor slots, k, v;
  if (!k_ext.has_value()) {
    slots = m_blocks->reshape({-1, D}).to(at::kBFloat16).contiguous();
    const int64_t L = slots.size(0);
    k = at::empty({L, D}, x.options().dtype(at::kBFloat16));
    v = at::empty({L, D}, x.options().dtype(at::kBFloat16));
    check(naylis_mom_bank_kv_fwd(slots.data_ptr(), w_k.data_ptr(), w_v.data_ptr(), k.data_ptr(), v.data_ptr(), L, D,
                                 D, st),
          "bank_kv_fwd");
  } else {
    k = *k_ext;
    v = *v_ext;
  }
  // ---- q projection, token order, gated read (model.py:251, 258-276)
  at::Tensor q = at::linear(x, w_q);
  const int64_t words = naylis_mom_read_order_words(B, T, num_blocks, top_k);
  if (words <= 0) check(NAYLIS_ERR_ARG, "read_order_words");
  at::Tensor order = at::empty({words}, x.options().dtype(at::kInt));
  {
    at::Tensor ows = workspace(naylis_mom_read_order_workspace_bytes(B, T, num_blocks, top_k), x);
    check(naylis_mom_read_order(top_idx.data_ptr<int32_t>(), order.data_ptr<int32_t>(), ows.data_ptr(), ows.numel(),
                                B, T, num_blocks, top_k, st),
          "read_order");
  }
  at::Tensor out = at::empty_like(q);
  at::Tensor side;
  const size_t side_bytes = naylis_mom_read_side_bytes(B, T, H, HD, num_blocks, block_size, top_k);
  if (side_bytes > 0) side = at::empty({(int64_t)side_bytes}, x.options().dtype(at::kByte));
  at::Tensor lse = at::empty({H, B, T}, f32);
  check(naylis_mom_read_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), top_idx.data_ptr<int32_t>(),
                            gates.data_ptr<float>(), order.data_ptr<int32_t>(), out.data_ptr(),
                            side.defined() ? side.data_ptr() : nullptr, lse.data_ptr<float>(), nullptr, 0, B, T, H, HD,
                            num_blocks, block_size, top_k, st),
        "read_fwd");
  // ---- o projection with the ReZero gate folded into the weight (model.py:251, 239)
  at::Tensor w_os = at::empty_like(w_o);
  check(naylis_mom_rezero_scale(w_o.data_ptr(), dtype_code(w_o), scale.data_ptr<float>(), w_os.data_ptr(),
                                dtype_code(w_os), w_o.numel(), st),
        "rezero_scale");
  at::Tensor y = at::mm(out.view({B * T, D}), w_os.t(), at::kFloat).view({B, T, D});
  return {y, probs, top_idx, act, gates, slots, k, v, q, order, out, side, lse, w_os};
}

// Returns [dx, d_m, dw_down, dw_up, dw_q, dw_k, dw_v, dw_o, ds, dk_ext,
// dv_ext]; with an external bank d_m, dw_k, dw_v are undefined and dk_ext,
// dv_ext the bank's K / V gradients, else the reverse.
std::vector<at::Tensor> layer_bwd(c10::optional<at::Tensor> dy, c10::optional<at::Tensor> d_probs, at::Tensor x,
                                  c10::optional<at::Tensor> slots, at::Tensor w_down, at::Tensor w_up,
                                  at::Tensor w_q, at::Tensor w_k, at::Tensor w_v, at::Tensor w_o, at::Tensor scale,
                                  at::Tensor act, at::Tensor probs, at::Tensor top_idx, at::Tensor gates,
                                  at::Tensor k, at::Tensor v, at::Tensor q, at::Tensor order, at::Tensor out,
                                  c10::optional<at::Tensor> side, at::Tensor lse, at::Tensor w_os, int64_t n_heads,
                                  int64_t num_blocks, int64_t block_size, int64_t top_k, bool external_bank,
                                  std::vector<int64_t> m_shape, bool m_bf16, int64_t stream) {
  at::DeviceGuard guard(x.device());
  void* st = reinterpret_cast<void*>(stream);
  const int64_t B = x.size(0), T = x.size(1), D = x.size(2);
  const int64_t R = w_down.size(0), E = w_up.size(0), H = n_heads, HD = D / n_heads, L = k.size(0), N = B * T;
  const auto f32 = x.options().dtype(at::kFloat);
  // ---- o projection with the folded gate: d out, dW_o, ds
  at::Tensor dy_t = dy.has_value() && dy->defined() ? *dy : at::zeros({B, T, D}, x.options().dtype(at::kBFloat16));
  at::Tensor dy2 = dy_t.reshape({N, D}).to(at::kBFloat16).contiguous();
  at::Tensor out2 = out.view({N, D});
  at::Tensor dout2 = at::mm(dy2, w_os);
  const int64_t D_in = out2.size(1), D_out = dy2.size(1);
  at::Tensor dw_o = at::empty_like(w_o), ds = at::empty({1}, f32);
  if (out2.scalar_type() == at::kBFloat16 && w_o.scalar_type() == at::kBFloat16 && w_o.is_contiguous() &&
      out2.is_contiguous() && N % 8 == 0 && D_in % 8 == 0 && D_out % 8 == 0) {
    at::Tensor ws = workspace(naylis_mom_gated_wgrad_workspace_bytes(N, D_in, D_out), x);
    check(naylis_mom_gated_wgrad(out2.data_ptr(), dy2.data_ptr(), w_o.data_ptr(), scale.data_ptr<float>(),
                                 dw_o.data_ptr(), ds.data_ptr<float>(), ws.data_ptr(), ws.numel(), N, D_in, D_out, st),
          "gated_wgrad");
  } else {
    at::Tensor dw_s = library_wgrad(out2, dy2, at::kFloat, st);
    at::Tensor ws = workspace(naylis_mom_rezero_workspace_bytes(w_o.numel()), x);
    check(naylis_mom_rezero_bwd(dw_s.data_ptr(), dtype_code(dw_s), w_o.data_ptr(), dtype_code(w_o),
                                scale.data_ptr<float>(), dw_o.data_ptr(), ds.data_ptr<float>(), ws.data_ptr(),
                                ws.numel(), w_o.numel(), st),
          "rezero_bwd");
  }
  // ---- gated read
  at::Tensor dq = at::empty_like(q), dk = at::empty_like(k), dv = at::empty_like(v), dgates = at::empty_like(gates);
  {
    const size_t nbytes = naylis_mom_read_workspace_bytes(B, T, H, HD, num_blocks, block_size, top_k);
    if (nbytes == 0) check(NAYLIS_ERR_ARG, "read_workspace_bytes");
    at::Tensor rws = workspace(nbytes, x);
    check(naylis_mom_read_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), top_idx.data_ptr<int32_t>(),
                              gates.data_ptr<float>(), order.data_ptr<int32_t>(), out.data_ptr(), opt_ptr(side),
                              lse.data_ptr<float>(), dout2.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                              dgates.data_ptr<float>(), rws.data_ptr(), rws.numel(), B, T, H, HD, num_blocks,
                              block_size, top_k, st),
          "read_bwd");
  }
  dout2 = at::Tensor();
  // ---- bank K/V (the caller's grouped node takes dK, dV when it projected the bank)
  at::Tensor d_m, dw_k, dw_v, dk_ext, dv_ext;
  if (external_bank) {
    dk_ext = dk;
    dv_ext = dv;
  } else {
    at::Tensor d_slots = at::empty({L, D}, x.options().dtype(m_bf16 ? at::kBFloat16 : at::kFloat));
    dw_k = at::empty_like(w_k);
    dw_v = at::empty_like(w_v);
    check(naylis_mom_bank_kv_bwd(slots->data_ptr(), w_k.data_ptr(), w_v.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                 d_slots.data_ptr(), m_bf16 ? kBF16 : kF32, dw_k.data_ptr(), dw_v.data_ptr(), kBF16,
                                 L, D, D, st),
          "bank_kv_bwd");
    d_m = d_slots.view(m_shape);
  }
  // ---- q projection: dx = dq W_q (the router adds its part below), dW_q = dq^T x
  at::Tensor dq2 = dq.view({N, D});
  at::Tensor dx = at::mm(dq2, w_q).view({B, T, D});
  at::Tensor dw_q = library_wgrad(x.view({N, D}), dq2, w_q.scalar_type(), st);
  // ---- router, accumulating into dx; d_probs as one row with stride 0 when it
  // is an expanded row, else dense (the hip_router.d_probs_arg rule)
  at::Tensor dp;
  int64_t dp_stride = E;
  if (d_probs.has_value() && d_probs->defined()) {
    const at::Tensor& g = *d_probs;
    bool row = g.scalar_type() == at::kFloat && g.stride(-1) == 1;
    for (int64_t i = 0; row && i + 1 < g.dim(); ++i) row = g.stride(i) == 0;
    if (row) {
      dp = g;
      dp_stride = 0;
    } else {
      dp = g.to(at::kFloat).contiguous();
    }
  }
  at::Tensor dw_down = at::empty({R, D}, f32), dw_up = at::empty({E, R}, f32);
  {
    at::Tensor rws = workspace(naylis_mom_router_workspace_bytes(B, T, D, R, E, top_k), x);
    check(naylis_mom_router_bwd(x.data_ptr(), kBF16, w_down.data_ptr<float>(), w_up.data_ptr<float>(),
                                act.data_ptr<float>(), probs.data_ptr<float>(), top_idx.data_ptr<int32_t>(),
                                gates.data_ptr<float>(), dgates.data_ptr<float>(),
                                dp.defined() ? dp.data_ptr<float>() : nullptr, dp_stride, nullptr, dx.data_ptr(), 1,
                                dw_down.data_ptr<float>(), dw_up.data_ptr<float>(), rws.data_ptr(), rws.numel(), B,
                                T, D, R, E, top_k, st),
          "router_bwd");
  }
  return {dx, d_m, dw_down, dw_up, dw_q, dw_k, dw_v, dw_o, ds, dk_ext, dv_ext};
}

namespace {

c10::optional<at::Tensor> opt(const at::Tensor& t) {
  return t.defined() ? c10::optional<at::Tensor>(t) : c10::nullopt;
}

// Inputs as MomLayerFunction.forward takes them; the autograd function takes
// only defined tensors, so an absent noise draw is passed as x with
// has_noise false, and the bank (m_blocks) or the external K / V that the
// call does not use likewise (external tells which); no gradient flows to
// those placeholders.  Outputs y, probs, top_idx.
struct MomLayerNode : public torch::autograd::Function<MomLayerNode> {
  static torch::autograd::variable_list forward(torch::autograd::AutogradContext* ctx, at::Tensor x,
                                                at::Tensor m_blocks, at::Tensor w_down, at::Tensor w_up,
                                                at::Tensor w_q, at::Tensor w_k, at::Tensor w_v, at::Tensor w_o,
                                                at::Tensor scale, at::Tensor noise, bool has_noise,
                                                double noise_scale, int64_t n_heads, int64_t num_blocks,
                                                int64_t block_size, int64_t top_k, int64_t noise_kind,
                                                at::Tensor k_ext, at::Tensor v_ext, bool external, int64_t stream) {
    const at::Tensor none;
    x = x.contiguous();
    std::vector<at::Tensor> r =
        layer_fwd(x, external ? c10::nullopt : opt(m_blocks), w_down, w_up, w_q, w_k, w_v, w_o, scale,
                  has_noise ? opt(noise) : c10::nullopt, noise_scale, n_heads, num_blocks, block_size, top_k,
                  noise_kind, external ? opt(k_ext) : c10::nullopt, external ? opt(v_ext) : c10::nullopt, stream);
    // r: y, probs, top_idx, act, gates, slots, k, v, q, order, out, side, lse, w_os
    ctx->save_for_backward({x, r[5], w_down, w_up, w_q, w_k, w_v, w_o, scale, r[3], r[1], r[2], r[4], r[6], r[7],
                            r[8], r[9], r[10], r[11], r[12], r[13]});
    ctx->saved_data["geom"] = std::vector<int64_t>{n_heads, num_blocks, block_size, top_k, stream};
    ctx->saved_data["external"] = external;
    ctx->saved_data["m_shape"] = external ? std::vector<int64_t>{} : m_blocks.sizes().vec();
    ctx->saved_data["m_bf16"] = !external && m_blocks.scalar_type() == at::kBFloat16;
    ctx->mark_non_differentiable({r[2]});
    ctx->set_materialize_grads(false);
    return {r[0], r[1], r[2]};
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    const torch::autograd::variable_list s = ctx->get_saved_variables();
    const std::vector<int64_t> geom = ctx->saved_data["geom"].toIntVector();
    const bool external = ctx->saved_data["external"].toBool();
    std::vector<int64_t> m_shape = ctx->saved_data["m_shape"].toIntVector();
    const bool m_bf16 = ctx->saved_data["m_bf16"].toBool();
    // s: x, slots, w_down, w_up, w_q, w_k, w_v, w_o, scale, act, probs, top_idx, gates, k, v, q, order,
    // out, side, lse, w_os
    std::vector<at::Tensor> r =
        layer_bwd(opt(grads[0]), opt(grads[1]), s[0], opt(s[1]), s[2], s[3], s[4], s[5], s[6], s[7], s[8], s[9],
                  s[10], s[11], s[12], s[13], s[14], s[15], s[16], s[17], opt(s[18]), s[19], s[20], geom[0],
                  geom[1], geom[2], geom[3], external, m_shape, m_bf16, geom[4]);
    // r: dx, d_m, dw_down, dw_up, dw_q, dw_k, dw_v, dw_o, ds, dk_ext, dv_ext
    const at::Tensor none;
    return {r[0], r[1],  r[2], r[3], r[4], r[5], r[6], r[7], r[8].view(s[8].sizes()), none, none,
            none, none, none, none, none, none, r[9], r[10], none, none};
  }
};

std::vector<at::Tensor> mom_layer_node(at::Tensor x, c10::optional<at::Tensor> m_blocks, at::Tensor w_down,
                                       at::Tensor w_up, at::Tensor w_q, at::Tensor w_k, at::Tensor w_v,
                                       at::Tensor w_o, at::Tensor scale, c10::optional<at::Tensor> noise,
                                       double noise_scale, int64_t n_heads, int64_t num_blocks, int64_t block_size,
                                       int64_t top_k, int64_t noise_kind, c10::optional<at::Tensor> k_ext,
                                       c10::optional<at::Tensor> v_ext, int64_t stream) {
  const bool external = k_ext.has_value() && k_ext->defined();
  const bool has_noise = noise.has_value() && noise->defined();
  TORCH_CHECK(external || (m_blocks.has_value() && m_blocks->defined()), "mom_layer: no bank and no external K / V");
  TORCH_CHECK(!external || (v_ext.has_value() && v_ext->defined()), "mom_layer: external K without V");
  return MomLayerNode::apply(x, external ? x : *m_blocks, w_down, w_up, w_q, w_k, w_v, w_o, scale,
                             has_noise ? *noise : x, has_noise, noise_scale, n_heads, num_blocks, block_size, top_k,
                             noise_kind, external ? *k_ext : x, external ? *v_ext : x, external, stream);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "Fused MoM layer node over the C ABI of libnaylis_mom.so";
  m.def("layer_fwd", &layer_fwd, "MoM layer forward (router, bank K/V, q projection, read, o projection)");
  m.def("layer_bwd", &layer_bwd, "MoM layer backward (the forward's gradients in one fixed order)");
  m.def("mom_layer", &mom_layer_node,
        "The fused layer node as a C++ autograd function: returns (y, probs, top_idx) with its backward attached");
}
