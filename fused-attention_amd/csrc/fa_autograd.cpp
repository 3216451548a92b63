// fa_autograd.cpp - the autograd op behind fused_attention_autograd and
// fused_gqa_attention_autograd, in C++ over the C ABI of libfa.so.
//
// Same contract as the Python autograd.Function it stands in for
// (attention/backward/fused_backward.py:151-206 of the reference: FusedAttentionFn,
// whose forward runs the fused kernel with the log-sum-exp output and saves
// Q, K, V, O and LSE, and whose backward runs the two gradient kernels):
//   forward : O, LSE = fa_fwd(Q, K, V); saves Q, K, V, O, LSE and the tiles
//   backward: dQ, dK, dV = fa_bwd_gqa(Q, K, V, O, dO, LSE) with its workspace
//             taken from torch's caching allocator on the launch stream
// H_kv may divide H (GQA/MQA): fa_bwd_gqa sums dK and dV over each K/V head's
// query heads.  The results are those of the Python Function bitwise (the same
// entry points with the same arguments); what changes is the host path: the
// autograd engine runs this node's backward without calling back into Python,
// and the step makes no ctypes calls.  Short sequences are bound by that path
// (B=2 H=8 N=128: about 18 us of kernels in a step of 70-120 us).
//
// Argument validation (dtypes, shapes, tiles) stays in the Python wrappers,
// which raise the reference's exception types before this op is called; a
// status other than FA_OK here (a launch failure) raises RuntimeError.
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <cmath>

#include "fa.h"

namespace {

// log2(e) / sqrt(D) and 1 / sqrt(D), formed in double and rounded once to float, as the
// Python layer passes them (so both paths hand the kernels the same scales)
float scale_log2(int D) { return static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(D))); }
float sm_scale(int D) { return static_cast<float>(1.0 / std::sqrt(static_cast<double>(D))); }

void* launch_stream(const at::Tensor& t) {
  return static_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

int dtype_code(const at::Tensor& t) { return t.scalar_type() == at::kBFloat16 ? FA_BF16 : FA_F16; }

void check(int status, const char* entry) {
  TORCH_CHECK(status == FA_OK, entry, ": ", fa_strerror(status), " (status ", status, ")");
}

struct FusedAttention : public torch::autograd::Function<FusedAttention> {
  static at::Tensor forward(torch::autograd::AutogradContext* ctx, const at::Tensor& q_in,
                            const at::Tensor& k_in, const at::Tensor& v_in, int64_t tile_m, int64_t tile_n) {
    const c10::DeviceGuard guard(q_in.device());
    const at::Tensor q = q_in.contiguous(), k = k_in.contiguous(), v = v_in.contiguous();
    const int B = q.size(0), H = q.size(1), S = q.size(2), D = q.size(3), H_kv = k.size(1);
    at::Tensor o = at::empty_like(q);
    at::Tensor lse = at::empty({B, H, S}, q.options().dtype(at::kFloat));
    check(fa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr<float>(), B, H, H_kv, S,
                 D, dtype_code(q), scale_log2(D), static_cast<int>(tile_m),
                 static_cast<int>(tile_n), launch_stream(q)),
          "fa_fwd");
    ctx->save_for_backward({q, k, v, o, lse});
    ctx->saved_data["tile_m"] = tile_m;
    ctx->saved_data["tile_n"] = tile_n;
    return o;
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grad_out) {
    const auto saved = ctx->get_saved_variables();
    const at::Tensor &q = saved[0], &k = saved[1], &v = saved[2], &o = saved[3], &lse = saved[4];
    const c10::DeviceGuard guard(q.device());
    const at::Tensor d_o = grad_out[0].contiguous().to(q.scalar_type());
    const int B = q.size(0), H = q.size(1), S = q.size(2), D = q.size(3), H_kv = k.size(1);
    at::Tensor dq = at::empty_like(q), dk = at::empty_like(k), dv = at::empty_like(v);
    const size_t nbytes = fa_bwd_gqa_workspace_size(B, H, H_kv, S, D);
    at::Tensor ws = at::empty({static_cast<int64_t>(nbytes)}, q.options().dtype(at::kByte));
    check(fa_bwd_gqa(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), d_o.data_ptr(), lse.data_ptr<float>(),
                     dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, H, H_kv, S, D, dtype_code(q),
                     scale_log2(D), sm_scale(D),
                     static_cast<int>(ctx->saved_data["tile_m"].toInt()),
                     static_cast<int>(ctx->saved_data["tile_n"].toInt()), nbytes ? ws.data_ptr() : nullptr, nbytes,
                     launch_stream(q)),
          "fa_bwd_gqa");
    return {dq, dk, dv, at::Tensor(), at::Tensor()};
  }
};

at::Tensor fused_attention(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, int64_t tile_m,
                           int64_t tile_n) {
  return FusedAttention::apply(q, k, v, tile_m, tile_n);
}

}  // namespace

PYBIND11_MODULE(fa_autograd, m) {
  m.doc() = "Causal fused attention with autograd (forward + recompute backward), C++ node over libfa.so";
  m.def("fused_attention", &fused_attention, "O = attention(q, k, v) with a backward; k, v may have fewer heads",
        pybind11::arg("q"), pybind11::arg("k"), pybind11::arg("v"), pybind11::arg("tile_m"), pybind11::arg("tile_n"));
}
