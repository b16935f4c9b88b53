// fa_torch.cpp - PyTorch binding of the C ABI (include/fa_gfx950.h) for the autograd path.
//
// The per-call host work of the drop-in -- tensor checks, output and workspace allocation (the
// caching allocator), the current HIP stream, filling fa_fwd_params / fa_bwd_params and the
// launch -- in C++, so a forward + backward costs a few microseconds of host time instead of
// the tens that per-field ctypes marshalling takes.  Every FLOP still runs in libfa_gfx950.so;
// this module only calls fa_fwd / fa_bwd / fa_fwd_sinks / fa_bwd_sinks / fa_bwd_workspace_bytes /
// fa_strerror.  swda / swda_sinks are the autograd functions themselves in C++ (forward, saved
// tensors, backward), which the functional forms of the Python package call.
//
// Error behaviour matches the ctypes path (_ops.py): tensors not on a GPU -> RuntimeError,
// unsupported dtype or shape -> ValueError, a C ABI status -> ValueError (argument) or
// RuntimeError (launch), with fa_strerror's text.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <stdexcept>
#include <string>

#include "../../include/fa_gfx950.h"

namespace {

int32_t dtype_code(const at::Tensor& t) {
  if (t.scalar_type() == at::kBFloat16) return FA_DTYPE_BF16;
  if (t.scalar_type() == at::kHalf) return FA_DTYPE_F16;
  if (t.scalar_type() == at::kFloat) return FA_DTYPE_F32;
  throw std::invalid_argument("q has dtype " + std::string(c10::toString(t.scalar_type())) +
                              "; supported dtypes are bfloat16, float16 and float32");
}

void check(const std::vector<std::pair<const at::Tensor*, const char*>>& ts) {
  const at::Tensor& first = *ts[0].first;
  if (!first.is_cuda())
    throw std::runtime_error(std::string(ts[0].second) + " is on " + first.device().str() +
                             ": the gfx950 attention kernels need GPU tensors (there is no CPU implementation)");
  dtype_code(first);
  for (const auto& [t, name] : ts) {
    if (t->dim() != 4) throw std::invalid_argument(std::string(name) + " must be 4-D [B, H, L, D]");
    if (t->device() != first.device())
      throw std::runtime_error(std::string(name) + " is on " + t->device().str() + " but " + ts[0].second +
                               " is on " + first.device().str());
    if (t->scalar_type() != first.scalar_type())
      throw std::invalid_argument(std::string(name) + " has a different dtype than " + ts[0].second);
  }
}

// Inputs the kernels cannot read directly (head-dim stride != 1, strides not whole multiples of
// 16 bytes, base not 16-byte aligned) are copied to a contiguous layout first.
at::Tensor kernel_ready(const at::Tensor& t) {
  const auto st = t.strides();
  const int64_t m = 16 / int64_t(t.element_size()) - 1;
  const auto misaligned = [&](const at::Tensor& x) { return (reinterpret_cast<uintptr_t>(x.data_ptr()) & 15) != 0; };
  if (st[3] != 1 || (st[0] & m) || (st[1] & m) || (st[2] & m) || misaligned(t)) {
    at::Tensor c = t.contiguous();
    if (misaligned(c)) c = c.clone(at::MemoryFormat::Contiguous);
    return c;
  }
  return t;
}

void strides3(int64_t dst[3], const at::Tensor& t) {
  dst[0] = t.stride(0);
  dst[1] = t.stride(1);
  dst[2] = t.stride(2);
}

int32_t clamp_i32(int64_t x) {
  return x < INT32_MIN ? INT32_MIN : (x > INT32_MAX ? INT32_MAX : int32_t(x));
}

void raise_for_status(int rc, const char* what) {
  if (rc == FA_OK) return;
  const std::string msg = std::string(what) + ": " + fa_strerror(rc);
  if (rc == FA_ERR_LAUNCH) throw std::runtime_error(msg);
  throw std::invalid_argument(msg);
}

void* current_stream(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// Learned sink logits as the C ABI takes them: float32 [Hq], contiguous, on q's device.
at::Tensor sinks_ready(const at::Tensor& sinks, int64_t Hq, const at::Tensor& q) {
  if (sinks.dim() != 1 || sinks.size(0) != Hq)
    throw std::invalid_argument("sinks must have shape [" + std::to_string(Hq) +
                                "] (one logit per query head)");
  if (sinks.device() != q.device())
    throw std::runtime_error("sinks is on " + sinks.device().str() + " but q is on " + q.device().str());
  return sinks.to(at::kFloat).contiguous();
}

// forward: returns (o, lse) for q [B,Hq,L,D], k/v [B,Hkv,L,D]; o has q's memory layout (as
// torch.empty_like(q) in the reference, flash_attention_gpt_oss.py:356).  With learned sink
// logits (float32-convertible [Hq]) it calls fa_fwd_sinks.
std::vector<at::Tensor> fwd(const at::Tensor& q_in, const at::Tensor& k_in, const at::Tensor& v_in, int64_t window,
                            int64_t sink, double scale, const c10::optional<at::Tensor>& sinks_in) {
  check({{&q_in, "q"}, {&k_in, "k"}, {&v_in, "v"}});
  const c10::DeviceGuard guard(q_in.device());
  const at::Tensor q = kernel_ready(q_in), k = kernel_ready(k_in), v = kernel_ready(v_in);
  const int64_t B = q.size(0), Hq = q.size(1), L = q.size(2), D = q.size(3);
  const at::Tensor sinks = sinks_in.has_value() ? sinks_ready(*sinks_in, Hq, q) : at::Tensor();
  at::Tensor o = at::empty_like(q);
  at::Tensor lse = at::empty({B, Hq, L}, q.options().dtype(at::kFloat));
  fa_fwd_params p{};
  p.q = q.data_ptr();
  p.k = k.data_ptr();
  p.v = v.data_ptr();
  p.o = o.data_ptr();
  p.lse = lse.data_ptr<float>();
  strides3(p.q_stride, q);
  strides3(p.k_stride, k);
  strides3(p.v_stride, v);
  strides3(p.o_stride, o);
  p.lse_stride[0] = lse.stride(0);
  p.lse_stride[1] = lse.stride(1);
  p.lse_stride[2] = lse.stride(2);
  p.batch = clamp_i32(B);
  p.heads_q = clamp_i32(Hq);
  p.heads_kv = clamp_i32(k.size(1));
  p.seqlen = clamp_i32(L);
  p.head_dim = clamp_i32(D);
  p.window = clamp_i32(window);
  p.sink = clamp_i32(sink);
  p.softmax_scale = float(scale);
  p.dtype = dtype_code(q);
  if (sinks.defined())
    raise_for_status(fa_fwd_sinks(&p, sinks.data_ptr<float>(), current_stream(q)), "fa_fwd_sinks");
  else
    raise_for_status(fa_fwd(&p, current_stream(q)), "fa_fwd");
  return {o, lse};
}

// backward: returns (dq, dk, dv) in the input dtype and the layouts of q, k, v; with learned
// sink logits, (dq, dk, dv, dsinks) through fa_bwd_sinks, dsinks float32 [Hq]
std::vector<at::Tensor> bwd(const at::Tensor& q_in, const at::Tensor& k_in, const at::Tensor& v_in,
                            const at::Tensor& o_in, const at::Tensor& lse, const at::Tensor& do_in, int64_t window,
                            int64_t sink, double scale, const c10::optional<at::Tensor>& sinks_in) {
  check({{&q_in, "q"}, {&k_in, "k"}, {&v_in, "v"}, {&o_in, "o"}, {&do_in, "do"}});
  const c10::DeviceGuard guard(q_in.device());
  const at::Tensor q = kernel_ready(q_in), k = kernel_ready(k_in), v = kernel_ready(v_in);
  const at::Tensor o = kernel_ready(o_in), dout = kernel_ready(do_in);
  const int64_t B = q.size(0), Hq = q.size(1), L = q.size(2), D = q.size(3), Hkv = k.size(1);
  const at::Tensor sinks = sinks_in.has_value() ? sinks_ready(*sinks_in, Hq, q) : at::Tensor();
  at::Tensor dq = at::empty_like(q);
  at::Tensor dk = at::empty_like(k);
  at::Tensor dv = at::empty_like(v);
  const size_t ws_bytes = fa_bwd_workspace_bytes(clamp_i32(B), clamp_i32(Hq), clamp_i32(Hkv), clamp_i32(L),
                                                 clamp_i32(D), clamp_i32(window), clamp_i32(sink));
  at::Tensor ws = at::empty({int64_t(ws_bytes > 256 ? ws_bytes : 256)}, q.options().dtype(at::kByte));
  fa_bwd_params p{};
  p.q = q.data_ptr();
  p.k = k.data_ptr();
  p.v = v.data_ptr();
  p.o = o.data_ptr();
  p.dout = dout.data_ptr();
  p.lse = lse.data_ptr<float>();
  p.dq = dq.data_ptr();
  p.dk = dk.data_ptr();
  p.dv = dv.data_ptr();
  strides3(p.q_stride, q);
  strides3(p.k_stride, k);
  strides3(p.v_stride, v);
  strides3(p.o_stride, o);
  strides3(p.do_stride, dout);
  p.lse_stride[0] = lse.stride(0);
  p.lse_stride[1] = lse.stride(1);
  p.lse_stride[2] = lse.stride(2);
  strides3(p.dq_stride, dq);
  strides3(p.dk_stride, dk);
  strides3(p.dv_stride, dv);
  p.batch = clamp_i32(B);
  p.heads_q = clamp_i32(Hq);
  p.heads_kv = clamp_i32(Hkv);
  p.seqlen = clamp_i32(L);
  p.head_dim = clamp_i32(D);
  p.window = clamp_i32(window);
  p.sink = clamp_i32(sink);
  p.softmax_scale = float(scale);
  p.dtype = dtype_code(q);
  if (sinks.defined()) {
    at::Tensor dsinks = at::empty({Hq}, q.options().dtype(at::kFloat));
    raise_for_status(fa_bwd_sinks(&p, sinks.data_ptr<float>(), dsinks.data_ptr<float>(), ws.data_ptr(),
                                  size_t(ws.numel()), current_stream(q)),
                     "fa_bwd_sinks");
    return {dq, dk, dv, dsinks};
  }
  raise_for_status(fa_bwd(&p, ws.data_ptr(), size_t(ws.numel()), current_stream(q)), "fa_bwd");
  return {dq, dk, dv};
}

// The autograd function of flash_attention_gpt_oss.py:340-438 (FlashSWDAWithSink) in C++: the
// forward saves (q, k, v, o, lse) and the window / sink / scale, the backward returns dq, dk, dv
// and no gradient for the other four arguments.  The autograd engine runs this backward on its
// device thread without taking the Python interpreter lock, so a training step spends no Python
// time in the backward; the computation is the same fa_fwd / fa_bwd calls as fwd() / bwd().
struct SwdaFunction : public torch::autograd::Function<SwdaFunction> {
  static at::Tensor forward(torch::autograd::AutogradContext* ctx, const at::Tensor& q, const at::Tensor& k,
                            const at::Tensor& v, int64_t window, int64_t sink, double scale) {
    std::vector<at::Tensor> r = fwd(q, k, v, window, sink, scale, c10::nullopt);
    ctx->save_for_backward({q, k, v, r[0], r[1]});
    ctx->saved_data["window"] = window;
    ctx->saved_data["sink"] = sink;
    ctx->saved_data["scale"] = scale;
    return r[0];
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    const torch::autograd::variable_list s = ctx->get_saved_variables();
    std::vector<at::Tensor> g = bwd(s[0], s[1], s[2], s[3], s[4], grads[0], ctx->saved_data["window"].toInt(),
                                    ctx->saved_data["sink"].toInt(), ctx->saved_data["scale"].toDouble(), c10::nullopt);
    return {g[0], g[1], g[2], at::Tensor(), at::Tensor(), at::Tensor()};
  }
};

// The same with GPT-OSS learned sink logits (sinks [Hq]): the backward also returns d sinks, in
// the dtype of sinks.
struct SwdaSinksFunction : public torch::autograd::Function<SwdaSinksFunction> {
  static at::Tensor forward(torch::autograd::AutogradContext* ctx, const at::Tensor& q, const at::Tensor& k,
                            const at::Tensor& v, const at::Tensor& sinks, int64_t window, int64_t sink, double scale) {
    std::vector<at::Tensor> r = fwd(q, k, v, window, sink, scale, sinks);
    ctx->save_for_backward({q, k, v, r[0], r[1], sinks});
    ctx->saved_data["window"] = window;
    ctx->saved_data["sink"] = sink;
    ctx->saved_data["scale"] = scale;
    return r[0];
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    const torch::autograd::variable_list s = ctx->get_saved_variables();
    std::vector<at::Tensor> g = bwd(s[0], s[1], s[2], s[3], s[4], grads[0], ctx->saved_data["window"].toInt(),
                                    ctx->saved_data["sink"].toInt(), ctx->saved_data["scale"].toDouble(), s[5]);
    return {g[0], g[1], g[2], g[3].to(s[5].scalar_type()), at::Tensor(), at::Tensor(), at::Tensor()};
  }
};

at::Tensor swda(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, int64_t window, int64_t sink,
                double scale) {
  return SwdaFunction::apply(q, k, v, window, sink, scale);
}

at::Tensor swda_sinks(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& sinks,
                      int64_t window, int64_t sink, double scale) {
  return SwdaSinksFunction::apply(q, k, v, sinks, window, sink, scale);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("swda", &swda,
        "autograd forward of causal sliding-window + sink attention: (q, k, v, window, sink, scale) -> o",
        py::arg("q"), py::arg("k"), py::arg("v"), py::arg("window"), py::arg("sink"), py::arg("scale"));
  m.def("swda_sinks", &swda_sinks,
        "autograd forward with learned sink logits: (q, k, v, sinks, window, sink, scale) -> o", py::arg("q"),
        py::arg("k"), py::arg("v"), py::arg("sinks"), py::arg("window"), py::arg("sink"), py::arg("scale"));
  m.doc() = "PyTorch binding of libfa_gfx950.so (fa_fwd / fa_bwd)";
  m.def("fwd", &fwd, "forward: (q, k, v, window, sink, scale, sinks=None) -> (o, lse)", py::arg("q"), py::arg("k"),
        py::arg("v"), py::arg("window"), py::arg("sink"), py::arg("scale"), py::arg("sinks") = py::none());
  m.def("bwd", &bwd, "backward: (q, k, v, o, lse, do, window, sink, scale, sinks=None) -> (dq, dk, dv[, dsinks])",
        py::arg("q"), py::arg("k"), py::arg("v"), py::arg("o"), py::arg("lse"), py::arg("do"), py::arg("window"),
        py::arg("sink"), py::arg("scale"), py::arg("sinks") = py::none());
}
