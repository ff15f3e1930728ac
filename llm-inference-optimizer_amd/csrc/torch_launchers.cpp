// Host-side launchers of the per-token kernels as a thin torch extension over
// the C ABI (include/mi355_fused.h): argument checks, the row / stride logic
// and the output allocation of the Python launchers in kernels/*.py, done in
// C++ so an eager call costs one pybind11 dispatch instead of Python
// attribute accesses, a torch.empty from Python and a 12-argument ctypes
// call.  Torch types stop here: every kernel is reached through the
// plain-pointer entry points of libmi355_fused.so, on torch's current HIP
// stream.
//
// The behaviour is the Python launchers', which keep the reference's
// launcher contracts (src/kernels/fused_rmsnorm_triton.py:52-71,
// src/kernels/fused_swiglu_triton.py:39-53, src/kernels/w8a16_matmul_triton.py:
// 102-134): a failed precondition raises AssertionError with the same
// message, a malformed weight shape the ValueError of Python's tuple
// unpacking, and a failing C-ABI call the package's KernelError (registered
// by _lib at import) with the library's message.
#include <torch/extension.h>
#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>

#include <sstream>
#include <string>

#include "../../include/mi355_fused.h"

namespace py = pybind11;

namespace {

// The package's KernelError class.  Held through a pointer that is never
// freed: a py::object with static storage would be released after the
// interpreter has finalised, at process exit.
py::object* g_kernel_error = nullptr;

[[noreturn]] void fail_assert(const std::string& msg) {
  PyErr_SetString(PyExc_AssertionError, msg.c_str());
  throw py::error_already_set();
}

void check(const char* fn, int status) {
  if (status == MI355_OK) return;
  const std::string msg = mi355_last_error();
  if (g_kernel_error != nullptr) {
    PyErr_SetObject(g_kernel_error->ptr(), py::make_tuple(fn, status, msg).ptr());
    throw py::error_already_set();
  }
  throw std::runtime_error(std::string(fn) + " failed with status " + std::to_string(status) + ": " + msg);
}

int code_of(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return MI355_F32;
    case at::kHalf: return MI355_F16;
    case at::kBFloat16: return MI355_BF16;
    default: return -1;
  }
}

// str(torch.dtype) as Python prints it, for the assertion messages.
std::string dtype_str(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return "torch.float32";
    case at::kHalf: return "torch.float16";
    case at::kBFloat16: return "torch.bfloat16";
    case at::kDouble: return "torch.float64";
    case at::kChar: return "torch.int8";
    case at::kByte: return "torch.uint8";
    case at::kShort: return "torch.int16";
    case at::kInt: return "torch.int32";
    case at::kLong: return "torch.int64";
    case at::kBool: return "torch.bool";
    default: return std::string("torch.") + c10::toString(t);
  }
}

// tuple(t.shape) as Python prints it.
std::string shape_str(at::IntArrayRef s) {
  std::ostringstream o;
  o << "(";
  for (size_t i = 0; i < s.size(); ++i) o << (i ? ", " : "") << s[i];
  if (s.size() == 1) o << ",";
  o << ")";
  return o.str();
}

// `n, k = w.shape` for a 2-D weight; Python's unpacking error otherwise.
std::pair<int64_t, int64_t> unpack2(const at::Tensor& w) {
  if (w.dim() > 2) throw py::value_error("too many values to unpack (expected 2)");
  if (w.dim() < 2) throw py::value_error("not enough values to unpack (expected 2, got " + std::to_string(w.dim()) + ")");
  return {w.size(0), w.size(1)};
}

// Launch context: `dev` current for the call (switched only when it is not),
// torch's current stream on it.
struct Launch {
  c10::optional<c10::hip::HIPGuard> guard;
  void* stream;
  explicit Launch(int dev) {
    if (c10::hip::current_device() != dev) guard.emplace(static_cast<c10::DeviceIndex>(dev));
    stream = c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(dev)).stream();
  }
};

// Rows view of t over its last dimension n: (view, row count, row stride),
// copying only when the last dimension itself is strided (a row-strided view
// is passed with its stride).
struct Rows {
  at::Tensor t;
  int64_t m, stride;
};
Rows rows_of(const at::Tensor& t, int64_t n) {
  if (t.is_contiguous()) return {t, n ? t.numel() / n : 0, n};
  at::Tensor t2 = t.reshape({-1, n});
  if (t2.stride(-1) != 1 || (t2.size(0) > 1 && t2.stride(0) < n)) t2 = t2.contiguous();
  const int64_t m = t2.size(0);
  return {t2, m, m > 1 ? t2.stride(0) : n};
}

// x as [rows, k] rows a projection kernel can stream: unit element stride
// and, over more than one row, rows that do not overlap (row stride >= k).
// A broadcast or overlapping view -- expand() gives row stride 0 -- is
// copied, as the reference's `x.reshape(-1, K).contiguous()` copies it.
at::Tensor matrix_rows(const at::Tensor& x, int64_t k) {
  at::Tensor x2 = x.reshape({-1, k});
  if (x2.stride(-1) != 1 || (x2.size(0) > 1 && x2.stride(0) < k)) x2 = x2.contiguous();
  return x2;
}

// Weight matrices [n, k] the kernels stream row by row: each with unit
// element stride and non-overlapping rows, and (for a pair read together)
// one shared row stride; copied otherwise.
bool streamable(const at::Tensor& w) {
  return w.stride(-1) == 1 && (w.size(0) <= 1 || w.stride(0) >= w.size(1));
}
std::pair<at::Tensor, at::Tensor> weight_pair(const at::Tensor& a, const at::Tensor& b) {
  if (streamable(a) && streamable(b) && a.stride(0) == b.stride(0)) return {a, b};
  return {a.contiguous(), b.contiguous()};
}

std::vector<int64_t> with_last(at::IntArrayRef s, int64_t last) {
  std::vector<int64_t> v(s.begin(), s.end());
  v.back() = last;
  return v;
}

void* ptr(const at::Tensor& t) { return t.data_ptr(); }

// ------------------------------------------------------------------ RMSNorm

at::Tensor rmsnorm(const at::Tensor& x, const at::Tensor& weight, double eps) {
  if (!(x.is_cuda() && weight.is_cuda())) fail_assert("x and weight must be ROCm GPU tensors");
  const int64_t N = x.size(-1);
  if (!(weight.dim() == 1 && weight.size(0) == N))
    fail_assert("weight shape " + shape_str(weight.sizes()) + " != (" + std::to_string(N) + ",)");
  const int code = code_of(x.scalar_type()), wcode = code_of(weight.scalar_type());
  if (code < 0 || wcode < 0)
    fail_assert("unsupported dtypes x=" + dtype_str(x.scalar_type()) + " weight=" + dtype_str(weight.scalar_type()) +
                " (fp16, bf16, fp32)");
  const int dev = x.get_device();
  if (weight.get_device() != dev) fail_assert("x and weight must be on the same device");
  const Rows r = rows_of(x, N);
  const at::Tensor w = weight.stride(0) != 1 ? weight.contiguous() : weight;
  at::Tensor out = x.is_contiguous() ? at::empty_like(x) : at::empty(x.sizes(), x.options());
  if (r.m && N) {
    Launch l(dev);
    check("mi355_rmsnorm_fwd", mi355_rmsnorm_fwd(ptr(r.t), ptr(w), ptr(out), r.m, N, r.stride, N,
                                                 static_cast<float>(eps), code, wcode, code, l.stream));
  }
  return out;
}

std::tuple<at::Tensor, at::Tensor> add_rmsnorm(const at::Tensor& x, const at::Tensor& residual,
                                               const at::Tensor& weight, double eps) {
  if (!(x.is_cuda() && residual.is_cuda() && weight.is_cuda()))
    fail_assert("x, residual and weight must be ROCm GPU tensors");
  if (x.sizes() != residual.sizes())
    fail_assert("shape mismatch " + shape_str(x.sizes()) + " vs " + shape_str(residual.sizes()));
  if (x.scalar_type() != residual.scalar_type())
    fail_assert("dtype mismatch " + dtype_str(x.scalar_type()) + " vs " + dtype_str(residual.scalar_type()));
  const int64_t N = x.size(-1);
  if (!(weight.dim() == 1 && weight.size(0) == N))
    fail_assert("weight shape " + shape_str(weight.sizes()) + " != (" + std::to_string(N) + ",)");
  const int code = code_of(x.scalar_type()), wcode = code_of(weight.scalar_type());
  if (code < 0 || wcode < 0)
    fail_assert("unsupported dtypes x=" + dtype_str(x.scalar_type()) + " weight=" + dtype_str(weight.scalar_type()) +
                " (fp16, bf16, fp32)");
  const int dev = x.get_device();
  if (residual.get_device() != dev || weight.get_device() != dev)
    fail_assert("x, residual and weight must be on the same device");
  const Rows xr = rows_of(x, N), rr = rows_of(residual, N);
  const at::Tensor w = weight.stride(0) != 1 ? weight.contiguous() : weight;
  at::Tensor out = at::empty(x.sizes(), x.options());
  at::Tensor h = at::empty(x.sizes(), x.options());
  if (xr.m && N) {
    Launch l(dev);
    check("mi355_add_rmsnorm_fwd",
          mi355_add_rmsnorm_fwd(ptr(xr.t), ptr(rr.t), ptr(w), ptr(out), ptr(h), xr.m, N, xr.stride, rr.stride, N, N,
                                static_cast<float>(eps), code, wcode, code, l.stream));
  }
  return {out, h};
}

// ------------------------------------------------------------- SiLU-and-mul

at::Tensor silu_mul(const at::Tensor& gate, const at::Tensor& up) {
  if (gate.sizes() != up.sizes())
    fail_assert("shape mismatch " + shape_str(gate.sizes()) + " vs " + shape_str(up.sizes()));
  if (!(gate.is_cuda() && up.is_cuda())) fail_assert("gate and up must be ROCm GPU tensors");
  int code = code_of(gate.scalar_type());
  const int ucode = code_of(up.scalar_type());
  if (code < 0 || ucode < 0)
    fail_assert("unsupported dtypes gate=" + dtype_str(gate.scalar_type()) + " up=" + dtype_str(up.scalar_type()) +
                " (fp16, bf16, fp32)");
  const int dev = gate.get_device();
  if (up.get_device() != dev) fail_assert("gate and up must be on the same device");
  at::Tensor g, u;
  if (code != ucode) {
    // the reference widens each input to fp32 separately; widening both here
    // is exact, and the fp32 result is rounded once below
    g = gate.contiguous().to(at::kFloat);
    u = up.contiguous().to(at::kFloat);
    code = MI355_F32;
  } else {
    g = gate.is_contiguous() ? gate : gate.contiguous();
    u = up.is_contiguous() ? up : up.contiguous();
  }
  at::Tensor out = at::empty_like(g);
  const int64_t n = g.numel();
  if (n) {
    Launch l(dev);
    check("mi355_silu_mul_fwd", mi355_silu_mul_fwd(ptr(g), ptr(u), ptr(out), n, code, code, l.stream));
  }
  if (out.scalar_type() != gate.scalar_type()) out = out.to(gate.scalar_type());
  return out.view(gate.sizes());
}

// ------------------------------------------------- gate/up + SiLU-and-mul

at::Tensor gate_up_silu(const at::Tensor& x, const at::Tensor& w_gate, const at::Tensor& w_up, bool out_f32) {
  if (!(x.is_cuda() && w_gate.is_cuda() && w_up.is_cuda())) fail_assert("x and the weights must be ROCm GPU tensors");
  if (x.scalar_type() != at::kHalf && x.scalar_type() != at::kBFloat16)
    fail_assert("x must be fp16 or bf16, got " + dtype_str(x.scalar_type()));
  if (w_gate.scalar_type() != x.scalar_type() || w_up.scalar_type() != x.scalar_type())
    fail_assert("dtype mismatch x=" + dtype_str(x.scalar_type()) + " w_gate=" + dtype_str(w_gate.scalar_type()) +
                " w_up=" + dtype_str(w_up.scalar_type()));
  const int64_t k = x.size(-1);
  if (!(w_gate.dim() == 2 && w_gate.sizes() == w_up.sizes() && w_gate.size(1) == k))
    fail_assert("weights must be [n_out, " + std::to_string(k) + "], got " + shape_str(w_gate.sizes()) + " and " +
                shape_str(w_up.sizes()));
  const int dev = x.get_device();
  if (w_gate.get_device() != dev || w_up.get_device() != dev) fail_assert("x and the weights must share a device");
  const at::ScalarType odt = out_f32 ? at::kFloat : x.scalar_type();

  const int64_t n_out = w_gate.size(0);
  const at::Tensor x2 = matrix_rows(x, k);
  const auto [wg, wu] = weight_pair(w_gate, w_up);
  const int64_t rows = x2.size(0);
  at::Tensor out = at::empty({rows, n_out}, x.options().dtype(odt));
  if (rows && n_out) {
    // a single row's stride is arbitrary in torch (even 0); the kernel reads one row then
    const int64_t xs = rows > 1 ? x2.stride(0) : k;
    const int64_t ws = n_out > 1 ? wg.stride(0) : k;
    Launch l(dev);
    check("mi355_gate_up_silu_fwd",
          mi355_gate_up_silu_fwd(ptr(x2), ptr(wg), ptr(wu), ptr(out), rows, k, n_out, xs, ws, n_out,
                                 code_of(x.scalar_type()), code_of(odt), l.stream));
  }
  return out.view(with_last(x.sizes(), n_out));
}

// ------------------------------------------------------------ 16-bit linear

at::Tensor linear16(const at::Tensor& x, const at::Tensor& weight, const c10::optional<at::Tensor>& bias,
                    bool out_f32) {
  if (!(x.is_cuda() && weight.is_cuda())) fail_assert("x and weight must be ROCm GPU tensors");
  if (x.scalar_type() != at::kHalf && x.scalar_type() != at::kBFloat16)
    fail_assert("x must be fp16 or bf16, got " + dtype_str(x.scalar_type()));
  if (weight.scalar_type() != x.scalar_type())
    fail_assert("dtype mismatch x=" + dtype_str(x.scalar_type()) + " weight=" + dtype_str(weight.scalar_type()));
  if (weight.dim() != 2) fail_assert("weight must be (N, K), got " + shape_str(weight.sizes()));
  const int64_t N = weight.size(0), K = weight.size(1);
  if (x.size(-1) != K)
    fail_assert("x last dim " + std::to_string(x.size(-1)) + " != weight in_features " + std::to_string(K));
  const bool has_bias = bias.has_value() && bias->defined();
  if (has_bias && !(bias->is_cuda() && bias->dim() == 1 && bias->size(0) == N && code_of(bias->scalar_type()) >= 0))
    fail_assert("bias must be a (" + std::to_string(N) + ",) float GPU tensor, got " + shape_str(bias->sizes()) + " " +
                dtype_str(bias->scalar_type()));
  const int dev = x.get_device();
  if (weight.get_device() != dev || (has_bias && bias->get_device() != dev))
    fail_assert("x, weight and bias must share a device");
  const at::ScalarType odt = out_f32 ? at::kFloat : x.scalar_type();

  const at::Tensor x2 = matrix_rows(x, K);
  const at::Tensor w = streamable(weight) ? weight : weight.contiguous();
  const at::Tensor b = has_bias ? bias->contiguous() : at::Tensor();
  const int64_t M = x2.size(0);
  at::Tensor out = at::empty({M, N}, x.options().dtype(odt));
  if (M && N) {
    const int64_t xs = M > 1 ? x2.stride(0) : K;
    const int64_t ws = N > 1 ? w.stride(0) : K;
    Launch l(dev);
    check("mi355_linear16_fwd",
          mi355_linear16_fwd(ptr(x2), ptr(w), has_bias ? ptr(b) : nullptr, ptr(out), M, K, N, xs, ws, N,
                             code_of(x.scalar_type()), has_bias ? code_of(b.scalar_type()) : 0, code_of(odt),
                             l.stream));
  }
  return out.reshape(with_last(x.sizes(), N));
}

// ------------------------------------------------------------------- W8A16

at::Tensor w8a16_linear(const at::Tensor& x, const at::Tensor& w_q, const at::Tensor& scale,
                        const c10::optional<at::Tensor>& bias, bool out_f32) {
  if (!(x.is_cuda() && w_q.is_cuda())) fail_assert("x and w_q must be ROCm GPU tensors");
  if (w_q.scalar_type() != at::kChar) fail_assert("w_q must be int8, got " + dtype_str(w_q.scalar_type()));
  const auto [N, K] = unpack2(w_q);
  if (x.size(-1) != K)
    fail_assert("x last dim " + std::to_string(x.size(-1)) + " != weight in_features " + std::to_string(K));
  if (x.scalar_type() != at::kHalf && x.scalar_type() != at::kBFloat16)
    fail_assert("x must be fp16 or bf16, got " + dtype_str(x.scalar_type()));
  if (!(scale.is_cuda() && scale.dim() == 1 && scale.size(0) == N && code_of(scale.scalar_type()) >= 0))
    fail_assert("scale must be a (" + std::to_string(N) + ",) float GPU tensor, got " + shape_str(scale.sizes()) + " " +
                dtype_str(scale.scalar_type()));
  const bool has_bias = bias.has_value() && bias->defined();
  if (has_bias && !(bias->is_cuda() && bias->dim() == 1 && bias->size(0) == N && code_of(bias->scalar_type()) >= 0))
    fail_assert("bias must be a (" + std::to_string(N) + ",) float GPU tensor, got " + shape_str(bias->sizes()) + " " +
                dtype_str(bias->scalar_type()));
  const int dev = x.get_device();
  if (w_q.get_device() != dev || scale.get_device() != dev || (has_bias && bias->get_device() != dev))
    fail_assert("x, w_q, scale and bias must share a device");
  const at::ScalarType odt = out_f32 ? at::kFloat : x.scalar_type();

  const at::Tensor x2 = matrix_rows(x, K);
  const at::Tensor q = streamable(w_q) ? w_q : w_q.contiguous();
  const at::Tensor s = scale.contiguous();
  const at::Tensor b = has_bias ? bias->contiguous() : at::Tensor();
  const int64_t M = x2.size(0);
  at::Tensor out = at::empty({M, N}, x.options().dtype(odt));
  if (M && N) {
    const int64_t xs = M > 1 ? x2.stride(0) : K;
    const int64_t ws = N > 1 ? q.stride(0) : K;
    Launch l(dev);
    check("mi355_w8a16_linear_fwd",
          mi355_w8a16_linear_fwd(ptr(x2), ptr(q), ptr(s), has_bias ? ptr(b) : nullptr, ptr(out), M, K, N, xs, ws, N,
                                 code_of(x.scalar_type()), code_of(s.scalar_type()),
                                 has_bias ? code_of(b.scalar_type()) : 0, code_of(odt), l.stream));
  }
  return out.reshape(with_last(x.sizes(), N));
}

at::Tensor gate_up_silu_w8a16(const at::Tensor& x, const at::Tensor& wq_gate, const at::Tensor& scale_gate,
                              const at::Tensor& wq_up, const at::Tensor& scale_up, bool out_f32) {
  if (!(x.is_cuda() && wq_gate.is_cuda() && wq_up.is_cuda())) fail_assert("x and the weights must be ROCm GPU tensors");
  if (!(wq_gate.scalar_type() == at::kChar && wq_up.scalar_type() == at::kChar)) fail_assert("weights must be int8");
  if (wq_gate.sizes() != wq_up.sizes())
    fail_assert("weight shapes differ: " + shape_str(wq_gate.sizes()) + " vs " + shape_str(wq_up.sizes()));
  const auto [N, K] = unpack2(wq_gate);
  if (x.size(-1) != K)
    fail_assert("x last dim " + std::to_string(x.size(-1)) + " != weight in_features " + std::to_string(K));
  if (x.scalar_type() != at::kHalf && x.scalar_type() != at::kBFloat16)
    fail_assert("x must be fp16 or bf16, got " + dtype_str(x.scalar_type()));
  for (const at::Tensor* sc : {&scale_gate, &scale_up}) {
    if (!(sc->is_cuda() && sc->dim() == 1 && sc->size(0) == N && code_of(sc->scalar_type()) >= 0))
      fail_assert("scales must be (" + std::to_string(N) + ",) float GPU tensors, got " + shape_str(sc->sizes()) + " " +
                  dtype_str(sc->scalar_type()));
  }
  if (scale_gate.scalar_type() != scale_up.scalar_type()) fail_assert("the two scales must share a dtype");
  const int dev = x.get_device();
  for (const at::Tensor* t : {&wq_gate, &wq_up, &scale_gate, &scale_up}) {
    if (t->get_device() != dev) fail_assert("all inputs must share a device");
  }
  const at::ScalarType odt = out_f32 ? at::kFloat : x.scalar_type();

  const at::Tensor x2 = matrix_rows(x, K);
  const auto [qg, qu] = weight_pair(wq_gate, wq_up);
  const at::Tensor sg = scale_gate.contiguous(), su = scale_up.contiguous();
  const int64_t M = x2.size(0);
  at::Tensor out = at::empty({M, N}, x.options().dtype(odt));
  if (M && N) {
    const int64_t xs = M > 1 ? x2.stride(0) : K;
    const int64_t ws = N > 1 ? qg.stride(0) : K;
    Launch l(dev);
    check("mi355_gate_up_silu_w8a16_fwd",
          mi355_gate_up_silu_w8a16_fwd(ptr(x2), ptr(qg), ptr(qu), ptr(sg), ptr(su), ptr(out), M, K, N, xs, ws, N,
                                       code_of(x.scalar_type()), code_of(sg.scalar_type()), code_of(odt), l.stream));
  }
  return out.reshape(with_last(x.sizes(), N));
}

}  // namespace

PYBIND11_MODULE(_mi355_torch, m) {
  m.doc() = "Host-side launchers of the MI355X fused kernels (torch tensors -> the C ABI of libmi355_fused.so)";
  m.def("set_kernel_error", [](py::object cls) {
    if (g_kernel_error == nullptr) g_kernel_error = new py::object(cls);
    else *g_kernel_error = cls;
  });
  m.def("abi_version", []() { return mi355_abi_version(); });
  m.def("rmsnorm", &rmsnorm, py::arg("x"), py::arg("weight"), py::arg("eps"));
  m.def("add_rmsnorm", &add_rmsnorm, py::arg("x"), py::arg("residual"), py::arg("weight"), py::arg("eps"));
  m.def("silu_mul", &silu_mul, py::arg("gate"), py::arg("up"));
  m.def("gate_up_silu", &gate_up_silu, py::arg("x"), py::arg("w_gate"), py::arg("w_up"), py::arg("out_f32"));
  m.def("linear16", &linear16, py::arg("x"), py::arg("weight"), py::arg("bias"), py::arg("out_f32"));
  m.def("w8a16_linear", &w8a16_linear, py::arg("x"), py::arg("w_q"), py::arg("scale"), py::arg("bias"),
        py::arg("out_f32"));
  m.def("gate_up_silu_w8a16", &gate_up_silu_w8a16, py::arg("x"), py::arg("wq_gate"), py::arg("scale_gate"),
        py::arg("wq_up"), py::arg("scale_up"), py::arg("out_f32"));
}
