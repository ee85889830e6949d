// fa_native.cpp — C++ autograd binding of libfa_gfx950.so for the public API's
// training path (host code only; built with g++ against PyTorch's headers).
//
// TritonAttention (the reference's torch.autograd.Function bridge,
// attention.py:673-771) runs its forward and backward in Python. At small
// shapes that costs more than the kernels: the Python Function's bookkeeping
// and the backward's trip through the autograd engine into Python take ~90 us
// per fwd+bwd on top of the op layer. This binding makes the same library
// calls from a C++ torch::autograd::Function: fa_fwd_kv (or fa_fwd_ws when the
// forward splits its keys) and fa_bwd, with the same arguments, the same
// workspaces and on torch's current stream, so its results are identical bit
// for bit. forward() serves calls that need no gradient the same way (the op
// layer's flash_fwd, without the Python around it). Both serve the plain case
// only: a positive scale and one kernel head size (32, 64 or 128) for q, k and
// v; attention.py keeps the Python path for the rest (negative or zero scales,
// padded head sizes, forward-mode AD).
//
// The library's entry points come from the copy Python has already loaded
// (init() takes their addresses), so one libfa_gfx950.so serves both paths.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace {

using FwdKv = int (*)(const void*, const void*, const void*, void*, void*, int64_t, int64_t,
                      int64_t, int64_t, int64_t, int64_t, float, int, void*);
using FwdWs = int (*)(const void*, const void*, const void*, void*, void*, int64_t, int64_t,
                      int64_t, int64_t, int64_t, int64_t, float, int, void*, int64_t, void*);
using WsBytes = int64_t (*)(int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int);
using Bwd = int (*)(const void*, const void*, const void*, const void*, const void*,
                    const void*, void*, void*, void*, void*, int64_t, int64_t, int64_t, int64_t,
                    int64_t, int64_t, float, int, void*, int64_t, void*);
using LastError = const char* (*)();

// Entry points; index 0 = fp16, 1 = bf16.
struct Entries {
  FwdKv fwd_kv[2] = {nullptr, nullptr};
  FwdWs fwd_ws[2] = {nullptr, nullptr};
  Bwd bwd[2] = {nullptr, nullptr};
  WsBytes fwd_ws_bytes = nullptr;
  WsBytes bwd_ws_bytes = nullptr;
  LastError last_error = nullptr;
};
Entries g;

bool ready() {
  return g.fwd_kv[0] && g.fwd_kv[1] && g.fwd_ws[0] && g.fwd_ws[1] && g.bwd[0] && g.bwd[1] &&
         g.fwd_ws_bytes && g.bwd_ws_bytes && g.last_error;
}

// The library's error as the Python binding words it (_lib.FlashAttentionError).
[[noreturn]] void fail(int64_t code) {
  throw std::runtime_error("libfa_gfx950 error " + std::to_string(code) + ": " +
                           std::string(g.last_error()));
}

void check(int64_t code) {
  if (code != 0) fail(code);
}

int elem_index(const at::Tensor& t) {
  if (t.scalar_type() == at::kHalf) return 0;
  if (t.scalar_type() == at::kBFloat16) return 1;
  throw std::invalid_argument("gfx950 attention: tensors must be float16 or bfloat16");
}

// The kernels move 128-bit vectors: a view whose data pointer is not 16-byte
// aligned is copied into a fresh allocation (as _ops._aligned does).
at::Tensor aligned(const at::Tensor& t) {
  const at::Tensor c = t.contiguous();
  return reinterpret_cast<uintptr_t>(c.data_ptr()) % 16 == 0
             ? c
             : c.clone(at::MemoryFormat::Contiguous);
}

void* stream_of(const at::Tensor& t) {
  return static_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

// The uint8 workspace of `bytes` bytes (none for 0) from torch's caching allocator.
at::Tensor workspace(int64_t bytes, const at::Tensor& like) {
  if (bytes < 0) fail(bytes);
  return bytes > 0 ? at::empty({bytes}, like.options().dtype(at::kByte)) : at::Tensor();
}

struct Dims {
  int64_t B, Hq, Hkv, N, Nkv, D;
};

Dims dims_of(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v) {
  TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4,
              "q, k, v must be 4-D [batch, heads, sequence, head_dim]");
  TORCH_CHECK(k.sizes() == v.sizes() && k.size(0) == q.size(0) && k.size(3) == q.size(3),
              "k and v must have shape [B, Hkv, N_kv, D] matching q");
  TORCH_CHECK(q.scalar_type() == k.scalar_type() && q.scalar_type() == v.scalar_type(),
              "q, k, v must share one dtype");
  TORCH_CHECK(q.is_cuda() && k.device() == q.device() && v.device() == q.device(),
              "q, k, v must be on one GPU");
  return {q.size(0), q.size(1), k.size(1), q.size(2), k.size(2), q.size(3)};
}

// The forward launch (the op layer's flash_fwd): O and the base-2 LSE of
// aligned q, k, v on the current stream of their device.
struct Forward {
  at::Tensor q, k, v, o, lse;
};

Forward run_forward(const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
                    bool causal, double scale) {
  const Dims d = dims_of(query, key, value);
  const int e = elem_index(query);
  Forward f{aligned(query), aligned(key), aligned(value), at::Tensor(), at::Tensor()};
  c10::DeviceGuard guard(f.q.device());
  f.o = at::empty_like(f.q);
  f.lse = at::empty({d.B, d.Hq, d.N}, f.q.options().dtype(at::kFloat));
  const int c = causal ? 1 : 0;
  const float s = static_cast<float>(scale);
  const int64_t ws_bytes = g.fwd_ws_bytes(d.B, d.Hq, d.Hkv, d.N, d.Nkv, d.D, c);
  const at::Tensor ws = workspace(ws_bytes, f.q);
  void* stream = stream_of(f.q);
  if (ws_bytes > 0)
    check(g.fwd_ws[e](f.q.data_ptr(), f.k.data_ptr(), f.v.data_ptr(), f.o.data_ptr(),
                      f.lse.data_ptr(), d.B, d.Hq, d.Hkv, d.N, d.Nkv, d.D, s, c, ws.data_ptr(),
                      ws_bytes, stream));
  else
    check(g.fwd_kv[e](f.q.data_ptr(), f.k.data_ptr(), f.v.data_ptr(), f.o.data_ptr(),
                      f.lse.data_ptr(), d.B, d.Hq, d.Hkv, d.N, d.Nkv, d.D, s, c, stream));
  return f;
}

class FlashAttention : public torch::autograd::Function<FlashAttention> {
 public:
  static at::Tensor forward(torch::autograd::AutogradContext* ctx, const at::Tensor& query,
                            const at::Tensor& key, const at::Tensor& value, bool causal,
                            double scale) {
    Forward f = run_forward(query, key, value, causal, scale);
    ctx->save_for_backward({f.q, f.k, f.v, f.o, f.lse});
    ctx->saved_data["causal"] = causal;
    ctx->saved_data["scale"] = scale;
    return f.o;
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    const auto saved = ctx->get_saved_variables();
    const at::Tensor &q = saved[0], &k = saved[1], &v = saved[2], &o = saved[3], &lse = saved[4];
    const bool causal = ctx->saved_data["causal"].toBool();
    const float s = static_cast<float>(ctx->saved_data["scale"].toDouble());
    const Dims d = dims_of(q, k, v);
    const int e = elem_index(q);
    const at::Tensor dO = aligned(grads[0]);
    c10::DeviceGuard guard(q.device());
    const int c = causal ? 1 : 0;
    const int64_t ws_bytes = g.bwd_ws_bytes(d.B, d.Hq, d.Hkv, d.N, d.Nkv, d.D, c);
    at::Tensor delta = at::empty({d.B, d.Hq, d.N}, q.options().dtype(at::kFloat));
    at::Tensor dq = at::empty_like(q), dk = at::empty_like(k), dv = at::empty_like(v);
    const at::Tensor ws = workspace(ws_bytes, q);
    check(g.bwd[e](q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), dO.data_ptr(),
                   lse.data_ptr(), delta.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                   d.B, d.Hq, d.Hkv, d.N, d.Nkv, d.D, s, c,
                   ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes, stream_of(q)));
    return {dq, dk, dv, at::Tensor(), at::Tensor()};
  }
};

// O = attention(query, key, value) with the library's kernels, differentiable
// in query, key and value (see the file comment for the cases served).
at::Tensor attention(const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
                     bool causal, double scale) {
  if (!ready()) throw std::runtime_error("gfx950 attention: init() has not run");
  return FlashAttention::apply(query, key, value, causal, scale);
}

// O without autograd (inference: no input needs a gradient).
at::Tensor forward_only(const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
                        bool causal, double scale) {
  if (!ready()) throw std::runtime_error("gfx950 attention: init() has not run");
  return run_forward(query, key, value, causal, scale).o;
}

// Takes the entry points' addresses: fa_fwd_kv, fa_fwd_kv_bf16, fa_fwd_ws,
// fa_fwd_ws_bf16, fa_bwd, fa_bwd_bf16, fa_fwd_workspace_bytes,
// fa_bwd_workspace_bytes, fa_last_error.
void init(int64_t fwd_kv, int64_t fwd_kv_bf16, int64_t fwd_ws, int64_t fwd_ws_bf16, int64_t bwd,
          int64_t bwd_bf16, int64_t fwd_ws_bytes, int64_t bwd_ws_bytes, int64_t last_error) {
  auto fn = [](int64_t a) { return reinterpret_cast<void*>(static_cast<uintptr_t>(a)); };
  Entries e;
  e.fwd_kv[0] = reinterpret_cast<FwdKv>(fn(fwd_kv));
  e.fwd_kv[1] = reinterpret_cast<FwdKv>(fn(fwd_kv_bf16));
  e.fwd_ws[0] = reinterpret_cast<FwdWs>(fn(fwd_ws));
  e.fwd_ws[1] = reinterpret_cast<FwdWs>(fn(fwd_ws_bf16));
  e.bwd[0] = reinterpret_cast<Bwd>(fn(bwd));
  e.bwd[1] = reinterpret_cast<Bwd>(fn(bwd_bf16));
  e.fwd_ws_bytes = reinterpret_cast<WsBytes>(fn(fwd_ws_bytes));
  e.bwd_ws_bytes = reinterpret_cast<WsBytes>(fn(bwd_ws_bytes));
  e.last_error = reinterpret_cast<LastError>(fn(last_error));
  g = e;
  if (!ready()) throw std::invalid_argument("gfx950 attention: a null entry point was passed");
}

}  // namespace

PYBIND11_MODULE(_fa_native, m) {
  m.doc() = "C++ autograd binding of libfa_gfx950.so (fa_fwd_kv / fa_fwd_ws and fa_bwd)";
  m.def("init", &init);
  m.def("ready", &ready);
  m.def("attention", &attention);
  m.def("forward", &forward_only);
}
