// Native per-token decode entry for the Python host (torch extension).
//
// The hot path of tao_attention_decode (operator.py:130-138 ->
// StreamCache.decode) is one call per token per layer. This object is built
// by the Python host after the full argument checks of a decode call; later
// calls with operands of the same layout go through call(): it re-checks
// every operand (shape, strides, dtype, device, 16-byte alignment) and the
// fusion parameters against the checked layout, writes the operand pointers
// into the C-ABI token struct, allocates the output and calls
// tao_stream_decode (include/tao_memory.h). Any mismatch returns None and
// the host falls back to its full checks; driver errors raise with the
// library's message. No arithmetic happens here.
#include <torch/extension.h>

#include <array>
#include <cstdint>
#include <vector>

#include "../../../include/tao_memory.h"

namespace {

using StreamDecodeFn = int (*)(void*, const tao_tokens*, const tao_fusion*, void*,
                               const int64_t*, void*, int64_t*);
using LastErrorFn = const char* (*)();

class DecodeCall {
 public:
  DecodeCall(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& rq,
             const at::Tensor& rk, const at::Tensor& fa, const at::Tensor& fb, double alpha,
             uintptr_t fn, uintptr_t last_error, uintptr_t handle, uintptr_t tok,
             uintptr_t fu, uintptr_t info, uintptr_t out_s)
      : sizes_(q.sizes().vec()),
        device_(q.device()),
        fa_impl_(fa.unsafeGetTensorImpl()),
        fb_impl_(fb.unsafeGetTensorImpl()),
        fa_ptr_(fa.data_ptr()),
        fb_ptr_(fb.data_ptr()),
        alpha_(alpha),
        fn_(reinterpret_cast<StreamDecodeFn>(fn)),
        last_error_(reinterpret_cast<LastErrorFn>(last_error)),
        handle_(reinterpret_cast<void*>(handle)),
        tok_(reinterpret_cast<tao_tokens*>(tok)),
        fu_(reinterpret_cast<const tao_fusion*>(fu)),
        info_(reinterpret_cast<int64_t*>(info)),
        out_s_(reinterpret_cast<const int64_t*>(out_s)) {
    const at::Tensor* ts[5] = {&q, &k, &v, &rq, &rk};
    for (int i = 0; i < 5; ++i) strides_[i] = ts[i]->strides().vec();
  }

  // Returns the output tensor (eager), True (graph replay: the heads are in
  // the epoch's output buffer, info[5]) or None (layout differs: take the
  // full path).
  py::object call(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                  const at::Tensor& rq, const at::Tensor& rk, const at::Tensor& fa,
                  const at::Tensor& fb, double alpha, int64_t position, uintptr_t stream) {
    const at::Tensor* ts[5] = {&q, &k, &v, &rq, &rk};
    void* ptrs[5];
    for (int i = 0; i < 5; ++i) {
      const at::Tensor& t = *ts[i];
      if (t.scalar_type() != at::kBFloat16 || t.device() != device_ ||
          t.sizes() != at::IntArrayRef(sizes_) || t.strides() != at::IntArrayRef(strides_[i]))
        return py::none();
      ptrs[i] = t.data_ptr();
      if (reinterpret_cast<uintptr_t>(ptrs[i]) & 15) return py::none();
    }
    if (fa.unsafeGetTensorImpl() != fa_impl_ || fb.unsafeGetTensorImpl() != fb_impl_ ||
        fa.data_ptr() != fa_ptr_ || fb.data_ptr() != fb_ptr_ || alpha != alpha_)
      return py::none();
    tok_->q = ptrs[0];
    tok_->k = ptrs[1];
    tok_->v = ptrs[2];
    tok_->raw_q = ptrs[3];
    tok_->raw_k = ptrs[4];
    (void)position;
    at::Tensor out = at::empty_like(q);
    const int rc = fn_(handle_, tok_, fu_, out.data_ptr(), out_s_,
                       reinterpret_cast<void*>(stream), info_);
    if (rc < 0) throw py::value_error(last_error_());
    if (rc > 0) throw std::runtime_error(std::string("HIP error: ") + last_error_());
    if (info_[5]) return py::bool_(true);
    return py::cast(out);
  }

 private:
  std::vector<int64_t> sizes_;
  std::array<std::vector<int64_t>, 5> strides_;
  c10::Device device_;
  const void* fa_impl_;
  const void* fb_impl_;
  const void* fa_ptr_;
  const void* fb_ptr_;
  double alpha_;
  StreamDecodeFn fn_;
  LastErrorFn last_error_;
  void* handle_;
  tao_tokens* tok_;
  const tao_fusion* fu_;
  int64_t* info_;
  const int64_t* out_s_;
};

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  py::class_<DecodeCall>(m, "DecodeCall")
      .def(py::init<const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                    const at::Tensor&, const at::Tensor&, const at::Tensor&, double, uintptr_t,
                    uintptr_t, uintptr_t, uintptr_t, uintptr_t, uintptr_t, uintptr_t>())
      .def("__call__", &DecodeCall::call);
}
