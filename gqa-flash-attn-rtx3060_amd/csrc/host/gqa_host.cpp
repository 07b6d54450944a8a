// gqa_host.cpp — torch-tensor binding of the split-KV decode call.
//
// The decode route of gqa_flash_attn (reference gqa_kernels/dispatch.py:49-56,
// gqa_split.py:153-194) is one gqa_split_launch per step.  Driven through
// ctypes, building its 21 arguments (four stride arrays, pointers read off
// the tensors one Python call at a time) costs more host time per step than
// the GPU spends on a short cache (8192 keys: ~12.5 us of host time against
// ~9.8 us of kernels), so a loop of decode steps waits on the host.  This
// binding takes the tensors themselves, reads pointers, strides and the
// current HIP stream natively, allocates the output (and LSE) with torch,
// and calls the same C entry point (include/gqa_attn.h) — the library
// boundary is unchanged; only the marshalling moves out of Python.
//
// Host-only C++ (no kernels); built by build.py into gqa_kernels/ next to
// libgqa_hip.so, which it links against.
#include <torch/extension.h>

#include <c10/hip/HIPStream.h>

#include <stdexcept>
#include <string>

#include "gqa_attn.h"

namespace {

void strides_of(const at::Tensor& t, int64_t (&s)[4]) {
  for (int i = 0; i < 4; ++i) s[i] = t.stride(i);
}

// q, k, v: 4-d (B, H, S, D) tensors the kernels can read (unit last-dim
// stride, 16-byte aligned rows — the caller's fast-path test, checked again
// by the C entry point); ws: the stream's fp32 workspace of at least
// gqa_split_workspace_bytes(...) bytes.  Returns o, or (o, lse).
py::object split_decode(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& ws,
                        int64_t splits, bool causal, double scale_log2, int64_t dtype, bool return_lse) {
  if (q.dim() != 4 || k.dim() != 4 || v.dim() != 4) throw std::invalid_argument("split_decode: 4-d q, k, v expected");
  if (ws.scalar_type() != at::kFloat) throw std::invalid_argument("split_decode: fp32 workspace expected");
  const int64_t B = q.size(0), Hq = q.size(1), Sq = q.size(2), D = q.size(3);
  const int64_t Hkv = k.size(1), Skv = k.size(2);
  at::Tensor o = at::empty_like(q);
  at::Tensor lse;
  if (return_lse) lse = at::empty({B, Hq, Sq}, q.options().dtype(at::kFloat));
  int64_t qs[4], ks[4], vs[4], os[4];
  strides_of(q, qs);
  strides_of(k, ks);
  strides_of(v, vs);
  strides_of(o, os);
  hipStream_t stream = c10::hip::getCurrentHIPStream(q.get_device()).stream();
  const int rc = gqa_split_launch(q.data_ptr(), qs, k.data_ptr(), ks, v.data_ptr(), vs, o.data_ptr(), os,
                                  return_lse ? lse.data_ptr<float>() : nullptr, ws.data_ptr<float>(),
                                  static_cast<int>(splits), static_cast<int>(B), static_cast<int>(Hq),
                                  static_cast<int>(Hkv), static_cast<int>(Sq), static_cast<int>(Skv),
                                  static_cast<int>(D), static_cast<float>(scale_log2), causal ? 1 : 0,
                                  static_cast<int>(dtype), stream);
  if (rc != GQA_OK) {
    // The package's own error path (gqa_kernels._lib.check raises GQAError
    // with the library's message), as for the ctypes-bound entry points.
    py::module_::import("gqa_kernels._lib").attr("check")(rc);
    throw std::runtime_error(std::string("gqa_split_launch failed: ") + gqa_strerror(rc));
  }
  if (return_lse) return py::make_tuple(o, lse);
  return py::cast(o);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "torch-tensor binding of gqa_split_launch (the split-KV decode step)";
  m.def("split_decode", &split_decode, "split-KV decode: first pass and combine through gqa_split_launch",
        py::arg("q"), py::arg("k"), py::arg("v"), py::arg("ws"), py::arg("splits"), py::arg("causal"),
        py::arg("scale_log2"), py::arg("dtype"), py::arg("return_lse"));
  m.attr("ABI_VERSION") = gqa_abi_version();
}
