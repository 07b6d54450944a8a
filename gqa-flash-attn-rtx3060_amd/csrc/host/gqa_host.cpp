// gqa_host.cpp — torch-tensor bindings of the split-KV decode call and of
// the paged-cache launches.
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
// boundary is unchanged; only the marshalling moves out of Python.  The
// paged routes (paged_forward: split-KV first pass + combine, single pass,
// key chunks) and the paged cache write get the same treatment: through
// ctypes a paged decode step spent ~18 us on the host against ~10 us of
// kernels.
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

[[noreturn]] void raise_rc(int rc, const char* what) {
  py::module_::import("gqa_kernels._lib").attr("check")(rc);
  throw std::runtime_error(std::string(what) + " failed: " + gqa_strerror(rc));
}

// The three kernel routes of paged attention (gqa_kernels.paged.paged_attention,
// after its checks and route choice), launched from the tensors:
//   route 0: gqa_paged_split_first_launch into ws, then the combine into out
//            (gqa_split_reduce_varlen_launch with variable query lengths,
//            else gqa_split_reduce_lse_launch or gqa_split_reduce_launch);
//   route 1: gqa_paged_fwd_launch, or with `splits` > 0 split query blocks
//            gqa_paged_fwd_split_launch (ws, zeroed counters);
//   route 2: gqa_paged_fwd_chunks_launch (ws, `splits` key chunks).
// q and out are (batch, heads, seq_q, head_dim), or token-major
// (tokens, heads, head_dim) when q_start / q_len are given.
void paged_forward(int64_t route, const at::Tensor& q, const at::Tensor& k_cache, const at::Tensor& v_cache,
                   const at::Tensor& block_table, int64_t table_stride, const at::Tensor& seq_lens,
                   const std::optional<at::Tensor>& q_start, const std::optional<at::Tensor>& q_len,
                   int64_t max_seq_len, const at::Tensor& out, const std::optional<at::Tensor>& lse,
                   const std::optional<at::Tensor>& ws, const std::optional<at::Tensor>& counters,
                   int64_t splits, int64_t batch, int64_t seq_q,
                   double scale_log2, bool causal, int64_t dtype) {
  if (k_cache.dim() != 4 || v_cache.dim() != 4) throw std::invalid_argument("paged_forward: 4-d caches expected");
  const bool varlen = q_start.has_value() && q_len.has_value();
  if (varlen ? q.dim() != 3 || out.dim() != 3 : q.dim() != 4 || out.dim() != 4)
    throw std::invalid_argument("paged_forward: q / out rank does not match the query layout");
  if ((route != 1 || splits > 0) && !ws.has_value()) throw std::invalid_argument("paged_forward: workspace expected");
  if (route == 1 && splits > 0 && !counters.has_value())
    throw std::invalid_argument("paged_forward: counters expected");
  const int H = static_cast<int>(q.size(1)), D = static_cast<int>(q.size(-1));
  const int Hkv = static_cast<int>(k_cache.size(2)), bs = static_cast<int>(k_cache.size(1));
  int64_t qs[4], os[4], ks[4], vs[4];
  if (varlen) {
    const int64_t qv[4] = {0, q.stride(1), q.stride(0), 1}, ov[4] = {0, out.stride(1), out.stride(0), 1};
    for (int i = 0; i < 4; ++i) qs[i] = qv[i], os[i] = ov[i];
  } else {
    strides_of(q, qs);
    strides_of(out, os);
  }
  strides_of(k_cache, ks);
  strides_of(v_cache, vs);
  const int* qst = varlen ? q_start->data_ptr<int>() : nullptr;
  const int* qln = varlen ? q_len->data_ptr<int>() : nullptr;
  float* lse_p = lse.has_value() ? lse->data_ptr<float>() : nullptr;
  float* ws_p = ws.has_value() ? ws->data_ptr<float>() : nullptr;
  const int B = static_cast<int>(batch), Sq = static_cast<int>(seq_q), S = static_cast<int>(splits);
  const int dt = static_cast<int>(dtype), ms = static_cast<int>(max_seq_len), ts = static_cast<int>(table_stride);
  const float sl2 = static_cast<float>(scale_log2);
  hipStream_t stream = c10::hip::getCurrentHIPStream(q.get_device()).stream();
  const int* table = block_table.data_ptr<int>();
  const int* lens = seq_lens.data_ptr<int>();
  int rc;
  if (route == 1 && S > 0) {
    rc = gqa_paged_fwd_split_launch(q.data_ptr(), qs, k_cache.data_ptr(), ks, v_cache.data_ptr(), vs, table, ts,
                                    lens, qst, qln, bs, ms, out.data_ptr(), os, lse_p, ws_p,
                                    counters->data_ptr<int>(), S, B, H, Hkv, Sq, D, sl2, causal ? 1 : 0, dt, stream);
    if (rc != GQA_OK) raise_rc(rc, "gqa_paged_fwd_split_launch");
    return;
  }
  if (route == 1) {
    rc = gqa_paged_fwd_launch(q.data_ptr(), qs, k_cache.data_ptr(), ks, v_cache.data_ptr(), vs, table, ts, lens,
                              qst, qln, bs, ms, out.data_ptr(), os, lse_p, B, H, Hkv, Sq, D, sl2, causal ? 1 : 0,
                              dt, stream);
    if (rc != GQA_OK) raise_rc(rc, "gqa_paged_fwd_launch");
    return;
  }
  if (route == 2) {
    rc = gqa_paged_fwd_chunks_launch(q.data_ptr(), qs, k_cache.data_ptr(), ks, v_cache.data_ptr(), vs, table, ts,
                                     lens, qst, qln, bs, ms, out.data_ptr(), os, lse_p, ws_p, S, B, H, Hkv, Sq, D,
                                     sl2, causal ? 1 : 0, dt, stream);
    if (rc != GQA_OK) raise_rc(rc, "gqa_paged_fwd_chunks_launch");
    return;
  }
  if (route != 0) throw std::invalid_argument("paged_forward: route must be 0, 1 or 2");
  rc = gqa_paged_split_first_launch(q.data_ptr(), qs, k_cache.data_ptr(), ks, v_cache.data_ptr(), vs, table, ts,
                                    lens, qst, qln, bs, ms, ws_p, S, B, H, Hkv, Sq, D, sl2, causal ? 1 : 0, dt,
                                    stream);
  if (rc != GQA_OK) raise_rc(rc, "gqa_paged_split_first_launch");
  if (varlen)
    rc = gqa_split_reduce_varlen_launch(ws_p, S, out.data_ptr(), os, lse_p, qst, qln, B, H, Sq, D, dt, stream);
  else if (lse_p != nullptr)
    rc = gqa_split_reduce_lse_launch(ws_p, S, out.data_ptr(), os, lse_p, B, H, Sq, D, dt, stream);
  else
    rc = gqa_split_reduce_launch(ws_p, S, out.data_ptr(), os, B, H, Sq, D, dt, stream);
  if (rc != GQA_OK) raise_rc(rc, "gqa_split_reduce_launch");
}

// gqa_paged_cache_write_launch from the tensors (gqa_kernels.paged.write_kv
// after its checks): key / value (tokens, kv heads, head_dim), int64 slots.
void cache_write(const at::Tensor& key, const at::Tensor& value, const at::Tensor& k_cache,
                 const at::Tensor& v_cache, const at::Tensor& slot_mapping, int64_t dtype) {
  if (key.dim() != 3 || value.dim() != 3 || k_cache.dim() != 4 || v_cache.dim() != 4)
    throw std::invalid_argument("cache_write: 3-d key / value and 4-d caches expected");
  const int64_t kst[3] = {key.stride(0), key.stride(1), key.stride(2)};
  const int64_t vst[3] = {value.stride(0), value.stride(1), value.stride(2)};
  int64_t kcs[4], vcs[4];
  strides_of(k_cache, kcs);
  strides_of(v_cache, vcs);
  hipStream_t stream = c10::hip::getCurrentHIPStream(key.get_device()).stream();
  const int rc = gqa_paged_cache_write_launch(
      key.data_ptr(), kst, value.data_ptr(), vst, k_cache.data_ptr(), kcs, v_cache.data_ptr(), vcs,
      slot_mapping.data_ptr<int64_t>(), static_cast<int>(key.size(0)), static_cast<int>(key.size(1)),
      static_cast<int>(key.size(2)), static_cast<int>(k_cache.size(1)), static_cast<int>(dtype), stream);
  if (rc != GQA_OK) raise_rc(rc, "gqa_paged_cache_write_launch");
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "torch-tensor binding of gqa_split_launch (the split-KV decode step)";
  m.def("split_decode", &split_decode, "split-KV decode: first pass and combine through gqa_split_launch",
        py::arg("q"), py::arg("k"), py::arg("v"), py::arg("ws"), py::arg("splits"), py::arg("causal"),
        py::arg("scale_log2"), py::arg("dtype"), py::arg("return_lse"));
  m.def("paged_forward", &paged_forward, "paged attention: one of the three kernel routes from tensors",
        py::arg("route"), py::arg("q"), py::arg("k_cache"), py::arg("v_cache"), py::arg("block_table"),
        py::arg("table_stride"), py::arg("seq_lens"), py::arg("q_start"), py::arg("q_len"), py::arg("max_seq_len"),
        py::arg("out"), py::arg("lse"), py::arg("ws"), py::arg("counters"), py::arg("splits"), py::arg("batch"),
        py::arg("seq_q"),
        py::arg("scale_log2"), py::arg("causal"), py::arg("dtype"));
  m.def("cache_write", &cache_write, "store new tokens' K/V at their paged cache slots", py::arg("key"),
        py::arg("value"), py::arg("k_cache"), py::arg("v_cache"), py::arg("slot_mapping"), py::arg("dtype"));
  m.attr("ABI_VERSION") = gqa_abi_version();
}
