// Thin pybind11 binding of the per-call hot entry points for torch callers.
//
// The reference's callers issue one gather/scatter call per chunk or per
// layer (lmcache_ascend/v1/npu_connector/npu_connectors.py:1146-1158,
// 608-616), so host cost per call matters.  This module reads at::Tensor
// geometry and the current HIP stream in C++ and calls the C ABI of
// liblmcache_amd.so directly; argument meaning, defaults and exception types
// are those of the reference's pybind module (csrc/pybind.cpp:364-481).
//
// The module does not link liblmcache_amd.so: `bind()` receives the
// addresses of the C ABI functions from the library instance the Python
// package already loaded, so both call paths share one library.
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <cstdint>
#include <string>
#include <vector>

#include "../../include/lmcache_amd.h"

namespace py = pybind11;

namespace {

using MultiFn = int (*)(const lmc_tensor *, const lmc_tensor *, const lmc_tensor *, int32_t, int64_t,
                        int32_t, int32_t, int32_t, int64_t, int64_t, int64_t, void *);
using SingleFn = int (*)(const lmc_tensor *, const lmc_tensor *, int32_t, const lmc_tensor *, int32_t,
                         int32_t, int32_t, int32_t, int64_t, int64_t, int64_t, void *);
using FlashFn = int (*)(const lmc_tensor *, const lmc_tensor *, const lmc_tensor *, const lmc_tensor *,
                        int32_t, void *);
using RopeFn = int (*)(const lmc_tensor *, const lmc_tensor *, const lmc_tensor *, int64_t,
                       const lmc_tensor *, int32_t, void *);
using BlendFn = int (*)(const lmc_tensor *, int32_t, const int64_t *, const lmc_tensor *, int32_t,
                        const lmc_tensor *, const lmc_tensor *, const lmc_tensor *, const lmc_tensor *,
                        int64_t, int32_t, int32_t, int32_t, void *);
using CdfFn = int (*)(const lmc_tensor *, int32_t, const lmc_tensor *, void *);
using Codec4Fn = int (*)(const lmc_tensor *, const lmc_tensor *, const lmc_tensor *, const lmc_tensor *, void *);
using ErrFn = const char *(*)();

struct Table {
  MultiFn multi = nullptr;
  SingleFn single = nullptr;
  FlashFn load_flash = nullptr;
  FlashFn reshape_flash = nullptr;
  RopeFn rope = nullptr;
  BlendFn blend = nullptr;
  CdfFn cdf = nullptr;
  Codec4Fn encode = nullptr;
  Codec4Fn decode = nullptr;
  ErrFn last_error = nullptr;
} g;

int32_t dtype_code(at::ScalarType t) {
  switch (t) {
  case at::kByte: return LMC_U8;
  case at::kChar: return LMC_I8;
  case at::kShort: return LMC_I16;
  case at::kInt: return LMC_I32;
  case at::kLong: return LMC_I64;
  case at::kHalf: return LMC_F16;
  case at::kBFloat16: return LMC_BF16;
  case at::kFloat: return LMC_F32;
  default: throw std::runtime_error("tensor dtype has no lmc_tensor code");
  }
}

lmc_tensor desc(const at::Tensor &t) {
  lmc_tensor d{};
  const int64_t n = t.dim();
  if (n > LMC_MAX_DIMS) throw std::runtime_error("tensors of more than 6 dims are not supported");
  d.data = t.data_ptr();
  d.dtype = dtype_code(t.scalar_type());
  if (t.is_cuda()) d.device = t.get_device();
  else if (t.is_cpu()) d.device = -1;
  else throw std::runtime_error("Invalid device. Device must be a GPU or pinned cpu.");
  d.ndim = static_cast<int32_t>(n);
  const auto sz = t.sizes();
  const auto st = t.strides();
  for (int64_t i = 0; i < n; ++i) {
    d.sizes[i] = sz[i];
    d.strides[i] = st[i];
  }
  return d;
}

void check_bound() {
  if (g.last_error == nullptr) throw std::runtime_error("lmcache_amd binding used before bind()");
}

void raise_for(int status) {
  if (status == LMC_OK) return;
  const std::string msg = g.last_error ? g.last_error() : "";
  if (status == LMC_ERR_VALUE) throw py::value_error(msg);
  if (status == LMC_ERR_NOT_IMPLEMENTED) {
    PyErr_SetString(PyExc_NotImplementedError, msg.c_str());
    throw py::error_already_set();
  }
  throw std::runtime_error(msg);
}

void *stream_of(int device) { return c10::hip::getCurrentHIPStream(device).stream(); }

int device_of(const at::Device &d, const at::Tensor &fallback) {
  if (d.is_cuda()) return d.has_index() ? d.index() : c10::hip::current_device();
  if (fallback.is_cuda()) return fallback.get_device();
  return c10::hip::current_device();
}

void multi_layer_kv_transfer(at::Tensor &key_value, const at::Tensor &key_value_ptrs,
                             const at::Tensor &slot_mapping, const at::Device &paged_memory_device,
                             int64_t page_buffer_size, bool direction, bool use_mla,
                             int64_t kvcache_format_raw, int64_t k_hidden_dims,
                             int64_t v_hidden_dims, int64_t dsa_hidden_dims) {
  check_bound();
  const int dev = device_of(paged_memory_device, key_value_ptrs);
  const lmc_tensor a = desc(key_value), p = desc(key_value_ptrs), s = desc(slot_mapping);
  raise_for(g.multi(&a, &p, &s, dev, page_buffer_size, direction, use_mla,
                    static_cast<int32_t>(kvcache_format_raw), k_hidden_dims, v_hidden_dims,
                    dsa_hidden_dims, stream_of(dev)));
}

std::vector<at::Tensor> normalize_kv_caches(const py::object &obj) {
  // csrc/pybind.cpp:22-31: a Tensor or a tuple of Tensors.
  if (THPVariable_Check(obj.ptr())) return {obj.cast<at::Tensor>()};
  if (py::isinstance<py::tuple>(obj)) return obj.cast<std::vector<at::Tensor>>();
  throw std::runtime_error("vllm_kv_caches is neither a Tensor nor a tuple of Tensors");
}

void single_layer_kv_transfer(at::Tensor &lmc, const py::object &caches_obj,
                              const at::Tensor &slot_mapping, bool direction,
                              int64_t kvcache_format_raw, bool token_major, bool vllm_two_major,
                              int64_t k_hidden_dims, int64_t v_hidden_dims,
                              int64_t dsa_hidden_dims) {
  check_bound();
  const std::vector<at::Tensor> caches = normalize_kv_caches(caches_obj);
  std::vector<lmc_tensor> cd;
  cd.reserve(caches.size());
  int dev = -1;
  for (const auto &c : caches) {
    cd.push_back(desc(c));
    if (dev < 0 && c.is_cuda()) dev = c.get_device();
  }
  if (dev < 0) dev = slot_mapping.is_cuda() ? slot_mapping.get_device() : c10::hip::current_device();
  const lmc_tensor a = desc(lmc), s = desc(slot_mapping);
  raise_for(g.single(&a, cd.data(), static_cast<int32_t>(cd.size()), &s, direction,
                     static_cast<int32_t>(kvcache_format_raw), token_major, vllm_two_major,
                     k_hidden_dims, v_hidden_dims, dsa_hidden_dims, stream_of(dev)));
}

void flash(FlashFn fn, at::Tensor &kv, at::Tensor &kc, at::Tensor &vc, at::Tensor &slots,
           int64_t layer_idx) {
  check_bound();
  const int dev = kc.is_cuda() ? kc.get_device() : c10::hip::current_device();
  const lmc_tensor a = desc(kv), k = desc(kc), v = desc(vc), s = desc(slots);
  raise_for(fn(&a, &k, &v, &s, static_cast<int32_t>(layer_idx), stream_of(dev)));
}

void rotary_embedding_k_fused(const at::Tensor &old_pos, const at::Tensor &new_pos, at::Tensor &key,
                              int64_t head_size, const at::Tensor &cos_sin_cache, bool is_neox) {
  check_bound();
  const int dev = key.is_cuda() ? key.get_device() : c10::hip::current_device();
  const lmc_tensor a = desc(old_pos), b = desc(new_pos), k = desc(key), c = desc(cos_sin_cache);
  raise_for(g.rope(&a, &b, &k, head_size, &c, is_neox, stream_of(dev)));
}

// One layer of the CacheBlend retrieve in one kernel (lmc_blend_layer_to_paged).
// Returns false when the library answers LMC_ERR_NOT_IMPLEMENTED (a shape
// the fused kernel does not take), before any work, so the caller can run
// the connector's own sequence; every other failure raises.
bool blend_layer_to_paged(const std::vector<at::Tensor> &objs, const std::vector<int64_t> &token_starts,
                          const py::object &caches_obj, const at::Tensor &slot_mapping,
                          const c10::optional<at::Tensor> &old_positions,
                          const c10::optional<at::Tensor> &new_positions,
                          const c10::optional<at::Tensor> &cos_sin_cache, int64_t head_size, bool is_neox,
                          int64_t kvcache_format_raw, bool vllm_two_major) {
  check_bound();
  if (objs.size() != token_starts.size()) throw py::value_error("memory_objs and token_starts differ in length");
  const std::vector<at::Tensor> caches = normalize_kv_caches(caches_obj);
  std::vector<lmc_tensor> cd, od;
  cd.reserve(caches.size());
  od.reserve(objs.size());
  int dev = -1;
  for (const auto &c : caches) {
    cd.push_back(desc(c));
    if (dev < 0 && c.is_cuda()) dev = c.get_device();
  }
  if (dev < 0) dev = slot_mapping.is_cuda() ? slot_mapping.get_device() : c10::hip::current_device();
  for (const auto &o : objs) od.push_back(desc(o));
  const bool rope = old_positions.has_value() || new_positions.has_value();
  if (rope && !(old_positions.has_value() && new_positions.has_value() && cos_sin_cache.has_value()))
    throw py::value_error("old_positions, new_positions and cos_sin_cache go together");
  const lmc_tensor s = desc(slot_mapping);
  lmc_tensor a{}, b{}, c{};
  if (rope) {
    a = desc(*old_positions);
    b = desc(*new_positions);
    c = desc(*cos_sin_cache);
  }
  const int status = g.blend(od.data(), static_cast<int32_t>(od.size()), token_starts.data(), cd.data(),
                             static_cast<int32_t>(cd.size()), &s, rope ? &a : nullptr, rope ? &b : nullptr,
                             rope ? &c : nullptr, head_size, is_neox, static_cast<int32_t>(kvcache_format_raw),
                             vllm_two_major, stream_of(dev));
  if (status == LMC_ERR_NOT_IMPLEMENTED) return false;
  raise_for(status);
  return true;
}

// CacheGen (csrc/cachegen_kernels.cpp:17-155).  calculate_cdf returns an
// int16 [L, C, n_bins + 1] tensor; the reference zero-fills it first, but
// the kernels write every entry of it, so it is allocated without a fill.
at::Tensor calculate_cdf(const at::Tensor &input, int64_t n_bins) {
  check_bound();
  if (!input.is_cuda()) throw std::runtime_error("calculate_cdf: input must be a GPU tensor");
  if (input.dim() != 3) throw std::runtime_error("input must be [layers, tokens, channels]");
  at::Tensor out = at::empty({input.size(0), input.size(2), n_bins + 1},
                             input.options().dtype(at::kShort));
  const lmc_tensor a = desc(input), o = desc(out);
  raise_for(g.cdf(&a, static_cast<int32_t>(n_bins), &o, stream_of(input.get_device())));
  return out;
}

void codec4(Codec4Fn fn, const at::Tensor &t0, const at::Tensor &t1, const at::Tensor &t2,
            const at::Tensor &t3, const at::Tensor &dev_of) {
  check_bound();
  const int dev = dev_of.is_cuda() ? dev_of.get_device() : c10::hip::current_device();
  const lmc_tensor a = desc(t0), b = desc(t1), c = desc(t2), d = desc(t3);
  raise_for(fn(&a, &b, &c, &d, stream_of(dev)));
}

void bind(uintptr_t multi, uintptr_t single, uintptr_t load_flash, uintptr_t reshape_flash,
          uintptr_t rope, uintptr_t blend, uintptr_t cdf, uintptr_t encode, uintptr_t decode,
          uintptr_t last_error) {
  g.multi = reinterpret_cast<MultiFn>(multi);
  g.single = reinterpret_cast<SingleFn>(single);
  g.load_flash = reinterpret_cast<FlashFn>(load_flash);
  g.reshape_flash = reinterpret_cast<FlashFn>(reshape_flash);
  g.rope = reinterpret_cast<RopeFn>(rope);
  g.blend = reinterpret_cast<BlendFn>(blend);
  g.cdf = reinterpret_cast<CdfFn>(cdf);
  g.encode = reinterpret_cast<Codec4Fn>(encode);
  g.decode = reinterpret_cast<Codec4Fn>(decode);
  g.last_error = reinterpret_cast<ErrFn>(last_error);
}

} // namespace

PYBIND11_MODULE(_c_ops_ext, m) {
  m.def("bind", &bind);
  m.def("multi_layer_kv_transfer", &multi_layer_kv_transfer);
  m.def("single_layer_kv_transfer", &single_layer_kv_transfer, py::arg("lmc_key_value_cache"),
        py::arg("vllm_kv_caches"), py::arg("slot_mapping"), py::arg("direction"),
        py::arg("kvcache_format_raw"), py::arg("token_major") = false,
        py::arg("vllm_two_major") = false, py::arg("k_hidden_dims") = 0,
        py::arg("v_hidden_dims") = 0, py::arg("dsa_hidden_dims") = 0);
  m.def("load_and_reshape_flash",
        [](at::Tensor &kv, at::Tensor &kc, at::Tensor &vc, at::Tensor &s, int64_t layer) {
          flash(g.load_flash, kv, kc, vc, s, layer);
        });
  m.def("reshape_and_cache_back_flash",
        [](at::Tensor &kv, at::Tensor &kc, at::Tensor &vc, at::Tensor &s, int64_t layer) {
          flash(g.reshape_flash, kv, kc, vc, s, layer);
        });
  m.def("rotary_embedding_k_fused", &rotary_embedding_k_fused);
  m.def("blend_layer_to_paged", &blend_layer_to_paged);
  m.def("calculate_cdf", &calculate_cdf);
  m.def("encode_fast_new", [](const at::Tensor &cdf, const at::Tensor &sym, at::Tensor &out, at::Tensor &lens) {
    codec4(g.encode, cdf, sym, out, lens, sym);
  });
  m.def("decode_fast_prefsum",
        [](const at::Tensor &cdf, const at::Tensor &bytes, const at::Tensor &lens, at::Tensor &out) {
          codec4(g.decode, cdf, bytes, lens, out, bytes);
        });
}
