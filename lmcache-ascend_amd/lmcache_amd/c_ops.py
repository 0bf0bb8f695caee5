"""The `c_ops` operator surface of LMCache-Ascend, on MI355X.

Each function keeps the name, positional arity, argument meaning and
exception types of the reference's pybind module (csrc/pybind.cpp:243-483)
so the LMCache v1 engine, the vLLM connector and the CacheGen serde can call
it unchanged once `lmcache_amd.install()` has put this module at
`sys.modules["lmcache.c_ops"]`.

This layer only describes tensors (pointer, dtype, device, sizes, strides)
and picks the current HIP stream; planning, validation and the kernels live
behind the C ABI in liblmcache_amd.so (include/lmcache_amd.h).  Work is
enqueued on `torch.cuda.current_stream()` of the op's device, as the
reference enqueues on the current NPU stream (csrc/utils.cpp:96,203).
"""

from __future__ import annotations

import ctypes
from enum import IntEnum
from typing import Sequence

import torch

from . import _lib

_L = _lib.load()


def _addr(name: str) -> int:
    return ctypes.cast(getattr(_L, name), ctypes.c_void_p).value


# The C++ binding (csrc/torch_binding.cpp) reads tensor geometry and the HIP
# stream in C++ for the per-call entry points; it calls the functions of the
# library loaded above.  Without it the same functions are called through
# ctypes.
try:
    from . import _c_ops_ext as _ext

    _ext.bind(
        _addr("lmc_multi_layer_kv_transfer"),
        _addr("lmc_single_layer_kv_transfer"),
        _addr("lmc_load_and_reshape_flash"),
        _addr("lmc_reshape_and_cache_back_flash"),
        _addr("lmc_rotary_embedding_k_fused"),
        _addr("lmc_last_error"),
    )
except ImportError:
    _ext = None

_DTYPES = {
    torch.uint8: _lib.U8,
    torch.int8: _lib.I8,
    torch.int16: _lib.I16,
    torch.int32: _lib.I32,
    torch.int64: _lib.I64,
    torch.float16: _lib.F16,
    torch.bfloat16: _lib.BF16,
    torch.float32: _lib.F32,
}


class GPUKVFormat(IntEnum):
    """Layout enum upstream LMCache reads from c_ops; provided like the
    reference's mock (lmcache_ascend/__init__.py:349-361)."""

    NB_NL_TWO_BS_NH_HS = 0
    NL_X_TWO_NB_BS_NH_HS = 1
    NL_X_NB_TWO_BS_NH_HS = 2
    NL_X_NB_BS_HS = 3
    TWO_X_NL_X_NBBS_NH_HS = 4
    NL_X_NBBS_ONE_HS = 5
    NL_X_TWO_NB_NH_BS_HS = 6
    NL_X_NB_TWO_NH_BS_HS = 7


_DIMS = ctypes.c_int64 * _lib.MAX_DIMS


def _desc(t: torch.Tensor) -> _lib.LmcTensor:
    """lmc_tensor descriptor of a tensor (pointer, dtype, device, geometry)."""
    try:
        dt = _DTYPES[t.dtype]
    except KeyError:
        raise RuntimeError(f"ScalarType not supported: {t.dtype}") from None
    except AttributeError:
        raise TypeError(f"expected a torch.Tensor, got {type(t).__name__}") from None
    if t.is_cuda:
        idx = t.device.index
        dev = idx if idx is not None else torch.cuda.current_device()
    elif t.device.type == "cpu":
        dev = -1
    else:
        raise RuntimeError("Invalid device. Device must be a GPU or pinned cpu.")
    n = t.dim()
    if n > _lib.MAX_DIMS:
        raise RuntimeError(f"tensors of more than {_lib.MAX_DIMS} dims are not supported")
    return _lib.LmcTensor(t.data_ptr(), dt, dev, n, 0, _DIMS(*t.shape), _DIMS(*t.stride()))


def _ref(d: _lib.LmcTensor):
    return ctypes.byref(d)


def _device_index(*candidates) -> int:
    for c in candidates:
        if isinstance(c, torch.device):
            if c.type == "cuda":
                return c.index if c.index is not None else torch.cuda.current_device()
        elif isinstance(c, torch.Tensor) and c.is_cuda:
            return c.device.index
    return torch.cuda.current_device()


def _stream(device_index: int) -> int:
    return torch.cuda.current_stream(device_index).cuda_stream


def _run(status: int) -> None:
    if status != _lib.OK:
        _lib.raise_for(status)


# ---------------------------------------------------------------------------
# Paged-KV gather / scatter
# ---------------------------------------------------------------------------


def multi_layer_kv_transfer(
    key_value: torch.Tensor,
    key_value_ptrs: torch.Tensor,
    slot_mapping: torch.Tensor,
    paged_memory_device: torch.device,
    page_buffer_size: int,
    direction: bool,
    use_mla: bool,
    kvcache_format_raw: int,
    k_hidden_dims: int = 0,
    v_hidden_dims: int = 0,
    dsa_hidden_dims: int = 0,
) -> None:
    """csrc/mem_kernels.cpp:75-111.  direction=True: paged -> key_value."""
    if _ext is not None:
        _ext.multi_layer_kv_transfer(
            key_value, key_value_ptrs, slot_mapping, torch.device(paged_memory_device),
            int(page_buffer_size), bool(direction), bool(use_mla), int(kvcache_format_raw),
            int(k_hidden_dims), int(v_hidden_dims), int(dsa_hidden_dims),
        )
        return
    _multi_layer_kv_transfer_ctypes(
        key_value, key_value_ptrs, slot_mapping, paged_memory_device, page_buffer_size, direction,
        use_mla, kvcache_format_raw, k_hidden_dims, v_hidden_dims, dsa_hidden_dims,
    )


def _multi_layer_kv_transfer_ctypes(
    key_value, key_value_ptrs, slot_mapping, paged_memory_device, page_buffer_size, direction,
    use_mla, kvcache_format_raw, k_hidden_dims=0, v_hidden_dims=0, dsa_hidden_dims=0,
) -> None:
    dev = _device_index(paged_memory_device, key_value_ptrs)
    a, p, s = _desc(key_value), _desc(key_value_ptrs), _desc(slot_mapping)
    _run(
        _L.lmc_multi_layer_kv_transfer(
            _ref(a), _ref(p), _ref(s), dev, int(page_buffer_size), int(bool(direction)),
            int(bool(use_mla)), int(kvcache_format_raw), int(k_hidden_dims),
            int(v_hidden_dims), int(dsa_hidden_dims), _stream(dev),
        )
    )


def multi_layer_kv_transfer_batched(
    key_values: Sequence[torch.Tensor],
    key_value_ptrs: torch.Tensor,
    slot_mapping: torch.Tensor,
    token_starts: Sequence[int],
    paged_memory_device: torch.device,
    page_buffer_size: int,
    direction: bool,
    use_mla: bool,
    kvcache_format_raw: int,
    k_hidden_dims: int = 0,
    v_hidden_dims: int = 0,
    dsa_hidden_dims: int = 0,
) -> None:
    """One launch for a batch of memory objects.

    key_values[i] ([kv, L, T_i, W]) takes tokens
    slot_mapping[token_starts[i] : token_starts[i] + T_i]; the bytes moved
    are those of one multi_layer_kv_transfer call per chunk, the loop the
    reference's connector runs (npu_connectors.py:1278-1284, 1465-1469).
    """
    n = len(key_values)
    if n != len(token_starts):
        raise ValueError("key_values and token_starts differ in length")
    dev = _device_index(paged_memory_device, key_value_ptrs)
    arr = (_lib.LmcTensor * max(n, 1))()
    for i, kv in enumerate(key_values):
        arr[i] = _desc(kv)
    starts = (ctypes.c_int64 * max(n, 1))(*[int(x) for x in token_starts])
    p, s = _desc(key_value_ptrs), _desc(slot_mapping)
    _run(
        _L.lmc_multi_layer_kv_transfer_batched(
            arr, n, starts, _ref(p), _ref(s), dev, int(page_buffer_size),
            int(bool(direction)), int(bool(use_mla)), int(kvcache_format_raw),
            int(k_hidden_dims), int(v_hidden_dims), int(dsa_hidden_dims), _stream(dev),
        )
    )


def fused_multi_layer_kv_transfer(
    key_value: torch.Tensor,
    staging_cache: torch.Tensor,
    key_value_ptrs: torch.Tensor,
    slot_mapping: torch.Tensor,
    paged_memory_device: torch.device,
    page_buffer_size: int,
    direction: bool,
    use_mla: bool,
    kvcache_format_raw: int,
    k_hidden_dims: int = 0,
    v_hidden_dims: int = 0,
    dsa_hidden_dims: int = 0,
) -> None:
    """csrc/mem_kernels.cpp:113-213: gather/scatter through a device staging
    buffer plus one DMA copy to/from the host key_value."""
    dev = _device_index(paged_memory_device, staging_cache)
    a, g = _desc(key_value), _desc(staging_cache)
    p, s = _desc(key_value_ptrs), _desc(slot_mapping)
    _run(
        _L.lmc_fused_multi_layer_kv_transfer(
            _ref(a), _ref(g), _ref(p), _ref(s), dev, int(page_buffer_size),
            int(bool(direction)), int(bool(use_mla)), int(kvcache_format_raw),
            int(k_hidden_dims), int(v_hidden_dims), int(dsa_hidden_dims), _stream(dev),
        )
    )


def multi_layer_kv_transfer_unilateral(*args, **kwargs):
    """csrc/mem_kernels.cpp:255-263: not implemented in the reference either."""
    raise NotImplementedError("multi_layer_kv_transfer_unilateral is not implemented.")


def _normalize_kv_caches(obj):
    # csrc/pybind.cpp:22-31: a Tensor or a tuple of Tensors.
    if isinstance(obj, torch.Tensor):
        return [obj]
    if isinstance(obj, tuple):
        return list(obj)
    raise RuntimeError("vllm_kv_caches must be a Tensor or a tuple of Tensors")


def single_layer_kv_transfer(
    lmc_key_value_cache: torch.Tensor,
    vllm_kv_caches,
    slot_mapping: torch.Tensor,
    direction: bool,
    kvcache_format_raw: int,
    token_major: bool = False,
    vllm_two_major: bool = False,
    k_hidden_dims: int = 0,
    v_hidden_dims: int = 0,
    dsa_hidden_dims: int = 0,
) -> None:
    """csrc/mem_kernels.cpp:265-334 (pybind keywords csrc/pybind.cpp:367-372)."""
    if _ext is not None:
        _ext.single_layer_kv_transfer(
            lmc_key_value_cache, vllm_kv_caches, slot_mapping, bool(direction), int(kvcache_format_raw),
            bool(token_major), bool(vllm_two_major), int(k_hidden_dims), int(v_hidden_dims),
            int(dsa_hidden_dims),
        )
        return
    _single_layer_kv_transfer_ctypes(
        lmc_key_value_cache, vllm_kv_caches, slot_mapping, direction, kvcache_format_raw, token_major,
        vllm_two_major, k_hidden_dims, v_hidden_dims, dsa_hidden_dims,
    )


def _single_layer_kv_transfer_ctypes(
    lmc_key_value_cache, vllm_kv_caches, slot_mapping, direction, kvcache_format_raw, token_major=False,
    vllm_two_major=False, k_hidden_dims=0, v_hidden_dims=0, dsa_hidden_dims=0,
) -> None:
    caches = _normalize_kv_caches(vllm_kv_caches)
    n = len(caches)
    arr = (_lib.LmcTensor * max(n, 1))()
    for i, c in enumerate(caches):
        arr[i] = _desc(c)
    dev = _device_index(*(caches + [slot_mapping, lmc_key_value_cache]))
    a, s = _desc(lmc_key_value_cache), _desc(slot_mapping)
    _run(
        _L.lmc_single_layer_kv_transfer(
            _ref(a), arr, n, _ref(s), int(bool(direction)), int(kvcache_format_raw),
            int(bool(token_major)), int(bool(vllm_two_major)), int(k_hidden_dims),
            int(v_hidden_dims), int(dsa_hidden_dims), _stream(dev),
        )
    )


def load_and_reshape_flash(key_value, key_cache, value_cache, slot_mapping, layer_idx) -> None:
    """csrc/mem_kernels.cpp:1341-1387: key_value[:, layer_idx] <- paged rows."""
    if _ext is not None:
        _ext.load_and_reshape_flash(key_value, key_cache, value_cache, slot_mapping, int(layer_idx))
        return
    dev = _device_index(key_cache)
    a, k, v, s = _desc(key_value), _desc(key_cache), _desc(value_cache), _desc(slot_mapping)
    _run(_L.lmc_load_and_reshape_flash(_ref(a), _ref(k), _ref(v), _ref(s), int(layer_idx), _stream(dev)))


def reshape_and_cache_back_flash(key_value, key_cache, value_cache, slot_mapping, layer_idx) -> None:
    """csrc/mem_kernels.cpp:1389-1440: paged rows <- key_value[:, layer_idx]."""
    if _ext is not None:
        _ext.reshape_and_cache_back_flash(key_value, key_cache, value_cache, slot_mapping, int(layer_idx))
        return
    dev = _device_index(key_cache)
    a, k, v, s = _desc(key_value), _desc(key_cache), _desc(value_cache), _desc(slot_mapping)
    _run(
        _L.lmc_reshape_and_cache_back_flash(_ref(a), _ref(k), _ref(v), _ref(s), int(layer_idx), _stream(dev))
    )


# ---------------------------------------------------------------------------
# CacheGen
# ---------------------------------------------------------------------------


def calculate_cdf(input: torch.Tensor, n_bins: int) -> torch.Tensor:
    """csrc/cachegen_kernels.cpp:119-155: int16 [L, C, n_bins + 1] CDF of the
    [L, T, C] symbols; the output is zero-initialised like the reference's."""
    if not input.is_cuda:
        raise RuntimeError("calculate_cdf: input must be a GPU tensor")
    L, _, C = input.shape
    out = torch.zeros((L, C, int(n_bins) + 1), dtype=torch.int16, device=input.device)
    dev = input.device.index
    a, o = _desc(input), _desc(out)
    _run(_L.lmc_calculate_cdf(_ref(a), int(n_bins), _ref(o), _stream(dev)))
    return out


def encode_fast_new(cdf, input_sym, output_buffer, output_lengths) -> None:
    """csrc/cachegen_kernels.cpp:17-58."""
    dev = _device_index(input_sym)
    c, i, o, n = _desc(cdf), _desc(input_sym), _desc(output_buffer), _desc(output_lengths)
    _run(_L.lmc_encode_fast_new(_ref(c), _ref(i), _ref(o), _ref(n), _stream(dev)))


def decode_fast_new(cdf, bytestreams, lengths, output) -> None:
    """csrc/cachegen_kernels.cpp:60-65: raises NotImplementedError."""
    raise NotImplementedError("Please use decode_fast_prefsum.")


def decode_fast_prefsum(cdf, bytestreams, lengths, output) -> None:
    """csrc/cachegen_kernels.cpp:67-112; lengths are inclusive prefix sums."""
    dev = _device_index(bytestreams)
    c, b, n, o = _desc(cdf), _desc(bytestreams), _desc(lengths), _desc(output)
    _run(_L.lmc_decode_fast_prefsum(_ref(c), _ref(b), _ref(n), _ref(o), _stream(dev)))


# ---------------------------------------------------------------------------
# Fused K re-rotation
# ---------------------------------------------------------------------------


def rotary_embedding_k_fused(oldPositions, newPositions, key, headSize, cosSinCache, isNeox) -> None:
    """csrc/pos_kernels.cpp:158-196: key rotated in place, old -> new."""
    if _ext is not None:
        _ext.rotary_embedding_k_fused(oldPositions, newPositions, key, int(headSize), cosSinCache, bool(isNeox))
        return
    dev = _device_index(key)
    a, b, k, c = _desc(oldPositions), _desc(newPositions), _desc(key), _desc(cosSinCache)
    _run(
        _L.lmc_rotary_embedding_k_fused(
            _ref(a), _ref(b), _ref(k), int(headSize), _ref(c), int(bool(isNeox)), _stream(dev)
        )
    )


# ---------------------------------------------------------------------------
# Pinned host memory
# ---------------------------------------------------------------------------


def get_device_ptr(ptr_addr: int, required_size: int = 1) -> int:
    """csrc/common/managed_mem.cpp:189-236; 0 when unmapped."""
    out = ctypes.c_size_t(0)
    _run(_L.lmc_get_device_ptr(int(ptr_addr), int(required_size), ctypes.byref(out)))
    return int(out.value)


def register_mapping(host_ptr: int, dev_ptr: int, size: int) -> int:
    out = ctypes.c_size_t(0)
    _run(_L.lmc_register_mapping(int(host_ptr), int(dev_ptr), int(size), ctypes.byref(out)))
    return int(out.value)


def unregister_ptr(ptr_addr: int) -> int:
    out = ctypes.c_int32(0)
    _run(_L.lmc_unregister_ptr(int(ptr_addr), ctypes.byref(out)))
    return int(out.value)


def alloc_pinned_ptr(size: int, flags: int = 0) -> int:
    """csrc/common/mem_alloc.cpp:19-44."""
    out = ctypes.c_size_t(0)
    _run(_L.lmc_alloc_pinned_ptr(int(size), int(flags), ctypes.byref(out)))
    return int(out.value)


def free_pinned_ptr(ptr: int) -> None:
    _run(_L.lmc_free_pinned_ptr(int(ptr)))


def get_gpu_pci_bus_id(device: int) -> str:
    buf = ctypes.create_string_buffer(64)
    _run(_L.lmc_get_gpu_pci_bus_id(int(device), buf, len(buf)))
    return buf.value.decode()
