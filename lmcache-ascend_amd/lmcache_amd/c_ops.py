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
from typing import Optional, Sequence

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
        _addr("lmc_blend_layer_to_paged"),
        _addr("lmc_calculate_cdf"),
        _addr("lmc_encode_fast_new"),
        _addr("lmc_decode_fast_prefsum"),
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
        raise RuntimeError(f"no lmc_tensor dtype code for {t.dtype}") from None
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


# Bytes of the library's per-GPU staging area used by
# fused_multi_layer_kv_transfer_noalloc.
NOALLOC_STAGING_BYTES = 64 << 20


def fused_multi_layer_kv_transfer_noalloc(
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
    """fused_multi_layer_kv_transfer without a staging_cache argument, for
    callers that cannot allocate device memory: the library stages through
    its own NOALLOC_STAGING_BYTES area on the cache device and allocates
    nothing.  A store zeroes the staging bytes first, so rows of skipped
    slots arrive as zeros.  Every call on one GPU shares that area: eager
    calls are ordered across streams and threads (each waits for the
    previous call's work), calls captured into a HIP graph are not, so a
    replay overlapping another call on the same GPU races with it."""
    dev = _device_index(paged_memory_device, key_value_ptrs)
    a, p, s = _desc(key_value), _desc(key_value_ptrs), _desc(slot_mapping)
    _run(
        _L.lmc_fused_multi_layer_kv_transfer_noalloc(
            _ref(a), _ref(p), _ref(s), dev, int(page_buffer_size),
            int(bool(direction)), int(bool(use_mla)), int(kvcache_format_raw),
            int(k_hidden_dims), int(v_hidden_dims), int(dsa_hidden_dims), _stream(dev),
        )
    )


def multi_layer_kv_transfer_unilateral(*args, **kwargs):
    """csrc/mem_kernels.cpp:255-263: not implemented in the reference either."""
    raise NotImplementedError("multi_layer_kv_transfer_unilateral is not implemented.")


def multi_layer_kv_transfer_310p(*args, **kwargs):
    """csrc/mem_kernels.cpp:215-253: the Ascend 310P's fractal (NZ) paged
    layout, whose kernel lives outside the reference tree.  No MI355X
    attention backend stores KV in that layout; callers reach this only when
    the device reports itself as a 310P."""
    raise NotImplementedError("multi_layer_kv_transfer_310p: the 310P NZ KV layout has no MI355X counterpart.")


def _normalize_kv_caches(obj):
    # csrc/pybind.cpp:22-31: a Tensor or a tuple of Tensors.
    if isinstance(obj, torch.Tensor):
        return [obj]
    if isinstance(obj, tuple):
        return list(obj)
    raise RuntimeError("vllm_kv_caches is neither a Tensor nor a tuple of Tensors")


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
    """csrc/mem_kernels.cpp:1341-1389: key_value[:, layer_idx] <- paged rows."""
    if _ext is not None:
        _ext.load_and_reshape_flash(key_value, key_cache, value_cache, slot_mapping, int(layer_idx))
        return
    dev = _device_index(key_cache)
    a, k, v, s = _desc(key_value), _desc(key_cache), _desc(value_cache), _desc(slot_mapping)
    _run(_L.lmc_load_and_reshape_flash(_ref(a), _ref(k), _ref(v), _ref(s), int(layer_idx), _stream(dev)))


def reshape_and_cache_back_flash(key_value, key_cache, value_cache, slot_mapping, layer_idx) -> None:
    """csrc/mem_kernels.cpp:1391-1440: paged rows <- key_value[:, layer_idx]."""
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
    [L, T, C] symbols, one row per (layer, channel) stream: aligned
    power-of-two intervals in symbol order, the code length in the low 4
    bits, the lengths those of an optimal alphabetic code (Garsia-Wachs)
    within 8 bits for at most 256 counted symbols (12 above), else Shannon
    lengths.  The reference zero-fills the output first; the kernel writes
    every entry of it, so it is allocated without a fill."""
    if _ext is not None:
        return _ext.calculate_cdf(input, int(n_bins))
    if not input.is_cuda:
        raise RuntimeError("calculate_cdf: input must be a GPU tensor")
    L, _, C = input.shape
    out = torch.empty((L, C, int(n_bins) + 1), dtype=torch.int16, device=input.device)
    dev = input.device.index
    a, o = _desc(input), _desc(out)
    _run(_L.lmc_calculate_cdf(_ref(a), int(n_bins), _ref(o), _stream(dev)))
    return out


def encode_fast_new(cdf, input_sym, output_buffer, output_lengths) -> None:
    """csrc/cachegen_kernels.cpp:17-58."""
    if _ext is not None:
        _ext.encode_fast_new(cdf, input_sym, output_buffer, output_lengths)
        return
    dev = _device_index(input_sym)
    c, i, o, n = _desc(cdf), _desc(input_sym), _desc(output_buffer), _desc(output_lengths)
    _run(_L.lmc_encode_fast_new(_ref(c), _ref(i), _ref(o), _ref(n), _stream(dev)))


def decode_fast_new(cdf, bytestreams, lengths, output) -> None:
    """csrc/cachegen_kernels.cpp:60-65: raises NotImplementedError."""
    raise NotImplementedError("Please use decode_fast_prefsum.")


def decode_fast_prefsum(cdf, bytestreams, lengths, output) -> None:
    """csrc/cachegen_kernels.cpp:67-112; lengths are inclusive prefix sums."""
    if _ext is not None:
        _ext.decode_fast_prefsum(cdf, bytestreams, lengths, output)
        return
    dev = _device_index(bytestreams)
    c, b, n, o = _desc(cdf), _desc(bytestreams), _desc(lengths), _desc(output)
    _run(_L.lmc_decode_fast_prefsum(_ref(c), _ref(b), _ref(n), _ref(o), _stream(dev)))


# ---------------------------------------------------------------------------
# Fused K re-rotation
# ---------------------------------------------------------------------------


def blend_layer_to_paged(
    memory_objs: Sequence[torch.Tensor],
    token_starts: Sequence[int],
    vllm_kv_caches,
    slot_mapping: torch.Tensor,
    old_positions: Optional[torch.Tensor] = None,
    new_positions: Optional[torch.Tensor] = None,
    cos_sin_cache: Optional[torch.Tensor] = None,
    head_size: int = 0,
    is_neox: bool = True,
    kvcache_format_raw: int = 2,
    vllm_two_major: bool = False,
) -> None:
    """One layer of the CacheBlend connector's retrieve
    (lmcache_ascend/v1/npu_connector/npu_connectors.py:556-689) in one
    kernel, with no device buffer.  The paged caches end as after

        buf = zeros([2, N, W]); buf[:, s:s + n_i] = memory_objs[i]
        rotary_embedding_k_fused(old_positions, new_positions, buf[0], ...)
        single_layer_kv_transfer(buf, vllm_kv_caches, slot_mapping, False,
                                 kvcache_format_raw, False, vllm_two_major)

    with N = slot_mapping.numel(), the objects KV_2TD [2, n_i, W] (device or
    pinned host tensors, not overlapping), and no re-rotation when the
    positions are None.  Shapes the kernel does not take (keys other than
    bf16/fp16, rows or heads not in 16-byte pieces, rotary halves not a
    multiple of 8 dims) run that same sequence with this library's ops."""
    caches = _normalize_kv_caches(vllm_kv_caches)
    objs = list(memory_objs)
    if len(objs) != len(token_starts):
        raise ValueError("memory_objs and token_starts differ in length")
    rope = old_positions is not None or new_positions is not None
    if rope and (old_positions is None or new_positions is None or cos_sin_cache is None):
        raise ValueError("old_positions, new_positions and cos_sin_cache go together")
    if _ext is not None:
        done = _ext.blend_layer_to_paged(
            objs, [int(x) for x in token_starts], vllm_kv_caches, slot_mapping, old_positions, new_positions,
            cos_sin_cache, int(head_size), bool(is_neox), int(kvcache_format_raw), bool(vllm_two_major))
        if not done:
            _blend_connector_sequence(objs, token_starts, vllm_kv_caches, slot_mapping, old_positions,
                                      new_positions, cos_sin_cache, head_size, is_neox, kvcache_format_raw,
                                      vllm_two_major)
        return
    dev = _device_index(*(caches + [slot_mapping]))
    carr = (_lib.LmcTensor * max(len(caches), 1))()
    for i, c in enumerate(caches):
        carr[i] = _desc(c)
    oarr = (_lib.LmcTensor * max(len(objs), 1))()
    for i, o in enumerate(objs):
        oarr[i] = _desc(o)
    starts = (ctypes.c_int64 * max(len(objs), 1))(*[int(x) for x in token_starts])
    s = _desc(slot_mapping)
    a = _desc(old_positions) if rope else None
    b = _desc(new_positions) if rope else None
    c = _desc(cos_sin_cache) if rope else None
    status = _L.lmc_blend_layer_to_paged(
        oarr, len(objs), starts, carr, len(caches), _ref(s),
        _ref(a) if rope else None, _ref(b) if rope else None, _ref(c) if rope else None,
        int(head_size), int(bool(is_neox)), int(kvcache_format_raw), int(bool(vllm_two_major)), _stream(dev),
    )
    if status != _lib.ERR_NOT_IMPLEMENTED:
        _run(status)
        return
    _blend_connector_sequence(objs, token_starts, vllm_kv_caches, slot_mapping, old_positions, new_positions,
                              cos_sin_cache, head_size, is_neox, kvcache_format_raw, vllm_two_major)


def _blend_connector_sequence(objs, token_starts, vllm_kv_caches, slot_mapping, old_positions, new_positions,
                              cos_sin_cache, head_size, is_neox, kvcache_format_raw, vllm_two_major) -> None:
    """The connector's own sequence (npu_connectors.py:597-680), on device,
    for shapes the fused kernel does not take.  The layer buffer lives on
    the caches' device; a slot mapping in pinned host memory, which the
    fused entry point accepts, is copied there first."""
    caches = _normalize_kv_caches(vllm_kv_caches)
    rope = old_positions is not None
    k0 = caches[0]
    dev = k0.device
    slot_mapping = slot_mapping.to(dev)
    width = k0.shape[-2] * k0.shape[-1]
    n_tok = int(slot_mapping.numel())
    buf = torch.zeros((2, n_tok, width), dtype=k0.dtype, device=dev)
    for o, st in zip(objs, token_starts):
        buf[:, int(st):int(st) + o.shape[1]].copy_(o, non_blocking=True)
    if rope:
        rotary_embedding_k_fused(old_positions, new_positions, buf[0], head_size, cos_sin_cache, is_neox)
        # Rows no object covers are zeroed after the re-rotation, as the
        # connector does (npu_connectors.py:647-649).
        cursor = 0
        for o, st in sorted(zip(objs, token_starts), key=lambda x: int(x[1])):
            if int(st) > cursor:
                buf[:, cursor:int(st)] = 0
            cursor = max(cursor, int(st) + o.shape[1])
        if cursor < n_tok:
            buf[:, cursor:] = 0
    single_layer_kv_transfer(buf, vllm_kv_caches, slot_mapping, False, kvcache_format_raw, False, vllm_two_major)


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
# Sparse, direct and staged-batch single-layer transfers
# (csrc/mem_kernels.cpp:336-1339; csrc/pybind.cpp:45-340, 373-472)
# ---------------------------------------------------------------------------

_MLA_DSA = (3, 4, 5, 6)


def _cache_array(caches):
    arr = (_lib.LmcTensor * max(len(caches), 1))()
    for i, c in enumerate(caches):
        arr[i] = _desc(c)
    return arr


def _tensor_array(tensors):
    return _cache_array(list(tensors))


def _i64_array(values):
    vals = [int(v) for v in values]
    return (ctypes.c_int64 * max(len(vals), 1))(*vals)


def _geom_desc(shape, strides, dtype) -> _lib.LmcTensor:
    """Geometry-only descriptor (no data) of an LMC layout sample."""
    return _lib.LmcTensor(0, _DTYPES[dtype], -1, len(shape), 0, _DIMS(*shape), _DIMS(*strides))


def _check_caches(caches, fmt, two_major=False, kH=0, vH=0, dsaH=0) -> None:
    arr = _cache_array(caches)
    _run(_L.lmc_check_kv_caches(arr, len(caches), int(fmt), int(bool(two_major)), int(kH), int(vH), int(dsaH)))


def _chunk_ptrs_for(lmc_tensors, device) -> torch.Tensor:
    """Device int64 table of the memory objects' kernel-visible addresses
    (csrc/mem_kernels.cpp:618-633)."""
    ptrs = []
    for t in lmc_tensors:
        if t.is_cuda:
            ptrs.append(t.data_ptr())
            continue
        p = get_device_ptr(t.data_ptr(), max(1, t.numel() * t.element_size()))
        if p == 0:
            raise RuntimeError("host tensor is not in pinned, device-mapped memory: no device address for it")
        ptrs.append(p)
    return torch.tensor(ptrs, dtype=torch.int64, device=device)


def _mla_plane_elems(caches, fmt, kH, vH, dsaH) -> int:
    """Elements of one token over all MLA/DSA planes, with the reference's
    hidden-dim defaults (csrc/utils.cpp:310-339)."""
    fmt = int(fmt)
    k = caches[0]
    if fmt == 6:
        return int(dsaH) if dsaH > 0 else k.shape[-2] * k.shape[-1]
    kH = int(kH) if kH > 0 else k.shape[-2] * k.shape[-1]
    vH = int(vH) if vH > 0 else caches[1].shape[-2] * caches[1].shape[-1]
    if fmt == 4:
        return kH + vH + (int(dsaH) if dsaH > 0 else caches[2].shape[-2] * caches[2].shape[-1])
    return kH + vH


def _check_chunk_capacity(lmc_tensors, caches, fmt, kH, vH, dsaH, chunk_size, total_tokens) -> None:
    """Memory object c must hold its min(chunk_size, total - c * chunk_size)
    tokens (the kernels address them from the object's base)."""
    if int(fmt) in _MLA_DSA:
        per_token = _mla_plane_elems(caches, fmt, kH, vH, dsaH)
        need = [min(chunk_size, total_tokens - c * chunk_size) * per_token for c in range(len(lmc_tensors))]
    else:
        need = [lmc_tensors[0].numel()] * len(lmc_tensors)
    for c, (t, n) in enumerate(zip(lmc_tensors, need)):
        if t.numel() < n:
            raise RuntimeError(f"memory object {c} holds {t.numel()} elements, its chunk needs {n}")


def _require_cpu_chunks(lmc_tensors, what: str) -> None:
    if len(lmc_tensors) == 0:
        raise RuntimeError("lmc_tensors lists no memory object")
    for t in lmc_tensors:
        if t.device.type != "cpu":
            raise RuntimeError(what)


def sparse_single_layer_kv_transfer(
    lmc_key_value_cache, vllm_kv_caches, slot_mapping_packed, selected_token_idx, kvcache_format_raw,
    token_major=False, vllm_two_major=False, k_hidden_dims=0, v_hidden_dims=0, dsa_hidden_dims=0,
) -> None:
    """Retrieve only: paged[slot_mapping_packed[i]] = LMC[selected_token_idx[i]]
    (csrc/mem_kernels.cpp:418-497; tests/v1/test_mem_kernels.py:1445-1543)."""
    caches = _normalize_kv_caches(vllm_kv_caches)
    arr = _cache_array(caches)
    dev = _device_index(*(caches + [slot_mapping_packed]))
    a, s, x = _desc(lmc_key_value_cache), _desc(slot_mapping_packed), _desc(selected_token_idx)
    _run(
        _L.lmc_sparse_single_layer_kv_transfer(
            _ref(a), arr, len(caches), _ref(s), _ref(x), int(kvcache_format_raw), int(bool(token_major)),
            int(bool(vllm_two_major)), int(k_hidden_dims), int(v_hidden_dims), int(dsa_hidden_dims), _stream(dev),
        )
    )


def batched_fused_single_layer_kv_transfer(
    lmc_tensors, staging_cache, vllm_kv_caches, slot_mapping_full, chunk_offsets, chunk_sizes, direction,
    kvcache_format_raw, token_major=False, vllm_two_major=False, k_hidden_dims=0, v_hidden_dims=0,
    dsa_hidden_dims=0,
) -> None:
    """Single-layer copy through `staging_cache` plus one DMA copy per chunk
    and plane (csrc/mem_kernels.cpp:336-416; tests/v1/test_mem_kernels.py:
    791-1062).  direction True: paged -> staging -> lmc_tensors."""
    caches = _normalize_kv_caches(vllm_kv_caches)
    arr = _cache_array(caches)
    objs = _tensor_array(lmc_tensors)
    if len(chunk_offsets) != len(lmc_tensors) or len(chunk_sizes) != len(lmc_tensors):
        raise RuntimeError("chunk_offsets and chunk_sizes need one entry per memory object")
    dev = _device_index(*(caches + [slot_mapping_full, staging_cache]))
    st, s = _desc(staging_cache), _desc(slot_mapping_full)
    _run(
        _L.lmc_batched_fused_single_layer_kv_transfer(
            objs, len(lmc_tensors), _ref(st), arr, len(caches), _ref(s), _i64_array(chunk_offsets),
            _i64_array(chunk_sizes), int(bool(direction)), int(kvcache_format_raw), int(bool(token_major)),
            int(bool(vllm_two_major)), int(k_hidden_dims), int(v_hidden_dims), int(dsa_hidden_dims), _stream(dev),
        )
    )


def batched_fused_sparse_single_layer_kv_transfer(
    lmc_tensors, staging_cache, vllm_kv_caches, slot_mapping_packed, selected_token_idx, chunk_offsets,
    chunk_sizes, kvcache_format_raw, token_major=False, vllm_two_major=False, k_hidden_dims=0,
    v_hidden_dims=0, dsa_hidden_dims=0, sparse_indices_cpu=None,
) -> None:
    """lmc_tensors -> staging, then sparse_single_layer_kv_transfer from the
    staging buffer (csrc/mem_kernels.cpp:1308-1339).  `sparse_indices_cpu`
    only steers the reference's choice of per-token copies; every chunk is
    staged whole here."""
    caches = _normalize_kv_caches(vllm_kv_caches)
    arr = _cache_array(caches)
    objs = _tensor_array(lmc_tensors)
    if len(chunk_offsets) != len(lmc_tensors) or len(chunk_sizes) != len(lmc_tensors):
        raise RuntimeError("chunk_offsets and chunk_sizes need one entry per memory object")
    dev = _device_index(*(caches + [slot_mapping_packed, staging_cache]))
    st, s, x = _desc(staging_cache), _desc(slot_mapping_packed), _desc(selected_token_idx)
    _run(
        _L.lmc_batched_fused_sparse_single_layer_kv_transfer(
            objs, len(lmc_tensors), _ref(st), arr, len(caches), _ref(s), _ref(x), _i64_array(chunk_offsets),
            _i64_array(chunk_sizes), int(kvcache_format_raw), int(bool(token_major)), int(bool(vllm_two_major)),
            int(k_hidden_dims), int(v_hidden_dims), int(dsa_hidden_dims), _stream(dev),
        )
    )


class SparseDirectLayerState:
    """prepare_sparse_direct_layer_state's result (csrc/utils.cpp:408-423):
    one layer's caches and LMC layout, checked once."""

    __slots__ = ("caches", "kvcache_format", "token_major", "vllm_two_major", "k_hidden_dims",
                 "v_hidden_dims", "dsa_hidden_dims", "layout", "lmc_num_tokens")


class SparseDirectDestinationState:
    """prepare_sparse_direct_destination_state's result (csrc/utils.cpp:
    425-498): one layer's MLA/DSA caches, checked once."""

    __slots__ = ("caches", "kvcache_format", "k_hidden_dims", "v_hidden_dims", "dsa_hidden_dims")


def prepare_sparse_direct_layer_state(
    lmc_layout_sample, vllm_kv_caches, slot_mapping_ref, token_major, vllm_two_major, kvcache_format_raw,
    k_hidden_dims, v_hidden_dims, dsa_hidden_dims, lmc_num_tokens,
) -> SparseDirectLayerState:
    caches = _normalize_kv_caches(vllm_kv_caches)
    _check_caches(caches, kvcache_format_raw, vllm_two_major, k_hidden_dims, v_hidden_dims, dsa_hidden_dims)
    st = SparseDirectLayerState()
    st.caches = tuple(caches)
    st.kvcache_format = int(kvcache_format_raw)
    st.token_major = bool(token_major)
    st.vllm_two_major = bool(vllm_two_major)
    st.k_hidden_dims, st.v_hidden_dims, st.dsa_hidden_dims = int(k_hidden_dims), int(v_hidden_dims), int(dsa_hidden_dims)
    st.layout = (tuple(lmc_layout_sample.shape), tuple(lmc_layout_sample.stride()), lmc_layout_sample.dtype)
    st.lmc_num_tokens = int(lmc_num_tokens)
    return st


def prepare_sparse_direct_destination_state(
    vllm_kv_caches, slot_mapping_ref, kvcache_format_raw, k_hidden_dims, v_hidden_dims, dsa_hidden_dims,
) -> SparseDirectDestinationState:
    caches = _normalize_kv_caches(vllm_kv_caches)
    _check_caches(caches, kvcache_format_raw, False, k_hidden_dims, v_hidden_dims, dsa_hidden_dims)
    if int(kvcache_format_raw) not in _MLA_DSA:
        raise RuntimeError("prepared sparse destination states serve MLA/DSA formats (3-6) only")
    st = SparseDirectDestinationState()
    st.caches = tuple(caches)
    st.kvcache_format = int(kvcache_format_raw)
    st.k_hidden_dims, st.v_hidden_dims, st.dsa_hidden_dims = int(k_hidden_dims), int(v_hidden_dims), int(dsa_hidden_dims)
    return st


def _sparse_direct(caches, fmt, token_major, two_major, kH, vH, dsaH, layout, slot_mapping_packed,
                   selected_token_idx, chunk_ptrs, counts, chunk_size, total_tokens, interleaved, validate):
    arr = _cache_array(caches)
    dev = _device_index(*(list(caches) + [slot_mapping_packed]))
    p, s, x = _desc(chunk_ptrs), _desc(slot_mapping_packed), _desc(selected_token_idx)
    lay = _geom_desc(*layout) if layout is not None else None
    cnt = _desc(counts) if counts is not None else None
    _run(
        _L.lmc_sparse_direct_kv_transfer(
            _ref(p), _ref(lay) if lay is not None else None, arr, len(caches), _ref(s), _ref(x),
            _ref(cnt) if cnt is not None else None, int(chunk_size), int(total_tokens), int(fmt),
            int(bool(token_major)), int(bool(two_major)), int(kH), int(vH), int(dsaH), int(bool(interleaved)),
            int(bool(validate)), _stream(dev),
        )
    )


def sparse_mla_dsa_batched_direct_kv_transfer(
    lmc_tensors, vllm_kv_caches, slot_mapping_packed, selected_token_idx, chunk_size, total_tokens,
    kvcache_format_raw, token_major=False, vllm_two_major=False, k_hidden_dims=0, v_hidden_dims=0,
    dsa_hidden_dims=0, lmc_host_interleaved=False, chunk_ptrs_npu=None, selected_token_counts=None,
) -> None:
    """Retrieve selected tokens straight from pinned memory objects
    (csrc/mem_kernels.cpp:588-682; tools/cpu_vllm_runtime.py:288-343)."""
    caches = _normalize_kv_caches(vllm_kv_caches)
    _check_caches(caches, kvcache_format_raw, vllm_two_major, k_hidden_dims, v_hidden_dims, dsa_hidden_dims)
    if int(chunk_size) <= 0:
        raise RuntimeError("chunk_size is not positive")
    if int(total_tokens) <= 0:
        raise RuntimeError("total_tokens is not positive")
    _require_cpu_chunks(lmc_tensors, "direct sparse retrieval reads memory objects in pinned host memory only")
    _check_chunk_capacity(lmc_tensors, caches, kvcache_format_raw, k_hidden_dims, v_hidden_dims, dsa_hidden_dims,
                          int(chunk_size), int(total_tokens))
    if selected_token_idx.numel() == 0:
        return
    if chunk_ptrs_npu is None or chunk_ptrs_npu.numel() != len(lmc_tensors):
        chunk_ptrs_npu = _chunk_ptrs_for(lmc_tensors, slot_mapping_packed.device)
    s0 = lmc_tensors[0]
    _sparse_direct(caches, kvcache_format_raw, token_major, vllm_two_major, k_hidden_dims, v_hidden_dims,
                   dsa_hidden_dims, (tuple(s0.shape), tuple(s0.stride()), s0.dtype), slot_mapping_packed,
                   selected_token_idx, chunk_ptrs_npu, selected_token_counts, chunk_size, total_tokens,
                   lmc_host_interleaved, True)


def sparse_mla_dsa_batched_direct_kv_transfer_fast(
    layer_state, slot_mapping_packed, selected_token_idx, chunk_ptrs_npu, chunk_size, total_tokens,
    lmc_host_interleaved, validate_inputs=False, selected_token_counts=None,
) -> None:
    """csrc/mem_kernels.cpp:684-752."""
    st = layer_state
    if selected_token_idx.numel() == 0 and not validate_inputs:
        return
    _sparse_direct(st.caches, st.kvcache_format, st.token_major, st.vllm_two_major, st.k_hidden_dims,
                   st.v_hidden_dims, st.dsa_hidden_dims, st.layout, slot_mapping_packed, selected_token_idx,
                   chunk_ptrs_npu, selected_token_counts, chunk_size, total_tokens, lmc_host_interleaved,
                   validate_inputs)


def sparse_mla_dsa_batched_direct_kv_transfer_prepared(
    destination_state, slot_mapping_packed, selected_token_idx, chunk_ptrs_npu, chunk_size, total_tokens,
    lmc_host_interleaved, selected_token_counts=None, diagnostic_layer_id=-1,
) -> None:
    """csrc/mem_kernels.cpp:833-976 (the diagnostic timing is not kept)."""
    st = destination_state
    if selected_token_idx.numel() == 0:
        return
    _sparse_direct(st.caches, st.kvcache_format, False, False, st.k_hidden_dims, st.v_hidden_dims,
                   st.dsa_hidden_dims, None, slot_mapping_packed, selected_token_idx, chunk_ptrs_npu,
                   selected_token_counts, chunk_size, total_tokens, lmc_host_interleaved, False)


def _dense_direct(caches, fmt, kH, vH, dsaH, slot_mapping_full, chunk_ptrs, chunk_offsets, chunk_sizes,
                  total_tokens, fixed_chunk_size, interleaved, direction, validate, two_major=False):
    arr = _cache_array(caches)
    dev = _device_index(*(list(caches) + [slot_mapping_full]))
    p, s = _desc(chunk_ptrs), _desc(slot_mapping_full)
    o, z = _desc(chunk_offsets), _desc(chunk_sizes)
    _run(
        _L.lmc_dense_direct_kv_transfer(
            _ref(p), arr, len(caches), _ref(s), _ref(o), _ref(z), int(total_tokens), int(fixed_chunk_size),
            int(fmt), int(bool(two_major)), int(kH), int(vH), int(dsaH), int(bool(interleaved)),
            int(bool(direction)), int(bool(validate)), _stream(dev),
        )
    )


def dense_mla_dsa_batched_direct_kv_transfer(
    lmc_tensors, vllm_kv_caches, slot_mapping_full, chunk_offsets_npu, chunk_sizes_npu, total_tokens,
    kvcache_format_raw, token_major=False, vllm_two_major=False, k_hidden_dims=0, v_hidden_dims=0,
    dsa_hidden_dims=0, lmc_host_interleaved=False, direction=False, chunk_ptrs_npu=None, fixed_chunk_size=0,
) -> None:
    """Every token of each memory object, either direction
    (csrc/mem_kernels.cpp:1036-1114; tools/cpu_vllm_runtime.py:353-411)."""
    caches = _normalize_kv_caches(vllm_kv_caches)
    _check_caches(caches, kvcache_format_raw, vllm_two_major, k_hidden_dims, v_hidden_dims, dsa_hidden_dims)
    if int(kvcache_format_raw) not in _MLA_DSA:
        raise RuntimeError("dense direct transfers move MLA/DSA formats (3-6) only")
    _require_cpu_chunks(lmc_tensors, "dense direct transfers take memory objects in pinned host memory only")
    if int(fixed_chunk_size) > 0:
        _check_chunk_capacity(lmc_tensors, caches, kvcache_format_raw, k_hidden_dims, v_hidden_dims,
                              dsa_hidden_dims, int(fixed_chunk_size), int(total_tokens))
    if chunk_ptrs_npu is None or chunk_ptrs_npu.numel() != len(lmc_tensors):
        chunk_ptrs_npu = _chunk_ptrs_for(lmc_tensors, slot_mapping_full.device)
    _dense_direct(caches, kvcache_format_raw, k_hidden_dims, v_hidden_dims, dsa_hidden_dims, slot_mapping_full,
                  chunk_ptrs_npu, chunk_offsets_npu, chunk_sizes_npu, total_tokens, fixed_chunk_size,
                  lmc_host_interleaved, direction, True, vllm_two_major)


def dense_mla_dsa_batched_direct_kv_transfer_fast(
    layer_state, slot_mapping_full, chunk_ptrs_npu, chunk_offsets_npu, chunk_sizes_npu, total_tokens,
    lmc_host_interleaved, direction, validate_inputs=False, fixed_chunk_size=0,
) -> None:
    """csrc/mem_kernels.cpp:1116-1166."""
    st = layer_state
    _dense_direct(st.caches, st.kvcache_format, st.k_hidden_dims, st.v_hidden_dims, st.dsa_hidden_dims,
                  slot_mapping_full, chunk_ptrs_npu, chunk_offsets_npu, chunk_sizes_npu, total_tokens,
                  fixed_chunk_size, lmc_host_interleaved, direction, validate_inputs, st.vllm_two_major)


def dense_mla_dsa_batched_direct_kv_transfer_prepared(
    destination_state, slot_mapping_full, chunk_ptrs_npu, chunk_offsets_npu, chunk_sizes_npu, total_tokens,
    lmc_host_interleaved, validate_inputs=False, fixed_chunk_size=0,
) -> None:
    """Retrieve (memory objects -> paged), csrc/mem_kernels.cpp:1168-1219."""
    st = destination_state
    _dense_direct(st.caches, st.kvcache_format, st.k_hidden_dims, st.v_hidden_dims, st.dsa_hidden_dims,
                  slot_mapping_full, chunk_ptrs_npu, chunk_offsets_npu, chunk_sizes_npu, total_tokens,
                  fixed_chunk_size, lmc_host_interleaved, False, validate_inputs)


def _dense_group(layer_states, slot_mapping_full, layer_chunk_ptrs_npu, chunk_offsets_npu, chunk_sizes_npu,
                 total_tokens, lmc_host_interleaved, direction, validate_inputs, fixed_chunk_size):
    """One dense direct transfer per layer, layer l using row l of the
    [layers, chunks] pointer table (csrc/mem_kernels.cpp:1221-1306)."""
    if len(layer_states) == 0:
        raise RuntimeError("layer_states lists no layer")
    if layer_chunk_ptrs_npu.dim() != 2:
        raise RuntimeError("layer_chunk_ptrs_npu is not a [layers, chunks] table")
    if layer_chunk_ptrs_npu.size(0) != len(layer_states):
        raise RuntimeError("layer_chunk_ptrs_npu rows and layer_states differ in count")
    if layer_chunk_ptrs_npu.size(1) <= 0:
        raise RuntimeError("layer_chunk_ptrs_npu has no chunk column")
    if not layer_chunk_ptrs_npu.is_contiguous():
        raise RuntimeError("layer_chunk_ptrs_npu is not contiguous")
    for layer_id, st in enumerate(layer_states):
        _dense_direct(st.caches, st.kvcache_format, st.k_hidden_dims, st.v_hidden_dims, st.dsa_hidden_dims,
                      slot_mapping_full, layer_chunk_ptrs_npu[layer_id], chunk_offsets_npu, chunk_sizes_npu,
                      total_tokens, fixed_chunk_size, lmc_host_interleaved, direction,
                      validate_inputs and layer_id == 0, st.vllm_two_major)


def dense_mla_dsa_group_direct_kv_transfer_fast(
    layer_states, layer_tensors, slot_mapping_full, chunk_offsets_npu, chunk_sizes_npu, total_tokens,
    lmc_host_interleaved, direction, validate_inputs=False, fixed_chunk_size=0,
):
    """Dense direct transfer of several layers into registered host memory
    objects; returns (host_pointer_rows, layer_chunk_ptrs_npu)
    (csrc/pybind.cpp:187-240)."""
    layer_states = list(layer_states)
    if len(layer_states) == 0:
        raise RuntimeError("layer_states lists no layer")
    if len(layer_tensors) != len(layer_states):
        raise RuntimeError("layer tensor rows and layer_states differ in count")
    rows, flat, num_chunks = [], [], None
    for layer_id, tensors in enumerate(layer_tensors):
        if num_chunks is None:
            num_chunks = len(tensors)
            if num_chunks <= 0:
                raise RuntimeError("a group store layer lists no chunk")
        if len(tensors) != num_chunks:
            raise RuntimeError("group store layers differ in chunk count")
        row = []
        for chunk_id, t in enumerate(tensors):
            if t.device.type != "cpu":
                raise RuntimeError("group direct stores write host tensors only")
            p = get_device_ptr(t.data_ptr())
            if p == 0:
                raise RuntimeError(
                    "group direct store target has no device mapping: "
                    f"layer={layer_id}, chunk={chunk_id}"
                )
            row.append(p)
            flat.append(p)
        rows.append(row)
    table = torch.tensor(flat, dtype=torch.int64, device=slot_mapping_full.device).reshape(
        len(layer_states), num_chunks
    )
    _dense_group(layer_states, slot_mapping_full, table, chunk_offsets_npu, chunk_sizes_npu, total_tokens,
                 lmc_host_interleaved, direction, validate_inputs, fixed_chunk_size)
    return rows, table


def dense_mla_dsa_group_direct_kv_transfer_prepared(
    objects, slots, pointers, offsets, sizes, tokens, interleaved, validate, fixed_chunk_size,
) -> None:
    """Store (paged -> memory objects) of several layers through a prepared
    [layers, chunks] pointer table (csrc/pybind.cpp:312-327)."""
    _dense_group(list(objects), slots, pointers, offsets, sizes, tokens, interleaved, True, validate,
                 fixed_chunk_size)


def sparse_graph_kv_transfer(destination_state, slots, selected, counts, ptrs, limits, chunk_size,
                             max_aiv_cores=0) -> None:
    """Graph-replay sparse copy into a prepared MLA destination
    (csrc/mem_kernels.cpp:754-831; csrc/graph/sparse_graph_kernel.cpp):
    rows of `selected` / `slots` per request, `counts` and `limits` per row,
    `ptrs` the [2, requests * chunks] K and PE chunk-source tables."""
    st = destination_state
    k, pe = st.caches[0], st.caches[1]
    a, b = _desc(k), _desc(pe)
    d = [_desc(x) for x in (slots, selected, counts, ptrs, limits)]
    dev = _device_index(selected, k)
    _run(
        _L.lmc_sparse_graph_kv_transfer(
            _ref(a), _ref(b), int(st.k_hidden_dims), int(st.v_hidden_dims), *[_ref(x) for x in d],
            int(chunk_size), int(max_aiv_cores), _stream(dev),
        )
    )


# ---------------------------------------------------------------------------
# Indexer key / C8 packet transport (csrc/indexer_c8.cpp; pybind.cpp:243-262)
# ---------------------------------------------------------------------------

INDEXER_C8_BLOCK_MAP_ABI = 1


class IndexerC8State:
    """One layer's indexer cache: float16/bfloat16 keys [NB, 128, 1, 128],
    or int8 keys with float16 scales [NB, 128, 1, 1]; physical slot factor
    1 (or 2 for int8) or an int32 block permutation (csrc/indexer_c8.cpp:
    13-50).  The layer's descriptors are built once, here."""

    def __init__(self, keys, scales=None, slot_factor=1, block_map=None):
        kd = _desc(keys)
        sd = _desc(scales) if scales is not None else None
        md = _desc(block_map) if block_map is not None else None
        _run(_L.lmc_indexer_c8_check_state(_ref(kd), _ref(sd) if sd is not None else None, int(slot_factor),
                                           _ref(md) if md is not None else None))
        self.keys, self.scales, self.block_map = keys, scales, block_map
        self.slot_factor = int(slot_factor)
        self.cache_slots = keys.numel() // 128 // self.slot_factor
        self.key_bytes = 128 * keys.element_size()
        self._descs = (kd, sd, md)
        self._table = None

    def _layer_table(self):
        if self._table is None:
            self._table = _c8_table([self])
        return self._table


class IndexerC8GroupState:
    """Several layers moved by one launch (csrc/indexer_c8.cpp:52-74)."""

    def __init__(self, layers):
        layers = list(layers)
        if not layers:
            raise RuntimeError("C8 group holds no layer")
        for st in layers:
            if st.keys.device != layers[0].keys.device or st.cache_slots != layers[0].cache_slots:
                raise RuntimeError("C8 group layers differ in GPU or in slot capacity")
        self.layers = layers
        self.max_key_bytes = max([128] + [st.key_bytes for st in layers])
        self._table = _c8_table(layers)

    def _layer_table(self):
        return self._table


def _c8_table(layers):
    """ctypes arrays of the layers' key / scale / block-map descriptors and
    slot factors, with the device index; they keep the descriptors alive."""
    n = len(layers)
    P = ctypes.POINTER(_lib.LmcTensor)
    ka = (P * n)(*[ctypes.pointer(st._descs[0]) for st in layers])
    sa = (P * n)(*[ctypes.pointer(st._descs[1]) if st._descs[1] is not None else P() for st in layers])
    ma = (P * n)(*[ctypes.pointer(st._descs[2]) if st._descs[2] is not None else P() for st in layers])
    fa = (ctypes.c_int64 * n)(*[st.slot_factor for st in layers])
    return ka, sa, ma, fa, n, _device_index(layers[0].keys)


def _c8(table, packet_ptrs, chunk_offsets, chunk_counts, slot_mapping, chunk_capacity, from_npu, fixed_chunks):
    ka, sa, ma, fa, n, dev = table
    d = [_desc(x) for x in (packet_ptrs, chunk_offsets, chunk_counts, slot_mapping)]
    _run(
        _L.lmc_indexer_c8_transfer(
            ka, sa, ma, fa, n, *[_ref(x) for x in d], int(chunk_capacity), int(bool(from_npu)),
            int(bool(fixed_chunks)), _stream(dev),
        )
    )


def indexer_c8_transfer_prepared(state, packet_ptrs, chunk_offsets, chunk_counts, slot_mapping, chunk_capacity,
                                 from_npu, fixed_chunks=False) -> None:
    """csrc/indexer_c8.cpp:139-158."""
    _c8(state._layer_table(), packet_ptrs, chunk_offsets, chunk_counts, slot_mapping, chunk_capacity, from_npu,
        fixed_chunks)


def indexer_c8_group_transfer_prepared(state, packet_ptrs, chunk_offsets, chunk_counts, slot_mapping,
                                       chunk_capacity, from_npu, fixed_chunks=False) -> None:
    """csrc/indexer_c8.cpp:160-184: packet_ptrs is [layers, chunks]."""
    _c8(state._layer_table(), packet_ptrs, chunk_offsets, chunk_counts, slot_mapping, chunk_capacity, from_npu,
        fixed_chunks)


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


def alloc_pinned_numa_ptr(size: int, node: int) -> int:
    """csrc/common/mem_alloc.cpp:56-92: zeroed pinned memory on NUMA `node`,
    device-mapped and registered like alloc_pinned_ptr."""
    out = ctypes.c_size_t(0)
    _run(_L.lmc_alloc_pinned_numa_ptr(int(size), int(node), ctypes.byref(out)))
    return int(out.value)


def free_pinned_numa_ptr(ptr: int, size: int) -> None:
    """csrc/common/mem_alloc.cpp:94-106."""
    _run(_L.lmc_free_pinned_numa_ptr(int(ptr), int(size)))


def _shm_name(shm_name) -> bytes:
    if not isinstance(shm_name, str):
        raise TypeError("shm_name must be a str")
    return shm_name.encode()


def alloc_shm_pinned_ptr(size: int, shm_name: str, interleave_nodes=()) -> int:
    """csrc/common/mem_alloc.cpp:252-321: creates shared CPU cache slab
    `shm_name` of `size` bytes, interleaved over `interleave_nodes`.  The
    slab is host memory reached by staged copies (not device-mapped)."""
    nodes = [int(n) for n in interleave_nodes]
    arr = (ctypes.c_int32 * max(1, len(nodes)))(*nodes)
    out = ctypes.c_size_t(0)
    _run(_L.lmc_alloc_shm_pinned_ptr(int(size), _shm_name(shm_name), arr, len(nodes),
                                     ctypes.byref(out)))
    return int(out.value)


def attach_shm_pinned_ptr(size: int, shm_name: str, writable: bool = True) -> int:
    """csrc/common/mem_alloc.cpp:323-357."""
    out = ctypes.c_size_t(0)
    _run(_L.lmc_attach_shm_pinned_ptr(int(size), _shm_name(shm_name), 1 if writable else 0,
                                      ctypes.byref(out)))
    return int(out.value)


def free_shm_pinned_ptr(ptr: int, size: int, shm_name: str) -> None:
    """csrc/common/mem_alloc.cpp:359-381."""
    _run(_L.lmc_free_shm_pinned_ptr(int(ptr), int(size), _shm_name(shm_name)))


def detach_shm_pinned_ptr(ptr: int, size: int) -> None:
    """csrc/common/mem_alloc.cpp:383-403."""
    _run(_L.lmc_detach_shm_pinned_ptr(int(ptr), int(size)))


def unlink_shm(shm_name: str) -> None:
    """csrc/common/mem_alloc.cpp:405-410."""
    _run(_L.lmc_unlink_shm(_shm_name(shm_name)))


def _dma_rows(copies) -> "np.ndarray":
    import numpy as np

    rows = np.asarray(copies if len(copies) else np.empty((0, 3)), dtype=np.uint64)
    if rows.ndim != 2 or rows.shape[1] != 3:
        raise TypeError("copies must be a sequence of (dst, src, bytes) tuples")
    return np.ascontiguousarray(rows)


def layerwise_prefill_dma_copy(copies, device_to_host: bool) -> None:
    """csrc/pybind.cpp:295-310: (dst, src, bytes) rows copied host<->device on
    the current stream by the copy engines; rows are merged and batched when
    no two destinations overlap."""
    rows = _dma_rows(copies)
    stream = torch.cuda.current_stream().cuda_stream
    _run(_L.lmc_layerwise_prefill_dma_copy(rows.ctypes.data, rows.shape[0], 1 if device_to_host else 0, stream))


def layerwise_prefill_dma_copy_diagnose(copies, device_to_host: bool):
    """csrc/pybind.cpp:263-294: one copy per row; returns (stream_us,
    stream_address, copy_us) with the host time to obtain the current stream
    and each row's submission time, in microseconds."""
    import time

    import numpy as np

    rows = _dma_rows(copies)
    t0 = time.perf_counter()
    stream = torch.cuda.current_stream().cuda_stream
    stream_us = (time.perf_counter() - t0) * 1e6
    copy_us = np.zeros(rows.shape[0], dtype=np.float64)
    _run(_L.lmc_layerwise_prefill_dma_copy_diagnose(rows.ctypes.data, rows.shape[0], 1 if device_to_host else 0,
                                                    stream, copy_us.ctypes.data))
    return stream_us, int(stream or 0), copy_us.tolist()


def get_gpu_pci_bus_id(device: int) -> str:
    buf = ctypes.create_string_buffer(64)
    _run(_L.lmc_get_gpu_pci_bus_id(int(device), buf, len(buf)))
    return buf.value.decode()
