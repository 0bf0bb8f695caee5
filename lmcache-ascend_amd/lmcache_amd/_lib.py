"""Loader and ctypes bindings for liblmcache_amd.so (the C ABI in
include/lmcache_amd.h).

The library is the only implementation of every op: when it is missing the
import fails loudly; nothing falls back to a CPU path.
"""

from __future__ import annotations

import ctypes
import os

# LMCACHE_AMD_LIB selects another build of the library (for example one
# compiled with different launch geometry).
LIB_PATH = os.environ.get("LMCACHE_AMD_LIB") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "liblmcache_amd.so"
)

MAX_DIMS = 6

# Status codes (enum lmc_status).
OK = 0
ERR_VALUE = 1
ERR_RUNTIME = 2
ERR_NOT_IMPLEMENTED = 3
ERR_HIP = 4

# dtype codes (enum lmc_dtype).
U8, I8, I16, I32, I64, F16, BF16, F32 = range(8)


class LmcTensor(ctypes.Structure):
    """struct lmc_tensor."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("device", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("sizes", ctypes.c_int64 * MAX_DIMS),
        ("strides", ctypes.c_int64 * MAX_DIMS),
    ]


_T = ctypes.POINTER(LmcTensor)
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_up = ctypes.c_size_t  # uintptr_t
_sz = ctypes.c_size_t

# name -> argtypes; every entry point returns int (status).
SIGNATURES = {
    "lmc_multi_layer_kv_transfer": [_T, _T, _T, _i32, _i64, _i32, _i32, _i32, _i64, _i64, _i64, _vp],
    "lmc_multi_layer_kv_transfer_batched": [
        _T, _i32, ctypes.POINTER(_i64), _T, _T, _i32, _i64, _i32, _i32, _i32, _i64, _i64, _i64, _vp,
    ],
    "lmc_fused_multi_layer_kv_transfer": [_T, _T, _T, _T, _i32, _i64, _i32, _i32, _i32, _i64, _i64, _i64, _vp],
    "lmc_fused_multi_layer_kv_transfer_noalloc": [_T, _T, _T, _i32, _i64, _i32, _i32, _i32, _i64, _i64, _i64, _vp],
    "lmc_blend_layer_to_paged": [_T, _i32, ctypes.POINTER(_i64), _T, _i32, _T, _T, _T, _T, _i64, _i32, _i32, _i32,
                                 _vp],
    "lmc_single_layer_kv_transfer": [_T, _T, _i32, _T, _i32, _i32, _i32, _i32, _i64, _i64, _i64, _vp],
    "lmc_load_and_reshape_flash": [_T, _T, _T, _T, _i32, _vp],
    "lmc_reshape_and_cache_back_flash": [_T, _T, _T, _T, _i32, _vp],
    "lmc_sparse_single_layer_kv_transfer": [_T, _T, _i32, _T, _T, _i32, _i32, _i32, _i64, _i64, _i64, _vp],
    "lmc_sparse_direct_kv_transfer": [
        _T, _T, _T, _i32, _T, _T, _T, _i64, _i64, _i32, _i32, _i32, _i64, _i64, _i64, _i32, _i32, _vp,
    ],
    "lmc_dense_direct_kv_transfer": [
        _T, _T, _i32, _T, _T, _T, _i64, _i64, _i32, _i32, _i64, _i64, _i64, _i32, _i32, _i32, _vp,
    ],
    "lmc_batched_fused_single_layer_kv_transfer": [
        _T, _i32, _T, _T, _i32, _T, ctypes.POINTER(_i64), ctypes.POINTER(_i64), _i32, _i32, _i32, _i32,
        _i64, _i64, _i64, _vp,
    ],
    "lmc_batched_fused_sparse_single_layer_kv_transfer": [
        _T, _i32, _T, _T, _i32, _T, _T, ctypes.POINTER(_i64), ctypes.POINTER(_i64), _i32, _i32, _i32,
        _i64, _i64, _i64, _vp,
    ],
    "lmc_check_kv_caches": [_T, _i32, _i32, _i32, _i64, _i64, _i64],
    "lmc_sparse_graph_kv_transfer": [_T, _T, _i64, _i64, _T, _T, _T, _T, _T, _i64, _i64, _vp],
    "lmc_indexer_c8_check_state": [_T, _T, _i64, _T],
    "lmc_indexer_c8_transfer": [
        ctypes.POINTER(_T), ctypes.POINTER(_T), ctypes.POINTER(_T), ctypes.POINTER(_i64), _i32, _T, _T, _T, _T,
        _i64, _i32, _i32, _vp,
    ],
    "lmc_calculate_cdf": [_T, _i32, _T, _vp],
    "lmc_encode_fast_new": [_T, _T, _T, _T, _vp],
    "lmc_decode_fast_new": [_T, _T, _T, _T, _vp],
    "lmc_decode_fast_prefsum": [_T, _T, _T, _T, _vp],
    "lmc_rotary_embedding_k_fused": [_T, _T, _T, _i64, _T, _i32, _vp],
    "lmc_get_device_ptr": [_up, _sz, ctypes.POINTER(_up)],
    "lmc_register_mapping": [_up, _up, _sz, ctypes.POINTER(_up)],
    "lmc_unregister_ptr": [_up, ctypes.POINTER(_i32)],
    "lmc_alloc_pinned_ptr": [_sz, ctypes.c_uint32, ctypes.POINTER(_up)],
    "lmc_free_pinned_ptr": [_up],
    "lmc_alloc_pinned_numa_ptr": [_sz, _i32, ctypes.POINTER(_up)],
    "lmc_free_pinned_numa_ptr": [_up, _sz],
    "lmc_alloc_shm_pinned_ptr": [_sz, ctypes.c_char_p, ctypes.POINTER(_i32), _i32, ctypes.POINTER(_up)],
    "lmc_attach_shm_pinned_ptr": [_sz, ctypes.c_char_p, _i32, ctypes.POINTER(_up)],
    "lmc_free_shm_pinned_ptr": [_up, _sz, ctypes.c_char_p],
    "lmc_detach_shm_pinned_ptr": [_up, _sz],
    "lmc_unlink_shm": [ctypes.c_char_p],
    "lmc_layerwise_prefill_dma_copy": [_vp, _i64, _i32, _vp],
    "lmc_layerwise_prefill_dma_copy_diagnose": [_vp, _i64, _i32, _vp, _vp],
    "lmc_get_gpu_pci_bus_id": [_i32, ctypes.c_char_p, _i32],
}

_lib = None


def load() -> ctypes.CDLL:
    """Loads the library once; raises ImportError when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with "
            "`python lmcache-ascend_amd/build.py` (hipcc, gfx950)"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    lib.lmc_last_error.argtypes = []
    lib.lmc_last_error.restype = ctypes.c_char_p
    lib.lmc_version.argtypes = []
    lib.lmc_version.restype = ctypes.c_char_p
    _lib = lib
    return lib


def exported_symbols():
    """Names the header declares (used by the ABI test)."""
    return list(SIGNATURES) + ["lmc_last_error", "lmc_version"]


def raise_for(status: int) -> None:
    """Raises the Python exception the reference raises for this status."""
    if status == OK:
        return
    msg = _lib.lmc_last_error().decode(errors="replace") if _lib is not None else ""
    if status == ERR_VALUE:
        raise ValueError(msg)
    if status == ERR_NOT_IMPLEMENTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)
