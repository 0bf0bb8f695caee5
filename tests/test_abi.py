"""CPU checks of the C ABI library: it loads, it exports every function
include/lmcache_amd.h declares, the ctypes table covers them, and argument
validation that runs before any device call maps to the reference's
exception types (no kernel is launched here)."""

import ctypes
import os
import re

import pytest

from lmcache_amd import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "lmcache_amd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lmc_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "lmc_multi_layer_kv_transfer" in names
    assert len(names) >= 19


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_ctypes_table_matches_header():
    assert sorted(_lib.exported_symbols()) == declared_functions()


def test_version_string():
    lib = _lib.load()
    assert b"gfx950" in lib.lmc_version()


def _t(dtype=_lib.BF16, device=0, shape=(1,)):
    d = _lib.LmcTensor()
    d.data = 0x1000
    d.dtype = dtype
    d.device = device
    d.ndim = len(shape)
    stride = 1
    for i in reversed(range(len(shape))):
        d.sizes[i] = shape[i]
        d.strides[i] = stride
        stride *= shape[i]
    return d


def test_single_layer_invalid_format_is_value_error():
    # csrc/utils.cpp:908-920
    lib = _lib.load()
    lmc = _t(shape=(2, 4, 16))
    caches = (_lib.LmcTensor * 1)(_t(shape=(2, 4, 2, 2, 4)))
    slots = _t(_lib.I64, shape=(4,))
    st = lib.lmc_single_layer_kv_transfer(ctypes.byref(lmc), caches, 1, ctypes.byref(slots),
                                          1, 9, 0, 0, 0, 0, 0, None)
    assert st == _lib.ERR_VALUE
    assert b"9 is not a KV cache format" in lib.lmc_last_error()
    with pytest.raises(ValueError, match="is not a KV cache format"):
        _lib.raise_for(st)


@pytest.mark.parametrize(
    "fmt,n,msg",
    [
        (2, 1, b"a SEPARATE_KV layer takes two caches"),
        (1, 2, b"a MERGED_KV layer takes one cache"),
        (4, 2, b"a DSA_KV layer takes three caches"),
        (3, 1, b"an MLA_KV or MLA_LATENT layer takes two caches"),
    ],
)
def test_single_layer_tuple_size_checks(fmt, n, msg):
    # csrc/utils.cpp:922-963
    lib = _lib.load()
    lmc = _t(shape=(2, 4, 16))
    caches = (_lib.LmcTensor * n)(*[_t(shape=(4, 2, 2, 4)) for _ in range(n)])
    slots = _t(_lib.I64, shape=(4,))
    st = lib.lmc_single_layer_kv_transfer(ctypes.byref(lmc), caches, n, ctypes.byref(slots),
                                          1, fmt, 0, 0, 0, 0, 0, None)
    assert st == _lib.ERR_VALUE
    assert msg in lib.lmc_last_error()


def test_single_layer_separate_shape_mismatch():
    lib = _lib.load()
    lmc = _t(shape=(2, 4, 16))
    caches = (_lib.LmcTensor * 2)(_t(shape=(4, 2, 2, 4)), _t(shape=(5, 2, 2, 4)))
    slots = _t(_lib.I64, shape=(4,))
    st = lib.lmc_single_layer_kv_transfer(ctypes.byref(lmc), caches, 2, ctypes.byref(slots),
                                          1, 2, 0, 0, 0, 0, 0, None)
    assert st == _lib.ERR_VALUE
    assert b"K and V caches differ in shape" in lib.lmc_last_error()


def test_multi_layer_unsupported_format_is_runtime_error():
    # csrc/utils.cpp:83 (TORCH_CHECK -> RuntimeError)
    lib = _lib.load()
    kv = _t(shape=(2, 4, 8, 16))
    ptrs = _t(_lib.I64, shape=(8,))
    slots = _t(_lib.I64, shape=(8,))
    st = lib.lmc_multi_layer_kv_transfer(ctypes.byref(kv), ctypes.byref(ptrs), ctypes.byref(slots),
                                         0, 64, 1, 0, 7, 0, 0, 0, None)
    assert st == _lib.ERR_RUNTIME
    assert b"no plane layout for KV format 7" in lib.lmc_last_error()


def test_multi_layer_rejects_short_pointer_table():
    lib = _lib.load()
    kv = _t(shape=(2, 4, 8, 16))
    ptrs = _t(_lib.I64, shape=(7,))  # SEPARATE needs 2 per layer = 8
    slots = _t(_lib.I64, shape=(8,))
    st = lib.lmc_multi_layer_kv_transfer(ctypes.byref(kv), ctypes.byref(ptrs), ctypes.byref(slots),
                                         0, 64, 1, 0, 2, 0, 0, 0, None)
    assert st == _lib.ERR_RUNTIME
    assert b"key_value_ptrs" in lib.lmc_last_error()


def test_get_device_ptr_of_null_is_zero():
    lib = _lib.load()
    out = ctypes.c_size_t(123)
    assert lib.lmc_get_device_ptr(0, 1, ctypes.byref(out)) == _lib.OK
    assert out.value == 0


def test_decode_fast_new_not_implemented():
    # csrc/cachegen_kernels.cpp:60-65
    lib = _lib.load()
    t = _t(_lib.U8)
    st = lib.lmc_decode_fast_new(ctypes.byref(t), ctypes.byref(t), ctypes.byref(t), ctypes.byref(t), None)
    assert st == _lib.ERR_NOT_IMPLEMENTED
