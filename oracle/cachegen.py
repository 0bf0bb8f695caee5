"""Python entry to the CacheGen oracle (oracle/cachegen.c).  TEST
INFRASTRUCTURE ONLY: used by tests, smoke() and bench.py's cpu_baseline.

The codec rules (L1-L6) are documented at the top of oracle/cachegen.c.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

from . import build_oracle

_lib = None


def load_library(path: str):
    """Binds the oracle's C functions from the shared library at `path`."""
    lib = ctypes.CDLL(path)
    P = ctypes.c_void_p
    i = ctypes.c_int
    lib.oc_calculate_cdf.argtypes = [P, i, i, i, i, P]
    lib.oc_encode.argtypes = [P, P, i, i, i, i, P, i, P]
    lib.oc_decode.argtypes = [P, P, ctypes.c_int64, P, i, i, i, i, P]
    for f in (lib.oc_calculate_cdf, lib.oc_encode, lib.oc_decode):
        f.restype = None
    return lib


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(build_oracle.LIB):
            build_oracle.build()
        _lib = load_library(build_oracle.LIB)
    return _lib




def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def calculate_cdf(sym: np.ndarray, n_bins: int) -> np.ndarray:
    """[L, T, C] u8 symbols -> int16 [L, C, n_bins + 1] (rule L4)."""
    sym = np.ascontiguousarray(sym).view(np.uint8)
    L, T, C = sym.shape
    out = np.zeros((L, C, n_bins + 1), np.int16)
    _load().oc_calculate_cdf(_p(sym), L, T, C, n_bins, _p(out))
    return out


def encode(cdf: np.ndarray, sym: np.ndarray, chunk: int, out: np.ndarray = None):
    """Rule L5.  Returns (bytes [L, C, chunk] u8, lengths [L, C] int32)."""
    cdf = np.ascontiguousarray(cdf, dtype=np.int16)
    sym = np.ascontiguousarray(sym).view(np.uint8)
    L, T, C = sym.shape
    nb = cdf.shape[2] - 1
    if out is None:
        out = np.zeros((L, C, chunk), np.uint8)
    lens = np.zeros((L, C), np.int32)
    _load().oc_encode(_p(cdf), _p(sym), L, T, C, nb, _p(out), chunk, _p(lens))
    return out, lens


def concat_streams(out: np.ndarray, lens: np.ndarray):
    """Concatenates streams in (layer, channel) order; returns (bytes,
    inclusive prefix sums [L, C] int32) as decode_fast_prefsum takes them."""
    L, C, chunk = out.shape
    flat = lens.reshape(-1)
    parts = [out.reshape(L * C, chunk)[i, : min(int(n), chunk)] for i, n in enumerate(flat)]
    stream = np.concatenate(parts) if parts else np.zeros(0, np.uint8)
    pref = np.cumsum(np.minimum(flat, chunk)).astype(np.int32).reshape(L, C)
    return np.ascontiguousarray(stream, dtype=np.uint8), pref


def decode(cdf: np.ndarray, stream: np.ndarray, prefix: np.ndarray, T: int) -> np.ndarray:
    """Rule L6.  Returns [L, T, C] u8."""
    cdf = np.ascontiguousarray(cdf, dtype=np.int16)
    stream = np.ascontiguousarray(stream, dtype=np.uint8)
    prefix = np.ascontiguousarray(prefix, dtype=np.int32)
    L, C, nb1 = cdf.shape
    out = np.zeros((L, T, C), np.uint8)
    _load().oc_decode(_p(cdf), _p(stream), stream.size, _p(prefix), L, T, C, nb1 - 1, _p(out))
    return out


def quantize(x: np.ndarray, bins) -> np.ndarray:
    """Per-(layer, channel) symmetric quantiser for [L, T, C] float data:
    q = round(x / max|x| * (bins/2 - 1)) + bins/2 - 1, in [0, bins - 2].
    `bins` is a scalar or one value per layer.  (The upstream LMCache
    quantiser is not available offline; this one only has to produce
    realistic symbols for the codec.)"""
    x = np.asarray(x, np.float32)
    L = x.shape[0]
    b = np.broadcast_to(np.asarray(bins, np.int64), (L,)).reshape(L, 1, 1)
    half = (b // 2 - 1).astype(np.float32)
    amax = np.abs(x).max(axis=1, keepdims=True)
    amax = np.where(amax == 0, 1.0, amax).astype(np.float32)
    q = np.rint(x / amax * half) + half
    return np.clip(q, 0, (b - 1).astype(np.float32)).astype(np.uint8)
