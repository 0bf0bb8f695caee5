"""CPU oracle for rotary_embedding_k_fused.  TEST INFRASTRUCTURE ONLY: used by
tests, smoke() and bench.py's cpu_baseline, never by the product.

The op (csrc/pos_kernels.cpp:158-196) rotates K in place from its old
positions to new ones: k <- R(new) R(old)^-1 k, per head, on the first
`rot = cos_sin_cache.size(-1)` dims, in the neox (halves) or GPT-J
(interleaved pairs) convention; R(p)^-1 is the rotation by -angle, which the
reference builds by shuffling halves around the forward rope
(lmcache_ascend/v1/blend/positional_encoding.py:62-92).

`fused_rerotate_f32` restates the arithmetic the kernel performs in float32,
one IEEE operation at a time (products, then sums; no fused multiply-add),
followed by one round to the key dtype, so its bf16 output is the kernel's
bit for bit.  `fused_rerotate` evaluates the same rotation in float64 (the
mathematical value) for tolerance checks, and `rope_forward` is the plain
forward rope used by the reference's invariant tests
(tests/v1/test_pos_kernels.py:98-142).
"""

from __future__ import annotations

import numpy as np
import torch


def cos_sin_cache(max_position: int, rot: int, base: float) -> torch.Tensor:
    """[max_position, rot] float32 cache, vLLM's layout: cos | sin halves of
    angle p * base^(-2i/rot)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, rot, 2, dtype=torch.float32) / rot))
    t = torch.arange(max_position, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)


def _pairs(rot: int, neox: bool):
    half = rot // 2
    i = np.arange(half)
    if neox:
        return i, i + half
    return 2 * i, 2 * i + 1


def fused_rerotate_f32(k: np.ndarray, old: np.ndarray, new: np.ndarray, cache: np.ndarray,
                       head_size: int, neox: bool) -> np.ndarray:
    """Float32 restatement of the kernel: k [T, H*hs] float32 values of the
    key dtype; cache [P, rot] float32 values of the cache dtype.  Returns the
    float32 result before the final rounding."""
    k = np.asarray(k, np.float32)
    cache = np.asarray(cache, np.float32)
    T, HD = k.shape
    H = HD // head_size
    rot = cache.shape[1]
    half = rot // 2
    a, b = _pairs(rot, neox)
    kh = k.reshape(T, H, head_size).copy()
    co, so = cache[old, :half][:, None, :], cache[old, half:][:, None, :]
    cn, sn = cache[new, :half][:, None, :], cache[new, half:][:, None, :]
    x1, x2 = kh[:, :, a], kh[:, :, b]
    y1 = (x1 * co).astype(np.float32) + (x2 * so).astype(np.float32)
    y2 = (x2 * co).astype(np.float32) - (x1 * so).astype(np.float32)
    z1 = (y1 * cn).astype(np.float32) - (y2 * sn).astype(np.float32)
    z2 = (y2 * cn).astype(np.float32) + (y1 * sn).astype(np.float32)
    kh[:, :, a] = z1
    kh[:, :, b] = z2
    return kh.reshape(T, HD)


def fused_rerotate(k, old, new, cache, head_size: int, neox: bool) -> np.ndarray:
    """Float64 value of R(new) R(old)^-1 k (no intermediate rounding)."""
    k = np.asarray(k, np.float64)
    cache = np.asarray(cache, np.float64)
    T, HD = k.shape
    H = HD // head_size
    rot = cache.shape[1]
    half = rot // 2
    a, b = _pairs(rot, neox)
    kh = k.reshape(T, H, head_size).copy()
    co, so = cache[old, :half][:, None, :], cache[old, half:][:, None, :]
    cn, sn = cache[new, :half][:, None, :], cache[new, half:][:, None, :]
    x1, x2 = kh[:, :, a], kh[:, :, b]
    y1 = x1 * co + x2 * so
    y2 = x2 * co - x1 * so
    kh[:, :, a] = y1 * cn - y2 * sn
    kh[:, :, b] = y2 * cn + y1 * sn
    return kh.reshape(T, HD)


def rope_forward(k, pos, cache, head_size: int, neox: bool) -> np.ndarray:
    """Forward rope R(pos) k in float64."""
    k = np.asarray(k, np.float64)
    cache = np.asarray(cache, np.float64)
    T, HD = k.shape
    H = HD // head_size
    rot = cache.shape[1]
    half = rot // 2
    a, b = _pairs(rot, neox)
    kh = k.reshape(T, H, head_size).copy()
    c, s = cache[pos, :half][:, None, :], cache[pos, half:][:, None, :]
    x1, x2 = kh[:, :, a], kh[:, :, b]
    kh[:, :, a] = x1 * c - x2 * s
    kh[:, :, b] = x2 * c + x1 * s
    return kh.reshape(T, HD)


def round_to(x: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """Round float32 values to `dtype` (round to nearest even) and back."""
    return torch.from_numpy(np.asarray(x, np.float32)).to(dtype).float().numpy()
