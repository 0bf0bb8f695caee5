"""The per-call ops through both host paths: the C++ binding (the default
when it is built) and ctypes (`c_ops._ext` set to None).  Both call the same
C ABI, so every output byte must agree; the binding path itself is checked
against the oracle by the other GPU tests."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvutil import block_slots, ptr_table, randn_bf16, to_bytes

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
L, NB, BS, H, D = 4, 32, 16, 8, 128
W = H * D


@pytest.fixture(scope="module")
def ops():
    import lmcache_amd

    return lmcache_amd.c_ops


def _both(ops, monkeypatch, run):
    """run(ops) on fresh state with the binding, then with ctypes; returns
    the two outputs (lists of tensors)."""
    if ops._ext is None:
        pytest.skip("the C++ binding is not built")
    a = run(ops)
    torch.cuda.synchronize()
    monkeypatch.setattr(ops, "_ext", None)
    b = run(ops)
    torch.cuda.synchronize()
    return a, b


def _assert_same(a, b):
    for x, y in zip(a, b):
        assert np.array_equal(to_bytes(x), to_bytes(y))


def _caches(seed):
    gen = torch.Generator().manual_seed(seed)
    return [randn_bf16((NB, BS, H, D), gen).to(DEV) for _ in range(2 * L)]


def _slots(n, seed):
    rng = np.random.default_rng(seed)
    blocks = rng.permutation(NB)[: (n + BS - 1) // BS].tolist()
    s = torch.tensor(block_slots(blocks, BS, [n]), dtype=torch.int64)
    s[3] = -1
    return s.to(DEV)


@pytest.mark.parametrize("direction", [True, False])
def test_multi_layer_paths_agree(ops, monkeypatch, direction):
    T = 100

    def run(o):
        caches = _caches(1)
        kv = randn_bf16((2, L, T, W), torch.Generator().manual_seed(2)).to(DEV)
        o.multi_layer_kv_transfer(kv, ptr_table(caches, DEV), _slots(T, 3), torch.device(DEV), NB * BS,
                                  direction, False, 2)
        return [kv] + caches

    _assert_same(*_both(ops, monkeypatch, run))


@pytest.mark.parametrize("direction", [True, False])
def test_single_layer_paths_agree(ops, monkeypatch, direction):
    T = 90

    def run(o):
        caches = _caches(4)[:2]
        buf = randn_bf16((2, T, W), torch.Generator().manual_seed(5)).to(DEV)
        o.single_layer_kv_transfer(buf, tuple(caches), _slots(T, 6), direction, 2)
        return [buf] + caches

    _assert_same(*_both(ops, monkeypatch, run))


@pytest.mark.parametrize("load", [True, False])
def test_flash_paths_agree(ops, monkeypatch, load):
    T = 70

    def run(o):
        kc, vc = _caches(7)[:2]
        kv = randn_bf16((2, L, T, W), torch.Generator().manual_seed(8)).to(DEV)
        fn = o.load_and_reshape_flash if load else o.reshape_and_cache_back_flash
        fn(kv, kc.view(-1, H, D), vc.view(-1, H, D), _slots(T, 9), 2)
        return [kv, kc, vc]

    _assert_same(*_both(ops, monkeypatch, run))


def test_rope_paths_agree(ops, monkeypatch):
    T, max_pos = 64, 512
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    ang = torch.outer(torch.arange(max_pos, dtype=torch.float32), inv)
    cache = torch.cat((ang.cos(), ang.sin()), dim=-1).to(torch.bfloat16).to(DEV)
    old = torch.arange(T, dtype=torch.int64, device=DEV)
    new = old + 100

    def run(o):
        key = randn_bf16((T, W), torch.Generator().manual_seed(10)).to(DEV)
        o.rotary_embedding_k_fused(old, new, key, D, cache, True)
        return [key]

    _assert_same(*_both(ops, monkeypatch, run))
