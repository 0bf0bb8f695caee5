"""GPU checks of lmc_fused_multi_layer_kv_transfer_noalloc, the staged
multi-layer transfer that stages through the library's static per-GPU area
instead of a caller's staging_cache.

Its output must equal lmc_fused_multi_layer_kv_transfer's
(csrc/mem_kernels.cpp:113-213) given a zeroed staging_cache: byte for byte
in the host memory object after a store (rows of skipped slots are zeros in
both) and in the paged caches after a load.  Each direction runs two calls
in a row, the second with fewer tokens and more skipped slots than the
first, so the second store also shows that the area's stale contents from
the first call do not leak into rows of skipped slots.  The op is also
captured into HIP graphs (as the first call of the process) and replayed,
and eager calls on two streams are checked to be ordered.
"""

from __future__ import annotations

import pytest
import torch

from kvutil import ptr_table, randn_bf16

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
L, NB, BS, H, D = 4, 64, 16, 8, 128
W = H * D
PBS = NB * BS


@pytest.fixture(scope="module")
def ops():
    import lmcache_amd

    return lmcache_amd.c_ops


def _planes(fmt, gen):
    if fmt == 1:  # MERGED: one two-major [2, NB, BS, H, D] tensor per layer
        return [randn_bf16((2, NB, BS, H, D), gen).to(DEV) for _ in range(L)]
    return [randn_bf16((NB, BS, H, D), gen).to(DEV) for _ in range(2 * L)]


def _slots(T, seed, n_skip):
    g = torch.Generator().manual_seed(seed)
    s = torch.randperm(PBS, generator=g)[:T].to(torch.int64)
    skip = torch.randperm(T, generator=g)[:n_skip]
    s[skip[: n_skip // 2]] = -1
    s[skip[n_skip // 2:]] = PBS + 7  # out of range: skipped as well
    return s.to(DEV)


CALLS = [(256, 12), (96, 40)]  # (tokens, skipped slots): the second call is smaller


def _staged(ops, host, ptrs, slots, direction, fmt):
    T = slots.shape[0]
    staging = torch.zeros((2, L, T, W), dtype=torch.bfloat16, device=DEV)
    ops.fused_multi_layer_kv_transfer(host, staging, ptrs, slots, torch.device(DEV), PBS, direction, False, fmt,
                                      W, W, 0)


def test_noalloc_first_call_under_graph_capture(ops):
    """Defined first in this file, so in a test session it makes the
    process's first call of the entry point, inside a HIP graph capture
    (where the staging area is resolved).  Store and load graphs are
    replayed three times each on new cache or host-object contents written
    eagerly between replays; every replay equals the staged op given a
    zeroed staging tensor."""
    fmt = 2
    gen = torch.Generator().manual_seed(300)
    caches = _planes(fmt, gen)
    ptrs = ptr_table(caches, DEV)
    T, n_skip = 256, 12
    slots = _slots(T, 31, n_skip)
    got = torch.zeros((2, L, T, W), dtype=torch.bfloat16).pin_memory()
    torch.cuda.synchronize()
    g_store = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_store):
        ops.fused_multi_layer_kv_transfer_noalloc(got, ptrs, slots, torch.device(DEV), PBS, True, False, fmt,
                                                  W, W, 0)
    src = randn_bf16((2, L, T, W), gen).pin_memory()
    dst = [torch.zeros_like(t) for t in caches]
    dptrs = ptr_table(dst, DEV)
    g_load = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_load):
        ops.fused_multi_layer_kv_transfer_noalloc(src, dptrs, slots, torch.device(DEV), PBS, False, False, fmt,
                                                  W, W, 0)
    for r in range(3):
        for t in caches:
            t.copy_(randn_bf16(tuple(t.shape), gen))
        got.fill_(7.0)
        torch.cuda.synchronize()
        g_store.replay()
        torch.cuda.synchronize()
        want = torch.full((2, L, T, W), 7.0, dtype=torch.bfloat16).pin_memory()
        _staged(ops, want, ptrs, slots, True, fmt)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"store replay {r} differs"
        src.copy_(randn_bf16((2, L, T, W), gen))
        for t in dst:
            t.fill_(5.0)
        torch.cuda.synchronize()
        g_load.replay()
        torch.cuda.synchronize()
        ref = [torch.full_like(t, 5.0) for t in dst]
        _staged(ops, src, ptr_table(ref, DEV), slots, False, fmt)
        torch.cuda.synchronize()
        for a, b in zip(dst, ref):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"load replay {r} differs"


def test_noalloc_calls_on_two_streams_are_ordered(ops):
    """A store on one stream and a load on another, enqueued back to back
    without synchronising: both use the one staging area, and the second
    call's stream waits for the first's work, so both results equal the
    staged op's."""
    fmt = 1
    gen = torch.Generator().manual_seed(400)
    caches = _planes(fmt, gen)
    ptrs = ptr_table(caches, DEV)
    dst = [torch.full_like(t, 5.0) for t in caches]
    dptrs = ptr_table(dst, DEV)
    T = 256
    s_store, s_load = _slots(T, 41, 10), _slots(T, 43, 10)
    got = torch.zeros((2, L, T, W), dtype=torch.bfloat16).pin_memory()
    src = randn_bf16((2, L, T, W), gen).pin_memory()
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    for _ in range(3):
        with torch.cuda.stream(a):
            ops.fused_multi_layer_kv_transfer_noalloc(got, ptrs, s_store, torch.device(DEV), PBS, True, False, fmt,
                                                      W, W, 0)
        with torch.cuda.stream(b):
            ops.fused_multi_layer_kv_transfer_noalloc(src, dptrs, s_load, torch.device(DEV), PBS, False, False,
                                                      fmt, W, W, 0)
    torch.cuda.synchronize()
    want = torch.zeros((2, L, T, W), dtype=torch.bfloat16).pin_memory()
    _staged(ops, want, ptrs, s_store, True, fmt)
    ref = [torch.full_like(t, 5.0) for t in caches]
    _staged(ops, src, ptr_table(ref, DEV), s_load, False, fmt)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    for x, y in zip(dst, ref):
        assert torch.equal(x.view(torch.int16), y.view(torch.int16))


@pytest.mark.parametrize("fmt", [1, 2])
def test_noalloc_store_equals_staged_store(ops, fmt):
    gen = torch.Generator().manual_seed(100 + fmt)
    caches = _planes(fmt, gen)
    ptrs = ptr_table(caches, DEV)
    for T, n_skip in CALLS:
        slots = _slots(T, 7 * T + fmt, n_skip)
        want = torch.full((2, L, T, W), 3.0, dtype=torch.bfloat16).pin_memory()
        got = torch.full((2, L, T, W), 3.0, dtype=torch.bfloat16).pin_memory()
        staging = torch.zeros((2, L, T, W), dtype=torch.bfloat16, device=DEV)
        ops.fused_multi_layer_kv_transfer(want, staging, ptrs, slots, torch.device(DEV), PBS, True, False, fmt,
                                          W, W, 0)
        ops.fused_multi_layer_kv_transfer_noalloc(got, ptrs, slots, torch.device(DEV), PBS, True, False, fmt,
                                                  W, W, 0)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"store T={T} differs"
        skipped = (slots < 0) | (slots >= PBS)
        assert int(skipped.sum()) == n_skip
        assert not got.view(torch.int16)[:, :, skipped.cpu()].any(), "skipped rows must arrive as zeros"


@pytest.mark.parametrize("fmt", [1, 2])
def test_noalloc_load_equals_staged_load(ops, fmt):
    gen = torch.Generator().manual_seed(200 + fmt)
    shape = _planes(fmt, gen)
    for T, n_skip in CALLS:
        slots = _slots(T, 11 * T + fmt, n_skip)
        src = randn_bf16((2, L, T, W), gen).pin_memory()
        want = [torch.full_like(t, 5.0) for t in shape]
        got = [torch.full_like(t, 5.0) for t in shape]
        staging = torch.zeros((2, L, T, W), dtype=torch.bfloat16, device=DEV)
        ops.fused_multi_layer_kv_transfer(src, staging, ptr_table(want, DEV), slots, torch.device(DEV), PBS, False,
                                          False, fmt, W, W, 0)
        ops.fused_multi_layer_kv_transfer_noalloc(src, ptr_table(got, DEV), slots, torch.device(DEV), PBS, False,
                                                  False, fmt, W, W, 0)
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"load T={T} differs"


def test_noalloc_refuses_more_than_its_staging_area(ops):
    T = 1024
    big = torch.empty((2, 32, T, W), dtype=torch.bfloat16)  # 128 MiB, above the 64 MiB area
    assert big.numel() * 2 > ops.NOALLOC_STAGING_BYTES
    caches = [torch.zeros((8, BS, H, D), dtype=torch.bfloat16, device=DEV) for _ in range(64)]
    slots = torch.arange(T, dtype=torch.int64, device=DEV)
    with pytest.raises(RuntimeError, match="exceeds the library's staging area"):
        ops.fused_multi_layer_kv_transfer_noalloc(big, ptr_table(caches, DEV), slots, torch.device(DEV), 8 * BS,
                                                  True, False, 2, W, W, 0)
