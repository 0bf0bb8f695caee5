"""GPU parity of layerwise_prefill_dma_copy (csrc/pybind.cpp:263-310)
against the oracle's in-order memcpy of every row: the planner's rows for
consecutive blocks (rectangular runs over chunks), scattered blocks (one
copy per row), rows adjacent in both address spaces (merged), overlapping
destinations (caller's order kept), overlapping sources, odd offsets and
sizes, zero-byte rows, pageable host memory, and the diagnostic variant."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_transfer as ok

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def ops():
    import lmcache_amd

    return lmcache_amd.c_ops


def _np(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().copy()


def _rand_u8(n, gen, pinned=True):
    t = torch.randint(0, 256, (n,), dtype=torch.uint8, generator=gen)
    return t.pin_memory() if pinned else t


def _spaces(host, caches):
    return [(host.data_ptr(), _np(host))] + [(c.data_ptr(), _np(c)) for c in caches]


@pytest.mark.parametrize("consecutive", [True, False])
@pytest.mark.parametrize("pinned", [True, False])
@pytest.mark.parametrize("widths", [(1024, 1024), (512, 64)])
def test_planner_rows_load_and_store(ops, consecutive, pinned, widths):
    gen = torch.Generator().manual_seed(consecutive * 2 + pinned + widths[1])
    bs, chunk, n_chunks = 16, 64, 4
    T = chunk * n_chunks
    nb = T // bs
    NB = 3 * nb
    pb = [w * 2 for w in widths]
    rng = np.random.default_rng(7)
    blocks = np.arange(5, 5 + nb) if consecutive else rng.permutation(NB)[:nb]
    host = _rand_u8(T * sum(pb), gen, pinned)
    caches = [torch.zeros(NB * bs * b, dtype=torch.uint8, device=DEV) for b in pb]
    starts = [c * chunk for c in range(n_chunks)]
    ends = [(c + 1) * chunk for c in range(n_chunks)]
    chunk_addrs = [host.data_ptr() + c * chunk * sum(pb) for c in range(n_chunks)]
    cache_addrs = [c.data_ptr() for c in caches]
    rows = ok.layerwise_dma_rows(chunk_addrs, [chunk] * n_chunks, cache_addrs, pb, blocks, bs, starts, ends, False)
    spaces = _spaces(host, caches)
    ok.layerwise_dma_copy(spaces, rows)  # also checks every row lies inside its buffers
    ops.layerwise_prefill_dma_copy(rows, False)
    torch.cuda.synchronize()
    for c, (_, want) in zip(caches, spaces[1:]):
        assert np.array_equal(_np(c), want)
    # store: caches -> a zeroed host buffer
    back = torch.zeros_like(host)
    if pinned:
        back = back.pin_memory()
    addrs = [back.data_ptr() + c * chunk * sum(pb) for c in range(n_chunks)]
    rows_out = ok.layerwise_dma_rows(addrs, [chunk] * n_chunks, cache_addrs, pb, blocks, bs, starts, ends, True)
    ok.layerwise_dma_copy(_spaces(back, caches), rows_out)
    ops.layerwise_prefill_dma_copy(rows_out, True)
    torch.cuda.synchronize()
    assert torch.equal(back, host)


def _random_disjoint_rows(rng, dst_base, dst_len, src_base, src_len, n, align):
    """n rows with disjoint destinations (random gaps), random sources."""
    cuts = np.sort(rng.choice(np.arange(1, dst_len // align), size=2 * n, replace=False)) * align
    rows = []
    for k in range(n):
        d0, d1 = int(cuts[2 * k]), int(cuts[2 * k + 1])
        size = d1 - d0
        s0 = int(rng.integers(0, (src_len - size) // align + 1)) * align
        rows.append((dst_base + d0, src_base + s0, size))
    order = rng.permutation(n)
    return [rows[i] for i in order]


@pytest.mark.parametrize("align", [1, 2, 16])
@pytest.mark.parametrize("d2h", [False, True])
def test_random_disjoint_rows(ops, align, d2h):
    rng = np.random.default_rng(align * 3 + d2h)
    gen = torch.Generator().manual_seed(align)
    hsz, dsz = 1 << 20, 1 << 20
    host = _rand_u8(hsz, gen)
    dev = torch.randint(0, 256, (dsz,), dtype=torch.uint8, generator=gen).to(DEV)
    if d2h:
        rows = _random_disjoint_rows(rng, host.data_ptr(), hsz, dev.data_ptr(), dsz, 200, align)
    else:
        rows = _random_disjoint_rows(rng, dev.data_ptr(), dsz, host.data_ptr(), hsz, 200, align)
    rows.append((rows[0][0], rows[0][1], 0))  # zero bytes: skipped
    spaces = _spaces(host, [dev])
    ok.layerwise_dma_copy(spaces, rows)
    ops.layerwise_prefill_dma_copy(rows, d2h)
    torch.cuda.synchronize()
    assert np.array_equal(host.numpy(), spaces[0][1])
    assert np.array_equal(_np(dev), spaces[1][1])


@pytest.mark.parametrize("pinned", [True, False])
@pytest.mark.parametrize("d2h", [False, True])
def test_merge_and_rectangular_runs(ops, d2h, pinned):
    """Rows adjacent on both sides (merged), equal-pitch runs (one
    rectangular copy when the host side is pageable, the copy kernel when it
    is pinned), a pitch smaller than the row on the source side (overlapping
    sources: one copy per row) and a broadcast source."""
    gen = torch.Generator().manual_seed(11 + d2h)
    host = _rand_u8(1 << 18, gen, pinned)
    dev = torch.randint(0, 256, (1 << 18,), dtype=torch.uint8, generator=gen).to(DEV)
    h, d = host.data_ptr(), dev.data_ptr()
    rows = []
    far, near = (h, d) if d2h else (d, h)  # (destination space, source space)
    for i in range(8):                       # adjacent both sides -> one row
        rows.append((far + 1000 + 96 * i, near + 50 + 96 * i, 96))
    for i in range(16):                      # dst pitch 512, src pitch 200
        rows.append((far + 20000 + 512 * i, near + 10000 + 200 * i, 160))
    for i in range(6):                       # src pitch 50 < 160 bytes
        rows.append((far + 40000 + 400 * i, near + 30000 + 50 * i, 160))
    for i in range(5):                       # same source for every row
        rows.append((far + 60000 + 1024 * i, near + 50000, 300))
    for i in range(3):                       # pitch 4096, odd length
        rows.append((far + 100001 + 4096 * i, near + 80003 + 1000 * i, 777))
    spaces = _spaces(host, [dev])
    ok.layerwise_dma_copy(spaces, rows)
    ops.layerwise_prefill_dma_copy(rows, d2h)
    torch.cuda.synchronize()
    assert np.array_equal(host.numpy(), spaces[0][1])
    assert np.array_equal(_np(dev), spaces[1][1])


@pytest.mark.parametrize("d2h", [False, True])
def test_run_across_two_allocations(ops, d2h):
    """Four rows at constant pitches over pageable host memory whose device
    side lies in two separate allocations: the runtime refuses one rectangle
    over them, and the rows still land."""
    gen = torch.Generator().manual_seed(21 + d2h)
    host = _rand_u8(1 << 20, gen, pinned=False)
    size = 64 << 20
    a = torch.randint(0, 256, (size,), dtype=torch.uint8, generator=gen).to(DEV)
    b = torch.randint(0, 256, (size,), dtype=torch.uint8, generator=gen).to(DEV)
    lo, hi = sorted([a, b], key=lambda t: t.data_ptr())
    n, a = 4096, 1000
    h = host.data_ptr()
    gap = hi.data_ptr() - lo.data_ptr()
    pitch = (gap + 1) // 2                 # rows 0-1 in `lo`, rows 2-3 in `hi`
    offs = [a + k * pitch for k in range(4)]
    dev_rows = [lo.data_ptr() + o if o + n <= size else hi.data_ptr() + o - gap for o in offs]
    inside = [lo.data_ptr() <= r and r + n <= lo.data_ptr() + size or
              hi.data_ptr() <= r and r + n <= hi.data_ptr() + size for r in dev_rows]
    if not all(inside) or pitch < n:
        pytest.skip(f"the allocations are {gap} bytes apart: too far for one run over both")
    host_rows = [h + 8192 * k for k in range(4)]
    rows = [(hr, dr, n) if d2h else (dr, hr, n) for dr, hr in zip(dev_rows, host_rows)]
    spaces = _spaces(host, [lo, hi])
    ok.layerwise_dma_copy(spaces, rows)
    ops.layerwise_prefill_dma_copy(rows, d2h)
    torch.cuda.synchronize()
    assert np.array_equal(host.numpy(), spaces[0][1])
    assert np.array_equal(_np(lo), spaces[1][1]) and np.array_equal(_np(hi), spaces[2][1])
    # a later launch does not see the refused rectangle as its error
    x = torch.ones(1 << 20, device=DEV)
    assert float((x * 2).sum()) == 2.0 * (1 << 20)


@pytest.mark.parametrize("d2h", [False, True])
def test_registered_host_memory_and_large_rows(ops, d2h):
    """Host memory from alloc_pinned_ptr (the library's own registry), many
    scattered rows (copied by the kernel) mixed with rows of 5 MiB (copy
    engines)."""
    import ctypes

    size = 24 << 20
    p = ops.alloc_pinned_ptr(size, 0)
    try:
        host = torch.frombuffer((ctypes.c_ubyte * size).from_address(p), dtype=torch.uint8)
        gen = torch.Generator().manual_seed(31 + d2h)
        host.copy_(torch.randint(0, 256, (size,), dtype=torch.uint8, generator=gen))
        dev = torch.randint(0, 256, (size,), dtype=torch.uint8, generator=gen).to(DEV)
        rng = np.random.default_rng(5)
        slots = rng.permutation(size // 32768 - 400)[:100] + 320  # 32 KiB rows past the big ones
        far, near = (p, dev.data_ptr()) if d2h else (dev.data_ptr(), p)
        rows = [(far + int(k) * 32768, near + int(j) * 32768, 32768) for j, k in enumerate(slots)]
        rows += [(far + i * (5 << 20), near + (size - (i + 1) * (5 << 20)), 5 << 20) for i in range(2)]
        spaces = _spaces(host, [dev])
        ok.layerwise_dma_copy(spaces, rows)
        ops.layerwise_prefill_dma_copy(rows, d2h)
        torch.cuda.synchronize()
        assert np.array_equal(host.numpy(), spaces[0][1])
        assert np.array_equal(_np(dev), spaces[1][1])
    finally:
        ops.free_pinned_ptr(p)


def test_overlapping_destinations_keep_order(ops):
    gen = torch.Generator().manual_seed(3)
    host = _rand_u8(1 << 16, gen)
    dev = torch.zeros(1 << 16, dtype=torch.uint8, device=DEV)
    d, h = dev.data_ptr(), host.data_ptr()
    rows = [(d + 0, h + 0, 4096), (d + 2048, h + 8192, 4096), (d + 100, h + 20000, 50), (d + 4096, h + 4096, 4096)]
    spaces = _spaces(host, [dev])
    ok.layerwise_dma_copy(spaces, rows)
    ops.layerwise_prefill_dma_copy(rows, False)
    torch.cuda.synchronize()
    assert np.array_equal(_np(dev), spaces[1][1])


def test_empty_and_null_rows(ops):
    ops.layerwise_prefill_dma_copy([], False)
    dev = torch.zeros(64, dtype=torch.uint8, device=DEV)
    with pytest.raises(RuntimeError, match="null address"):
        ops.layerwise_prefill_dma_copy([(dev.data_ptr(), 0, 16)], False)
    with pytest.raises(TypeError):
        ops.layerwise_prefill_dma_copy([(1, 2)], False)


def test_diagnose_submits_every_row(ops):
    gen = torch.Generator().manual_seed(4)
    host = _rand_u8(1 << 16, gen)
    dev = torch.zeros(1 << 16, dtype=torch.uint8, device=DEV)
    rows = [(dev.data_ptr() + 4096 * i, host.data_ptr() + 4096 * (15 - i), 4096) for i in range(16)]
    ok.layerwise_dma_copy(_spaces(host, [dev]), rows)
    stream_us, stream_addr, copy_us = ops.layerwise_prefill_dma_copy_diagnose(rows, False)
    torch.cuda.synchronize()
    assert len(copy_us) == 16 and all(u >= 0 for u in copy_us) and stream_us >= 0
    assert stream_addr == (torch.cuda.current_stream().cuda_stream or 0)
    want = host.view(16, 4096).flip(0).reshape(-1)
    assert torch.equal(dev.cpu(), want)


def test_runs_on_the_current_stream(ops):
    """The copies are ordered after work already queued on the current
    stream and before work queued after them."""
    gen = torch.Generator().manual_seed(6)
    s = torch.cuda.Stream()
    host = _rand_u8(1 << 22, gen)
    dev = torch.zeros(1 << 22, dtype=torch.uint8, device=DEV)
    with torch.cuda.stream(s):
        dev.fill_(7)
        ops.layerwise_prefill_dma_copy([(dev.data_ptr(), host.data_ptr(), 1 << 21)], False)
        tail = dev[1 << 21:].clone()
        head = dev[: 1 << 21].clone()
    s.synchronize()
    assert torch.equal(head.cpu(), host[: 1 << 21])
    assert bool((tail == 7).all())
