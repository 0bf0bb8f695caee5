"""Pins the oracle's sparse, direct and staged-batch restatements
(oracle/kv_transfer.py) without trusting its byte arithmetic.

Each closed form below is written the way the reference's CPU runtime and
tests state these ops: numpy views of the caches as [-1, width] rows and of
the memory objects as their stacked or interleaved planes, then fancy
indexing (tools/cpu_vllm_runtime.py:288-411; tests/v1/test_mem_kernels.py:
791-1062, 1445-1543).  Invariants tie the ops together (a sparse transfer of
every token in order equals the dense one; store then load restores the
cache), and planted mistakes (swapped index roles, the wrong chunk layout,
ignored counts) must fail the closed forms.
"""

import numpy as np
import pytest

from oracle import kv_transfer as ok

pytestmark = []

ES = 2


def tb(a: np.ndarray) -> ok.TensorBytes:
    a = np.ascontiguousarray(a)
    return ok.TensorBytes(a.view(np.uint8).reshape(-1), a.shape, [s // a.itemsize for s in a.strides], a.itemsize)


def rnd(rng, shape):
    return rng.integers(0, 65535, size=shape, dtype=np.uint16)


def mla_caches(rng, NB=8, BS=4, kH=16, vH=8, dsaH=0):
    c = [rnd(rng, (NB, BS, 1, kH)), rnd(rng, (NB, BS, 1, vH))]
    if dsaH:
        c.append(rnd(rng, (NB, BS, 1, dsaH)))
    return c


# --------------------------------------------------------------------------
# sparse_single_layer_kv_transfer
# --------------------------------------------------------------------------


def test_sparse_single_layer_mla_closed_form():
    rng = np.random.default_rng(0)
    kH, vH, N = 16, 8, 10
    caches = mla_caches(rng, kH=kH, vH=vH)
    want = [c.copy() for c in caches]
    lmc = rnd(rng, N * (kH + vH))
    sel = np.array([3, 0, 9, 12, -1, 5], dtype=np.int32)          # 12 and -1 out of range
    slots = np.array([7, 31, 2, 4, 5, -1], dtype=np.int64)        # -1 skipped
    ok.sparse_single_layer_kv_transfer(tb(lmc), [tb(c) for c in caches], slots, sel, ok.MLA_KV)
    kplane, vplane = lmc[: N * kH].reshape(N, kH), lmc[N * kH:].reshape(N, vH)
    for i in range(len(sel)):
        if 0 <= sel[i] < N and 0 <= slots[i] < 32:
            want[0].reshape(-1, kH)[slots[i]] = kplane[sel[i]]
            want[1].reshape(-1, vH)[slots[i]] = vplane[sel[i]]
    for g, w in zip(caches, want):
        assert np.array_equal(g, w)


@pytest.mark.parametrize("token_major", [False, True])
@pytest.mark.parametrize("two_major", [False, True])
def test_sparse_single_layer_merged_closed_form(token_major, two_major):
    rng = np.random.default_rng(1)
    NB, BS, H, D, N = 6, 4, 2, 4, 9
    W = H * D
    cache = rnd(rng, (2, NB, BS, H, D) if two_major else (NB, 2, BS, H, D))
    want = cache.copy()
    lmc = rnd(rng, (N, 2, W) if token_major else (2, N, W))
    sel = rng.permutation(N)[:5].astype(np.int32)
    slots = rng.permutation(NB * BS)[:5].astype(np.int64)
    ok.sparse_single_layer_kv_transfer(tb(lmc), [tb(cache)], slots, sel, ok.MERGED_KV, token_major, two_major)
    for p in range(2):
        plane = want[p] if two_major else want[:, p]
        rows = plane.reshape(-1, W) if two_major else plane.reshape(NB * BS, W)
        src = lmc[:, p] if token_major else lmc[p]
        rows[slots] = src[sel]
        if not two_major:
            want[:, p] = rows.reshape(NB, BS, H, D)
    assert np.array_equal(cache, want)


def test_sparse_of_every_token_equals_single_layer_retrieve():
    rng = np.random.default_rng(2)
    NB, BS, H, D, T = 6, 4, 2, 4, 11
    k, v = rnd(rng, (NB, BS, H, D)), rnd(rng, (NB, BS, H, D))
    k2, v2 = k.copy(), v.copy()
    lmc = rnd(rng, (2, T, H * D))
    slots = rng.permutation(NB * BS)[:T].astype(np.int64)
    ok.single_layer_kv_transfer(tb(lmc), [tb(k), tb(v)], slots, False, ok.SEPARATE_KV)
    ok.sparse_single_layer_kv_transfer(tb(lmc), [tb(k2), tb(v2)], slots, np.arange(T, dtype=np.int32),
                                       ok.SEPARATE_KV)
    assert np.array_equal(k, k2) and np.array_equal(v, v2)


def test_planted_swapped_index_roles_fail_the_closed_form():
    rng = np.random.default_rng(3)
    kH, vH, N = 16, 8, 12
    caches = mla_caches(rng, kH=kH, vH=vH)
    lmc = rnd(rng, N * (kH + vH))
    sel = np.array([1, 4, 7], dtype=np.int32)
    slots = np.array([9, 2, 11], dtype=np.int64)
    planted = [c.copy() for c in caches]
    ok.sparse_single_layer_kv_transfer(tb(lmc), [tb(c) for c in planted], sel.astype(np.int64),
                                       slots.astype(np.int32), ok.MLA_KV)
    want = [c.copy() for c in caches]
    want[0].reshape(-1, kH)[slots] = lmc[: N * kH].reshape(N, kH)[sel]
    assert not np.array_equal(planted[0], want[0])


# --------------------------------------------------------------------------
# direct (host-chunk) transfers
# --------------------------------------------------------------------------


def chunk_views(raw: np.ndarray, count: int, widths, interleaved: bool):
    """The CPU runtime's plane views of one memory object
    (tools/cpu_vllm_runtime.py:366-373)."""
    out, prefix = [], 0
    for w in widths:
        if interleaved:
            out.append(raw.reshape(count, sum(widths))[:, prefix: prefix + w])
        else:
            out.append(raw[prefix * count: (prefix + w) * count].reshape(count, w))
        prefix += w
    return out


def dense_closed_form(caches, chunks, slots, total, offsets, sizes, fixed, interleaved, direction):
    widths = [c.shape[-1] for c in caches]
    for c, raw in enumerate(chunks):
        start = c * fixed if fixed else int(offsets[c])
        count = min(fixed, total - start) if fixed else int(sizes[c])
        sel = slots[start: start + count]
        valid = sel >= 0
        for cache, cpu in zip(caches, chunk_views(raw, count, widths, interleaved)):
            view = cache.reshape(-1, cache.shape[-1])
            if direction:
                cpu[valid] = view[sel[valid]]
            else:
                view[sel[valid]] = cpu[valid]


@pytest.mark.parametrize("interleaved", [False, True])
@pytest.mark.parametrize("fixed", [0, 4])
@pytest.mark.parametrize("dsa", [0, 8])
def test_dense_direct_closed_form_both_directions(interleaved, fixed, dsa):
    rng = np.random.default_rng(4)
    kH, vH, total = 16, 8, 14
    fmt = ok.DSA_KV if dsa else ok.MLA_KV
    pe = kH + vH + dsa
    sizes = [4, 4, 4, 2] if fixed else [5, 3, 6]
    offsets = np.cumsum([0] + sizes[:-1])
    caches = mla_caches(rng, kH=kH, vH=vH, dsaH=dsa)
    slots = rng.permutation(32)[:total].astype(np.int64)
    slots[[2, 9]] = -1
    # load: chunks -> paged
    chunks = [rnd(rng, n * pe) for n in sizes]
    got, want = [c.copy() for c in caches], [c.copy() for c in caches]
    ok.dense_direct_kv_transfer([c.view(np.uint8) for c in chunks], [tb(c) for c in got], slots, total,
                                offsets, sizes, fixed, fmt, interleaved=interleaved, direction=False)
    dense_closed_form(want, chunks, slots, total, offsets, sizes, fixed, interleaved, False)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)
    # store: paged -> chunks
    got_c = [np.zeros(n * pe, np.uint16) for n in sizes]
    want_c = [np.zeros(n * pe, np.uint16) for n in sizes]
    ok.dense_direct_kv_transfer([c.view(np.uint8) for c in got_c], [tb(c) for c in caches], slots, total,
                                offsets, sizes, fixed, fmt, interleaved=interleaved, direction=True)
    dense_closed_form(caches, want_c, slots, total, offsets, sizes, fixed, interleaved, True)
    for g, w in zip(got_c, want_c):
        assert np.array_equal(g, w)


def test_dense_direct_store_then_load_restores():
    rng = np.random.default_rng(5)
    caches = mla_caches(rng)
    total, fixed = 10, 4
    sizes = [4, 4, 2]
    slots = rng.permutation(32)[:total].astype(np.int64)
    chunks = [np.zeros(n * 24, np.uint16) for n in sizes]
    ok.dense_direct_kv_transfer([c.view(np.uint8) for c in chunks], [tb(c) for c in caches], slots, total,
                                None, None, fixed, ok.MLA_KV, direction=True)
    restored = [np.zeros_like(c) for c in caches]
    ok.dense_direct_kv_transfer([c.view(np.uint8) for c in chunks], [tb(c) for c in restored], slots, total,
                                None, None, fixed, ok.MLA_KV, direction=False)
    for c, r in zip(caches, restored):
        assert np.array_equal(c.reshape(-1, c.shape[-1])[slots], r.reshape(-1, r.shape[-1])[slots])


def test_planted_interleave_flip_fails_dense_closed_form():
    rng = np.random.default_rng(6)
    caches = mla_caches(rng)
    total, fixed = 8, 4
    slots = rng.permutation(32)[:total].astype(np.int64)
    chunks = [rnd(rng, 4 * 24) for _ in range(2)]
    got, want = [c.copy() for c in caches], [c.copy() for c in caches]
    ok.dense_direct_kv_transfer([c.view(np.uint8) for c in chunks], [tb(c) for c in got], slots, total,
                                None, None, fixed, ok.MLA_KV, interleaved=True)
    dense_closed_form(want, chunks, slots, total, None, None, fixed, False, False)
    assert not np.array_equal(got[0], want[0])


def sparse_closed_form(caches, chunks, slots, selected, chunk_size, total, interleaved, counts=None):
    widths = [c.shape[-1] for c in caches]
    dest, tok = slots.reshape(-1).astype(np.int64), selected.reshape(-1).astype(np.int64)
    keep = np.ones(len(tok), bool)
    if counts is not None:
        w = len(tok) // len(counts)
        keep &= (np.arange(len(tok)) % w) < np.repeat(counts, w)
    keep &= (tok >= 0) & (tok < total) & (dest >= 0)
    for d, t in zip(dest[keep], tok[keep]):
        c = t // chunk_size
        n = min(chunk_size, total - c * chunk_size)
        for cache, cpu in zip(caches, chunk_views(chunks[c], n, widths, interleaved)):
            cache.reshape(-1, cache.shape[-1])[d] = cpu[t % chunk_size]


@pytest.mark.parametrize("interleaved", [False, True])
@pytest.mark.parametrize("with_counts", [False, True])
def test_sparse_direct_closed_form(interleaved, with_counts):
    rng = np.random.default_rng(7)
    kH, vH, cs, total = 16, 8, 4, 14
    caches = mla_caches(rng, kH=kH, vH=vH)
    chunks = [rnd(rng, min(cs, total - c * cs) * (kH + vH)) for c in range(4)]
    sel = np.array([[0, 3, 13, 7], [4, 15, 9, 1]], dtype=np.int32)   # 15 >= total: skipped
    slots = np.array([[1, 2, 3, 4], [5, 6, -1, 8]], dtype=np.int64)
    counts = np.array([3, 4], dtype=np.int32) if with_counts else None
    got, want = [c.copy() for c in caches], [c.copy() for c in caches]
    ok.sparse_direct_kv_transfer([c.view(np.uint8) for c in chunks], [tb(c) for c in got], slots, sel, cs, total,
                                 ok.MLA_KV, interleaved=interleaved, counts=counts)
    sparse_closed_form(want, chunks, slots, sel, cs, total, interleaved, counts)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


def test_planted_ignored_counts_fail_the_closed_form():
    rng = np.random.default_rng(8)
    caches = mla_caches(rng)
    chunks = [rnd(rng, 4 * 24) for _ in range(2)]
    sel = np.array([0, 1, 2, 3, 4, 5, 6, 7], dtype=np.int32)
    slots = np.arange(8, dtype=np.int64) + 10
    counts = np.array([2, 1], dtype=np.int32)
    got, want = [c.copy() for c in caches], [c.copy() for c in caches]
    ok.sparse_direct_kv_transfer([c.view(np.uint8) for c in chunks], [tb(c) for c in got], slots, sel, 4, 8,
                                 ok.MLA_KV)
    sparse_closed_form(want, chunks, slots, sel, 4, 8, False, counts)
    assert not np.array_equal(got[0], want[0])


def test_sparse_direct_of_every_token_equals_dense_load():
    rng = np.random.default_rng(9)
    caches = mla_caches(rng, dsaH=8)
    total, cs = 10, 4
    chunks = [rnd(rng, min(cs, total - c * cs) * 32) for c in range(3)]
    slots = rng.permutation(32)[:total].astype(np.int64)
    a, b = [c.copy() for c in caches], [c.copy() for c in caches]
    ok.sparse_direct_kv_transfer([c.view(np.uint8) for c in chunks], [tb(c) for c in a], slots,
                                 np.arange(total, dtype=np.int32), cs, total, ok.DSA_KV)
    ok.dense_direct_kv_transfer([c.view(np.uint8) for c in chunks], [tb(c) for c in b], slots, total, None, None, cs,
                                ok.DSA_KV)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


@pytest.mark.parametrize("token_major", [False, True])
def test_sparse_direct_separate_uses_the_layout_sample(token_major):
    rng = np.random.default_rng(10)
    NB, BS, H, D, cs, total = 6, 4, 2, 4, 4, 8
    W = H * D
    k, v = rnd(rng, (NB, BS, H, D)), rnd(rng, (NB, BS, H, D))
    chunks = [rnd(rng, (cs, 2, W) if token_major else (2, cs, W)) for _ in range(2)]
    sel = np.array([6, 1, 3], dtype=np.int32)
    slots = np.array([20, 2, 13], dtype=np.int64)
    want_k, want_v = k.copy(), v.copy()
    for i in range(3):
        c, t = divmod(int(sel[i]), cs)
        src = chunks[c][t] if token_major else chunks[c][:, t]
        want_k.reshape(-1, W)[slots[i]] = src[0]
        want_v.reshape(-1, W)[slots[i]] = src[1]
    ok.sparse_direct_kv_transfer([c.reshape(-1).view(np.uint8) for c in chunks], [tb(k), tb(v)], slots, sel, cs,
                                 total, ok.SEPARATE_KV, layout=tb(chunks[0]), token_major=token_major)
    assert np.array_equal(k, want_k) and np.array_equal(v, want_v)


# --------------------------------------------------------------------------
# staged batch copies
# --------------------------------------------------------------------------


@pytest.mark.parametrize("token_major", [False, True])
def test_stage_chunks_merged_closed_form(token_major):
    rng = np.random.default_rng(11)
    NB, BS, H, D, T = 6, 4, 2, 4, 9
    W = H * D
    cache = rnd(rng, (NB, 2, BS, H, D))
    staging = rnd(rng, (T, 2, W) if token_major else (2, T, W))
    sizes, offs = [4, 2, 3], [0, 4, 6]
    objs = [np.zeros((n, 2, W) if token_major else (2, n, W), np.uint16) for n in sizes]
    ok.stage_chunks(tb(staging), [tb(cache)], [tb(o) for o in objs], offs, sizes, ok.MERGED_KV, token_major, True)
    for o, off, n in zip(objs, offs, sizes):
        want = staging[off: off + n] if token_major else staging[:, off: off + n]
        assert np.array_equal(o, want)


@pytest.mark.parametrize("token_major", [False, True])
def test_stage_chunks_mla_closed_form(token_major):
    rng = np.random.default_rng(12)
    kH, vH, T = 16, 8, 9
    caches = mla_caches(rng, kH=kH, vH=vH)
    staging = rnd(rng, T * (kH + vH))
    sizes, offs = [5, 4], [0, 5]
    objs = [np.zeros(n * (kH + vH), np.uint16) for n in sizes]
    ok.stage_chunks(tb(staging), [tb(c) for c in caches], [tb(o) for o in objs], offs, sizes, ok.MLA_KV,
                    token_major, True)
    kp, vp = staging[: T * kH].reshape(T, kH), staging[T * kH:].reshape(T, vH)
    for o, off, n in zip(objs, offs, sizes):
        ko, vo = chunk_views(o, n, [kH, vH], token_major)
        assert np.array_equal(ko, kp[off: off + n]) and np.array_equal(vo, vp[off: off + n])
