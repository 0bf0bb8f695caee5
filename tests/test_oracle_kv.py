"""Pins the gather/scatter oracle (oracle/kv_transfer.py) on the CPU.

The oracle restates the reference's byte-offset arithmetic.  These tests
check it against formulations that share none of that arithmetic:
shape-indexed numpy gathers (the textbook definition: row `slot` of the
cache viewed as [-1, W], or [block, offset] of a 4-/5-D cache), per-element
loops on tiny inputs, and the reference's invariants (round trip,
multi_layer == per-layer load_and_reshape_flash).  One test plants a mistake
in the oracle and checks that the closed form catches it.
"""

import json
import os

import numpy as np
import pytest

from oracle import kv_transfer as ok

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _rng(seed):
    return np.random.default_rng(seed)


def _u16(shape, rng):
    return rng.integers(0, 1 << 16, size=shape, dtype=np.uint16)


def _b(a):
    return a.reshape(-1).view(np.uint8)


@pytest.mark.parametrize("fmt,use_mla", [(1, False), (2, False), (1, True), (2, True)])
@pytest.mark.parametrize("direction", [True, False])
def test_multi_layer_planar_closed_form(fmt, use_mla, direction):
    rng = _rng(fmt * 10 + use_mla)
    L, NB, BS, W, T = 3, 7, 4, 24, 11
    pbs = NB * BS
    slots = rng.permutation(pbs)[:T].astype(np.int64)
    if fmt == 1 and not use_mla:
        caches = [_u16((2, NB, BS, W), rng) for _ in range(L)]
        table = [_b(c) for c in caches]
        planes = lambda l: [caches[l][0].reshape(-1, W), caches[l][1].reshape(-1, W)]
    elif use_mla:
        caches = [_u16((NB, BS, W), rng) for _ in range(L)]
        table = [_b(c) for c in caches]
        planes = lambda l: [caches[l].reshape(-1, W)]
    else:
        caches = [(_u16((NB, BS, W), rng), _u16((NB, BS, W), rng)) for _ in range(L)]
        table = [_b(x) for kv in caches for x in kv]
        planes = lambda l: [caches[l][0].reshape(-1, W), caches[l][1].reshape(-1, W)]
    P = 1 if use_mla else 2
    lmc = _u16((P, L, T, W), rng)
    lmc0 = lmc.copy()
    expected_lmc = lmc0.copy()
    expected_paged = [[p.copy() for p in planes(l)] for l in range(L)]
    for l in range(L):
        for p in range(P):
            if direction:
                expected_lmc[p, l] = planes(l)[p][slots]
            else:
                expected_paged[l][p][slots] = lmc0[p, l]
    ok.multi_layer_kv_transfer(_b(lmc), table, slots, pbs, direction, use_mla, fmt, L, W, 2)
    if direction:
        assert np.array_equal(lmc, expected_lmc)
    else:
        for l in range(L):
            for p in range(P):
                assert np.array_equal(planes(l)[p], expected_paged[l][p])


@pytest.mark.parametrize("fmt", [3, 4, 5, 6])
def test_multi_layer_concatenated_closed_form(fmt):
    rng = _rng(fmt)
    L, NB, BS, T = 2, 5, 4, 9
    kH, vH, dsaH = 16, 8, 12
    pbs = NB * BS
    slots = rng.permutation(pbs)[:T].astype(np.int64)
    widths = {3: [kH, vH], 5: [kH, vH], 4: [kH, vH, dsaH], 6: [dsaH]}[fmt]
    caches = [[_u16((NB, BS, 1, w), rng) for w in widths] for _ in range(L)]
    table = [_b(x) for layer in caches for x in layer]
    wsum = sum(widths)
    lmc = np.zeros((1, L, T, wsum), np.uint16)
    ok.multi_layer_kv_transfer(_b(lmc), table, slots, pbs, True, False, fmt, L, wsum, 2, kH, vH, dsaH)
    for l in range(L):
        row = np.concatenate([caches[l][p].reshape(-1, w)[slots] for p, w in enumerate(widths)], axis=1)
        assert np.array_equal(lmc[0, l], row)
    # retrieve into zeroed caches reproduces exactly the mapped rows
    zero = [[np.zeros_like(x) for x in layer] for layer in caches]
    ztable = [_b(x) for layer in zero for x in layer]
    ok.multi_layer_kv_transfer(_b(lmc), ztable, slots, pbs, False, False, fmt, L, wsum, 2, kH, vH, dsaH)
    for l in range(L):
        for p, w in enumerate(widths):
            got = zero[l][p].reshape(-1, w)
            want = np.zeros_like(got)
            want[slots] = caches[l][p].reshape(-1, w)[slots]
            assert np.array_equal(got, want)


def test_multi_layer_skips_out_of_range_slots():
    rng = _rng(7)
    L, NB, BS, W, T = 2, 4, 4, 8, 10
    pbs = NB * BS
    slots = rng.permutation(pbs)[:T].astype(np.int64)
    slots[[1, 4, 7]] = -1
    slots[8] = pbs + 3
    caches = [(_u16((NB, BS, W), rng), _u16((NB, BS, W), rng)) for _ in range(L)]
    table = [_b(x) for kv in caches for x in kv]
    guard = 0xA5A5
    lmc = np.full((2, L, T, W), guard, np.uint16)
    ok.multi_layer_kv_transfer(_b(lmc), table, slots, pbs, True, False, 2, L, W, 2)
    for t in (1, 4, 7, 8):
        assert (lmc[:, :, t] == guard).all()
    before = [np.array(x, copy=True) for kv in caches for x in kv]
    ok.multi_layer_kv_transfer(_b(lmc), table, slots, pbs, False, False, 2, L, W, 2)
    # retrieve of the just-stored rows is the identity on valid slots, and the
    # skipped tokens' guard rows went nowhere
    after = [x for kv in caches for x in kv]
    for b, a in zip(before, after):
        assert np.array_equal(b, a)


def test_multi_layer_equals_per_layer_flash():
    # tests/v1/test_mem_kernels.py:124-127 cross-checks multi_layer against
    # layer-by-layer load_and_reshape_flash on the MERGED layout.
    rng = _rng(11)
    L, NB, BS, W, T = 3, 6, 4, 16, 13
    pbs = NB * BS
    slots = rng.permutation(pbs)[:T].astype(np.int64)
    caches = [_u16((2, NB, BS, W), rng) for _ in range(L)]
    a = np.zeros((2, L, T, W), np.uint16)
    ok.multi_layer_kv_transfer(_b(a), [_b(c) for c in caches], slots, pbs, True, False, 1, L, W, 2)
    b = np.zeros((2, L, T, W), np.uint16)
    for l in range(L):
        ok.load_and_reshape_flash(_b(b), L, W, 2, _b(caches[l][0]), _b(caches[l][1]), slots, l)
    assert np.array_equal(a, b)
    # and reshape_and_cache_back_flash inverts it
    z = [np.zeros_like(c) for c in caches]
    for l in range(L):
        ok.load_and_reshape_flash(_b(b), L, W, 2, _b(z[l][0]), _b(z[l][1]), slots, l, page2lmc=False)
    for l in range(L):
        for p in range(2):
            want = np.zeros((pbs, W), np.uint16)
            want[slots] = caches[l][p].reshape(-1, W)[slots]
            assert np.array_equal(z[l][p].reshape(-1, W), want)


def _tb(a, es=2):
    strides = [s // a.itemsize for s in a.strides]
    return ok.TensorBytes(_b(a), a.shape, strides, es)


@pytest.mark.parametrize("token_major", [True, False])
@pytest.mark.parametrize("two_major", [True, False])
def test_single_layer_merged_brute_force(token_major, two_major):
    rng = _rng(3 + token_major * 2 + two_major)
    NB, BS, H, D, T = 5, 4, 2, 3, 7
    W = H * D
    shape = (2, NB, BS, H, D) if two_major else (NB, 2, BS, H, D)
    cache = _u16(shape, rng)
    slots = rng.permutation(NB * BS)[:T].astype(np.int64)
    lmc = np.zeros((T, 2, W) if token_major else (2, T, W), np.uint16)
    ok.single_layer_kv_transfer(_tb(lmc), [_tb(cache)], slots, True, 1, token_major, two_major)
    for t in range(T):
        blk, off = divmod(int(slots[t]), BS)
        for kv in range(2):
            src = cache[kv, blk, off] if two_major else cache[blk, kv, off]
            dst = lmc[t, kv] if token_major else lmc[kv, t]
            for h in range(H):
                for d in range(D):
                    assert dst[h * D + d] == src[h, d]
    # retrieve into a zeroed cache writes exactly these rows
    zc = np.zeros_like(cache)
    ok.single_layer_kv_transfer(_tb(lmc), [_tb(zc)], slots, False, 1, token_major, two_major)
    mask = np.zeros_like(cache, dtype=bool)
    for t in range(T):
        blk, off = divmod(int(slots[t]), BS)
        for kv in range(2):
            if two_major:
                mask[kv, blk, off] = True
            else:
                mask[blk, kv, off] = True
    assert np.array_equal(zc[mask], cache[mask])
    assert (zc[~mask] == 0).all()


@pytest.mark.parametrize("token_major", [True, False])
def test_single_layer_separate_strided_blocks(token_major):
    # K and V are block-strided views (every other block of a larger tensor):
    # only stride(0) differs from BS*H*D, as csrc/utils.cpp:266-272 reads it.
    rng = _rng(21 + token_major)
    NB, BS, H, D, T = 6, 4, 2, 4, 9
    W = H * D
    big_k = _u16((2 * NB, BS, H, D), rng)
    big_v = _u16((2 * NB, BS, H, D), rng)
    k, v = big_k[::2], big_v[::2]
    slots = rng.permutation(NB * BS)[:T].astype(np.int64)
    lmc = np.zeros((T, 2, W) if token_major else (2, T, W), np.uint16)
    kb = ok.TensorBytes(_b(big_k), k.shape, [s // 2 for s in k.strides], 2)
    vb = ok.TensorBytes(_b(big_v), v.shape, [s // 2 for s in v.strides], 2)
    ok.single_layer_kv_transfer(_tb(lmc), [kb, vb], slots, True, 2, token_major, False)
    for t in range(T):
        blk, off = divmod(int(slots[t]), BS)
        want_k = k[blk, off].reshape(-1)
        want_v = v[blk, off].reshape(-1)
        got_k = lmc[t, 0] if token_major else lmc[0, t]
        got_v = lmc[t, 1] if token_major else lmc[1, t]
        assert np.array_equal(got_k, want_k) and np.array_equal(got_v, want_v)


@pytest.mark.parametrize("fmt", [3, 4, 6])
def test_single_layer_mla_dsa_stacked_planes(fmt):
    rng = _rng(40 + fmt)
    NB, BS, T, N = 4, 4, 6, 8  # the LMC buffer holds N >= T tokens
    kH, vH, dsaH = 8, 4, 6
    k = _u16((NB, BS, 1, kH), rng)
    v = _u16((NB, BS, 1, vH), rng)
    dsa = _u16((NB, BS, 1, dsaH), rng)
    caches = {3: [k, v], 4: [k, v, dsa], 6: [dsa]}[fmt]
    widths = {3: [kH, vH], 4: [kH, vH, dsaH], 6: [dsaH]}[fmt]
    slots = rng.permutation(NB * BS)[:T].astype(np.int64)
    lmc = np.zeros(N * sum(widths), np.uint16)
    ok.single_layer_kv_transfer(_tb(lmc), [_tb(c) for c in caches], slots, True, fmt)
    off = 0
    for c, w in zip(caches, widths):
        plane = lmc[off: off + N * w].reshape(N, w)
        assert np.array_equal(plane[:T], c.reshape(-1, w)[slots])
        assert (plane[T:] == 0).all()
        off += N * w


def test_planted_plane_swap_is_caught(monkeypatch):
    """A plausible oracle mistake (K and V planes swapped in the pointer
    table) must fail the closed-form check above."""
    real = ok.multi_layer_planes

    def swapped(*a, **k):
        planes, ppl, concat = real(*a, **k)
        if len(planes) == 2:
            planes[0].ptr_index, planes[1].ptr_index = planes[1].ptr_index, planes[0].ptr_index
        return planes, ppl, concat

    monkeypatch.setattr(ok, "multi_layer_planes", swapped)
    with pytest.raises(AssertionError):
        test_multi_layer_planar_closed_form(2, False, True)


def test_planted_merged_offset_is_caught(monkeypatch):
    """A MERGED V plane placed one row too early must fail the closed form."""
    real = ok.multi_layer_planes

    def shifted(fmt, use_mla, last_dim, kH, vH, dsaH, pbs, es):
        planes, ppl, concat = real(fmt, use_mla, last_dim, kH, vH, dsaH, pbs, es)
        if fmt == 1 and len(planes) == 2:
            planes[1].paged_off -= last_dim * es
        return planes, ppl, concat

    monkeypatch.setattr(ok, "multi_layer_planes", shifted)
    with pytest.raises(AssertionError):
        test_multi_layer_planar_closed_form(1, False, True)


def test_fused_required_size():
    # csrc/mem_kernels.cpp:143-165
    assert ok.fused_required_size(1, False, 4, 256, 1024, 0, 0, 0, 2) == 2 * 4 * 256 * 1024 * 2
    assert ok.fused_required_size(3, False, 4, 10, 0, 512, 64, 0, 2) == 4 * 10 * 576 * 2
    assert ok.fused_required_size(4, False, 4, 10, 0, 512, 64, 128, 2) == 4 * 10 * 704 * 2
    assert ok.fused_required_size(6, False, 4, 10, 0, 0, 0, 128, 2) == 4 * 10 * 128 * 2


def test_c1_golden_digest():
    """The C1 plumbing case (4 layers, SEPARATE_KV, 256 tokens) reproduces the
    committed digests."""
    from tests.golden import gen_kv_golden as g

    with open(os.path.join(GOLDEN, "kv_c1.json")) as f:
        want = json.load(f)
    got = g.c1_digests()
    assert got == want
