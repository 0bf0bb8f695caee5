"""Pins the oracle's sparse-graph and indexer C8 restatements
(oracle/kv_transfer.py) with the closed forms the reference's own tests use
(tests/standalone/test_indexer_c8_native.py: packet = keys[slots] bytes ||
scales[slots] bytes, the factor-2 physical mapping, the block permutation;
tests/v1/test_sparse_graph_transfer.py: per-row selected tokens from chunk
sources), written here with numpy indexing, and planted mistakes that must
fail them."""

import numpy as np
import pytest

from oracle import kv_transfer as ok


def c8_layer(blocks, quantized=True, factor=1, block_map=None, seed=0):
    rng = np.random.default_rng(seed)
    kb = 128 if quantized else 256
    keys = rng.integers(0, 256, size=blocks * 128 * kb, dtype=np.uint8)
    scales = rng.integers(0, 256, size=blocks * 128 * 2, dtype=np.uint8) if quantized else None
    return ok.C8Layer(keys, scales, kb, factor, block_map, blocks * 128 // factor)


@pytest.mark.parametrize("fixed", [False, True])
@pytest.mark.parametrize("strided", [False, True])
def test_c8_packets_closed_form_and_round_trip(fixed, strided):
    counts = [256, 256, 7] if fixed else [1, 7, 127, 128, 129, 40]
    tokens = sum(counts)
    slots = np.arange(tokens, dtype=np.int64) * (2 if strided else 1)
    blocks = (int(slots[-1]) + 128) // 128
    L = c8_layer(blocks)
    keys0, scales0 = L.keys.copy(), L.scales.copy()
    packets = [np.full(130 * n, 173, np.uint8) for n in counts]
    offs = np.concatenate([[0], np.cumsum(counts)[:-1]])
    ok.indexer_c8_transfer([L], [packets], offs, counts, slots, 256 if fixed else 1024, True, fixed)
    o = 0
    for n, p in zip(counts, packets):
        sel = slots[o:o + n]
        want = np.concatenate([keys0.reshape(-1, 128)[sel].reshape(-1), scales0.reshape(-1, 2)[sel].reshape(-1)])
        assert np.array_equal(p, want)
        o += n
    L.keys[:] = 42
    L.scales[:] = 0xFF
    ok.indexer_c8_transfer([L], [packets], offs, counts, slots, 256 if fixed else 1024, False, fixed)
    assert np.array_equal(L.keys.reshape(-1, 128)[slots], keys0.reshape(-1, 128)[slots])
    assert np.array_equal(L.scales.reshape(-1, 2)[slots], scales0.reshape(-1, 2)[slots])
    untouched = np.ones(blocks * 128, bool)
    untouched[slots] = False
    assert (L.keys.reshape(-1, 128)[untouched] == 42).all()


@pytest.mark.parametrize("factor", [1, 2])
def test_c8_physical_mapping_closed_form(factor):
    tokens = 259
    L = c8_layer(4 * factor, factor=factor)
    keys0 = L.keys.copy()
    packet = np.zeros(tokens * 130, np.uint8)
    slots = np.arange(tokens, dtype=np.int64)
    ok.indexer_c8_transfer([L], [[packet]], [0], [tokens], slots, tokens, True, False)
    physical = np.arange(tokens) + (np.arange(tokens) // 128) * (factor - 1) * 128
    assert np.array_equal(packet[: tokens * 128].reshape(tokens, 128), keys0.reshape(-1, 128)[physical])


def test_c8_block_map_closed_form_and_planted_factor():
    t = 3
    mapping = np.empty(18 * t, np.int32)
    for u in range(t):
        ids = [*range(8 * u, 8 * u + 8), *range(8 * (t + u), 8 * (t + u) + 8), 16 * t + u, 17 * t + u]
        mapping[ids] = [*range(16 * u, 16 * u + 16), 16 * t + 2 * u, 16 * t + 2 * u + 1]
    L = c8_layer(18 * t, block_map=mapping)
    host_slots = np.concatenate([np.arange(b * 128 + 126, b * 128 + 129) for b in (23, 47, 50)])
    physical = mapping[host_slots // 128].astype(np.int64) * 128 + host_slots % 128
    n = len(host_slots)
    packet = np.zeros(n * 130, np.uint8)
    ok.indexer_c8_transfer([L], [[packet]], [0], [n], host_slots, n, True, False)
    want = np.concatenate([L.keys.reshape(-1, 128)[physical].reshape(-1), L.scales.reshape(-1, 2)[physical].reshape(-1)])
    assert np.array_equal(packet, want)
    # planted: ignoring the block map reads the logical slots
    planted = np.zeros_like(packet)
    L2 = ok.C8Layer(L.keys, L.scales, 128, 1, None, L.cache_slots)
    ok.indexer_c8_transfer([L2], [[planted]], [0], [n], host_slots, n, True, False)
    assert not np.array_equal(planted, want)


def test_c8_skips_bad_chunks_and_slots():
    L = c8_layer(2)
    keys0 = L.keys.copy()
    slots = np.array([0, -1, 300, 5, 7, 9], dtype=np.int64)   # -1 and 300 >= 256 skipped
    p0 = np.full(4 * 130, 9, np.uint8)
    p1 = np.full(2 * 130, 9, np.uint8)
    ok.indexer_c8_transfer([L], [[p0, None, p1]], [0, 4, 4], [4, 2, 9], slots, 4, True, False)
    assert np.array_equal(p0[:128], keys0[:128])
    assert (p0[128:256] == 9).all() and (p0[256:384] == 9).all()
    assert (p1 == 9).all()                                   # count 9 > capacity 4: skipped


def graph_closed_form(k_rows, pe_rows, kb, pb, slots, sel, counts, limits, ks, ps, cs):
    R, W = sel.shape
    cpr = len(ks) // R
    dest = min(k_rows.size // kb, pe_rows.size // pb)
    active = np.where((limits <= 0) | (counts <= 0), 0, np.minimum(counts, W))
    cols = np.arange(W)[None, :] < active[:, None]
    ok_tok = (sel >= 0) & (sel < limits[:, None]) & (slots >= 0) & (slots < dest) & cols
    chunk = np.where(ok_tok, sel // cs, 0)
    ok_tok &= chunk < cpr
    for r, j in zip(*np.nonzero(ok_tok)):
        i = r * cpr + chunk[r, j]
        if ks[i] is None or ps[i] is None:
            continue
        k = ks[i].reshape(-1, kb)[sel[r, j] % cs]
        p = ps[i].reshape(-1, pb)[sel[r, j] % cs]
        k_rows.reshape(-1, kb)[slots[r, j]] = k
        pe_rows.reshape(-1, pb)[slots[r, j]] = p


def test_sparse_graph_closed_form_and_planted_swap():
    rng = np.random.default_rng(3)
    R, W, cs, cpr, kb, pb = 3, 12, 8, 3, 64, 32
    ks = [rng.integers(0, 256, cs * kb, dtype=np.uint8) for _ in range(R * cpr)]
    ps = [rng.integers(0, 256, cs * pb, dtype=np.uint8) for _ in range(R * cpr)]
    ks[4] = None
    sel = rng.integers(-2, cs * cpr + 3, size=(R, W))
    slots = rng.permutation(64)[: R * W].reshape(R, W)
    slots[0, 2] = -1
    counts = np.array([5, 20, 0])
    limits = np.array([20, 24, 9])
    got_k, got_p = np.zeros(64 * kb, np.uint8), np.zeros(64 * pb, np.uint8)
    want_k, want_p = got_k.copy(), got_p.copy()
    ok.sparse_graph_kv_transfer(got_k, got_p, kb, pb, slots, sel, counts, limits, ks, ps, cs)
    graph_closed_form(want_k, want_p, kb, pb, slots, sel, counts, limits, ks, ps, cs)
    assert np.array_equal(got_k, want_k) and np.array_equal(got_p, want_p)
    assert got_k.any()
    bad_k = np.zeros_like(got_k)
    ok.sparse_graph_kv_transfer(bad_k, np.zeros_like(got_p), kb, pb, slots, sel, counts, limits,
                                ks[1:] + ks[:1], ps, cs)
    assert not np.array_equal(bad_k, want_k)
