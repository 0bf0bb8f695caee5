"""Pins the oracle's layerwise prefill DMA restatement
(oracle/kv_transfer.py: layerwise_dma_copy, layerwise_dma_rows) with the
reference's own planner case (tests/standalone/test_layerwise_prefill_dma.py:
31-51: block ids 10..13 of 4 tokens give slots 40, 44, 48, 52), a numpy
gather/scatter closed form over several planes, and planted mistakes."""

import numpy as np
import pytest

from oracle import kv_transfer as ok


def test_reference_planner_case():
    rows = ok.layerwise_dma_rows([100, 200, 300, 400], [4, 4, 4, 4], [1000], [2 * 2], [10, 11, 12, 13], 4,
                                 [0, 4, 8, 12], [4, 8, 12, 16], False)
    assert len(rows) == 4
    assert [(r[0] - 1000) // 4 for r in rows] == [40, 44, 48, 52]
    assert [r[1] for r in rows] == [100, 200, 300, 400]
    assert sum(r[2] for r in rows) == 16 * 4
    d2h = ok.layerwise_dma_rows([100, 200, 300, 400], [4, 4, 4, 4], [1000], [4], [10, 11, 12, 13], 4,
                                [0, 4, 8, 12], [4, 8, 12, 16], True)
    assert d2h == [(s, d, n) for d, s, n in rows]


def test_empty_range_has_no_rows():
    assert ok.layerwise_dma_rows([], [], [1000], [4], [], 4, [], [], False) == []


def _layout(seed, consecutive, chunk=48, n_chunks=3, bs=16, widths=(64, 64, 32)):
    rng = np.random.default_rng(seed)
    T = chunk * n_chunks
    nb = T // bs
    NB = 4 * nb
    blocks = np.arange(3, 3 + nb) if consecutive else rng.permutation(NB)[:nb]
    pb = [w * 2 for w in widths]
    host = rng.integers(0, 256, T * sum(pb), dtype=np.uint8)
    caches = [np.zeros(NB * bs * b, np.uint8) for b in pb]
    host_base, cache_bases = 1 << 40, [(2 + i) << 40 for i in range(len(pb))]
    starts = [c * chunk for c in range(n_chunks)]
    ends = [(c + 1) * chunk for c in range(n_chunks)]
    chunk_addrs = [host_base + c * chunk * sum(pb) for c in range(n_chunks)]
    return dict(blocks=blocks, pb=pb, host=host, caches=caches, host_base=host_base, cache_bases=cache_bases,
                starts=starts, ends=ends, chunk_addrs=chunk_addrs, chunk=chunk, bs=bs, T=T)


@pytest.mark.parametrize("consecutive", [True, False])
def test_rows_scatter_closed_form(consecutive):
    L = _layout(5, consecutive)
    rows = ok.layerwise_dma_rows(L["chunk_addrs"], [L["chunk"]] * 3, L["cache_bases"], L["pb"], L["blocks"],
                                 L["bs"], L["starts"], L["ends"], False)
    spaces = [(L["host_base"], L["host"])] + list(zip(L["cache_bases"], L["caches"]))
    ok.layerwise_dma_copy(spaces, rows)
    t = np.arange(L["T"])
    slot = L["blocks"][t // L["bs"]] * L["bs"] + t % L["bs"]
    chunks = L["host"].reshape(3, -1)
    off = 0
    for p, b in enumerate(L["pb"]):
        # chunk layout [plane][token][bytes]
        src = chunks[:, L["chunk"] * off:L["chunk"] * (off + b)].reshape(3, L["chunk"], b).reshape(-1, b)
        assert np.array_equal(L["caches"][p].reshape(-1, b)[slot], src)
        off += b
    if consecutive:
        assert len(rows) == 3 * len(L["pb"])      # one range per chunk
    else:
        assert len(rows) > 3 * len(L["pb"])
    # the store direction reproduces the host bytes
    back = np.zeros_like(L["host"])
    rows_out = ok.layerwise_dma_rows(L["chunk_addrs"], [L["chunk"]] * 3, L["cache_bases"], L["pb"], L["blocks"],
                                     L["bs"], L["starts"], L["ends"], True)
    ok.layerwise_dma_copy([(L["host_base"], back)] + list(zip(L["cache_bases"], L["caches"])), rows_out)
    assert np.array_equal(back, L["host"])


def test_later_row_wins_and_planted_order():
    src = np.arange(64, dtype=np.uint8)
    dst = np.zeros(32, np.uint8)
    rows = [(1000, 0, 16), (1008, 32, 16), (1000, 48, 4)]
    spaces = [(0, src), (1000, dst)]
    ok.layerwise_dma_copy(spaces, rows)
    want = np.zeros(32, np.uint8)
    want[0:16] = src[0:16]
    want[8:24] = src[32:48]
    want[0:4] = src[48:52]
    assert np.array_equal(dst, want)
    rev = np.zeros(32, np.uint8)
    ok.layerwise_dma_copy([(0, src), (1000, rev)], rows[::-1])
    assert not np.array_equal(rev, want)


def test_out_of_range_address_is_refused():
    with pytest.raises(ValueError):
        ok.layerwise_dma_copy([(0, np.zeros(8, np.uint8))], [(4, 0, 8)])
