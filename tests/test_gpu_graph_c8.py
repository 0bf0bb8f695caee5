"""GPU parity of the sparse-graph copy (sfa_copy) and the indexer C8 packet
transport, through the C ABI.

Every indexer case derives its expected bytes from the CPU oracle
(oracle/kv_transfer.py: indexer_c8_transfer), on random cache contents:
offset and fixed chunks with int32/int64 metadata, guard bytes around every
packet, int8 keys with float16 scales at slot factor 1 and 2 and bf16 keys,
groups of mixed key widths with unaligned packet starts, pinned host
packets, two streams unpacking disjoint slots, and int32 block maps.  The
chunk sizes, the guard value 173, the slot factors and the block-end slots
are the data the reference's qualification tests use
(tests/standalone/test_indexer_c8_native.py).  Random cases with skipped
chunks, slots and sources are compared bit for bit with the oracle too.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from kvutil import to_bytes
from oracle import kv_transfer as ok

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def c_ops():
    import lmcache_amd

    return lmcache_amd.c_ops


# ---------------------------------------------------------------------------
# indexer C8: packets, groups, pinned packets, streams and block maps, each
# checked byte for byte against oracle.indexer_c8_transfer
# ---------------------------------------------------------------------------

GUARD, PAD = 173, 32


def _c8_cache(rng, blocks, kind, slot_factor=1):
    """Random cache contents for one layer on the CPU: int8 keys with
    float16 scales ([blocks * slot_factor, 128, 1, 128/1]) or bf16 keys."""
    if kind == "int8":
        nb = blocks * slot_factor
        keys = torch.from_numpy(rng.integers(-128, 128, size=(nb, 128, 1, 128), dtype=np.int8))
        scales = torch.from_numpy(rng.integers(0, 0x7BFF, size=(nb, 128, 1, 1), dtype=np.uint16).view(np.float16))
        return keys, scales
    keys = torch.from_numpy(rng.integers(0, 1 << 16, size=(blocks, 128, 1, 128), dtype=np.uint16).view(np.int16))
    return keys.view(torch.bfloat16), None


def _oracle_layer(keys, scales, slot_factor=1, block_map=None):
    return ok.C8Layer(to_bytes(keys), to_bytes(scales) if scales is not None else None, 128 * keys.element_size(),
                      slot_factor, None if block_map is None else block_map.numpy().astype(np.int64),
                      keys.numel() // 128 // slot_factor)


def _packet_bytes(layer: ok.C8Layer, n: int) -> int:
    return n * (layer.key_bytes + (2 if layer.scales is not None else 0))


class _Packets:
    """Packets of one layer, each inside PAD guard bytes of its own device
    (or pinned host) buffer."""

    def __init__(self, sizes, host=False):
        self.sizes = sizes
        self.bufs = []
        for n in sizes:
            if host:
                b = torch.full((n + 2 * PAD,), GUARD, dtype=torch.uint8).pin_memory()
            else:
                b = torch.full((n + 2 * PAD,), GUARD, dtype=torch.uint8, device=DEV)
            self.bufs.append(b)

    def pointers(self, c_ops, host=False):
        out = []
        for b, n in zip(self.bufs, self.sizes):
            out.append(c_ops.get_device_ptr(b.data_ptr() + PAD, max(n, 1)) if host else b.data_ptr() + PAD)
        return out

    def inner(self):
        return [b.cpu().numpy()[PAD: PAD + n].copy() for b, n in zip(self.bufs, self.sizes)]

    def guards_intact(self):
        return all((b.cpu().numpy()[:PAD] == GUARD).all() and (b.cpu().numpy()[PAD + n:] == GUARD).all()
                   for b, n in zip(self.bufs, self.sizes))

    def fill(self, arrays):
        for b, a in zip(self.bufs, arrays):
            b[PAD: PAD + a.size].copy_(torch.from_numpy(a))


def _chunks(counts, fixed, capacity):
    if fixed:
        return [c * capacity for c in range(len(counts))], counts
    return list(np.cumsum([0] + counts[:-1])), counts


@pytest.mark.parametrize("kind,slot_factor", [("int8", 1), ("int8", 2), ("bf16", 1)])
@pytest.mark.parametrize("fixed", [False, True])
@pytest.mark.parametrize("metadata_dtype", [torch.int32, torch.int64])
def test_c8_pack_unpack_vs_oracle(c_ops, kind, slot_factor, fixed, metadata_dtype):
    """Chunked packets (offset chunks of 1..1024 tokens, or fixed 1024-token
    chunks with a short last one), guard bytes around every packet, then an
    unpack into a cleared cache: every byte of packets and cache equals the
    oracle's."""
    rng = np.random.default_rng(17 + slot_factor * 3 + fixed * 5 + (metadata_dtype == torch.int64))
    capacity = 1024
    counts = [1024, 1024, 7] if fixed else [1, 7, 127, 128, 129, 754, 1024]
    tokens = sum(counts)
    blocks = (tokens + 255) // 128
    keys, scales = _c8_cache(rng, blocks, kind, slot_factor)
    slots = rng.permutation(blocks * 128)[:tokens].astype(np.int64)
    layer = _oracle_layer(keys, scales, slot_factor)
    starts, lens = _chunks(counts, fixed, capacity)
    pk = _Packets([_packet_bytes(layer, n) for n in counts])
    state = c_ops.IndexerC8State(keys.to(DEV), scales.to(DEV) if scales is not None else None, slot_factor)
    meta_starts = torch.tensor(starts, dtype=metadata_dtype, device=DEV)
    meta_lens = torch.tensor(lens, dtype=metadata_dtype, device=DEV)
    ptrs = torch.tensor(pk.pointers(c_ops), dtype=torch.int64, device=DEV)
    slot_t = torch.from_numpy(slots).to(device=DEV, dtype=metadata_dtype)
    c_ops.indexer_c8_transfer_prepared(state, ptrs, meta_starts, meta_lens, slot_t, capacity, True,
                                       fixed_chunks=fixed)
    want = [np.full(n, GUARD, np.uint8) for n in pk.sizes]
    ok.indexer_c8_transfer([layer], [want], starts, lens, slots, capacity, True, fixed)
    torch.cuda.synchronize()
    for got, w in zip(pk.inner(), want):
        assert np.array_equal(got, w)
    assert pk.guards_intact()
    # unpack into a cleared cache
    state.keys.fill_(42)
    if state.scales is not None:
        state.scales.view(torch.int16).fill_(-1)
    cleared = _oracle_layer(state.keys.cpu(), state.scales.cpu() if state.scales is not None else None, slot_factor)
    c_ops.indexer_c8_transfer_prepared(state, ptrs, meta_starts, meta_lens, slot_t, capacity, False,
                                       fixed_chunks=fixed)
    ok.indexer_c8_transfer([cleared], [want], starts, lens, slots, capacity, False, fixed)
    torch.cuda.synchronize()
    assert np.array_equal(to_bytes(state.keys), cleared.keys)
    if state.scales is not None:
        assert np.array_equal(to_bytes(state.scales), cleared.scales)


@pytest.mark.parametrize("kinds", [["int8"], ["bf16", "int8", "int8"], ["int8", "bf16"]])
@pytest.mark.parametrize("slot_factor", [1, 2])
def test_c8_group_vs_oracle(c_ops, kinds, slot_factor):
    """One launch over several layers of different key widths.  Each layer's
    packets sit back to back in one buffer, so every layer after the first
    starts at an address that is not 16-byte aligned."""
    rng = np.random.default_rng(len(kinds) * 10 + slot_factor)
    blocks, capacity = 6, 300
    counts = [300, 41, 259]
    starts = [0, 300, 341]
    tokens = sum(counts)
    slots = rng.permutation(blocks * 128)[:tokens].astype(np.int64)
    caches, layers = [], []
    for kd in kinds:
        sf = slot_factor if kd == "int8" else 1
        k, s = _c8_cache(rng, blocks, kd, sf)
        caches.append((k.to(DEV), s.to(DEV) if s is not None else None, sf))
        layers.append(_oracle_layer(k, s, sf))
    state = c_ops.IndexerC8GroupState([c_ops.IndexerC8State(k, s, sf) for k, s, sf in caches])
    sizes = [[_packet_bytes(L, n) for n in counts] for L in layers]
    total = sum(sum(x) for x in sizes)
    buf = torch.full((total + 2 * PAD,), GUARD, dtype=torch.uint8, device=DEV)
    ptr_rows, pos = [], PAD
    for row in sizes:
        ptr_rows.append([])
        for n in row:
            ptr_rows[-1].append(buf.data_ptr() + pos)
            pos += n
    ptrs = torch.tensor(ptr_rows, dtype=torch.int64, device=DEV)
    offs = torch.tensor(starts, dtype=torch.int32, device=DEV)
    cnts = torch.tensor(counts, dtype=torch.int32, device=DEV)
    slot_t = torch.from_numpy(slots).to(DEV)
    c_ops.indexer_c8_group_transfer_prepared(state, ptrs, offs, cnts, slot_t, capacity, True)
    want = [[np.full(n, GUARD, np.uint8) for n in row] for row in sizes]
    ok.indexer_c8_transfer(layers, want, starts, counts, slots, capacity, True, False)
    torch.cuda.synchronize()
    got = buf.cpu().numpy()
    assert np.array_equal(got[PAD: PAD + total], np.concatenate([w for row in want for w in row]))
    assert (got[:PAD] == GUARD).all() and (got[PAD + total:] == GUARD).all()
    # unpack every layer into cleared caches
    for k, s, _ in caches:
        k.view(torch.uint8).fill_(9)
        if s is not None:
            s.view(torch.uint8).fill_(9)
    cleared = [_oracle_layer(k.cpu(), s.cpu() if s is not None else None, sf) for k, s, sf in caches]
    c_ops.indexer_c8_group_transfer_prepared(state, ptrs, offs, cnts, slot_t, capacity, False)
    ok.indexer_c8_transfer(cleared, want, starts, counts, slots, capacity, False, False)
    torch.cuda.synchronize()
    for (k, s, _), L in zip(caches, cleared):
        assert np.array_equal(to_bytes(k), L.keys)
        if s is not None:
            assert np.array_equal(to_bytes(s), L.scales)


@pytest.mark.parametrize("tokens", [1, 7, 129])
def test_c8_pinned_host_packet_vs_oracle(c_ops, tokens):
    """A packet in pinned host memory (alloc_pinned_ptr), addressed through
    get_device_ptr: packed and unpacked over PCIe."""
    rng = np.random.default_rng(tokens)
    keys, scales = _c8_cache(rng, 4, "int8")
    layer = _oracle_layer(keys, scales)
    slots = rng.permutation(4 * 128)[:tokens].astype(np.int64)
    n = _packet_bytes(layer, tokens)
    alloc = int(c_ops.alloc_pinned_ptr(n + 2 * PAD, 0))
    try:
        ctypes.memset(alloc, GUARD, n + 2 * PAD)
        dev_ptr = int(c_ops.get_device_ptr(alloc + PAD, n))
        assert dev_ptr
        state = c_ops.IndexerC8State(keys.to(DEV), scales.to(DEV))
        args = (torch.tensor([dev_ptr], dtype=torch.int64, device=DEV), torch.tensor([0], dtype=torch.int32, device=DEV),
                torch.tensor([tokens], dtype=torch.int32, device=DEV), torch.from_numpy(slots).to(DEV), tokens)
        c_ops.indexer_c8_transfer_prepared(state, *args, True)
        want = np.full(n, GUARD, np.uint8)
        ok.indexer_c8_transfer([layer], [[want]], [0], [tokens], slots, tokens, True, False)
        torch.cuda.synchronize()
        host = np.frombuffer(ctypes.string_at(alloc, n + 2 * PAD), dtype=np.uint8)
        assert np.array_equal(host[PAD: PAD + n], want)
        assert (host[:PAD] == GUARD).all() and (host[PAD + n:] == GUARD).all()
        state.keys.zero_()
        state.scales.zero_()
        cleared = _oracle_layer(state.keys.cpu(), state.scales.cpu())
        c_ops.indexer_c8_transfer_prepared(state, *args, False)
        ok.indexer_c8_transfer([cleared], [[want]], [0], [tokens], slots, tokens, False, False)
        torch.cuda.synchronize()
        assert np.array_equal(to_bytes(state.keys), cleared.keys)
        assert np.array_equal(to_bytes(state.scales), cleared.scales)
    finally:
        torch.cuda.synchronize()
        c_ops.free_pinned_ptr(alloc)


def test_c8_unpack_on_two_streams_vs_oracle(c_ops):
    """Two streams unpack their own packets, repeatedly, into disjoint slots
    of one cache; the result equals the oracle applying both (the slot sets
    are disjoint, so the order of the streams does not matter)."""
    rng = np.random.default_rng(3)
    blocks, tokens = 5, 257
    keys, scales = _c8_cache(rng, blocks, "int8")
    state = c_ops.IndexerC8State(keys.to(DEV), scales.to(DEV))
    layer = _oracle_layer(keys, scales)
    perm = rng.permutation(blocks * 128)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    keep = []
    for i, st in enumerate(streams):
        slots = perm[i * tokens: (i + 1) * tokens].astype(np.int64)
        packet = rng.integers(0, 256, size=_packet_bytes(layer, tokens), dtype=np.uint8)
        dev_packet = torch.from_numpy(packet).to(DEV)
        args = (torch.tensor([dev_packet.data_ptr()], dtype=torch.int64, device=DEV),
                torch.zeros(1, dtype=torch.int32, device=DEV), torch.tensor([tokens], dtype=torch.int32, device=DEV),
                torch.from_numpy(slots).to(DEV), tokens)
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            for _ in range(16):
                c_ops.indexer_c8_transfer_prepared(state, *args, False)
        keep.append((dev_packet, args))
        ok.indexer_c8_transfer([layer], [[packet]], [0], [tokens], slots, tokens, False, False)
    torch.cuda.synchronize()
    assert np.array_equal(to_bytes(state.keys), layer.keys)
    assert np.array_equal(to_bytes(state.scales), layer.scales)


@pytest.mark.parametrize("grouped", [False, True])
def test_c8_block_map_vs_oracle(c_ops, grouped):
    """An int32 block map sends logical block b to physical block map[b];
    the selected slots straddle block ends (offsets 126..128), alone and
    behind a bf16 layer in a group."""
    assert getattr(c_ops, "INDEXER_C8_BLOCK_MAP_ABI", 0) >= 1
    rng = np.random.default_rng(11 + grouped)
    blocks = 54
    keys, scales = _c8_cache(rng, blocks, "int8")
    block_map = torch.from_numpy(rng.permutation(blocks).astype(np.int32))
    slots = np.concatenate([np.arange(b * 128 + 126, b * 128 + 129) for b in (23, 47, 50)]).astype(np.int64)
    n = len(slots)
    c8 = c_ops.IndexerC8State(keys.to(DEV), scales.to(DEV), 1, block_map.to(DEV))
    layers = [_oracle_layer(keys, scales, 1, block_map)]
    states = [c8]
    if grouped:
        bf_keys, _ = _c8_cache(rng, blocks, "bf16")
        states.insert(0, c_ops.IndexerC8State(bf_keys.to(DEV)))
        layers.insert(0, _oracle_layer(bf_keys, None))
    packets = [torch.zeros(_packet_bytes(L, n), dtype=torch.uint8, device=DEV) for L in layers]
    args = (torch.tensor([[p.data_ptr()] for p in packets], dtype=torch.int64, device=DEV) if grouped else
            torch.tensor([packets[0].data_ptr()], dtype=torch.int64, device=DEV),
            torch.tensor([0], dtype=torch.int32, device=DEV), torch.tensor([n], dtype=torch.int32, device=DEV),
            torch.from_numpy(slots).to(DEV), n)
    run = c_ops.indexer_c8_group_transfer_prepared if grouped else c_ops.indexer_c8_transfer_prepared
    state = c_ops.IndexerC8GroupState(states) if grouped else c8
    run(state, *args, True)
    want = [[np.zeros(_packet_bytes(L, n), np.uint8)] for L in layers]
    ok.indexer_c8_transfer(layers, want, [0], [n], slots, n, True, False)
    torch.cuda.synchronize()
    for p, w in zip(packets, want):
        assert np.array_equal(to_bytes(p), w[0])
    for st in states:
        st.keys.zero_()
        if st.scales is not None:
            st.scales.zero_()
    cleared = [_oracle_layer(st.keys.cpu(), st.scales.cpu() if st.scales is not None else None, 1,
                             st.block_map.cpu() if st.block_map is not None else None) for st in states]
    run(state, *args, False)
    ok.indexer_c8_transfer(cleared, want, [0], [n], slots, n, False, False)
    torch.cuda.synchronize()
    for st, L in zip(states, cleared):
        assert np.array_equal(to_bytes(st.keys), L.keys)
        if st.scales is not None:
            assert np.array_equal(to_bytes(st.scales), L.scales)


@pytest.mark.parametrize("build,message", [
    (lambda c, d: c.IndexerC8State(torch.empty(2, 128, 1, 128, dtype=torch.int8, device=d),
                                   torch.empty(2, 128, 1, 1, dtype=torch.bfloat16, device=d)), "float16 scales"),
    (lambda c, d: c.IndexerC8State(torch.empty(2, 64, 1, 128, dtype=torch.bfloat16, device=d)), r"not a contiguous \[blocks, 128, 1, 128\] cache"),
    (lambda c, d: c.IndexerC8State(torch.empty(2, 128, 1, 128, dtype=torch.bfloat16, device=d), None, 2),
     "block factor"),
])
def test_c8_state_validation(c_ops, build, message):
    with pytest.raises(RuntimeError, match=message):
        build(c_ops, DEV)


def test_c8_metadata_must_be_device_vectors(c_ops):
    keys = torch.empty(2, 128, 1, 128, dtype=torch.int8, device=DEV)
    scales = torch.empty(2, 128, 1, 1, dtype=torch.float16, device=DEV)
    state = c_ops.IndexerC8State(keys, scales)
    dev_meta = torch.empty(0, dtype=torch.int64, device=DEV)
    with pytest.raises(RuntimeError, match="int32/int64 vectors"):
        c_ops.indexer_c8_transfer_prepared(state, dev_meta.cpu(), dev_meta, dev_meta, dev_meta, 1024, False)


# ---------------------------------------------------------------------------
# indexer C8: random cases against the oracle
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("from_npu", [True, False])
def test_c8_random_against_oracle(c_ops, from_npu):
    rng = np.random.default_rng(5)
    blocks, capacity = 8, 200
    keys = torch.from_numpy(rng.integers(-128, 128, size=(blocks, 128, 1, 128), dtype=np.int8)).to(DEV)
    scales = torch.from_numpy(rng.integers(0, 65535, size=(blocks, 128, 1, 1), dtype=np.uint16).view(np.float16)).to(DEV)
    counts = [150, 0, 201, 60, 120]              # 0 and > capacity: skipped
    offs = [0, 150, 150, 150, 210]
    # distinct slots (duplicate destinations have no defined write order),
    # some of them outside the cache
    slots_np = (rng.permutation(blocks * 128 + 45)[: sum([150, 60, 120]) + 20] - 5).astype(np.int64)
    packets = [torch.from_numpy(rng.integers(0, 256, size=max(n, 1) * 130, dtype=np.uint8)).to(DEV) for n in counts]
    ptr_list = [p.data_ptr() for p in packets]
    ptr_list[3] = 0                              # null packet: skipped
    state = c_ops.IndexerC8State(keys, scales)
    L = ok.C8Layer(to_bytes(keys), to_bytes(scales), 128, 1, None, blocks * 128)
    ref_packets = [to_bytes(p) if ptr else None for p, ptr in zip(packets, ptr_list)]
    ok.indexer_c8_transfer([L], [ref_packets], offs, counts, slots_np, capacity, from_npu, False)
    c_ops.indexer_c8_transfer_prepared(
        state, torch.tensor(ptr_list, dtype=torch.int64, device=DEV), torch.tensor(offs, dtype=torch.int32, device=DEV),
        torch.tensor(counts, dtype=torch.int32, device=DEV), torch.from_numpy(slots_np).to(DEV), capacity, from_npu)
    torch.cuda.synchronize()
    assert np.array_equal(to_bytes(keys), L.keys) and np.array_equal(to_bytes(scales), L.scales)
    for p, want in zip(packets, ref_packets):
        if want is not None:
            assert np.array_equal(to_bytes(p), want)


# ---------------------------------------------------------------------------
# sparse graph (sfa_copy)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("sel_dtype,slot_dtype", [(torch.int32, torch.int32), (torch.int64, torch.int64),
                                                  (torch.int32, torch.int64)])
@pytest.mark.parametrize("host_sources", [False, True])
def test_sparse_graph_against_oracle(c_ops, sel_dtype, slot_dtype, host_sources):
    rng = np.random.default_rng(7 + host_sources)
    R, W, cs, cpr, KH, PH = 3, 96, 64, 4, 512, 64
    kb, pb = KH * 2, PH * 2
    NB, BS = 32, 16
    k = torch.from_numpy(rng.integers(0, 65535, size=(NB, BS, 1, KH), dtype=np.uint16).view(np.int16)).view(
        torch.bfloat16).to(DEV)
    pe = torch.from_numpy(rng.integers(0, 65535, size=(NB, BS, 1, PH), dtype=np.uint16).view(np.int16)).view(
        torch.bfloat16).to(DEV)
    srcs_k, srcs_p = [], []
    for _ in range(R * cpr):
        a = torch.from_numpy(rng.integers(0, 256, size=cs * kb, dtype=np.uint8))
        b = torch.from_numpy(rng.integers(0, 256, size=cs * pb, dtype=np.uint8))
        if host_sources:
            srcs_k.append(a.pin_memory())
            srcs_p.append(b.pin_memory())
        else:
            srcs_k.append(a.to(DEV))
            srcs_p.append(b.to(DEV))
    kp = [c_ops.get_device_ptr(t.data_ptr(), t.numel()) if host_sources else t.data_ptr() for t in srcs_k]
    pp = [c_ops.get_device_ptr(t.data_ptr(), t.numel()) if host_sources else t.data_ptr() for t in srcs_p]
    kp[5] = 0                                    # null K source: skipped
    ptrs = torch.tensor([kp, pp], dtype=torch.int64, device=DEV)
    sel = rng.integers(-3, cs * cpr + 5, size=(R, W))
    slots = rng.permutation(NB * BS)[: R * W].reshape(R, W)
    slots[1, 4] = -1
    slots[2, 7] = NB * BS + 9
    counts = np.array([[70, 0], [300, 0], [0, 0]], dtype=np.int32)   # counts read at stride 2
    limits = np.array([200, 256, 100], dtype=np.int32)
    st = c_ops.prepare_sparse_direct_destination_state((k, pe), torch.zeros(1, device=DEV), 5, 0, 0, 0)
    want_k, want_p = to_bytes(k), to_bytes(pe)
    ok.sparse_graph_kv_transfer(want_k, want_p, kb, pb, slots, sel, counts[:, 0], limits,
                                [to_bytes(t) if p else None for t, p in zip(srcs_k, kp)],
                                [to_bytes(t) for t in srcs_p], cs)
    c_ops.sparse_graph_kv_transfer(st, torch.from_numpy(slots).to(slot_dtype).to(DEV),
                                   torch.from_numpy(sel).to(sel_dtype).to(DEV),
                                   torch.from_numpy(counts).to(DEV), ptrs, torch.from_numpy(limits).to(DEV), cs)
    torch.cuda.synchronize()
    assert np.array_equal(to_bytes(k), want_k) and np.array_equal(to_bytes(pe), want_p)
    assert not np.array_equal(want_k, to_bytes(torch.zeros_like(k)))


def test_sparse_graph_errors(c_ops):
    k = torch.zeros((4, 16, 1, 512), dtype=torch.bfloat16, device=DEV)
    pe = torch.zeros((4, 16, 1, 64), dtype=torch.bfloat16, device=DEV)
    st = c_ops.prepare_sparse_direct_destination_state((k, pe), torch.zeros(1, device=DEV), 5, 0, 0, 0)
    sel = torch.zeros((2, 4), dtype=torch.int32, device=DEV)
    cnt = torch.zeros(2, dtype=torch.int32, device=DEV)
    ptrs = torch.zeros((2, 2), dtype=torch.int64, device=DEV)
    with pytest.raises(RuntimeError, match="contiguous \\[rows, columns\\] matrix"):
        c_ops.sparse_graph_kv_transfer(st, sel[:, :2], sel[:, ::2], cnt, ptrs, cnt, 16)
    with pytest.raises(RuntimeError, match="contiguous int64 \\[2, chunks\\] table"):
        c_ops.sparse_graph_kv_transfer(st, sel, sel, cnt, ptrs[:1], cnt, 16)
    with pytest.raises(RuntimeError, match="one contiguous int32 per row"):
        c_ops.sparse_graph_kv_transfer(st, sel, sel, cnt, ptrs, cnt[:1], 16)
