"""The drop-in ops captured in a HIP graph (torch.cuda.CUDAGraph on ROCm).

A serving loop can capture a launch-bound sequence, such as the per-chunk
multi_layer_kv_transfer calls of one request, into a HIP graph and replay it
with one launch.  Each op here enqueues kernels on the current stream and
nothing else (no allocation, synchronisation or memset inside the op), so a
replay re-runs the captured launches on whatever the captured buffers hold.
Every test replays several times, writing new contents into the captured
buffers eagerly between replays, and checks every replay: the copies against
torch's own gathers, RoPE against the op run eagerly on the same key, the
CacheGen kernels against the eager op and by round trip.
"""

from __future__ import annotations

import pytest
import torch

from kvutil import block_slots, ptr_table, randn_bf16

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
REPLAYS = 3


@pytest.fixture(scope="module")
def ops():
    import lmcache_amd

    return lmcache_amd.c_ops


def _capture(fn):
    """Runs fn once eagerly on a side stream (lazy set-up happens outside the
    capture), then captures it."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def _kv_setup(gen):
    """SEPARATE_KV, 4 layers of [64 blocks, 16 slots, 8 heads, 128] bf16; two
    requests (100 and 130 tokens, 4 padding slots set to -1) in chunks of 64
    tokens, the last one partial."""
    L, NB, BS, H, D = 4, 64, 16, 8, 128
    W = H * D
    caches = [(randn_bf16([NB, BS, H, D], gen).to(DEV), randn_bf16([NB, BS, H, D], gen).to(DEV))
              for _ in range(L)]
    flat = [t for kv in caches for t in kv]
    blocks = torch.randperm(NB, generator=gen).tolist()
    slots = block_slots(blocks, BS, [100, 130])
    for i in (3, 50, 101, 229):
        slots[i] = -1
    slots = torch.tensor(slots, dtype=torch.int64, device=DEV)
    starts = list(range(0, slots.numel(), 64))
    chunks = [torch.zeros((2, L, min(64, slots.numel() - s), W), dtype=torch.bfloat16, device=DEV)
              for s in starts]
    views = [slots[s: s + c.shape[2]] for s, c in zip(starts, chunks)]
    return L, NB * BS, W, flat, ptr_table(flat, DEV), slots, starts, chunks, views


def test_per_chunk_store_replays_match_gather(ops):
    """Per-chunk stores (paged caches -> memory objects) captured once; each
    replay after new cache contents matches index_select at the valid slots
    and leaves the rows of -1 slots as the previous contents."""
    gen = torch.Generator().manual_seed(11)
    L, pbs, W, flat, ptrs, slots, starts, chunks, views = _kv_setup(gen)

    def store():
        for x, s in zip(chunks, views):
            ops.multi_layer_kv_transfer(x, ptrs, s, torch.device(DEV), pbs, True, False, 2, W, W, 0)

    g = _capture(store)
    for r in range(REPLAYS):
        for t in flat:
            t.copy_(randn_bf16(list(t.shape), gen).to(DEV))
        for x in chunks:
            x.fill_(float(r + 7))
        g.replay()
        torch.cuda.synchronize()
        for x, s in zip(chunks, views):
            valid = s >= 0
            for p in range(2):
                for l in range(L):
                    rows = flat[2 * l + p].view(-1, W)
                    want = torch.index_select(rows, 0, s[valid])
                    assert torch.equal(x[p, l][valid], want), (r, p, l)
                    assert bool((x[p, l][~valid] == float(r + 7)).all()), (r, p, l)


def test_per_chunk_retrieve_replays_match_scatter(ops):
    """Per-chunk retrieves (memory objects -> paged caches) captured once;
    each replay after new memory-object contents writes exactly the valid
    slots."""
    gen = torch.Generator().manual_seed(12)
    L, pbs, W, flat, ptrs, slots, starts, chunks, views = _kv_setup(gen)

    def retrieve():
        for x, s in zip(chunks, views):
            ops.multi_layer_kv_transfer(x, ptrs, s, torch.device(DEV), pbs, False, False, 2, W, W, 0)

    g = _capture(retrieve)
    valid_slots = slots[slots >= 0]
    untouched = torch.ones(pbs, dtype=torch.bool, device=DEV)
    untouched[valid_slots] = False
    for r in range(REPLAYS):
        for x in chunks:
            x.copy_(randn_bf16(list(x.shape), gen).to(DEV))
        for t in flat:
            t.zero_()
        g.replay()
        torch.cuda.synchronize()
        for x, s in zip(chunks, views):
            valid = s >= 0
            for p in range(2):
                for l in range(L):
                    rows = flat[2 * l + p].view(-1, W)
                    assert torch.equal(torch.index_select(rows, 0, s[valid]), x[p, l][valid]), (r, p, l)
        for t in flat:
            assert not bool(t.view(-1, W)[untouched].any()), r


@pytest.mark.parametrize("neox", [True, False])
def test_rope_replays_match_eager(ops, neox):
    """rotary_embedding_k_fused (in place) captured once; each replay on a
    new key equals the eager op on a copy of that key, bit for bit."""
    gen = torch.Generator().manual_seed(13)
    T, H, D = 96, 8, 128
    key = randn_bf16([T, H * D], gen).to(DEV)
    old = torch.arange(T, dtype=torch.int64, device=DEV)
    new = old + 1000
    inv = 1.0 / (500000.0 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    ang = torch.arange(T + 1000, dtype=torch.float32)[:, None] * inv[None, :]
    cache = torch.cat([ang.cos(), ang.sin()], dim=1).to(torch.bfloat16).to(DEV)

    g = _capture(lambda: ops.rotary_embedding_k_fused(old, new, key, D, cache, neox))
    for r in range(REPLAYS):
        fresh = randn_bf16([T, H * D], gen).to(DEV)
        want = fresh.clone()
        ops.rotary_embedding_k_fused(old, new, want, D, cache, neox)
        key.copy_(fresh)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(key, want), r


def _symbols(gen, L, T, C):
    x = torch.randn((L, T, C), generator=gen) * torch.rand((1, 1, C), generator=gen) * 5
    return (x.round() + 15).clamp(0, 30).to(torch.uint8).to(DEV)


def test_cachegen_replays_round_trip(ops):
    """calculate_cdf, encode_fast_new and decode_fast_prefsum captured as
    three graphs.  Each replay on new symbols: the CDF and the bitstreams
    equal the eager op's, and decoding the replayed streams returns the
    symbols."""
    gen = torch.Generator().manual_seed(14)
    L, T, C, nb = 2, 256, 128, 32
    sym = _symbols(gen, L, T, C)
    cap = 4 * T
    out = torch.zeros((L, C, cap), dtype=torch.uint8, device=DEV)
    lens = torch.zeros((L, C), dtype=torch.int32, device=DEV)
    stream = torch.zeros(L * C * cap, dtype=torch.uint8, device=DEV)
    prefix = torch.zeros((L, C), dtype=torch.int32, device=DEV)
    dec = torch.zeros((L, T, C), dtype=torch.uint8, device=DEV)
    cdf = ops.calculate_cdf(sym, nb)

    cdf_holder = []
    g_cdf = _capture(lambda: cdf_holder.append(ops.calculate_cdf(sym, nb)))
    cdf_g = cdf_holder[-1]
    g_enc = _capture(lambda: ops.encode_fast_new(cdf, sym, out, lens))
    g_dec = _capture(lambda: ops.decode_fast_prefsum(cdf, stream, prefix, dec))
    for r in range(REPLAYS):
        sym.copy_(_symbols(gen, L, T, C))
        want_cdf = ops.calculate_cdf(sym, nb)
        g_cdf.replay()
        torch.cuda.synchronize()
        assert torch.equal(cdf_g, want_cdf), r

        cdf.copy_(want_cdf)
        want_out = torch.zeros_like(out)
        want_lens = torch.zeros_like(lens)
        ops.encode_fast_new(cdf, sym, want_out, want_lens)
        g_enc.replay()
        torch.cuda.synchronize()
        assert torch.equal(lens, want_lens), r
        n = lens.view(-1).tolist()
        rows = out.view(-1, cap)
        want_rows = want_out.view(-1, cap)
        for i, k in enumerate(n):
            assert torch.equal(rows[i, :k], want_rows[i, :k]), (r, i)

        flat = torch.cat([rows[i, :k] for i, k in enumerate(n)])
        stream.zero_()
        stream[: flat.numel()].copy_(flat)
        prefix.copy_(lens.view(-1).cumsum(0).to(torch.int32).view(L, C))
        dec.fill_(0xEE)
        g_dec.replay()
        torch.cuda.synchronize()
        assert torch.equal(dec, sym), r


@pytest.mark.parametrize("host_sources", [False, True])
def test_sparse_graph_replays_follow_device_counts(ops, host_sources):
    """sparse_graph_kv_transfer is the reference's graph-replay copy
    (csrc/graph/sparse_graph_kernel.cpp): captured once, each replay reads
    the selections, slots, counts and limits the captured tensors hold at
    that replay.  Every replay writes new values into them and matches the
    oracle on the same bytes."""
    import numpy as np

    from kvutil import to_bytes
    from oracle import kv_transfer as ok

    rng = np.random.default_rng(31 + host_sources)
    R, W, cs, cpr, KH, PH = 3, 64, 64, 4, 512, 64
    kb, pb = KH * 2, PH * 2
    NB, BS = 32, 16
    k = torch.zeros((NB, BS, 1, KH), dtype=torch.bfloat16, device=DEV)
    pe = torch.zeros((NB, BS, 1, PH), dtype=torch.bfloat16, device=DEV)
    srcs_k, srcs_p = [], []
    for _ in range(R * cpr):
        a = torch.from_numpy(rng.integers(0, 256, size=cs * kb, dtype=np.uint8))
        b = torch.from_numpy(rng.integers(0, 256, size=cs * pb, dtype=np.uint8))
        srcs_k.append(a.pin_memory() if host_sources else a.to(DEV))
        srcs_p.append(b.pin_memory() if host_sources else b.to(DEV))
    addr = (lambda t: ops.get_device_ptr(t.data_ptr(), t.numel())) if host_sources else (lambda t: t.data_ptr())
    ptrs = torch.tensor([[addr(t) for t in srcs_k], [addr(t) for t in srcs_p]], dtype=torch.int64, device=DEV)
    sel = torch.zeros((R, W), dtype=torch.int32, device=DEV)
    slots = torch.full((R, W), -1, dtype=torch.int64, device=DEV)
    counts = torch.zeros((R,), dtype=torch.int32, device=DEV)
    limits = torch.zeros((R,), dtype=torch.int32, device=DEV)
    st = ops.prepare_sparse_direct_destination_state((k, pe), torch.zeros(1, device=DEV), 5, 0, 0, 0)
    g = _capture(lambda: ops.sparse_graph_kv_transfer(st, slots, sel, counts, ptrs, limits, cs))
    for r in range(REPLAYS):
        s_np = rng.integers(-2, cs * cpr + 3, size=(R, W)).astype(np.int32)
        d_np = rng.permutation(NB * BS)[: R * W].reshape(R, W).astype(np.int64)
        c_np = rng.integers(0, W + 8, size=R).astype(np.int32)
        l_np = rng.integers(0, cs * cpr + 1, size=R).astype(np.int32)
        c_np[r % R] = 0
        sel.copy_(torch.from_numpy(s_np))
        slots.copy_(torch.from_numpy(d_np))
        counts.copy_(torch.from_numpy(c_np))
        limits.copy_(torch.from_numpy(l_np))
        k.zero_()
        pe.zero_()
        want_k, want_p = to_bytes(k), to_bytes(pe)
        ok.sparse_graph_kv_transfer(want_k, want_p, kb, pb, d_np, s_np, c_np, l_np,
                                    [to_bytes(t) for t in srcs_k], [to_bytes(t) for t in srcs_p], cs)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(to_bytes(k), want_k), r
        assert np.array_equal(to_bytes(pe), want_p), r
        assert want_k.any(), r


@pytest.mark.parametrize("from_npu", [True, False])
def test_c8_prepared_replays_follow_device_metadata(ops, from_npu):
    """indexer_c8_transfer_prepared captured once; each replay reads the
    packet contents, chunk offsets, counts and slots the captured tensors
    hold at that replay (a zero count and slots outside the cache included)
    and matches the oracle on the same bytes, in both directions."""
    import numpy as np

    from kvutil import to_bytes
    from oracle import kv_transfer as ok

    rng = np.random.default_rng(41 + from_npu)
    blocks, capacity, chunks = 8, 128, 4
    keys = torch.zeros((blocks, 128, 1, 128), dtype=torch.int8, device=DEV)
    scales = torch.zeros((blocks, 128, 1, 1), dtype=torch.float16, device=DEV)
    packets = [torch.zeros(capacity * 130, dtype=torch.uint8, device=DEV) for _ in range(chunks)]
    ptrs = torch.tensor([p.data_ptr() for p in packets], dtype=torch.int64, device=DEV)
    offs = torch.zeros(chunks, dtype=torch.int32, device=DEV)
    counts = torch.zeros(chunks, dtype=torch.int32, device=DEV)
    slots = torch.full((chunks * capacity,), -1, dtype=torch.int64, device=DEV)
    state = ops.IndexerC8State(keys, scales)
    g = _capture(lambda: ops.indexer_c8_transfer_prepared(state, ptrs, offs, counts, slots, capacity, from_npu))
    for r in range(REPLAYS):
        cnt = rng.integers(1, capacity + 1, size=chunks).astype(np.int32)
        cnt[r % chunks] = 0
        off = np.concatenate([[0], np.cumsum(cnt)[:-1]]).astype(np.int32)
        n = int(cnt.sum())
        s_np = np.full(chunks * capacity, -1, np.int64)
        s_np[:n] = rng.permutation(blocks * 128 + 20)[:n] - 10    # distinct; a few outside the cache
        keys.copy_(torch.from_numpy(rng.integers(-128, 128, size=tuple(keys.shape), dtype=np.int8)))
        scales.copy_(torch.from_numpy(rng.integers(0, 65535, size=tuple(scales.shape), dtype=np.uint16)
                                      .view(np.float16)))
        for p in packets:
            p.copy_(torch.from_numpy(rng.integers(0, 256, size=p.numel(), dtype=np.uint8)))
        offs.copy_(torch.from_numpy(off))
        counts.copy_(torch.from_numpy(cnt))
        slots.copy_(torch.from_numpy(s_np))
        layer = ok.C8Layer(to_bytes(keys), to_bytes(scales), 128, 1, None, blocks * 128)
        ref_packets = [to_bytes(p) for p in packets]
        ok.indexer_c8_transfer([layer], [ref_packets], off.tolist(), cnt.tolist(), s_np, capacity, from_npu, False)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(to_bytes(keys), layer.keys), r
        assert np.array_equal(to_bytes(scales), layer.scales), r
        for p, want in zip(packets, ref_packets):
            assert np.array_equal(to_bytes(p), want), r
