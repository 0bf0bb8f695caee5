"""GPU parity of the sparse-graph copy (sfa_copy) and the indexer C8 packet
transport, through the C ABI.

The indexer tests are the reference's device qualification tests
(tests/standalone/test_indexer_c8_native.py) run on the MI355X: their
expected bytes are torch indexing of the caches (short scale tails with
guard bytes, fixed and offset chunks, int32/int64 metadata, a registered
host packet, two streams, mixed bf16 / int8 groups, the slot factor and the
block permutation).  Random cases with skipped chunks, slots and sources are
compared bit for bit with the CPU oracle (oracle/kv_transfer.py).
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
# indexer C8: the reference's qualification tests
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("strided_slots", [False, True])
@pytest.mark.parametrize("fixed", [False, True])
@pytest.mark.parametrize("metadata_dtype", [torch.int32, torch.int64])
def test_c8_packets_round_trip_with_short_scales(c_ops, strided_slots, fixed, metadata_dtype):
    counts = [1024, 1024, 7] if fixed else [1, 7, 127, 128, 129, 754, 1024]
    tokens = sum(counts)
    slots = torch.arange(tokens, dtype=torch.int64) * (2 if strided_slots else 1)
    blocks = (int(slots[-1]) + 128) // 128
    keys_cpu = torch.arange(blocks * 128 * 128).to(torch.int8).reshape(blocks, 128, 1, 128)
    scales_cpu = ((torch.arange(blocks * 128, dtype=torch.int32) * 97).to(torch.int16).view(torch.float16)
                  .reshape(blocks, 128, 1, 1))
    keys, scales = keys_cpu.to(DEV), scales_cpu.to(DEV)
    state = c_ops.IndexerC8State(keys, scales)
    buffers = [torch.full((130 * n + 64,), 173, dtype=torch.uint8, device=DEV) for n in counts]
    ptrs = torch.tensor([b.data_ptr() + 32 for b in buffers], dtype=torch.int64, device=DEV)
    lengths = torch.tensor(counts, dtype=metadata_dtype, device=DEV)
    starts = torch.tensor([0, *torch.tensor(counts).cumsum(0).tolist()[:-1]], dtype=metadata_dtype, device=DEV)
    slot_map = slots.to(device=DEV, dtype=metadata_dtype)
    if fixed:
        starts = lengths = torch.empty(1, dtype=metadata_dtype, device=DEV)
    c_ops.indexer_c8_transfer_prepared(state, ptrs, starts, lengths, slot_map, 1024, True, fixed_chunks=fixed)
    torch.cuda.synchronize()
    offset = 0
    for n, buffer in zip(counts, buffers):
        selected = slots[offset: offset + n]
        expected = torch.cat((keys_cpu.view(-1, 128)[selected].contiguous().view(torch.uint8).flatten(),
                              scales_cpu.view(-1, 1)[selected].contiguous().view(torch.uint8).flatten()))
        actual = buffer.cpu()
        assert torch.equal(actual[32:-32], expected)
        assert torch.all(actual[:32] == 173) and torch.all(actual[-32:] == 173)
        offset += n
    keys.fill_(42)
    scales.fill_(-1)
    c_ops.indexer_c8_transfer_prepared(state, ptrs, starts, lengths, slot_map, 1024, False, fixed_chunks=fixed)
    actual_keys, actual_scales = keys.cpu().view(-1, 128), scales.cpu().view(-1, 1)
    assert torch.equal(actual_keys[slots], keys_cpu.view(-1, 128)[slots])
    assert torch.equal(actual_scales.view(torch.int16)[slots], scales_cpu.view(-1, 1).view(torch.int16)[slots])
    untouched = torch.ones(blocks * 128, dtype=torch.bool)
    untouched[slots] = False
    assert torch.all(actual_keys[untouched] == 42)
    assert torch.all(actual_scales[untouched] == -1)


def test_c8_rejects_wrong_scale_dtype_and_metadata(c_ops):
    keys = torch.empty(2, 128, 1, 128, dtype=torch.int8, device=DEV)
    scales = torch.empty(2, 128, 1, 1, dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError, match="float16 scales"):
        c_ops.IndexerC8State(keys, scales.bfloat16())
    state = c_ops.IndexerC8State(keys, scales)
    meta = torch.empty(0, dtype=torch.int64, device=DEV)
    with pytest.raises(RuntimeError, match="int32/int64 vectors"):
        c_ops.indexer_c8_transfer_prepared(state, meta.cpu(), meta, meta, meta, 1024, False)
    with pytest.raises(RuntimeError, match="PA_BSND"):
        c_ops.IndexerC8State(torch.empty(2, 64, 1, 128, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(RuntimeError, match="block factor"):
        c_ops.IndexerC8State(torch.empty(2, 128, 1, 128, dtype=torch.bfloat16, device=DEV), None, 2)


@pytest.mark.parametrize("layers", [1, 3])
def test_c8_group_keeps_layers_and_planes_separate(c_ops, layers):
    keys = [torch.full((2, 128, 1, 128), i + 1, dtype=torch.int8, device=DEV) for i in range(layers)]
    scales = [torch.full((2, 128, 1, 1), (i + 1) / 16, dtype=torch.float16, device=DEV) for i in range(layers)]
    state = c_ops.IndexerC8GroupState([c_ops.IndexerC8State(k, s) for k, s in zip(keys, scales)])
    # Adjacent layer packets have unaligned starts after layer 0.
    packet = torch.full((layers * 7 * 130,), 255, dtype=torch.uint8, device=DEV)
    pointers = torch.tensor([[packet.data_ptr() + i * 7 * 130] for i in range(layers)], dtype=torch.int64,
                            device=DEV)
    offsets = torch.tensor([0], dtype=torch.int32, device=DEV)
    counts = torch.tensor([7], dtype=torch.int32, device=DEV)
    slots = torch.arange(7, dtype=torch.int64, device=DEV)
    c_ops.indexer_c8_group_transfer_prepared(state, pointers, offsets, counts, slots, 7, True)
    actual = packet.cpu().view(layers, 7 * 130)
    for i in range(layers):
        assert torch.all(actual[i, : 7 * 128].view(torch.int8) == i + 1)
        assert torch.all(actual[i, 7 * 128:].view(torch.float16) == (i + 1) / 16)


@pytest.mark.parametrize("tokens", [1, 7, 129])
def test_c8_registered_cpu_packet_round_trip(c_ops, tokens):
    keys = torch.arange(4 * 128 * 128).to(torch.int8).reshape(4, 128, 1, 128).to(DEV)
    scales = ((torch.arange(4 * 128, dtype=torch.int32) * 97).to(torch.int16).view(torch.float16)
              .reshape(4, 128, 1, 1).to(DEV))
    state = c_ops.IndexerC8State(keys, scales)
    slots_cpu = torch.arange(tokens, dtype=torch.int64) * 2
    slots = slots_cpu.to(DEV)
    expected_keys = keys.cpu().view(-1, 128)[slots_cpu]
    expected_scales = scales.cpu().view(-1, 1)[slots_cpu]
    payload = torch.cat((expected_keys.contiguous().view(torch.uint8).flatten(),
                         expected_scales.contiguous().view(torch.uint8).flatten()))
    allocation = int(c_ops.alloc_pinned_ptr(tokens * 130 + 64, 0))
    try:
        ctypes.memset(allocation, 173, tokens * 130 + 64)
        device_pointer = int(c_ops.get_device_ptr(allocation + 32, tokens * 130))
        assert device_pointer
        pointers = torch.tensor([device_pointer], dtype=torch.int64, device=DEV)
        offsets = torch.tensor([0], dtype=torch.int32, device=DEV)
        counts = torch.tensor([tokens], dtype=torch.int32, device=DEV)
        c_ops.indexer_c8_transfer_prepared(state, pointers, offsets, counts, slots, tokens, True)
        torch.cuda.synchronize()
        assert ctypes.string_at(allocation + 32, tokens * 130) == payload.numpy().tobytes()
        assert ctypes.string_at(allocation, 32) == bytes([173]) * 32
        assert ctypes.string_at(allocation + 32 + tokens * 130, 32) == bytes([173]) * 32
        keys.zero_()
        scales.zero_()
        c_ops.indexer_c8_transfer_prepared(state, pointers, offsets, counts, slots, tokens, False)
        torch.cuda.synchronize()
        assert torch.equal(keys.cpu().view(-1, 128)[slots_cpu], expected_keys)
        assert torch.equal(scales.cpu().view(-1, 1).view(torch.int16)[slots_cpu], expected_scales.view(torch.int16))
    finally:
        torch.cuda.synchronize()
        c_ops.free_pinned_ptr(allocation)


def test_c8_repeated_copy_on_two_streams_keeps_disjoint_slots(c_ops):
    tokens = 257
    keys = torch.full((5, 128, 1, 128), -7, dtype=torch.int8, device=DEV)
    scales = torch.full((5, 128, 1, 1), -1, dtype=torch.float16, device=DEV)
    state = c_ops.IndexerC8State(keys, scales)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    owners = []
    for rank, stream in enumerate(streams):
        key_bits = ((torch.arange(tokens * 128) + rank * 37) % 256).to(torch.uint8)
        scale_bits = ((torch.arange(tokens) + rank * 991) * 97).to(torch.int16)
        packet = torch.cat((key_bits, scale_bits.view(torch.uint8))).to(DEV)
        pointers = torch.tensor([packet.data_ptr()], dtype=torch.int64, device=DEV)
        offsets = torch.zeros(1, dtype=torch.int32, device=DEV)
        counts = torch.tensor([tokens], dtype=torch.int32, device=DEV)
        slots = (torch.arange(tokens, dtype=torch.int64) * 2 + rank).to(DEV)
        stream.wait_stream(torch.cuda.current_stream())
        owners.append((packet, pointers, offsets, counts, slots, key_bits, scale_bits))
        with torch.cuda.stream(stream):
            for _ in range(16):
                c_ops.indexer_c8_transfer_prepared(state, pointers, offsets, counts, slots, tokens, False)
    torch.cuda.synchronize()
    key_result = keys.cpu().view(-1, 128).view(torch.uint8)
    scale_result = scales.cpu().view(-1).view(torch.int16)
    for _, _, _, _, slots, expected_keys, expected_scales in owners:
        indices = slots.cpu()
        assert torch.equal(key_result[indices].flatten(), expected_keys)
        assert torch.equal(scale_result[indices], expected_scales)
    assert torch.all(keys.cpu().view(-1, 128)[tokens * 2:] == -7)
    assert torch.all(scales.cpu().view(-1)[tokens * 2:] == -1)


@pytest.mark.parametrize("slot_factor", [1, 2])
def test_c8_mixed_group_preserves_bf16_bits_and_c8_physical_mapping(c_ops, slot_factor):
    tokens = 259
    bf16_cpu = torch.arange(4 * 128 * 128).to(torch.int16).view(torch.bfloat16).reshape(4, 128, 1, 128)
    c8_cpu = torch.arange(4 * slot_factor * 128 * 128).to(torch.int8).reshape(4 * slot_factor, 128, 1, 128)
    scale_cpu = ((torch.arange(4 * slot_factor * 128) * 97).to(torch.int16).view(torch.float16)
                 .reshape(4 * slot_factor, 128, 1, 1))
    bf16, c8, scale = bf16_cpu.to(DEV), c8_cpu.to(DEV), scale_cpu.to(DEV)
    state = c_ops.IndexerC8GroupState([c_ops.IndexerC8State(bf16), c_ops.IndexerC8State(c8, scale, slot_factor)])
    packets = [torch.empty(tokens * width, dtype=torch.uint8, device=DEV) for width in (256, 130)]
    pointers = torch.tensor([[p.data_ptr()] for p in packets], dtype=torch.int64, device=DEV)
    offsets = torch.tensor([0], dtype=torch.int32, device=DEV)
    sizes = torch.tensor([tokens], dtype=torch.int32, device=DEV)
    slots = torch.arange(tokens, dtype=torch.int64, device=DEV)
    physical = torch.arange(tokens) + (torch.arange(tokens) // 128) * (slot_factor - 1) * 128
    c_ops.indexer_c8_group_transfer_prepared(state, pointers, offsets, sizes, slots, tokens, True)
    expected_bf16 = bf16_cpu.view(-1, 128)[:tokens].contiguous().view(torch.uint8).flatten()
    expected_c8 = torch.cat((c8_cpu.view(-1, 128)[physical].contiguous().view(torch.uint8).flatten(),
                             scale_cpu.view(-1, 1)[physical].contiguous().view(torch.uint8).flatten()))
    assert torch.equal(packets[0].cpu(), expected_bf16)
    assert torch.equal(packets[1].cpu(), expected_c8)
    bf16.zero_()
    c8.zero_()
    scale.zero_()
    c_ops.indexer_c8_group_transfer_prepared(state, pointers, offsets, sizes, slots, tokens, False)
    assert torch.equal(bf16.cpu().view(-1, 128)[:tokens].contiguous().view(torch.uint8).flatten(), expected_bf16)
    assert torch.equal(c8.cpu().view(-1, 128)[physical], c8_cpu.view(-1, 128)[physical])
    assert torch.equal(scale.cpu().view(torch.int16).view(-1)[physical],
                       scale_cpu.view(torch.int16).view(-1)[physical])


@pytest.mark.parametrize("grouped", [False, True])
def test_c8_paired_bank_copy_roundtrip_and_unused_rows(c_ops, grouped):
    assert getattr(c_ops, "INDEXER_C8_BLOCK_MAP_ABI", 0) >= 1
    t = 3
    mapping = torch.empty(18 * t, dtype=torch.int32)
    for u in range(t):
        ids = [*range(8 * u, 8 * u + 8), *range(8 * (t + u), 8 * (t + u) + 8), 16 * t + u, 17 * t + u]
        mapping[ids] = torch.tensor([*range(16 * u, 16 * u + 16), 16 * t + 2 * u, 16 * t + 2 * u + 1],
                                    dtype=torch.int32)
    keys = torch.arange(18 * t * 128 * 128).to(torch.int8).reshape(18 * t, 128, 1, 128).to(DEV)
    scales = ((torch.arange(18 * t * 128) * 97).to(torch.int16).view(torch.float16)
              .reshape(18 * t, 128, 1, 1).to(DEV))
    state = c_ops.IndexerC8State(keys, scales, 1, mapping.to(DEV))
    host_slots = torch.cat([torch.arange(b * 128 + 126, b * 128 + 129) for b in (23, 47, 50)])
    physical = mapping[host_slots // 128].long() * 128 + host_slots % 128
    expected = torch.cat([keys.cpu().view(-1, 128)[physical].contiguous().view(torch.uint8).flatten(),
                          scales.cpu().view(-1)[physical].contiguous().view(torch.uint8).flatten()])
    packet = torch.zeros_like(expected, device=DEV)
    ptr = torch.tensor([packet.data_ptr()], dtype=torch.int64, device=DEV)
    offsets = torch.tensor([0], dtype=torch.int32, device=DEV)
    counts = torch.tensor([len(host_slots)], dtype=torch.int32, device=DEV)
    slots = host_slots.to(DEV)
    if grouped:
        bf = torch.full_like(keys, 5, dtype=torch.bfloat16)
        bf_packet = torch.empty(len(host_slots) * 256, dtype=torch.uint8, device=DEV)
        state = c_ops.IndexerC8GroupState([c_ops.IndexerC8State(bf), state])
        ptr = torch.tensor([[bf_packet.data_ptr()], [packet.data_ptr()]], dtype=torch.int64, device=DEV)
    fn = c_ops.indexer_c8_group_transfer_prepared if grouped else c_ops.indexer_c8_transfer_prepared
    fn(state, ptr, offsets, counts, slots, len(host_slots), True)
    torch.cuda.synchronize()
    assert torch.equal(packet.cpu(), expected)
    keys.zero_()
    scales.zero_()
    fn(state, ptr, offsets, counts, slots, len(host_slots), False)
    torch.cuda.synchronize()
    actual = torch.cat([keys.cpu().view(-1, 128)[physical].contiguous().view(torch.uint8).flatten(),
                        scales.cpu().view(-1)[physical].contiguous().view(torch.uint8).flatten()])
    assert torch.equal(actual, expected)
    unused = torch.ones(18 * t * 128, dtype=torch.bool)
    unused[physical] = False
    assert keys.cpu().view(-1, 128)[unused].eq(0).all()
    assert scales.cpu().view(-1)[unused].eq(0).all()


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
    with pytest.raises(RuntimeError, match="contiguous matrix"):
        c_ops.sparse_graph_kv_transfer(st, sel[:, :2], sel[:, ::2], cnt, ptrs, cnt, 16)
    with pytest.raises(RuntimeError, match="two contiguous int64 plane tables"):
        c_ops.sparse_graph_kv_transfer(st, sel, sel, cnt, ptrs[:1], cnt, 16)
    with pytest.raises(RuntimeError, match="one contiguous int32 value per row"):
        c_ops.sparse_graph_kv_transfer(st, sel, sel, cnt, ptrs, cnt[:1], 16)
