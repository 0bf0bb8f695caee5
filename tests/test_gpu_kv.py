"""GPU parity of the gather/scatter ops against the CPU oracle.

Every test runs the op on the MI355X through the C ABI (lmcache_amd.c_ops ->
liblmcache_amd.so) and compares bytes with oracle/kv_transfer.py on the same
seeded inputs: bit-exact, plus guard bytes around the LMCache buffers and
untouched unmapped slots.  Shapes follow the reference's tests
(tests/v1/test_mem_kernels.py) at sizes the oracle finishes in seconds; the
Llama-3-8B-shape case (32 layers, 4096 tokens, 2048 blocks of 128) is checked
through size-independent properties (round trip, equality with torch's
index_select gather, checksums).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvutil import block_slots, ptr_table, randn_bf16, sample_slots, to_bytes
from oracle import kv_transfer as ok

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def ops():
    import lmcache_amd

    return lmcache_amd.c_ops


def _sync():
    torch.cuda.synchronize()


def _paged(fmt, L, NB, BS, H, D, gen, two_major=True, mla_widths=None):
    """Per-layer caches in the reference connector's structure, on the GPU."""
    layers = []
    for _ in range(L):
        if fmt == 1:
            shape = [2, NB, BS, H, D] if two_major else [NB, 2, BS, H, D]
            layers.append(randn_bf16(shape, gen).to(DEV))
        elif fmt == 2:
            layers.append((randn_bf16([NB, BS, H, D], gen).to(DEV), randn_bf16([NB, BS, H, D], gen).to(DEV)))
        else:
            layers.append(tuple(randn_bf16([NB, BS, 1, w], gen).to(DEV) for w in mla_widths))
    return layers


def _flat_tensors(layers):
    out = []
    for x in layers:
        out.extend(x if isinstance(x, tuple) else [x])
    return out


# ---------------------------------------------------------------------------
# multi_layer_kv_transfer
# ---------------------------------------------------------------------------


def test_c1_plumbing_case_matches_golden(ops):
    """C1: 4 layers SEPARATE_KV, 256 tokens; store then retrieve into zeroed
    caches, bit-exact against the oracle's digests."""
    import json
    import os
    import hashlib

    from tests.golden import gen_kv_golden as g

    caches, slots = g.c1_inputs()
    gpu = [(k.to(DEV), v.to(DEV)) for k, v in caches]
    flat = _flat_tensors(gpu)
    ptrs = ptr_table(flat, DEV)
    s = slots.to(DEV)
    # guard bytes around the memory object
    guard2 = torch.full((2 * 4 * 256 * 1024 * 2 + 8192,), 173, dtype=torch.uint8, device=DEV)
    lmc = guard2[4096: 4096 + 2 * 4 * 256 * 1024 * 2].view(torch.bfloat16).view(2, 4, 256, 1024)
    ops.multi_layer_kv_transfer(lmc, ptrs, s, torch.device(DEV), 64 * 16, True, False, 2, 1024, 1024, 0)
    _sync()
    want = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kv_c1.json")))
    assert hashlib.sha256(to_bytes(lmc).tobytes()).hexdigest() == want["lmc_sha256"]
    gb = guard2.cpu().numpy()
    assert (gb[:4096] == 173).all() and (gb[-4096:] == 173).all()
    zero = [torch.zeros_like(t) for t in flat]
    ops.multi_layer_kv_transfer(lmc, ptr_table(zero, DEV), s, torch.device(DEV), 64 * 16, False, False, 2,
                                1024, 1024, 0)
    _sync()
    cat = np.concatenate([to_bytes(z) for z in zero])
    assert hashlib.sha256(cat.tobytes()).hexdigest() == want["retrieved_caches_sha256"]


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("num_tokens,chunk", [(256, 256), (500, 256), (1024, 512)])
@pytest.mark.parametrize("num_layers", [1, 8])
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_multi_layer_store_retrieve_vs_oracle(ops, fmt, num_tokens, chunk, num_layers, slot_dtype):
    gen = torch.Generator().manual_seed(1000 + fmt * 7 + num_tokens + num_layers)
    NB, BS, H, D = 96, 16, 8, 64
    W = H * D
    pbs = NB * BS
    layers = _paged(fmt, num_layers, NB, BS, H, D, gen)
    flat = _flat_tensors(layers)
    ptrs = ptr_table(flat, DEV)
    slots_all = torch.tensor(sample_slots(pbs, num_tokens, seed=num_tokens), dtype=slot_dtype)
    table_np = [to_bytes(t) for t in flat]
    for c0 in range(0, num_tokens, chunk):
        sl = slots_all[c0: c0 + chunk]
        T = sl.shape[0]
        lmc = torch.zeros((2, num_layers, T, W), dtype=torch.bfloat16, device=DEV)
        ops.multi_layer_kv_transfer(lmc, ptrs, sl.to(DEV), torch.device(DEV), pbs, True, False, fmt, W, W, 0)
        want = np.zeros(2 * num_layers * T * W * 2, np.uint8)
        ok.multi_layer_kv_transfer(want, table_np, sl.numpy().astype(np.int64), pbs, True, False, fmt,
                                   num_layers, W, 2)
        _sync()
        assert np.array_equal(to_bytes(lmc), want)
        # retrieve into zeroed caches
        zero = [torch.zeros_like(t) for t in flat]
        ops.multi_layer_kv_transfer(lmc, ptr_table(zero, DEV), sl.to(DEV), torch.device(DEV), pbs, False,
                                    False, fmt, W, W, 0)
        zero_np = [np.zeros_like(x) for x in table_np]
        ok.multi_layer_kv_transfer(want, zero_np, sl.numpy().astype(np.int64), pbs, False, False, fmt,
                                   num_layers, W, 2)
        _sync()
        for z, zn in zip(zero, zero_np):
            assert np.array_equal(to_bytes(z), zn)


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("num_heads,head_size", [(8, 256), (1, 256), (4, 128)])
def test_multi_layer_row_widths(ops, fmt, num_heads, head_size):
    """tests/v1/test_mem_kernels.py:24-284 use head_size 256: 4 KiB rows
    (two slices per row); 1 head gives 512-byte rows (tiles)."""
    gen = torch.Generator().manual_seed(fmt * 100 + num_heads + head_size)
    L, NB, BS, T = 4, 64, 128, 500
    W = num_heads * head_size
    pbs = NB * BS
    layers = _paged(fmt, L, NB, BS, num_heads, head_size, gen)
    flat = _flat_tensors(layers)
    slots = torch.tensor(sample_slots(pbs, T, seed=7), dtype=torch.int64)
    table_np = [to_bytes(t) for t in flat]
    lmc = torch.zeros((2, L, T, W), dtype=torch.bfloat16, device=DEV)
    ops.multi_layer_kv_transfer(lmc, ptr_table(flat, DEV), slots.to(DEV), torch.device(DEV), pbs, True, False, fmt,
                                W, W, 0)
    want = np.zeros(2 * L * T * W * 2, np.uint8)
    ok.multi_layer_kv_transfer(want, table_np, slots.numpy(), pbs, True, False, fmt, L, W, 2)
    _sync()
    assert np.array_equal(to_bytes(lmc), want)
    zero = [torch.zeros_like(t) for t in flat]
    ops.multi_layer_kv_transfer(lmc, ptr_table(zero, DEV), slots.to(DEV), torch.device(DEV), pbs, False, False, fmt,
                                W, W, 0)
    zero_np = [np.zeros_like(x) for x in table_np]
    ok.multi_layer_kv_transfer(want, zero_np, slots.numpy(), pbs, False, False, fmt, L, W, 2)
    _sync()
    for z, zn in zip(zero, zero_np):
        assert np.array_equal(to_bytes(z), zn)


def test_multi_layer_equals_load_and_reshape_flash(ops):
    """tests/v1/test_mem_kernels.py:24-168: multi_layer (MERGED) equals the
    layer-by-layer load_and_reshape_flash result, and the retrieve restores
    the mapped rows into fresh caches."""
    gen = torch.Generator().manual_seed(5)
    L, NB, BS, H, D, T = 8, 64, 128, 2, 128, 500
    W = H * D
    pbs = NB * BS
    layers = _paged(1, L, NB, BS, H, D, gen)
    ptrs = ptr_table(layers, DEV)
    slots = torch.tensor(sample_slots(pbs, T, seed=2), device=DEV)
    a = torch.zeros((2, L, T, W), dtype=torch.bfloat16, device=DEV)
    b = torch.zeros_like(a)
    ops.multi_layer_kv_transfer(a, ptrs, slots, torch.device(DEV), pbs, True, False, 1, W, W, 0)
    for l in range(L):
        ops.load_and_reshape_flash(b, layers[l][0], layers[l][1], slots, l)
    _sync()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    fresh = _paged(1, L, NB, BS, H, D, gen)
    for l in range(L):
        ops.reshape_and_cache_back_flash(b, fresh[l][0], fresh[l][1], slots, l)
    _sync()
    for l in range(L):
        for p in range(2):
            left = layers[l][p].reshape(-1, W)[slots]
            right = fresh[l][p].reshape(-1, W)[slots]
            assert torch.equal(left.view(torch.int16), right.view(torch.int16))


@pytest.mark.parametrize("fmt", [3, 4, 5, 6])
def test_multi_layer_mla_dsa_vs_oracle(ops, fmt):
    gen = torch.Generator().manual_seed(30 + fmt)
    L, NB, BS, T = 4, 64, 16, 300
    kH, vH, dsaH = 512, 64, 128
    widths = {3: [kH, vH], 5: [kH, vH], 4: [kH, vH, dsaH], 6: [dsaH]}[fmt]
    layers = _paged(fmt, L, NB, BS, 1, 1, gen, mla_widths=widths)
    flat = _flat_tensors(layers)
    pbs = NB * BS
    slots = torch.tensor(sample_slots(pbs, T, seed=fmt), dtype=torch.int64)
    wsum = sum(widths)
    lmc = torch.zeros((1, L, T, wsum), dtype=torch.bfloat16, device=DEV)
    ops.multi_layer_kv_transfer(lmc, ptr_table(flat, DEV), slots.to(DEV), torch.device(DEV), pbs, True, False,
                                fmt, kH, vH, dsaH)
    table_np = [to_bytes(t) for t in flat]
    want = np.zeros(L * T * wsum * 2, np.uint8)
    ok.multi_layer_kv_transfer(want, table_np, slots.numpy(), pbs, True, False, fmt, L, wsum, 2, kH, vH, dsaH)
    _sync()
    assert np.array_equal(to_bytes(lmc), want)
    zero = [torch.zeros_like(t) for t in flat]
    ops.multi_layer_kv_transfer(lmc, ptr_table(zero, DEV), slots.to(DEV), torch.device(DEV), pbs, False,
                                False, fmt, kH, vH, dsaH)
    _sync()
    zero_np = [np.zeros_like(x) for x in table_np]
    ok.multi_layer_kv_transfer(want, zero_np, slots.numpy(), pbs, False, False, fmt, L, wsum, 2, kH, vH, dsaH)
    for z, zn in zip(zero, zero_np):
        assert np.array_equal(to_bytes(z), zn)


def test_mla_single_plane_576_with_padding_slots(ops):
    """DeepSeek-V3-style latent cache: one [NB, BS, 576] tensor per layer,
    use_mla=True; 1152-byte rows (not a multiple of one 1 KiB wave access);
    5% of slots are -1 and must be skipped."""
    gen = torch.Generator().manual_seed(61)
    L, NB, BS, W, T = 6, 128, 64, 576, 2048
    caches = [(torch.randn((NB, BS, W), generator=gen) * 0.5).to(torch.bfloat16).to(DEV) for _ in range(L)]
    pbs = NB * BS
    blocks = torch.randperm(NB, generator=gen)[: T // BS].tolist()
    slots = torch.tensor(block_slots(blocks, BS), dtype=torch.int64)
    pad = torch.randperm(T, generator=gen)[: int(round(0.05 * T))]
    slots[pad] = -1
    guard = 0x5A5A
    lmc = torch.full((1, L, T, W), 0, dtype=torch.int16, device=DEV)
    lmc.fill_(guard)
    lmc = lmc.view(torch.bfloat16)
    ops.multi_layer_kv_transfer(lmc, ptr_table(caches, DEV), slots.to(DEV), torch.device(DEV), pbs, True, True,
                                1, 0, 0, 0)
    table_np = [to_bytes(t) for t in caches]
    want = to_bytes(lmc.cpu().view(torch.int16).fill_(guard).view(torch.bfloat16))
    ok.multi_layer_kv_transfer(want, table_np, slots.numpy(), pbs, True, True, 1, L, W, 2)
    _sync()
    got = to_bytes(lmc)
    assert np.array_equal(got, want)
    assert (lmc.view(torch.int16)[:, :, pad] == guard).all()
    # retrieve into zeroed caches: padded tokens write nothing
    zero = [torch.zeros_like(t) for t in caches]
    ops.multi_layer_kv_transfer(lmc, ptr_table(zero, DEV), slots.to(DEV), torch.device(DEV), pbs, False, True,
                                1, 0, 0, 0)
    _sync()
    valid = slots[slots >= 0].to(DEV)
    for z, c in zip(zero, caches):
        zr, cr = z.reshape(-1, W), c.reshape(-1, W)
        assert torch.equal(zr[valid].view(torch.int16), cr[valid].view(torch.int16))
        mask = torch.ones(pbs, dtype=torch.bool, device=DEV)
        mask[valid] = False
        assert (zr[mask].view(torch.int16) == 0).all()


def test_batched_equals_per_chunk(ops):
    gen = torch.Generator().manual_seed(77)
    L, NB, BS, H, D = 8, 64, 128, 8, 128
    W = H * D
    pbs = NB * BS
    layers = _paged(2, L, NB, BS, H, D, gen)
    flat = _flat_tensors(layers)
    ptrs = ptr_table(flat, DEV)
    lengths = [1000, 1100, 996, 1000]
    blocks = torch.randperm(NB, generator=gen).tolist()
    slots = torch.tensor(block_slots(blocks, BS, lengths), dtype=torch.int64, device=DEV)
    n = slots.shape[0]
    starts = list(range(0, n, 256))
    per = [torch.zeros((2, L, min(256, n - s), W), dtype=torch.bfloat16, device=DEV) for s in starts]
    bat = [torch.zeros_like(x) for x in per]
    for x, s in zip(per, starts):
        ops.multi_layer_kv_transfer(x, ptrs, slots[s: s + x.shape[2]], torch.device(DEV), pbs, True, False, 2, W,
                                    W, 0)
    ops.multi_layer_kv_transfer_batched(bat, ptrs, slots, starts, torch.device(DEV), pbs, True, False, 2, W, W, 0)
    _sync()
    for x, y in zip(per, bat):
        assert torch.equal(x.view(torch.int16), y.view(torch.int16))
    # batched retrieve into zeroed caches equals per-chunk retrieve
    z1 = [torch.zeros_like(t) for t in flat]
    z2 = [torch.zeros_like(t) for t in flat]
    for x, s in zip(per, starts):
        ops.multi_layer_kv_transfer(x, ptr_table(z1, DEV), slots[s: s + x.shape[2]], torch.device(DEV), pbs, False,
                                    False, 2, W, W, 0)
    ops.multi_layer_kv_transfer_batched(bat, ptr_table(z2, DEV), slots, starts, torch.device(DEV), pbs, False,
                                        False, 2, W, W, 0)
    _sync()
    for a, b in zip(z1, z2):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("direction", [True, False])
def test_fused_equals_non_fused(ops, direction):
    """tests/v1/test_mem_kernels.py:287-591: the staged path moves the same
    bytes as the direct one; the staging buffer is a sliced view."""
    gen = torch.Generator().manual_seed(90 + direction)
    L, NB, BS, H, D, T, chunk = 4, 64, 128, 8, 128, 200, 256
    W = H * D
    pbs = NB * BS
    layers = _paged(1, L, NB, BS, H, D, gen)
    ptrs = ptr_table(layers, DEV)
    slots = torch.tensor(sample_slots(pbs, T, seed=3), device=DEV)
    staging = torch.empty((2, L, chunk, W), dtype=torch.bfloat16, device=DEV)[:, :, :T, :]
    if direction:
        host = torch.zeros((2, L, T, W), dtype=torch.bfloat16).pin_memory()
        ops.fused_multi_layer_kv_transfer(host, staging, ptrs, slots, torch.device(DEV), pbs, True, False, 1, W, W,
                                          0)
        ref = torch.zeros((2, L, T, W), dtype=torch.bfloat16, device=DEV)
        ops.multi_layer_kv_transfer(ref, ptrs, slots, torch.device(DEV), pbs, True, False, 1, W, W, 0)
        _sync()
        assert torch.equal(host.view(torch.int16), ref.cpu().view(torch.int16))
    else:
        host = randn_bf16((2, L, T, W), gen).pin_memory()
        fresh = _paged(1, L, NB, BS, H, D, gen)
        ops.fused_multi_layer_kv_transfer(host, staging, ptr_table(fresh, DEV), slots, torch.device(DEV), pbs,
                                          False, False, 1, W, W, 0)
        _sync()
        for l in range(L):
            for p in range(2):
                got = fresh[l][p].reshape(-1, W)[slots]
                assert torch.equal(got.cpu().view(torch.int16), host[p, l].view(torch.int16))


def test_fused_staging_too_small_raises(ops):
    L, W, T = 2, 256, 64
    layers = [torch.zeros((2, 8, 16, 2, 128), dtype=torch.bfloat16, device=DEV) for _ in range(L)]
    host = torch.zeros((2, L, T, W), dtype=torch.bfloat16).pin_memory()
    staging = torch.empty((2, L, T - 1, W), dtype=torch.bfloat16, device=DEV)
    slots = torch.arange(T, device=DEV)
    with pytest.raises(RuntimeError, match="staging_cache is smaller than the transfer"):
        ops.fused_multi_layer_kv_transfer(host, staging, ptr_table(layers, DEV), slots, torch.device(DEV), 128,
                                          True, False, 1, W, W, 0)


@pytest.mark.parametrize("direction", [True, False])
def test_pinned_host_zero_copy(ops, direction):
    """The memory object lives in pinned host memory: the kernel reads/writes
    it over PCIe through its mapped device address."""
    gen = torch.Generator().manual_seed(120 + direction)
    L, NB, BS, H, D, T = 4, 64, 16, 8, 128, 256
    W = H * D
    pbs = NB * BS
    layers = _paged(2, L, NB, BS, H, D, gen)
    flat = _flat_tensors(layers)
    slots = torch.tensor(sample_slots(pbs, T, seed=9), dtype=torch.int64)
    table_np = [to_bytes(t) for t in flat]
    if direction:
        host = torch.zeros((2, L, T, W), dtype=torch.bfloat16).pin_memory()
        ops.multi_layer_kv_transfer(host, ptr_table(flat, DEV), slots.to(DEV), torch.device(DEV), pbs, True, False,
                                    2, W, W, 0)
        want = np.zeros(2 * L * T * W * 2, np.uint8)
        ok.multi_layer_kv_transfer(want, table_np, slots.numpy(), pbs, True, False, 2, L, W, 2)
        _sync()
        assert np.array_equal(to_bytes(host), want)
    else:
        host = randn_bf16((2, L, T, W), gen).pin_memory()
        zero = [torch.zeros_like(t) for t in flat]
        ops.multi_layer_kv_transfer(host, ptr_table(zero, DEV), slots.to(DEV), torch.device(DEV), pbs, False, False,
                                    2, W, W, 0)
        zero_np = [np.zeros_like(x) for x in table_np]
        ok.multi_layer_kv_transfer(to_bytes(host), zero_np, slots.numpy(), pbs, False, False, 2, L, W, 2)
        _sync()
        for z, zn in zip(zero, zero_np):
            assert np.array_equal(to_bytes(z), zn)


def test_alloc_pinned_and_device_ptr(ops):
    size = 1 << 20
    p = ops.alloc_pinned_ptr(size, 0)
    assert p != 0
    d = ops.get_device_ptr(p + 100, 10)
    assert d != 0
    assert ops.get_device_ptr(p + size - 5, 10) == 0  # range overflows the record
    ops.free_pinned_ptr(p)
    assert ops.register_mapping(0x7000_0000_0000, 0x7100_0000_0000, 4096) == 0x7100_0000_0000
    assert ops.get_device_ptr(0x7000_0000_0010, 16) == 0x7100_0000_0010
    assert ops.unregister_ptr(0x7000_0000_0000) == 0
    assert ops.unregister_ptr(0x7000_0000_0000) == -1


def _first_allowed_node() -> int:
    for line in open("/proc/self/status"):
        if line.startswith("Mems_allowed_list:"):
            return int(line.split(":")[1].strip().split(",")[0].split("-")[0])
    return 0


@pytest.mark.parametrize("direction", [True, False])
def test_numa_pinned_host_zero_copy(ops, direction):
    """csrc/common/mem_alloc.cpp:56-106: memory from alloc_pinned_numa_ptr on
    a node this process may use is zeroed, registered, and the transfer kernel reads/writes it
    through its mapped device address; freeing drops the registry record."""
    import ctypes

    gen = torch.Generator().manual_seed(140 + direction)
    L, NB, BS, H, D, T = 2, 32, 16, 8, 128, 200
    W = H * D
    pbs = NB * BS
    size = 2 * L * T * W * 2
    p = ops.alloc_pinned_numa_ptr(size, _first_allowed_node())
    try:
        raw = (ctypes.c_ubyte * size).from_address(p)
        assert not any(raw[i] for i in range(0, size, 4099))
        assert ops.get_device_ptr(p, size) != 0
        host = torch.frombuffer(raw, dtype=torch.bfloat16).view(2, L, T, W)
        assert host.data_ptr() == p
        layers = _paged(2, L, NB, BS, H, D, gen)
        flat = _flat_tensors(layers)
        slots = torch.tensor(sample_slots(pbs, T, seed=31), dtype=torch.int64)
        table_np = [to_bytes(t) for t in flat]
        if direction:
            ops.multi_layer_kv_transfer(host, ptr_table(flat, DEV), slots.to(DEV), torch.device(DEV), pbs, True,
                                        False, 2, W, W, 0)
            want = np.zeros(size, np.uint8)
            ok.multi_layer_kv_transfer(want, table_np, slots.numpy(), pbs, True, False, 2, L, W, 2)
            _sync()
            assert np.array_equal(to_bytes(host), want)
        else:
            host.copy_(randn_bf16((2, L, T, W), gen))
            zero = [torch.zeros_like(t) for t in flat]
            ops.multi_layer_kv_transfer(host, ptr_table(zero, DEV), slots.to(DEV), torch.device(DEV), pbs, False,
                                        False, 2, W, W, 0)
            zero_np = [np.zeros_like(x) for x in table_np]
            ok.multi_layer_kv_transfer(to_bytes(host), zero_np, slots.numpy(), pbs, False, False, 2, L, W, 2)
            _sync()
            for z, zn in zip(zero, zero_np):
                assert np.array_equal(to_bytes(z), zn)
    finally:
        ops.free_pinned_numa_ptr(p, size)
    assert ops.get_device_ptr(p, 1) == 0


def test_numa_pinned_bad_node_is_refused(ops):
    with pytest.raises(RuntimeError, match="NUMA node"):
        ops.alloc_pinned_numa_ptr(4096, 1024)
    with pytest.raises(RuntimeError, match="binding the thread to NUMA node 1023 failed"):
        ops.alloc_pinned_numa_ptr(4096, 1023)  # no host has 1024 NUMA nodes


def test_unpinned_host_buffer_is_rejected(ops):
    layers = [torch.zeros((2, 8, 16, 2, 128), dtype=torch.bfloat16, device=DEV)]
    host = torch.zeros((2, 1, 16, 256), dtype=torch.bfloat16)  # pageable
    with pytest.raises(RuntimeError, match="no device address"):
        ops.multi_layer_kv_transfer(host, ptr_table(layers, DEV), torch.arange(16, device=DEV), torch.device(DEV),
                                    128, True, False, 1, 256, 256, 0)


def test_pci_bus_id(ops):
    bus = ops.get_gpu_pci_bus_id(0)
    assert ":" in bus


# ---------------------------------------------------------------------------
# single_layer_kv_transfer
# ---------------------------------------------------------------------------


def _tb(t: torch.Tensor) -> ok.TensorBytes:
    """Oracle view of a (possibly strided) tensor: bytes of its whole storage
    span from element 0, with its element strides."""
    base = t.untyped_storage()
    es = t.element_size()
    full = torch.empty(0, dtype=t.dtype, device=t.device).set_(base, 0, (base.nbytes() // es,), (1,))
    data = to_bytes(full)[t.storage_offset() * es:]
    return ok.TensorBytes(data, list(t.shape), list(t.stride()), es)


@pytest.mark.parametrize("num_tokens", [256, 500])
@pytest.mark.parametrize("num_heads", [8, 1])
@pytest.mark.parametrize("token_major", [True, False])
@pytest.mark.parametrize("two_major", [True, False])
def test_single_layer_merged(ops, num_tokens, num_heads, token_major, two_major):
    """tests/v1/test_mem_kernels.py:595-681."""
    gen = torch.Generator().manual_seed(num_tokens + num_heads * 3 + token_major * 5 + two_major * 7)
    NB, BS, D = 100, 16, 128
    W = num_heads * D
    cache = _paged(1, 1, NB, BS, num_heads, D, gen, two_major=two_major)[0]
    slots = torch.tensor(sample_slots(NB * BS, num_tokens, seed=num_tokens), dtype=torch.int64)
    shape = (num_tokens, 2, W) if token_major else (2, num_tokens, W)
    lmc = torch.zeros(shape, dtype=torch.bfloat16, device=DEV)
    ops.single_layer_kv_transfer(lmc, cache, slots.to(DEV), True, 1, token_major, two_major)
    want_lmc = ok.TensorBytes(np.zeros(lmc.numel() * 2, np.uint8), list(lmc.shape), list(lmc.stride()), 2)
    ok.single_layer_kv_transfer(want_lmc, [_tb(cache)], slots.numpy(), True, 1, token_major, two_major)
    _sync()
    assert np.array_equal(to_bytes(lmc), want_lmc.data)
    fresh = torch.zeros_like(cache)
    ops.single_layer_kv_transfer(lmc, fresh, slots.to(DEV), False, 1, token_major, two_major)
    zb = _tb(torch.zeros_like(cache).cpu())
    ok.single_layer_kv_transfer(want_lmc, [zb], slots.numpy(), False, 1, token_major, two_major)
    _sync()
    assert np.array_equal(to_bytes(fresh), zb.data)


@pytest.mark.parametrize("token_major", [True, False])
def test_single_layer_separate_strided_views(ops, token_major):
    """SEPARATE_KV with block-strided K/V views (every other block of a
    larger allocation) and a strided LMC view."""
    gen = torch.Generator().manual_seed(300 + token_major)
    NB, BS, H, D, T = 60, 16, 8, 128, 500
    W = H * D
    big_k = randn_bf16([2 * NB, BS, H, D], gen).to(DEV)
    big_v = randn_bf16([2 * NB, BS, H, D], gen).to(DEV)
    k, v = big_k[::2], big_v[::2]
    slots = torch.tensor(sample_slots(NB * BS, T, seed=11), dtype=torch.int64)
    big = torch.zeros((T + 8, 2, W) if token_major else (2, T + 8, W), dtype=torch.bfloat16, device=DEV)
    lmc = big[:T] if token_major else big[:, :T]
    ops.single_layer_kv_transfer(lmc, (k, v), slots.to(DEV), True, 2, token_major)
    want = _tb(big.cpu())
    want = ok.TensorBytes(want.data, list(lmc.shape), list(lmc.stride()), 2)
    ok.single_layer_kv_transfer(want, [_tb(k), _tb(v)], slots.numpy(), True, 2, token_major)
    _sync()
    assert np.array_equal(to_bytes(big), want.data)
    fk, fv = torch.zeros_like(big_k), torch.zeros_like(big_v)
    ops.single_layer_kv_transfer(lmc, (fk[::2], fv[::2]), slots.to(DEV), False, 2, token_major)
    _sync()
    sk, sv = k.reshape(-1, W), v.reshape(-1, W)
    gk, gv = fk[::2].reshape(-1, W), fv[::2].reshape(-1, W)
    s = slots.to(DEV)
    assert torch.equal(gk[s].view(torch.int16), sk[s].view(torch.int16))
    assert torch.equal(gv[s].view(torch.int16), sv[s].view(torch.int16))
    assert (fk[1::2].view(torch.int16) == 0).all() and (fv[1::2].view(torch.int16) == 0).all()


@pytest.mark.parametrize("fmt", [3, 4, 5, 6])
def test_single_layer_mla_dsa(ops, fmt):
    gen = torch.Generator().manual_seed(400 + fmt)
    NB, BS, T, N = 64, 16, 300, 320
    kH, vH, dsaH = 512, 64, 128
    widths = {3: [kH, vH], 5: [kH, vH], 4: [kH, vH, dsaH], 6: [dsaH]}[fmt]
    caches = tuple(randn_bf16([NB, BS, 1, w], gen).to(DEV) for w in widths)
    slots = torch.tensor(sample_slots(NB * BS, T, seed=fmt), dtype=torch.int64)
    lmc = torch.zeros(N * sum(widths), dtype=torch.bfloat16, device=DEV)
    ops.single_layer_kv_transfer(lmc, caches, slots.to(DEV), True, fmt)
    want = ok.TensorBytes(np.zeros(lmc.numel() * 2, np.uint8), [lmc.numel()], [1], 2)
    ok.single_layer_kv_transfer(want, [_tb(c) for c in caches], slots.numpy(), True, fmt)
    _sync()
    assert np.array_equal(to_bytes(lmc), want.data)
    fresh = tuple(torch.zeros_like(c) for c in caches)
    ops.single_layer_kv_transfer(lmc, fresh, slots.to(DEV), False, fmt)
    _sync()
    s = slots.to(DEV)
    for c, f, w in zip(caches, fresh, widths):
        assert torch.equal(c.reshape(-1, w)[s].view(torch.int16), f.reshape(-1, w)[s].view(torch.int16))


def test_single_layer_rejects_list(ops):
    with pytest.raises(RuntimeError, match="neither a Tensor nor a tuple"):
        ops.single_layer_kv_transfer(torch.zeros(4, device=DEV), [torch.zeros(4, device=DEV)],
                                     torch.zeros(1, dtype=torch.int64, device=DEV), True, 1)


def test_single_layer_bad_format_value_error(ops):
    with pytest.raises(ValueError, match="is not a KV cache format"):
        ops.single_layer_kv_transfer(torch.zeros(4, device=DEV), torch.zeros(4, device=DEV),
                                     torch.zeros(1, dtype=torch.int64, device=DEV), True, 0)


# ---------------------------------------------------------------------------
# Llama-3-8B shape, full size: size-independent properties
# ---------------------------------------------------------------------------


def test_llama8b_shape_full_size_round_trip(ops):
    """32 layers, 8x128 bf16, block 128, 2048-block pool per layer, 4096
    tokens in 16 chunks of 256 (4 requests, partial last blocks).  Store must
    equal torch's index_select gather, and retrieve into the zeroed touched
    slots must restore the pool bit for bit."""
    L, NB, BS, H, D = 32, 2048, 128, 8, 128
    W = H * D
    pbs = NB * BS
    torch.manual_seed(0)
    flat = []
    for _ in range(L):
        flat.append(torch.randn((NB, BS, H, D), device=DEV, dtype=torch.bfloat16))
        flat.append(torch.randn((NB, BS, H, D), device=DEV, dtype=torch.bfloat16))
    ptrs = ptr_table(flat, DEV)
    gen = torch.Generator().manual_seed(1)
    blocks = torch.randperm(NB, generator=gen).tolist()
    slots = torch.tensor(block_slots(blocks, BS, [1000, 1100, 996, 1000]), dtype=torch.int64, device=DEV)
    starts = list(range(0, 4096, 256))
    chunks = [torch.empty((2, L, 256, W), dtype=torch.bfloat16, device=DEV) for _ in starts]
    ops.multi_layer_kv_transfer_batched(chunks, ptrs, slots, starts, torch.device(DEV), pbs, True, False, 2, W, W, 0)
    _sync()
    for c, s0 in zip(chunks, starts):
        sl = slots[s0: s0 + 256]
        for l in (0, 13, 31):
            for p in range(2):
                want = flat[2 * l + p].reshape(-1, W).index_select(0, sl)
                assert torch.equal(c[p, l].view(torch.int16), want.view(torch.int16))
    checksum_before = [t.view(torch.int16).to(torch.int64).sum().item() for t in flat[:4]]
    saved = [t.reshape(-1, W)[slots].clone() for t in flat]
    for t in flat:
        t.reshape(-1, W)[slots] = 0
    ops.multi_layer_kv_transfer_batched(chunks, ptrs, slots, starts, torch.device(DEV), pbs, False, False, 2, W, W,
                                        0)
    _sync()
    for t, s in zip(flat, saved):
        assert torch.equal(t.reshape(-1, W)[slots].view(torch.int16), s.view(torch.int16))
    checksum_after = [t.view(torch.int16).to(torch.int64).sum().item() for t in flat[:4]]
    assert checksum_before == checksum_after


def test_llama8b_shape_full_size_pinned_round_trip(ops):
    """The same Llama-3-8B-shape batch with its 16 memory objects in
    page-locked host memory, one batched launch per direction (the
    pinned-host mode of the benchmark, kernel reads and writes over PCIe).
    Store: every object equals torch's index_select gather of all 32 layers
    and both planes.  Retrieve into the zeroed touched slots restores them
    and leaves the other rows' checksums unchanged."""
    L, NB, BS, H, D = 32, 2048, 128, 8, 128
    W = H * D
    pbs = NB * BS
    torch.manual_seed(2)
    flat = [torch.randn((NB, BS, H, D), device=DEV, dtype=torch.bfloat16) for _ in range(2 * L)]
    ptrs = ptr_table(flat, DEV)
    gen = torch.Generator().manual_seed(1)
    blocks = torch.randperm(NB, generator=gen).tolist()
    slots = torch.tensor(block_slots(blocks, BS, [1000, 1100, 996, 1000]), dtype=torch.int64, device=DEV)
    starts = list(range(0, 4096, 256))
    chunks = [torch.empty((2, L, 256, W), dtype=torch.bfloat16).pin_memory() for _ in starts]
    ops.multi_layer_kv_transfer_batched(chunks, ptrs, slots, starts, torch.device(DEV), pbs, True, False, 2, W, W, 0)
    _sync()
    for c, s0 in zip(chunks, starts):
        sl = slots[s0: s0 + 256]
        want = torch.stack([torch.stack([flat[2 * l + p].reshape(-1, W).index_select(0, sl) for l in range(L)])
                            for p in range(2)])
        assert torch.equal(c.to(DEV).view(torch.int16), want.view(torch.int16))
    checksum_before = [t.view(torch.int16).to(torch.int64).sum().item() for t in flat[:4]]
    saved = [t.reshape(-1, W)[slots].clone() for t in flat]
    for t in flat:
        t.reshape(-1, W)[slots] = 0
    ops.multi_layer_kv_transfer_batched(chunks, ptrs, slots, starts, torch.device(DEV), pbs, False, False, 2, W, W,
                                        0)
    _sync()
    for t, s in zip(flat, saved):
        assert torch.equal(t.reshape(-1, W)[slots].view(torch.int16), s.view(torch.int16))
    checksum_after = [t.view(torch.int16).to(torch.int64).sum().item() for t in flat[:4]]
    assert checksum_before == checksum_after
    del flat, chunks, saved
    torch.cuda.empty_cache()


def test_binding_and_ctypes_paths_agree(ops):
    """The C++ binding and the ctypes calls reach the same library functions
    and move the same bytes."""
    gen = torch.Generator().manual_seed(808)
    L, NB, BS, H, D, T = 4, 64, 16, 8, 128, 300
    W = H * D
    pbs = NB * BS
    layers = _paged(2, L, NB, BS, H, D, gen)
    flat = _flat_tensors(layers)
    ptrs = ptr_table(flat, DEV)
    slots = torch.tensor(sample_slots(pbs, T, seed=8), device=DEV)
    a = torch.zeros((2, L, T, W), dtype=torch.bfloat16, device=DEV)
    b = torch.zeros_like(a)
    assert ops._ext is not None, "the C++ binding was not built"
    ops.multi_layer_kv_transfer(a, ptrs, slots, torch.device(DEV), pbs, True, False, 2, W, W, 0)
    ops._multi_layer_kv_transfer_ctypes(b, ptrs, slots, torch.device(DEV), pbs, True, False, 2, W, W, 0)
    _sync()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    c = torch.zeros((2, T, W), dtype=torch.bfloat16, device=DEV)
    d = torch.zeros_like(c)
    ops.single_layer_kv_transfer(c, layers[1], slots, True, 2)
    ops._single_layer_kv_transfer_ctypes(d, layers[1], slots, True, 2)
    _sync()
    assert torch.equal(c.view(torch.int16), d.view(torch.int16))
    assert torch.equal(c.view(torch.int16), a[:, 1].view(torch.int16))


def test_zero_token_calls_leave_everything_unchanged(ops):
    """An empty slot mapping (a chunk with no tokens) is a no-op for every
    gather/scatter entry point, both directions, and for the K re-rotation:
    no launch, no error, caches and buffers unchanged."""
    gen = torch.Generator().manual_seed(21)
    L, NB, BS, H, D = 2, 8, 16, 2, 128
    W = H * D
    pbs = NB * BS
    layers = _paged(1, L, NB, BS, H, D, gen)
    ptrs = ptr_table(layers, DEV)
    before = [x.clone() for x in layers]
    none = torch.empty(0, dtype=torch.int64, device=DEV)
    kv = torch.empty((2, L, 0, W), dtype=torch.bfloat16, device=DEV)
    for direction in (True, False):
        ops.multi_layer_kv_transfer(kv, ptrs, none, torch.device(DEV), pbs, direction, False, 1, W, W, 0)
    ops.multi_layer_kv_transfer_batched([kv], ptrs, none, [0], torch.device(DEV), pbs, False, False, 1, W, W, 0)
    for l in range(L):
        ops.load_and_reshape_flash(kv, layers[l][0], layers[l][1], none, l)
        ops.reshape_and_cache_back_flash(kv, layers[l][0], layers[l][1], none, l)
        ops.single_layer_kv_transfer(torch.empty((2, 0, W), dtype=torch.bfloat16, device=DEV), layers[l],
                                     none, False, 1, vllm_two_major=True)
    key = torch.empty((0, W), dtype=torch.bfloat16, device=DEV)
    cache = torch.zeros((16, D), dtype=torch.bfloat16, device=DEV)
    ops.rotary_embedding_k_fused(none, none, key, D, cache, True)
    _sync()
    for a, b in zip(before, layers):
        assert torch.equal(a, b)
