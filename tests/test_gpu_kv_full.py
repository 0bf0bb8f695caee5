"""Full-size gather/scatter configurations on the GPU, checked through
size-independent properties: equality with torch's index_select gather on
sampled (chunk, layer, plane) slices, guard values left in rows whose slot
is -1, and bit-exact restoration of the pool after a retrieve into zeroed
touched slots."""

import pytest
import torch

from kvutil import block_slots, ptr_table

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def ops():
    import lmcache_amd

    return lmcache_amd.c_ops


def _eq(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_qwen32b_long_prefix_with_padding(ops):
    """64 layers x 8x128 bf16, block 128, 4096-block pool; one 32768-token
    request in 128 chunks of 256; 5% of slots are -1.  Multi-layer batched
    store/retrieve and single_layer_kv_transfer layer by layer."""
    L, NB, BS, H, D, T = 64, 4096, 128, 8, 128, 32768
    W = H * D
    torch.manual_seed(3)
    flat = [torch.randn((NB, BS, H, D), device=DEV, dtype=torch.bfloat16) for _ in range(2 * L)]
    ptrs = ptr_table(flat, DEV)
    gen = torch.Generator().manual_seed(3)
    blocks = torch.randperm(NB, generator=gen)[: T // BS].tolist()
    slots = torch.tensor(block_slots(blocks, BS, [T]), dtype=torch.int64)
    pad = torch.randperm(T, generator=gen)[: round(0.05 * T)]
    slots[pad] = -1
    slots = slots.to(DEV)
    valid_mask = slots >= 0
    valid = slots[valid_mask]
    starts = list(range(0, T, 256))
    guard = 0x7B7B
    chunks = [torch.full((2, L, 256, W), guard, dtype=torch.int16, device=DEV).view(torch.bfloat16) for _ in starts]
    ops.multi_layer_kv_transfer_batched(chunks, ptrs, slots, starts, torch.device(DEV), NB * BS, True, False, 2,
                                        W, W, 0)
    torch.cuda.synchronize()
    for ci in (0, 37, 127):
        sl = slots[starts[ci]: starts[ci] + 256]
        m = sl >= 0
        for l in (0, 31, 63):
            for p in range(2):
                rows = chunks[ci][p, l]
                want = flat[2 * l + p].reshape(-1, W).index_select(0, sl[m])
                assert _eq(rows[m], want)
                assert (rows[~m].view(torch.int16) == guard).all()
    saved = [t.reshape(-1, W).index_select(0, valid) for t in flat]
    for t in flat:
        t.reshape(-1, W)[valid] = 0
    ops.multi_layer_kv_transfer_batched(chunks, ptrs, slots, starts, torch.device(DEV), NB * BS, False, False, 2,
                                        W, W, 0)
    torch.cuda.synchronize()
    for t, s in zip(flat, saved):
        assert _eq(t.reshape(-1, W).index_select(0, valid), s)
    # single_layer_kv_transfer, layer by layer, [2, T, W] staging
    buf = torch.full((2, T, W), guard, dtype=torch.int16, device=DEV).view(torch.bfloat16)
    for l in (0, 17, 63):
        k, v = flat[2 * l], flat[2 * l + 1]
        ops.single_layer_kv_transfer(buf, (k, v), slots, True, 2)
        torch.cuda.synchronize()
        assert _eq(buf[0][valid_mask], k.reshape(-1, W).index_select(0, valid))
        assert _eq(buf[1][valid_mask], v.reshape(-1, W).index_select(0, valid))
        assert (buf[:, ~valid_mask].view(torch.int16) == guard).all()
        k.reshape(-1, W)[valid] = 0
        v.reshape(-1, W)[valid] = 0
        ops.single_layer_kv_transfer(buf, (k, v), slots, False, 2)
        torch.cuda.synchronize()
        assert _eq(k.reshape(-1, W).index_select(0, valid), saved[2 * l])
        assert _eq(v.reshape(-1, W).index_select(0, valid), saved[2 * l + 1])
    del flat, chunks, saved, buf
    torch.cuda.empty_cache()


def test_mla_576_full_size(ops):
    """61 layers of one [1024, 64, 576] bf16 latent tensor each (use_mla),
    8 requests x 2048 tokens, memory objects [1, 61, 2048, 576]."""
    L, NB, BS, W, NR, TR = 61, 1024, 64, 576, 8, 2048
    torch.manual_seed(4)
    caches = [torch.randn((NB, BS, W), device=DEV, dtype=torch.bfloat16) * 0.5 for _ in range(L)]
    ptrs = ptr_table(caches, DEV)
    gen = torch.Generator().manual_seed(4)
    blocks = torch.randperm(NB, generator=gen).tolist()
    slots = torch.tensor(block_slots(blocks, BS, [TR] * NR), dtype=torch.int64, device=DEV)
    starts = [i * TR for i in range(NR)]
    objs = [torch.empty((1, L, TR, W), dtype=torch.bfloat16, device=DEV) for _ in range(NR)]
    ops.multi_layer_kv_transfer_batched(objs, ptrs, slots, starts, torch.device(DEV), NB * BS, True, True, 1, 0, 0, 0)
    torch.cuda.synchronize()
    for r in (0, 7):
        sl = slots[starts[r]: starts[r] + TR]
        for l in (0, 30, 60):
            assert _eq(objs[r][0, l], caches[l].reshape(-1, W).index_select(0, sl))
    saved = [c.reshape(-1, W).index_select(0, slots) for c in caches]
    for c in caches:
        c.reshape(-1, W)[slots] = 0
    ops.multi_layer_kv_transfer_batched(objs, ptrs, slots, starts, torch.device(DEV), NB * BS, False, True, 1, 0, 0,
                                        0)
    torch.cuda.synchronize()
    for c, s in zip(caches, saved):
        assert _eq(c.reshape(-1, W).index_select(0, slots), s)
    del caches, objs, saved
    torch.cuda.empty_cache()
