"""GPU parity of the whole-row gather/scatter kernels, the flash ops and the
staged (fused) op against the CPU oracle.

Rows of 2 KiB and wider take the row kernels; which one runs depends on the
geometry (lean kernel: every plane the same power-of-two number of 2 KiB
slices, 16-byte access, power-of-two block size; otherwise the general row
kernel).  Each case below is chosen to land on one of them: 2 KiB and 4 KiB
rows, 6 KiB rows (three slices), block sizes 16 and 48, memory objects
offset by 8 or 2 bytes (8- and 2-byte accesses), a pointer-table entry that
is only 2-byte aligned (the byte path), one, two and three planes, empty
chunks inside a batch.  Every case runs int32 and int64 slot mappings with
-1 padding and out-of-range slots mixed in, and checks guard bytes around
every buffer the op writes.

load_and_reshape_flash / reshape_and_cache_back_flash
(csrc/mem_kernels.cpp:1341-1440) and fused_multi_layer_kv_transfer
(csrc/mem_kernels.cpp:113-213) are compared with the oracle at the 4-layer
256-token plumbing shape and at one Llama-3-8B-shape layer (4096 tokens,
block 128), for MERGED and SEPARATE caches.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvutil import ptr_table, randn_bf16, sample_slots, to_bytes
from oracle import kv_transfer as ok

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
GUARD = 173
PAD = 4096


@pytest.fixture(scope="module")
def ops():
    import lmcache_amd

    return lmcache_amd.c_ops


def _sync():
    torch.cuda.synchronize()


class Guarded:
    """A byte buffer with PAD guard bytes on each side of a window that
    starts `offset` bytes past the left pad."""

    def __init__(self, nbytes: int, offset: int = 0, device=DEV, pinned=False, fill=None):
        total = nbytes + 2 * PAD + offset
        if device == "cpu":
            self.buf = torch.full((total,), GUARD, dtype=torch.uint8)
            if pinned:
                self.buf = self.buf.pin_memory()
        else:
            self.buf = torch.full((total,), GUARD, dtype=torch.uint8, device=device)
        self.lo = PAD + offset
        self.hi = self.lo + nbytes
        self.window = self.buf[self.lo: self.hi]
        if fill is not None:
            self.window.copy_(fill.reshape(-1).view(torch.uint8))

    def view(self, shape, dtype=torch.bfloat16):
        return self.window.view(dtype).view(shape)

    def guards_intact(self) -> bool:
        b = self.buf.cpu().numpy()
        return bool((b[: self.lo] == GUARD).all() and (b[self.hi:] == GUARD).all())

    def bytes(self) -> np.ndarray:
        return self.window.cpu().numpy().copy()


def _slots(n_slots: int, n: int, seed: int, dtype) -> torch.Tensor:
    """Distinct valid slots, with about 5% -1 padding and 2% out of range."""
    s = np.array(sample_slots(n_slots, n, seed=seed), dtype=np.int64)
    rng = np.random.default_rng(seed)
    pick = rng.permutation(n)
    s[pick[: max(1, n // 20)]] = -1
    big = np.iinfo(np.int32).max if dtype == torch.int32 else (1 << 40)
    oor = pick[max(1, n // 20): max(1, n // 20) + max(1, n // 50)]
    s[oor[::2]] = n_slots
    s[oor[1::2]] = big
    return torch.tensor(s, dtype=dtype)


# ---------------------------------------------------------------------------
# multi_layer_kv_transfer through the row kernels
# ---------------------------------------------------------------------------


def _mk_planes(fmt, L, NB, BS, W, gen):
    if fmt == 1:
        return [randn_bf16([2, NB, BS, W // 128, 128], gen).to(DEV) for _ in range(L)]
    return [randn_bf16([NB, BS, W // 128, 128], gen).to(DEV) for _ in range(2 * L)]


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("heads", [8, 16, 24])  # 2, 4 and 6 KiB rows
@pytest.mark.parametrize("lmc_offset", [0, 8, 2])
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_multi_layer_rows_vs_oracle(ops, fmt, heads, lmc_offset, slot_dtype):
    gen = torch.Generator().manual_seed(fmt * 1000 + heads * 10 + lmc_offset)
    L, NB, BS, T = 3, 32, 16, 301
    W = heads * 128
    pbs = NB * BS
    tens = _mk_planes(fmt, L, NB, BS, W, gen)
    ptrs = ptr_table(tens, DEV)
    slots = _slots(pbs, T, seed=heads + lmc_offset, dtype=slot_dtype)
    nbytes = 2 * L * T * W * 2
    g = Guarded(nbytes, lmc_offset)
    lmc = g.view((2, L, T, W))
    ops.multi_layer_kv_transfer(lmc, ptrs, slots.to(DEV), torch.device(DEV), pbs, True, False, fmt, W, W, 0)
    table_np = [to_bytes(t) for t in tens]
    want = np.full(nbytes, GUARD, np.uint8)
    ok.multi_layer_kv_transfer(want, table_np, slots.numpy().astype(np.int64), pbs, True, False, fmt, L, W, 2)
    _sync()
    assert np.array_equal(g.bytes(), want)
    assert g.guards_intact()
    # retrieve into guard-filled caches: untouched rows keep the guard value
    filled = [torch.full_like(t.view(torch.uint8), GUARD).view(torch.bfloat16) for t in tens]
    src = randn_bf16((2, L, T, W), gen)
    g2 = Guarded(nbytes, lmc_offset, fill=src.to(DEV))
    ops.multi_layer_kv_transfer(g2.view((2, L, T, W)), ptr_table(filled, DEV), slots.to(DEV),
                                torch.device(DEV), pbs, False, False, fmt, W, W, 0)
    want_t = [np.full(t.numel() * 2, GUARD, np.uint8) for t in tens]
    ok.multi_layer_kv_transfer(to_bytes(src), want_t, slots.numpy().astype(np.int64), pbs, False, False, fmt,
                               L, W, 2)
    _sync()
    for f, w in zip(filled, want_t):
        assert np.array_equal(to_bytes(f), w)
    assert g2.guards_intact()


@pytest.mark.parametrize("fmt,widths", [(4, [1024, 1024, 1024]), (6, [1024]), (3, [1024, 1024]),
                                        (4, [2048, 2048, 2048])])
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_multi_layer_concatenated_planes_rows_vs_oracle(ops, fmt, widths, slot_dtype):
    """MLA/DSA memory objects [1, L, T, sum(W)] whose planes are whole 2 KiB
    slices: one, two and three planes per token in the lean kernel."""
    gen = torch.Generator().manual_seed(fmt * 77 + len(widths) + widths[0])
    L, NB, BS, T = 3, 24, 16, 200
    pbs = NB * BS
    tens = [randn_bf16([NB, BS, 1, w], gen).to(DEV) for _ in range(L) for w in widths]
    kH, vH, dsaH = (widths + [0, 0])[:3] if fmt != 6 else (0, 0, widths[0])
    wsum = sum(widths)
    slots = _slots(pbs, T, seed=fmt + wsum, dtype=slot_dtype)
    nbytes = L * T * wsum * 2
    g = Guarded(nbytes)
    ops.multi_layer_kv_transfer(g.view((1, L, T, wsum)), ptr_table(tens, DEV), slots.to(DEV), torch.device(DEV),
                                pbs, True, False, fmt, kH, vH, dsaH)
    want = np.full(nbytes, GUARD, np.uint8)
    table_np = [to_bytes(t) for t in tens]
    ok.multi_layer_kv_transfer(want, table_np, slots.numpy().astype(np.int64), pbs, True, False, fmt, L, wsum, 2,
                               kH, vH, dsaH)
    _sync()
    assert np.array_equal(g.bytes(), want)
    assert g.guards_intact()
    filled = [torch.full_like(t.view(torch.uint8), GUARD).view(torch.bfloat16) for t in tens]
    ops.multi_layer_kv_transfer(g.view((1, L, T, wsum)), ptr_table(filled, DEV), slots.to(DEV), torch.device(DEV),
                                pbs, False, False, fmt, kH, vH, dsaH)
    want_t = [np.full(t.numel() * 2, GUARD, np.uint8) for t in tens]
    ok.multi_layer_kv_transfer(want, want_t, slots.numpy().astype(np.int64), pbs, False, False, fmt, L, wsum, 2,
                               kH, vH, dsaH)
    _sync()
    for f, w in zip(filled, want_t):
        assert np.array_equal(to_bytes(f), w)


def test_multi_layer_misaligned_table_entry_takes_byte_path(ops):
    """A pointer-table entry 2 bytes past an allocation's start (a device
    value the host cannot check) is copied byte by byte, still exactly."""
    gen = torch.Generator().manual_seed(9)
    L, NB, BS, W, T = 2, 16, 16, 1024, 120
    pbs = NB * BS
    plane_bytes = pbs * W * 2
    raw = [torch.full((plane_bytes + 64,), GUARD, dtype=torch.uint8, device=DEV) for _ in range(2 * L)]
    for r in raw:
        r[2: 2 + plane_bytes].copy_(randn_bf16([plane_bytes // 2], gen).view(torch.uint8).to(DEV))
    ptrs = torch.tensor([r.data_ptr() + 2 for r in raw], dtype=torch.int64, device=DEV)
    slots = _slots(pbs, T, seed=5, dtype=torch.int64)
    g = Guarded(2 * L * T * W * 2)
    ops.multi_layer_kv_transfer(g.view((2, L, T, W)), ptrs, slots.to(DEV), torch.device(DEV), pbs, True, False, 2,
                                W, W, 0)
    table_np = [r.cpu().numpy()[2: 2 + plane_bytes].copy() for r in raw]
    want = np.full(2 * L * T * W * 2, GUARD, np.uint8)
    ok.multi_layer_kv_transfer(want, table_np, slots.numpy(), pbs, True, False, 2, L, W, 2)
    _sync()
    assert np.array_equal(g.bytes(), want)
    assert g.guards_intact()
    # retrieve into the same (2-byte offset) caches, cleared
    for r in raw:
        r.fill_(GUARD)
    ops.multi_layer_kv_transfer(g.view((2, L, T, W)), ptrs, slots.to(DEV), torch.device(DEV), pbs, False, False, 2,
                                W, W, 0)
    want_t = [np.full(plane_bytes, GUARD, np.uint8) for _ in raw]
    ok.multi_layer_kv_transfer(want, want_t, slots.numpy(), pbs, False, False, 2, L, W, 2)
    _sync()
    for r, w in zip(raw, want_t):
        b = r.cpu().numpy()
        assert np.array_equal(b[2: 2 + plane_bytes], w)
        assert (b[:2] == GUARD).all() and (b[2 + plane_bytes:] == GUARD).all()


@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_batched_with_empty_chunks_vs_oracle(ops, slot_dtype):
    """A batch whose memory objects include zero-token ones, in the middle
    and at the end; every object equals the oracle's single-chunk result."""
    gen = torch.Generator().manual_seed(12)
    L, NB, BS, W = 4, 32, 16, 1024
    pbs = NB * BS
    tens = _mk_planes(2, L, NB, BS, W, gen)
    ptrs = ptr_table(tens, DEV)
    counts = [100, 0, 77, 256, 0]
    starts = [0, 100, 100, 177, 433]
    slots = _slots(pbs, 433, seed=3, dtype=slot_dtype)
    objs = [Guarded(2 * L * max(c, 0) * W * 2) for c in counts]
    views = [o.view((2, L, c, W)) for o, c in zip(objs, counts)]
    ops.multi_layer_kv_transfer_batched(views, ptrs, slots.to(DEV), starts, torch.device(DEV), pbs, True, False, 2,
                                        W, W, 0)
    table_np = [to_bytes(t) for t in tens]
    _sync()
    for o, c, s in zip(objs, counts, starts):
        want = np.full(2 * L * c * W * 2, GUARD, np.uint8)
        ok.multi_layer_kv_transfer(want, table_np, slots.numpy().astype(np.int64)[s: s + c], pbs, True, False, 2,
                                   L, W, 2)
        assert np.array_equal(o.bytes(), want)
        assert o.guards_intact()


# ---------------------------------------------------------------------------
# single_layer_kv_transfer through the row kernels
# ---------------------------------------------------------------------------


def _tb(t: torch.Tensor) -> ok.TensorBytes:
    base = t.untyped_storage()
    es = t.element_size()
    full = torch.empty(0, dtype=t.dtype, device=t.device).set_(base, 0, (base.nbytes() // es,), (1,))
    data = to_bytes(full)[t.storage_offset() * es:]
    return ok.TensorBytes(data, list(t.shape), list(t.stride()), es)


@pytest.mark.parametrize("fmt,two_major", [(1, True), (1, False), (2, False)])
@pytest.mark.parametrize("block_size", [16, 48])
@pytest.mark.parametrize("heads", [8, 24])
@pytest.mark.parametrize("token_major", [True, False])
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_single_layer_rows_vs_oracle(ops, fmt, two_major, block_size, heads, token_major, slot_dtype):
    gen = torch.Generator().manual_seed(block_size + heads * 3 + token_major * 5 + two_major * 7 + fmt)
    NB, D, T = 20, 128, 203
    W = heads * D
    if fmt == 1:
        shape = [2, NB, block_size, heads, D] if two_major else [NB, 2, block_size, heads, D]
        caches = randn_bf16(shape, gen).to(DEV)
        cache_list = [caches]
    else:
        caches = (randn_bf16([NB, block_size, heads, D], gen).to(DEV),
                  randn_bf16([NB, block_size, heads, D], gen).to(DEV))
        cache_list = list(caches)
    slots = _slots(NB * block_size, T, seed=heads + block_size, dtype=slot_dtype)
    shape = (T, 2, W) if token_major else (2, T, W)
    g = Guarded(2 * T * W * 2)
    lmc = g.view(shape)
    ops.single_layer_kv_transfer(lmc, caches, slots.to(DEV), True, fmt, token_major, two_major)
    want = ok.TensorBytes(np.full(2 * T * W * 2, GUARD, np.uint8), list(shape), list(lmc.stride()), 2)
    ok.single_layer_kv_transfer(want, [_tb(c) for c in cache_list], slots.numpy().astype(np.int64), True, fmt,
                                token_major, two_major)
    _sync()
    assert np.array_equal(g.bytes(), want.data)
    assert g.guards_intact()
    filled = [torch.full_like(c.view(torch.uint8), GUARD).view(torch.bfloat16) for c in cache_list]
    arg = filled[0] if fmt == 1 else tuple(filled)
    ops.single_layer_kv_transfer(lmc, arg, slots.to(DEV), False, fmt, token_major, two_major)
    want_c = [_tb(f.cpu()) for f in filled]
    ok.single_layer_kv_transfer(want, want_c, slots.numpy().astype(np.int64), False, fmt, token_major, two_major)
    _sync()
    for f, w in zip(filled, want_c):
        assert np.array_equal(to_bytes(f), w.data)


# ---------------------------------------------------------------------------
# load_and_reshape_flash / reshape_and_cache_back_flash against the oracle
# ---------------------------------------------------------------------------


FLASH_SHAPES = {
    # name: (layers in the memory object, tokens, blocks, block size, heads);
    # the op moves layer 1 of the object.
    "plumbing_4L_256": (4, 256, 64, 16, 8),
    "llama8b_layer_4096": (2, 4096, 512, 128, 8),
}


@pytest.mark.parametrize("shape", list(FLASH_SHAPES))
@pytest.mark.parametrize("merged", [True, False])
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_flash_vs_oracle(ops, shape, merged, slot_dtype):
    L, T, NB, BS, H = FLASH_SHAPES[shape]
    D, W = 128, H * 128
    gen = torch.Generator().manual_seed(T + merged * 3 + (slot_dtype == torch.int32))
    layer = 1 if L > 1 else 0
    if merged:
        kvc = randn_bf16([2, NB, BS, H, D], gen).to(DEV)
        kc, vc = kvc[0], kvc[1]
    else:
        kc = randn_bf16([NB, BS, H, D], gen).to(DEV)
        vc = randn_bf16([NB, BS, H, D], gen).to(DEV)
    slots = _slots(NB * BS, T, seed=T + 1, dtype=slot_dtype)
    nbytes = 2 * L * T * W * 2
    g = Guarded(nbytes)
    kv = g.view((2, L, T, W))
    ops.load_and_reshape_flash(kv, kc, vc, slots.to(DEV), layer)
    want = np.full(nbytes, GUARD, np.uint8)
    ok.load_and_reshape_flash(want, L, W, 2, to_bytes(kc), to_bytes(vc), slots.numpy().astype(np.int64), layer,
                              page2lmc=True)
    _sync()
    assert np.array_equal(g.bytes(), want)
    assert g.guards_intact()
    # reshape back into guard-filled caches from a fresh random object
    src = randn_bf16((2, L, T, W), gen)
    g2 = Guarded(nbytes, fill=src.to(DEV))
    if merged:
        f = torch.full_like(kvc.view(torch.uint8), GUARD).view(torch.bfloat16)
        fk, fv = f[0], f[1]
    else:
        fk = torch.full_like(kc.view(torch.uint8), GUARD).view(torch.bfloat16)
        fv = torch.full_like(vc.view(torch.uint8), GUARD).view(torch.bfloat16)
    ops.reshape_and_cache_back_flash(g2.view((2, L, T, W)), fk, fv, slots.to(DEV), layer)
    wk = np.full(kc.numel() * 2, GUARD, np.uint8)
    wv = np.full(vc.numel() * 2, GUARD, np.uint8)
    ok.load_and_reshape_flash(to_bytes(src), L, W, 2, wk, wv, slots.numpy().astype(np.int64), layer,
                              page2lmc=False)
    _sync()
    assert np.array_equal(to_bytes(fk), wk)
    assert np.array_equal(to_bytes(fv), wv)
    assert g2.guards_intact()


# ---------------------------------------------------------------------------
# fused_multi_layer_kv_transfer against the oracle
# ---------------------------------------------------------------------------


FUSED_SHAPES = {
    "plumbing_4L_256": (4, 256, 64, 16, 8),
    "llama8b_2L_4096": (2, 4096, 512, 128, 8),
}


@pytest.mark.parametrize("shape", list(FUSED_SHAPES))
@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_fused_vs_oracle(ops, shape, fmt, slot_dtype):
    """The staged op's host object and staging buffer both end as the
    oracle's memory object (store); the caches end as the oracle's retrieve
    (load).  The staging buffer is a sliced view inside a guarded buffer."""
    L, T, NB, BS, H = FUSED_SHAPES[shape]
    W = H * 128
    pbs = NB * BS
    gen = torch.Generator().manual_seed(L * 11 + fmt + T)
    tens = _mk_planes(fmt, L, NB, BS, W, gen)
    slots = _slots(pbs, T, seed=fmt + T, dtype=slot_dtype)
    nbytes = 2 * L * T * W * 2
    table_np = [to_bytes(t) for t in tens]
    # store: paged -> staging -> pinned host object
    stg = Guarded(nbytes + 2 * L * 16 * W * 2)  # room for a larger chunk
    staging = stg.view((2, L, T + 16, W))[:, :, :T, :]
    host = Guarded(nbytes, device="cpu", pinned=True)
    ops.fused_multi_layer_kv_transfer(host.view((2, L, T, W)), staging, ptr_table(tens, DEV), slots.to(DEV),
                                      torch.device(DEV), pbs, True, False, fmt, W, W, 0)
    want = np.full(nbytes, GUARD, np.uint8)
    ok.multi_layer_kv_transfer(want, table_np, slots.numpy().astype(np.int64), pbs, True, False, fmt, L, W, 2)
    _sync()
    assert np.array_equal(host.bytes(), want)
    assert host.guards_intact()
    assert np.array_equal(stg.bytes()[:nbytes], want)
    assert stg.guards_intact()
    # load: pinned host object -> staging -> paged
    src = randn_bf16((2, L, T, W), gen)
    host2 = Guarded(nbytes, device="cpu", pinned=True, fill=src)
    filled = [torch.full_like(t.view(torch.uint8), GUARD).view(torch.bfloat16) for t in tens]
    stg2 = Guarded(nbytes)
    ops.fused_multi_layer_kv_transfer(host2.view((2, L, T, W)), stg2.view((2, L, T, W)), ptr_table(filled, DEV),
                                      slots.to(DEV), torch.device(DEV), pbs, False, False, fmt, W, W, 0)
    want_t = [np.full(t.numel() * 2, GUARD, np.uint8) for t in tens]
    ok.multi_layer_kv_transfer(to_bytes(src), want_t, slots.numpy().astype(np.int64), pbs, False, False, fmt, L,
                               W, 2)
    _sync()
    for f, w in zip(filled, want_t):
        assert np.array_equal(to_bytes(f), w)
    assert stg2.guards_intact()


# ---------------------------------------------------------------------------
# multi_layer_kv_transfer_batched over page-locked host memory objects
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_batched_pinned_vs_oracle(ops, fmt, slot_dtype):
    """Five memory objects in page-locked host memory, one launch per
    direction: the general row kernel with plain cache hints over several
    objects, the launch the pinned-host benchmark mode times.  An empty
    object sits mid-batch and a one-token object at the end.  Store: every
    object equals the oracle's single-chunk result, guard bytes intact.
    Retrieve: caches filled with the guard value end as the oracle's."""
    gen = torch.Generator().manual_seed(40 + fmt)
    L, NB, BS, W = 4, 64, 16, 1024
    pbs = NB * BS
    tens = _mk_planes(fmt, L, NB, BS, W, gen)
    counts = [256, 0, 77, 100, 1]
    starts = [0, 256, 256, 333, 433]
    slots = _slots(pbs, 434, seed=50 + fmt, dtype=slot_dtype)
    s64 = slots.numpy().astype(np.int64)
    objs = [Guarded(2 * L * c * W * 2, device="cpu", pinned=True) for c in counts]
    views = [o.view((2, L, c, W)) for o, c in zip(objs, counts)]
    ops.multi_layer_kv_transfer_batched(views, ptr_table(tens, DEV), slots.to(DEV), starts, torch.device(DEV), pbs,
                                        True, False, fmt, W, W, 0)
    table_np = [to_bytes(t) for t in tens]
    _sync()
    for o, c, s in zip(objs, counts, starts):
        want = np.full(2 * L * c * W * 2, GUARD, np.uint8)
        ok.multi_layer_kv_transfer(want, table_np, s64[s: s + c], pbs, True, False, fmt, L, W, 2)
        assert np.array_equal(o.bytes(), want)
        assert o.guards_intact()
    srcs = [randn_bf16((2, L, c, W), gen) for c in counts]
    objs2 = [Guarded(2 * L * c * W * 2, device="cpu", pinned=True, fill=x) for x, c in zip(srcs, counts)]
    views2 = [o.view((2, L, c, W)) for o, c in zip(objs2, counts)]
    filled = [torch.full_like(t.view(torch.uint8), GUARD).view(torch.bfloat16) for t in tens]
    ops.multi_layer_kv_transfer_batched(views2, ptr_table(filled, DEV), slots.to(DEV), starts, torch.device(DEV),
                                        pbs, False, False, fmt, W, W, 0)
    want_t = [np.full(t.numel() * 2, GUARD, np.uint8) for t in tens]
    for x, c, s in zip(srcs, counts, starts):
        ok.multi_layer_kv_transfer(to_bytes(x), want_t, s64[s: s + c], pbs, False, False, fmt, L, W, 2)
    _sync()
    for f, w in zip(filled, want_t):
        assert np.array_equal(to_bytes(f), w)
    for o, x in zip(objs2, srcs):
        assert np.array_equal(o.bytes(), to_bytes(x)) and o.guards_intact()


# ---------------------------------------------------------------------------
# fused_multi_layer_kv_transfer for the MLA / DSA formats and use_mla
# ---------------------------------------------------------------------------


FUSED_FORMATS = {
    # name: (format, use_mla, row widths of the planes each layer points to)
    "mla_kv": (3, False, [512, 64]),
    "dsa_kv": (4, False, [512, 64, 128]),
    "mla_latent": (5, False, [512, 64]),
    "dsa_index": (6, False, [128]),
    "use_mla_merged": (1, True, [576]),
    "use_mla_separate": (2, True, [576]),
}


@pytest.mark.parametrize("case", list(FUSED_FORMATS))
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_fused_formats_vs_oracle(ops, case, slot_dtype):
    """The staged op sizes its staging copy per format
    (csrc/mem_kernels.cpp:143-165): L * T * (kH + vH (+ dsaH)) elements for
    the MLA / DSA formats, L * T * W for use_mla single-plane caches.  The
    staging buffer is a sliced view inside a guarded buffer with room to
    spare: store leaves the oracle's object in the host object and in the
    first `required` staging bytes and nothing after them; load scatters the
    host object into caches filled with the guard value."""
    fmt, use_mla, widths = FUSED_FORMATS[case]
    kH, vH, dsaH = (0, 0, 0) if use_mla else (512, 64, 128)
    gen = torch.Generator().manual_seed(60 + fmt * 3 + use_mla)
    L, NB, BS, T = 4, 64, 16, 300
    pbs = NB * BS
    wsum = sum(widths)
    tens = [randn_bf16([NB, BS, 1, w], gen).to(DEV) for _ in range(L) for w in widths]
    table_np = [to_bytes(t) for t in tens]
    slots = _slots(pbs, T, seed=70 + fmt, dtype=slot_dtype)
    s64 = slots.numpy().astype(np.int64)
    required = L * T * wsum * 2
    spare = L * 16 * wsum * 2
    stg = Guarded(required + spare)
    staging = stg.view((1, L, T + 16, wsum))[:, :, :T, :]
    host = Guarded(required, device="cpu", pinned=True)
    ops.fused_multi_layer_kv_transfer(host.view((1, L, T, wsum)), staging, ptr_table(tens, DEV), slots.to(DEV),
                                      torch.device(DEV), pbs, True, use_mla, fmt, kH, vH, dsaH)
    want = np.full(required, GUARD, np.uint8)
    ok.multi_layer_kv_transfer(want, table_np, s64, pbs, True, use_mla, fmt, L, wsum, 2, kH, vH, dsaH)
    _sync()
    assert np.array_equal(host.bytes(), want)
    assert host.guards_intact()
    sb = stg.bytes()
    assert np.array_equal(sb[:required], want)
    assert (sb[required:] == GUARD).all()
    assert stg.guards_intact()
    src = randn_bf16((1, L, T, wsum), gen)
    host2 = Guarded(required, device="cpu", pinned=True, fill=src)
    filled = [torch.full_like(t.view(torch.uint8), GUARD).view(torch.bfloat16) for t in tens]
    stg2 = Guarded(required + spare)
    staging2 = stg2.view((1, L, T + 16, wsum))[:, :, :T, :]
    ops.fused_multi_layer_kv_transfer(host2.view((1, L, T, wsum)), staging2, ptr_table(filled, DEV), slots.to(DEV),
                                      torch.device(DEV), pbs, False, use_mla, fmt, kH, vH, dsaH)
    want_t = [np.full(t.numel() * 2, GUARD, np.uint8) for t in tens]
    ok.multi_layer_kv_transfer(to_bytes(src), want_t, s64, pbs, False, use_mla, fmt, L, wsum, 2, kH, vH, dsaH)
    _sync()
    for f, w in zip(filled, want_t):
        assert np.array_equal(to_bytes(f), w)
    assert np.array_equal(stg2.bytes()[:required], to_bytes(src))
    assert stg2.guards_intact()
