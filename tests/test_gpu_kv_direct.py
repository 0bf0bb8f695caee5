"""GPU parity of the sparse, direct and staged-batch single-layer transfers
against the CPU oracle (oracle/kv_transfer.py), through the C ABI.

Shapes follow the reference's tests (tests/v1/test_mem_kernels.py:791-1543;
tests/v1/test_sparse_direct_kernel_minimal.py) at sizes the oracle finishes
in seconds; memory objects of the direct paths are page-locked host tensors
read and written by the GPU over PCIe.  Results are compared bit for bit,
including rows that must stay untouched (skipped slots, padding entries).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvutil import randn_bf16, to_bytes
from oracle import kv_transfer as ok

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def ops():
    import lmcache_amd

    return lmcache_amd.c_ops


def tb(t: torch.Tensor) -> ok.TensorBytes:
    """Oracle view (bytes + geometry) of a contiguous tensor."""
    assert t.is_contiguous()
    return ok.TensorBytes(to_bytes(t), list(t.shape), list(t.stride()), t.element_size())


def same(t: torch.Tensor, b: ok.TensorBytes) -> bool:
    return np.array_equal(to_bytes(t), b.data)


def pinned(shape, gen, dtype=torch.bfloat16):
    x = torch.empty(shape, dtype=dtype, pin_memory=True)
    x.copy_(randn_bf16(shape, gen).to(dtype))
    return x


def mla_caches(gen, NB=32, BS=16, widths=(512, 64)):
    return tuple(randn_bf16([NB, BS, 1, w], gen).to(DEV) for w in widths)


def paged_caches(fmt, gen, NB=32, BS=16, H=4, D=64, two_major=False):
    if fmt == ok.MERGED_KV:
        return (randn_bf16([2, NB, BS, H, D] if two_major else [NB, 2, BS, H, D], gen).to(DEV),)
    if fmt == ok.SEPARATE_KV:
        return (randn_bf16([NB, BS, H, D], gen).to(DEV), randn_bf16([NB, BS, H, D], gen).to(DEV))
    if fmt == ok.DSA_KV:
        return mla_caches(gen, NB, BS, (512, 64, 128))
    if fmt == ok.DSA_INDEX:
        return mla_caches(gen, NB, BS, (128,))
    return mla_caches(gen, NB, BS)


def plane_elems(fmt, caches):
    if fmt in (ok.MERGED_KV, ok.SEPARATE_KV):
        return 2 * caches[0].shape[-2] * caches[0].shape[-1]
    return sum(c.shape[-1] for c in caches)


def arg_caches(caches):
    return caches[0] if len(caches) == 1 else caches


# ---------------------------------------------------------------------------
# sparse_single_layer_kv_transfer
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("num_lmc_tokens,num_sparse", [(256, 64), (512, 512)])
def test_sparse_single_layer_reference_mla_case(ops, num_lmc_tokens, num_sparse):
    """tests/v1/test_mem_kernels.py:1445-1543: staging filled by a
    single-layer store, then a sparse scatter into other slots."""
    g = torch.Generator().manual_seed(num_sparse)
    src, dst = mla_caches(g, NB=64), mla_caches(g, NB=64)
    NBBS = 64 * 16
    full = torch.randperm(NBBS, generator=g)[:num_lmc_tokens].to(DEV)
    staging = torch.empty(num_lmc_tokens * 576, dtype=torch.bfloat16, device=DEV)
    ops.single_layer_kv_transfer(staging, src, full, True, 3, False, False, 0, 0, 0)
    sel = torch.randperm(num_lmc_tokens, generator=g)[:num_sparse].to(torch.int32).to(DEV)
    slots = torch.randperm(NBBS, generator=g)[:num_sparse].to(DEV)
    want = [tb(c) for c in dst]
    ok.sparse_single_layer_kv_transfer(tb(staging), want, slots.cpu().numpy(), sel.cpu().numpy(), ok.MLA_KV)
    ops.sparse_single_layer_kv_transfer(staging, dst, slots, sel, 3, False, False, 0, 0, 0)
    torch.cuda.synchronize()
    for c, w in zip(dst, want):
        assert same(c, w)
    k_src, v_src = src[0].reshape(-1, 512), src[1].reshape(-1, 64)
    k_dst, v_dst = dst[0].reshape(-1, 512), dst[1].reshape(-1, 64)
    for i in range(0, num_sparse, 7):
        s_src, s_dst = full[sel[i]].item(), slots[i].item()
        assert torch.equal(k_dst[s_dst], k_src[s_src]) and torch.equal(v_dst[s_dst], v_src[s_src])


@pytest.mark.parametrize(
    "fmt,token_major,two_major",
    [(1, False, False), (1, True, True), (1, False, True), (2, False, False), (2, True, False),
     (3, False, False), (4, False, False), (5, False, False), (6, False, False)],
)
@pytest.mark.parametrize("two_d", [False, True])
def test_sparse_single_layer_formats(ops, fmt, token_major, two_major, two_d):
    g = torch.Generator().manual_seed(fmt * 10 + token_major + 2 * two_major)
    caches = paged_caches(fmt, g, two_major=two_major)
    N, n = 96, 64
    pe = plane_elems(fmt, caches)
    if fmt in (ok.MERGED_KV, ok.SEPARATE_KV):
        W = pe // 2
        lmc = randn_bf16([N, 2, W] if token_major else [2, N, W], g).to(DEV)
    else:
        lmc = randn_bf16([N * pe], g).to(DEV)
    sel = torch.randint(0, N, (n,), generator=g, dtype=torch.int32)
    sel[5], sel[9] = N + 3, -2                      # out of range: skipped
    slots = torch.randperm(32 * 16, generator=g)[:n]
    slots[11] = -1
    if two_d:
        sel, slots = sel.reshape(4, 16), slots.reshape(4, 16)
    sel, slots = sel.to(DEV), slots.to(torch.int32 if fmt % 2 else torch.int64).to(DEV)
    want = [tb(c) for c in caches]
    ok.sparse_single_layer_kv_transfer(tb(lmc), want, slots.cpu().numpy(), sel.cpu().numpy(), fmt, token_major,
                                       two_major)
    ops.sparse_single_layer_kv_transfer(lmc, arg_caches(caches), slots, sel, fmt, token_major, two_major)
    torch.cuda.synchronize()
    for c, w in zip(caches, want):
        assert same(c, w)


def test_sparse_single_layer_errors(ops):
    g = torch.Generator().manual_seed(0)
    caches = mla_caches(g)
    lmc = torch.zeros(64 * 576, dtype=torch.bfloat16, device=DEV)
    s1 = torch.zeros(8, dtype=torch.int64, device=DEV)
    with pytest.raises(ValueError, match="one is 1-D and the other 2-D"):
        ops.sparse_single_layer_kv_transfer(lmc, caches, s1, torch.zeros((2, 4), dtype=torch.int32, device=DEV), 3)
    with pytest.raises(ValueError, match="differ in shape"):
        ops.sparse_single_layer_kv_transfer(lmc, caches, s1, torch.zeros(7, dtype=torch.int32, device=DEV), 3)
    with pytest.raises(ValueError, match="holds int32 token indices"):
        ops.sparse_single_layer_kv_transfer(lmc, caches, s1, torch.zeros(8, dtype=torch.int64, device=DEV), 3)
    with pytest.raises(ValueError, match="is not a KV cache format"):
        ops.sparse_single_layer_kv_transfer(lmc, caches, s1, torch.zeros(8, dtype=torch.int32, device=DEV), 9)


# ---------------------------------------------------------------------------
# batched_fused_single_layer_kv_transfer / batched_fused_sparse_...
# ---------------------------------------------------------------------------


def _chunks_of(T, num_chunks):
    base, rem = divmod(T, num_chunks)
    sizes = [base + (1 if i < rem else 0) for i in range(num_chunks)]
    offs = [sum(sizes[:i]) for i in range(num_chunks)]
    return offs, sizes


def _obj_shape(fmt, n, pe, token_major):
    if fmt in (ok.MERGED_KV, ok.SEPARATE_KV):
        return [n, 2, pe // 2] if token_major else [2, n, pe // 2]
    return [n * pe]


@pytest.mark.parametrize("fmt,two_major", [(1, False), (1, True), (2, False), (3, False), (4, False)])
@pytest.mark.parametrize("token_major", [False, True])
@pytest.mark.parametrize("num_chunks", [1, 3, 5])
@pytest.mark.parametrize("objects", ["pinned", "pageable", "gap"])
def test_batched_fused_single_layer(ops, fmt, two_major, token_major, num_chunks, objects):
    """tests/v1/test_mem_kernels.py:791-1062: equal, byte for byte (memory
    objects, paged caches and the staging buffer), to one single-layer copy
    through the staging buffer plus per-chunk copies, both directions, with
    some slots -1.  Pinned objects covering the staging tokens take the
    one-pass kernel; pageable objects and a chunk list with a gap take the
    two-step path."""
    T = 256
    g = torch.Generator().manual_seed(100 * fmt + 10 * num_chunks + token_major)
    src = paged_caches(fmt, g, two_major=two_major)
    dst = paged_caches(fmt, g, two_major=two_major)
    pe = plane_elems(fmt, src)
    slots = torch.randperm(32 * 16, generator=g)[:T]
    slots[[5, 130]] = -1
    slots = slots.to(DEV)
    offs, sizes = _chunks_of(T, num_chunks)
    if objects == "gap":
        sizes[-1] -= 3
    stg_shape = _obj_shape(fmt, T, pe, token_major)
    staging = randn_bf16(stg_shape, g).to(DEV)
    pin = objects != "pageable"
    objs = [torch.zeros(_obj_shape(fmt, n, pe, token_major), dtype=torch.bfloat16, pin_memory=pin) for n in sizes]
    # from_gpu
    want_stg = tb(staging)
    want_objs = [tb(o) for o in objs]
    ok.single_layer_kv_transfer(want_stg, [tb(c) for c in src], slots.cpu().numpy(), True, fmt, token_major,
                                two_major)
    ok.stage_chunks(want_stg, [tb(c) for c in src], want_objs, offs, sizes, fmt, token_major, True, two_major)
    ops.batched_fused_single_layer_kv_transfer(objs, staging, arg_caches(src), slots, offs, sizes, True, fmt,
                                               token_major, two_major)
    torch.cuda.synchronize()
    for o, w in zip(objs, want_objs):
        assert same(o, w)
    assert same(staging, want_stg)
    # to_gpu (objects perturbed first so staging rows change)
    for o in objs:
        o.add_(1.0)
    want_objs = [tb(o) for o in objs]
    want_dst = [tb(c) for c in dst]
    ok.stage_chunks(want_stg, [tb(c) for c in dst], want_objs, offs, sizes, fmt, token_major, False, two_major)
    ok.single_layer_kv_transfer(want_stg, want_dst, slots.cpu().numpy(), False, fmt, token_major, two_major)
    ops.batched_fused_single_layer_kv_transfer(objs, staging, arg_caches(dst), slots, offs, sizes, False, fmt,
                                               token_major, two_major)
    torch.cuda.synchronize()
    for c, w in zip(dst, want_dst):
        assert same(c, w)
    assert same(staging, want_stg)
    # the reference test's own check: dst rows now equal src rows + 1
    if fmt in (ok.MERGED_KV, ok.SEPARATE_KV) and objects != "gap":
        slots = slots[slots >= 0]
        for a, b in zip(src, dst):
            a = a + 1.0
            if fmt == ok.MERGED_KV:
                for p in range(2):
                    ap = a[p] if two_major else a[:, p]
                    bp = b[p] if two_major else b[:, p]
                    W = ap.shape[-2] * ap.shape[-1]
                    assert torch.equal(ap.reshape(-1, W)[slots], bp.reshape(-1, W)[slots])
            else:
                W = a.shape[-2] * a.shape[-1]
                assert torch.equal(a.reshape(-1, W)[slots], b.reshape(-1, W)[slots])


@pytest.mark.parametrize("fmt", [2, 3])
def test_batched_fused_sparse_single_layer(ops, fmt):
    T, num_chunks, n = 200, 3, 80
    g = torch.Generator().manual_seed(fmt)
    dst = paged_caches(fmt, g)
    pe = plane_elems(fmt, dst)
    offs, sizes = _chunks_of(T, num_chunks)
    objs = [pinned(_obj_shape(fmt, m, pe, False), g) for m in sizes]
    staging = torch.zeros(_obj_shape(fmt, T, pe, False), dtype=torch.bfloat16, device=DEV)
    sel = torch.randperm(T, generator=g)[:n].to(torch.int32).to(DEV)
    slots = torch.randperm(32 * 16, generator=g)[:n].to(DEV)
    want = [tb(c) for c in dst]
    stg = tb(staging)
    ok.stage_chunks(stg, want, [tb(o) for o in objs], offs, sizes, fmt, False, False)
    ok.sparse_single_layer_kv_transfer(stg, want, slots.cpu().numpy(), sel.cpu().numpy(), fmt)
    ops.batched_fused_sparse_single_layer_kv_transfer(objs, staging, arg_caches(dst), slots, sel, offs, sizes, fmt)
    torch.cuda.synchronize()
    for c, w in zip(dst, want):
        assert same(c, w)


# ---------------------------------------------------------------------------
# sparse_mla_dsa_batched_direct_kv_transfer (+ _fast / _prepared)
# ---------------------------------------------------------------------------


def test_sparse_direct_reference_minimal_case(ops):
    """tests/v1/test_sparse_direct_kernel_minimal.py:30-150 with its values."""
    chunk_size, num_chunks, kH, vH = 4, 2, 512, 128
    total = chunk_size * num_chunks
    selected, scratch = [0, 3, 4, 7], [0, 1, 2, 3]
    chunks = []
    for c in range(num_chunks):
        t = torch.empty(chunk_size * (kH + vH), dtype=torch.bfloat16, pin_memory=True)
        kp, vp = t[: chunk_size * kH].view(chunk_size, kH), t[chunk_size * kH:].view(chunk_size, vH)
        for j in range(chunk_size):
            kp[j].fill_(float(c * chunk_size + j + 1))
            vp[j].fill_(float(c * chunk_size + j + 101))
        chunks.append(t)
    k = torch.full((4, 16, 1, kH), -7.0, dtype=torch.bfloat16, device=DEV)
    v = torch.full((4, 16, 1, vH), -7.0, dtype=torch.bfloat16, device=DEV)
    ops.sparse_mla_dsa_batched_direct_kv_transfer(
        chunks, (k, v), torch.tensor(scratch, dtype=torch.long, device=DEV),
        torch.tensor(selected, dtype=torch.int32, device=DEV), chunk_size, total, 3, False, False, kH, vH, 0, False,
        None)
    torch.cuda.synchronize()
    kf, vf = k.reshape(-1, kH), v.reshape(-1, vH)
    for row, token in enumerate(selected):
        assert torch.all(kf[scratch[row]] == float(token + 1))
        assert torch.all(vf[scratch[row]] == float(token + 101))
    assert torch.all(kf[len(scratch):] == -7.0) and torch.all(vf[len(scratch):] == -7.0)


@pytest.mark.parametrize("fmt", [3, 4, 6])
@pytest.mark.parametrize("interleaved", [False, True])
@pytest.mark.parametrize("counted", [False, True])
def test_sparse_direct_mla_dsa(ops, fmt, interleaved, counted):
    g = torch.Generator().manual_seed(fmt * 4 + interleaved * 2 + counted)
    caches = paged_caches(fmt, g)
    pe = plane_elems(fmt, caches)
    cs, total = 64, 240
    chunks = [pinned([min(cs, total - c * cs) * pe], g) for c in range((total + cs - 1) // cs)]
    n = 128
    sel = torch.randint(0, total + 8, (2, n // 2), generator=g, dtype=torch.int32)
    slots = torch.randperm(32 * 16, generator=g)[:n].reshape(2, n // 2)
    slots[0, 3] = -1
    counts = torch.tensor([50, 64], dtype=torch.int32) if counted else None
    want = [tb(c) for c in caches]
    ok.sparse_direct_kv_transfer([to_bytes(c) for c in chunks], want, slots.numpy(), sel.numpy(), cs, total, fmt,
                                 interleaved=interleaved, counts=None if counts is None else counts.numpy())
    ops.sparse_mla_dsa_batched_direct_kv_transfer(
        chunks, arg_caches(caches), slots.to(DEV), sel.to(DEV), cs, total, fmt, False, False, 0, 0, 0, interleaved,
        None, None if counts is None else counts.to(DEV))
    torch.cuda.synchronize()
    for c, w in zip(caches, want):
        assert same(c, w)


@pytest.mark.parametrize("token_major", [False, True])
def test_sparse_direct_separate_kv(ops, token_major):
    g = torch.Generator().manual_seed(11 + token_major)
    caches = paged_caches(ok.SEPARATE_KV, g)
    W = caches[0].shape[-2] * caches[0].shape[-1]
    cs, total = 32, 96
    chunks = [pinned([cs, 2, W] if token_major else [2, cs, W], g) for _ in range(3)]
    sel = torch.randperm(total, generator=g)[:40].to(torch.int32)
    slots = torch.randperm(32 * 16, generator=g)[:40]
    want = [tb(c) for c in caches]
    ok.sparse_direct_kv_transfer([to_bytes(c) for c in chunks], want, slots.numpy(), sel.numpy(), cs, total,
                                 ok.SEPARATE_KV, layout=tb(chunks[0]), token_major=token_major)
    ops.sparse_mla_dsa_batched_direct_kv_transfer(chunks, caches, slots.to(DEV), sel.to(DEV), cs, total, 2,
                                                  token_major)
    torch.cuda.synchronize()
    for c, w in zip(caches, want):
        assert same(c, w)


def test_sparse_direct_fast_and_prepared_match(ops):
    g = torch.Generator().manual_seed(21)
    cs, total, n = 64, 256, 96
    chunks = [pinned([cs * 576], g) for _ in range(total // cs)]
    sel = torch.randperm(total, generator=g)[:n].to(torch.int32).to(DEV)
    slots = torch.randperm(32 * 16, generator=g)[:n].to(DEV)
    ptrs = ops._chunk_ptrs_for(chunks, DEV)
    outs = []
    for mode in range(3):
        caches = mla_caches(torch.Generator().manual_seed(5))
        if mode == 0:
            ops.sparse_mla_dsa_batched_direct_kv_transfer(chunks, caches, slots, sel, cs, total, 3,
                                                          chunk_ptrs_npu=ptrs)
        elif mode == 1:
            st = ops.prepare_sparse_direct_layer_state(chunks[0], caches, slots, False, False, 3, 0, 0, 0, cs)
            ops.sparse_mla_dsa_batched_direct_kv_transfer_fast(st, slots, sel, ptrs, cs, total, False, True)
        else:
            st = ops.prepare_sparse_direct_destination_state(caches, slots, 3, 0, 0, 0)
            ops.sparse_mla_dsa_batched_direct_kv_transfer_prepared(st, slots, sel, ptrs, cs, total, False)
        torch.cuda.synchronize()
        outs.append([to_bytes(c) for c in caches])
    for o in outs[1:]:
        assert all(np.array_equal(a, b) for a, b in zip(outs[0], o))


def test_sparse_direct_misaligned_chunk_base(ops):
    """A chunk address that is not 16-byte aligned takes the bytewise path."""
    g = torch.Generator().manual_seed(31)
    cs, total = 16, 32
    backing = [pinned([cs * 576 + 8], g) for _ in range(2)]
    chunks = [b[1: 1 + cs * 576] for b in backing]        # 2-byte offset views
    caches = mla_caches(g)
    sel = torch.arange(total, dtype=torch.int32)
    slots = torch.randperm(32 * 16, generator=g)[:total]
    want = [tb(c) for c in caches]
    ok.sparse_direct_kv_transfer([to_bytes(c) for c in chunks], want, slots.numpy(), sel.numpy(), cs, total, 3)
    ops.sparse_mla_dsa_batched_direct_kv_transfer(chunks, caches, slots.to(DEV), sel.to(DEV), cs, total, 3)
    torch.cuda.synchronize()
    for c, w in zip(caches, want):
        assert same(c, w)


def test_sparse_direct_errors(ops):
    g = torch.Generator().manual_seed(0)
    caches = mla_caches(g)
    chunk = torch.zeros(64 * 576, dtype=torch.bfloat16, pin_memory=True)
    s = torch.zeros(4, dtype=torch.int64, device=DEV)
    x = torch.zeros(4, dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="chunk_size is not positive"):
        ops.sparse_mla_dsa_batched_direct_kv_transfer([chunk], caches, s, x, 0, 64, 3)
    with pytest.raises(RuntimeError, match="in pinned host memory only"):
        ops.sparse_mla_dsa_batched_direct_kv_transfer([chunk.to(DEV)], caches, s, x, 64, 64, 3)
    with pytest.raises(RuntimeError, match="MLA/DSA formats \\(3-6\\) only"):
        ops.prepare_sparse_direct_destination_state(paged_caches(2, g), s, 2, 0, 0, 0)
    with pytest.raises(ValueError, match="of equal shape"):
        ops.prepare_sparse_direct_destination_state((caches[0], caches[0]), s, 3, 0, 0, 0)


# ---------------------------------------------------------------------------
# dense_mla_dsa_batched_direct_kv_transfer (+ _fast / _prepared / group)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("fmt", [3, 4, 6])
@pytest.mark.parametrize("interleaved", [False, True])
@pytest.mark.parametrize("fixed", [0, 64])
def test_dense_direct_both_directions(ops, fmt, interleaved, fixed):
    g = torch.Generator().manual_seed(fmt * 7 + interleaved * 3 + (fixed > 0))
    caches = paged_caches(fmt, g)
    pe = plane_elems(fmt, caches)
    total = 224
    sizes = [64, 64, 64, 32] if fixed else [50, 90, 84]
    offs = [sum(sizes[:i]) for i in range(len(sizes))]
    slots = torch.randperm(32 * 16, generator=g)[:total]
    slots[[3, 77]] = -1
    chunks = [torch.zeros(n * pe, dtype=torch.bfloat16, pin_memory=True) for n in sizes]
    o_t = torch.tensor(offs, dtype=torch.int32, device=DEV)
    z_t = torch.tensor(sizes, dtype=torch.int32, device=DEV)
    # store: paged -> chunks
    want_chunks = [to_bytes(c) for c in chunks]
    ok.dense_direct_kv_transfer(want_chunks, [tb(c) for c in caches], slots.numpy(), total, offs, sizes, fixed, fmt,
                                interleaved=interleaved, direction=True)
    ops.dense_mla_dsa_batched_direct_kv_transfer(chunks, arg_caches(caches), slots.to(DEV), o_t, z_t, total, fmt,
                                                 lmc_host_interleaved=interleaved, direction=True,
                                                 fixed_chunk_size=fixed)
    torch.cuda.synchronize()
    for c, w in zip(chunks, want_chunks):
        assert np.array_equal(to_bytes(c), w)
    # load: chunks -> other paged caches
    dst = paged_caches(fmt, g)
    want = [tb(c) for c in dst]
    ok.dense_direct_kv_transfer(want_chunks, want, slots.numpy(), total, offs, sizes, fixed, fmt,
                                interleaved=interleaved, direction=False)
    ops.dense_mla_dsa_batched_direct_kv_transfer(chunks, arg_caches(dst), slots.to(DEV), o_t, z_t, total, fmt,
                                                 lmc_host_interleaved=interleaved, direction=False,
                                                 fixed_chunk_size=fixed)
    torch.cuda.synchronize()
    for c, w in zip(dst, want):
        assert same(c, w)


def test_dense_direct_fast_prepared_group_match(ops):
    g = torch.Generator().manual_seed(41)
    L, total, cs = 3, 192, 64
    layers = [mla_caches(g) for _ in range(L)]
    slots = torch.randperm(32 * 16, generator=g)[:total].to(DEV)
    o_t = torch.tensor([0, 64, 128], dtype=torch.int32, device=DEV)
    z_t = torch.tensor([64, 64, 64], dtype=torch.int32, device=DEV)
    objs = [[torch.zeros(cs * 576, dtype=torch.bfloat16, pin_memory=True) for _ in range(3)] for _ in range(L)]
    states = [ops.prepare_sparse_direct_layer_state(objs[0][0], c, slots, False, False, 3, 0, 0, 0, cs)
              for c in layers]
    rows, table = ops.dense_mla_dsa_group_direct_kv_transfer_fast(states, objs, slots, o_t, z_t, total, False, True,
                                                                  True)
    torch.cuda.synchronize()
    assert table.shape == (L, 3) and len(rows) == L
    for l in range(L):
        want = [to_bytes(c) for c in objs[l]]
        ok.dense_direct_kv_transfer(want, [tb(c) for c in layers[l]], slots.cpu().numpy(), total, [0, 64, 128],
                                    [64, 64, 64], 0, 3, direction=True)
        assert all(np.array_equal(to_bytes(c), w) for c, w in zip(objs[l], want))
    # prepared group store into fresh objects equals the fast group store
    objs2 = [[torch.zeros(cs * 576, dtype=torch.bfloat16, pin_memory=True) for _ in range(3)] for _ in range(L)]
    table2 = ops._chunk_ptrs_for([t for r in objs2 for t in r], DEV).reshape(L, 3)
    ops.dense_mla_dsa_group_direct_kv_transfer_prepared(states, slots, table2, o_t, z_t, total, False, True, 0)
    # _fast and _prepared retrieve of layer 0 into fresh caches agree
    fresh = [mla_caches(torch.Generator().manual_seed(9)) for _ in range(2)]
    ops.dense_mla_dsa_batched_direct_kv_transfer_fast(
        ops.prepare_sparse_direct_layer_state(objs[0][0], fresh[0], slots, False, False, 3, 0, 0, 0, cs),
        slots, table[0], o_t, z_t, total, False, False, True)
    ops.dense_mla_dsa_batched_direct_kv_transfer_prepared(
        ops.prepare_sparse_direct_destination_state(fresh[1], slots, 3, 0, 0, 0), slots, table[0], o_t, z_t, total,
        False, True)
    torch.cuda.synchronize()
    for l in range(L):
        assert all(torch.equal(a, b) for a, b in zip(objs[l], objs2[l]))
    assert all(torch.equal(a, b) for a, b in zip(fresh[0], fresh[1]))
    for c in range(2):
        assert torch.equal(fresh[0][c].reshape(-1, fresh[0][c].shape[-1])[slots],
                           layers[0][c].reshape(-1, layers[0][c].shape[-1])[slots])


def test_dense_direct_errors(ops):
    g = torch.Generator().manual_seed(0)
    s = torch.zeros(8, dtype=torch.int64, device=DEV)
    o = torch.zeros(1, dtype=torch.int32, device=DEV)
    chunk = torch.zeros(8 * 576, dtype=torch.bfloat16, pin_memory=True)
    with pytest.raises(RuntimeError, match="MLA/DSA formats \\(3-6\\) only"):
        ops.dense_mla_dsa_batched_direct_kv_transfer([chunk], paged_caches(2, g), s, o, o, 8, 2)
    with pytest.raises(RuntimeError, match="do not span total_tokens"):
        ops.dense_mla_dsa_batched_direct_kv_transfer([chunk], mla_caches(g), s, o, o, 16, 3, fixed_chunk_size=4)
    with pytest.raises(RuntimeError, match="longer than total_tokens"):
        ops.dense_mla_dsa_batched_direct_kv_transfer([chunk], mla_caches(g), s, o, o, 4, 3, fixed_chunk_size=4)
