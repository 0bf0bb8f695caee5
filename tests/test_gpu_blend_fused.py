"""GPU parity of blend_layer_to_paged, the CacheBlend connector's per-layer
retrieve in one kernel (no reference counterpart; it replaces the sequence
of lmcache_ascend/v1/npu_connector/npu_connectors.py:597-680 for one layer).

Expected caches come from the oracle applied to the connector's sequence
on the CPU: a zeroed [2, N, W] buffer receives the KV_2TD memory objects at
their token offsets, its K half is re-rotated by the oracle's float32
restatement of rotary_embedding_k_fused (rounded once; tokens whose old or
new position lies outside the cache keep their values), the rows of tokens
no object covers are zeroed again (the connector zeroes them after the
re-rotation), and the oracle's single-layer scatter writes it into the
paged caches.  Every byte of every
cache is compared, so rows of skipped slots must keep their values and
tokens no object covers must arrive as zero rows.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvutil import sample_slots, to_bytes
from oracle import kv_transfer as ok
from oracle import rope as orope

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
NB, BS, H, D = 48, 16, 8, 128
W = H * D


@pytest.fixture(scope="module")
def ops():
    import lmcache_amd

    return lmcache_amd.c_ops


def _tb(t: torch.Tensor) -> ok.TensorBytes:
    return ok.TensorBytes(to_bytes(t), list(t.shape), list(t.stride()), t.element_size())


def _caches(fmt, two_major, dtype, gen):
    if fmt == 2:
        return (torch.randn((NB, BS, H, D), generator=gen).to(dtype), torch.randn((NB, BS, H, D), generator=gen).to(dtype))
    shape = (2, NB, BS, H, D) if two_major else (NB, 2, BS, H, D)
    return torch.randn(shape, generator=gen).to(dtype)


def _expected(caches, fmt, two_major, objs, starts, n_tok, slots, rope):
    """The connector's sequence on the CPU, through the oracle."""
    dtype = objs[0].dtype if objs else torch.bfloat16
    buf = torch.zeros((2, n_tok, W), dtype=dtype)
    for o, s in zip(objs, starts):
        buf[:, s:s + o.shape[1]] = o.cpu()
    if rope is not None:
        old, new, cache, head_size, neox = rope
        max_pos = cache.shape[0]
        ok_rows = (old >= 0) & (old < max_pos) & (new >= 0) & (new < max_pos)
        k = buf[0].float().numpy()
        rows = np.nonzero(ok_rows.numpy())[0]
        if rows.size:
            z = orope.fused_rerotate_f32(k[rows], old.numpy()[rows], new.numpy()[rows], cache.float().numpy(),
                                         head_size, neox)
            k_new = buf[0].clone()
            k_new[torch.from_numpy(rows)] = torch.from_numpy(orope.round_to(z, dtype)).to(dtype)
            buf[0] = k_new
    # Gap rows are zeroed after the re-rotation, as the connector does
    # (npu_connectors.py:647-649): rotating a zero row can give -0.0.
    covered = torch.zeros(n_tok, dtype=torch.bool)
    for o, s in zip(objs, starts):
        covered[s:s + o.shape[1]] = True
    buf[:, ~covered] = 0
    want = [_tb(c) for c in ((caches,) if isinstance(caches, torch.Tensor) else caches)]
    ok.single_layer_kv_transfer(_tb(buf.contiguous()), want, slots.numpy(), False, fmt, False, two_major)
    return want


def _run_case(ops, fmt, two_major, dtype, objs_on, rope_kind, neox, rot, layout, seed, slot_dtype=torch.int64,
              slots_on="device"):
    gen = torch.Generator().manual_seed(seed)
    caches = _caches(fmt, two_major, dtype, gen)
    gpu = caches.to(DEV) if isinstance(caches, torch.Tensor) else tuple(c.to(DEV) for c in caches)
    # Objects of 64, 100 and 37 tokens at token offsets with gaps before,
    # between and after them (layout "gaps"), or back to back ("dense").
    sizes = [64, 100, 37]
    if layout == "gaps":
        starts = [5, 64 + 5 + 11, 64 + 5 + 11 + 100 + 3]
        n_tok = starts[-1] + sizes[-1] + 9
    else:
        starts = [0, 64, 164]
        n_tok = 201
    objs = [torch.randn((2, n, W), generator=gen).to(dtype) for n in sizes]
    slots = torch.tensor(sample_slots(NB * BS, n_tok, seed=seed), dtype=torch.int64)
    slots[::17] = -1
    slots[3] = NB * BS + 5  # out of range: skipped
    if objs_on == "pinned":
        dobjs = [o.pin_memory() for o in objs]
    else:
        dobjs = [o.to(DEV) for o in objs]
    rope = None
    kwargs = {}
    if rope_kind != "none":
        pdt = torch.int64 if rope_kind == "i64" else torch.int32
        max_pos = n_tok + 1500
        cache = orope.cos_sin_cache(max_pos, rot, 500000.0).to(torch.bfloat16 if rot == D else torch.float32)
        old = torch.arange(n_tok, dtype=torch.int64)
        new = old + 1000
        new[7] = max_pos + 3   # out of the cache: the row keeps its values
        old[9] = -1
        rope = (old, new, cache, D, neox)
        kwargs = dict(old_positions=old.to(pdt).to(DEV), new_positions=new.to(pdt).to(DEV),
                      cos_sin_cache=cache.to(DEV), head_size=D, is_neox=neox)
    want = _expected(caches, fmt, two_major, objs, starts, n_tok, slots, rope)
    sl = slots.to(slot_dtype)
    sl = sl.pin_memory() if slots_on == "pinned" else sl.to(DEV)
    ops.blend_layer_to_paged(dobjs, starts, gpu, sl, kvcache_format_raw=fmt,
                             vllm_two_major=two_major,
                             **kwargs)
    torch.cuda.synchronize()
    got = (gpu,) if isinstance(gpu, torch.Tensor) else gpu
    for g, w in zip(got, want):
        assert np.array_equal(to_bytes(g), w.data)


@pytest.mark.parametrize("objs_on", ["pinned", "device"])
@pytest.mark.parametrize("rope_kind", ["none", "i64", "i32"])
@pytest.mark.parametrize("layout", ["gaps", "dense"])
def test_blend_layer_separate_vs_oracle(ops, objs_on, rope_kind, layout):
    _run_case(ops, 2, False, torch.bfloat16, objs_on, rope_kind, True, D, layout, seed=11)


@pytest.mark.parametrize("objs_on", ["pinned", "device"])
@pytest.mark.parametrize("two_major", [True, False])
@pytest.mark.parametrize("neox", [True, False])
def test_blend_layer_merged_vs_oracle(ops, objs_on, two_major, neox):
    _run_case(ops, 1, two_major, torch.bfloat16, objs_on, "i64", neox, D, "gaps", seed=13 + two_major + 2 * neox)


@pytest.mark.parametrize("objs_on", ["pinned", "device"])
@pytest.mark.parametrize("neox", [True, False])
def test_blend_layer_fp16_keys_whole_heads(ops, objs_on, neox):
    """fp16 keys rotated whole (the 16-lane group kernel) with a bf16
    cos/sin cache, from pinned and from device objects."""
    _run_case(ops, 2, False, torch.float16, objs_on, "i32", neox, D, "dense", seed=47 + neox)


@pytest.mark.parametrize("neox", [True, False])
def test_blend_layer_partial_rotary_fp32_cache_fp16_keys(ops, neox):
    """rot = 64 of 128 dims (the rest pass through), an fp32 cos/sin cache
    and fp16 keys."""
    _run_case(ops, 2, False, torch.float16, "device", "i64", neox, 64, "gaps", seed=17 + neox)


def test_blend_layer_fp32_keys_take_the_connector_sequence(ops):
    """fp32 caches are outside the fused kernel: the op runs the connector's
    own sequence with this library's ops, with the same bytes."""
    _run_case(ops, 2, False, torch.float32, "device", "i64", True, D, "gaps", seed=19)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_blend_layer_slots_in_pinned_host_memory(ops, dtype):
    """A slot mapping in pinned host memory, which the entry point accepts:
    the fused kernel reads it over PCIe (bf16), and the connector sequence
    (fp32 keys) copies it to the caches' device first."""
    _run_case(ops, 2, False, dtype, "pinned", "i64", True, D, "gaps", seed=53, slots_on="pinned")


def test_blend_layer_without_objects_zeroes_every_named_slot(ops):
    gen = torch.Generator().manual_seed(23)
    caches = _caches(2, False, torch.bfloat16, gen)
    gpu = tuple(c.to(DEV) for c in caches)
    slots = torch.tensor(sample_slots(NB * BS, 50, seed=23), dtype=torch.int64)
    ops.blend_layer_to_paged([], [], gpu, slots.to(DEV), kvcache_format_raw=2)
    want = _expected(caches, 2, False, [], [], 50, slots, None)
    torch.cuda.synchronize()
    for g, w in zip(gpu, want):
        assert np.array_equal(to_bytes(g), w.data)


def test_blend_layer_rejects_overlapping_objects(ops):
    gen = torch.Generator().manual_seed(29)
    gpu = tuple(c.to(DEV) for c in _caches(2, False, torch.bfloat16, gen))
    objs = [torch.zeros((2, 10, W), dtype=torch.bfloat16, device=DEV) for _ in range(2)]
    slots = torch.arange(30, dtype=torch.int64, device=DEV)
    with pytest.raises(RuntimeError, match="must not overlap"):
        ops.blend_layer_to_paged(objs, [0, 5], gpu, slots, kvcache_format_raw=2)
    with pytest.raises(RuntimeError, match="exceeds slot_mapping"):
        ops.blend_layer_to_paged(objs[:1], [25], gpu, slots, kvcache_format_raw=2)


def test_blend_layer_int32_slots(ops):
    _run_case(ops, 2, False, torch.bfloat16, "pinned", "i64", True, D, "gaps", seed=31, slot_dtype=torch.int32)


def test_blend_layer_rejects_host_positions(ops):
    gen = torch.Generator().manual_seed(37)
    gpu = tuple(c.to(DEV) for c in _caches(2, False, torch.bfloat16, gen))
    objs = [torch.zeros((2, 10, W), dtype=torch.bfloat16, device=DEV)]
    slots = torch.arange(10, dtype=torch.int64, device=DEV)
    cache = orope.cos_sin_cache(64, D, 10000.0).to(torch.bfloat16).to(DEV)
    pos = torch.arange(10, dtype=torch.int64)
    with pytest.raises(RuntimeError, match="on the caches' device"):
        ops.blend_layer_to_paged(objs, [0], gpu, slots, old_positions=pos, new_positions=pos.to(DEV),
                                 cos_sin_cache=cache, head_size=D, kvcache_format_raw=2)
    with pytest.raises(RuntimeError, match="non-negative"):
        ops.blend_layer_to_paged(objs, [-1], gpu, slots, kvcache_format_raw=2)


def test_blend_layer_graph_replays(ops):
    """Captured once in a HIP graph; each replay reads the objects' current
    contents and positions (refilled by eager copies between replays) and
    must equal the oracle's connector sequence on them."""
    gen = torch.Generator().manual_seed(41)
    caches = _caches(2, False, torch.bfloat16, gen)
    gpu = tuple(c.to(DEV) for c in caches)
    sizes, starts = [64, 100], [0, 70]
    n_tok = 180
    objs = [torch.randn((2, n, W), generator=gen).to(torch.bfloat16).pin_memory() for n in sizes]
    slots = torch.tensor(sample_slots(NB * BS, n_tok, seed=41), dtype=torch.int64)
    max_pos = 2048
    cache = orope.cos_sin_cache(max_pos, D, 500000.0).to(torch.bfloat16)
    old = torch.zeros(n_tok, dtype=torch.int64, device=DEV)
    new = torch.zeros(n_tok, dtype=torch.int64, device=DEV)
    dslots, dcache = slots.to(DEV), cache.to(DEV)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        ops.blend_layer_to_paged(objs, starts, gpu, dslots, old_positions=old, new_positions=new,
                                 cos_sin_cache=dcache, head_size=D, is_neox=True, kvcache_format_raw=2)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.blend_layer_to_paged(objs, starts, gpu, dslots, old_positions=old, new_positions=new,
                                 cos_sin_cache=dcache, head_size=D, is_neox=True, kvcache_format_raw=2)
    torch.cuda.synchronize()
    for rep in range(3):
        for o in objs:
            o.copy_(torch.randn(o.shape, generator=gen).to(torch.bfloat16))
        o_pos = torch.randint(0, max_pos - 600, (n_tok,), generator=gen)
        n_pos = o_pos + 100 * (rep + 1)
        old.copy_(o_pos)
        new.copy_(n_pos)
        torch.cuda.synchronize()
        want = _expected(tuple(c.cpu() for c in gpu), 2, False, objs, starts, n_tok, slots,
                         (o_pos, n_pos, cache, D, True))
        graph.replay()
        torch.cuda.synchronize()
        for g, w in zip(gpu, want):
            assert np.array_equal(to_bytes(g), w.data), f"replay {rep}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_blend_layer_through_ctypes(ops, monkeypatch, dtype):
    """The same op with the C++ binding absent (the ctypes path), fused
    (bf16) and through the connector's sequence (fp32)."""
    monkeypatch.setattr(ops, "_ext", None)
    _run_case(ops, 2, False, dtype, "pinned", "i64", True, D, "gaps", seed=43)


@pytest.mark.parametrize("rope_kind", ["none", "i64"])
def test_blend_layer_grid_stride_over_a_long_object(ops, rope_kind):
    """One pinned object of 9000 tokens: more tokens than the capped grid for
    host objects covers in one pass, so groups stride over the segment.
    Tokens past the cache's 768 slots get -1 (skipped)."""
    gen = torch.Generator().manual_seed(53)
    caches = _caches(2, False, torch.bfloat16, gen)
    gpu = tuple(c.to(DEV) for c in caches)
    n_tok = 9000
    obj = torch.randn((2, n_tok, W), generator=gen).to(torch.bfloat16)
    slots = torch.full((n_tok,), -1, dtype=torch.int64)
    perm = torch.tensor(sample_slots(NB * BS, NB * BS, seed=53), dtype=torch.int64)
    pick = torch.randperm(n_tok, generator=gen)[: NB * BS]
    slots[pick] = perm
    rope, kwargs = None, {}
    if rope_kind != "none":
        max_pos = 12000
        cache = orope.cos_sin_cache(max_pos, D, 500000.0).to(torch.bfloat16)
        old = torch.arange(n_tok, dtype=torch.int64)
        new = old + 7
        rope = (old, new, cache, D, True)
        kwargs = dict(old_positions=old.to(DEV), new_positions=new.to(DEV), cos_sin_cache=cache.to(DEV),
                      head_size=D, is_neox=True)
    want = _expected(caches, 2, False, [obj], [0], n_tok, slots, rope)
    ops.blend_layer_to_paged([obj.pin_memory()], [0], gpu, slots.to(DEV), kvcache_format_raw=2, **kwargs)
    torch.cuda.synchronize()
    for g, w in zip(gpu, want):
        assert np.array_equal(to_bytes(g), w.data)
