"""CPU oracle for the paged-KV gather/scatter ops.  TEST INFRASTRUCTURE ONLY.

This module is the reference the tests, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` compare the HIP kernels against.  It is
never on the product path: the `lmcache_amd` package does not import it.

Every buffer is a flat numpy uint8 array (the bytes of a tensor); every op is
restated as explicit byte-offset arithmetic from the reference's host code,
so the oracle is independent of the kernels' geometry tables.  All ops are
pure copies: results must match bit for bit.

Pinning (see tests/test_oracle_kv.py): closed forms (numpy fancy indexing as
the textbook gather/scatter), the reference's own invariants (store ->
retrieve round trip; multi_layer == per-layer load_and_reshape_flash,
tests/v1/test_mem_kernels.py:124-127; fused == non-fused, :400) and
brute-force per-element loops on tiny inputs.

Slots outside [0, num_slots) are skipped (no read, no write): the reference's
in-tree kernels and CPU substitutes skip negative slots
(csrc/graph/sparse_graph_kernel.cpp:45-48; tools/cpu_vllm_runtime.py:379-380).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Sequence

import numpy as np

MERGED_KV, SEPARATE_KV, MLA_KV, DSA_KV, MLA_LATENT, DSA_INDEX = 1, 2, 3, 4, 5, 6


@dataclass
class _Plane:
    width: int        # elements per row
    ptr_index: int    # index within the layer's pointer-table entries
    paged_off: int    # byte offset added to the table pointer
    col: int          # element column inside a concatenated LMC row


def multi_layer_planes(fmt: int, use_mla: bool, last_dim: int, kH: int, vH: int,
                       dsaH: int, page_buffer_size: int, es: int):
    """(planes, pointers_per_layer, concatenated) for a multi-layer call.

    csrc/utils.cpp:59-83 fixes the plane count and width per format;
    csrc/mem_kernels.cpp:58-69 the MERGED K/V split at page_buffer_size rows;
    lmcache_ascend/v1/npu_connector/npu_connectors.py:889-925 the pointer
    table order (K, V, DSA per layer); npu_connectors.py:1472-1485 the
    [1, L, T, kH+vH(+dsaH)] memory-object shape of MLA/DSA, whose rows are
    the per-(layer, token) concatenation [K | V | DSA].  use_mla with the
    MERGED/SEPARATE codes selects the single-plane MLA cache
    (csrc/mindspore/mem_kernels.cpp:85-88).
    """
    if fmt == MERGED_KV:
        if use_mla:
            return [_Plane(last_dim, 0, 0, 0)], 1, False
        return [_Plane(last_dim, 0, 0, 0),
                _Plane(last_dim, 0, page_buffer_size * last_dim * es, 0)], 1, False
    if fmt == SEPARATE_KV:
        if use_mla:
            return [_Plane(last_dim, 0, 0, 0)], 1, False
        return [_Plane(last_dim, 0, 0, 0), _Plane(last_dim, 1, 0, 0)], 2, False
    if fmt in (MLA_KV, MLA_LATENT):
        return [_Plane(kH, 0, 0, 0), _Plane(vH, 1, 0, kH)], 2, True
    if fmt == DSA_KV:
        return [_Plane(kH, 0, 0, 0), _Plane(vH, 1, 0, kH), _Plane(dsaH, 2, 0, kH + vH)], 3, True
    if fmt == DSA_INDEX:
        return [_Plane(dsaH, 0, 0, 0)], 1, True
    raise RuntimeError(f"no plane layout for KV format {fmt}")


def multi_layer_kv_transfer(lmc: np.ndarray, table: Sequence[np.ndarray], slots: np.ndarray,
                            page_buffer_size: int, direction: bool, use_mla: bool, fmt: int,
                            num_layers: int, last_dim: int, es: int,
                            kH: int = 0, vH: int = 0, dsaH: int = 0) -> None:
    """multi_layer_kv_transfer (csrc/mem_kernels.cpp:54-111), in place.

    lmc: bytes of the memory object ([kv, L, T, W] or [1, L, T, sum W]).
    table: bytes of the tensor behind each pointer-table entry, in table order.
    direction True: paged -> lmc (store); False: lmc -> paged (retrieve).
    """
    planes, ppl, concat = multi_layer_planes(fmt, use_mla, last_dim, kH, vH, dsaH,
                                             page_buffer_size, es)
    T = int(slots.shape[0])
    L = int(num_layers)
    wsum = sum(p.width for p in planes)
    valid = (slots >= 0) & (slots < page_buffer_size)
    t_idx = np.nonzero(valid)[0]
    s_idx = slots[valid].astype(np.int64)
    for pi, pl in enumerate(planes):
        rb = pl.width * es
        for l in range(L):
            buf = table[l * ppl + pl.ptr_index]
            paged = buf[pl.paged_off: pl.paged_off + page_buffer_size * rb].reshape(page_buffer_size, rb)
            if concat:
                lm = lmc[: L * T * wsum * es].reshape(L, T, wsum * es)[l, :, pl.col * es: pl.col * es + rb]
            else:
                base = (pi * L + l) * T * rb
                lm = lmc[base: base + T * rb].reshape(T, rb)
            if direction:
                lm[t_idx] = paged[s_idx]
            else:
                paged[s_idx] = lm[t_idx]


def _gather_rows(buf: np.ndarray, offs: np.ndarray, nbytes: int) -> np.ndarray:
    return buf[offs[:, None] + np.arange(nbytes, dtype=np.int64)[None, :]]


def _scatter_rows(buf: np.ndarray, offs: np.ndarray, rows: np.ndarray) -> None:
    buf[offs[:, None] + np.arange(rows.shape[1], dtype=np.int64)[None, :]] = rows


@dataclass
class TensorBytes:
    """A tensor as bytes plus the geometry the reference host code reads."""
    data: np.ndarray          # flat uint8, element 0 at index 0
    shape: Sequence[int]
    strides: Sequence[int]    # elements
    es: int

    @property
    def numel(self) -> int:
        n = 1
        for s in self.shape:
            n *= int(s)
        return n


def _layer_planes(caches: List[TensorBytes], fmt: int, vllm_two_major: bool, kH: int, vH: int,
                  dsaH: int):
    """Paged side of one layer (csrc/utils.cpp:212-406): a list of
    (cache, row bytes, paged offset, row pitch, block stride, width,
    prefix) per plane, plus num_slots, block_size and the LMC token width
    (sum of plane widths)."""
    es = caches[0].es
    planes = []
    if fmt in (MLA_KV, DSA_KV, MLA_LATENT, DSA_INDEX):
        k = caches[0]
        v = caches[1] if fmt != DSA_INDEX else None
        dsa = caches[2] if fmt == DSA_KV else None
        if kH <= 0:
            kH = k.shape[-2] * k.shape[-1]
        if vH <= 0 and v is not None:
            vH = v.shape[-2] * v.shape[-1]
        if dsaH <= 0 and dsa is not None:
            dsaH = dsa.shape[-2] * dsa.shape[-1]
        if fmt == DSA_INDEX:
            kH = dsaH if dsaH > 0 else k.shape[-2] * k.shape[-1]
            vH = 0
        widths = [kH, vH if fmt != DSA_INDEX else 0, dsaH if fmt == DSA_KV else 0]
        num_slots, pre = None, 0
        for w, tb in zip(widths, [k, v, dsa]):
            if w > 0 and tb is not None:
                planes.append((tb, w * es, 0, w * es, 0, w, pre))
                ns = tb.numel // w
                num_slots = ns if num_slots is None else min(num_slots, ns)
            pre += w
        return planes, num_slots, 0, sum(widths)
    k = caches[0]
    H, D, BS = k.shape[-2], k.shape[-1], k.shape[-3]
    W = H * D
    if fmt == MERGED_KV:
        blk = k.strides[1] if vllm_two_major else k.strides[0]
        voff = k.strides[0] if vllm_two_major else k.strides[1]
        NB = k.shape[1] if vllm_two_major else k.shape[0]
        planes = [(k, W * es, 0, W * es, blk * es, W, 0), (k, W * es, voff * es, W * es, blk * es, W, W)]
        return planes, NB * BS, BS, 2 * W
    v = caches[1]
    planes = [(k, W * es, 0, W * es, k.strides[0] * es, W, 0),
              (v, W * es, 0, W * es, v.strides[0] * es, W, W)]
    return planes, min(k.shape[0], v.shape[0]) * BS, BS, 2 * W


def _single_layer_lmc(lmc: TensorBytes, planes, plane_elems: int, mla_dsa: bool, token_major: bool):
    """LMC side of a single-layer buffer: (byte offset of plane p's token 0,
    byte stride per token) per plane, and the tokens it holds
    (csrc/utils.cpp:222-244, 350-357)."""
    es = lmc.es
    if mla_dsa:
        N = lmc.numel // plane_elems
        return [(pre * N * es, w * es) for (_, _, _, _, _, w, pre) in planes], N
    if token_major:
        tok_stride, val_off = lmc.strides[0], lmc.strides[1]
    else:
        tok_stride, val_off = lmc.strides[1], lmc.strides[0]
    N = lmc.shape[0] if token_major else lmc.shape[1]
    return [(0, tok_stride * es), (val_off * es, tok_stride * es)], N


def _paged_offsets(slot: np.ndarray, plane, block_size: int) -> np.ndarray:
    _, _, poff, pitch, blk, _, _ = plane
    if block_size:
        return poff + (slot // block_size) * blk + (slot % block_size) * pitch
    return poff + slot * pitch


def single_layer_kv_transfer(lmc: TensorBytes, caches: List[TensorBytes], slots: np.ndarray,
                             direction: bool, fmt: int, token_major: bool = False,
                             vllm_two_major: bool = False, kH: int = 0, vH: int = 0,
                             dsaH: int = 0) -> None:
    """single_layer_kv_transfer (csrc/mem_kernels.cpp:265-334), in place.

    Strides follow csrc/utils.cpp:212-285; MLA/DSA hidden-dim defaults and the
    stacked-plane LMC layout follow csrc/utils.cpp:310-357.
    """
    T = int(slots.shape[0])
    mla = fmt in (MLA_KV, DSA_KV, MLA_LATENT, DSA_INDEX)
    planes, num_slots, block_size, pe = _layer_planes(caches, fmt, vllm_two_major, kH, vH, dsaH)
    lmc_geo, N = _single_layer_lmc(lmc, planes, pe, mla, token_major)
    assert T <= N, "LMC buffer too small"
    valid = (slots >= 0) & (slots < num_slots)
    s = slots[valid].astype(np.int64)
    t = np.nonzero(valid)[0].astype(np.int64)
    for plane, (l0, lstride) in zip(planes, lmc_geo):
        tb, rb = plane[0], plane[1]
        p_off = _paged_offsets(s, plane, block_size)
        l_off = l0 + t * lstride
        if direction:
            _scatter_rows(lmc.data, l_off, _gather_rows(tb.data, p_off, rb))
        else:
            _scatter_rows(tb.data, p_off, _gather_rows(lmc.data, l_off, rb))


def sparse_single_layer_kv_transfer(lmc: TensorBytes, caches: List[TensorBytes],
                                    slots_packed: np.ndarray, selected: np.ndarray, fmt: int,
                                    token_major: bool = False, vllm_two_major: bool = False,
                                    kH: int = 0, vH: int = 0, dsaH: int = 0) -> None:
    """sparse_single_layer_kv_transfer (csrc/mem_kernels.cpp:418-497;
    tests/v1/test_mem_kernels.py:1445-1543): for each i, paged row
    slots_packed[i] <- LMC token selected[i]; entries whose slot or token is
    out of range are skipped."""
    mla = fmt in (MLA_KV, DSA_KV, MLA_LATENT, DSA_INDEX)
    planes, num_slots, block_size, pe = _layer_planes(caches, fmt, vllm_two_major, kH, vH, dsaH)
    lmc_geo, N = _single_layer_lmc(lmc, planes, pe, mla, token_major)
    slots_packed = slots_packed.reshape(-1).astype(np.int64)
    selected = selected.reshape(-1).astype(np.int64)
    valid = (slots_packed >= 0) & (slots_packed < num_slots) & (selected >= 0) & (selected < N)
    s, t = slots_packed[valid], selected[valid]
    for plane, (l0, lstride) in zip(planes, lmc_geo):
        _scatter_rows(plane[0].data, _paged_offsets(s, plane, block_size),
                      _gather_rows(lmc.data, l0 + t * lstride, plane[1]))


def _chunk_row_offset(plane, pe: int, n_c: int, t: int, es: int, interleaved: bool) -> int:
    """Byte offset of token t of plane `plane` inside an MLA/DSA memory
    object of n_c tokens: stacked planes [K: n_c*kH | V: n_c*vH | DSA] or
    per-token [K | V | DSA] rows (tools/cpu_vllm_runtime.py:322-330,
    366-373)."""
    w, pre = plane[5], plane[6]
    if interleaved:
        return (t * pe + pre) * es
    return (pre * n_c + t * w) * es


def dense_direct_kv_transfer(chunks: Sequence[np.ndarray], caches: List[TensorBytes],
                             slots: np.ndarray, total_tokens: int, chunk_offsets, chunk_sizes,
                             fixed_chunk_size: int, fmt: int, kH: int = 0, vH: int = 0,
                             dsaH: int = 0, interleaved: bool = False,
                             direction: bool = False) -> None:
    """dense_mla_dsa_batched_direct_kv_transfer, following the reference's
    CPU restatement (tools/cpu_vllm_runtime.py:353-411): chunk c covers
    tokens [start, start + count) of slot_mapping (start = c * fixed or
    chunk_offsets[c]); direction True: paged -> chunk."""
    planes, num_slots, block_size, pe = _layer_planes(caches, fmt, False, kH, vH, dsaH)
    es = caches[0].es
    slots = slots.astype(np.int64)
    for c, buf in enumerate(chunks):
        if fixed_chunk_size:
            start = c * fixed_chunk_size
            count = min(fixed_chunk_size, total_tokens - start)
        else:
            start, count = int(chunk_offsets[c]), int(chunk_sizes[c])
        for t in range(count):
            g = start + t
            if g >= slots.shape[0]:
                break
            s = int(slots[g])
            if s < 0 or s >= num_slots:
                continue
            for plane in planes:
                rb = plane[1]
                po = int(_paged_offsets(np.int64(s), plane, block_size))
                lo = _chunk_row_offset(plane, pe, count, t, es, interleaved)
                if direction:
                    buf[lo: lo + rb] = plane[0].data[po: po + rb]
                else:
                    plane[0].data[po: po + rb] = buf[lo: lo + rb]


def sparse_direct_kv_transfer(chunks: Sequence[np.ndarray], caches: List[TensorBytes],
                              slots_packed: np.ndarray, selected: np.ndarray, chunk_size: int,
                              total_tokens: int, fmt: int, kH: int = 0, vH: int = 0,
                              dsaH: int = 0, interleaved: bool = False, counts=None,
                              layout: TensorBytes = None, token_major: bool = False,
                              vllm_two_major: bool = False) -> None:
    """sparse_mla_dsa_batched_direct_kv_transfer, following the reference's
    CPU restatement (tools/cpu_vllm_runtime.py:288-343): entry i moves token
    selected[i] (chunk selected[i] // chunk_size, n_c = min(chunk_size,
    total_tokens - chunk * chunk_size)) into paged row slots_packed[i].
    `counts` (csrc/mem_kernels.cpp:636-650): the entries form len(counts)
    rows of equal width; only the first counts[r] of row r are valid.
    MERGED/SEPARATE memory objects have the layout of `layout` (shape and
    strides of the first chunk)."""
    mla = fmt in (MLA_KV, DSA_KV, MLA_LATENT, DSA_INDEX)
    planes, num_slots, block_size, pe = _layer_planes(caches, fmt, vllm_two_major, kH, vH, dsaH)
    es = caches[0].es
    slots_packed = slots_packed.reshape(-1).astype(np.int64)
    selected = selected.reshape(-1).astype(np.int64)
    n = selected.shape[0]
    row_w = n // len(counts) if counts is not None else 0
    if not mla:
        lmc_geo, _ = _single_layer_lmc(layout, planes, pe, False, token_major)
    for i in range(n):
        if counts is not None:
            r = i // row_w
            if r >= len(counts) or i - r * row_w >= int(counts[r]):
                continue
        tok, s = int(selected[i]), int(slots_packed[i])
        if tok < 0 or tok >= total_tokens or s < 0 or s >= num_slots:
            continue
        c = tok // chunk_size
        if c >= len(chunks):
            continue
        t = tok - c * chunk_size
        n_c = min(chunk_size, total_tokens - c * chunk_size)
        for q, plane in enumerate(planes):
            rb = plane[1]
            po = int(_paged_offsets(np.int64(s), plane, block_size))
            if mla:
                lo = _chunk_row_offset(plane, pe, n_c, t, es, interleaved)
            else:
                lo = lmc_geo[q][0] + t * lmc_geo[q][1]
            plane[0].data[po: po + rb] = chunks[c][lo: lo + rb]


def stage_chunks(staging: TensorBytes, caches: List[TensorBytes], objs: Sequence[TensorBytes],
                 offsets, sizes, fmt: int, token_major: bool, to_objects: bool,
                 vllm_two_major: bool = False, kH: int = 0, vH: int = 0, dsaH: int = 0) -> None:
    """The DMA copies of the batched fused paths (csrc/utils.cpp:500-733):
    staging tokens [offsets[i], + sizes[i]) <-> memory object i.
    MLA/DSA objects: stacked planes, or per-token [K|V|DSA] rows when
    token_major; MERGED/SEPARATE objects: [n, 2, W] (token_major, one range)
    or [2, n, W] (K range, then V range at the object's stride 0)."""
    mla = fmt in (MLA_KV, DSA_KV, MLA_LATENT, DSA_INDEX)
    planes, _, _, pe = _layer_planes(caches, fmt, vllm_two_major, kH, vH, dsaH)
    lmc_geo, N = _single_layer_lmc(staging, planes, pe, mla, token_major)
    es = staging.es

    def move(stg_off, obj, obj_off, nbytes):
        if to_objects:
            obj.data[obj_off: obj_off + nbytes] = staging.data[stg_off: stg_off + nbytes]
        else:
            staging.data[stg_off: stg_off + nbytes] = obj.data[obj_off: obj_off + nbytes]

    for obj, off, n in zip(objs, offsets, sizes):
        off, n = int(off), int(n)
        assert off + n <= N
        if mla:
            for plane, (l0, lstride) in zip(planes, lmc_geo):
                rb = plane[1]
                for t in range(n):
                    move(l0 + (off + t) * lstride, obj, _chunk_row_offset(plane, pe, n, t, es, token_major), rb)
        elif token_major:
            tok = lmc_geo[0][1]
            move(off * tok, obj, 0, n * tok)
        else:
            tok = lmc_geo[0][1]
            move(off * tok, obj, 0, n * tok)
            move(lmc_geo[1][0] + off * tok, obj, obj.strides[0] * es, n * tok)


def load_and_reshape_flash(kv: np.ndarray, num_layers: int, width: int, es: int,
                           key_cache: np.ndarray, value_cache: np.ndarray,
                           slots: np.ndarray, layer_idx: int, page2lmc: bool = True) -> None:
    """load_and_reshape_flash / reshape_and_cache_back_flash
    (csrc/mem_kernels.cpp:1341-1440): layer `layer_idx` of [2, L, T, W]
    against key_cache / value_cache viewed as [-1, W] rows."""
    T = int(slots.shape[0])
    rb = width * es
    ns = min(key_cache.size, value_cache.size) // rb
    valid = (slots >= 0) & (slots < ns)
    t = np.nonzero(valid)[0]
    s = slots[valid].astype(np.int64)
    for p, cache in enumerate((key_cache, value_cache)):
        base = (p * num_layers + layer_idx) * T * rb
        lm = kv[base: base + T * rb].reshape(T, rb)
        paged = cache[: ns * rb].reshape(ns, rb)
        if page2lmc:
            lm[t] = paged[s]
        else:
            paged[s] = lm[t]


def fused_required_size(fmt: int, use_mla: bool, L: int, T: int, W: int, kH: int, vH: int,
                        dsaH: int, es: int) -> int:
    """Bytes moved by the staging DMA copy (csrc/mem_kernels.cpp:143-165)."""
    if fmt in (MLA_KV, MLA_LATENT):
        return L * T * (kH + vH) * es
    if fmt == DSA_KV:
        return L * T * (kH + vH + dsaH) * es
    if fmt == DSA_INDEX:
        return L * T * dsaH * es
    return (1 if use_mla else 2) * L * T * W * es


def sparse_graph_kv_transfer(k_rows: np.ndarray, pe_rows: np.ndarray, k_bytes: int, pe_bytes: int,
                             slots: np.ndarray, selected: np.ndarray, row_counts, limits,
                             k_sources: Sequence, pe_sources: Sequence, chunk_size: int) -> None:
    """sparse_graph_kv_transfer (csrc/graph/sparse_graph_kernel.cpp:6-72):
    k_rows / pe_rows are the destination caches' bytes (flat rows);
    selected / slots are [requests, row_width]; row_counts[r] is the row's
    count (counts[r * stride]); k_sources / pe_sources list, per request and
    chunk (index r * chunks_per_request + chunk), a byte array or None."""
    R, width = selected.shape
    cpr = len(k_sources) // R
    dest_slots = min(k_rows.size // k_bytes, pe_rows.size // pe_bytes)
    for r in range(R):
        lim, cnt = int(limits[r]), int(row_counts[r])
        active = 0 if lim <= 0 or cnt <= 0 else min(cnt, width)
        for j in range(active):
            tok, dst = int(selected[r, j]), int(slots[r, j])
            if tok < 0 or tok >= lim or dst < 0 or dst >= dest_slots:
                continue
            chunk, off = divmod(tok, chunk_size)
            if chunk >= cpr:
                continue
            ks, ps = k_sources[r * cpr + chunk], pe_sources[r * cpr + chunk]
            if ks is None or ps is None:
                continue
            k_rows[dst * k_bytes:(dst + 1) * k_bytes] = ks[off * k_bytes:(off + 1) * k_bytes]
            pe_rows[dst * pe_bytes:(dst + 1) * pe_bytes] = ps[off * pe_bytes:(off + 1) * pe_bytes]


@dataclass
class C8Layer:
    """One indexer layer: key rows (key_bytes per physical slot), optional
    2-byte scales, slot factor, optional int32 block map, logical slots."""
    keys: np.ndarray
    scales: np.ndarray
    key_bytes: int
    slot_factor: int
    block_map: np.ndarray
    cache_slots: int


def indexer_c8_transfer(layers: Sequence[C8Layer], packets: Sequence[Sequence], offsets, counts,
                        slots: np.ndarray, capacity: int, from_npu: bool, fixed: bool) -> None:
    """indexer_c8_transfer_prepared / _group_ (csrc/indexer_c8/kernel.cpp:
    29-121): packets[l][c] is chunk c's packet of layer l (bytes, or None):
    `count` key rows then `count` 2-byte scales."""
    slot_count = slots.shape[0]
    for l, L in enumerate(layers):
        for c, packet in enumerate(packets[l]):
            start = c * capacity if fixed else int(offsets[c])
            count = min(slot_count - start, capacity) if fixed else int(counts[c])
            if (packet is None or count <= 0 or count > capacity or start < 0 or start > slot_count
                    or count > slot_count - start):
                continue
            for t in range(count):
                s = int(slots[start + t])
                if s < 0 or s >= L.cache_slots:
                    continue
                if L.block_map is not None:
                    phys = int(L.block_map[s // 128]) * 128 + s % 128
                else:
                    phys = s + (s // 128) * (L.slot_factor - 1) * 128
                if phys < 0 or phys + 1 > L.cache_slots * L.slot_factor:
                    continue
                kb = L.key_bytes
                pk, ck = slice(t * kb, (t + 1) * kb), slice(phys * kb, (phys + 1) * kb)
                if from_npu:
                    packet[pk] = L.keys[ck]
                else:
                    L.keys[ck] = packet[pk]
                if L.scales is not None:
                    ps, cs = slice(count * kb + 2 * t, count * kb + 2 * t + 2), slice(2 * phys, 2 * phys + 2)
                    if from_npu:
                        packet[ps] = L.scales[cs]
                    else:
                        L.scales[cs] = packet[ps]


def layerwise_dma_copy(spaces: Sequence[tuple], rows) -> None:
    """csrc/pybind.cpp:295-310: every (dst, src, bytes) row is one memcpy,
    applied in the given order (a later row wins where destinations
    overlap).  `spaces` lists (base_address, flat uint8 buffer) pairs; an
    address is resolved to the buffer whose range holds it."""

    def resolve(addr: int, n: int):
        for base, buf in spaces:
            if base <= addr and addr + n <= base + buf.size:
                return buf, addr - base
        raise ValueError(f"address {addr:#x}+{n} is outside every buffer")

    for dst, src, n in rows:
        if n == 0:
            continue
        sbuf, so = resolve(int(src), int(n))
        dbuf, do = resolve(int(dst), int(n))
        dbuf[do:do + n] = sbuf[so:so + n].copy()


def layerwise_dma_rows(chunk_addrs, chunk_tokens, cache_addrs, plane_bytes, block_ids, block_size,
                       starts, ends, device_to_host: bool):
    """Rows as the reference's planner binds them
    (lmcache_ascend/v1/npu_connector/layerwise_dma.py:147-211, 558-594),
    without its bundle-period edges: token ranges split at chunk bounds and
    where the next block id is not the previous one plus one; for range
    [t0, t1) of chunk c, one row per plane p with host side chunk_addrs[c] +
    chunk_tokens[c] * (sum of the earlier planes' row bytes) + (t0 -
    starts[c]) * plane_bytes[p], device side cache_addrs[p] + slot(t0) *
    plane_bytes[p], and plane_bytes[p] * (t1 - t0) bytes, where slot(t) =
    block_ids[t // block_size] * block_size + t % block_size."""
    rows = []
    plane_off = np.concatenate([[0], np.cumsum(plane_bytes)[:-1]])
    for c, (s, e) in enumerate(zip(starts, ends)):
        t = s
        while t < e:
            b = t // block_size
            while (b + 1) * block_size < e and block_ids[b + 1] == block_ids[b] + 1:
                b += 1
            t1 = min(e, (b + 1) * block_size)
            slot = block_ids[t // block_size] * block_size + t % block_size
            for p, pb in enumerate(plane_bytes):
                host = chunk_addrs[c] + chunk_tokens[c] * int(plane_off[p]) + (t - s) * pb
                dev = cache_addrs[p] + slot * pb
                n = (t1 - t) * pb
                rows.append((host, dev, n) if device_to_host else (dev, host, n))
            t = t1
    return rows
