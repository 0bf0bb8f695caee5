"""CPU oracle for the paged-KV gather/scatter ops.  TEST INFRASTRUCTURE ONLY.

This module is the checker the tests, `__graft_entry__.smoke()` and the
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
    raise RuntimeError(f"Unsupported KVCacheFormat: {fmt}")


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


def single_layer_kv_transfer(lmc: TensorBytes, caches: List[TensorBytes], slots: np.ndarray,
                             direction: bool, fmt: int, token_major: bool = False,
                             vllm_two_major: bool = False, kH: int = 0, vH: int = 0,
                             dsaH: int = 0) -> None:
    """single_layer_kv_transfer (csrc/mem_kernels.cpp:265-334), in place.

    Strides follow csrc/utils.cpp:212-285; MLA/DSA hidden-dim defaults and the
    stacked-plane LMC layout follow csrc/utils.cpp:310-357.
    """
    es = caches[0].es
    T = int(slots.shape[0])
    rows = []  # (lmc byte offsets[T], paged buffer, paged byte offsets[T], row bytes)
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
        tensors = [k, v, dsa]
        plane_elems = sum(widths)
        N = lmc.numel // plane_elems
        assert T <= N, "LMC buffer too small"
        off = 0
        num_slots = None
        for w, tb in zip(widths, tensors):
            if w > 0 and tb is not None:
                t = np.arange(T, dtype=np.int64)
                lmc_off = (off + t * w) * es
                rows.append((lmc_off, tb, w * es, 0, w * es, 0))
                ns = tb.numel // w
                num_slots = ns if num_slots is None else min(num_slots, ns)
            off += N * w
        block_size = 0
    else:
        k = caches[0]
        H, D, BS = k.shape[-2], k.shape[-1], k.shape[-3]
        W = H * D
        if token_major:
            tok_stride, val_off = lmc.strides[0], lmc.strides[1]
        else:
            tok_stride, val_off = lmc.strides[1], lmc.strides[0]
        t = np.arange(T, dtype=np.int64)
        if fmt == MERGED_KV:
            blk = k.strides[1] if vllm_two_major else k.strides[0]
            voff = k.strides[0] if vllm_two_major else k.strides[1]
            NB = k.shape[1] if vllm_two_major else k.shape[0]
            rows.append((t * tok_stride * es, k, W * es, 0, W * es, blk * es))
            rows.append(((t * tok_stride + val_off) * es, k, W * es, voff * es, W * es, blk * es))
            num_slots = NB * BS
        else:
            v = caches[1]
            rows.append((t * tok_stride * es, k, W * es, 0, W * es, k.strides[0] * es))
            rows.append(((t * tok_stride + val_off) * es, v, W * es, 0, W * es, v.strides[0] * es))
            num_slots = min(k.shape[0], v.shape[0]) * BS
        block_size = BS
    valid = (slots >= 0) & (slots < num_slots)
    s = slots[valid].astype(np.int64)
    for lmc_off, tb, rb, poff, pitch, blk in rows:
        if block_size:
            p_off = poff + (s // block_size) * blk + (s % block_size) * pitch
        else:
            p_off = poff + s * pitch
        l_off = lmc_off[valid]
        if direction:
            _scatter_rows(lmc.data, l_off, _gather_rows(tb.data, p_off, rb))
        else:
            _scatter_rows(tb.data, p_off, _gather_rows(lmc.data, l_off, rb))


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
