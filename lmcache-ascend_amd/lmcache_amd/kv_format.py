"""KV cache storage formats: the integer contract between the connector and
the gather/scatter ops (lmcache_ascend/v1/kv_format.py:13-219).

The values must equal the reference's, since callers pass `fmt.value` as
`kvcache_format_raw`.  `pointers_per_layer` is what the connector puts into
the per-layer pointer table (the reference's Python get_kv_size, which counts
pointers: MERGED = 1); `planes` counts the rows copied per (layer, token)
(the reference's C++ kv_size, csrc/utils.cpp:59-83: MERGED = 2).
"""

from __future__ import annotations

from enum import IntEnum
from typing import Sequence, Tuple, Union

import torch


class KVCacheFormat(IntEnum):
    UNDEFINED = 0
    MERGED_KV = 1     # layer: [2, NB, BS, H, D] (or [NB, 2, BS, H, D])
    SEPARATE_KV = 2   # layer: (K, V), each [NB, BS, H, D]
    MLA_KV = 3        # layer: (k_nope [NB, BS, 1, kv_lora], k_pe [NB, BS, 1, rope])
    DSA_KV = 4        # layer: (k_nope, k_pe, indexer_k)
    MLA_LATENT = 5    # two-group MLA latent pair
    DSA_INDEX = 6     # two-group indexer only: (indexer_k,)

    def pointers_per_layer(self) -> int:
        if self == KVCacheFormat.DSA_KV:
            return 3
        if self in (KVCacheFormat.SEPARATE_KV, KVCacheFormat.MLA_KV, KVCacheFormat.MLA_LATENT):
            return 2
        if self in (KVCacheFormat.MERGED_KV, KVCacheFormat.DSA_INDEX):
            return 1
        return 0

    def planes(self) -> int:
        if self == KVCacheFormat.DSA_KV:
            return 3
        if self == KVCacheFormat.DSA_INDEX:
            return 1
        if self == KVCacheFormat.UNDEFINED:
            return 0
        return 2

    def is_tuple_format(self) -> bool:
        return self in (
            KVCacheFormat.SEPARATE_KV,
            KVCacheFormat.MLA_KV,
            KVCacheFormat.DSA_KV,
            KVCacheFormat.MLA_LATENT,
            KVCacheFormat.DSA_INDEX,
        )

    @staticmethod
    def detect(
        kvcaches: Sequence[Union[torch.Tensor, Tuple[torch.Tensor, ...]]],
        use_mla: bool = False,
        dsa_two_groups: bool = False,
    ) -> "KVCacheFormat":
        """Format of a vLLM kv_caches list, by structure
        (lmcache_ascend/v1/kv_format.py:126-219)."""
        if not kvcaches:
            return KVCacheFormat.UNDEFINED
        first = kvcaches[0]
        if isinstance(kvcaches, list) and len(kvcaches) == 2:
            if isinstance(first, torch.Tensor) and first.ndim == 5:
                return KVCacheFormat.SEPARATE_KV  # layer-concatenated K, V
        if isinstance(first, tuple):
            n = len(first)
            if n == 3 and all(isinstance(t, torch.Tensor) for t in first):
                if first[0].shape != first[1].shape:
                    return KVCacheFormat.DSA_KV
            if n == 1 and dsa_two_groups and isinstance(first[0], torch.Tensor):
                return KVCacheFormat.DSA_INDEX
            if n == 2 and all(isinstance(t, torch.Tensor) for t in first):
                if use_mla or first[0].shape != first[1].shape:
                    return KVCacheFormat.MLA_LATENT if dsa_two_groups else KVCacheFormat.MLA_KV
                return KVCacheFormat.SEPARATE_KV
            return KVCacheFormat.SEPARATE_KV
        if isinstance(first, torch.Tensor) and first.ndim == 5:
            if first.shape[0] == 2 or first.shape[1] == 2:
                return KVCacheFormat.MERGED_KV
        return KVCacheFormat.UNDEFINED
