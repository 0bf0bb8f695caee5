"""Helpers shared by the KV gather/scatter tests: byte views of tensors,
seeded cache builders and pointer tables (as the reference's connector builds
them, lmcache_ascend/v1/npu_connector/npu_connectors.py:862-979)."""

from __future__ import annotations

import random
from typing import List, Sequence

import numpy as np
import torch


def to_bytes(t: torch.Tensor) -> np.ndarray:
    """Flat uint8 copy of a tensor's storage bytes in logical (row-major) order."""
    t = t.detach().contiguous().cpu()
    return t.view(-1).view(torch.uint8).numpy().copy()


def from_bytes(b: np.ndarray, like: torch.Tensor) -> torch.Tensor:
    return torch.from_numpy(b.copy()).view(like.dtype).reshape(like.shape)


def randn_bf16(shape, gen: torch.Generator, std: float = 1.0) -> torch.Tensor:
    return (torch.randn(shape, generator=gen, dtype=torch.float32) * std).to(torch.bfloat16)


def ptr_table(tensors: Sequence[torch.Tensor], device) -> torch.Tensor:
    return torch.tensor([t.data_ptr() for t in tensors], dtype=torch.int64, device=device)


def block_slots(block_ids: Sequence[int], block_size: int, lengths: Sequence[int] = None) -> List[int]:
    """Slots of requests laid out in the given blocks (contiguous within a block)."""
    out = []
    if lengths is None:
        for b in block_ids:
            out.extend(range(b * block_size, (b + 1) * block_size))
        return out
    it = iter(block_ids)
    for n in lengths:
        nb = (n + block_size - 1) // block_size
        blocks = [next(it) for _ in range(nb)]
        for i in range(n):
            out.append(blocks[i // block_size] * block_size + i % block_size)
    return out


def sample_slots(n_slots: int, n: int, seed: int) -> List[int]:
    rng = random.Random(seed)
    return rng.sample(range(n_slots), n)
