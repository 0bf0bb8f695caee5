"""Writes tests/golden/kv_c1.json: digests of the C1 plumbing case run through
the gather/scatter oracle.

C1: 4 layers, 8 KV heads x 128, bf16, SEPARATE_KV caches [64, 16, 8, 128] per
layer and plane, N(0,1) from torch.Generator seed 0 drawn K0, V0, K1, ...;
16 distinct blocks from randperm(64), slots contiguous inside each block
(256 tokens); store into a zeroed [2, 4, 256, 1024] memory object, then
retrieve into zeroed caches.

    python tests/golden/gen_kv_golden.py
"""

from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

from oracle import kv_transfer as ok  # noqa: E402

L, NB, BS, H, D, T = 4, 64, 16, 8, 128, 256
W = H * D


def c1_inputs():
    g = torch.Generator().manual_seed(0)
    caches = []
    for _ in range(L):
        k = torch.randn((NB, BS, H, D), generator=g, dtype=torch.float32).to(torch.bfloat16)
        v = torch.randn((NB, BS, H, D), generator=g, dtype=torch.float32).to(torch.bfloat16)
        caches.append((k, v))
    blocks = torch.randperm(NB, generator=g)[:16]
    slots = (blocks[:, None] * BS + torch.arange(BS)[None, :]).reshape(-1).to(torch.int64)
    return caches, slots


def _bytes(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(-1).view(torch.uint8).numpy().copy()


def _sha(a: np.ndarray) -> str:
    return hashlib.sha256(a.tobytes()).hexdigest()


def c1_outputs():
    caches, slots = c1_inputs()
    table = [_bytes(x) for kv in caches for x in kv]
    lmc = np.zeros(2 * L * T * W * 2, np.uint8)
    s = slots.numpy()
    ok.multi_layer_kv_transfer(lmc, table, s, NB * BS, True, False, 2, L, W, 2)
    zero = [np.zeros_like(x) for x in table]
    ok.multi_layer_kv_transfer(lmc, zero, s, NB * BS, False, False, 2, L, W, 2)
    return caches, slots, lmc, zero


def c1_digests() -> dict:
    _, slots, lmc, zero = c1_outputs()
    return {
        "case": "C1 SEPARATE_KV L=4 T=256 W=1024 bf16 seed=0",
        "slots_head": [int(x) for x in slots[:20]],
        "lmc_sha256": _sha(lmc),
        "retrieved_caches_sha256": _sha(np.concatenate(zero)),
        "lmc_row_p1_l3_t255_first8": [int(x) for x in lmc.reshape(2, L, T, W * 2)[1, 3, 255, :8]],
    }


if __name__ == "__main__":
    out = os.path.join(HERE, "kv_c1.json")
    with open(out, "w") as f:
        json.dump(c1_digests(), f, indent=1)
        f.write("\n")
    print(f"wrote {out}")
