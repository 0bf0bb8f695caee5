"""GPU parity of the CacheBlend layerwise retrieve pipeline, in the
reference connector's call pattern (lmcache_ascend/v1/npu_connector/
npu_connectors.py:556-689): per layer, pinned KV_2TD memory objects are
copied into a load buffer on a load stream, the K half of the buffer loaded
one step earlier is re-rotated in place by rotary_embedding_k_fused, and the
buffer of two steps earlier is scattered into the paged caches by
single_layer_kv_transfer, with a device-wide synchronize between steps and
two ping-pong buffers.

Expected caches: the oracle's fused re-rotation (float32, one rounding; the
kernel matches it exactly) and the oracle's single-layer scatter, applied
layer by layer on the CPU.  Every byte of every cache is compared, so rows
the slot mapping does not name must keep their values.
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


@pytest.fixture(scope="module")
def ops():
    import lmcache_amd

    return lmcache_amd.c_ops


def _tb(t: torch.Tensor) -> ok.TensorBytes:
    return ok.TensorBytes(to_bytes(t), list(t.shape), list(t.stride()), t.element_size())


@pytest.mark.parametrize("layers,chunk,n_obj", [(3, 128, 3), (5, 256, 2)])
def test_blend_layerwise_pipeline_vs_oracle(ops, layers, chunk, n_obj):
    gen = torch.Generator().manual_seed(layers * 10 + n_obj)
    NB, BS, H, D = 48, 16, 8, 128
    W = H * D
    T = chunk * n_obj
    caches = [(torch.randn((NB, BS, H, D), generator=gen).to(torch.bfloat16),
               torch.randn((NB, BS, H, D), generator=gen).to(torch.bfloat16)) for _ in range(layers)]
    gpu = [(k.to(DEV), v.to(DEV)) for k, v in caches]
    slots = torch.tensor(sample_slots(NB * BS, T, seed=T + layers), dtype=torch.int64)
    host = torch.randn((layers, n_obj, 2, chunk, W), generator=gen).to(torch.bfloat16).pin_memory()
    cache = orope.cos_sin_cache(T + 2048, D, 500000.0).to(torch.bfloat16)
    old = torch.arange(T, dtype=torch.int64)
    new = old + 1000
    dold, dnew, dcache, dslots = old.to(DEV), new.to(DEV), cache.to(DEV), slots.to(DEV)
    bufs = [torch.empty((2, T, W), dtype=torch.bfloat16, device=DEV) for _ in range(2)]
    load_stream = torch.cuda.Stream(DEV)

    compute, load = bufs
    mapping = {}
    for layer_id in range(layers + 2):
        if layer_id > 1:
            ops.single_layer_kv_transfer(mapping.pop(layer_id - 2), gpu[layer_id - 2], dslots, False, 2, False,
                                         False)
        if 0 < layer_id <= layers:
            torch.cuda.synchronize()
            compute, load = load, compute
            ops.rotary_embedding_k_fused(dold, dnew, compute[0], D, dcache, True)
            mapping[layer_id - 1] = compute
        if layer_id < layers:
            with torch.cuda.stream(load_stream):
                for c in range(n_obj):
                    load[0][c * chunk:(c + 1) * chunk].copy_(host[layer_id, c, 0], non_blocking=True)
                    load[1][c * chunk:(c + 1) * chunk].copy_(host[layer_id, c, 1], non_blocking=True)
    torch.cuda.synchronize()
    assert not mapping

    for layer in range(layers):
        buf = torch.cat([host[layer, c] for c in range(n_obj)], dim=1)  # [2, T, W]
        k32 = orope.fused_rerotate_f32(buf[0].float().numpy(), old.numpy(), new.numpy(), cache.float().numpy(),
                                       D, True)
        buf[0] = torch.from_numpy(orope.round_to(k32, torch.bfloat16)).to(torch.bfloat16)
        lmc = _tb(buf.contiguous())
        want = [_tb(caches[layer][0]), _tb(caches[layer][1])]
        ok.single_layer_kv_transfer(lmc, want, slots.numpy(), False, 2, False, False)
        assert np.array_equal(to_bytes(gpu[layer][0]), want[0].data), f"layer {layer} K"
        assert np.array_equal(to_bytes(gpu[layer][1]), want[1].data), f"layer {layer} V"
