"""GPU tests of the format helpers (lmcache_amd/formats.py).

* CacheGen chunks: encode_chunk's CDF, per-stream lengths and concatenated
  streams are bit-exact against the CPU oracle's calculate_cdf / encode /
  concatenation; chunk -> bytes -> chunk -> decode_chunk returns the
  symbols (the reference's round trip, tests/v1/test_cachegen_kernels.py:
  242-345, at the 2 x 32-layer K+V stacking).
* Memory objects: every layer slice of a KV_2LTD object written by
  multi_layer_kv_transfer equals the KV_T2D / KV_2TD object that
  single_layer_kv_transfer writes for that layer, in the layout the format
  names.
"""

import numpy as np
import pytest
import torch

from kvutil import ptr_table, randn_bf16, sample_slots
from oracle import cachegen as oc

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def F():
    from lmcache_amd import formats

    return formats


@pytest.mark.parametrize("L,T,C,nb", [(8, 256, 64, 32), (2, 1, 32, 16), (64, 256, 128, 16)])
def test_chunk_codec_round_trip_vs_oracle(F, L, T, C, nb):
    rng = np.random.default_rng(L * T + C)
    x = rng.normal(0, 2, size=(L, T, C)).astype(np.float32)
    sym = oc.quantize(x, nb)
    chunk = F.encode_chunk(torch.from_numpy(sym).to(DEV), nb)
    torch.cuda.synchronize()
    cdf = oc.calculate_cdf(sym, nb)
    rows, lens = oc.encode(cdf, sym, 2 * T)
    stream, _ = oc.concat_streams(rows, lens)
    assert np.array_equal(chunk.cdf.cpu().numpy(), cdf)
    assert np.array_equal(chunk.lengths.cpu().numpy(), lens)
    assert np.array_equal(chunk.streams.cpu().numpy(), stream)
    back = F.CacheGenChunk.from_bytes(chunk.to_bytes(), device=DEV)
    out = F.decode_chunk(back)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), sym)


def _quantize_planes(x, bins):
    """Symmetric per-(plane, channel) quantiser over a chunk's tokens into
    [0, bins - 2] (this library's own; the reference's sits in upstream
    LMCache)."""
    half = (bins // 2 - 1).to(torch.float32).view(-1, 1, 1)
    amax = x.abs().amax(dim=1, keepdim=True).clamp_min(1e-30)
    return (torch.round(x / amax * half) + half).to(torch.uint8)


@pytest.mark.parametrize("n_tokens", [1, 20, 256, 8000])
@pytest.mark.parametrize("n_layers", [1, 28])
@pytest.mark.parametrize("chunk_size", [128, 256])
@pytest.mark.parametrize("num_heads", [1, 8])
def test_chunked_encode_into_decode(F, n_tokens, n_layers, chunk_size, num_heads):
    """The reference's end-to-end CacheGen test, in its parameter grid
    (tests/v1/test_cachegen_kernels.py:242-345): bf16 K and V of
    [n_layers, n_tokens, num_heads x 128] from N(0, 2), K layers 0-9 at 32
    bins and the rest at 16, V layers 0-1 at 32 and the rest at 16 (one
    layer: 32 for both), cut into chunks of chunk_size tokens; each chunk is
    quantised, encoded, serialized, read back and decoded, and the decoded
    symbols equal the quantised ones."""
    torch.manual_seed(n_tokens * 7 + n_layers * 3 + chunk_size + num_heads)
    C = num_heads * 128
    kv = (torch.randn((n_layers, 2, n_tokens, C), device=DEV) * 2).to(torch.bfloat16)
    if n_layers == 1:
        kb = vb = torch.tensor([32], device=DEV)
    else:
        kb = torch.full((n_layers,), 16, device=DEV)
        kb[:10] = 32
        vb = torch.full((n_layers,), 16, device=DEV)
        vb[:2] = 32
    bins = torch.cat([kb, vb])
    for t0 in range(0, n_tokens, chunk_size):
        part = kv[:, :, t0:t0 + chunk_size].float()
        planes = torch.cat([part[:, 0], part[:, 1]]).contiguous()  # [2L, T, C]: K layers, then V
        sym = _quantize_planes(planes, bins)
        chunk = F.encode_chunk(sym, 32)
        back = F.CacheGenChunk.from_bytes(chunk.to_bytes(), device=DEV)
        assert back.shape == (2 * n_layers, sym.shape[1], C)
        out = F.decode_chunk(back)
        torch.cuda.synchronize()
        assert torch.equal(out, sym), (t0, n_tokens)


def test_chunk_encode_refuses_cpu_symbols(F):
    with pytest.raises(ValueError):
        F.encode_chunk(torch.zeros(1, 4, 32, dtype=torch.uint8), 16)


@pytest.mark.parametrize("fmt", [1, 2])
def test_kv_2ltd_layers_equal_single_layer_objects(F, fmt):
    from lmcache_amd import c_ops
    from lmcache_amd.kv_format import KVCacheFormat

    gen = torch.Generator().manual_seed(fmt)
    L, NB, BS, H, D, T = 4, 32, 16, 2, 64, 100
    W = H * D
    if fmt == 1:
        layers = [randn_bf16([2, NB, BS, H, D], gen).to(DEV) for _ in range(L)]
        flat = layers
        per_layer = layers
    else:
        layers = [(randn_bf16([NB, BS, H, D], gen).to(DEV), randn_bf16([NB, BS, H, D], gen).to(DEV))
                  for _ in range(L)]
        flat = [t for kv in layers for t in kv]
        per_layer = layers
    slots = torch.tensor(sample_slots(NB * BS, T, seed=3), dtype=torch.int64, device=DEV)
    shape = F.memory_obj_shape(KVCacheFormat(fmt), L, T, hidden_dim_size=W)
    obj = torch.zeros(shape, dtype=torch.bfloat16, device=DEV)
    F.check_memory_obj(obj, F.MemoryFormat.KV_2LTD, F.memory_format_for(False), num_layers=L, width=W)
    c_ops.multi_layer_kv_transfer(obj, ptr_table(flat, DEV), slots, torch.device(DEV), NB * BS, True, False, fmt,
                                  W, W, 0)
    for fmt1 in (F.MemoryFormat.KV_T2D, F.MemoryFormat.KV_2TD):
        tm = F.single_layer_token_major(fmt1)
        for li in range(L):
            one = torch.zeros((T, 2, W) if tm else (2, T, W), dtype=torch.bfloat16, device=DEV)
            F.check_memory_obj(one, fmt1, fmt1, width=W)
            c_ops.single_layer_kv_transfer(one, per_layer[li], slots, True, fmt, token_major=tm,
                                           vllm_two_major=True)
            torch.cuda.synchronize()
            want = obj[:, li].transpose(0, 1) if tm else obj[:, li]
            assert torch.equal(one.view(torch.int16), want.contiguous().view(torch.int16))
            assert F.num_tokens_of(fmt1, one.shape) == T
