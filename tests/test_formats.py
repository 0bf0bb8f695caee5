"""CPU tests of the memory-object format helpers and the CacheGen chunk
container (lmcache_amd/formats.py): shapes from the connector's get_shape
(lmcache_ascend/v1/npu_connector/npu_connectors.py:1472-1485), token counts
(lmcache_ascend/v1/proxy_memory_obj.py:452-462), the connector's format
checks, and the chunk's explicit binary layout (round trip, corrupted and
truncated input refused).  No GPU call is made."""

import struct

import pytest
import torch

from lmcache_amd import formats as F
from lmcache_amd.kv_format import KVCacheFormat


def test_memory_obj_shapes():
    # Llama-3-8B shape: [2, 32, T, 1024]; DeepSeek MLA: [1, 61, T, 512 + 64]
    assert F.memory_obj_shape(KVCacheFormat.SEPARATE_KV, 32, 256, hidden_dim_size=1024) == (2, 32, 256, 1024)
    assert F.memory_obj_shape(KVCacheFormat.MERGED_KV, 4, 7, hidden_dim_size=64) == (2, 4, 7, 64)
    assert F.memory_obj_shape(KVCacheFormat.MLA_KV, 61, 2048, kv_lora_rank=512, qk_rope_head_dim=64) == (
        1, 61, 2048, 576)
    assert F.memory_obj_shape(3, 61, 16, kv_lora_rank=512, qk_rope_head_dim=64) == (1, 61, 16, 576)
    assert F.memory_obj_shape(KVCacheFormat.DSA_KV, 61, 16, kv_lora_rank=512, qk_rope_head_dim=64,
                              dsa_head_dim=128) == (1, 61, 16, 704)


def test_tags_and_token_counts():
    assert F.memory_format_for(True) is F.MemoryFormat.KV_MLA_FMT
    assert F.memory_format_for(False) is F.MemoryFormat.KV_2LTD
    assert F.num_tokens_of(F.MemoryFormat.KV_2LTD, (2, 32, 256, 1024)) == 256
    assert F.num_tokens_of(F.MemoryFormat.KV_MLA_FMT, (1, 61, 99, 576)) == 99
    assert F.num_tokens_of(F.MemoryFormat.KV_2TD, (2, 17, 1024)) == 17
    assert F.num_tokens_of(F.MemoryFormat.KV_T2D, (17, 2, 1024)) == 17
    assert F.num_tokens_of(F.MemoryFormat.KV_T2D, (2, 1024)) == 0
    assert F.single_layer_token_major(F.MemoryFormat.KV_T2D) is True
    assert F.single_layer_token_major(F.MemoryFormat.KV_2TD) is False
    with pytest.raises(ValueError):
        F.single_layer_token_major(F.MemoryFormat.KV_2LTD)


def test_connector_checks():
    obj = torch.zeros(2, 4, 8, 64)
    F.check_memory_obj(obj, F.MemoryFormat.KV_2LTD, F.MemoryFormat.KV_2LTD, num_layers=4, width=64)
    with pytest.raises(ValueError, match="tagged KV_MLA_FMT; this transfer takes KV_2LTD"):
        F.check_memory_obj(obj, F.MemoryFormat.KV_MLA_FMT, F.MemoryFormat.KV_2LTD)
    with pytest.raises(ValueError, match="layers"):
        F.check_memory_obj(obj, F.MemoryFormat.KV_2LTD, F.MemoryFormat.KV_2LTD, num_layers=3)
    with pytest.raises(ValueError, match="wide"):
        F.check_memory_obj(obj, F.MemoryFormat.KV_2LTD, F.MemoryFormat.KV_2LTD, width=32)
    with pytest.raises(ValueError, match="leading plane"):
        F.check_memory_obj(torch.zeros(1, 4, 8, 64), F.MemoryFormat.KV_2LTD, F.MemoryFormat.KV_2LTD)
    with pytest.raises(ValueError, match="4-D"):
        F.check_memory_obj(torch.zeros(2, 8, 64), F.MemoryFormat.KV_MLA_FMT, F.MemoryFormat.KV_MLA_FMT)
    F.check_memory_obj(torch.zeros(8, 2, 64), F.MemoryFormat.KV_T2D, F.MemoryFormat.KV_T2D)
    with pytest.raises(ValueError, match=r"\[T, 2, W\]"):
        F.check_memory_obj(torch.zeros(2, 8, 64), F.MemoryFormat.KV_T2D, F.MemoryFormat.KV_T2D)


def _chunk(L=3, T=5, C=4, nb=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    cdf = torch.randint(-32768, 32767, (L, C, nb + 1), dtype=torch.int16, generator=g)
    lengths = torch.randint(0, 9, (L, C), dtype=torch.int32, generator=g)
    streams = torch.randint(0, 256, (int(lengths.sum()),), dtype=torch.uint8, generator=g)
    return F.CacheGenChunk(cdf, lengths, streams, T)


def test_chunk_round_trip_and_layout():
    c = _chunk()
    data = c.to_bytes()
    head = struct.unpack_from("<4sHxxIIIIQ", data, 0)
    assert head == (b"LMCG", 1, 3, 5, 4, 9, c.streams.numel())
    assert len(data) == 32 + 3 * 4 * 9 * 2 + 3 * 4 * 4 + c.streams.numel()
    # the arrays follow the header, little-endian, in the order cdf, lengths, streams
    assert data[32:34] == int(c.cdf.view(-1)[0]).to_bytes(2, "little", signed=True)
    back = F.CacheGenChunk.from_bytes(data)
    assert back.shape == (3, 5, 4)
    assert torch.equal(back.cdf, c.cdf) and torch.equal(back.lengths, c.lengths)
    assert torch.equal(back.streams, c.streams) and back.num_tokens == 5


def test_chunk_without_stream_bytes():
    c = F.CacheGenChunk(torch.zeros(1, 2, 3, dtype=torch.int16), torch.zeros(1, 2, dtype=torch.int32),
                        torch.zeros(0, dtype=torch.uint8), 0)
    back = F.CacheGenChunk.from_bytes(c.to_bytes())
    assert back.streams.numel() == 0 and back.shape == (1, 0, 2)


def test_corrupted_chunks_are_refused():
    data = _chunk().to_bytes()
    with pytest.raises(ValueError, match="header"):
        F.CacheGenChunk.from_bytes(data[:20])
    with pytest.raises(ValueError, match="known version"):
        F.CacheGenChunk.from_bytes(b"XXXX" + data[4:])
    with pytest.raises(ValueError, match="size does not match"):
        F.CacheGenChunk.from_bytes(data[:-1])
    with pytest.raises(ValueError, match="size does not match"):
        F.CacheGenChunk.from_bytes(data + b"\0")
    # lengths that no longer add up to the stream bytes
    bad = bytearray(data)
    off = 32 + 3 * 4 * 9 * 2
    bad[off:off + 4] = (int.from_bytes(bad[off:off + 4], "little") + 1).to_bytes(4, "little")
    with pytest.raises(ValueError, match="lengths"):
        F.CacheGenChunk.from_bytes(bytes(bad))
    c = _chunk()
    c.streams = c.streams[:-1]
    with pytest.raises(ValueError, match="add up"):
        c.to_bytes()
