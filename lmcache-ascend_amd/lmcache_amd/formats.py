"""Data formats either side of the ops: LMCache memory-object layouts and a
CacheGen chunk container.

Memory objects.  LMCache tags every memory object with a `MemoryFormat`
(upstream `lmcache.v1.memory_management`, not part of the reference tree);
the connector checks the tag before a transfer and sets it after one
(lmcache_ascend/v1/npu_connector/npu_connectors.py:1007-1017, 1100, 1258)
and sizes objects with `get_shape` (:1472-1485).  Each format is a tensor
layout that one family of ops reads and writes:

  KV_2LTD     [2, L, T, W]            multi_layer_kv_transfer (MERGED /
                                      SEPARATE), fused_..., load_and_reshape_flash
  KV_MLA_FMT  [1, L, T, kH + vH (+ dsaH)]  multi_layer_kv_transfer (MLA / DSA)
  KV_T2D      [T, 2, W]               single_layer_kv_transfer(token_major=True)
  KV_2TD      [2, T, W]               single_layer_kv_transfer(token_major=False)

Only the names are shared with LMCache: this module's enum values are its
own (upstream's integers are outside the reference tree).

CacheGen chunks.  Upstream LMCache's CacheGen serde wraps the codec ops in
`CacheGenGPUEncoderOutput` (call sites tests/v1/test_cachegen_kernels.py:
299-335): the CDF, the encoded streams concatenated in (layer, channel)
order, and per-stream lengths, which `decode_fast_prefsum` takes as
inclusive prefix sums.  `CacheGenChunk` holds the same pieces and
serializes them with an explicit little-endian layout (a magic, a version,
the dimensions, then the raw arrays), so loading bytes runs no code from
them.  Byte-level interop with upstream's serialized objects is not claimed:
upstream defines that format and is absent here.
"""

from __future__ import annotations

import struct
from dataclasses import dataclass
from enum import Enum
from typing import Tuple

import torch

from . import c_ops
from .kv_format import KVCacheFormat

__all__ = [
    "MemoryFormat",
    "memory_obj_shape",
    "memory_format_for",
    "num_tokens_of",
    "check_memory_obj",
    "single_layer_token_major",
    "CacheGenChunk",
    "encode_chunk",
    "decode_chunk",
]


class MemoryFormat(Enum):
    KV_2LTD = "KV_2LTD"
    KV_MLA_FMT = "KV_MLA_FMT"
    KV_T2D = "KV_T2D"
    KV_2TD = "KV_2TD"


def memory_obj_shape(kv_format: KVCacheFormat, num_layers: int, num_tokens: int, hidden_dim_size: int = 0,
                     kv_lora_rank: int = 0, qk_rope_head_dim: int = 0, dsa_head_dim: int = 0) -> torch.Size:
    """Shape of a multi-layer memory object for `num_tokens` tokens
    (npu_connectors.py:1472-1485): [1, L, T, kv_lora + rope (+ dsa)] for
    MLA_KV / DSA_KV, else [2, L, T, hidden_dim_size]."""
    kv_format = KVCacheFormat(kv_format)
    if kv_format == KVCacheFormat.MLA_KV:
        return torch.Size([1, num_layers, num_tokens, kv_lora_rank + qk_rope_head_dim])
    if kv_format == KVCacheFormat.DSA_KV:
        return torch.Size([1, num_layers, num_tokens, kv_lora_rank + qk_rope_head_dim + dsa_head_dim])
    return torch.Size([2, num_layers, num_tokens, hidden_dim_size])


def memory_format_for(use_mla: bool) -> MemoryFormat:
    """The tag the connector expects on multi-layer objects
    (npu_connectors.py:1005-1017) and sets after a store (:1100, 1258)."""
    return MemoryFormat.KV_MLA_FMT if use_mla else MemoryFormat.KV_2LTD


def num_tokens_of(fmt: MemoryFormat, shape) -> int:
    """Token count of an object of this format and shape
    (lmcache_ascend/v1/proxy_memory_obj.py:452-462)."""
    shape = tuple(shape)
    if fmt in (MemoryFormat.KV_2LTD, MemoryFormat.KV_MLA_FMT):
        return shape[2] if len(shape) == 4 else 0
    if fmt == MemoryFormat.KV_2TD:
        return shape[1] if len(shape) == 3 else 0
    if fmt == MemoryFormat.KV_T2D:
        return shape[0] if len(shape) == 3 else 0
    return 0


def single_layer_token_major(fmt: MemoryFormat) -> bool:
    """The `token_major` flag single_layer_kv_transfer needs for an object
    of this format."""
    if fmt == MemoryFormat.KV_T2D:
        return True
    if fmt == MemoryFormat.KV_2TD:
        return False
    raise ValueError(f"{fmt.name} is not a single-layer format")


def check_memory_obj(tensor: torch.Tensor, fmt: MemoryFormat, expected_fmt: MemoryFormat,
                     num_layers: int = 0, width: int = 0) -> None:
    """The connector's checks before a transfer (npu_connectors.py:1005-1017):
    the object carries the expected tag, and its tensor has that format's
    rank and, where given, its layer count and row width."""
    if fmt != expected_fmt:
        raise ValueError(f"memory object is tagged {fmt.name}; this transfer takes {expected_fmt.name} objects")
    rank = 4 if fmt in (MemoryFormat.KV_2LTD, MemoryFormat.KV_MLA_FMT) else 3
    if tensor.dim() != rank:
        raise ValueError(f"{fmt.name} objects are {rank}-D, got shape {tuple(tensor.shape)}")
    lead = {MemoryFormat.KV_2LTD: 2, MemoryFormat.KV_MLA_FMT: 1}.get(fmt)
    if lead is not None and tensor.shape[0] != lead:
        raise ValueError(f"{fmt.name} objects have {lead} leading plane(s), got shape {tuple(tensor.shape)}")
    if fmt == MemoryFormat.KV_T2D and tensor.shape[1] != 2:
        raise ValueError(f"KV_T2D objects are [T, 2, W], got shape {tuple(tensor.shape)}")
    if fmt == MemoryFormat.KV_2TD and tensor.shape[0] != 2:
        raise ValueError(f"KV_2TD objects are [2, T, W], got shape {tuple(tensor.shape)}")
    if num_layers and rank == 4 and tensor.shape[1] != num_layers:
        raise ValueError(f"object holds {tensor.shape[1]} layers, expected {num_layers}")
    if width and tensor.shape[-1] != width:
        raise ValueError(f"object rows are {tensor.shape[-1]} wide, expected {width}")


# ---------------------------------------------------------------------------
# CacheGen chunks
# ---------------------------------------------------------------------------

_MAGIC = b"LMCG"
_VERSION = 1
# magic, version, layers, tokens, channels, cdf entries per stream, stream bytes
_HEADER = struct.Struct("<4sHxxIIIIQ")


@dataclass
class CacheGenChunk:
    """One encoded chunk: `cdf` int16 [L, C, n_bins + 1], `lengths` int32
    [L, C] bytes per stream, `streams` uint8 [sum(lengths)] (the streams
    concatenated in (layer, channel) order), and the token count."""

    cdf: torch.Tensor
    lengths: torch.Tensor
    streams: torch.Tensor
    num_tokens: int

    @property
    def shape(self) -> Tuple[int, int, int]:
        return int(self.cdf.shape[0]), int(self.num_tokens), int(self.cdf.shape[1])

    def to_bytes(self) -> bytes:
        L, T, C = self.shape
        cdf = self.cdf.detach().to("cpu", torch.int16).contiguous()
        lengths = self.lengths.detach().to("cpu", torch.int32).contiguous()
        streams = self.streams.detach().to("cpu", torch.uint8).contiguous()
        if int(lengths.sum()) != streams.numel():
            raise ValueError("stream lengths do not add up to the stream bytes")
        head = _HEADER.pack(_MAGIC, _VERSION, L, T, C, int(cdf.shape[2]), streams.numel())
        return b"".join([head, cdf.numpy().tobytes(), lengths.numpy().tobytes(), streams.numpy().tobytes()])

    @staticmethod
    def from_bytes(data: bytes, device=None) -> "CacheGenChunk":
        if len(data) < _HEADER.size:
            raise ValueError("CacheGen chunk is shorter than its header")
        magic, version, L, T, C, E, n = _HEADER.unpack_from(data, 0)
        if magic != _MAGIC or version != _VERSION:
            raise ValueError("not a CacheGen chunk of a known version")
        if E < 2 or E > 65:
            raise ValueError(f"CacheGen chunk has {E} CDF entries per stream")
        sizes = (L * C * E * 2, L * C * 4, n)
        if len(data) != _HEADER.size + sum(sizes):
            raise ValueError("CacheGen chunk size does not match its header")
        off = _HEADER.size
        cdf = _array(data, off, sizes[0], torch.int16, (L, C, E))
        off += sizes[0]
        lengths = _array(data, off, sizes[1], torch.int32, (L, C))
        off += sizes[1]
        streams = _array(data, off, n, torch.uint8, (n,))
        if int(lengths.to(torch.int64).sum()) != n or bool((lengths < 0).any()):
            raise ValueError("CacheGen chunk stream lengths do not match its stream bytes")
        chunk = CacheGenChunk(cdf, lengths, streams, int(T))
        return chunk.to(device) if device is not None else chunk

    def to(self, device) -> "CacheGenChunk":
        return CacheGenChunk(self.cdf.to(device), self.lengths.to(device), self.streams.to(device),
                             self.num_tokens)


def _array(data: bytes, off: int, size: int, dtype, shape) -> torch.Tensor:
    if size == 0:
        return torch.empty(shape, dtype=dtype)
    return torch.frombuffer(bytearray(data[off:off + size]), dtype=dtype).view(shape)


def encode_chunk(symbols: torch.Tensor, n_bins: int, max_stream_bytes: int = 0) -> CacheGenChunk:
    """Encodes uint8 symbols [L, T, C] (values below n_bins) on the GPU:
    calculate_cdf, encode_fast_new into per-stream rows of
    `max_stream_bytes` (default: enough for 16 bits per symbol), then the
    rows' used bytes concatenated in (layer, channel) order."""
    if not symbols.is_cuda or symbols.dtype != torch.uint8 or symbols.dim() != 3:
        raise ValueError("encode_chunk takes uint8 GPU symbols [L, T, C]")
    L, T, C = symbols.shape
    cap = int(max_stream_bytes) or 2 * T
    cdf = c_ops.calculate_cdf(symbols, int(n_bins))
    rows = torch.zeros((L, C, cap), dtype=torch.uint8, device=symbols.device)
    lengths = torch.zeros((L, C), dtype=torch.int32, device=symbols.device)
    c_ops.encode_fast_new(cdf, symbols, rows, lengths)
    used = torch.arange(cap, device=symbols.device).view(1, 1, cap) < lengths.unsqueeze(-1)
    return CacheGenChunk(cdf, lengths, rows[used], int(T))


def decode_chunk(chunk: CacheGenChunk) -> torch.Tensor:
    """Decodes a chunk on the GPU into uint8 symbols [L, T, C]
    (decode_fast_prefsum over the concatenated streams)."""
    L, T, C = chunk.shape
    dev = chunk.cdf.device
    if dev.type != "cuda":
        raise ValueError("decode_chunk takes a chunk on the GPU (CacheGenChunk.to)")
    prefix = torch.cumsum(chunk.lengths.to(torch.int64).view(-1), 0).to(torch.int32).view(L, C)
    streams = chunk.streams.to(dev)
    if streams.numel() == 0:  # the op needs an addressable buffer
        streams = torch.zeros(1, dtype=torch.uint8, device=dev)
    # decode_fast_prefsum writes all T symbols of every stream.
    out = torch.empty((L, T, C), dtype=torch.uint8, device=dev)
    c_ops.decode_fast_prefsum(chunk.cdf, streams, prefix, out)
    return out
