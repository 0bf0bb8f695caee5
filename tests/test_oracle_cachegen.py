"""Pins the CacheGen oracle (oracle/cachegen.c) on the CPU.

Checks, in order of strength:
  * the reference's own known-answer tests (tests/v1/test_cachegen_kernels.py):
    uniform 2^n CDF -> n-bit binary codes, MSB first, zero-padded, exact byte
    lengths (:31-122); the non-uniform [0, 0, 2, 3] case (:125-161); the
    closed-form decode with low-bit lengths and prefix sums (:164-239);
  * closed forms of calculate_cdf: a uniform 2^n histogram gives exactly the
    reference decode test's CDF; a dyadic histogram gives the optimal code;
  * an independent Python restatement of the CDF rule on small inputs;
  * structural invariants (prefix-free, aligned, Kraft <= 1) and round trips;
  * a planted bit-order mistake in the oracle must fail the encode KAT.
"""

import os
import subprocess
import tempfile

import numpy as np
import pytest
import torch

from oracle import cachegen as oc

MAX_TOKENS_PER_CHUNK = 256  # bytes per encoded stream in the reference tests


def _wrap16(values):
    """The reference builds CDFs as floats and casts them to int16."""
    return torch.tensor(values, dtype=torch.float32).to(torch.int16).numpy()


def _binary_stream(bits, max_sym):
    s = "".join(format(t, f"0{bits}b") for t in range(max_sym))
    if len(s) % 8:
        s += "0" * (8 - len(s) % 8)
    return [int(s[i: i + 8], 2) for i in range(0, len(s), 8)]


@pytest.mark.parametrize("layers", [1, 2])
@pytest.mark.parametrize("channels", [1, 32, 256])
@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6])
def test_reference_basic_encode(layers, channels, bits):
    max_sym = 2 ** bits
    syms = np.array([s for s in range(max_sym) for _ in range(channels)] * layers, np.int8)
    syms = syms.reshape(layers, max_sym, channels)
    bins = max_sym + 1
    cdf = _wrap16([b * (0x10000 / (bins - 1)) for b in range(bins)] * layers * channels)
    cdf = cdf.reshape(layers, channels, bins)
    out, lens = oc.encode(cdf, syms, MAX_TOKENS_PER_CHUNK)
    expected = _binary_stream(bits, max_sym)
    row = np.zeros(MAX_TOKENS_PER_CHUNK, np.uint8)
    row[: len(expected)] = expected
    assert (out == row).all()
    assert (lens == len(expected)).all()


def test_reference_non_uniform_encode():
    cdf = _wrap16([0x0000, 0x8000, 0x8000, 0xC000, 0x10000]).reshape(1, 1, 5)
    syms = np.array([0, 0, 2, 3], np.int8).reshape(1, 4, 1)
    out, lens = oc.encode(cdf, syms, 4)
    assert out[0, 0, 0] == 0b00101100
    assert lens[0, 0] == 1


@pytest.mark.parametrize("layers", [1, 2])
@pytest.mark.parametrize("channels", [32, 256])
@pytest.mark.parametrize("bits", [2, 3, 4, 5])
def test_reference_basic_decode(layers, channels, bits):
    max_sym = 2 ** bits
    stream = _binary_stream(bits, max_sym)
    byte_stream = np.array(stream * layers * channels, np.uint8)
    lens = np.cumsum([len(stream)] * layers * channels).astype(np.int32).reshape(layers, channels)
    bins = max_sym + 1
    factor = 0x10000 / (bins - 1)
    cdf = _wrap16([int(b * factor) | bits for b in range(bins)] * layers * channels)
    cdf = cdf.reshape(layers, channels, bins)
    out = oc.decode(cdf, byte_stream, lens, max_sym)
    want = np.array([s for s in range(max_sym) for _ in range(channels)] * layers, np.uint8)
    assert (out == want.reshape(layers, max_sym, channels)).all()


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6])
def test_cdf_of_uniform_histogram_is_reference_decode_cdf(bits):
    # 2^n equally frequent symbols: every code is n bits and the CDF is the
    # one test_basic_decode builds (cdf[b] = b * 2^(16-n) | n), except the end
    # entry, which this library stores as the wrapped 0x10000 = 0.
    n = 2 ** bits
    syms = np.tile(np.arange(n, dtype=np.uint8), 4).reshape(1, 4 * n, 1)
    cdf = oc.calculate_cdf(syms, n)
    want = _wrap16([int(b * (0x10000 / n)) | bits for b in range(n)] + [0])
    assert (cdf.reshape(-1) == want).all()


def test_cdf_dyadic_histogram_is_optimal():
    syms = np.array([0] * 128 + [1] * 64 + [2] * 32 + [3] * 32, np.uint8).reshape(1, 256, 1)
    cdf = oc.calculate_cdf(syms, 4).reshape(-1).view(np.uint16)
    assert list(cdf) == [0x0000 | 1, 0x8000 | 2, 0xC000 | 3, 0xE000 | 3, 0]


def test_cdf_single_and_empty():
    syms = np.full((1, 10, 1), 2, np.uint8)
    cdf = oc.calculate_cdf(syms, 4).reshape(-1).view(np.uint16)
    # symbols 0 and 1 absent (base of symbol 2 = 0), 2 has a 1-bit code,
    # symbol 3 absent at the end of the used range (0x8000)
    assert list(cdf) == [0, 0, 0 | 1, 0x8000, 0]
    empty = oc.calculate_cdf(np.zeros((2, 0, 3), np.uint8), 8)
    assert (empty == 0).all()


def _py_cdf_row(counts):
    """Independent restatement of rule L4 with Python integers."""
    n = sum(counts)
    nb = len(counts)
    lens = [0] * nb
    for s, c in enumerate(counts):
        if c:
            lens[s] = min(12, max(1, ((n + c - 1) // c - 1).bit_length()))
    while sum(2 ** (16 - l) for l in lens if l) > 2 ** 16:
        cands = [s for s in range(nb) if 0 < lens[s] < 12]
        s = min(cands, key=lambda i: (counts[i], -i))
        lens[s] += 1
    base = [None] * nb
    pos = 0
    for s in range(nb):
        if lens[s]:
            w = 2 ** (16 - lens[s])
            if pos:
                w = min(w, pos & -pos)
            lens[s] = 16 - (w.bit_length() - 1)
            base[s] = pos
            pos += w
    nxt = pos
    for s in reversed(range(nb)):
        if base[s] is None:
            base[s] = nxt
        else:
            nxt = base[s]
    return [((b | l) & 0xFFFF) for b, l in zip(base, lens)] + [0]


@pytest.mark.parametrize("seed", range(12))
def test_cdf_matches_python_restatement(seed):
    rng = np.random.default_rng(seed)
    nb = int(rng.choice([2, 5, 16, 32, 64]))
    T = int(rng.choice([1, 3, 17, 256, 1000]))
    C = 7
    p = rng.dirichlet(np.full(nb, 0.3))
    syms = rng.choice(nb, size=(2, T, C), p=p).astype(np.uint8)
    syms[0, :, 0] = nb + 3 if nb < 200 else 0  # out-of-range symbols are not counted
    cdf = oc.calculate_cdf(syms, nb).view(np.uint16)
    for l in range(2):
        for c in range(C):
            counts = np.bincount(syms[l, :, c][syms[l, :, c] < nb], minlength=nb).tolist()
            assert list(cdf[l, c]) == _py_cdf_row(counts), (l, c)


def _intervals(cdf_row_u16):
    nb = len(cdf_row_u16) - 1
    base = [int(v) & 0xFFF0 for v in cdf_row_u16[:nb]]
    for s in range(1, nb):
        if base[s] < base[s - 1]:
            base[s:] = [0x10000] * (nb - s)
            break
    lens = [int(v) & 0xF for v in cdf_row_u16[:nb]]
    return base, lens


@pytest.mark.parametrize("seed", range(6))
def test_cdf_structural_invariants(seed):
    rng = np.random.default_rng(100 + seed)
    nb = 32
    p = rng.dirichlet(np.full(nb, 0.2))
    syms = rng.choice(nb, size=(3, 256, 64), p=p).astype(np.uint8)
    cdf = oc.calculate_cdf(syms, nb).view(np.uint16)
    for l in range(3):
        for c in range(64):
            base, lens = _intervals(cdf[l, c])
            present = np.bincount(syms[l, :, c], minlength=nb) > 0
            assert all((ln > 0) == bool(pr) for ln, pr in zip(lens, present))
            assert all(1 <= ln <= 12 for ln in lens if ln)
            kraft = sum(2.0 ** -ln for ln in lens if ln)
            assert kraft <= 1.0
            end = 0
            for s in range(nb):
                if lens[s]:
                    w = 2 ** (16 - lens[s])
                    assert base[s] % w == 0          # aligned: fixed code
                    assert base[s] >= end            # disjoint, in order
                    end = base[s] + w
            assert end <= 0x10000


@pytest.mark.parametrize("seed", range(8))
def test_round_trip(seed):
    rng = np.random.default_rng(seed)
    L, T, C = 3, int(rng.choice([1, 20, 256])), 64
    nb = int(rng.choice([16, 32]))
    x = rng.normal(size=(L, T, C)).astype(np.float32)
    syms = oc.quantize(x, nb)
    syms[1, :, :8] = 5                              # deterministic channels
    cdf = oc.calculate_cdf(syms, nb)
    out, lens = oc.encode(cdf, syms, 512)
    assert lens.max() <= 512
    stream, pref = oc.concat_streams(out, lens)
    assert (oc.decode(cdf, stream, pref, T) == syms).all()


def test_encode_truncates_at_chunk_and_reports_full_length():
    syms = np.tile(np.arange(16, dtype=np.uint8), 8).reshape(1, 128, 1)
    cdf = oc.calculate_cdf(syms, 16)                # 4 bits per symbol: 64 bytes
    out = np.full((1, 1, 40), 0xEE, np.uint8)
    out, lens = oc.encode(cdf, syms, 40, out=out)
    assert lens[0, 0] == 64
    full, _ = oc.encode(cdf, syms, 64)
    assert (out[0, 0] == full[0, 0, :40]).all()


def test_planted_lsb_first_fails_reference_kat():
    """A plausible mistake (LSB-first bit packing) built into the oracle must
    be caught by the reference's encode KAT."""
    src = os.path.join(os.path.dirname(oc.__file__), "cachegen.c")
    with tempfile.TemporaryDirectory() as d:
        lib = os.path.join(d, "planted.so")
        subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-DOC_PLANT_LSB_FIRST", src, "-o", lib],
                       check=True)
        planted = oc.load_library(lib)
        real = oc._load()
        try:
            oc._lib = planted
            with pytest.raises(AssertionError):
                test_reference_basic_encode(1, 1, 3)
        finally:
            oc._lib = real
