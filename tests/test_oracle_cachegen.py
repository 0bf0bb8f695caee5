"""Pins the CacheGen oracle (oracle/cachegen.c) on the CPU.

Checks, in order of strength:
  * the reference's own known-answer tests (tests/v1/test_cachegen_kernels.py):
    uniform 2^n CDF -> n-bit binary codes, MSB first, zero-padded, exact byte
    lengths (:31-122); the non-uniform [0, 0, 2, 3] case (:125-161); the
    closed-form decode with low-bit lengths and prefix sums (:164-239);
  * closed forms of calculate_cdf: a uniform 2^n histogram gives exactly the
    reference decode test's CDF; a dyadic histogram gives the optimal code;
  * the defining properties of Shannon code lengths, checked on random
    histograms: no symbol's interval exceeds its frequency share, and one
    bit less would, wherever the alignment step did not shorten it;
  * an independent Python restatement of the CDF rule, on small inputs and
    on a constructed 65536-token case where the Kraft repair runs;
  * structural invariants (prefix-free, aligned, Kraft <= 1) and round trips;
  * planted mistakes built into the oracle: LSB-first bit packing must fail
    the encode KAT, floor instead of ceil code lengths must fail the share
    bound, and the other Kraft-repair tie rule fails only the repair case
    (no chunk of at most 4096 tokens can tell the two tie rules apart).
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


# ---------------------------------------------------------------------------
# Shannon-length properties of calculate_cdf, and planted CDF mistakes
# ---------------------------------------------------------------------------


def _share_and_minimality(syms, nb):
    """Checks the defining properties of Shannon code lengths on every
    stream of `syms` ([L, T, C]) whose T <= 4096 (no length reaches the
    12-bit cap, so no Kraft repair runs):
      share: a present symbol's interval is at most its frequency share,
             2^-l <= c / n;
      minimality: where the alignment step did not halve the interval (the
             base is a multiple of twice the width), one bit less would
             exceed the share: 2^-(l-1) > c / n, for l > 1.
    Returns the number of symbols checked."""
    cdf = oc.calculate_cdf(syms, nb).view(np.uint16)
    L, T, C = syms.shape
    assert T <= 4096
    checked = 0
    for l in range(L):
        for c in range(C):
            counts = np.bincount(syms[l, :, c][syms[l, :, c] < nb], minlength=nb)
            n = int(counts.sum())
            base, lens = _intervals(cdf[l, c])
            for s in range(nb):
                if counts[s] == 0:
                    continue
                cs, ls = int(counts[s]), lens[s]
                assert n <= cs << ls, ("share", l, c, s)
                width = 1 << (16 - ls)
                if ls > 1 and base[s] % (2 * width) == 0:
                    assert n > cs << (ls - 1), ("minimality", l, c, s)
                checked += 1
    return checked


@pytest.mark.parametrize("seed", range(8))
def test_cdf_shannon_share_bound_and_minimality(seed):
    rng = np.random.default_rng(300 + seed)
    nb = int(rng.choice([8, 16, 32, 64]))
    T = int(rng.choice([17, 100, 256, 1000, 4096]))
    p = rng.dirichlet(np.full(nb, float(rng.choice([0.1, 0.5, 2.0]))))
    syms = rng.choice(nb, size=(2, T, 16), p=p).astype(np.uint8)
    assert _share_and_minimality(syms, nb) > 0


# 65536 tokens over 37 symbols: exact power-of-two counts plus six rare
# symbols whose 13..14-bit Shannon lengths are capped at 12, which pushes
# the Kraft sum over 1; the repair then lengthens two of several equally
# frequent symbols, so the tie rule decides the code.
REPAIR_CASE_COUNTS = [512, 1024, 512, 2048, 32, 12, 10, 5, 1024, 32768, 128, 16, 15, 64, 8192, 64, 256, 64, 1024,
                      16, 16, 2048, 64, 4096, 2048, 256, 6, 256, 64, 16, 32, 64, 16, 8192, 32, 32, 512]


def _repair_case():
    nb = 64
    counts = REPAIR_CASE_COUNTS + [0] * (nb - len(REPAIR_CASE_COUNTS))
    syms = np.repeat(np.arange(nb, dtype=np.uint8), counts)
    syms = np.random.default_rng(0).permutation(syms).reshape(1, -1, 1)
    return syms, counts, nb


def test_cdf_kraft_repair_case_matches_python_restatement():
    syms, counts, nb = _repair_case()
    cdf = oc.calculate_cdf(syms, nb).view(np.uint16)
    assert list(cdf[0, 0]) == _py_cdf_row(counts)
    base, lens = _intervals(cdf[0, 0])
    assert sum(2.0 ** -ln for ln in lens if ln) <= 1.0


def _run_checks():
    """Every CPU check of calculate_cdf, by name -> passed?"""
    checks = {
        "uniform closed form": lambda: [test_cdf_of_uniform_histogram_is_reference_decode_cdf(b) for b in range(1, 7)],
        "dyadic closed form": test_cdf_dyadic_histogram_is_optimal,
        "single and empty": test_cdf_single_and_empty,
        "structural invariants": lambda: [test_cdf_structural_invariants(s) for s in range(6)],
        "round trip": lambda: [test_round_trip(s) for s in range(8)],
        "share bound and minimality": lambda: [test_cdf_shannon_share_bound_and_minimality(s) for s in range(8)],
        "python restatement": lambda: [test_cdf_matches_python_restatement(s) for s in range(12)],
        "restatement on the Kraft repair case": test_cdf_kraft_repair_case_matches_python_restatement,
    }
    out = {}
    for name, fn in checks.items():
        try:
            fn()
            out[name] = True
        except AssertionError:
            out[name] = False
    return out


def _with_planted(flag, fn):
    src = os.path.join(os.path.dirname(oc.__file__), "cachegen.c")
    with tempfile.TemporaryDirectory() as d:
        lib = os.path.join(d, "planted.so")
        subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-D" + flag, src, "-o", lib], check=True)
        planted = oc.load_library(lib)
        real = oc._load()
        try:
            oc._lib = planted
            return fn()
        finally:
            oc._lib = real


def test_planted_floor_length_is_caught_by_the_shannon_properties():
    """floor(log2(n/c)) instead of ceil: the closed forms (uniform, dyadic)
    cannot see it (their shares are exact powers of two) and the Kraft
    repair keeps every structural invariant and round trip intact; the
    share bound catches it, as does the restatement."""
    passed = _with_planted("OC_PLANT_FLOOR_LEN", _run_checks)
    assert not passed["share bound and minimality"]
    assert not passed["python restatement"]
    for name in ("uniform closed form", "dyadic closed form", "single and empty", "structural invariants",
                 "round trip"):
        assert passed[name], name


def test_planted_tie_break_is_caught_only_by_the_repair_case():
    """Ties in the Kraft repair going to the lowest symbol instead of the
    highest: no property can tell the two rules apart (both yield valid
    prefix codes of equal cost), only the restatement on a case where the
    repair runs.  The repair needs a length capped at 12 bits, i.e. more
    than 4096 tokens, so no CDF of a chunk of at most 4096 tokens (LMCache
    chunks hold 256) depends on the tie rule."""
    passed = _with_planted("OC_PLANT_TIE_LOW", _run_checks)
    assert not passed["restatement on the Kraft repair case"]
    assert all(ok for name, ok in passed.items() if name != "restatement on the Kraft repair case"), passed
    rng = np.random.default_rng(9)
    syms = np.concatenate([rng.choice(32, size=(1, 4096, 64), p=rng.dirichlet(np.full(32, a))).astype(np.uint8)
                           for a in (0.05, 0.3, 1.0)])
    real = oc.calculate_cdf(syms, 32)
    planted = _with_planted("OC_PLANT_TIE_LOW", lambda: oc.calculate_cdf(syms, 32))
    assert np.array_equal(real, planted)
