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


def _py_gw_depths(weights):
    """Garsia-Wachs restated with Python lists (the C oracle keeps parent
    links instead): items are (weight, leaves); combining two items adds one
    to the depth of each of their leaves."""
    items = [(w, [i]) for i, w in enumerate(weights)]
    depth = [0] * len(weights)
    while len(items) > 1:
        ws = [w for w, _ in items] + [float("inf")]
        k = next(i for i in range(len(items) - 1) if ws[i] <= ws[i + 2])
        (x, lx), (y, ly) = items[k], items[k + 1]
        for leaf in lx + ly:
            depth[leaf] += 1
        del items[k:k + 2]
        j = max([i for i in range(k) if items[i][0] >= x + y], default=-1)
        items.insert(j + 1, (x + y, lx + ly))
    return depth


def _py_shannon_lengths(counts):
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
    return lens


def _py_lengths(counts):
    """Rule L4's code lengths: Garsia-Wachs depths when the longest fits
    Lmax (8 bits for at most 256 counted symbols, else 12), else Shannon."""
    n = sum(counts)
    present = [s for s, c in enumerate(counts) if c]
    lens = [0] * len(counts)
    if len(present) == 1:
        lens[present[0]] = 1
    elif len(present) >= 2:
        d = _py_gw_depths([counts[s] for s in present])
        if max(d) > (8 if n <= 256 else 12):
            return _py_shannon_lengths(counts), False
        for s, l in zip(present, d):
            lens[s] = l
    return lens, True


def _py_cdf_row(counts):
    """Independent restatement of rule L4 with Python integers."""
    nb = len(counts)
    lens, _ = _py_lengths(counts)
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


def _cdf_of_counts(counts):
    """calculate_cdf of one stream holding counts[s] copies of symbol s."""
    nb = len(counts)
    syms = np.repeat(np.arange(nb, dtype=np.uint8), counts)
    syms = np.random.default_rng(len(syms)).permutation(syms).reshape(1, -1, 1)
    return oc.calculate_cdf(syms, nb).view(np.uint16)[0, 0]


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


def _check_structure(row, counts, full=False):
    """Structural invariants of one CDF row: present symbols (and only they)
    have lengths 1..12 (at most 8 when at most 256 symbols are counted);
    each interval is aligned to its width (a fixed code); the intervals are
    gap-free in symbol order (the first starts at 0, each starts where the
    previous present symbol's ends), so the last one ends at the sum of the
    widths, which is at most 0x10000 (Kraft <= 1), and exactly 0x10000 for
    a code that is a full binary tree (`full`: the Garsia-Wachs rows)."""
    n = int(sum(counts))
    base, lens = _intervals(row)
    assert all((ln > 0) == bool(c) for ln, c in zip(lens, counts)), "present <=> length"
    assert all(1 <= ln <= (8 if n <= 256 else 12) for ln in lens if ln), "length limit"
    end = 0
    total = 0
    for s in range(len(lens)):
        if lens[s]:
            w = 2 ** (16 - lens[s])
            assert base[s] % w == 0, "aligned"
            assert base[s] == end, "gap-free"
            end = base[s] + w
            total += w
    assert end == total <= 0x10000, "Kraft"
    if full:
        assert total == 0x10000, "complete code"


# Counts that force the Shannon fallback: a Fibonacci run makes a caterpillar
# Garsia-Wachs tree deeper than 8 levels within 256 symbols.
FIB = [1, 1, 2, 3, 5, 8, 13, 21, 34, 55, 89]


def _fallback_cases(rng, k):
    """k count rows over 16 or 32 bins, at most 256 symbols, whose
    Garsia-Wachs tree is 9 or more levels deep: a Fibonacci run of 10 or 11
    counts, forwards or backwards, beside a few rare symbols."""
    out = []
    i = 0
    while len(out) < k:
        nb = int(rng.choice([16, 32]))
        run = FIB[:10 + i % 2]
        i += 1
        tail = [int(x) for x in rng.integers(0, 3, size=nb - len(run))]
        counts = (run + tail) if rng.random() < 0.5 else (tail[::-1] + run[::-1])
        if sum(counts) <= 256 and max(_py_gw_depths([c for c in counts if c])) > 8:
            out.append(counts)
    return out


@pytest.mark.parametrize("seed", range(6))
def test_cdf_structural_invariants(seed):
    rng = np.random.default_rng(100 + seed)
    nb = 32
    p = rng.dirichlet(np.full(nb, 0.2))
    syms = rng.choice(nb, size=(3, 256, 64), p=p).astype(np.uint8)
    cdf = oc.calculate_cdf(syms, nb).view(np.uint16)
    full_rows = 0
    for l in range(3):
        for c in range(64):
            counts = np.bincount(syms[l, :, c], minlength=nb)
            full = int((counts > 0).sum()) >= 2 and _py_lengths(counts.tolist())[1]
            full_rows += full
            _check_structure(cdf[l, c], counts, full)
    assert full_rows > 0
    for counts in _fallback_cases(rng, 8):
        assert not _py_lengths(counts)[1]
        _check_structure(_cdf_of_counts(counts), counts)


def test_cdf_of_uniform_and_dyadic_histograms():
    """Closed forms: 2^n equal counts give n-bit codes (every optimal code of
    equally likely symbols is balanced); a dyadic histogram gives lengths
    log2(n / c), the entropy."""
    for bits in range(1, 7):
        row = _cdf_of_counts([3] * 2 ** bits)
        assert list(row) == [(b << (16 - bits)) | bits for b in range(2 ** bits)] + [0]
    assert _intervals(_cdf_of_counts([128, 64, 32, 16, 8, 8]))[1] == [1, 2, 3, 4, 5, 5]
    assert _intervals(_cdf_of_counts([8, 8, 16, 32, 64, 128]))[1] == [5, 5, 4, 3, 2, 1]


def test_cdf_hand_worked_tie_rules():
    """Rows worked by hand from the rule's statement where equally good
    codes exist, so only the tie rules decide:
      [1, 1, 1]: the triple (1, 1, 1) qualifies at once (1 <= 1): symbols 0
        and 1 combine into 2, re-inserted at the front (no weight to its
        left): [2, 1] -> lengths 2, 2, 1 (x < z would give 1, 2, 2);
      [2, 1, 1, 2]: (2, 1, 1) fails (2 > 1), (1, 1, 2) qualifies: symbols 1
        and 2 combine into 2, re-inserted right after the first 2 (2 >= 2):
        [2, 2, 2]; that triple qualifies: the first pair combines into 4,
        at the front: [4, 2] -> lengths 2, 3, 3, 1;
      [5, 1, 1, 5]: (5, 1, 1) fails, (1, 1, 5) qualifies: 2 goes right
        after the 5: [5, 2, 5]; (5, 2, 5) qualifies (5 <= 5): 7 at the
        front: [7, 5] -> lengths 2, 3, 3, 1."""
    assert _intervals(_cdf_of_counts([1, 1, 1]))[1] == [2, 2, 1]
    assert _intervals(_cdf_of_counts([5, 1, 1, 5]))[1] == [2, 3, 3, 1]
    assert _intervals(_cdf_of_counts([2, 1, 1, 2]))[1] == [2, 3, 3, 1]


def _all_alphabetic_codes(m, lmax):
    """Every order-preserving prefix code of m symbols with lengths 1..lmax:
    the length vectors whose intervals, placed in symbol order each at the
    first multiple of its width, fit in [0, 2^16)."""
    lens = np.array(np.meshgrid(*[np.arange(1, lmax + 1)] * m, indexing="ij")).reshape(m, -1).T
    pos = np.zeros(lens.shape[0], np.int64)
    for j in range(m):
        w = np.int64(1) << (16 - lens[:, j])
        pos = (pos + w - 1) // w * w + w
    return lens[pos <= 1 << 16]


@pytest.mark.parametrize("m", [2, 3, 4, 5, 6])
def test_cdf_is_optimal_by_brute_force(m):
    """For alphabets of up to 6 present symbols (at most 256 tokens), the
    code costs exactly the minimum over every order-preserving prefix code
    with lengths 1..8, found by enumeration."""
    codes = _all_alphabetic_codes(m, 8)
    rng = np.random.default_rng(m)
    for _ in range(60):
        nb = int(rng.integers(m, m + 3))
        present = np.sort(rng.choice(nb, size=m, replace=False))
        counts = np.zeros(nb, np.int64)
        counts[present] = rng.choice([1, 1, 2, 3, 5, 9, 20, 40], size=m)
        row = _cdf_of_counts(counts.tolist())
        lens = np.array(_intervals(row)[1])
        assert int(counts @ lens) == int((codes @ counts[present]).min()), counts.tolist()


def _optimal_alphabetic_cost(w):
    """Textbook interval dynamic program: the cheapest alphabetic tree over
    w[i..j] costs sum(w[i..j]) + the cheapest split into two subtrees."""
    m = len(w)
    pre = np.concatenate([[0], np.cumsum(w)])
    f = [[0] * m for _ in range(m)]
    for d in range(1, m):
        for i in range(m - d):
            j = i + d
            f[i][j] = int(pre[j + 1] - pre[i]) + min(f[i][k] + f[k + 1][j] for k in range(i, j))
    return f[0][m - 1]


@pytest.mark.parametrize("seed", range(4))
def test_cdf_is_optimal_by_interval_dp(seed):
    """Quantised Gaussian chunks of 256 tokens with 16 and 32 bins (up to
    31 present symbols): every row whose optimal code fits 8 bits costs
    exactly the interval program's optimum; the others (Shannon fallback)
    cost more and keep the structural invariants."""
    rng = np.random.default_rng(400 + seed)
    x = rng.normal(size=(2, 256, 48)).astype(np.float32)
    syms = oc.quantize(x, [32, 16])
    cdf = oc.calculate_cdf(syms, 32).view(np.uint16)
    fell_back = 0
    for l in range(2):
        for c in range(48):
            counts = np.bincount(syms[l, :, c], minlength=32)
            lens = np.array(_intervals(cdf[l, c])[1])
            cost = int(counts @ lens)
            best = _optimal_alphabetic_cost(counts[counts > 0].tolist())
            if _py_lengths(counts.tolist())[1]:
                assert cost == best, (l, c)
            else:
                fell_back += 1
                assert cost > best
                _check_structure(cdf[l, c], counts)
    assert fell_back < 24  # about 1 in 10 32-bin rows, none of the 16-bin ones


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
# The Shannon fallback's properties, and planted CDF mistakes
# ---------------------------------------------------------------------------


def _share_and_minimality(cases):
    """The defining properties of Shannon code lengths, on rows that take
    the fallback and need no Kraft repair (no length reaches 12):
      share: a present symbol's interval is at most its frequency share,
             2^-l <= c / n;
      minimality: where the alignment step did not halve the interval (the
             base is a multiple of twice the width), one bit less would
             exceed the share: 2^-(l-1) > c / n, for l > 1.
    Returns the number of symbols checked."""
    checked = 0
    for counts in cases:
        n = sum(counts)
        base, lens = _intervals(_cdf_of_counts(counts))
        for s, cs in enumerate(counts):
            if cs == 0:
                continue
            ls = lens[s]
            assert n <= cs << ls, ("share", counts, s)
            width = 1 << (16 - ls)
            if ls > 1 and base[s] % (2 * width) == 0:
                assert n > cs << (ls - 1), ("minimality", counts, s)
            checked += 1
    return checked


@pytest.mark.parametrize("seed", range(4))
def test_cdf_shannon_share_bound_and_minimality(seed):
    cases = _fallback_cases(np.random.default_rng(300 + seed), 12)
    assert all(not _py_lengths(c)[1] for c in cases)
    assert _share_and_minimality(cases) > 0


# 65536 counted symbols over 29 bins: a run 1, 1, 2, 4, ..., 8192 whose
# Garsia-Wachs tree is a 15-level caterpillar (above the 12-bit limit, so the
# Shannon rule applies), then power-of-two counts.  The run's five rarest
# symbols have Shannon lengths capped at 12, which pushes the Kraft sum to
# 1 + 2^-10; the repair lengthens four of the seven symbols of count 32
# (from 11 to 12 bits), so the tie rule decides the code.
REPAIR_CASE_COUNTS = [1] + [2 ** j for j in range(14)] + [32, 4096, 32, 512, 32768, 32, 64, 2048, 32, 256, 8192,
                                                         32, 1024, 32]


def test_cdf_kraft_repair_case_matches_python_restatement():
    counts = REPAIR_CASE_COUNTS + [0] * (64 - len(REPAIR_CASE_COUNTS))
    assert sum(counts) == 65536
    assert max(_py_gw_depths([c for c in counts if c])) > 12
    row = _cdf_of_counts(counts)
    assert list(row) == _py_cdf_row(counts)
    assert sum(2.0 ** -ln for ln in _intervals(row)[1] if ln) <= 1.0


def _run_checks():
    """Every CPU check of calculate_cdf that is not the restatement, by
    name -> passed?  The restatement and the repair case, which compare
    with it, are listed last."""
    checks = {
        "uniform and dyadic closed forms": test_cdf_of_uniform_and_dyadic_histograms,
        "hand-worked tie rules": test_cdf_hand_worked_tie_rules,
        "single and empty": test_cdf_single_and_empty,
        "structural invariants": lambda: [test_cdf_structural_invariants(s) for s in range(6)],
        "round trip": lambda: [test_round_trip(s) for s in range(8)],
        "brute-force optimality": lambda: [test_cdf_is_optimal_by_brute_force(m) for m in range(2, 7)],
        "interval-program optimality": lambda: [test_cdf_is_optimal_by_interval_dp(s) for s in range(4)],
        "share bound and minimality": lambda: [test_cdf_shannon_share_bound_and_minimality(s) for s in range(4)],
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


# Planted mistake -> the checks other than the restatement that must fail
# it (every other non-restatement check may pass it).
PLANTED = {
    # the combined weight left at the pair's place: not optimal
    "OC_PLANT_GW_IN_PLACE": {"brute-force optimality", "interval-program optimality"},
    # re-inserted one place too far left: not optimal
    "OC_PLANT_GW_BEFORE": {"brute-force optimality", "interval-program optimality"},
    # the first triple with x < z: equally optimal codes, other ties
    "OC_PLANT_GW_STRICT": {"hand-worked tie rules"},
    # a 9-bit limit for chunks of at most 256 symbols
    "OC_PLANT_LMAX9": {"structural invariants"},
    # the fallback's base rounded up to the width, the length kept: aligned,
    # disjoint and decodable, but with gaps
    "OC_PLANT_ROUND_UP": {"structural invariants"},
    # floor(log2(n / c)) in the fallback: the Kraft repair keeps the code
    # valid, the share bound catches it
    "OC_PLANT_FLOOR_LEN": {"share bound and minimality"},
}


@pytest.mark.parametrize("flag", list(PLANTED))
def test_planted_cdf_mistake_is_caught(flag):
    passed = _with_planted(flag, _run_checks)
    for name in PLANTED[flag]:
        assert not passed[name], (flag, name, passed)


def test_planted_tie_break_is_caught_only_by_the_repair_case():
    """Ties in the fallback's Kraft repair going to the lowest symbol instead
    of the highest: no property can tell the two rules apart (both yield
    valid prefix codes of equal cost), only the restatement on a case where
    the repair runs.  The repair needs a length capped at 12 bits, i.e. more
    than 4096 symbols and a Garsia-Wachs tree deeper than 12 levels, so no
    CDF of a chunk of at most 4096 tokens (LMCache chunks hold 256) depends
    on the tie rule."""
    passed = _with_planted("OC_PLANT_TIE_LOW", _run_checks)
    assert not passed["restatement on the Kraft repair case"]
    assert all(ok for name, ok in passed.items() if name != "restatement on the Kraft repair case"), passed
    rng = np.random.default_rng(9)
    syms = np.concatenate([rng.choice(32, size=(1, 4096, 64), p=rng.dirichlet(np.full(32, a))).astype(np.uint8)
                           for a in (0.05, 0.3, 1.0)])
    real = oc.calculate_cdf(syms, 32)
    planted = _with_planted("OC_PLANT_TIE_LOW", lambda: oc.calculate_cdf(syms, 32))
    assert np.array_equal(real, planted)
