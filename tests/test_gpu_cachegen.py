"""GPU parity of the CacheGen kernels (calculate_cdf, encode_fast_new,
decode_fast_prefsum) through the C ABI.

* The reference's own tests (tests/v1/test_cachegen_kernels.py) re-run on the
  MI355X with their known answers;
* bit-exact CDFs, bitstreams, byte lengths and decoded symbols against the
  CPU oracle at the 32-layer x 256-token x 1024-channel K+V chunk shape
  (K layers 0-9 quantised to 32 bins, later K layers and all V layers to 16);
* edge cases: one token, one bin, constant channels, out-of-range symbols,
  streams longer than the output row, and the reference's limits.
"""

import numpy as np
import pytest
import torch

from oracle import cachegen as oc

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
MAX_TOKENS_PER_CHUNK = 256


@pytest.fixture(scope="module")
def ops():
    import lmcache_amd

    return lmcache_amd.c_ops


def _wrap16(values):
    return torch.tensor(values, dtype=torch.float32).to(torch.int16)


def _binary_stream(bits, max_sym):
    s = "".join(format(t, f"0{bits}b") for t in range(max_sym))
    if len(s) % 8:
        s += "0" * (8 - len(s) % 8)
    return [int(s[i: i + 8], 2) for i in range(0, len(s), 8)]


@pytest.mark.parametrize("layers", [1, 2])
@pytest.mark.parametrize("channels", [1, 32, 256])
@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6])
def test_basic_encode(ops, layers, channels, bits):
    """tests/v1/test_cachegen_kernels.py:31-122."""
    max_sym = 2 ** bits
    symbols = [s for s in range(max_sym) for _ in range(channels)] * layers
    syms = torch.tensor(symbols).to(DEV).to(torch.int8).reshape(layers, max_sym, channels)
    bins = max_sym + 1
    cdf = torch.Tensor([b * (0x10000 / (bins - 1)) for b in range(bins)] * layers * channels)
    cdf = cdf.to(DEV).to(torch.int16).reshape(layers, channels, bins)
    out = torch.zeros(MAX_TOKENS_PER_CHUNK * layers * channels, dtype=torch.uint8).to(DEV)
    out = out.reshape(layers, channels, MAX_TOKENS_PER_CHUNK)
    lens = torch.zeros((layers, channels), dtype=torch.int32, device=DEV)
    ops.encode_fast_new(cdf, syms, out, lens)
    torch.cuda.synchronize()
    expected = _binary_stream(bits, max_sym)
    n = len(expected)
    expected += [0] * (MAX_TOKENS_PER_CHUNK - n)
    exp_t = torch.tensor(expected, dtype=torch.uint8, device=DEV).broadcast_to(out.shape)
    assert (exp_t == out).all()
    assert (lens == n).all()


def test_basic_non_uniform_encode(ops):
    """tests/v1/test_cachegen_kernels.py:125-161."""
    syms = torch.Tensor([0, 0, 2, 3]).to(DEV).to(torch.int8).reshape(1, 4, 1)
    cdf = torch.Tensor([0x0000, 0x8000, 0x8000, 0xC000, 0x10000]).to(DEV).to(torch.int16).reshape(1, 1, 5)
    out = torch.zeros(4, dtype=torch.uint8, device=DEV).reshape(1, 1, 4)
    lens = torch.zeros((1, 1), dtype=torch.int32, device=DEV)
    ops.encode_fast_new(cdf, syms, out, lens)
    torch.cuda.synchronize()
    assert out[0][0][0].tolist() == int("00101100", 2)


@pytest.mark.parametrize("layers", [1, 2])
@pytest.mark.parametrize("channels", [32, 256])
@pytest.mark.parametrize("bits", [2, 3, 4, 5])
def test_basic_decode(ops, layers, channels, bits):
    """tests/v1/test_cachegen_kernels.py:164-239."""
    max_sym = 2 ** bits
    stream = _binary_stream(bits, max_sym)
    bs = torch.tensor(stream * layers * channels, dtype=torch.uint8, device=DEV)
    lens = torch.tensor([len(stream)] * layers * channels, dtype=torch.int32, device=DEV)
    lens = lens.cumsum(0).to(torch.int32).reshape(layers, channels)
    bins = max_sym + 1
    factor = 0x10000 / (bins - 1)
    cdf = torch.Tensor([int(b * factor) | bits for b in range(bins)] * layers * channels)
    cdf = cdf.to(DEV).to(torch.int16).reshape(layers, channels, bins)
    out = torch.zeros((layers, max_sym, channels), dtype=torch.uint8, device=DEV)
    ops.decode_fast_prefsum(cdf, bs, lens, out)
    torch.cuda.synchronize()
    want = torch.tensor([s for s in range(max_sym) for _ in range(channels)] * layers, dtype=torch.uint8)
    assert (want.reshape(layers, max_sym, channels).to(DEV) == out).all()


def _kv_chunk_symbols(L=32, T=256, C=1024, seed=0):
    """[2L, T, C] symbols of one K+V chunk: K layers 0-9 at 32 bins, later K
    layers at 16; V layers at 16 (K stacked before V)."""
    rng = np.random.default_rng(seed)
    k = rng.normal(size=(L, T, C)).astype(np.float32)
    v = rng.normal(size=(L, T, C)).astype(np.float32)
    kb = np.where(np.arange(L) < 10, 32, 16)
    return np.concatenate([oc.quantize(k, kb), oc.quantize(v, 16)], axis=0)


def test_cachegen_kv_chunk_bit_exact(ops):
    syms = _kv_chunk_symbols()
    L2, T, C = syms.shape
    nb = 32
    d_syms = torch.from_numpy(syms).to(DEV)
    cdf = ops.calculate_cdf(d_syms, nb)
    want_cdf = oc.calculate_cdf(syms, nb)
    torch.cuda.synchronize()
    assert np.array_equal(cdf.cpu().numpy(), want_cdf)
    chunk = MAX_TOKENS_PER_CHUNK
    out = torch.zeros((L2, C, chunk), dtype=torch.uint8, device=DEV)
    lens = torch.zeros((L2, C), dtype=torch.int32, device=DEV)
    ops.encode_fast_new(cdf, d_syms, out, lens)
    want_out, want_len = oc.encode(want_cdf, syms, chunk)
    torch.cuda.synchronize()
    assert np.array_equal(lens.cpu().numpy(), want_len)
    assert np.array_equal(out.cpu().numpy(), want_out)
    assert want_len.max() <= chunk
    stream, pref = oc.concat_streams(want_out, want_len)
    dec = torch.zeros((L2, T, C), dtype=torch.uint8, device=DEV)
    ops.decode_fast_prefsum(cdf, torch.from_numpy(stream).to(DEV), torch.from_numpy(pref).to(DEV), dec)
    torch.cuda.synchronize()
    assert np.array_equal(dec.cpu().numpy(), syms)


@pytest.mark.parametrize("n_tokens", [1, 20, 256])
@pytest.mark.parametrize("n_layers", [1, 28])
@pytest.mark.parametrize("num_heads", [1, 8])
def test_encode_into_decode(ops, n_tokens, n_layers, num_heads):
    """tests/v1/test_cachegen_kernels.py:242-345 (with this library's quantiser)."""
    C = num_heads * 128
    rng = np.random.default_rng(n_tokens * 31 + n_layers)
    x = rng.normal(0, 2, size=(2 * n_layers, n_tokens, C)).astype(np.float32)
    bins = np.where(np.arange(2 * n_layers) % n_layers < 10, 32, 16) if n_layers > 1 else 32
    syms = oc.quantize(x, bins)
    d = torch.from_numpy(syms).to(DEV)
    cdf = ops.calculate_cdf(d, 32)
    out = torch.zeros((2 * n_layers, C, MAX_TOKENS_PER_CHUNK), dtype=torch.uint8, device=DEV)
    lens = torch.zeros((2 * n_layers, C), dtype=torch.int32, device=DEV)
    ops.encode_fast_new(cdf, d, out, lens)
    torch.cuda.synchronize()
    assert int(lens.max()) <= MAX_TOKENS_PER_CHUNK
    stream, pref = oc.concat_streams(out.cpu().numpy(), lens.cpu().numpy())
    dec = torch.zeros_like(d)
    ops.decode_fast_prefsum(cdf, torch.from_numpy(stream).to(DEV), torch.from_numpy(pref).to(DEV), dec)
    torch.cuda.synchronize()
    assert torch.equal(dec, d)


@pytest.mark.parametrize("T,C", [(300, 96), (256, 96), (255, 64), (256, 128), (97, 100), (1, 64)])
def test_edge_cases_vs_oracle(ops, T, C):
    """Tokens above 256 take the one-lane-per-stream kernels, 256 and below
    the tiled ones; C = 96 leaves a partial block of 32 streams, C = 100 is
    not a multiple of 16 (byte staging)."""
    rng = np.random.default_rng(5 + T + C)
    L, nb = 3, 16
    syms = rng.integers(0, nb, size=(L, T, C)).astype(np.uint8)
    syms[0, :, :5] = 7                    # constant channels: one 1-bit code
    syms[1, :, 10:20] = nb + 1            # out-of-range: not counted, not coded
    syms[2] = np.minimum(syms[2], 1)      # two symbols
    d = torch.from_numpy(syms).to(DEV)
    cdf = ops.calculate_cdf(d, nb)
    want_cdf = oc.calculate_cdf(syms, nb)
    torch.cuda.synchronize()
    assert np.array_equal(cdf.cpu().numpy(), want_cdf)
    chunk = 100                           # some streams overflow the row
    guard = np.full((L, C, chunk), 0xEE, np.uint8)
    out = torch.from_numpy(guard.copy()).to(DEV)
    lens = torch.zeros((L, C), dtype=torch.int32, device=DEV)
    ops.encode_fast_new(cdf, d, out, lens)
    want_out, want_len = oc.encode(want_cdf, syms, chunk, out=guard.copy())
    torch.cuda.synchronize()
    assert np.array_equal(lens.cpu().numpy(), want_len)
    assert np.array_equal(out.cpu().numpy(), want_out)
    if T >= 255:
        assert want_len.max() > chunk
    # round trip through the decoder where every stream fit its row
    if want_len.max() <= chunk and C % 32 == 0:
        stream, pref = oc.concat_streams(want_out, want_len)
        dec = torch.zeros_like(d)
        ops.decode_fast_prefsum(cdf, torch.from_numpy(stream).to(DEV), torch.from_numpy(pref).to(DEV), dec)
        torch.cuda.synchronize()
        assert np.array_equal(dec.cpu().numpy(), oc.decode(want_cdf, stream, pref, T))


def test_single_bin_and_single_token(ops):
    syms = np.zeros((2, 1, 32), np.uint8)
    d = torch.from_numpy(syms).to(DEV)
    cdf = ops.calculate_cdf(d, 1)
    torch.cuda.synchronize()
    assert np.array_equal(cdf.cpu().numpy(), oc.calculate_cdf(syms, 1))
    out = torch.zeros((2, 32, 8), dtype=torch.uint8, device=DEV)
    lens = torch.zeros((2, 32), dtype=torch.int32, device=DEV)
    ops.encode_fast_new(cdf, d, out, lens)
    torch.cuda.synchronize()
    assert (lens.cpu() == 1).all()


def test_decode_limits(ops):
    cdf = torch.zeros((1, 48, 17), dtype=torch.int16, device=DEV)
    with pytest.raises(RuntimeError, match="multiple of 32"):
        ops.decode_fast_prefsum(cdf, torch.zeros(4, dtype=torch.uint8, device=DEV),
                                torch.zeros((1, 48), dtype=torch.int32, device=DEV),
                                torch.zeros((1, 4, 48), dtype=torch.uint8, device=DEV))
    cdf = torch.zeros((1, 32, 65), dtype=torch.int16, device=DEV)
    with pytest.raises(RuntimeError, match="fewer than 64 bins"):
        ops.decode_fast_prefsum(cdf, torch.zeros(4, dtype=torch.uint8, device=DEV),
                                torch.zeros((1, 32), dtype=torch.int32, device=DEV),
                                torch.zeros((1, 4, 32), dtype=torch.uint8, device=DEV))
    with pytest.raises(NotImplementedError):
        ops.decode_fast_new(None, None, None, None)


def _arbitrary_cdf_rows(rng, L, C, nb, step=16):
    """CDF rows a caller may build by hand: non-decreasing 16-bit bases in
    multiples of `step` with gaps and repeats anywhere, a first base above
    zero in some rows, length nibbles 0 (derived from the width) to 15, and
    in some rows a decreasing entry after which every base reads as
    0x10000."""
    rows = np.zeros((L, C, nb + 1), np.uint16)
    for l in range(L):
        for c in range(C):
            bases = np.sort(rng.integers(0, 0x10000 // step, size=nb)) * step
            if c % 3 == 0:
                bases[0] = 0
            nib = rng.integers(0, 16, size=nb)
            nib[rng.random(nb) < 0.5] = 0
            row = bases | nib
            if c % 5 == 1 and nb > 2:
                k = int(rng.integers(1, nb))
                row[k] = (int(bases[k - 1]) // 2) & 0xFFF0
            rows[l, c, :nb] = row
    return rows.view(np.int16)


@pytest.mark.parametrize("step", [16, 256])
@pytest.mark.parametrize("nb", [2, 3, 17, 31, 32, 33, 40, 63])
def test_decode_arbitrary_cdf_rows_vs_oracle(ops, nb, step):
    """Random byte streams of random lengths (zero included) decoded under
    hand-built CDF rows, bit-exact against the oracle.  Bases in steps of
    16 put symbol boundaries inside most 8-bit window prefixes; steps of 256
    keep them on prefix boundaries, so short codes resolve in one lookup."""
    rng = np.random.default_rng(100 + nb + step)
    L, C, T = 2, 64, 96
    cdf = _arbitrary_cdf_rows(rng, L, C, nb, step)
    lengths = rng.integers(0, 60, size=L * C)
    lengths[::7] = 0
    prefix = np.cumsum(lengths).astype(np.int32).reshape(L, C)
    stream = rng.integers(0, 256, size=int(lengths.sum()), dtype=np.uint8)
    want = oc.decode(cdf, stream, prefix, T)
    out = torch.full((L, T, C), 0xEE, dtype=torch.uint8, device=DEV)
    ops.decode_fast_prefsum(torch.from_numpy(cdf).to(DEV), torch.from_numpy(stream).to(DEV),
                            torch.from_numpy(prefix).to(DEV), out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("nb", [2, 17, 32, 33, 64])
@pytest.mark.parametrize("T,C,chunk", [(256, 128, 600), (256, 64, 37), (130, 192, 300), (7, 64, 16), (1, 128, 5)])
def test_encode_arbitrary_cdf_rows_vs_oracle(ops, nb, T, C, chunk):
    """Encode under hand-built CDF rows (codes of 1 to 15 bits, wrapped
    rows, absent symbols) of random symbols, some of them >= n_bins, against
    the oracle: byte lengths, and every output byte including the untouched
    guard bytes past each stream and past short rows (chunk 37 and 5 are
    not multiples of 4; chunk 37, 16 and 5 truncate streams)."""
    rng = np.random.default_rng(300 + nb + T + C + chunk)
    L = 2
    cdf = _arbitrary_cdf_rows(rng, L, C, nb, 16)
    syms = rng.integers(0, nb + 3, size=(L, T, C)).astype(np.uint8)
    guard = np.full((L, C, chunk), 0xEE, np.uint8)
    out = torch.from_numpy(guard.copy()).to(DEV)
    lens = torch.zeros((L, C), dtype=torch.int32, device=DEV)
    ops.encode_fast_new(torch.from_numpy(cdf).to(DEV), torch.from_numpy(syms).to(DEV), out, lens)
    want_out, want_len = oc.encode(cdf, syms, chunk, out=guard.copy())
    torch.cuda.synchronize()
    assert np.array_equal(lens.cpu().numpy(), want_len)
    assert np.array_equal(out.cpu().numpy(), want_out)


@pytest.mark.parametrize("T", [5, 256])
def test_decode_random_streams_under_calculated_cdfs(ops, T):
    """Tables from calculate_cdf on 256-token chunks hold no escape entry,
    so whole blocks take the branch-free decode loop; random byte streams of
    random lengths (zero, shorter than the symbols need, longer) check its
    reads at and past each stream's end against the oracle."""
    rng = np.random.default_rng(7 + T)
    L, C, nb = 2, 128, 32
    syms = np.minimum(np.abs(rng.normal(0, 4, size=(L, 256, C))), nb - 2).astype(np.uint8)
    cdf = oc.calculate_cdf(syms, nb)
    lengths = rng.integers(0, 200, size=L * C)
    lengths[::9] = 0
    lengths[1::9] = 1
    prefix = np.cumsum(lengths).astype(np.int32).reshape(L, C)
    stream = rng.integers(0, 256, size=int(lengths.sum()), dtype=np.uint8)
    want = oc.decode(cdf, stream, prefix, T)
    out = torch.full((L, T, C), 0xEE, dtype=torch.uint8, device=DEV)
    ops.decode_fast_prefsum(torch.from_numpy(cdf).to(DEV), torch.from_numpy(stream).to(DEV),
                            torch.from_numpy(prefix).to(DEV), out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("T", [63, 64, 65, 128, 201, 256])
@pytest.mark.parametrize("C", [64, 96, 192])
def test_decode_valid_streams_across_lengths(ops, T, C):
    """Streams encoded by the oracle from quantised Gaussian symbols, decoded
    at token counts on both sides of the two-wave decoder's range (64..256)
    and with a partial last block of channels; bit-exact symbols."""
    rng = np.random.default_rng(1000 + 7 * T + C)
    L, nb = 3, 32
    scale = rng.uniform(0.5, 6.0, size=(1, 1, C))
    syms = np.clip(np.round(rng.normal(0, 1, size=(L, T, C)) * scale) + 15, 0, 30).astype(np.uint8)
    cdf = oc.calculate_cdf(syms, nb)
    enc, lens = oc.encode(cdf, syms, 4 * T)
    stream, pref = oc.concat_streams(enc, lens)
    out = torch.full((L, T, C), 0xEE, dtype=torch.uint8, device=DEV)
    ops.decode_fast_prefsum(torch.from_numpy(cdf).to(DEV), torch.from_numpy(stream).to(DEV),
                            torch.from_numpy(pref).to(DEV), out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), syms)


def test_codec_through_ctypes(ops, monkeypatch):
    """calculate_cdf, encode and decode with the C++ binding absent (the
    ctypes path), against the oracle."""
    monkeypatch.setattr(ops, "_ext", None)
    syms = _kv_chunk_symbols(L=2, T=200, C=192, seed=5)
    d = torch.from_numpy(syms).to(DEV)
    cdf = ops.calculate_cdf(d, 32)
    want_cdf = oc.calculate_cdf(syms, 32)
    out = torch.zeros((syms.shape[0], syms.shape[2], MAX_TOKENS_PER_CHUNK), dtype=torch.uint8, device=DEV)
    lens = torch.zeros((syms.shape[0], syms.shape[2]), dtype=torch.int32, device=DEV)
    ops.encode_fast_new(cdf, d, out, lens)
    want_out, want_len = oc.encode(want_cdf, syms, MAX_TOKENS_PER_CHUNK)
    torch.cuda.synchronize()
    assert np.array_equal(cdf.cpu().numpy(), want_cdf)
    assert np.array_equal(lens.cpu().numpy(), want_len)
    assert np.array_equal(out.cpu().numpy(), want_out)
    stream, pref = oc.concat_streams(want_out, want_len)
    dec = torch.zeros_like(d)
    ops.decode_fast_prefsum(cdf, torch.from_numpy(stream).to(DEV), torch.from_numpy(pref).to(DEV), dec)
    torch.cuda.synchronize()
    assert torch.equal(dec, d)


@pytest.mark.parametrize("T,C,nb", [(256, 1024, 32), (100, 100, 17), (300, 70, 32), (1, 64, 64), (0, 64, 32)])
def test_calculate_cdf_writes_every_entry(ops, T, C, nb):
    """calculate_cdf allocates its output without a fill: the kernels must
    write every entry.  Called through the C ABI into an output holding
    -1 everywhere (tiled kernel for 1 <= T <= 256, one lane per stream
    above and for T = 0, where every row is zeros: no symbol is present)."""
    rng = np.random.default_rng(T + C + nb)
    syms = rng.integers(0, nb, size=(3, T, C), dtype=np.uint8)
    d = torch.from_numpy(syms).to(DEV)
    out = torch.full((3, C, nb + 1), -1, dtype=torch.int16, device=DEV)
    a, o = ops._desc(d), ops._desc(out)
    ops._run(ops._L.lmc_calculate_cdf(ops._ref(a), nb, ops._ref(o), ops._stream(0)))
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), oc.calculate_cdf(syms, nb))


@pytest.mark.parametrize("C", [128, 96])
def test_decode_empty_streams_write_every_symbol(ops, C):
    """decode's output is allocated without a fill by decode_chunk: with
    every stream empty (all lengths 0), decode still writes every symbol
    (bits past a stream's end read as zeros, rule L6) into an output that
    holds 0xEE.  C = 128 is two full 64-stream blocks (per-lane regions),
    C = 96 adds a partial block (the shared-window path)."""
    rng = np.random.default_rng(77 + C)
    L, T, nb = 2, 40, 32
    syms = rng.integers(0, nb, size=(L, T, C), dtype=np.uint8)
    cdf = oc.calculate_cdf(syms, nb)
    stream = np.zeros(64, np.uint8)
    pref = np.zeros((L, C), np.int32)
    out = torch.full((L, T, C), 0xEE, dtype=torch.uint8, device=DEV)
    ops.decode_fast_prefsum(torch.from_numpy(cdf).to(DEV), torch.from_numpy(stream).to(DEV),
                            torch.from_numpy(pref).to(DEV), out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), oc.decode(cdf, stream, pref, T))


FIB = [1, 1, 2, 3, 5, 8, 13, 21, 34, 55, 89]


def _channels_from_counts(rng, counts_per_channel, T, nb):
    """[T, C] symbols: channel c holds counts[c][s] copies of symbol s in a
    random order, the rest of its T tokens out of range (not counted)."""
    C = len(counts_per_channel)
    out = np.full((T, C), nb + 1, np.uint8)
    for c, counts in enumerate(counts_per_channel):
        col = np.repeat(np.arange(len(counts), dtype=np.uint8), counts)
        assert col.size <= T
        out[: col.size, c] = col
        out[:, c] = rng.permutation(out[:, c])
    return out


def _gaussian_counts(rng, T, bins, nb):
    x = rng.normal(size=(T, 1)).astype(np.float32)
    q = oc.quantize(x[None], bins)[0, :, 0]
    return np.bincount(q, minlength=nb)[:nb].tolist()


def _fib_counts(rng, nb, extra):
    """A Fibonacci run (a Garsia-Wachs tree deeper than 8 levels within 256
    symbols) beside `extra` rare symbols, forwards or backwards."""
    tail = [int(x) for x in rng.integers(1, 3, size=extra)] + [0] * (nb - len(FIB) - extra)
    c = FIB + tail
    return c if rng.random() < 0.5 else c[::-1]


@pytest.mark.parametrize("case", ["one_lane", "quad32", "quad64", "quad64_not_exact", "fallback_one_lane",
                                  "fallback_quad", "long_few_counted", "long_wide_items", "quad_ties"])
def test_calculate_cdf_modes_vs_oracle(ops, case):
    """calculate_cdf picks, per block of 64 streams, one lane per stream
    (at most 16 present symbols) or a quad of lanes per stream with 32- or
    64-leaf items; each mode, rows that fall back to the Shannon lengths
    (Garsia-Wachs trees deeper than 8 levels), chunks longer than 256
    tokens with at most 256 counted symbols (8-bit limit) and chunks of
    65536 tokens or more (no 16-bit items) are bit-exact against the
    oracle.  `quad_ties` gives the node-id quads equal and two- or
    three-valued weights (several optimal trees, where the tie rule picks
    one) and 2..32 present symbols per stream within one block, so the
    lists of one wave end at different steps."""
    rng = np.random.default_rng(sum(map(ord, case)))
    T, nb, C = 256, 32, 128
    if case == "one_lane":
        rows = [_gaussian_counts(rng, T, 16, nb) for _ in range(C)]
    elif case == "quad32":
        rows = [_gaussian_counts(rng, T, 32, nb) for _ in range(C)]
    elif case in ("quad64", "quad64_not_exact"):
        nb = 64 if case == "quad64" else 50
        rows = [_gaussian_counts(rng, T, 64 if nb == 64 else 50, nb) for _ in range(C)]
    elif case == "fallback_one_lane":
        rows = [_fib_counts(rng, nb, int(rng.integers(0, 5))) if c % 3 == 0 else _gaussian_counts(rng, T, 16, nb)
                for c in range(C)]
    elif case == "fallback_quad":
        rows = [_fib_counts(rng, nb, int(rng.integers(5, 15))) if c % 3 == 0 else _gaussian_counts(rng, T, 32, nb)
                for c in range(C)]
    elif case == "long_few_counted":
        T = 700
        rows = [_gaussian_counts(rng, 200, 16 if c < 64 else 32, nb) for c in range(C)]
    elif case == "quad_ties":
        rows = []
        for c in range(C):
            m = 32 if c % 64 == 0 else int(rng.integers(2, 33))
            kind = c % 4
            if kind == 0:
                w = [8] * m
            elif kind == 1:
                w = [1 + (j % 2) for j in range(m)]
            elif kind == 2:
                w = [int(x) for x in rng.choice([1, 2, 4], size=m)]
            else:
                w = [int(x) for x in rng.integers(1, 4, size=m)]
            counts = [0] * nb
            for pos, x in zip(sorted(rng.choice(nb, size=m, replace=False)), w):
                counts[int(pos)] = x
            rows.append(counts)
    else:
        T, C = 65536, 64
        rows = [[4096] * 16 + [0] * 16 for _ in range(C)]
        rows[5] = [32769] + [2 ** j for j in range(15)] + [0] * 16  # a 15-level caterpillar: fallback
    syms = _channels_from_counts(rng, rows, T, nb)[None]
    d = torch.from_numpy(syms).to(DEV)
    cdf = ops.calculate_cdf(d, nb)
    want = oc.calculate_cdf(syms, nb)
    torch.cuda.synchronize()
    assert np.array_equal(cdf.cpu().numpy(), want)


@pytest.mark.parametrize("nb", [1, 2, 3, 5, 8, 15, 16, 17, 31, 32, 33, 48, 63, 64])
def test_calculate_cdf_bin_count_sweep_vs_oracle(ops, nb):
    """Every bin count from 1 to 64 that changes a bound in the kernel (the
    per-wave symbol shares, the register capacity of 32 or 64 bins, exact
    or not, the one-lane / node-id / 64-leaf step modes), with skewed
    histograms (Dirichlet weights, so some symbols are absent and some
    trees exceed the 8-bit limit), token counts around the 256-token piece,
    out-of-range symbols and a partial block of channels: bit-exact against
    the oracle."""
    rng = np.random.default_rng(700 + nb)
    for T in (1, 7, 256, 300):
        L, C = 2, 80
        syms = np.empty((L, T, C), np.uint8)
        for l in range(L):
            for c in range(C):
                p = rng.dirichlet(np.full(nb, float(rng.choice([0.1, 0.5, 3.0]))))
                syms[l, :, c] = rng.choice(nb, size=T, p=p)
        syms[1, :, 3] = nb + 2                # not counted
        d = torch.from_numpy(syms).to(DEV)
        cdf = ops.calculate_cdf(d, nb)
        want = oc.calculate_cdf(syms, nb)
        torch.cuda.synchronize()
        assert np.array_equal(cdf.cpu().numpy(), want), (nb, T)
