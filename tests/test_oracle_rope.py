"""Pins the fused K-RoPE oracle (oracle/rope.py) on the CPU.

* The forward rope is checked against complex multiplication (the textbook
  definition: each rotated pair is z * e^{i p theta_j});
* R(new) R(old)^-1 is checked against the reference's own invariant
  fused(old, new, rope(old, k)) == rope(new, k)
  (tests/v1/test_pos_kernels.py:98-142) and reverse(forward) == identity;
* the cos/sin cache against its closed form;
* the float32 restatement against the float64 value;
* a planted sign mistake in the inverse rotation must fail.
"""

import numpy as np
import pytest
import torch

from oracle import rope as orope


def _k(T, H, hs, seed):
    return np.random.default_rng(seed).normal(size=(T, H * hs))


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("hs,rot", [(64, 64), (128, 128), (128, 64)])
def test_forward_rope_is_complex_rotation(neox, hs, rot):
    T, H = 9, 3
    cache = orope.cos_sin_cache(64, rot, 10000.0).double().numpy()
    k = _k(T, H, hs, 1)
    pos = np.arange(T) * 3 + 1
    got = orope.rope_forward(k, pos, cache, hs, neox).reshape(T, H, hs)
    kh = k.reshape(T, H, hs)
    half = rot // 2
    theta = np.arctan2(cache[pos, half:], cache[pos, :half])[:, None, :]
    if neox:
        z = kh[:, :, :half] + 1j * kh[:, :, half:rot]
        r = z * np.exp(1j * theta)
        want = np.concatenate([r.real, r.imag, kh[:, :, rot:]], axis=-1)
    else:
        z = kh[:, :, 0:rot:2] + 1j * kh[:, :, 1:rot:2]
        r = z * np.exp(1j * theta)
        want = kh.copy()
        want[:, :, 0:rot:2] = r.real
        want[:, :, 1:rot:2] = r.imag
    np.testing.assert_allclose(got, want, atol=1e-12)


@pytest.mark.parametrize("neox", [True, False])
def test_fused_equals_rope_at_new_positions(neox):
    T, H, hs = 50, 4, 128
    cache = orope.cos_sin_cache(6000, hs, 500000.0).double().numpy()
    x = _k(T, H, hs, 2)
    old = np.arange(T)
    new = old + 1000
    k_old = orope.rope_forward(x, old, cache, hs, neox)
    got = orope.fused_rerotate(k_old, old, new, cache, hs, neox)
    # the float32-built cos/sin pairs are unit-norm to ~1e-7
    np.testing.assert_allclose(got, orope.rope_forward(x, new, cache, hs, neox), atol=1e-6)
    back = orope.fused_rerotate(got, new, old, cache, hs, neox)
    np.testing.assert_allclose(back, k_old, atol=1e-6)


def test_cos_sin_cache_closed_form():
    P, rot, base = 5096, 128, 500000.0
    cache = orope.cos_sin_cache(P, rot, base).double().numpy()
    p = np.arange(P)[:, None]
    inv = base ** (-np.arange(0, rot, 2) / rot)
    ang = p * inv[None, :]
    # the cache is built in float32 (angles up to ~5096 rad): compare loosely
    np.testing.assert_allclose(cache[:, : rot // 2], np.cos(ang), atol=2e-3)
    np.testing.assert_allclose(cache[:, rot // 2:], np.sin(ang), atol=2e-3)


@pytest.mark.parametrize("neox", [True, False])
def test_f32_restatement_close_to_f64(neox):
    T, H, hs = 64, 8, 128
    cache = orope.cos_sin_cache(5200, hs, 500000.0).to(torch.bfloat16).float().numpy()
    k = orope.round_to(_k(T, H, hs, 3).astype(np.float32), torch.bfloat16)
    old = np.arange(T)
    new = old + 1000
    f32 = orope.fused_rerotate_f32(k, old, new, cache, hs, neox)
    f64 = orope.fused_rerotate(k, old, new, cache, hs, neox)
    assert np.abs(f32 - f64).max() < 1e-5
    # after the single rounding to bf16 the error is at most half a bf16 ulp
    r = orope.round_to(f32, torch.bfloat16)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(f64), 1e-30))) - 7)
    assert (np.abs(r - f64) <= 0.5 * ulp + 1e-5).all()


def test_passthrough_dims_untouched():
    T, H, hs, rot = 5, 2, 128, 64
    cache = orope.cos_sin_cache(64, rot, 10000.0).float().numpy()
    k = _k(T, H, hs, 4).astype(np.float32)
    out = orope.fused_rerotate_f32(k, np.arange(T), np.arange(T) + 7, cache, hs, True)
    assert np.array_equal(out.reshape(T, H, hs)[:, :, rot:], k.reshape(T, H, hs)[:, :, rot:])


def test_planted_sign_mistake_is_caught(monkeypatch):
    """An oracle that applies R(new) R(old) (forgetting to invert the old
    rotation) must fail the invariant above."""

    def wrong(k, old, new, cache, hs, neox):
        return orope.rope_forward(orope.rope_forward(k, old, cache, hs, neox), new, cache, hs, neox)

    monkeypatch.setattr(orope, "fused_rerotate", wrong)
    with pytest.raises(AssertionError):
        test_fused_equals_rope_at_new_positions(True)
