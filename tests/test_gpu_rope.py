"""GPU parity of rotary_embedding_k_fused through the C ABI.

Tolerance: within 1e-2 absolute of the oracle's float32 restatement rounded
to the key dtype (the kernel is expected to match it exactly: same IEEE
operations, one final rounding), and within one unit in the last place of
the key dtype of the float64 value.  The reference's own accuracy invariant
(tests/v1/test_pos_kernels.py:72-177: fused(old, new, rope(old, k)) vs
rope(new, k), threshold 0.1) is checked too.
"""

import numpy as np
import pytest
import torch

from oracle import rope as orope

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL = 1e-2


@pytest.fixture(scope="module")
def ops():
    import lmcache_amd

    return lmcache_amd.c_ops


def _run(ops, k, old, new, cache, hs, neox, pos_dtype=torch.int64):
    kd = k.to(DEV).clone()
    ops.rotary_embedding_k_fused(old.to(DEV, pos_dtype), new.to(DEV, pos_dtype), kd, hs, cache.to(DEV), neox)
    torch.cuda.synchronize()
    return kd.cpu()


def _expected(k, old, new, cache, hs, neox):
    f32 = orope.fused_rerotate_f32(k.float().numpy(), old.numpy(), new.numpy(), cache.float().numpy(), hs, neox)
    return orope.round_to(f32, k.dtype), orope.fused_rerotate(
        k.float().numpy(), old.numpy(), new.numpy(), cache.float().numpy(), hs, neox)


@pytest.mark.parametrize("neox", [True, False])
def test_blend_shape_4096_tokens(ops, neox):
    """8 heads x 128 bf16 K of 4096 tokens re-positioned 0..4095 ->
    1000..5095, rope theta 500000."""
    T, H, hs = 4096, 8, 128
    cache = orope.cos_sin_cache(8192, hs, 500000.0).to(torch.bfloat16)
    k = torch.randn((T, H * hs), generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    old = torch.arange(T)
    new = old + 1000
    got = _run(ops, k, old, new, cache, hs, neox).float().numpy()
    want, exact = _expected(k, old, new, cache, hs, neox)
    err = np.abs(got - want).max()
    assert err <= TOL, err
    assert np.count_nonzero(got != want) == 0
    # one bf16 ulp of the exact value, plus the fp32 evaluation error, which
    # dominates for outputs near zero (cancellation of O(1) terms)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(exact), 1e-30))) - 7)
    assert (np.abs(got - exact) <= ulp + 1e-5).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("hs", [64, 128])
@pytest.mark.parametrize("neox", [True, False])
def test_reference_accuracy_invariant(ops, dtype, hs, neox):
    """fused(old, new, rope(old, k)) ~ rope(new, k) for sizes 512..4096."""
    for T in (512, 1024, 4096):
        cache = orope.cos_sin_cache(40960, hs, 500000.0).to(dtype)
        x = torch.rand((T, hs * 8), generator=torch.Generator().manual_seed(T)).to(dtype)
        old = torch.arange(T)
        new = torch.arange(100, 100 + T)
        cf = cache.float().numpy()
        k_old = torch.from_numpy(orope.rope_forward(x.float().numpy(), old.numpy(), cf, hs, neox)).to(dtype)
        target = orope.rope_forward(x.float().numpy(), new.numpy(), cf, hs, neox)
        got = _run(ops, k_old, old, new, cache, hs, neox).float().numpy()
        err = np.abs(got - target).max()
        assert err < 0.1, err                    # the reference's threshold
        want, _ = _expected(k_old, old, new, cache, hs, neox)
        assert np.abs(got - want).max() <= TOL


def test_mixed_cache_dtype_and_int32_positions(ops):
    T, H, hs = 300, 4, 128
    cache = orope.cos_sin_cache(2048, hs, 10000.0)  # fp32 cache, bf16 key
    k = torch.randn((T, H * hs), generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    old = torch.randint(0, 1000, (T,), generator=torch.Generator().manual_seed(2))
    new = old + 517
    got = _run(ops, k, old, new, cache, hs, True, pos_dtype=torch.int32).float().numpy()
    want, _ = _expected(k, old, new, cache, hs, True)
    assert np.abs(got - want).max() <= TOL
    assert np.count_nonzero(got != want) == 0


def test_partial_rotary_passthrough(ops):
    T, H, hs, rot = 64, 2, 128, 64
    cache = orope.cos_sin_cache(256, rot, 10000.0).to(torch.bfloat16)
    k = torch.randn((T, H * hs), generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    got = _run(ops, k, torch.arange(T), torch.arange(T) + 9, cache, hs, True)
    assert torch.equal(got.view(T, H, hs)[:, :, rot:].view(torch.int16), k.view(T, H, hs)[:, :, rot:].view(torch.int16))
    want, _ = _expected(k, torch.arange(T), torch.arange(T) + 9, cache, hs, True)
    assert np.abs(got.float().numpy() - want).max() <= TOL


def test_strided_key_view_and_out_of_range_positions(ops):
    """The blending path rotates buf[0] of a [2, T, W] load buffer; tokens
    whose positions fall outside the cache are left as they are."""
    T, H, hs = 128, 8, 128
    cache = orope.cos_sin_cache(512, hs, 500000.0).to(torch.bfloat16)
    buf = torch.randn((2, T, H * hs), generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    old = torch.arange(T)
    new = old + 300
    new[5] = 10_000                                 # outside the cache
    d = buf.to(DEV)
    ops.rotary_embedding_k_fused(old.to(DEV), new.to(DEV), d[0], hs, cache.to(DEV), True)
    torch.cuda.synchronize()
    got = d.cpu()
    assert torch.equal(got[1].view(torch.int16), buf[1].view(torch.int16))
    assert torch.equal(got[0, 5].view(torch.int16), buf[0, 5].view(torch.int16))
    keep = torch.ones(T, dtype=torch.bool)
    keep[5] = False
    want, _ = _expected(buf[0][keep], old[keep], new[keep], cache, hs, True)
    assert np.abs(got[0][keep].float().numpy() - want).max() <= TOL


def test_rejects_integer_key(ops):
    with pytest.raises(ValueError, match="bfloat16, float16 or float32"):
        ops.rotary_embedding_k_fused(torch.arange(4, device=DEV), torch.arange(4, device=DEV),
                                     torch.zeros((4, 128), dtype=torch.int32, device=DEV), 128,
                                     torch.zeros((8, 128), device=DEV), True)
