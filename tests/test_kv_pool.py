"""KV-pool store oracle pinning (CPU) and the fused HIP kernel's argument
checks. The oracle is checked against the reference's own steps written
with PyTorch's F.rms_norm and tensor ops in the key dtype
(src/white_matter/modules/kv_pool.py:163-172, rotary.py:30-34), and against
RoPE's rotation invariants."""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import kv_pool as ref


def _torch_steps(key, weight, cos, sin, eps):
    """The reference's `_apply_k_norm_rope` as eager PyTorch evaluates it."""
    normed = F.rms_norm(key, (key.shape[-1],), None, eps)
    k = normed * weight.view(1, weight.shape[0], 1, 1, weight.shape[1]).to(key.dtype)
    c = cos[:, None, None, :, :].to(key.dtype)
    s = sin[:, None, None, :, :].to(key.dtype)
    half = k.shape[-1] // 2
    rot = torch.cat((-k[..., half:], k[..., :half]), dim=-1)
    return (k * c) + (rot * s)


def _inputs(dtype, dim=64, seed=0, shape=(2, 3, 2, 5)):
    gen = torch.Generator().manual_seed(seed)
    b, c, h, t = shape
    key = (torch.randn(b, c, h, t, dim, generator=gen) * 2).to(dtype)
    weight = (1 + 0.1 * torch.randn(c, dim, generator=gen)).to(dtype)
    angle = torch.rand(b, t, dim // 2, generator=gen) * 6.0
    angle = torch.cat((angle, angle), -1)
    return key, weight, angle.cos(), angle.sin()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("dim", [64, 96, 128])
def test_oracle_matches_pytorch_steps(dtype, dim):
    key, weight, cos, sin = _inputs(dtype, dim)
    expected = _torch_steps(key, weight, cos, sin, 1e-6).double()
    actual = ref.k_norm_rope(key, weight, cos, sin, 1e-6)
    if dtype == torch.float32:
        torch.testing.assert_close(actual, expected, rtol=2e-6, atol=2e-6)
    else:
        # the rms mean is summed in another order: a rare 1-ulp flip of a bf16 step
        ulp = expected.abs().clamp_min(2**-126) * 2**-7
        assert ((actual - expected).abs() <= ulp).all()
        assert (actual == expected).float().mean() > 0.99


def test_rotation_invariants():
    key, weight, cos, sin = _inputs(torch.float64, 64, seed=3)
    eps = 1e-6
    plain = ref.k_norm_rope(key, weight, torch.ones_like(cos), torch.zeros_like(sin), eps)
    normed = key / torch.sqrt(key.pow(2).mean(-1, keepdim=True) + eps) * weight[None, :, None, None, :]
    torch.testing.assert_close(plain, normed, rtol=1e-6, atol=1e-6)  # identity rotation
    turned = ref.k_norm_rope(key, weight, -torch.ones_like(cos), torch.zeros_like(sin), eps)
    torch.testing.assert_close(turned, -plain, rtol=0, atol=0)  # half turn
    rotated = ref.k_norm_rope(key, weight, cos, sin, eps)
    half = 32  # RoPE rotates the pairs (d, d + D/2): their norms are kept
    pair = lambda x: x[..., :half] ** 2 + x[..., half:] ** 2  # noqa: E731
    torch.testing.assert_close(pair(rotated), pair(plain), rtol=1e-5, atol=1e-6)
    # a quarter turn maps (a, b) to (-b, a)
    quarter = ref.k_norm_rope(key, weight, torch.zeros_like(cos), torch.ones_like(sin), eps)
    torch.testing.assert_close(quarter, torch.cat((-plain[..., half:], plain[..., :half]), -1), rtol=1e-6, atol=1e-6)
    assert math.isclose(float(cos[0, 0, 0] ** 2 + sin[0, 0, 0] ** 2), 1.0, rel_tol=1e-6)


def test_planted_mistake_is_caught():
    """A rotate_half without the sign flip (a plausible slip) fails the check."""
    key, weight, cos, sin = _inputs(torch.float32, 64, seed=5)
    expected = _torch_steps(key, weight, cos, sin, 1e-6).double()
    x = ref.k_norm_rope(key, weight, torch.ones_like(cos), torch.zeros_like(sin), 1e-6)
    wrong = x * cos[:, None, None].double() + torch.cat((x[..., 32:], x[..., :32]), -1) * sin[:, None, None].double()
    assert not torch.allclose(wrong, expected, rtol=1e-3, atol=1e-3)


def test_write_pool_oracle_scatters_slots():
    key, weight, cos, sin = _inputs(torch.bfloat16, 64, seed=7)
    value = torch.randn(key.shape).bfloat16()
    pool_k = torch.full((2, 3, 2, 9, 64), 7.0).bfloat16()
    pool_v = pool_k.clone()
    slots = torch.tensor([8, 0, 3, 5, 1])
    out_k, out_v = ref.write_pool(key, value, weight, cos, sin, pool_k, pool_v, slots, 1e-6)
    k = ref.k_norm_rope(key, weight, cos, sin, 1e-6).bfloat16()
    for t, s in enumerate(slots.tolist()):
        assert torch.equal(out_k[:, :, :, s], k[:, :, :, t]) and torch.equal(out_v[:, :, :, s], value[:, :, :, t])
    untouched = [s for s in range(9) if s not in slots.tolist()]
    assert (out_k[:, :, :, untouched] == 7).all() and (out_v[:, :, :, untouched] == 7).all()


def test_write_pool_rejects_autograd_and_bad_shapes():
    from white_matter_amd import kv_pool

    key = torch.randn(1, 1, 1, 2, 64, requires_grad=True)
    w, cs = torch.ones(1, 64), torch.ones(1, 2, 64)
    pool = torch.zeros(1, 1, 1, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="forward-only"):
        kv_pool.write_pool(key, None, w, cs, cs, pool, None, torch.tensor([0, 1]))
    with torch.no_grad(), pytest.raises(ValueError, match="head_dim"):
        kv_pool.write_pool(torch.randn(1, 1, 1, 2, 32), None, torch.ones(1, 32), torch.ones(1, 2, 32),
                           torch.ones(1, 2, 32), torch.zeros(1, 1, 1, 4, 32, dtype=torch.bfloat16), None, torch.tensor([0, 1]))
