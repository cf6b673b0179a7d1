"""KV-pool oracle pinning (CPU) and the fused HIP kernels' argument checks.

The store oracle is checked against the reference's own steps written with
PyTorch's F.rms_norm and tensor ops in the key dtype
(src/white_matter/modules/kv_pool.py:163-172, rotary.py:30-34), and against
RoPE's rotation invariants. The producer oracle (`projection_inputs`) is
checked against the reference's formulation of kv_pool.py:103-136 and
routing.py:108-124 with F.rms_norm, F.linear and einsum, against the closed
form of the routing prior, and by planted mistakes at magnitudes where both
eps values matter."""

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


# ------------------------------------------------------------ producer ----
def _producer_inputs(seed, batch=2, tokens=3, sources=5, hidden=64, channels=3, scale=1.0, logit_scale=0.25):
    gen = torch.Generator().manual_seed(seed)
    stacked = torch.randn(batch, tokens, sources, hidden, generator=gen) * scale
    pre_mix = (1 + 0.2 * torch.randn(2, sources, hidden, generator=gen)).bfloat16()
    router = tuple(
        (
            (torch.randn(channels * sources, sources * hidden, generator=gen) * 0.02).bfloat16(),
            (torch.randn(channels * sources, generator=gen) * logit_scale).bfloat16(),
        )
        for _ in range(2)
    )
    gain = (1 + 0.2 * torch.randn(2, channels, hidden, generator=gen)).bfloat16()
    return stacked, pre_mix, router, gain


def _reference_formulation(stacked, pre_mix, router, gain, eps, mix_eps):
    """kv_pool.py:103-136 (fused bf16 inference form) with routing.py:108-124,
    as eager PyTorch evaluates it on the CPU."""
    batch, tokens, sources, hidden = stacked.shape
    channels = gain.shape[1]
    normed = F.rms_norm(stacked.float(), (hidden,), None, eps)
    out = []
    for side in range(2):
        premixed = (normed * pre_mix[side].float()).bfloat16()  # _premix
        weight, bias = router[side]
        logits = F.linear(premixed.reshape(batch, tokens, sources * hidden), weight, bias)
        logits = logits.view(batch, tokens, channels, sources)
        mixed = torch.einsum("btld,btkl->btkd", premixed, logits)
        mixed = F.rms_norm(mixed.float(), (hidden,), None, mix_eps)
        h = (mixed * gain[side].float()).bfloat16()  # _projection_input
        out.append(h.permute(2, 0, 1, 3).flatten(1, 2))
    return torch.stack(out).double()


def _close_in_bf16(actual, expected, share=0.97):
    """Equal but for rare roundings of a bf16 step that land on the other
    side (sums taken in another order): within 2 bf16 ulps of the result."""
    ulp = expected.abs().clamp_min(2**-126) * 2**-7
    return bool(((actual - expected).abs() <= 2 * ulp).all()) and float((actual == expected).double().mean()) > share


@pytest.mark.parametrize(
    ("scale", "logit_scale"),
    [(1.0, 0.25), (1e-3, 0.25), (1.0, 0.004), (1e-3, 0.004)],  # small magnitudes: both eps values matter
)
def test_producer_oracle_matches_reference_formulation(scale, logit_scale):
    inputs = _producer_inputs(3, scale=scale, logit_scale=logit_scale)
    expected = _reference_formulation(*inputs, 1e-6, 1e-4)
    actual = ref.projection_inputs(*inputs, 1e-6, 1e-4)
    assert actual.shape == (2, 3, 6, 64)
    assert _close_in_bf16(actual, expected)


@pytest.mark.parametrize("stride", [1, 2])
def test_training_recompute_matches_oracle_values_and_gradients(stride):
    """The training form's backward differentiates kv_pool's eager recompute
    of the producer (CPU here): its values equal the oracle's but for rare
    bf16 roundings, and its gradients match float64 autograd through the
    oracle (bf16 rounding points as casts, which pass gradients through). A
    recompute with the two eps values exchanged fails the gradient check."""
    from white_matter_amd import kv_pool

    stacked, pre_mix, _, gain = _producer_inputs(11, scale=1e-2)
    sources, hidden, channels = stacked.shape[2], stacked.shape[3], gain.shape[1]
    read = kv_pool.router_sources(sources, stride)
    gen = torch.Generator().manual_seed(12)
    router = tuple(
        ((torch.randn(channels * sources, len(read) * hidden, generator=gen) * 0.02).bfloat16(),
         (torch.randn(channels * sources, generator=gen) * 0.25).bfloat16())
        for _ in range(2)
    )
    leaves = [stacked, pre_mix[0], pre_mix[1], router[0][0], router[0][1], router[1][0], router[1][1], gain[0], gain[1]]

    def eager(ts, eps=1e-6, mix_eps=1e-4):
        return kv_pool._projection_inputs_eager(ts[0], (ts[1], ts[2]), ((ts[3], ts[4]), (ts[5], ts[6])),
                                                (ts[7], ts[8]), eps, mix_eps, read)

    def oracle(ts):
        return ref.projection_inputs(ts[0], torch.stack(ts[1:3]), ((ts[3], ts[4]), (ts[5], ts[6])),
                                     torch.stack(ts[7:9]), 1e-6, 1e-4, stride)

    ours = [t.clone().float().requires_grad_() for t in leaves]
    theirs = [t.clone().double().requires_grad_() for t in leaves]
    hk, hv = eager(ours)
    want = oracle(theirs)
    assert _close_in_bf16(torch.stack((hk, hv)).double(), want.detach())
    grad = torch.randn(want.shape, generator=gen)
    g_ours = torch.autograd.grad((hk, hv), ours, (grad[0].bfloat16(), grad[1].bfloat16()))
    g_want = torch.autograd.grad(want, theirs, grad.double())
    for g, r in zip(g_ours, g_want):
        assert (g.double() - r).norm() <= 2e-2 * r.norm()
    swapped = [t.clone().float().requires_grad_() for t in leaves]
    sk, sv = eager(swapped, eps=1e-4, mix_eps=1e-6)
    g_swapped = torch.autograd.grad((sk, sv), swapped, (grad[0].bfloat16(), grad[1].bfloat16()))
    assert (g_swapped[0].double() - g_want[0]).norm() > 2e-2 * g_want[0].norm()


def test_producer_oracle_routing_prior_closed_form():
    """The reference's "cyclic" prior with C = S and zero router weights
    (routing.py:9-25, 77-80): channel c reads source c with logit 2^-2, so
    the mixture is p_c / 4 exactly and its mix norm p_c / sqrt(mean(p_c^2) +
    16 mix_eps)."""
    channels = sources = 4
    stacked, pre_mix, _, gain = _producer_inputs(9, sources=sources, channels=channels, scale=0.01)
    bias = torch.zeros(channels, sources)
    bias[torch.arange(channels), torch.arange(channels)] = 0.25
    router = tuple((torch.zeros(channels * sources, sources * 64).bfloat16(), bias.reshape(-1).bfloat16()) for _ in range(2))
    eps, mix_eps = 1e-6, 1e-2  # a large mix eps, so that a mix norm that misses the 1/4 shows
    actual = ref.projection_inputs(stacked, pre_mix, router, gain, eps, mix_eps)
    x = stacked.double()
    normed = x / torch.sqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    for side in range(2):
        p = (normed * pre_mix[side].double()).bfloat16().double()  # (B, T, S, H)
        expected = p / torch.sqrt(p.pow(2).mean(-1, keepdim=True) + 16 * mix_eps) * gain[side].double()[None, None]
        expected = expected.bfloat16().double().permute(2, 0, 1, 3).reshape(channels, -1, 64)
        assert _close_in_bf16(actual[side], expected, share=0.99)


def test_producer_planted_mistakes_are_caught():
    """The two eps exchanged, or the logits read source-major (c + C*s for
    c*S + s): each fails the check above."""
    inputs = _producer_inputs(4, scale=1e-3, logit_scale=0.004)
    expected = _reference_formulation(*inputs, 1e-6, 1e-4)
    assert not _close_in_bf16(ref.projection_inputs(*inputs, 1e-4, 1e-6), expected)
    stacked, pre_mix, router, gain = inputs
    channels, sources = gain.shape[1], stacked.shape[2]
    transposed = tuple(
        (w.view(channels, sources, -1).transpose(0, 1).reshape(channels * sources, -1),
         b.view(channels, sources).t().reshape(-1))
        for w, b in router
    )
    assert not _close_in_bf16(ref.projection_inputs(stacked, pre_mix, transposed, gain, 1e-6, 1e-4), expected)


def _padded_router(router, sources, hidden, read):
    """The full-width router equal to a router whose context is the sources
    `read`: its weight columns of those sources hold that router's columns,
    the others zero."""
    padded = []
    for weight, bias in router:
        full = torch.zeros(weight.shape[0], sources, hidden, dtype=weight.dtype)
        full[:, list(read)] = weight.view(weight.shape[0], len(read), hidden)
        padded.append((full.reshape(weight.shape[0], -1), bias))
    return tuple(padded)


@pytest.mark.parametrize(("sources", "layer_stride"), [(5, 2), (7, 3), (25, 2), (4, 4), (6, 4), (8, 3)])
def test_producer_oracle_strided_router_equals_padded_full_router(sources, layer_stride):
    """A router reading every layer_stride-th source from (S - 1) %
    layer_stride (routing.py:66-72, 96-99) is the full-width router whose
    columns of the other sources are zero: the oracle's strided context gives
    the full-width oracle's result. A context starting at source 0 instead
    (a plausible slip where S - 1 is not a multiple of the stride) does not."""
    hidden, channels = 64, 3
    stacked, pre_mix, _, gain = _producer_inputs(11 + sources, sources=sources, hidden=hidden, channels=channels,
                                                 scale=1e-3, logit_scale=0.004)
    read = range((sources - 1) % layer_stride, sources, layer_stride)
    gen = torch.Generator().manual_seed(sources * layer_stride)
    router = tuple(
        ((torch.randn(channels * sources, len(read) * hidden, generator=gen) * 0.05).bfloat16(),
         (torch.randn(channels * sources, generator=gen) * 0.004).bfloat16())
        for _ in range(2)
    )
    strided = ref.projection_inputs(stacked, pre_mix, router, gain, 1e-6, 1e-4, layer_stride)
    full = ref.projection_inputs(stacked, pre_mix, _padded_router(router, sources, hidden, read), gain, 1e-6, 1e-4)
    assert torch.equal(strided, full)
    if read.start:
        slip = _padded_router(router, sources, hidden, range(0, sources, layer_stride)[: len(read)])
        assert not _close_in_bf16(ref.projection_inputs(stacked, pre_mix, slip, gain, 1e-6, 1e-4), full)
