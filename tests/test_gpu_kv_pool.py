"""The fused KV-pool store (wmx_kv_pool_store) against the float64 oracle
with the reference's rounding points, and against the reference's eager
PyTorch steps on the GPU. Keys: the bf16 bar (max-abs <= 1e-2 * max(1,
max|ref|), relative L2 <= 5e-3) and >= 99% bit-exact: the rms mean is
summed in another order, so a rare rounding step lands one ulp apart (and
RoPE's sum can cancel, which magnifies that ulp relative to the result);
values: exact.

The producer kernels (wmx_kv_premix, the router GEMM wmx_kv_router, wmx_kv_mix)
against the float64 oracle of kv_pool.py:103-136 / routing.py:108-124 and
against the torch formulation of the harness on the GPU: the bf16 bar and
>= 97% of the outputs bit-exact (a premixed row or a mixture summed in
another order can round one ulp apart, and a logit that moves by one ulp
moves its whole channel's mixture slightly)."""

import pytest
import torch
import torch.nn.functional as F

from oracle import kv_pool as ref
from tests.numerics import assert_bf16_close
from white_matter_amd import kv_pool
from white_matter_amd.cyclic_pass import FeedbackConfig, FeedbackModel, HipKernels

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(key_dtype, value_dtype, weight_dtype, rope_dtype, dim, shape=(2, 3, 2, 37), seed=0):
    gen = torch.Generator().manual_seed(seed)
    b, c, h, t = shape
    key = (torch.randn(b, c, h, t, dim, generator=gen) * 1.7).to(key_dtype)
    value = torch.randn(b, c, h, t, dim, generator=gen).to(value_dtype)
    weight = (1 + 0.2 * torch.randn(c, dim, generator=gen)).to(weight_dtype)
    angle = torch.rand(b, t, dim // 2, generator=gen) * 20.0
    angle = torch.cat((angle, angle), -1)
    return key, value, weight, angle.cos().to(rope_dtype), angle.sin().to(rope_dtype)


def _ulp_close(actual, expected):
    actual, expected = actual.double().cpu(), expected.double().cpu()
    assert_bf16_close(actual, expected, what="kv store keys")
    assert (actual == expected).double().mean() >= 0.99


@pytest.mark.parametrize("dim", [64, 96, 128])
@pytest.mark.parametrize(
    "dtypes",
    [
        (torch.bfloat16, torch.bfloat16, torch.float32, torch.float32),
        (torch.bfloat16, torch.bfloat16, torch.bfloat16, torch.bfloat16),
        (torch.float32, torch.float32, torch.float32, torch.float32),
        (torch.float32, torch.bfloat16, torch.bfloat16, torch.float32),
    ],
)
def test_store_matches_oracle(dim, dtypes):
    key, value, weight, cos, sin = _inputs(*dtypes, dim)
    pool_slots = 50
    keys = torch.full((2, 3, 2, pool_slots, dim), 3.0, dtype=torch.bfloat16)
    values = keys.clone()
    slots = torch.randperm(pool_slots, generator=torch.Generator().manual_seed(1))[:37]
    exp_k, exp_v = ref.write_pool(key, value, weight, cos, sin, keys, values, slots, 1e-6)
    pk, pv = keys.to(DEV), values.to(DEV)
    with torch.no_grad():
        kv_pool.write_pool(key.to(DEV), value.to(DEV), weight.to(DEV), cos.to(DEV), sin.to(DEV), pk, pv, slots.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(pv.cpu(), exp_v)
    untouched = [i for i in range(pool_slots) if i not in slots.tolist()]
    assert torch.equal(pk.cpu()[:, :, :, untouched], exp_k[:, :, :, untouched])
    _ulp_close(pk.cpu()[:, :, :, slots], exp_k[:, :, :, slots])


def test_pool_views_keys_only_and_out_of_range_slots():
    """Channel views of a larger pool (the decoder cache layout), the keys-only
    form, and a slot past the pool that is not written."""
    key, value, weight, cos, sin = _inputs(torch.bfloat16, torch.bfloat16, torch.float32, torch.float32, 64, (2, 2, 2, 9))
    big = torch.zeros(2, 5, 2, 16, 64, dtype=torch.bfloat16, device=DEV)
    view = big[:, 1:3]  # (B, C=2, H, N, D) view with the larger channel stride
    slots = torch.tensor([0, 2, 4, 6, 8, 10, 12, 14, 16])  # 16 is outside the pool
    with torch.no_grad():
        kv_pool.write_pool(key.to(DEV), None, weight.to(DEV), cos.to(DEV), sin.to(DEV), view, None, slots.to(DEV))
    torch.cuda.synchronize()
    k = ref.k_norm_rope(key, weight, cos, sin, 1e-6).bfloat16()
    _ulp_close(view[:, :, :, 0:16:2].cpu(), k[:, :, :, :8])
    assert (big[:, 1:3, :, 1::2] == 0).all() and (big[:, 0] == 0).all() and (big[:, 3:] == 0).all()
    with torch.no_grad():
        direct = kv_pool.k_norm_rope(key.to(DEV), weight.to(DEV), cos.to(DEV), sin.to(DEV))
    _ulp_close(direct, k)


def test_matches_reference_eager_sequence_on_gpu():
    """The reference's eager steps (kv_pool.py:163-172, 216; cyclic.py:448-458)
    on the GPU, bf16 keys: the fused store is within the bf16 tolerance."""
    key, value, weight, cos, sin = (t.to(DEV) for t in _inputs(torch.bfloat16, torch.bfloat16, torch.float32, torch.float32, 128, (2, 4, 2, 64)))
    slots = torch.arange(64, device=DEV) * 2
    keys = torch.zeros(2, 4, 2, 128, 128, dtype=torch.bfloat16, device=DEV)
    values = torch.zeros_like(keys)
    normed = F.rms_norm(key, (128,), None, 1e-6) * weight.view(1, 4, 1, 1, 128).to(key.dtype)
    c, s = cos[:, None, None].to(key.dtype), sin[:, None, None].to(key.dtype)
    eager = (normed * c + torch.cat((-normed[..., 64:], normed[..., :64]), -1) * s).to(torch.bfloat16)
    ek, ev = keys.clone(), values.clone()
    ek.index_copy_(3, slots, eager)
    ev.index_copy_(3, slots, value)
    with torch.no_grad():
        kv_pool.write_pool(key, value, weight, cos, sin, keys, values, slots)
    assert torch.equal(values, ev)
    assert_bf16_close(keys.double().cpu(), ek.double().cpu(), what="kv store vs eager")
    assert (keys[:, :, :, slots] == ek[:, :, :, slots]).float().mean() > 0.95


def _producer_inputs(batch, tokens, sources, hidden, channels, seed, src_dtype, weight_dtype, scale=1.0, stride=1):
    gen = torch.Generator().manual_seed(seed)
    stacked = (torch.randn(batch, tokens, sources, hidden, generator=gen) * scale).to(src_dtype)
    pre_mix = (1 + 0.2 * torch.randn(2, sources, hidden, generator=gen)).to(weight_dtype)
    width = len(range((sources - 1) % stride, sources, stride)) * hidden  # the sources the router reads
    router = tuple(
        (
            (torch.randn(channels * sources, width, generator=gen) * 0.5 / width**0.5).bfloat16(),
            (torch.randn(channels * sources, generator=gen) * 0.25).bfloat16(),
        )
        for _ in range(2)
    )
    gain = (1 + 0.2 * torch.randn(2, channels, hidden, generator=gen)).to(weight_dtype)
    return stacked, pre_mix, router, gain


def _hip_inputs(stacked, pre_mix, router, gain, stride=1):
    with torch.no_grad():
        return kv_pool.projection_inputs(
            stacked.to(DEV), tuple(pre_mix.to(DEV)), tuple((w.to(DEV), b.to(DEV)) for w, b in router),
            tuple(gain.to(DEV)), eps=1e-6, mix_eps=1e-4, router_layer_stride=stride,
        )


def _producer_close(actual, expected, what):
    actual, expected = actual.double().cpu(), expected.double().cpu()
    assert_bf16_close(actual, expected, what=what)
    assert (actual == expected).double().mean() >= 0.97, what


@pytest.mark.parametrize(
    ("batch", "tokens", "sources", "hidden", "channels"),
    [(2, 3, 5, 64, 3), (1, 9, 25, 1024, 8), (2, 2, 3, 2056, 11), (1, 1, 1, 8, 1), (3, 2, 40, 520, 17)],
)
@pytest.mark.parametrize(
    ("src_dtype", "weight_dtype"), [(torch.float32, torch.bfloat16), (torch.bfloat16, torch.float32)]
)
def test_producer_matches_oracle(batch, tokens, sources, hidden, channels, src_dtype, weight_dtype):
    inputs = _producer_inputs(batch, tokens, sources, hidden, channels, hidden + sources, src_dtype, weight_dtype)
    hk, hv = _hip_inputs(*inputs)
    assert hk.shape == hv.shape == (channels, batch * tokens, hidden) and hk.dtype == torch.bfloat16
    expected = ref.projection_inputs(*inputs, 1e-6, 1e-4)
    _producer_close(hk, expected[0], "h_K")
    _producer_close(hv, expected[1], "h_V")


@pytest.mark.parametrize(
    ("sources", "hidden", "channels", "stride"),
    # the model's shape (25 sources, stride 2: sources 0, 2, .., 24), a start
    # past source 0 ((S - 1) % stride = 2), one source read, and a width that
    # splits 64-input stages (the library GEMM path)
    [(25, 1024, 8, 2), (9, 256, 3, 3), (4, 128, 4, 4), (7, 520, 5, 2)],
)
def test_producer_strided_router_matches_oracle(sources, hidden, channels, stride):
    """router_layer_stride > 1 (reference modules/routing.py:66-99; the model
    configuration's default is 2): the router reads every stride-th source
    from the top, in place from the premixed rows."""
    inputs = _producer_inputs(2, 5, sources, hidden, channels, 31 + sources, torch.float32, torch.bfloat16, stride=stride)
    hk, hv = _hip_inputs(*inputs, stride=stride)
    expected = ref.projection_inputs(*inputs, 1e-6, 1e-4, stride)
    _producer_close(hk, expected[0], "h_K")
    _producer_close(hv, expected[1], "h_V")


def test_strided_router_logits_match_gathered_product():
    """wmx_kv_router over a strided source view: the fp32 product of the
    gathered sources' columns, within one bf16 step, and the same bits on a
    second run."""
    rows, sources, hidden, stride, logits = 300, 25, 1024, 2, 200
    gen = torch.Generator().manual_seed(8)
    p = torch.randn(2, rows, sources * hidden, generator=gen).bfloat16().to(DEV)
    read = range((sources - 1) % stride, sources, stride)
    w = [(torch.randn(logits, len(read) * hidden, generator=gen) * (len(read) * hidden) ** -0.5).bfloat16().to(DEV)
         for _ in range(2)]
    b = [torch.randn(logits, generator=gen).bfloat16().to(DEV) for _ in range(2)]
    alpha = torch.ops.white_matter.kv_router(p, w[0], b[0], w[1], b[1], hidden, stride)
    for side in range(2):
        gathered = p[side].view(rows, sources, hidden)[:, read.start :: read.step].reshape(rows, -1)
        exact = gathered.double() @ w[side].double().t() + b[side].double()
        err = (alpha[side].double() - exact).abs()
        assert bool((err <= exact.abs() * 2.0**-8 + 1e-3).all()), f"side {side}: max error {err.max().item():.3e}"
    assert torch.equal(torch.ops.white_matter.kv_router(p, w[0], b[0], w[1], b[1], hidden, stride), alpha)


def test_producer_repeated_source_view_and_small_magnitudes():
    """Sources given as one row per token repeated along S (stride 0: the
    pool's initial write of the embeddings), at magnitudes where both eps
    values move the result."""
    stacked, pre_mix, router, gain = _producer_inputs(2, 5, 7, 256, 4, 1, torch.float32, torch.bfloat16, scale=1e-3)
    router = tuple((w * 0.05, b * 0.02) for w, b in router)  # mixtures ~1e-2: mean(m^2) ~ mix_eps
    row = stacked[:, :, :1]
    hk, hv = _hip_inputs(row.expand(-1, -1, 7, -1), pre_mix, router, gain)
    expected = ref.projection_inputs(row.expand(-1, -1, 7, -1).contiguous(), pre_mix, router, gain, 1e-6, 1e-4)
    _producer_close(hk, expected[0], "h_K")
    _producer_close(hv, expected[1], "h_V")


@torch.no_grad()
def test_producer_matches_torch_formulation_at_c5_width():
    """The harness's C5 producer (25 sources of 1024, 8 channels) on 8 x 64
    tokens: the HIP kernels against the same steps as torch operations on
    the GPU (F.rms_norm, F.linear, matmul), both ending in the projection."""
    config = FeedbackConfig()
    model = FeedbackModel(config, device=DEV, seed=2)
    gen = torch.Generator(device=DEV).manual_seed(5)
    for side in "kv":  # a router with content weights, not only the prior
        weight, bias = model.router[side]
        weight.copy_((torch.randn(weight.shape, generator=gen, device=DEV) * 0.003).bfloat16())
    stacked = torch.randn(8, 64, config.num_sources, config.hidden_size, generator=gen, device=DEV)
    eager = model.projection_inputs(stacked)
    fused = HipKernels.mix(model, stacked)
    for side, a, e in zip("KV", fused, eager, strict=True):
        _producer_close(a, e, f"h_{side}")
    k_fused, v_fused = model.project(stacked, HipKernels)
    k_eager, v_eager = model.project(stacked)
    assert_bf16_close(k_fused.double().cpu(), k_eager.double().cpu(), what="projected keys")
    assert_bf16_close(v_fused.double().cpu(), v_eager.double().cpu(), what="projected values")


@pytest.mark.parametrize(("rows", "inputs", "logits"), [(300, 25 * 1024, 200), (130, 1088, 37), (5, 64, 256)])
def test_router_logits_match_fp32_product(rows, inputs, logits):
    """wmx_kv_router: bf16(p . W^T + b) over 1024-input chunks summed in order,
    against the fp32 product of the same bf16 operands (rows not a multiple
    of 128, a partial last chunk, the widest logit count): within one bf16
    rounding step of the fp32 result, and the same bits on a second run."""
    gen = torch.Generator().manual_seed(rows)
    p = torch.randn(2, rows, inputs, generator=gen).bfloat16().to(DEV)
    w = [(torch.randn(logits, inputs, generator=gen) * inputs**-0.5).bfloat16().to(DEV) for _ in range(2)]
    b = [torch.randn(logits, generator=gen).bfloat16().to(DEV) for _ in range(2)]
    alpha = torch.ops.white_matter.kv_router(p, w[0], b[0], w[1], b[1])
    assert alpha.shape == (2, rows, logits) and alpha.dtype == torch.bfloat16
    for side in range(2):
        exact = p[side].double() @ w[side].double().t() + b[side].double()
        err = (alpha[side].double() - exact).abs()
        assert bool((err <= exact.abs() * 2.0**-8 + 1e-3).all()), f"side {side}: max error {err.max().item():.3e}"
    assert torch.equal(torch.ops.white_matter.kv_router(p, w[0], b[0], w[1], b[1]), alpha)


@pytest.mark.parametrize(("sources", "hidden", "channels", "stride"), [(5, 64, 3, 1), (9, 128, 4, 2)])
def test_producer_training_form_gradients(sources, hidden, channels, stride):
    """Under autograd projection_inputs runs the HIP forward (the same bits as
    without autograd) and the backward differentiates the recomputed eager
    steps: gradients of every input against float64 autograd through the
    oracle (bf16 rounding points as casts, which pass gradients through)."""
    inputs = _producer_inputs(2, 4, sources, hidden, channels, 40 + sources, torch.float32, torch.float32,
                              stride=stride)
    stacked, pre_mix, router, gain = inputs
    leaves = [stacked.to(DEV), pre_mix[0].to(DEV), pre_mix[1].to(DEV), router[0][0].to(DEV), router[0][1].to(DEV),
              router[1][0].to(DEV), router[1][1].to(DEV), gain[0].to(DEV), gain[1].to(DEV)]
    leaves = [t.clone().requires_grad_() for t in leaves]
    hk, hv = kv_pool.projection_inputs(
        leaves[0], (leaves[1], leaves[2]), ((leaves[3], leaves[4]), (leaves[5], leaves[6])), (leaves[7], leaves[8]),
        eps=1e-6, mix_eps=1e-4, router_layer_stride=stride,
    )
    with torch.no_grad():
        plain = _hip_inputs(*inputs, stride=stride)
    assert torch.equal(hk, plain[0]) and torch.equal(hv, plain[1]), "the training form's forward is the HIP forward"
    gen = torch.Generator().manual_seed(7)
    gk = torch.randn(hk.shape, generator=gen)
    gv = torch.randn(hv.shape, generator=gen)
    grads = torch.autograd.grad((hk, hv), leaves, (gk.to(DEV, hk.dtype), gv.to(DEV, hv.dtype)))
    ref_leaves = [t.detach().cpu().double().requires_grad_() for t in leaves]
    want = ref.projection_inputs(
        ref_leaves[0], torch.stack(ref_leaves[1:3]), ((ref_leaves[3], ref_leaves[4]), (ref_leaves[5], ref_leaves[6])),
        torch.stack(ref_leaves[7:9]), 1e-6, 1e-4, stride,
    )
    ref_grads = torch.autograd.grad(want, ref_leaves, torch.stack((gk, gv)).double())
    names = ("stacked", "pre_mix_k", "pre_mix_v", "router_w_k", "router_b_k", "router_w_v", "router_b_v", "gain_k", "gain_v")
    for name, g, r in zip(names, grads, ref_grads):
        err = (g.double().cpu() - r).norm() / r.norm().clamp_min(1e-30)
        assert err <= 2e-2, f"{name}: rel-L2 {err:.3e} against float64 autograd of the oracle"


def test_producer_rejects_bad_shapes():
    stacked, pre_mix, router, gain = _producer_inputs(1, 2, 3, 64, 2, 0, torch.float32, torch.float32)
    args = (tuple(pre_mix.to(DEV)), tuple((w.to(DEV), b.to(DEV)) for w, b in router), tuple(gain.to(DEV)))
    with torch.no_grad(), pytest.raises(ValueError, match="multiples of 8"):
        kv_pool.projection_inputs(stacked[..., :60].to(DEV), tuple(p[:, :60] for p in args[0]), args[1], args[2])
    with torch.no_grad(), pytest.raises(ValueError, match="pre_mix"):
        kv_pool.projection_inputs(stacked[:, :, :2].to(DEV), *args)


@pytest.mark.parametrize("dim", [64, 96, 128])
@pytest.mark.parametrize("rope_dtype", [torch.float32, torch.bfloat16])
@torch.no_grad()
def test_store_rope_by_slot_equals_gathered_rows(dim, rope_dtype):
    """write_pool(rope_by_slot=True) reads each token's cos/sin row at its
    pool slot from (N, D) tables: the same bits as the gathered (B, T, D)
    rows, for one decode token and for several tokens; slots past the pool
    are not written either way."""
    gen = torch.Generator().manual_seed(dim)
    batch, channels, heads, capacity = 3, 2, 5, 40
    weight = (1 + 0.1 * torch.randn(channels, dim, generator=gen)).to(DEV)
    cos = torch.randn(capacity, dim, generator=gen).to(DEV, rope_dtype)
    sin = torch.randn(capacity, dim, generator=gen).to(DEV, rope_dtype)
    for slots in ([17], [3, 9, 38, 0], [39, 40]):
        print(f"rope by slot D={dim} {rope_dtype} slots {slots}", flush=True)
        slot_t = torch.tensor(slots, device=DEV)
        tokens = len(slots)
        key = torch.randn(batch, channels, heads, tokens, dim, generator=gen).to(DEV, torch.bfloat16)
        value = torch.randn(batch, channels, heads, tokens, dim, generator=gen).to(DEV, torch.bfloat16)
        pools = [torch.zeros(2, batch, channels, heads, capacity, dim, device=DEV, dtype=torch.bfloat16) for _ in range(2)]
        rows = slot_t.clamp(max=capacity - 1)
        kv_pool.write_pool(key, value, weight, cos[rows].expand(batch, tokens, dim), sin[rows].expand(batch, tokens, dim),
                           pools[0][0], pools[0][1], slot_t)
        kv_pool.write_pool(key, value, weight, cos, sin, pools[1][0], pools[1][1], slot_t, rope_by_slot=True)
        assert torch.equal(pools[0], pools[1])
        assert bool(pools[1][:, :, :, :, slot_t[slot_t < capacity]].ne(0).any())


@pytest.mark.parametrize("dim", [64, 96, 128])
@pytest.mark.parametrize("key_dtype", [torch.float32, torch.bfloat16])
def test_k_norm_rope_backward_matches_oracle(dim, key_dtype):
    """white_matter::k_norm_rope's backward (wmx_kv_store_bwd) against float64
    autograd of the oracle's transform (no rounding), on rows that do not
    fill the last workgroup (37 tokens); grad_weight sums 2 x 2 x 37 rows
    per channel through the fixed-order parts, so repeats are bit-identical."""
    key, _, weight, cos, sin = _inputs(key_dtype, torch.bfloat16, torch.float32, torch.float32, dim, seed=dim)
    k = key.to(DEV).requires_grad_()
    w = weight.to(DEV).requires_grad_()
    out = kv_pool.k_norm_rope(k, w, cos.to(DEV), sin.to(DEV))
    assert out.dtype == torch.bfloat16
    probe = torch.randn(out.shape, generator=torch.Generator().manual_seed(dim)).bfloat16()
    gk, gw = torch.autograd.grad(out, (k, w), probe.to(DEV))
    assert gk.dtype == key_dtype and gw.dtype == weight.dtype
    kr, wr = key.double().requires_grad_(), weight.double().requires_grad_()
    expected = ref.k_norm_rope(kr, wr, cos, sin, 1e-6, dtype=torch.float64)
    ek, ew = torch.autograd.grad(expected, (kr, wr), probe.double())
    if key_dtype == torch.bfloat16:
        assert_bf16_close(gk.double().cpu(), ek, what="grad key")
    else:
        torch.testing.assert_close(gk.double().cpu(), ek, rtol=2e-4, atol=2e-5 * ek.abs().max().item())
    torch.testing.assert_close(gw.double().cpu(), ew, rtol=1e-4, atol=1e-5 * ew.abs().max().item())
    gk2, gw2 = torch.autograd.grad(kv_pool.k_norm_rope(k, w, cos.to(DEV), sin.to(DEV)), (k, w), probe.to(DEV))
    assert torch.equal(gk, gk2) and torch.equal(gw, gw2)


def test_k_norm_rope_backward_in_a_training_step():
    """The reference's training use (kv_pool.py:213-216, cyclic.py:448-458):
    projected keys -> k_norm_rope -> index_copy_ into a pool copy -> a loss;
    gradients reach the projection input and the norm weight as with the
    eager torch steps (fp32 keys: to the fp32 bar)."""
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(2, 16, 64, generator=gen).to(DEV).requires_grad_()
    proj = (torch.randn(2, 2 * 64, 64, generator=gen) * 0.1).to(DEV)
    weight = (1 + 0.1 * torch.randn(2, 64, generator=gen)).to(DEV).requires_grad_()
    angle = torch.rand(1, 16, 32, generator=gen).to(DEV) * 9.0
    angle = torch.cat((angle, angle), -1)
    cos, sin = angle.cos(), angle.sin()
    slots = torch.arange(16, device=DEV) + 1
    target = torch.randn(1, 2, 2, 17, 64, generator=gen).to(DEV)

    def loss(transform):
        key = (x @ proj.transpose(1, 2)).view(2, 16, 2, 64).permute(0, 2, 1, 3)[None]  # (1, C=2, H=2, T, D)
        pool = torch.zeros(1, 2, 2, 17, 64, device=DEV).index_copy(3, slots, transform(key).float())
        return ((pool - target) ** 2).sum()

    def eager(key):
        normed = F.rms_norm(key, (64,), None, 1e-6) * weight.view(1, 2, 1, 1, 64)
        c, s = cos[:, None, None], sin[:, None, None]
        return (normed * c + torch.cat((-normed[..., 32:], normed[..., :32]), -1) * s).bfloat16()

    gx, gw = torch.autograd.grad(loss(lambda k: kv_pool.k_norm_rope(k, weight, cos, sin)), (x, weight))
    ex, ew = torch.autograd.grad(loss(eager), (x, weight))
    torch.testing.assert_close(gx, ex, rtol=1e-3, atol=1e-3 * ex.abs().max().item())
    torch.testing.assert_close(gw, ew, rtol=1e-3, atol=1e-3 * ew.abs().max().item())
