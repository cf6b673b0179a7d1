"""The KV-pool producer on the HIP kernels: the token-local mixing ahead of the
per-channel projection, and the fused store (key norm, RoPE, casts and the
pool write in one pass).

The reference builds the projection's inputs with an eager sequence
(src/white_matter/modules/kv_pool.py:97-136 `KVPool._project`, its bf16
inference form; modules/routing.py:77-124 `Router`, `_RoutedMixer`): an RMS
norm of every source row, the K- and V-side pre-mix products cast to bf16,
a router linear over the premixed row, the routed sum over the sources, the
mix norm and the channel gain cast to bf16 and permuted to (channel, token,
hidden). `projection_inputs` runs that as three HIP steps: wmx_kv_premix, the
router logits (wmx_kv_router: a split-K MFMA GEMM, since the library GEMM of
this shape, few logits over long rows, runs on a few workgroups) and
wmx_kv_mix. Under autograd the same kernels run forward and the backward
recomputes the eager steps and differentiates them (the reference's
selective checkpointing of _project).

The reference produces a group's keys with an eager sequence
(src/white_matter/modules/kv_pool.py:163-172 `_apply_k_norm_rope`, the
`.to(V_channels.dtype)` cast of :216) and writes them and the values into the
pool with two `index_copy_` along the token axis
(src/white_matter/blocks/_execution/cyclic.py:448-458 `_write_pool`). Here the
whole step is one HIP kernel (wmx_kv_pool_store) that reads each key and value
once and writes the pool slots, with the reference's rounding after every step
when the keys are bf16. The in-place pool write is forward-only; training
projects keys through `k_norm_rope`, an operator (white_matter::k_norm_rope)
whose backward is one HIP kernel pair (wmx_kv_store_bwd: the key gradient
and the norm weight's gradient summed in a fixed order).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _native

_DTYPES = {torch.float32: _native.DTYPE_F32, torch.bfloat16: _native.DTYPE_BF16}


def _dtype(t: torch.Tensor, what: str) -> int:
    if t.dtype not in _DTYPES:
        raise TypeError(f"{what} must be float32 or bfloat16, got {t.dtype}")
    return _DTYPES[t.dtype]


def _rows(t: torch.Tensor) -> torch.Tensor:
    """A view whose rows start 16-byte aligned with unit stride along the last
    dimension (a copy otherwise)."""
    elem = t.element_size()
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(s * elem % 16 == 0 for s in t.stride()[:-1])
    return t if ok else t.contiguous()


def write_pool(
    key: torch.Tensor,
    value: torch.Tensor | None,
    k_norm_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor | None,
    slots: torch.Tensor,
    *,
    eps: float = 1e-6,
    rope_by_slot: bool = False,
) -> None:
    """keys[:, :, :, slots] = bf16(rope(rms_norm(key) * k_norm_weight)) and
    values[:, :, :, slots] = bf16(value), in place.

    key/value (B, C, H, T, D) float32 or bfloat16 (the KV pool's projected
    channels), k_norm_weight (C, D), cos/sin (B, T, D) (the group's position
    embeddings), keys/values bf16 pool tensors or views (B, C, H, N, D),
    slots (T,) int64 distinct pool slots. head_dim 64, 96 or 128. With
    rope_by_slot, cos/sin are (N, D) tables of rows by pool slot and token t
    uses row slots[t] of them (a decode step then gathers nothing).
    """
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (key, value, k_norm_weight, cos, sin)):
        raise RuntimeError("write_pool is forward-only; under autograd produce the keys with k_norm_rope")
    if key.ndim != 5 or (value is not None and value.shape != key.shape):
        raise ValueError("key and value must be (B, C, H, T, D) of one shape")
    batch, channels, heads, tokens, dim = key.shape
    if dim not in (64, 96, 128):
        raise ValueError(f"head_dim {dim} is not supported (64, 96 or 128)")
    if k_norm_weight.shape != (channels, dim):
        raise ValueError("k_norm_weight must be (C, D)")
    if rope_by_slot:
        if cos.shape != (keys.shape[3], dim) or sin.shape != cos.shape or sin.dtype != cos.dtype:
            raise ValueError("with rope_by_slot, cos and sin must be (N, D) tables of one dtype")
    elif cos.shape != (batch, tokens, dim) or sin.shape != cos.shape or sin.dtype != cos.dtype:
        raise ValueError("cos and sin must be (B, T, D) of one dtype")
    if keys.ndim != 5 or keys.shape[:3] != (batch, channels, heads) or keys.shape[4] != dim or keys.dtype != torch.bfloat16:
        raise ValueError("keys must be a bf16 (B, C, H, N, D) pool")
    if (values is None) != (value is None) or (values is not None and (values.shape != keys.shape or values.dtype != torch.bfloat16)):
        raise ValueError("values must be a bf16 pool shaped like keys, given exactly when value is")
    if slots.shape != (tokens,):
        raise ValueError("slots must be (T,)")
    for pool in (keys, values):
        if pool is not None and (pool.stride(-1) != 1 or pool.data_ptr() % 16 or any(s % 8 for s in pool.stride()[:-1])):
            raise ValueError("pool views need unit stride along D and 16-byte aligned rows")
    a = _native.KvStoreArgs()
    key = _rows(key)
    cos, sin = _rows(cos), _rows(sin)  # the kernel reads both with cos's strides
    if sin.stride() != cos.stride():
        cos, sin = cos.contiguous(), sin.contiguous()
    weight = k_norm_weight.contiguous()
    slots = slots.to(device=key.device, dtype=torch.int64).contiguous()
    a.key, a.key_stride, a.key_dtype = key.data_ptr(), key.stride()[:4], _dtype(key, "key")
    if value is not None:
        value = _rows(value)
        a.value, a.value_stride, a.value_dtype = value.data_ptr(), value.stride()[:4], _dtype(value, "value")
        a.value_pool, a.value_pool_stride = values.data_ptr(), values.stride()[:4]
    a.k_norm_weight, a.weight_dtype = weight.data_ptr(), _dtype(weight, "k_norm_weight")
    rope_stride = (0, cos.stride(0)) if rope_by_slot else cos.stride()[:2]
    a.cos, a.sin, a.rope_stride, a.rope_dtype = cos.data_ptr(), sin.data_ptr(), rope_stride, _dtype(cos, "cos")
    a.rope_by_slot = int(rope_by_slot)
    a.key_pool, a.key_pool_stride = keys.data_ptr(), keys.stride()[:4]
    a.slots = slots.data_ptr()
    a.batch, a.channels, a.heads, a.tokens, a.head_dim = batch, channels, heads, tokens, dim
    a.pool_slots, a.eps = keys.shape[3], float(eps)
    _native.kv_pool_store(a, key.device)


@torch.library.custom_op("white_matter::k_norm_rope", mutates_args=())
def _k_norm_rope_op(key: torch.Tensor, k_norm_weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, eps: float) -> torch.Tensor:
    out = torch.empty(key.shape, device=key.device, dtype=torch.bfloat16)
    slots = torch.arange(key.shape[3], device=key.device)
    with torch.no_grad():
        write_pool(key, None, k_norm_weight, cos, sin, out, None, slots, eps=eps)
    return out


@_k_norm_rope_op.register_fake
def _(key, k_norm_weight, cos, sin, eps):
    return key.new_empty(key.shape, dtype=torch.bfloat16)


@torch.library.custom_op("white_matter::k_norm_rope_bwd", mutates_args=())
def _k_norm_rope_bwd_op(
    grad: torch.Tensor, key: torch.Tensor, k_norm_weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, eps: float
) -> tuple[torch.Tensor, torch.Tensor]:
    batch, channels, heads, tokens, dim = key.shape
    key = _rows(key)
    grad = _rows(grad.to(torch.bfloat16))
    cos, sin = _rows(cos), _rows(sin)
    if sin.stride() != cos.stride():
        cos, sin = cos.contiguous(), sin.contiguous()
    weight = k_norm_weight.contiguous()
    grad_key = torch.empty(key.shape, device=key.device, dtype=key.dtype)
    grad_weight = torch.empty(channels, dim, device=key.device, dtype=torch.float32)
    a = _native.KvStoreBwdArgs()
    a.key, a.key_stride, a.key_dtype = key.data_ptr(), key.stride()[:4], _dtype(key, "key")
    a.grad_out, a.grad_out_stride = grad.data_ptr(), grad.stride()[:4]
    a.grad_key, a.grad_key_stride = grad_key.data_ptr(), grad_key.stride()[:4]
    a.k_norm_weight, a.weight_dtype = weight.data_ptr(), _dtype(weight, "k_norm_weight")
    a.cos, a.sin, a.rope_stride, a.rope_dtype = cos.data_ptr(), sin.data_ptr(), cos.stride()[:2], _dtype(cos, "cos")
    a.grad_weight = grad_weight.data_ptr()
    a.batch, a.channels, a.heads, a.tokens, a.head_dim, a.eps = batch, channels, heads, tokens, dim, float(eps)
    need = _native.kv_store_bwd_workspace_size(a)
    workspace = torch.empty(max(need, 16), device=key.device, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = workspace.data_ptr(), need
    _native.kv_store_bwd(a, key.device)
    return grad_key, grad_weight.to(k_norm_weight.dtype)


@_k_norm_rope_bwd_op.register_fake
def _(grad, key, k_norm_weight, cos, sin, eps):
    return torch.empty_like(key), torch.empty_like(k_norm_weight)


def _k_norm_rope_setup(ctx, inputs, output):
    key, k_norm_weight, cos, sin, eps = inputs
    ctx.save_for_backward(key, k_norm_weight, cos, sin)
    ctx.eps = eps


def _k_norm_rope_backward(ctx, grad):
    key, k_norm_weight, cos, sin = ctx.saved_tensors
    grad_key, grad_weight = _k_norm_rope_bwd_op(grad, key, k_norm_weight, cos, sin, ctx.eps)
    return grad_key, grad_weight, None, None, None


_k_norm_rope_op.register_autograd(_k_norm_rope_backward, setup_context=_k_norm_rope_setup)


def k_norm_rope(key: torch.Tensor, k_norm_weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, *, eps: float = 1e-6) -> torch.Tensor:
    """bf16(rope(rms_norm(key) * k_norm_weight)) as a new (B, C, H, T, D)
    tensor: the reference's `_apply_k_norm_rope(...).to(bfloat16)`
    (modules/kv_pool.py:163-172, 216). Differentiable in key and
    k_norm_weight (cos and sin are position embeddings and get no gradient):
    the backward evaluates the exact gradient in fp32 on the HIP kernels."""
    return _k_norm_rope_op(key, k_norm_weight, cos, sin, float(eps))


def _weights(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return t.to(dtype).contiguous()


def _weight_dtype(*weights: torch.Tensor) -> torch.dtype:
    return torch.bfloat16 if all(t.dtype == torch.bfloat16 for t in weights) else torch.float32


@torch.library.custom_op("white_matter::kv_premix", mutates_args=())
def kv_premix(stacked: torch.Tensor, pre_mix_k: torch.Tensor, pre_mix_v: torch.Tensor, eps: float) -> torch.Tensor:
    """Both premixed stacks (2, B*T, S*hidden) bf16 of (B, T, S, hidden)
    sources (wmx_kv_premix; shapes checked by `projection_inputs`)."""
    batch, tokens, sources, hidden = stacked.shape
    ok = stacked.stride(-1) == 1 and stacked.data_ptr() % 16 == 0 and all(st % 8 == 0 for st in stacked.stride()[:3])
    x = stacked if ok else stacked.contiguous()
    wdtype = _weight_dtype(pre_mix_k, pre_mix_v)
    pre = [_weights(w, wdtype) for w in (pre_mix_k, pre_mix_v)]
    premixed = torch.empty(2, batch * tokens, sources * hidden, device=stacked.device, dtype=torch.bfloat16)
    a = _native.KvMixArgs()
    a.sources, a.source_stride = x.data_ptr(), x.stride()[:3]
    a.source_dtype, a.weight_dtype = _DTYPES[x.dtype], _DTYPES[wdtype]
    a.batch, a.tokens, a.num_sources, a.hidden, a.channels = batch, tokens, sources, hidden, 1
    a.eps = float(eps)
    for side in range(2):
        a.pre_mix[side] = pre[side].data_ptr()
        a.premixed[side] = premixed[side].data_ptr()
    _native.kv_premix(a, stacked.device)
    return premixed


@kv_premix.register_fake
def _(stacked, pre_mix_k, pre_mix_v, eps):
    batch, tokens, sources, hidden = stacked.shape
    return stacked.new_empty((2, batch * tokens, sources * hidden), dtype=torch.bfloat16)


@torch.library.custom_op("white_matter::kv_mix", mutates_args=())
def kv_mix(
    premixed: torch.Tensor, alpha_k: torch.Tensor, alpha_v: torch.Tensor, gain_k: torch.Tensor, gain_v: torch.Tensor,
    mix_eps: float,
) -> torch.Tensor:
    """The channel rows (2, C, B*T, hidden) bf16 (wmx_kv_mix) from both
    premixed stacks (2, B*T, S*hidden) and both sides' (B*T, C*S) logits."""
    _, rows, width = premixed.shape
    channels, hidden = gain_k.shape
    sources = width // hidden
    wdtype = _weight_dtype(gain_k, gain_v)
    gains = [_weights(g, wdtype) for g in (gain_k, gain_v)]
    alphas = [t if t.stride(-1) == 1 else t.contiguous() for t in (alpha_k, alpha_v)]
    if rows > 1 and alphas[0].stride(0) != alphas[1].stride(0):
        alphas = [t.contiguous() for t in alphas]
    premixed = premixed.contiguous()
    mixed = torch.empty(2, channels, rows, hidden, device=premixed.device, dtype=torch.bfloat16)
    a = _native.KvMixArgs()
    a.weight_dtype, a.source_dtype = _DTYPES[wdtype], _native.DTYPE_BF16
    a.batch, a.tokens, a.num_sources, a.hidden, a.channels = 1, rows, sources, hidden, channels
    a.mix_eps = float(mix_eps)
    a.alpha_stride = alphas[0].stride(0) if rows > 1 else channels * sources
    for side in range(2):
        a.premixed[side] = premixed[side].data_ptr()
        a.alpha[side] = alphas[side].data_ptr()
        a.gain[side] = gains[side].data_ptr()
        a.mixed[side] = mixed[side].data_ptr()
    _native.kv_mix(a, premixed.device)
    return mixed


@kv_mix.register_fake
def _(premixed, alpha_k, alpha_v, gain_k, gain_v, mix_eps):
    channels, hidden = gain_k.shape
    return premixed.new_empty((2, channels, premixed.shape[1], hidden), dtype=torch.bfloat16)


_ROUTER_WORKSPACE: dict[tuple[int, int], torch.Tensor] = {}


def _router_workspace(device: torch.device, need: int) -> torch.Tensor:
    """The router's fp32 partial sums (tens of MB at the model's width), kept
    per device and stream and grown when a call needs more, so that repeated
    calls do not churn the caching allocator with large blocks. Calls on one
    stream run in order, so they may share it."""
    key = (device.index if device.index is not None else torch.cuda.current_device(), torch.cuda.current_stream(device).cuda_stream)
    buf = _ROUTER_WORKSPACE.get(key)
    if buf is None or buf.numel() < need:
        buf = torch.empty(max(need, 16), device=device, dtype=torch.uint8)
        _ROUTER_WORKSPACE[key] = buf
    return buf


@torch.library.custom_op("white_matter::kv_router", mutates_args=())
def kv_router(
    premixed: torch.Tensor,
    weight_k: torch.Tensor,
    bias_k: torch.Tensor,
    weight_v: torch.Tensor,
    bias_v: torch.Tensor,
    hidden: int = 0,
    source_stride: int = 1,
) -> torch.Tensor:
    """Both sides' router logits (2, B*T, C*S) bf16 = bf16(context[side] .
    W_side^T + b_side) (wmx_kv_router) from both premixed stacks (2, B*T,
    S*hidden) and bf16 weights (C*S, n*hidden) and biases (C*S,). The context
    is the premixed row itself (source_stride 1), or the reference Router's
    strided view (routing.py:66-99): the n = len(range(start, S, stride))
    sources start, start + stride, ... with start = (S - 1) % stride, read in
    place from the row (hidden: the sources' width)."""
    _, rows, width = premixed.shape
    logits, inputs = weight_k.shape
    premixed = premixed.contiguous()
    weights = [w.to(torch.bfloat16).contiguous() for w in (weight_k, weight_v)]
    biases = [b.to(torch.bfloat16).contiguous() for b in (bias_k, bias_v)]
    alpha = torch.empty(2, rows, logits, device=premixed.device, dtype=torch.bfloat16)
    a = _native.KvRouterArgs()
    a.rows, a.inputs, a.logits = rows, inputs, logits
    if source_stride != 1:
        sources = width // hidden
        a.row_stride, a.source_width = width, hidden
        a.source_start, a.source_stride = (sources - 1) % source_stride, source_stride
    elif inputs != width:
        raise ValueError("router weights must span the premixed row")
    for side in range(2):
        a.premixed[side] = premixed[side].data_ptr()
        a.weight[side] = weights[side].data_ptr()
        a.bias[side] = biases[side].data_ptr()
        a.alpha[side] = alpha[side].data_ptr()
    need = _native.kv_router_workspace_size(a)
    workspace = _router_workspace(premixed.device, need)
    a.workspace, a.workspace_bytes = workspace.data_ptr(), need
    _native.kv_router(a, premixed.device)
    return alpha


@kv_router.register_fake
def _(premixed, weight_k, bias_k, weight_v, bias_v, hidden=0, source_stride=1):
    return premixed.new_empty((2, premixed.shape[1], weight_k.shape[0]), dtype=torch.bfloat16)


def router_sources(sources: int, layer_stride: int) -> range:
    """The sources a router with `layer_stride` reads (reference routing.py:
    66-72: from (S - 1) % stride, every stride-th, so the top source is
    always among them)."""
    if layer_stride < 1:
        raise ValueError("router_layer_stride must be positive")
    return range((sources - 1) % layer_stride, sources, layer_stride)


def _projection_inputs_eager(stacked, pre_mix, router, gain, eps, mix_eps, read):
    """The reference's _project steps up to the projection as torch operations
    (kv_pool.py:103-136, routing.py:108-124), differentiable: the recompute
    that the training form differentiates, as the reference's selective
    checkpointing recomputes its eager steps. Values are rounded to bf16 where
    the reference's bf16 steps round them; the products run in fp32 (their
    backward then never issues a bf16 batched product over transposed views)."""
    bf16, f32 = torch.bfloat16, torch.float32
    batch, tokens, sources, hidden = stacked.shape
    rows = batch * tokens
    channels = gain[0].shape[0]
    x = stacked.to(f32)
    normed = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    out = []
    for side in range(2):
        premixed = (normed * pre_mix[side].to(f32)).to(bf16).reshape(rows, sources, hidden)
        weight, bias = router[side]
        context = premixed[:, read.start :: read.step].reshape(rows, -1)
        logits = (context.to(f32) @ weight.to(bf16).to(f32).t() + bias.to(bf16).to(f32)).to(bf16)
        mixed = torch.bmm(logits.view(rows, channels, sources).to(f32), premixed.to(f32)).to(bf16)  # (rows, C, d)
        m = mixed.to(f32)
        h = (m * torch.rsqrt(m.pow(2).mean(-1, keepdim=True) + mix_eps) * gain[side].to(f32)[None]).to(bf16)
        out.append(h.permute(1, 0, 2))
    return out[0], out[1]


class _ProjectionInputsFn(torch.autograd.Function):
    """Training form: the forward runs the HIP kernels; the backward
    recomputes the reference's eager steps from the saved inputs and
    differentiates them (the reference trains _project under selective
    checkpointing with the same recompute)."""

    @staticmethod
    def forward(ctx, stacked, pre_k, pre_v, w_k, b_k, w_v, b_v, gain_k, gain_v, eps, mix_eps, stride):
        with torch.no_grad():
            h_k, h_v = _projection_inputs_hip(
                stacked, (pre_k, pre_v), ((w_k, b_k), (w_v, b_v)), (gain_k, gain_v), eps, mix_eps, stride
            )
        ctx.save_for_backward(stacked, pre_k, pre_v, w_k, b_k, w_v, b_v, gain_k, gain_v)
        ctx.config = (eps, mix_eps, stride)
        return h_k, h_v

    @staticmethod
    def backward(ctx, grad_k, grad_v):
        saved = ctx.saved_tensors
        eps, mix_eps, stride = ctx.config
        with torch.enable_grad():
            leaves = [t.detach().requires_grad_(need) for t, need in zip(saved, ctx.needs_input_grad)]
            stacked, pre_k, pre_v, w_k, b_k, w_v, b_v, gain_k, gain_v = leaves
            outs = _projection_inputs_eager(
                stacked, (pre_k, pre_v), ((w_k, b_k), (w_v, b_v)), (gain_k, gain_v), eps, mix_eps,
                router_sources(stacked.shape[2], stride),
            )
            pairs = [(o, g) for o, g in zip(outs, (grad_k, grad_v)) if g is not None]
            wanted = [t for t in leaves if t.requires_grad]
            grads = iter(torch.autograd.grad([o for o, _ in pairs], wanted, [g for _, g in pairs], allow_unused=True))
        out = [next(grads) if t.requires_grad else None for t in leaves]
        return (*out, None, None, None)


def projection_inputs(
    stacked: torch.Tensor,
    pre_mix: tuple[torch.Tensor, torch.Tensor],
    router: tuple[tuple[torch.Tensor, torch.Tensor], tuple[torch.Tensor, torch.Tensor]],
    gain: tuple[torch.Tensor, torch.Tensor],
    *,
    eps: float = 1e-6,
    mix_eps: float = 1e-4,
    router_layer_stride: int = 1,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(h_K, h_V), each (C, B*T, hidden) bf16: the inputs of the per-channel
    K and V projections (reference kv_pool.py:103-136 with its fused bf16
    casts, and routing.py:46-124 with the router reading every
    `router_layer_stride`-th source, as the reference's Router).

    stacked (B, T, S, hidden) float32 or bfloat16 (stride 0 along S repeats
    one row); pre_mix (K, V) weights (S, hidden); router ((W_K, b_K), (W_V,
    b_V)) with W (C*S, n*hidden), n the number of sources the router reads
    (router_sources), and b (C*S,), the logits of channel c and source s at
    c*S + s; gain (K, V) (C, hidden). Per side:
      p = bf16(rms_norm(x, eps) * pre_mix)           (HIP, wmx_kv_premix)
      alpha = bf16(p[read sources] . W^T + b)         (HIP, wmx_kv_router)
      m = bf16(sum_s alpha[c, s] * p[s])               (HIP, wmx_kv_mix)
      h = bf16(rms_norm(m, mix_eps) * gain[c])
    Under autograd (any input requiring grad) the forward still runs the HIP
    kernels and the backward recomputes the reference's eager steps and
    differentiates them, as the reference trains _project under selective
    checkpointing. The three HIP steps are the operators white_matter::kv_premix,
    white_matter::kv_router and white_matter::kv_mix, so the whole function
    traces under torch.compile. Router widths C*S beyond
    _native.KV_ROUTER_MAX_LOGITS, or S*hidden not a multiple of 64, take the
    library GEMM (F.linear) for the logits.
    """
    if torch.is_grad_enabled() and any(
        t.requires_grad for t in (stacked, *pre_mix, *gain, *router[0], *router[1])
    ):
        (w_k, b_k), (w_v, b_v) = router
        return _ProjectionInputsFn.apply(
            stacked, pre_mix[0], pre_mix[1], w_k, b_k, w_v, b_v, gain[0], gain[1], float(eps), float(mix_eps),
            int(router_layer_stride),
        )
    return _projection_inputs_hip(stacked, pre_mix, router, gain, eps, mix_eps, router_layer_stride)


def _projection_inputs_hip(stacked, pre_mix, router, gain, eps, mix_eps, router_layer_stride):
    """projection_inputs' forward on the HIP kernels (arguments checked here)."""
    if stacked.ndim != 4:
        raise ValueError("stacked must be (B, T, S, hidden)")
    sources, hidden = stacked.shape[2:]
    if not stacked.is_cuda:
        raise RuntimeError("projection_inputs runs on the HIP kernels: stacked must be a GPU tensor")
    if stacked.dtype not in _DTYPES:
        raise TypeError(f"stacked must be float32 or bfloat16, got {stacked.dtype}")
    if sources > _native.KV_MIX_MAX_SOURCES or hidden % 8 or hidden > _native.KV_MIX_MAX_HIDDEN:
        raise ValueError(
            f"projection_inputs supports up to {_native.KV_MIX_MAX_SOURCES} sources and hidden sizes that are "
            f"multiples of 8 up to {_native.KV_MIX_MAX_HIDDEN}"
        )
    channels = gain[0].shape[0]
    for w in pre_mix:
        if w.shape != (sources, hidden):
            raise ValueError("pre_mix weights must be (S, hidden)")
    for g in gain:
        if g.shape != (channels, hidden):
            raise ValueError("gains must be (C, hidden), one shape for both sides")
    read = router_sources(sources, router_layer_stride)
    for weight, bias in router:
        if weight.shape != (channels * sources, len(read) * hidden) or bias.shape != (channels * sources,):
            raise ValueError("router weights must be (C*S, n*hidden) with a (C*S,) bias, n the sources read")
    premixed = torch.ops.white_matter.kv_premix(stacked, pre_mix[0], pre_mix[1], float(eps))
    # the HIP product reads the selected sources in place when their width
    # keeps each 64-input stage inside one source
    gather_ok = router_layer_stride == 1 or hidden % 64 == 0
    if channels * sources <= _native.KV_ROUTER_MAX_LOGITS and (len(read) * hidden) % 64 == 0 and gather_ok:
        (w_k, b_k), (w_v, b_v) = router
        alphas = torch.ops.white_matter.kv_router(
            premixed, w_k, b_k, w_v, b_v, hidden, router_layer_stride
        ).unbind(0)
    else:
        rows = premixed.shape[1]
        alphas = [
            F.linear(
                premixed[side].view(rows, sources, hidden)[:, read.start :: read.step].reshape(rows, -1),
                weight.to(torch.bfloat16),
                bias.to(torch.bfloat16),
            )
            for side, (weight, bias) in enumerate(router)
        ]
    mixed = torch.ops.white_matter.kv_mix(premixed, alphas[0], alphas[1], gain[0], gain[1], float(mix_eps))
    return mixed[0], mixed[1]
