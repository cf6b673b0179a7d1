"""KV-pool store in float64 with the reference's rounding points - TEST
INFRASTRUCTURE ONLY (see oracle/__init__.py for who may import it).

Follows src/white_matter/modules/kv_pool.py:163-172 (`_apply_k_norm_rope`:
rms_norm over head_dim, times the per-channel k_norm weight, then
K*cos + rotate_half(K)*sin with cos/sin cast to the key dtype),
src/white_matter/modules/rotary.py:30-34 (`rotate_half`), the cast of
kv_pool.py:216 (`.to(V_channels.dtype)`) and
src/white_matter/blocks/_execution/cyclic.py:448-458 (`_write_pool`: two
index_copy_ along the token axis). Every step is evaluated in float64 and
rounded to the key dtype, as eager PyTorch evaluates it in that dtype; the
rms_norm mean is taken in float64 and its reciprocal square root rounded to
float32 (F.rms_norm computes in float32 for bf16 and float32 inputs).

Pinned (tests/test_kv_pool.py) against the same steps written with
PyTorch's own F.rms_norm and tensor ops on the CPU in the key dtype, and
against rotation invariants of RoPE (pairwise norm preservation, identity
and half-turn rotations).

`projection_inputs` follows src/white_matter/modules/kv_pool.py:97-136
(`KVPool._project` in its bf16 inference form: rms_norm of the sources,
`_premix` :15-19, the mixer, the mix norm with eps 1e-4, `_projection_input`
:22-25) and src/white_matter/modules/routing.py:46-124 (`Router.forward` with
its strided source view, `_RoutedMixer.forward`). Sums are
taken in float64, with a bf16 rounding wherever the reference casts or a
bf16 operation returns (premixed rows, logits, mixtures, outputs). Pinned
(tests/test_kv_pool.py) against the reference's formulation with PyTorch's
F.rms_norm, F.linear and einsum, against the closed form of the routing
prior (each channel reads one source scaled by 2^-2), at magnitudes where
both eps values move the result, by a planted exchange of the two eps, and,
for a strided router, against the full-width router whose weight columns of
the sources it does not read are zero (the same product).
"""

from __future__ import annotations

import torch


def _round(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return x.to(dtype).to(torch.float64)


def k_norm_rope(key, weight, cos, sin, eps, dtype=None):
    """Float64 result of the reference's `_apply_k_norm_rope`
    evaluated in `dtype` (default: key's dtype): key (B,C,H,T,D), weight
    (C,D), cos/sin (B,T,D). Returns float64 (B,C,H,T,D) holding values
    representable in `dtype`."""
    dtype = key.dtype if dtype is None else dtype
    x = key.to(torch.float64)
    inv = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps).to(torch.float32).to(torch.float64)
    y = _round(x * inv, dtype)
    w = _round(weight.to(torch.float64), dtype)[None, :, None, None, :]
    y = _round(y * w, dtype)
    c = _round(cos.to(torch.float64), dtype)[:, None, None, :, :]
    s = _round(sin.to(torch.float64), dtype)[:, None, None, :, :]
    half = y.shape[-1] // 2
    rot = torch.cat((-y[..., half:], y[..., :half]), dim=-1)
    return _round(_round(y * c, dtype) + _round(rot * s, dtype), dtype)


def write_pool(key, value, weight, cos, sin, keys, values, slots, eps):
    """The pool tensors after the reference's `_write_pool` step with the
    keys produced by `k_norm_rope` (cast to the pool dtype) and the values
    cast to the pool dtype. Returns new tensors; inputs are not modified."""
    out_k, out_v = keys.clone(), None if values is None else values.clone()
    out_k.index_copy_(3, slots, k_norm_rope(key, weight, cos, sin, eps).to(keys.dtype))
    if values is not None:
        out_v.index_copy_(3, slots, value.to(values.dtype))
    return out_k, out_v


def projection_inputs(stacked, pre_mix, router, gain, eps, mix_eps, layer_stride=1):
    """Float64 (2, C, B*T, hidden) holding bf16 values: the K-side and V-side
    inputs of the per-channel projections for sources stacked (B, T, S,
    hidden); pre_mix (2, S, hidden); router ((W_K, b_K), (W_V, b_V)) with W
    (C*S, n*hidden) and b (C*S,) (logit of channel c, source s at c*S + s);
    gain (2, C, hidden). The router's context is the premixed sources
    (S - 1) % layer_stride, + layer_stride, ... (n of them), concatenated
    (reference modules/routing.py:66-72, 96-99)."""
    bf16 = torch.bfloat16
    x = stacked.to(torch.float64)
    batch, tokens, sources, hidden = x.shape
    rows = batch * tokens
    channels = gain[0].shape[0]
    normed = x / torch.sqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    out = []
    for side in range(2):
        premixed = _round(normed * pre_mix[side].to(torch.float64), bf16).reshape(rows, sources, hidden)
        weight, bias = (t.to(torch.float64) for t in router[side])
        context = premixed[:, (sources - 1) % layer_stride :: layer_stride].reshape(rows, -1)
        logits = _round(context @ weight.t() + bias, bf16)
        logits = logits.reshape(rows, channels, sources)
        mixed = torch.zeros(rows, channels, hidden, dtype=torch.float64)
        for s in range(sources):  # the routed sum, one source at a time
            mixed += logits[:, :, s, None] * premixed[:, None, s, :]
        mixed = _round(mixed, bf16)
        scale = 1.0 / torch.sqrt(mixed.pow(2).mean(-1, keepdim=True) + mix_eps)
        out.append(_round(mixed * scale * gain[side].to(torch.float64)[None], bf16).permute(1, 0, 2))
    return torch.stack(out)
