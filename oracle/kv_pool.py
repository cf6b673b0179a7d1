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
