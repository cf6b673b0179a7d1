"""Fused KV-pool store: key norm, RoPE, casts and the pool write in one pass.

The reference produces a group's keys with an eager sequence
(src/white_matter/modules/kv_pool.py:163-172 `_apply_k_norm_rope`, the
`.to(V_channels.dtype)` cast of :216) and writes them and the values into the
pool with two `index_copy_` along the token axis
(src/white_matter/blocks/_execution/cyclic.py:448-458 `_write_pool`). Here the
whole step is one HIP kernel (wmx_kv_pool_store) that reads each key and value
once and writes the pool slots, with the reference's rounding after every step
when the keys are bf16. Forward only: under autograd the reference's eager
sequence (differentiable) remains the path.
"""

from __future__ import annotations

import torch

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
) -> None:
    """keys[:, :, :, slots] = bf16(rope(rms_norm(key) * k_norm_weight)) and
    values[:, :, :, slots] = bf16(value), in place.

    key/value (B, C, H, T, D) float32 or bfloat16 (the KV pool's projected
    channels), k_norm_weight (C, D), cos/sin (B, T, D) (the group's position
    embeddings), keys/values bf16 pool tensors or views (B, C, H, N, D),
    slots (T,) int64 distinct pool slots. head_dim 64, 96 or 128.
    """
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (key, value, k_norm_weight, cos, sin)):
        raise RuntimeError("write_pool is forward-only; use the reference's eager sequence under autograd")
    if key.ndim != 5 or (value is not None and value.shape != key.shape):
        raise ValueError("key and value must be (B, C, H, T, D) of one shape")
    batch, channels, heads, tokens, dim = key.shape
    if dim not in (64, 96, 128):
        raise ValueError(f"head_dim {dim} is not supported (64, 96 or 128)")
    if k_norm_weight.shape != (channels, dim):
        raise ValueError("k_norm_weight must be (C, D)")
    if cos.shape != (batch, tokens, dim) or sin.shape != cos.shape or sin.dtype != cos.dtype:
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
    a.cos, a.sin, a.rope_stride, a.rope_dtype = cos.data_ptr(), sin.data_ptr(), cos.stride()[:2], _dtype(cos, "cos")
    a.key_pool, a.key_pool_stride = keys.data_ptr(), keys.stride()[:4]
    a.slots = slots.data_ptr()
    a.batch, a.channels, a.heads, a.tokens, a.head_dim = batch, channels, heads, tokens, dim
    a.pool_slots, a.eps = keys.shape[3], float(eps)
    _native.kv_pool_store(a, key.device)


def k_norm_rope(key: torch.Tensor, k_norm_weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, *, eps: float = 1e-6) -> torch.Tensor:
    """bf16(rope(rms_norm(key) * k_norm_weight)) as a new (B, C, H, T, D)
    tensor: the reference's `_apply_k_norm_rope(...).to(bfloat16)`
    (modules/kv_pool.py:163-172, 216)."""
    out = torch.empty(key.shape, device=key.device, dtype=torch.bfloat16)
    slots = torch.arange(key.shape[3], device=key.device)
    write_pool(key, None, k_norm_weight, cos, sin, out, None, slots, eps=eps)
    return out
