"""The reference's FlashAttention entry points on the gfx950 HIP kernels.

Drop-in for ``white_matter.ops.flash_attention``
(src/white_matter/ops/flash_attention.py:1-236): the same public names,
signatures, registered operator names and output layouts, so the model's
ordinary-attention readers (layers/backends.py:22,61-116), the strict
operator and the FLOP counter (benchmarks/_flop_counter.py:88-123) find
what they import. Every name runs the kernels of libwmx_attn.so:

  flash_attention_decode     white_matter::flash_attention_decode (:15-49):
                             (B, Sq, H, D) queries over (B, N, Hkv, D) caches
                             with per-row lengths; one query token runs the
                             split-K decode kernel, several the dense kernel
                             with bottom-right causal rows (or all visible
                             slots when causal is False)
  torch_flash_decode         single-query decode on (B, H, N, D) caches (:52-103)
  can_use_torch_flash        whether the HIP kernels take these operands (:106-108)
  TorchFlashVarlen           packed varlen forward/backward (:125-167)
  TorchFlashDense            dense forward/backward writing (B, T, H, D) (:213-236)
  white_matter::torch_flash_dense_forward
                             its registered forward (:170-211)

Head dims that are not 64, 96 or 128 are zero-padded to the next of those
(exact for attention); above 128 the kernels refuse with RuntimeError. The
kernels compute in bf16 with fp32 accumulation; fp16 operands are rounded to
bf16 on the way in and results are returned in the operands' dtype.
"""

from __future__ import annotations

from typing import Any

import torch

from . import _kernels
from .strict_causal_attention import (
    StrictCausalMetadata,
    _schedule_flags,
    _work_units,
    strict_decode,
    strict_dense_bwd,
    strict_dense_fwd,
    strict_varlen_bwd,
    strict_varlen_fwd,
)

_EMPTY = None


def _unsupported(dim: int) -> RuntimeError:
    return RuntimeError(f"the gfx950 attention kernels: this path does not support head_dim {dim} (maximum 128)")


def _padded(dim: int) -> int:
    size = _kernels.kernel_head_dim(dim)
    if size is None:
        raise _unsupported(dim)
    return size


def _empty_rows(device: torch.device) -> torch.Tensor:
    return torch.empty(0, dtype=torch.long, device=device)


# ---------------------------------------------------------------- decode ----
@torch.library.custom_op("white_matter::flash_attention_decode", mutates_args=())
def flash_attention_decode(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    lengths: torch.Tensor,
    scale: float,
    causal: bool,
    num_splits: int = 0,
) -> torch.Tensor:
    """Attention of (B, Sq, H, D) queries over the first ``lengths[b]`` slots
    of (B, N, Hkv, D) key/value caches (flash_attn_with_kvcache with
    cache_seqlens, reference flash_attention.py:15-36). With ``causal`` query
    s sees slots j <= lengths[b] - Sq + s (bottom-right alignment); a single
    query sees every visible slot either way. Output (B, Sq, H, D) in the
    query dtype; a query that sees no slot outputs zeros."""
    batch, count, heads, dim = query.shape
    size = _padded(dim)
    q, k, v = (_kernels.pad_head_dim(t, size).transpose(1, 2) for t in (query, key, value))
    lengths = lengths.to(device=query.device)
    if count == 1:
        out = strict_decode(q, k, v, lengths, 0, None, None, False, scale, num_splits)
    else:
        limit = (lengths.to(torch.int64) - 1).to(torch.int32)
        first = (lengths.to(torch.int64) - count).to(torch.int32) if causal else limit
        out, _ = strict_dense_fwd(q, k, v, 0, first, limit, None, False, scale)
    return out[..., :dim].to(query.dtype)


@flash_attention_decode.register_fake
def _fake_decode(query, key, value, lengths, scale, causal, num_splits=0):
    return query.new_empty(query.shape)


def torch_flash_decode(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    lengths: torch.Tensor,
    scale: float,
    *,
    static_cache: bool = False,
) -> torch.Tensor:
    """Single-query attention over (B, Hkv, N, D) caches (channel views of a
    pool with any strides are read in place) with device-resident lengths:
    query (B, H, 1, D) sees slots j < lengths[b]. Returns (B, 1, H, D) in the
    query dtype (reference flash_attention.py:52-103). With ``static_cache``
    a compiled caller specialises on the batch, KV-head and capacity sizes as
    the reference's does; no offsets are built either way (the kernel reads
    the cache through its strides)."""
    if static_cache and torch.compiler.is_compiling():
        torch._dynamo.mark_static(query, 0)
        torch._dynamo.mark_static(key, 1)
        torch._dynamo.mark_static(key, 2)
    dim = query.shape[-1]
    size = _padded(dim)
    q, k, v = (_kernels.pad_head_dim(t, size) for t in (query, key, value))
    out = strict_decode(q, k, v, lengths.to(device=query.device), 0, None, None, False, scale, 0)
    return out[..., :dim].to(query.dtype)


def can_use_torch_flash(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    """Whether the HIP kernels take these (B, T, H, D) operands: ROCm device
    tensors of one 16-bit float dtype, head_dim <= 128, matching batch and
    head_dim, query heads a multiple of the key/value heads (reference
    flash_attention.py:106-108 asks PyTorch's FlashAttention the same)."""
    tensors = (q, k, v)
    if any(t.ndim != 4 or not t.is_cuda for t in tensors):
        return False
    if any(t.dtype not in (torch.bfloat16, torch.float16) or t.dtype != q.dtype for t in tensors):
        return False
    if k.shape != v.shape or q.shape[0] != k.shape[0] or q.shape[-1] != k.shape[-1]:
        return False
    if k.shape[2] < 1 or q.shape[2] % k.shape[2]:
        return False
    return _kernels.kernel_head_dim(q.shape[-1]) is not None


# ----------------------------------------------------------------- dense ----
def _dense_offset(length: int, keys: int, causal: bool) -> int:
    # bottom-right causal: query i sees keys j <= i + keys - length; otherwise all keys
    return keys - length if causal else keys - 1


@torch.library.custom_op("white_matter::torch_flash_dense_forward", mutates_args=())
def torch_flash_dense_forward(
    query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scale: float, causal: bool
) -> tuple[torch.Tensor, torch.Tensor]:
    """Dense attention of (B, H, T, D) queries over (B, Hkv, N, D) keys:
    output (B, T, H, D) in the query dtype and LSE (B, H, T) fp32 (reference
    flash_attention.py:170-190). ``causal`` aligns bottom-right."""
    batch, heads, length, dim = query.shape
    size = _padded(dim)
    q, k, v = (_kernels.pad_head_dim(t, size) for t in (query, key, value))
    out, lse = strict_dense_fwd(q, k, v, _dense_offset(length, key.shape[2], causal), None, None, None, False, scale)
    return out[..., :dim].to(query.dtype), lse


@torch_flash_dense_forward.register_fake
def _fake_dense_forward(query, key, value, scale, causal):
    batch, heads, length, dim = query.shape
    return query.new_empty(batch, length, heads, dim), query.new_empty(batch, heads, length, dtype=torch.float32)


class TorchFlashDense(torch.autograd.Function):
    """Dense attention writing contiguous (B, T, H, D) output from (B, H, T, D)
    operands, with its backward on the HIP kernels (reference
    flash_attention.py:213-236)."""

    @staticmethod
    def forward(
        ctx: Any, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scale: float, causal: bool
    ) -> torch.Tensor:
        output, lse = torch_flash_dense_forward(query, key, value, scale, causal)
        ctx.save_for_backward(query, key, value, output, lse)
        ctx.scale, ctx.causal = scale, causal
        return output

    @staticmethod
    def backward(ctx: Any, grad: torch.Tensor) -> tuple[torch.Tensor | None, ...]:
        query, key, value, output, lse = ctx.saved_tensors
        dim = query.shape[-1]
        size = _padded(dim)
        q, k, v = (_kernels.pad_head_dim(t, size) for t in (query, key, value))
        out, dout = (_kernels.pad_head_dim(t, size) for t in (output, grad))
        offset = _dense_offset(query.shape[2], key.shape[2], ctx.causal)
        dq, dk, dv = strict_dense_bwd(q, k, v, out, lse, dout, offset, None, None, None, False, ctx.scale)
        return (
            dq[..., :dim].to(query.dtype),
            dk[..., :dim].to(key.dtype),
            dv[..., :dim].to(value.dtype),
            None,
            None,
        )


# ---------------------------------------------------------------- varlen ----
def _packed_schedule(cu_q: torch.Tensor, cu_k: torch.Tensor, max_q: int, max_k: int, total_k: int):
    """A packed (total, H, D) batch as one row of varlen segments: segment s
    holds queries cu_q[s]:cu_q[s+1] and keys cu_k[s]:cu_k[s+1] of that row,
    bottom-right causal (FlashAttention's varlen causal alignment)."""
    total_q = int(cu_q[-1])
    device = cu_q.device
    return StrictCausalMetadata(
        torch.arange(total_q, device=device),
        torch.arange(total_k, device=device),
        cu_q.to(torch.int32),
        cu_k.to(torch.int32),
        total_q,
        max_k,
        total_k,
    )


class TorchFlashVarlen(torch.autograd.Function):
    """Packed varlen attention, causal with bottom-right alignment per segment:
    query (total_q, H, D), key/value (total_k, Hkv, D), cu_q/cu_k int32
    offsets; output (total_q, H, D) (reference flash_attention.py:125-167)."""

    @staticmethod
    def forward(
        ctx: Any,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        cu_q: torch.Tensor,
        cu_k: torch.Tensor,
        max_q: int,
        max_k: int,
        scale: float,
    ) -> torch.Tensor:
        dim = query.shape[-1]
        size = _padded(dim)
        q, k, v = (_kernels.pad_head_dim(t, size).unsqueeze(0).transpose(1, 2) for t in (query, key, value))
        schedule = _packed_schedule(cu_q, cu_k, max_q, max_k, key.shape[0])
        max_q_, max_k_, flags = _schedule_flags(schedule)
        units = _work_units(schedule, query_extent=query.shape[0])
        none = _empty_rows(query.device)
        out, lse = strict_varlen_fwd(
            q, k, v, schedule.query_indices, schedule.key_indices, schedule.cu_queries, schedule.cu_keys,
            max_q_, max_k_, flags, scale, none, none, none, *units,
        )
        ctx.save_for_backward(query, key, value, out, lse)
        ctx.schedule, ctx.scale = schedule, scale
        return out[0, :, :, :dim].to(query.dtype)

    @staticmethod
    def backward(ctx: Any, grad: torch.Tensor) -> tuple[torch.Tensor | None, ...]:
        query, key, value, out, lse = ctx.saved_tensors
        dim = query.shape[-1]
        size = out.shape[-1]
        q, k, v = (_kernels.pad_head_dim(t, size).unsqueeze(0).transpose(1, 2) for t in (query, key, value))
        dout = _kernels.pad_head_dim(grad, size).unsqueeze(0)
        s = ctx.schedule
        max_q, max_k, flags = _schedule_flags(s)
        none = _empty_rows(query.device)
        dq, dk, dv = strict_varlen_bwd(
            q, k, v, out, lse, dout, s.query_indices, s.key_indices, s.cu_queries, s.cu_keys,
            max_q, max_k, flags, ctx.scale, none, none, *_work_units(s, query_extent=query.shape[0]),
        )
        return (
            dq[0].transpose(0, 1)[..., :dim].to(query.dtype),
            dk[0].transpose(0, 1)[..., :dim].to(key.dtype),
            dv[0].transpose(0, 1)[..., :dim].to(value.dtype),
            None, None, None, None, None,
        )
