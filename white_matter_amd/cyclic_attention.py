"""Cyclic (strided-causal) attention with packed documents and a dummy slot.

Drop-in for ``white_matter.ops.cyclic_attention``
(src/white_matter/ops/cyclic_attention/functional.py:11-90) and its
registered operators ``white_matter::cyclic_attn_fwd``, ``cyclic_attn_bwd``,
``cyclic_attn_doc_fwd`` and ``cyclic_attn_doc_bwd``
(src/white_matter/ops/cyclic_attention/_tilelang/registration.py:164-302):
same names, argument names, validation messages and output layout. The
``"tilelang"`` backend literal runs the gfx950 HIP kernels of libwmx_attn.so.

Query i reads key slots j <= query_offset + query_stride * i (strictly below
for strict_past), intersected with the document rule of the metadata. The
HIP forward writes O in (B, Tq, H, D) storage and returns its (B, H, Tq, D)
view, so the output projection reads it without a transpose copy.
"""

from __future__ import annotations

from typing import Literal

import torch

from . import _kernels, portable
from .metadata import CyclicAttentionMetadata


def cyclic_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    query_stride: int = 1,
    query_offset: int = 0,
    strict_past: bool = False,
    metadata: CyclicAttentionMetadata | None = None,
    backend: Literal["reference", "tilelang"] = "reference",
) -> torch.Tensor:
    """Attend from query i to key slots j <= query_offset + query_stride * i.

    strict_past=True makes the bound strict (<). Tensors are
    (batch, heads, sequence, head_dim); K/V share heads and shape; query heads
    are grouped over KV heads. Scale is 1/sqrt(head_dim), no dropout.
    ``backend="reference"`` is the portable math path in the query dtype;
    ``backend="tilelang"`` runs the gfx950 kernels and needs ROCm BF16 with
    head_dim 64, 96 or 128. Metadata must satisfy the contract of
    prepare_cyclic_attention_metadata. Inputs are never mutated.
    """
    if backend not in ("reference", "tilelang"):
        raise ValueError(f"unknown cyclic attention backend: {backend!r}")
    if type(query_stride) is not int or query_stride < 1:
        raise ValueError("query_stride must be a positive integer")
    if type(query_offset) is not int or not 0 <= query_offset < query_stride:
        raise ValueError("query_offset must be in [0, query_stride)")
    if any(x.ndim != 4 for x in (query, key, value)):
        raise ValueError("Q/K/V must have shape (batch, heads, sequence, head_dim)")
    if min(*query.shape, *key.shape) < 1 or key.shape != value.shape:
        raise ValueError("Q/K/V must be nonempty, with matching K/V shapes")
    if query.shape[0] != key.shape[0] or query.shape[-1] != key.shape[-1] or query.shape[1] % key.shape[1]:
        raise ValueError("Q/K/V require matching batch/head_dim and divisible query/KV heads")
    if query_offset + query_stride * (query.shape[-2] - 1) >= key.shape[-2]:
        raise ValueError("query slots must be within the key sequence")
    if any(x.device != query.device or x.dtype != query.dtype for x in (key, value)):
        raise ValueError("Q/K/V must share dtype and device")
    if not query.is_floating_point():
        raise ValueError("Q/K/V must be floating-point tensors")
    if metadata is not None:
        if len(metadata) != 4:
            raise ValueError("document metadata requires four tensors")
        for tensor, length in zip(metadata, (query.shape[-2], key.shape[-2]) * 2):
            if tensor.shape != (query.shape[0], length) or tensor.device != query.device:
                raise ValueError("document metadata shape/device does not match Q/K/V")
            if tensor.dtype not in (torch.int32, torch.int64):
                raise ValueError("document metadata must be int32 or int64")
    query_offset -= int(strict_past)
    if backend == "reference":
        return portable.cyclic_attention_portable(
            query, key, value, query_stride=query_stride, query_offset=query_offset, metadata=metadata
        )
    if query.device.type != "cuda" or query.dtype != torch.bfloat16 or query.shape[-1] not in (64, 96, 128):
        raise ValueError("TileLang cyclic attention requires CUDA BF16 with head_dim 64, 96, or 128")
    # A strict-past residue of -1 is handled in the kernels: query 0 then sees no key.
    if metadata is None:
        return cyclic_attn_fwd(query, key, value, query_stride, query_offset, 64)[0]
    return cyclic_attn_doc_fwd(query, key, value, *metadata, query_stride, query_offset, 64)[0]


# --------------------------------------------------------------- operators ----
def _check_residue(K_stride: int, residue: int) -> None:
    # residue -1 is the strict-past shift of residue 0
    if not -1 <= residue < K_stride:
        raise ValueError(f"cyclic residue must be in [-1, {K_stride}), got {residue}")


def _documents(metadata, Q, K) -> tuple[torch.Tensor, ...] | None:
    if metadata is None:
        return None
    shapes = ((Q.shape[0], Q.shape[2]), (K.shape[0], K.shape[2])) * 2
    if any(tuple(t.shape) != shape or t.device != Q.device for t, shape in zip(metadata, shapes)):
        raise ValueError("document metadata shape/device does not match Q/K/V")
    return tuple(t.to(torch.int32).contiguous() for t in metadata)


def _check_shapes(Q, K, V) -> None:
    if Q.ndim != 4 or K.ndim != 4 or K.shape != V.shape or Q.shape[0] != K.shape[0] or Q.shape[3] != K.shape[3]:
        raise ValueError("Q/K/V require matching batch/head_dim and K/V shapes")
    if Q.shape[1] % K.shape[1]:
        raise ValueError("Q/K/V require divisible query/KV heads")


def _forward_impl(Q, K, V, metadata, K_stride, residue):
    _check_residue(K_stride, residue)
    _check_shapes(Q, K, V)
    q = _kernels.operand(Q)
    k, v = _kernels.operand(K), _kernels.operand(V)
    batch, heads, length, dim = Q.shape
    out = torch.empty(batch, length, heads, dim, device=Q.device, dtype=torch.bfloat16).transpose(1, 2)
    lse = torch.empty(batch, heads, length, device=Q.device, dtype=torch.float32)
    vis = _kernels.Visibility(query_stride=K_stride, query_offset=residue, documents=_documents(metadata, Q, K))
    _kernels.forward(q, k, v, out, lse, dim**-0.5, vis)
    return out.to(Q.dtype) if Q.dtype != torch.bfloat16 else out, lse


def _backward_impl(Q, K, V, metadata, Out, Lse, dOut, K_stride, residue):
    _check_residue(K_stride, residue)
    _check_shapes(Q, K, V)
    if Out.shape != Q.shape or dOut.shape != Q.shape or Lse.shape != Q.shape[:3]:
        raise ValueError("Out/dOut/Lse do not match Q")
    q, k, v = _kernels.operand(Q), _kernels.operand(K), _kernels.operand(V)
    o, g = _kernels.operand(Out), _kernels.operand(dOut)
    dq = torch.empty(Q.shape, device=Q.device, dtype=torch.bfloat16)
    dk = torch.empty(K.shape, device=Q.device, dtype=torch.bfloat16)
    dv = torch.empty(V.shape, device=Q.device, dtype=torch.bfloat16)
    vis = _kernels.Visibility(query_stride=K_stride, query_offset=residue, documents=_documents(metadata, Q, K))
    _kernels.backward(q, k, v, o, Lse.contiguous(), g, dq, dk, dv, Q.shape[-1] ** -0.5, vis)
    return tuple(t.to(Q.dtype) if Q.dtype != torch.bfloat16 else t for t in (dq, dk, dv))


@torch.library.custom_op("white_matter::cyclic_attn_fwd", mutates_args=())
def cyclic_attn_fwd(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    K_stride: int,
    residue: int,
    block_M: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(O, LSE) of cyclic attention; O is a (B, H, Tq, D) view of (B, Tq, H, D)
    storage, LSE the fp32 natural-log row normaliser (+inf for empty rows).
    ``block_M`` is accepted for schema compatibility; tiles are fixed per D."""
    return _forward_impl(Q, K, V, None, K_stride, residue)


def _fake_fwd(Q: torch.Tensor, *_: object, **__: object) -> tuple[torch.Tensor, torch.Tensor]:
    batch, heads, length, dim = Q.shape
    out = torch.empty((batch, length, heads, dim), dtype=Q.dtype, device=Q.device).transpose(1, 2)
    lse = torch.empty((batch, heads, length), dtype=torch.float32, device=Q.device)
    return out, lse


cyclic_attn_fwd.register_fake(_fake_fwd)


@torch.library.custom_op("white_matter::cyclic_attn_bwd", mutates_args=())
def cyclic_attn_bwd(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    Out: torch.Tensor,
    Lse: torch.Tensor,
    dOut: torch.Tensor,
    K_stride: int,
    residue: int,
    block_M: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dQ, dK, dV), contiguous in Q's dtype."""
    return _backward_impl(Q, K, V, None, Out, Lse, dOut, K_stride, residue)


def _fake_bwd(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, *_: object, **__: object):
    # must match the real op exactly: contiguous tensors in Q's dtype
    return (
        torch.empty(Q.shape, dtype=Q.dtype, device=Q.device),
        torch.empty(K.shape, dtype=Q.dtype, device=Q.device),
        torch.empty(V.shape, dtype=Q.dtype, device=Q.device),
    )


cyclic_attn_bwd.register_fake(_fake_bwd)


@torch.library.custom_op("white_matter::cyclic_attn_doc_fwd", mutates_args=())
def cyclic_attn_doc_fwd(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    QSeg: torch.Tensor,
    KSeg: torch.Tensor,
    QStart: torch.Tensor,
    KQEnd: torch.Tensor,
    K_stride: int,
    residue: int,
    block_M: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """cyclic_attn_fwd with the document rule of CyclicAttentionMetadata."""
    return _forward_impl(Q, K, V, (QSeg, KSeg, QStart, KQEnd), K_stride, residue)


cyclic_attn_doc_fwd.register_fake(_fake_fwd)


@torch.library.custom_op("white_matter::cyclic_attn_doc_bwd", mutates_args=())
def cyclic_attn_doc_bwd(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    QSeg: torch.Tensor,
    KSeg: torch.Tensor,
    QStart: torch.Tensor,
    KQEnd: torch.Tensor,
    Out: torch.Tensor,
    Lse: torch.Tensor,
    dOut: torch.Tensor,
    K_stride: int,
    residue: int,
    block_M: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return _backward_impl(Q, K, V, (QSeg, KSeg, QStart, KQEnd), Out, Lse, dOut, K_stride, residue)


cyclic_attn_doc_bwd.register_fake(_fake_bwd)


def _setup_ctx(ctx, inputs, output):
    *tensors, ctx.K_stride, ctx.residue, ctx.block_M = inputs
    ctx.save_for_backward(*tensors, *output)
    ctx.set_materialize_grads(False)  # Lse has no gradient: no zero fill for it


def _backward(ctx, dOut, dLse):
    tensors = ctx.saved_tensors
    if dOut is None:
        dOut = torch.zeros_like(tensors[-2])
    # Q/K/V, optionally four document tensors, then O and LSE
    if len(tensors) == 9:
        grads = cyclic_attn_doc_bwd(*tensors, dOut, ctx.K_stride, ctx.residue, ctx.block_M)
    else:
        grads = cyclic_attn_bwd(*tensors, dOut, ctx.K_stride, ctx.residue, ctx.block_M)
    return (*grads, *((None,) * (len(tensors) - 2)))


cyclic_attn_fwd.register_autograd(_backward, setup_context=_setup_ctx)
cyclic_attn_doc_fwd.register_autograd(_backward, setup_context=_setup_ctx)
