"""The portable PyTorch backend (``backend="reference"``) of both operators.

This is the reference's own portable algorithm, kept so that callers who
select it (CPU training, fp32 evaluation) find it in the drop-in: a dense
boolean visibility mask fed to PyTorch's math scaled-dot-product attention
(src/white_matter/ops/cyclic_attention/reference.py:10-42,
 src/white_matter/ops/strict_causal_attention.py:279-322,362-373).
It is selected only by the caller's backend argument (or "auto" on a CPU
tensor), never as a substitute for the HIP kernels on a ROCm device.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel


def _math_sdpa(query, key, value, keep, scale):
    with sdpa_kernel([SDPBackend.MATH]):
        return F.scaled_dot_product_attention(
            query,
            key.to(query.dtype),
            value.to(query.dtype),
            attn_mask=keep,
            dropout_p=0.0,
            scale=scale,
            enable_gqa=True,
        )


def cyclic_keep(q_len, k_len, query_stride, query_offset, metadata, device):
    """Visibility (Tq, Tk) or (B, 1, Tq, Tk): key j <= offset + stride * i, and the
    document rule when metadata is given."""
    q_slot = query_offset + query_stride * torch.arange(q_len, device=device)
    k_slot = torch.arange(k_len, device=device)
    keep = k_slot[None, :] <= q_slot[:, None]
    if metadata is None:
        return keep
    q_seg, k_seg, q_start, k_end = metadata
    shared = (k_seg == -1)[:, None, :]
    same_document = (q_seg[:, :, None] == k_seg[:, None, :]) | shared
    from_start = (k_slot[None, None, :] >= q_start[:, :, None]) | shared
    before_end = torch.arange(q_len, device=device)[None, :, None] < k_end[:, None, :]
    return (keep[None] & same_document & from_start & before_end)[:, None]


def cyclic_attention_portable(query, key, value, *, query_stride, query_offset, metadata=None):
    keep = cyclic_keep(query.shape[-2], key.shape[-2], query_stride, query_offset, metadata, query.device)
    return _math_sdpa(query, key, value, keep, query.shape[-1] ** -0.5)


def strict_causal_attention_portable(
    query, key, value, *, query_start, kv_lengths, use_dummy_token, metadata, key_mask, scale
):
    batch, heads, length, dim = query.shape
    offset = int(use_dummy_token)
    zero = (query[..., :0, :].sum() + key[..., :0, :].sum() + value[..., :0, :].sum()).to(query.dtype)
    if metadata is not None:
        # gather each segment, bottom-right causal inside it, scatter into zeros
        q = query.transpose(1, 2).flatten(0, 1)[metadata.query_indices]
        k = key.transpose(1, 2).flatten(0, 1)[metadata.key_indices]
        v = value.transpose(1, 2).flatten(0, 1)[metadata.key_indices]
        out = query.new_zeros(batch * length, heads, dim) + zero
        for qs, qe, ks, ke in metadata.segments:
            nq, nk = qe - qs, ke - ks
            local_keep = torch.arange(nk, device=query.device)[None, :] <= (
                nk - nq + torch.arange(nq, device=query.device)[:, None]
            )
            seg = _math_sdpa(
                q[qs:qe].transpose(0, 1)[None], k[ks:ke].transpose(0, 1)[None], v[ks:ke].transpose(0, 1)[None],
                local_keep, scale,
            )
            out = out.index_copy(0, metadata.query_indices[qs:qe], seg[0].transpose(0, 1))
        return out.view(batch, length, heads, dim)
    if isinstance(query_start, torch.Tensor):
        starts = query_start.to(device=query.device).expand(batch)
    else:
        starts = torch.full((batch,), query_start, device=query.device, dtype=torch.long)
    position = starts[:, None] + torch.arange(length, device=query.device)
    slot = torch.arange(key.shape[-2], device=query.device) - offset
    keep = slot[None, None, :] < position[:, :, None]
    if kv_lengths is not None:
        keep = keep & (slot[None, None, :] < kv_lengths[:, None, None])
    if use_dummy_token:
        keep[..., 0] = True
    if key_mask is not None:
        keep = keep & key_mask[:, None, :]
    # unread cache slots may hold NaN; zero them so they cannot reach the products
    read = keep.any(1)[:, None, :, None]
    key, value = key.masked_fill(~read, 0), value.masked_fill(~read, 0)
    return _math_sdpa(query, key, value, keep[:, None], scale).transpose(1, 2)
