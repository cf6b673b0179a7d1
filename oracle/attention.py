"""float64 attention under the reference's visibility rules (test oracle).

The reference's portable path is a dense boolean mask fed to math SDPA
(src/white_matter/ops/cyclic_attention/reference.py:10-42,
 src/white_matter/ops/strict_causal_attention.py:279-322,362-373). The
oracle builds the same masks and evaluates softmax(Q K^T * scale) V
explicitly in float64, with rows that see nothing giving zero output and
zero gradient (the math backend's safe softmax). Gradients come from
autograd through these float64 expressions.
"""

from __future__ import annotations

import numpy as np
import torch


def masked_attention(q, k, v, keep, scale, dtype=torch.float64):
    """q (B,Hq,Tq,D), k/v (B,Hkv,Tk,D), keep broadcastable to (B,Hq,Tq,Tk).
    Query head h reads KV head h // (Hq // Hkv). Computes and returns `dtype`
    (float64 for parity checks; float32 is the reference's CPU precision)."""
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    group = q.shape[1] // k.shape[1]
    k = k.repeat_interleave(group, dim=1)
    v = v.repeat_interleave(group, dim=1)
    scores = (q @ k.transpose(-1, -2)) * scale
    keep = keep.expand(scores.shape)
    scores = scores.masked_fill(~keep, float("-inf"))
    row_max = scores.amax(-1, keepdim=True)
    row_max = torch.where(torch.isfinite(row_max), row_max, torch.zeros_like(row_max)).detach()
    weights = torch.exp(scores - row_max)
    total = weights.sum(-1, keepdim=True)
    weights = weights / torch.where(total > 0, total, torch.ones_like(total))
    return weights @ v


def cyclic_keep(q_len, k_len, query_stride, query_offset, metadata=None):
    """reference.py:18-30: j <= offset + stride * i, and with metadata
    (q_seg == k_seg or k_seg == -1) and (j >= q_start or k_seg == -1) and i < k_end."""
    i = torch.arange(q_len)[:, None]
    j = torch.arange(k_len)[None, :]
    keep = j <= query_offset + query_stride * i
    if metadata is None:
        return keep[None, None]
    qseg, kseg, qstart, kend = (torch.as_tensor(np.asarray(t)).long().cpu() for t in metadata)
    dummy = kseg[:, None, :] == -1
    same = (qseg[:, :, None] == kseg[:, None, :]) | dummy
    after = (j[None] >= qstart[:, :, None]) | dummy
    before = i[None] < kend[:, None, :]
    return (keep[None] & same & after & before)[:, None]


def cyclic_attention(q, k, v, *, query_stride=1, query_offset=0, strict_past=False, metadata=None):
    """cyclic_attention(backend="reference") (functional.py:59-67, reference.py:10-42)."""
    keep = cyclic_keep(q.shape[2], k.shape[2], query_stride, query_offset - int(strict_past), metadata)
    return masked_attention(q, k, v, keep.to(q.device), q.shape[-1] ** -0.5)


def strict_keep(batch, length, slots, query_start, kv_lengths=None, use_dummy_token=False, key_mask=None):
    """strict_causal_attention.py:299-308: slot' = s - dummy; keep slot' < start + i
    and slot' < kv_len, slot 0 always with a dummy, and key_mask. (B, T, N) bool."""
    offset = int(use_dummy_token)
    starts = torch.as_tensor(query_start).long().cpu().expand(batch)
    position = starts[:, None] + torch.arange(length)[None, :]
    slot = torch.arange(slots) - offset
    keep = slot[None, None, :] < position[:, :, None]
    if kv_lengths is not None:
        keep = keep & (slot[None, None, :] < torch.as_tensor(kv_lengths).long().cpu()[:, None, None])
    if use_dummy_token:
        keep[..., 0] = True
    if key_mask is not None:
        keep = keep & torch.as_tensor(key_mask).bool().cpu()[:, None, :]
    return keep


def schedule_keep(metadata, batch, length, slots):
    """Visibility implied by a varlen schedule (strict_causal_attention.py:279-298):
    for segment (qs, qe, ks, ke), local key j is visible to local query i iff
    j <= (ke - ks) - (qe - qs) + i. Keys never leave their query's row, so the
    result is a per-row (B, T, N) mask; queries outside the schedule see nothing."""
    qi = np.asarray(metadata["query_indices"], dtype=np.int64)
    ki = np.asarray(metadata["key_indices"], dtype=np.int64)
    cq = np.asarray(metadata["cu_queries"], dtype=np.int64)
    ck = np.asarray(metadata["cu_keys"], dtype=np.int64)
    extent = int(metadata["key_extent"])
    keep = np.zeros((batch, length, slots), dtype=bool)
    for s in range(len(cq) - 1):
        nq, nk = cq[s + 1] - cq[s], ck[s + 1] - ck[s]
        for a in range(nq):
            b, t = divmod(int(qi[cq[s] + a]), length)
            for j in range(nk):
                if j <= nk - nq + a:
                    kb, slot = divmod(int(ki[ck[s] + j]), extent)
                    assert kb == b, "a schedule key left its query's row"
                    keep[b, t, slot] = True
    return torch.from_numpy(keep)


def strict_attention(
    q,
    k,
    v,
    *,
    query_start=0,
    kv_lengths=None,
    use_dummy_token=False,
    metadata=None,
    key_mask=None,
    softmax_scale=None,
):
    """strict_causal_attention(backend="reference") -> float64 (B, T, H, D)."""
    batch, heads, length, dim = q.shape
    scale = dim**-0.5 if softmax_scale is None else softmax_scale
    if metadata is not None:
        keep = schedule_keep(metadata, batch, length, k.shape[2])
    else:
        keep = strict_keep(batch, length, k.shape[2], query_start, kv_lengths, use_dummy_token, key_mask)
    # slots that no query reads may hold NaN in the cache; they never enter a product
    read = keep.any(1)[:, None, :, None].to(k.device)
    k = k.double().masked_fill(~read, 0)
    v = v.double().masked_fill(~read, 0)
    return masked_attention(q, k, v, keep[:, None].to(q.device), scale).transpose(1, 2)


def per_query_strict(q, k, v, starts, dummy, docs=None, lengths=None):
    """Explicit per-query softmax from document ids, building no schedule
    (restates the test oracle of tests/unit/test_strict_causal_attention.py:16-39).
    Query i of row b sits at slot starts[b] + i; it reads earlier slots of its
    document run (padding skipped), capped by lengths, plus the dummy.
    Returns float64 (B, T, H, D)."""
    batch, heads, count, dim = q.shape
    group = heads // k.shape[1]
    # rows that see nothing stay zero but keep autograd linkage to q/k/v
    linked = (q[..., :0, :].sum() + k[..., :0, :].sum() + v[..., :0, :].sum()).double()
    out = torch.zeros(batch, count, heads, dim, dtype=torch.float64) + linked
    for b in range(batch):
        for i in range(count):
            pos = int(starts[b]) + i
            limit = min(pos, k.shape[2] - int(dummy))
            if lengths is not None:
                limit = min(limit, int(lengths[b]))
            slots = list(range(max(limit, 0)))
            if docs is not None:
                first = pos
                while first and (docs[b, first - 1] < 0 or docs[b, first - 1] == docs[b, pos]):
                    first -= 1
                slots = [s for s in slots if s >= first and docs[b, s] >= 0 and docs[b, pos] >= 0]
            idx = ([0] if dummy and (docs is None or docs[b, pos] >= 0) else []) + [s + int(dummy) for s in slots]
            if not idx:
                continue
            kk = k[b][:, idx].double().repeat_interleave(group, 0)
            vv = v[b][:, idx].double().repeat_interleave(group, 0)
            w = ((q[b, :, i, None].double() * kk).sum(-1) * dim**-0.5).softmax(-1)
            out = out.index_put((torch.tensor(b), torch.tensor(i)), (w[..., None] * vv).sum(-2))
    return out


def bf16_pipeline(q, k, v, dout, keep, scale):
    """Outputs and gradients with the rounding points of the reference's
    accelerated path, evaluated in float64 (src/white_matter/ops/cyclic_attention/
    _tilelang/forward.py:99-131: unnormalised probabilities cast to bf16 before
    the PV product, output cast to bf16; backward_preprocess.py:34-49: delta from
    the bf16 output; backward_query.py:86-109 and backward_key_value.py:102-132:
    P and dS cast to bf16 before their products, gradients cast to bf16).

    q (B,Hq,Tq,D), k/v (B,Hkv,Tk,D), dout like q, keep broadcastable to
    (B,Hq,Tq,Tk). Returns (out, dq, dk, dv) in float64 (B,H,T,D) layouts.
    An exact kernel differs from this only by fp32 accumulation order.
    """

    def bf(x):
        return x.to(torch.bfloat16).double()

    q, k, v, dout = (t.double() for t in (q, k, v, dout))
    batch, heads, length, dim = q.shape
    group = heads // k.shape[1]
    kk, vv = k.repeat_interleave(group, 1), v.repeat_interleave(group, 1)
    s = (q @ kk.transpose(-1, -2)) * scale
    s = s.masked_fill(~keep.expand(s.shape), float("-inf"))
    m = s.amax(-1, keepdim=True)
    m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    unnorm = torch.exp(s - m)
    total = unnorm.sum(-1, keepdim=True)
    inv = torch.where(total > 0, 1 / total.clamp_min(1e-300), torch.zeros_like(total))
    out = bf((bf(unnorm) @ vv) * inv)
    p = unnorm * inv
    dp = dout @ vv.transpose(-1, -2)
    delta = (dout * out).sum(-1, keepdim=True)
    ds = bf(p * (dp - delta))
    dq = bf(ds @ kk * scale)
    dk = bf(((ds.transpose(-1, -2) @ q) * scale).view(batch, -1, group, k.shape[2], dim).sum(2))
    dv = bf((bf(p).transpose(-1, -2) @ dout).view(batch, -1, group, k.shape[2], dim).sum(2))
    return out, dq, dk, dv
