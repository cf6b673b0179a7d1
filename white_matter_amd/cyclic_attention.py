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

Document metadata whose documents are contiguous runs of slots (what
prepare_cyclic_attention_metadata and prepare_feedback_metadata build) is
packed once per metadata, stride and residue into varlen segments, one per
(row, document): the document's queries of this residue and the keys from
the document start to its last query's slot, after the dummy slots. The
varlen kernels then visit only those keys, with the strided bound
j <= nk - 1 - stride * (nq - 1 - i). Other metadata runs the document-mode
kernels, which evaluate the rule per pair.
"""

from __future__ import annotations

import weakref
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


def _check_documents(metadata, Q, K) -> None:
    shapes = ((Q.shape[0], Q.shape[2]), (K.shape[0], K.shape[2])) * 2
    if any(tuple(t.shape) != shape or t.device != Q.device for t, shape in zip(metadata, shapes)):
        raise ValueError("document metadata shape/device does not match Q/K/V")


def _documents(metadata, Q, K) -> tuple[torch.Tensor, ...] | None:
    if metadata is None:
        return None
    _check_documents(metadata, Q, K)
    return tuple(t.to(torch.int32).contiguous() for t in metadata)


# packed schedules per metadata, keyed on the id of the query-document tensor
# (checked against a weak reference, dropped when the tensor is freed)
_PACKED: dict[int, dict] = {}


def _packed_schedule(metadata, q_len: int, k_len: int, stride: int, offset: int):
    """The varlen schedule equivalent to `metadata` at this stride and residue
    offset (StrictCausalMetadata over Q rows b * Tq + i and K rows
    b * Tk + slot), or None when the metadata is not run-structured; cached
    while the four tensors are alive and unmodified."""
    qseg = metadata[0]
    entries = _PACKED.get(id(qseg))
    if entries is None or entries["tensor"]() is not qseg:
        entries = _PACKED[id(qseg)] = {"tensor": weakref.ref(qseg)}
        weakref.finalize(qseg, _PACKED.pop, id(qseg), None)
    key = (q_len, k_len, stride, offset)
    entry = entries.get(key)
    if entry is not None:
        refs, versions, schedule = entry
        if all(r() is t for r, t in zip(refs, metadata)) and versions == tuple(t._version for t in metadata):
            return schedule
    schedule = _build_packed_schedule(*metadata, q_len, k_len, stride, offset)
    if schedule is not None and schedule != "empty":
        from .strict_causal_attention import _schedule_facts

        if _schedule_facts(schedule)[2] == 0:
            # key rows other than the dummy slot repeat: dK/dV would accumulate
            # every row with atomics; the document-mode kernels keep one key
            # row per slot (dummy slots alone go through small accumulators)
            schedule = None
    entries[key] = (tuple(weakref.ref(t) for t in metadata), tuple(t._version for t in metadata), schedule)
    return schedule


def _build_packed_schedule(qseg, kseg, qstart, kqend, q_len: int, k_len: int, stride: int, offset: int):
    """Segments of (row, document run): the run's valid queries (consecutive
    indices with one document id and start) and keys = the row's dummy slots,
    then slots [document start, last query's slot]. Exact when the metadata
    satisfies what is checked here (all on the device, one read):
      - dummy slots (id < 0) form one leading prefix of every row, of one
        length nd, and every query may see them (their query end >= Tq);
      - the query end is constant over each run of equal key ids;
      - every query id is a document (>= 0), and a query that reaches real
        keys (slot >= its start) has its slot in a run of its own id that
        begins at or before its start (so [start, slot] is one run), a start
        past the dummies, and a query end beyond itself at its slot;
      - with dummies, every valid query's slot is >= its start - 1, so the
        strided bound keeps all of them visible.
    A query is valid (sees a key) when its slot is >= 0 and either dummies
    exist or its slot reaches its start. Every other row is covered too, so
    the kernels write all of O, LSE, dQ, dK and dV themselves: runs of
    queries that see nothing form segments without keys (zero output,
    infinite LSE, zero dQ) and runs of keys that no query sees form segments
    without queries (zero dK/dV). Returns a StrictCausalMetadata, the string
    "empty" when no query sees a key, or None."""
    from .strict_causal_attention import StrictCausalMetadata, _runs

    device = qseg.device
    qseg, kseg, qstart, kqend = (t.long() for t in (qseg, kseg, qstart, kqend))
    batch = qseg.shape[0]
    i = torch.arange(q_len, device=device)
    slot = (offset + stride * i).expand(batch, q_len)
    dummy = kseg < 0
    nd = dummy.long().cumprod(1).sum(1)
    new_run = torch.ones_like(dummy)
    new_run[:, 1:] = kseg[:, 1:] != kseg[:, :-1]
    run_start = torch.where(new_run, torch.arange(k_len, device=device), 0).cummax(1).values
    at = slot.clamp(0, k_len - 1)
    sees_real = slot >= qstart
    real_ok = (
        (kseg.gather(1, at) == qseg)
        & (run_start.gather(1, at) <= qstart)
        & (qstart >= nd[:, None])
        & (kqend.gather(1, at) > i)
    )
    valid = (slot >= 0) & ((nd[:, None] > 0) | sees_real)
    checks = torch.stack(
        (
            (dummy.sum(1) == nd).all(),
            (nd == nd[:1]).all(),
            ((kqend >= q_len) | ~dummy).all(),
            ((kqend[:, 1:] == kqend[:, :-1]) | new_run[:, 1:]).all(),
            (qseg >= 0).all(),
            (~sees_real | real_ok).all(),
            (~valid | (nd[:, None] == 0) | (slot >= qstart - 1)).all(),
        )
    )
    ok, dummies = torch.stack((checks.all().long(), nd[0])).tolist()
    if not ok:
        return None
    flat = valid.flatten().nonzero().flatten()
    n = flat.numel()
    if n == 0:
        return "empty"
    row = torch.div(flat, q_len, rounding_mode="floor")
    qi = flat - row * q_len
    q_start = qstart.flatten()[flat]
    q_doc = qseg.flatten()[flat]
    breaks = torch.ones(n, dtype=torch.bool, device=device)
    breaks[1:] = (row[1:] != row[:-1]) | (q_start[1:] != q_start[:-1]) | (q_doc[1:] != q_doc[:-1]) | (qi[1:] != qi[:-1] + 1)
    starts = breaks.nonzero().flatten()
    cu_queries = torch.cat((starts, starts.new_full((1,), n)))
    last = cu_queries[1:] - 1
    first_key = q_start[last]
    seg_row = row[last]
    last_key = offset + stride * qi[last]
    real = (last_key - first_key + 1).clamp_min(0)
    keys = real + dummies
    owner = torch.repeat_interleave(torch.arange(keys.numel(), device=device), keys)
    local = torch.arange(owner.numel(), device=device) - torch.cat((keys.new_zeros(1), keys.cumsum(0)))[owner]
    key_slot = torch.where(local < dummies, local, first_key[owner] + local - dummies)
    key_indices = seg_row[owner] * k_len + key_slot

    # keys no segment holds: the complement of the dummies and [first, last] ranges
    edges = torch.zeros(batch, k_len + 1, dtype=torch.long, device=device)
    has_real = real > 0
    edges.index_put_((seg_row[has_real], first_key[has_real]), torch.ones_like(first_key[has_real]), accumulate=True)
    edges.index_put_((seg_row[has_real], last_key[has_real] + 1), -torch.ones_like(first_key[has_real]), accumulate=True)
    covered = (edges[:, :k_len].cumsum(1) > 0) | dummy

    idle_q, idle_q_runs = _runs(~valid)
    idle_k, idle_k_runs = _runs(~covered)
    nq = torch.cat((torch.diff(cu_queries), idle_q_runs, torch.zeros_like(idle_k_runs)))
    nk = torch.cat((keys, torch.zeros_like(idle_q_runs), idle_k_runs))
    cu_queries = torch.cat((nq.new_zeros(1), nq.cumsum(0)))
    cu_keys = torch.cat((nk.new_zeros(1), nk.cumsum(0)))
    return StrictCausalMetadata(
        torch.cat((flat, idle_q)), torch.cat((key_indices, idle_k)), cu_queries.int(), cu_keys.int(), q_len, k_len, k_len
    )


def _packed_visibility(schedule, q, k, stride: int, backward: bool) -> _kernels.Visibility:
    from .strict_causal_attention import _schedule_flags, _varlen, _work_units

    max_q, max_k, flags = _schedule_flags(schedule)
    units = _work_units(schedule, stride)
    varlen = _varlen(
        q, k, schedule.query_indices, schedule.key_indices, schedule.cu_queries, schedule.cu_keys, max_q, max_k, flags,
        units[0], units[1], *(units[2:] if backward else (None, 0)),
    )
    return _kernels.Visibility(query_stride=stride, varlen=varlen)


def _packed_forward(q, k, v, schedule, stride: int):
    """Forward over the packed schedule: O (B, H, Tq, D) view of (B, Tq, H, D)
    storage and LSE (+inf for queries outside every segment)."""
    from .strict_causal_attention import _schedule_gaps

    batch, heads, length, dim = q.shape
    out = torch.empty(batch, length, heads, dim, device=q.device, dtype=torch.bfloat16)
    lse = torch.empty(batch, heads, length, device=q.device, dtype=torch.float32)
    if schedule == "empty":
        return out.zero_().transpose(1, 2), lse.fill_(float("inf"))
    out_gaps, _, _ = _schedule_gaps(schedule, batch, length, heads, k.shape[2], k.shape[1])
    if out_gaps.numel():
        out.view(batch * length, heads * dim).index_fill_(0, out_gaps, 0)
        # the same query rows of every head: (B*T) row r is query r % T of batch row r // T
        unscheduled = torch.zeros(batch * length, device=q.device, dtype=torch.bool).index_fill_(0, out_gaps, True)
        lse.masked_fill_(unscheduled.view(batch, 1, length), float("inf"))
    _kernels.forward(q, k, v, out.transpose(1, 2), lse, dim**-0.5, _packed_visibility(schedule, q, k, stride, False))
    return out.transpose(1, 2), lse


def _packed_backward(q, k, v, o, lse, g, schedule, stride: int):
    from .strict_causal_attention import _schedule_gaps

    dim = q.shape[3]
    dq = torch.empty(q.shape, device=q.device, dtype=torch.bfloat16)
    dk = torch.empty(k.shape, device=q.device, dtype=torch.bfloat16)
    dv = torch.empty(v.shape, device=q.device, dtype=torch.bfloat16)
    if schedule == "empty":
        return dq.zero_(), dk.zero_(), dv.zero_()
    _, dq_gaps, dkv_gaps = _schedule_gaps(schedule, q.shape[0], q.shape[2], q.shape[1], k.shape[2], k.shape[1])
    if dq_gaps.numel():
        dq.view(-1, dim).index_fill_(0, dq_gaps, 0)
    if dkv_gaps.numel():
        dk.view(-1, dim).index_fill_(0, dkv_gaps, 0)
        dv.view(-1, dim).index_fill_(0, dkv_gaps, 0)
    _kernels.backward(q, k, v, o, lse, g, dq, dk, dv, dim**-0.5, _packed_visibility(schedule, q, k, stride, True))
    return dq, dk, dv


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
    schedule = None
    if metadata is not None:
        _check_documents(metadata, Q, K)
        schedule = _packed_schedule(metadata, length, K.shape[2], K_stride, residue)
    if schedule is not None:
        out, lse = _packed_forward(q, k, v, schedule, K_stride)
    else:
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
    schedule = None
    if metadata is not None:
        _check_documents(metadata, Q, K)
        schedule = _packed_schedule(metadata, Q.shape[2], K.shape[2], K_stride, residue)
    if schedule is not None:
        grads = _packed_backward(q, k, v, o, Lse.contiguous(), g, schedule, K_stride)
    else:
        grads = tuple(torch.empty(t.shape, device=Q.device, dtype=torch.bfloat16) for t in (Q, K, V))
        vis = _kernels.Visibility(query_stride=K_stride, query_offset=residue, documents=_documents(metadata, Q, K))
        _kernels.backward(q, k, v, o, Lse.contiguous(), g, *grads, Q.shape[-1] ** -0.5, vis)
    return tuple(t.to(Q.dtype) if Q.dtype != torch.bfloat16 else t for t in grads)


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
