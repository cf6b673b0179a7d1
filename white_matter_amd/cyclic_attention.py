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

from typing import Literal

import torch

from . import _kernels, _native, portable
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


# ------------------------------------------------------- packed schedule ----
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


# ------------------------------------------------- registered operators ----
@torch.library.custom_op("white_matter::_cyclic_schedule", mutates_args=())
def _cyclic_schedule(
    qseg: torch.Tensor, kseg: torch.Tensor, qstart: torch.Tensor, kqend: torch.Tensor,
    q_len: int, k_len: int, stride: int, offset: int,
) -> list[torch.Tensor]:
    """The kernel form of one residue call's document metadata, built when the
    C++ operators (csrc/torch_ops.cpp) miss their schedule cache: a CPU int64
    facts tensor {status, num_segments, max_queries, max_keys, segment_layout,
    keys_unique, ds_elements, key_tile} and, for status 2 (packed segments), the varlen
    tensors query_indices, key_indices, cu_queries, cu_keys and the work lists
    q_units, k_units, ds_offsets, then the fused backward's segment list and the
    backward's query-tile and key-tile lists without those segments (used when
    the call has as many query heads as KV heads). Status 1: no query sees a key; status 0: the
    metadata is not run-structured, or key rows other than the dummy slots
    repeat (the document-mode kernels evaluate the rule per pair)."""
    _kernels.guard_capture("packing cyclic document metadata")
    schedule = _build_packed_schedule(qseg, kseg, qstart, kqend, q_len, k_len, stride, offset)

    def facts(*values: int) -> torch.Tensor:
        return torch.tensor(values + (0,) * (8 - len(values)), dtype=torch.int64)

    if schedule is None:
        return [facts(0)]
    if schedule == "empty":
        return [facts(1)]
    from .strict_causal_attention import _fused_units, _key_tile, _keys_unique_code, _schedule_flags, _work_units

    max_q, max_k, flags = _schedule_flags(schedule)
    unique = _keys_unique_code(flags)
    if unique == 0:
        # key rows other than the dummy slots repeat: dK/dV would accumulate
        # every row with atomics; the document-mode kernels keep one key row
        # per slot (dummy slots alone go through small accumulators)
        return [facts(0)]
    key_tile = _key_tile(schedule, stride)
    q_units, k_units, ds_offsets, ds_elements = _work_units(schedule, stride, query_extent=q_len, key_tile=key_tile)
    f_units, bq_units, bk_units = _fused_units(schedule, stride, q_len, key_tile)
    return [
        facts(2, schedule.cu_queries.numel() - 1, max_q, max_k, flags & 15, unique, ds_elements, key_tile),
        schedule.query_indices, schedule.key_indices, schedule.cu_queries, schedule.cu_keys,
        q_units, k_units, ds_offsets, f_units, bq_units, bk_units,
    ]


# The four cyclic operators are registered from C++ (libwmx_torch.so,
# csrc/torch_ops.cpp): same names, argument names and output layouts as the
# reference's torch.library registrations; their fakes are registered here.
_native.load_ops()


def _fake_fwd(Q: torch.Tensor, *_: object, **__: object) -> tuple[torch.Tensor, torch.Tensor]:
    batch, heads, length, dim = Q.shape
    out = torch.empty((batch, length, heads, dim), dtype=Q.dtype, device=Q.device).transpose(1, 2)
    lse = torch.empty((batch, heads, length), dtype=torch.float32, device=Q.device)
    return out, lse


def _fake_bwd(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, *_: object, **__: object):
    # must match the real op exactly: contiguous tensors in Q's dtype
    return (
        torch.empty(Q.shape, dtype=Q.dtype, device=Q.device),
        torch.empty(K.shape, dtype=Q.dtype, device=Q.device),
        torch.empty(V.shape, dtype=Q.dtype, device=Q.device),
    )


for _name, _fake in (
    ("cyclic_attn_fwd", _fake_fwd),
    ("cyclic_attn_bwd", _fake_bwd),
    ("cyclic_attn_doc_fwd", _fake_fwd),
    ("cyclic_attn_doc_bwd", _fake_bwd),
):
    torch.library.register_fake(f"white_matter::{_name}", _fake)

cyclic_attn_fwd = torch.ops.white_matter.cyclic_attn_fwd
cyclic_attn_bwd = torch.ops.white_matter.cyclic_attn_bwd
cyclic_attn_doc_fwd = torch.ops.white_matter.cyclic_attn_doc_fwd
cyclic_attn_doc_bwd = torch.ops.white_matter.cyclic_attn_doc_bwd
