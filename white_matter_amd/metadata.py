"""Document metadata for cyclic attention.

Mirrors the reference's public contract:
  - ``CyclicAttentionMetadata`` and ``prepare_cyclic_attention_metadata``
    (src/white_matter/ops/cyclic_attention/metadata.py:8-56),
  - ``prepare_feedback_metadata``, the model-side builder of per-residue
    metadata (src/white_matter/blocks/_execution/metadata.py:11-55).

Outputs are int32 tensors on the input device and must be bit-identical to
the reference's. Validation messages are the reference's (callers match on
them).
"""

from __future__ import annotations

from collections.abc import Sequence
from typing import NamedTuple

import torch

_INT32_MAX = torch.iinfo(torch.int32).max


class CyclicAttentionMetadata(NamedTuple):
    """Per-row document ids of query slots and key slots, plus bounds.

    ``query_key_start[b, i]`` is the first key slot of query i's document and
    ``key_query_end[b, j]`` the exclusive end of the queries that can read key
    j. A key id of -1 marks the globally visible dummy slot.
    """

    query_document_ids: torch.Tensor
    key_document_ids: torch.Tensor
    query_key_start: torch.Tensor
    key_query_end: torch.Tensor


def _validate_ids(query_ids: torch.Tensor, key_ids: torch.Tensor, use_dummy_token: bool) -> None:
    if query_ids.ndim != 2 or key_ids.ndim != 2:
        raise ValueError("segment IDs must have shape (batch, length)")
    if query_ids.shape[0] != key_ids.shape[0] or min(query_ids.shape[0], query_ids.shape[1], key_ids.shape[1]) < 1:
        raise ValueError("segment IDs require matching nonempty batches and sequences")
    if query_ids.device != key_ids.device:
        raise ValueError("segment IDs must be on the same device")
    for ids in (query_ids, key_ids):
        if ids.dtype not in (torch.int32, torch.int64):
            raise ValueError("segment IDs must be int32 or int64")
        if ids.dtype == torch.int64 and bool((ids > _INT32_MAX).any()):
            raise ValueError(f"segment IDs must fit int32 (maximum {_INT32_MAX})")
        if bool((ids.diff(dim=1) < 0).any()):
            raise ValueError("segment IDs must be nondecreasing within each row")
    first_real = int(use_dummy_token)
    if bool((query_ids < 0).any()) or bool((key_ids[:, first_real:] < 0).any()):
        raise ValueError("only the leading key dummy may have a negative segment ID")
    if use_dummy_token and not bool((key_ids[:, 0] == -1).all()):
        raise ValueError("document attention requires a leading dummy key with segment ID -1")


def prepare_cyclic_attention_metadata(
    query_document_ids: torch.Tensor, key_document_ids: torch.Tensor, *, use_dummy_token: bool = True
) -> CyclicAttentionMetadata:
    """Bounds from sorted per-row segment ids (reference metadata.py:17-56).

    Both inputs are (batch, length) int32/int64. With ``use_dummy_token`` key
    slot 0 must be the dummy (-1); every other id is >= 0 and nondecreasing.
    ``query_key_start`` is the row-wise left search of each query id among
    the key ids, ``key_query_end`` the right search of each key id among the
    query ids (the dummy's end is the query count).
    """
    _validate_ids(query_document_ids, key_document_ids, use_dummy_token)
    queries = query_document_ids.to(torch.int32).contiguous()
    keys = key_document_ids.to(torch.int32).contiguous()
    query_key_start = torch.searchsorted(keys, queries, right=False).to(torch.int32)
    key_query_end = torch.searchsorted(queries, keys, right=True).to(torch.int32)
    if use_dummy_token:
        key_query_end[:, 0] = queries.shape[1]
    return CyclicAttentionMetadata(queries, keys, query_key_start, key_query_end)


def _run_bounds(document_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """First token and exclusive end token of the run of equal ids holding
    every token: a run is numbered by counting the id changes before it, and
    its bounds are the positions of its own start and of the next run's start
    (rows are laid end to end, each row's first token opening a run)."""
    batch, length = document_ids.shape
    change = torch.ones(batch, length, dtype=torch.bool, device=document_ids.device)
    change[:, 1:] = document_ids[:, 1:] != document_ids[:, :-1]
    flat = change.reshape(-1)
    run = flat.cumsum(0) - 1  # run number of every token, over all rows
    starts = flat.nonzero().reshape(-1)  # flat position of every run's first token
    ends = torch.cat((starts[1:], starts.new_full((1,), flat.numel())))
    row_base = (torch.arange(batch, device=document_ids.device) * length)[:, None]
    run_first = starts[run].reshape(batch, length) - row_base
    run_end = ends[run].reshape(batch, length) - row_base
    return run_first, run_end


def _slots(position: torch.Tensor, device: torch.device) -> torch.Tensor:
    slots = torch.as_tensor(position, device=device)
    if slots.ndim != 1 or slots.dtype not in (torch.int32, torch.int64):
        raise ValueError("cyclic query positions must be 1-D integer index tensors")
    return slots.long()


def prepare_feedback_metadata(
    document_ids: torch.Tensor,
    query_positions: Sequence[torch.Tensor],
    key_length: int,
    *,
    use_dummy_token: bool = True,
) -> tuple[CyclicAttentionMetadata, ...]:
    """Per-residue cyclic metadata for packed documents (reference
    blocks/_execution/metadata.py:11-55).

    Group r holds query token slots ``query_positions[r]`` (r, r+s, r+2s, ...
    in the model's schedule, s = number of groups). Keys are token slots
    shifted by the optional dummy. Negative document ids (padding) become -2
    and form their own runs. On a GPU one HIP kernel builds every group's
    metadata without synchronising with the host; on the CPU the same values
    come from run numbering and gathers.
    """
    offset = int(use_dummy_token)
    groups = len(query_positions)
    if not groups:
        raise ValueError("cyclic query groups must be nonempty")
    batch, length = document_ids.shape
    if key_length > length + offset:
        raise ValueError(f"key_length={key_length} exceeds dummy-shifted token extent {length + offset}")
    slots = [_slots(p, document_ids.device) for p in query_positions]
    if document_ids.is_cuda:
        return _device_feedback(document_ids, slots, key_length, offset)
    run_first, run_end = _run_bounds(document_ids)
    ids = document_ids.to(torch.int32).masked_fill(document_ids < 0, -2)
    key_ids = torch.cat((ids.new_full((batch, offset), -1), ids), dim=1)[:, :key_length].contiguous()
    result = []
    for residue, slot in enumerate(slots):
        count = slot.numel()
        query_ids = ids.index_select(1, slot).contiguous()
        query_key_start = (run_first.index_select(1, slot) + offset).to(torch.int32).contiguous()
        # queries r + s*i (i < count) that precede a token's run end
        behind = (run_end - residue).clamp_min(0)
        visible_until = torch.div(behind + groups - 1, groups, rounding_mode="floor").clamp_max(count).to(torch.int32)
        key_query_end = torch.cat((ids.new_full((batch, offset), count), visible_until), dim=1)[:, :key_length]
        result.append(CyclicAttentionMetadata(query_ids, key_ids, query_key_start, key_query_end.contiguous()))
    return tuple(result)


def _device_feedback(
    document_ids: torch.Tensor, slots: list[torch.Tensor], key_length: int, offset: int
) -> tuple[CyclicAttentionMetadata, ...]:
    """prepare_feedback_metadata through the HIP kernel (wmx_feedback_meta):
    every group's outputs in one launch per 64 groups, no host synchronisation."""
    from . import _native

    batch, length = document_ids.shape
    device = document_ids.device
    groups = len(slots)
    ids = document_ids if document_ids.dtype in (torch.int32, torch.int64) else document_ids.long()
    if ids.stride(-1) != 1 or (batch > 1 and ids.stride(0) < length):
        ids = ids.contiguous()
    counts = [s.numel() for s in slots]
    starts = [0]
    for c in counts:
        starts.append(starts[-1] + c)
    flat_slots = torch.cat(slots).contiguous()
    key_ids = torch.empty(batch, key_length, device=device, dtype=torch.int32)
    key_query_end = torch.empty(groups, batch, key_length, device=device, dtype=torch.int32)
    query_ids = torch.empty(batch * starts[-1], device=device, dtype=torch.int32)
    query_key_start = torch.empty_like(query_ids)
    a = _native.FeedbackMetaArgs()
    a.document_ids = ids.data_ptr()
    a.doc_stride = ids.stride(0) if batch > 1 else length
    a.doc_dtype = _native.DTYPE_I32 if ids.dtype == torch.int32 else _native.DTYPE_I64
    a.batch, a.length, a.key_length, a.groups, a.use_dummy = batch, length, key_length, groups, offset
    need = _native.feedback_meta_workspace_size(a)
    workspace = torch.empty(max(need, 16), device=device, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = workspace.data_ptr(), need
    a.key_ids = key_ids.data_ptr()
    for base in range(0, groups, _native.FEEDBACK_MAX_GROUPS):
        count = min(_native.FEEDBACK_MAX_GROUPS, groups - base)
        o0 = starts[base]
        a.group_base, a.group_count = base, count
        for g in range(count + 1):
            a.group_offsets[g] = starts[base + g] - o0
        a.slots = flat_slots.data_ptr() + 8 * o0
        a.query_ids = query_ids.data_ptr() + 4 * batch * o0
        a.query_key_start = query_key_start.data_ptr() + 4 * batch * o0
        a.key_query_end = key_query_end.data_ptr() + 4 * base * batch * key_length
        _native.feedback_meta(a, device)
    result = []
    for r, count in enumerate(counts):
        span = slice(batch * starts[r], batch * starts[r + 1])
        result.append(
            CyclicAttentionMetadata(
                query_ids[span].view(batch, count),
                key_ids,
                query_key_start[span].view(batch, count),
                key_query_end[r],
            )
        )
    return tuple(result)
