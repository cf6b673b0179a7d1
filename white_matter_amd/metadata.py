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


def document_start_mask(document_ids: torch.Tensor) -> torch.Tensor:
    """True at each row's first token and wherever the id changes
    (reference src/white_matter/modules/documents.py:24-27)."""
    starts = torch.ones_like(document_ids, dtype=torch.bool)
    starts[:, 1:] = document_ids[:, 1:] != document_ids[:, :-1]
    return starts


def _run_bounds(document_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """First token and exclusive end token of the equal-id run of every token."""
    batch, length = document_ids.shape
    token = torch.arange(length, device=document_ids.device).expand(batch, length)
    starts = document_start_mask(document_ids)
    run_first = torch.where(starts, token, 0).cummax(dim=1).values
    # a run ends where the next one starts (or at the row end)
    next_start = torch.full_like(token, length)
    next_start[:, :-1] = torch.where(starts[:, 1:], token[:, 1:], length)
    run_end = next_start.flip(1).cummin(dim=1).values.flip(1)
    return run_first, run_end


def prepare_feedback_metadata(
    document_ids: torch.Tensor,
    query_positions: Sequence[torch.Tensor],
    key_length: int,
    *,
    use_dummy_token: bool = True,
) -> tuple[CyclicAttentionMetadata, ...]:
    """Per-residue cyclic metadata for packed documents (reference
    blocks/_execution/metadata.py:11-55).

    Group r holds query token slots ``query_positions[r]`` = r, r+s, r+2s, ...
    (s = number of groups). Keys are token slots shifted by the optional
    dummy. Negative document ids (padding) become -2 and form their own runs.
    """
    offset = int(use_dummy_token)
    groups = len(query_positions)
    if not groups:
        raise ValueError("cyclic query groups must be nonempty")
    batch, length = document_ids.shape
    if key_length > length + offset:
        raise ValueError(f"key_length={key_length} exceeds dummy-shifted token extent {length + offset}")
    run_first, run_end = _run_bounds(document_ids)
    ids = document_ids.to(torch.int32).masked_fill(document_ids < 0, -2)
    key_ids = torch.cat((ids.new_full((batch, offset), -1), ids), dim=1)[:, :key_length].contiguous()
    result = []
    for residue, slots in enumerate(query_positions):
        count = slots.numel()
        query_ids = ids.index_select(1, slots).contiguous()
        query_key_start = (run_first.index_select(1, slots) + offset).to(torch.int32).contiguous()
        # queries r + s*i (i < count) that precede a token's run end
        visible_until = torch.div((run_end - residue).clamp_min(0) + groups - 1, groups, rounding_mode="floor")
        visible_until = visible_until.clamp_max(count).to(torch.int32)
        key_query_end = torch.cat((ids.new_full((batch, offset), count), visible_until), dim=1)[:, :key_length]
        result.append(CyclicAttentionMetadata(query_ids, key_ids, query_key_start, key_query_end.contiguous()))
    return tuple(result)
