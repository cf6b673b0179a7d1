"""Strict-past attention for Jacobi passes, cached prefill and KV-pool decode.

Drop-in for ``white_matter.ops.strict_causal_attention``
(src/white_matter/ops/strict_causal_attention.py:36-474): same names,
signatures, validation messages, masking contract and output layout
(Q/K/V in (B, H, T, D), output (B, T, H, D)). On ROCm devices every
non-"reference" backend literal runs the gfx950 HIP kernels of
libwmx_attn.so:

  * packed documents (``metadata``)      -> varlen kernels, gather on load
  * int/tensor ``query_start``, ragged ``kv_lengths`` or single-query training
                                          -> dense kernels with per-row bounds
  * one query token without gradient      -> split-K decode kernel

``backend="reference"`` (and "auto" on CPU) is the reference's portable
PyTorch math path.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

import torch

from . import _kernels, _native, portable

_BACKENDS = ("auto", "reference", "torch_flash", "flash_attention_2")


def _standalone_flash_available() -> bool:
    """The reference picks "flash_attention_2" for "auto" when the flash_attn
    package is installed (strict_causal_attention.py:32-33,233-236). Here every
    non-reference literal runs the same HIP kernels, so no package is looked
    for; the FLOP counter (benchmarks/_flop_counter.py:90,98) then binds only
    the operators this package registers."""
    return False


@dataclass(frozen=True)
class StrictCausalMetadata:
    """Reusable varlen gather/scatter schedule, independent of heads and values
    (reference strict_causal_attention.py:36-72).

    Segment s holds queries ``query_indices[cu_queries[s]:cu_queries[s+1]]``
    (flat row * query_length + t) and keys ``key_indices[cu_keys[s]:cu_keys[s+1]]``
    (flat row * key_extent + slot); its local key j is visible to its local
    query i iff j <= (keys - queries) + i.
    """

    query_indices: torch.Tensor
    key_indices: torch.Tensor
    cu_queries: torch.Tensor
    cu_keys: torch.Tensor
    max_queries: int
    max_keys: int
    key_extent: int
    segments: tuple[tuple[int, int, int, int], ...] = ()

    def __post_init__(self) -> None:
        if not self.segments and self.cu_queries.numel() > 1:
            q = self.cu_queries.tolist()
            k = self.cu_keys.tolist()
            object.__setattr__(self, "segments", tuple((q[s], q[s + 1], k[s], k[s + 1]) for s in range(len(q) - 1)))

    def with_key_extent(self, key_extent: int) -> StrictCausalMetadata:
        """Address the same key slots in storage rows of width ``key_extent``."""
        if key_extent == self.key_extent:
            return self
        # one remapped schedule per storage width, so its host facts are computed once
        remapped_by_extent = self.__dict__.setdefault("_remapped", {})
        remapped = remapped_by_extent.get(key_extent)
        if remapped is None:
            row = torch.div(self.key_indices, self.key_extent, rounding_mode="floor")
            slot = self.key_indices % self.key_extent
            remapped = StrictCausalMetadata(
                self.query_indices,
                row * key_extent + slot,
                self.cu_queries,
                self.cu_keys,
                self.max_queries,
                self.max_keys,
                key_extent,
                self.segments,
            )
            remapped_by_extent[key_extent] = remapped
        return remapped


@torch.compiler.disable
def prepare_strict_causal_metadata(
    document_ids: torch.Tensor,
    query_length: int,
    *,
    query_start: int | torch.Tensor = 0,
    kv_lengths: torch.Tensor | None = None,
    use_dummy_token: bool = False,
) -> StrictCausalMetadata:
    """Pack document runs into varlen segments; negative ids are padding
    (reference strict_causal_attention.py:75-155).

    ``document_ids`` (B, extent) labels real key slots, the current query
    tokens included and the optional leading dummy excluded; query i of row b
    sits at slot query_start[b] + i. A run is a maximal sequence of present
    (id >= 0) slots with one id, padding slots in between not breaking it.
    Query at slot p sees the present slots of its run before min(p, kv_len),
    plus the dummy. Consecutive valid queries share a segment while they stay
    in one run and each sees exactly one more key than the previous one; a
    segment's keys are the visible set of its last query, dummy first.

    Integer ids on a ROCm device are scheduled by the HIP builder
    (wmx_strict_meta_count / _fill): one host synchronisation, to size the
    outputs. Elsewhere the same steps run as torch operations.
    """
    _kernels.guard_capture("prepare_strict_causal_metadata")
    if document_ids.is_cuda and not document_ids.is_floating_point() and document_ids.dtype != torch.bool:
        return _device_schedule(document_ids, query_length, query_start, kv_lengths, use_dummy_token)
    return _torch_schedule(document_ids, query_length, query_start, kv_lengths, use_dummy_token)


def _torch_schedule(
    document_ids: torch.Tensor,
    query_length: int,
    query_start: int | torch.Tensor,
    kv_lengths: torch.Tensor | None,
    use_dummy_token: bool,
) -> StrictCausalMetadata:
    """prepare_strict_causal_metadata as torch operations on the ids' device
    (the reference's formulation; synchronises at each data-dependent size)."""
    batch, extent = document_ids.shape
    device = document_ids.device
    offset = int(use_dummy_token)
    start = torch.as_tensor(query_start, device=device, dtype=torch.long).expand(batch)
    position = start[:, None] + torch.arange(query_length, device=device)
    if bool(((position < 0) | (position >= extent)).any()):
        raise ValueError("document_ids must label every query position")

    present = document_ids >= 0
    # rank[b, s]: present slots before s (width extent + 1 so rank[:, extent] is the row total)
    rank = torch.zeros(batch, extent + 1, device=device, dtype=torch.long)
    rank[:, 1:] = present.cumsum(1)
    slot = torch.arange(extent, device=device).expand(batch, extent)
    last_present = torch.where(present, slot, -1).cummax(1).values
    before = torch.full_like(last_present, -1)
    before[:, 1:] = last_present[:, :-1]
    run_begins = present & ((before < 0) | (document_ids != document_ids.gather(1, before.clamp_min(0))))
    # rank of the first slot of the run that holds (or last precedes) each slot
    run_rank = torch.where(run_begins, rank[:, :-1], 0).cummax(1).values

    first = run_rank.gather(1, position)
    reach = position if kv_lengths is None else torch.minimum(position, kv_lengths[:, None])
    visible_end = rank.gather(1, reach.clamp(0, extent))
    valid = (document_ids.gather(1, position) >= 0) & ((visible_end > first) | use_dummy_token)
    query_indices = valid.flatten().nonzero().flatten()

    # segment breaks: another row, another run, or a visible end that is not previous + 1
    q_row = torch.div(query_indices, max(query_length, 1), rounding_mode="floor")
    q_first = first.flatten()[query_indices]
    q_end = visible_end.flatten()[query_indices]
    breaks = torch.ones_like(query_indices, dtype=torch.bool)
    breaks[1:] = (q_row[1:] != q_row[:-1]) | (q_first[1:] != q_first[:-1]) | (q_end[1:] != q_end[:-1] + 1)
    seg_start = breaks.nonzero().flatten()
    cu_queries = torch.cat((seg_start, seg_start.new_full((1,), query_indices.numel())))
    key_extent = extent + offset
    if query_indices.numel() == 0:
        return StrictCausalMetadata(
            query_indices, query_indices, cu_queries.int(), cu_queries.int(), query_length, key_extent, key_extent
        )

    last = cu_queries[1:] - 1
    seg_row = q_row[last]
    seg_first = q_first[last]
    seg_keys = (q_end[last] - seg_first).clamp_min(0) + offset
    cu_keys = torch.zeros(seg_keys.numel() + 1, device=device, dtype=torch.long)
    cu_keys[1:] = seg_keys.cumsum(0)
    owner = torch.repeat_interleave(torch.arange(seg_keys.numel(), device=device), seg_keys)
    local = torch.arange(owner.numel(), device=device) - cu_keys[owner]
    # slot of the r-th present slot of a row: index into the row-major list of present slots
    present_slots = present.flatten().nonzero().flatten() % max(extent, 1)
    row_base = rank[:, extent].cumsum(0) - rank[:, extent]
    pick = (row_base[seg_row[owner]] + seg_first[owner] + local - offset).clamp_min(0)
    key_slot = present_slots[pick] + offset
    if use_dummy_token:
        key_slot = torch.where(local == 0, 0, key_slot)
    key_indices = seg_row[owner] * key_extent + key_slot
    metadata = StrictCausalMetadata(
        query_indices, key_indices, cu_queries.int(), cu_keys.int(), query_length, key_extent, key_extent
    )
    for tensor in (metadata.query_indices, metadata.key_indices, metadata.cu_queries, metadata.cu_keys):
        torch._dynamo.mark_dynamic(tensor, 0)
    return metadata


def _device_schedule(
    document_ids: torch.Tensor,
    query_length: int,
    query_start: int | torch.Tensor,
    kv_lengths: torch.Tensor | None,
    use_dummy_token: bool,
) -> StrictCausalMetadata:
    """prepare_strict_causal_metadata through the HIP builder: a count pass,
    one read of the per-row counts (validation and output sizes), a fill pass."""
    from . import _native

    batch, extent = document_ids.shape
    device = document_ids.device
    offset = int(use_dummy_token)
    key_extent = extent + offset
    ids = document_ids if document_ids.dtype in (torch.int32, torch.int64) else document_ids.long()
    if ids.stride(-1) != 1 or (batch > 1 and ids.stride(0) < extent):
        ids = ids.contiguous()
    a = _native.StrictMetaArgs()
    a.document_ids = ids.data_ptr()
    a.doc_stride = ids.stride(0) if batch > 1 else extent
    a.doc_dtype = _native.DTYPE_I32 if ids.dtype == torch.int32 else _native.DTYPE_I64
    keep = [ids]
    if isinstance(query_start, torch.Tensor):
        start = torch.as_tensor(query_start, device=device, dtype=torch.long).expand(batch).contiguous()
        keep.append(start)
        a.query_start = start.data_ptr()
    else:
        a.query_start_scalar = int(query_start)
    if kv_lengths is not None:
        kv = kv_lengths.to(device=device, dtype=torch.long).expand(batch).contiguous()
        keep.append(kv)
        a.kv_lengths = kv.data_ptr()
    a.batch, a.extent, a.query_length, a.use_dummy = batch, extent, query_length, offset
    workspace = torch.empty(max(_native.strict_meta_workspace_size(a), 16), device=device, dtype=torch.uint8)
    counts = torch.zeros(batch, 4, device=device, dtype=torch.long)
    a.workspace, a.workspace_bytes, a.counts = workspace.data_ptr(), workspace.numel(), counts.data_ptr()
    _native.strict_meta_count(a, device)
    host = counts.cpu()  # the one synchronisation: validation and output sizes
    if bool((host[:, 3] != 0).any()):
        raise ValueError("document_ids must label every query position")
    n_queries, n_segments, n_keys = (int(x) for x in host[:, :3].sum(0))
    if max(n_queries, n_keys) >= 2**31:
        raise ValueError("the schedule holds 2**31 or more queries or keys (cu_queries/cu_keys are int32)")
    if n_queries == 0:
        empty = torch.empty(0, device=device, dtype=torch.long)
        cu = torch.zeros(1, device=device, dtype=torch.int32)
        return StrictCausalMetadata(empty, empty, cu, cu, query_length, key_extent, key_extent)
    query_indices = torch.empty(n_queries, device=device, dtype=torch.long)
    key_indices = torch.empty(n_keys, device=device, dtype=torch.long)
    cu_queries = torch.empty(n_segments + 1, device=device, dtype=torch.int32)
    cu_keys = torch.empty(n_segments + 1, device=device, dtype=torch.int32)
    a.query_indices, a.key_indices = query_indices.data_ptr(), key_indices.data_ptr()
    a.cu_queries, a.cu_keys = cu_queries.data_ptr(), cu_keys.data_ptr()
    _native.strict_meta_fill(a, device)
    del keep, workspace, counts  # the stream orders the fill before any reuse of this memory
    cq, ck = torch.stack((cu_queries, cu_keys)).tolist()  # one copy for the host segment list
    segments = tuple((cq[s], cq[s + 1], ck[s], ck[s + 1]) for s in range(n_segments))
    metadata = StrictCausalMetadata(
        query_indices, key_indices, cu_queries, cu_keys, query_length, key_extent, key_extent, segments
    )
    for tensor in (metadata.query_indices, metadata.key_indices, metadata.cu_queries, metadata.cu_keys):
        torch._dynamo.mark_dynamic(tensor, 0)
    return metadata


# ---------------------------------------------------------------- schedules --
def _segment_layout(indices: torch.Tensor, cu: torch.Tensor, extent: int, skip_first: bool) -> tuple[bool, bool]:
    """(consecutive, one_row) over all segments: element e of a segment sits at
    slot first + e (from element 1 on when skip_first), and every element of a
    segment lies in the row of its first element."""
    n = indices.numel()
    if n == 0:
        return True, True
    owner = torch.repeat_interleave(torch.arange(cu.numel() - 1, device=indices.device), cu.diff().long())
    local = torch.arange(n, device=indices.device) - cu.long()[owner]
    start = indices[cu.long()[owner]]
    rows_ok = bool((torch.div(indices, extent, rounding_mode="floor") == torch.div(start, extent, rounding_mode="floor")).all())
    if skip_first:
        second = indices[(cu.long()[owner] + 1).clamp_max(n - 1)]
        expected = torch.where(local == 0, indices, second + local - 1)
    else:
        expected = start + local
    return bool((indices == expected).all()) and rows_ok, rows_ok


def _schedule_facts(metadata: StrictCausalMetadata) -> tuple[int, int, int, int, int, int, bool]:
    """Host facts the kernels need, computed once per metadata object and kept
    on it: largest segment (queries, keys), whether key rows repeat across
    segments (wmx_attn_args keys_unique: 1 none, 2 only slot 0, 0 others),
    the largest query and key index (for bounds checks), the
    segment layout bits of wmx_attn_args (consecutive / one-row slots), and
    whether query rows repeat."""
    facts = getattr(metadata, "_facts", None)
    if facts is None:
        _kernels.guard_capture("deriving the facts of a packed-document schedule")
        segments = metadata.segments
        max_q = max((qe - qs for qs, qe, _, _ in segments), default=0)
        max_k = max((ke - ks for _, _, ks, ke in segments), default=0)
        qi, ki = metadata.query_indices, metadata.key_indices
        if segments and (segments[-1][1] != qi.numel() or segments[-1][3] != ki.numel()):
            raise ValueError("metadata segments do not cover query_indices/key_indices")
        n = ki.numel()
        # 1: key rows unique; 2: only slot 0 of a batch row (a leading dummy
        # shared by the row's segments) repeats; 0: other rows repeat
        unique = 1 if n == 0 or int(torch.unique(ki).numel()) == n else 0
        if not unique:
            dummy = ki % metadata.key_extent == 0
            real = ki[~dummy]
            unique = 2 if int(torch.unique(real).numel()) == real.numel() else 0
            # code 2 keeps one part of the dummy's gradients per segment: a
            # segment holding two slot-0 keys takes the general path
            per_segment = torch.cat((dummy.new_zeros(1, dtype=torch.long), dummy.long().cumsum(0)))
            per_segment = per_segment[metadata.cu_keys.long()].diff()
            if unique == 2 and per_segment.numel() and int(per_segment.max()) > 1:
                unique = 0
        unique_q = qi.numel() == 0 or int(torch.unique(qi).numel()) == qi.numel()
        top_q = int(qi.max()) if qi.numel() else -1
        top_k = int(ki.max()) if n else -1
        if (qi.numel() and int(qi.min()) < 0) or (n and int(ki.min()) < 0):
            raise ValueError("metadata indices must be nonnegative")
        q_consecutive, q_one_row = _segment_layout(qi, metadata.cu_queries, metadata.max_queries, False)
        k_consecutive, k_one_row = _segment_layout(ki, metadata.cu_keys, metadata.key_extent, True)
        layout = (1 if q_consecutive else 0) | (2 if k_consecutive else 0) | (4 if q_one_row else 0) | (8 if k_one_row else 0)
        facts = (max_q, max_k, unique, top_q, top_k, layout, unique_q)
        object.__setattr__(metadata, "_facts", facts)
    return facts


# ------------------------------------------------------------ operators ----
# strict_packed_fwd/bwd, strict_dense_fwd/bwd and strict_decode are registered
# from C++ (libwmx_torch.so, csrc/torch_ops.cpp): their host work per call
# (operand checks, allocation, the argument block, the launches, autograd)
# runs without the Python interpreter. Their fakes are registered below; the
# packed operators' planner (_packed_plan) is the Python step they call once
# per schedule and call shape.
_native.load_ops()


_KEYS_UNIQUE = 16  # schedule_flags bits above the four segment-layout bits
_KEYS_UNIQUE_BUT_SLOT0 = 32


def _schedule_flags(metadata: StrictCausalMetadata) -> tuple[int, int, int]:
    """(max_queries, max_keys, flags) passed to the varlen operators."""
    max_q, max_k, unique, _, _, layout, _ = _schedule_facts(metadata)
    return max_q, max_k, layout | {1: _KEYS_UNIQUE, 2: _KEYS_UNIQUE_BUT_SLOT0}.get(unique, 0)


def _keys_unique_code(flags: int) -> int:
    """wmx_attn_args.keys_unique from the schedule flags."""
    return 1 if flags & _KEYS_UNIQUE else 2 if flags & _KEYS_UNIQUE_BUT_SLOT0 else 0


def _schedule_gaps(
    metadata: StrictCausalMetadata, batch: int, length: int, heads: int, key_extent: int, kv_heads: int
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Rows that no segment writes, as flat row indices of the outputs'
    storage, so the operators zero only these rows (one index_fill each)
    instead of filling whole tensors:
      - O rows of the (B*T, H*D) view of the (B, T, H, D) output,
      - dQ rows of the (B*H*T, D) view of the (B, H, T, D) gradient,
      - dK/dV rows of the (B*Hkv*N, D) view of the (B, Hkv, N, D) gradients.
    Where any key row may repeat, the fp32 accumulators are converted in
    full, which leaves no key gap; where only slot 0 repeats (keys_unique 2)
    the other rows are stored directly and their gaps are zeroed too. Cached
    on the metadata object per call shape."""
    cache = metadata.__dict__.setdefault("_gaps", {})
    key = (batch, length, heads, key_extent, kv_heads)
    gaps = cache.get(key)
    if gaps is None:
        _kernels.guard_capture("finding the rows a packed-document schedule leaves out")
        facts = _schedule_facts(metadata)
        unique_k, unique_q = facts[2], facts[6]
        device = metadata.query_indices.device
        none = torch.empty(0, dtype=torch.long, device=device)

        def missing(indices: torch.Tensor, total: int, unique: bool) -> torch.Tensor:
            if unique and indices.numel() == total:
                return none
            seen = torch.zeros(total, dtype=torch.bool, device=device)
            seen[indices] = True
            return torch.nonzero(~seen).flatten()

        def per_head(flat: torch.Tensor, extent: int, count: int) -> torch.Tensor:
            # flat b * extent + t -> (b * count + h) * extent + t for every head h
            b, t = flat // extent, flat % extent
            h = torch.arange(count, device=device)
            return ((b[:, None] * count + h[None, :]) * extent + t[:, None]).flatten()

        out_rows = missing(metadata.query_indices, batch * length, unique_q)
        key_flat = missing(metadata.key_indices, batch * key_extent, unique_k == 1) if unique_k else none
        gaps = cache[key] = (out_rows, per_head(out_rows, length, heads), per_head(key_flat, key_extent, kv_heads))
    return gaps


_TILE = 128  # rows of the kernels' query and key tiles
_STEP = 64  # rows of the tiles their loops step over


def _runs(mask: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Flat indices of the set entries of a (rows, width) mask, and the lengths
    of their runs of consecutive entries within one row."""
    width = mask.shape[1]
    at = mask.flatten().nonzero().flatten()
    if at.numel() == 0:
        return at, at
    starts = torch.ones_like(at, dtype=torch.bool)
    starts[1:] = (at[1:] != at[:-1] + 1) | (at[1:] % width == 0)
    first = starts.nonzero().flatten()
    return at, torch.diff(torch.cat((first, first.new_full((1,), at.numel()))))


def _covering_schedule(metadata: StrictCausalMetadata, batch: int, length: int, key_extent: int) -> StrictCausalMetadata:
    """The schedule the kernels run: `metadata` plus, for the rows it leaves
    out, runs of queries as segments without keys (the kernels write a zero
    output, infinite LSE and zero dQ for them) and runs of key rows as
    segments without queries (zero dK/dV), so every output row is written by
    a kernel and no fill is launched. Cached on the metadata per call shape."""
    cache = metadata.__dict__.setdefault("_covering", {})
    shape = (batch, length, key_extent)
    cover = cache.get(shape)
    if cover is None:
        _kernels.guard_capture("covering a packed-document schedule")
        device = metadata.query_indices.device
        seen_q = torch.zeros(batch * length, dtype=torch.bool, device=device)
        seen_q[metadata.query_indices] = True
        seen_k = torch.zeros(batch * key_extent, dtype=torch.bool, device=device)
        seen_k[metadata.key_indices] = True
        idle_q, q_runs = _runs(~seen_q.view(batch, length))
        idle_k, k_runs = _runs(~seen_k.view(batch, key_extent))
        if idle_q.numel() == 0 and idle_k.numel() == 0:
            cover = metadata
        else:
            nq = torch.cat((torch.diff(metadata.cu_queries.long()), q_runs, torch.zeros_like(k_runs)))
            nk = torch.cat((torch.diff(metadata.cu_keys.long()), torch.zeros_like(q_runs), k_runs))
            cover = StrictCausalMetadata(
                torch.cat((metadata.query_indices, idle_q)),
                torch.cat((metadata.key_indices, idle_k)),
                torch.cat((nq.new_zeros(1), nq.cumsum(0))).int(),
                torch.cat((nk.new_zeros(1), nk.cumsum(0))).int(),
                metadata.max_queries,
                metadata.max_keys,
                metadata.key_extent,
            )
        cache[shape] = cover
    return cover


def _work_units(
    metadata: StrictCausalMetadata, stride: int = 1, query_extent: int | None = None, key_tile: int = _TILE
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, int]:
    """The kernels' work lists and dS layout, cached on the metadata object per
    query stride, entry form and key tile: the (segment, tile) units of the
    query-tiled kernels (forward, dQ: 128 rows) and of the key-tiled kernel
    (dK/dV: `key_tile` keys, 128 or 64, wmx_attn_args key_tile), heaviest first, as int32 device tensors, and the int64
    (num_segments + 1) offsets of the segments' dS blocks (keys x queries
    rounded up to 128 elements each) with their total. A unit's cost is the
    number of 64-row tiles its loop visits (then its row count): query i of a
    segment with nq queries and nk keys sees keys 0 .. nk - 1 - stride *
    (nq - 1 - i) (bottom-right causal at stride 1); a query tile visits the
    key tiles up to its last row's bound, a key tile the query tiles from the
    one holding the first row that sees its first key.

    Without `query_extent` an entry is the (segment, tile) pair. With it (the
    query rows' storage width, query.shape[2] of the call) an entry holds
    _native.UNIT_FIELDS ints that also carry the segment's bounds, its first
    query and key rows and slots, and its dS offset (wmx_attn_args
    unit_fields): a workgroup then reads its entry alone before loading rows,
    not cu_queries, cu_keys and the index arrays one after another."""
    if key_tile not in (64, _TILE):
        raise ValueError(f"key_tile must be 64 or {_TILE}")
    by_stride = metadata.__dict__.setdefault("_units", {})
    units = by_stride.get((stride, query_extent, key_tile))
    if units is None:
        _kernels.guard_capture("building the work lists of a packed-document schedule")
        q_units, k_units, ds_blocks = [], [], []
        for s, (qs, qe, ks, ke) in enumerate(metadata.segments):
            nq, nk = qe - qs, ke - ks
            off = nk - 1 - stride * (nq - 1)  # bound of local query 0
            ds_blocks.append(nk * (-(-nq // _TILE) * _TILE))
            for t in range(0, -(-nq // _TILE)):
                rows = min(nq, (t + 1) * _TILE) - t * _TILE
                reach = min(nk, max(0, off + stride * (t * _TILE + rows - 1) + 1))
                q_units.append(((-(-reach // _STEP), rows), s, t))
            for t in range(0, -(-nk // key_tile)):
                keys = min(nk, (t + 1) * key_tile) - t * key_tile
                first = max(0, -(-(t * key_tile - off) // stride))
                steps = -(-(nq - first // _STEP * _STEP) // _STEP) if first < nq else 0
                k_units.append(((steps, keys), s, t))
        device = metadata.query_indices.device
        offsets = torch.tensor([0] + ds_blocks, dtype=torch.int64).cumsum(0)
        fields = None if query_extent is None else _segment_fields(metadata, query_extent, offsets)

        def table(entries):
            entries.sort(key=lambda e: (-e[0][0], -e[0][1], e[1], e[2]))
            if fields is None:
                flat = [v for _, seg, tile in entries for v in (seg, tile)]
                return torch.tensor(flat, dtype=torch.int32).view(-1, 2).to(device)
            seg = torch.tensor([seg for _, seg, _ in entries], dtype=torch.long)
            out = fields.index_select(0, seg)
            out[:, 1] = torch.tensor([tile for _, _, tile in entries], dtype=torch.int32)
            return out.to(device)

        units = by_stride[(stride, query_extent, key_tile)] = (
            table(q_units), table(k_units), offsets.to(device), int(offsets[-1])
        )
    return units


# Segments of at most this many queries take the fused backward
# (attn_bwd_seg.hip, which holds up to 128). A workgroup walks its segment's
# key tiles one after another, so the longest listed segment bounds the
# launch: at C3 stride 8 the limit 96 keeps the one 16-tile segment of 97-128
# queries on the tiled kernels (1.41-1.43 against 1.44-1.46 ms per pass with
# 128, 1.56 with none).
_FUSED_ROWS = 96
_FUSED_ROWS_MAX = 128  # the kernel's bound (wmx_attn_args f_units)


def _fused_units(
    metadata: StrictCausalMetadata, stride: int, query_extent: int, key_tile: int = _TILE
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The fused backward's work list and the other backward kernels' lists
    without its segments (wmx_attn_args f_units, q_units, k_units), cached on
    the metadata object like `_work_units`: every segment with 1 to
    _FUSED_ROWS queries and at least one key, heaviest first (most 64-key
    tiles, then most queries), as entries with the segment's fields; then
    `_work_units`' query-tile and key-tile entries of the other segments. The
    forward keeps `_work_units`' full query list."""
    if not 0 <= _FUSED_ROWS <= _FUSED_ROWS_MAX:
        raise ValueError(f"the fused backward holds at most {_FUSED_ROWS_MAX} queries")
    cache = metadata.__dict__.setdefault("_fused", {})
    lists = cache.get((stride, query_extent, key_tile, _FUSED_ROWS))
    if lists is None:
        _kernels.guard_capture("building the fused backward's work lists")
        q_units, k_units, ds_offsets, _ = _work_units(metadata, stride, query_extent=query_extent, key_tile=key_tile)
        fused = [
            (-(-(ke - ks) // _STEP), qe - qs, s)
            for s, (qs, qe, ks, ke) in enumerate(metadata.segments)
            if 1 <= qe - qs <= _FUSED_ROWS and ke > ks
        ]
        fused.sort(key=lambda e: (-e[0], -e[1], e[2]))
        ids = torch.tensor([s for _, _, s in fused], dtype=torch.long)
        fields = _segment_fields(metadata, query_extent, ds_offsets.cpu())
        f_units = fields.index_select(0, ids)
        f_units[:, 1] = 0
        device = metadata.query_indices.device

        def placed(rows: torch.Tensor) -> torch.Tensor:
            # an empty list keeps an allocation of its own (empty device
            # tensors share a null address, which reads as aliasing)
            if rows.shape[0] == 0:
                return torch.zeros(1, rows.shape[1], dtype=rows.dtype, device=device)[:0]
            return rows.contiguous().to(device)

        def others(units: torch.Tensor) -> torch.Tensor:
            host = units.cpu()
            return placed(host[~torch.isin(host[:, 0].long(), ids)])

        lists = cache[(stride, query_extent, key_tile, _FUSED_ROWS)] = (
            placed(f_units), others(q_units), others(k_units)
        )
    return lists


def _key_tile(metadata: StrictCausalMetadata, stride: int = 1) -> int:
    """Keys per dK/dV workgroup for a packed schedule (wmx_attn_args key_tile).
    Strided (cyclic) calls give each key tile few query tiles, so the per-unit
    setup (bounds, K/V rows, first query tiles) dominates: 64-key workgroups,
    two per CU, overlap one's setup with the other's loop (C3 strides 4 and 8:
    2-3% faster passes). Full-sequence schedules keep 128 keys per workgroup,
    whose query tiles then serve twice the keys (C2: 222 against 252 us)."""
    return 64 if stride >= 2 else _TILE


def _segment_fields(metadata: StrictCausalMetadata, query_extent: int, ds_offsets: torch.Tensor) -> torch.Tensor:
    """Per segment the int32 fields of a work-list entry (wmx_attn_args
    unit_fields, WMX_UNIT_* in wmx_attn.h): segment, tile (filled per entry),
    query start and count, key start and count, the row and the slots of
    index elements 0 and 1 of each side (slot 1 = slot 0 + 1 for a
    one-element side; zeros for an empty side), and the dS offset's halves."""
    segments = torch.tensor(metadata.segments, dtype=torch.int64).view(-1, 4)
    count = segments.shape[0]
    out = torch.zeros(count, _native.UNIT_FIELDS, dtype=torch.int64)
    out[:, 0] = torch.arange(count)
    out[:, 2], out[:, 3] = segments[:, 0], segments[:, 1] - segments[:, 0]
    out[:, 4], out[:, 5] = segments[:, 2], segments[:, 3] - segments[:, 2]
    for column, start, n, index, extent in (
        (6, out[:, 2], out[:, 3], metadata.query_indices, query_extent),
        (9, out[:, 4], out[:, 5], metadata.key_indices, metadata.key_extent),
    ):
        if index.numel():
            last = index.numel() - 1
            picked = index.index_select(0, torch.cat((start.clamp_max(last), (start + 1).clamp_max(last))).to(index.device))
            e0, e1 = picked.cpu().view(2, count)
            row = torch.div(e0, extent, rounding_mode="floor")
            slot0 = e0 - row * extent
            slot1 = torch.where(n > 1, e1 - row * extent, slot0 + 1)
            live = n > 0
            out[:, column] = torch.where(live, row, 0)
            out[:, column + 1] = torch.where(live, slot0, 0)
            out[:, column + 2] = torch.where(live, slot1, 0)
    ds = ds_offsets[:-1]
    out[:, 12], out[:, 13] = ds & 0xFFFFFFFF, ds >> 32
    if bool((out[:, :12].abs() > torch.iinfo(torch.int32).max).any()):
        raise ValueError("packed-document schedule fields exceed int32")
    return out.to(torch.int32)  # the offset's low half wraps into int32 bit for bit


def _varlen(
    query, key, query_indices, key_indices, cu_queries, cu_keys, max_q, max_k, flags, q_units=None, k_units=None,
    ds_offsets=None, ds_elements=0,
):
    return _kernels.Varlen(
        query_indices=query_indices.contiguous(),
        key_indices=key_indices.contiguous(),
        cu_queries=cu_queries.to(torch.int32).contiguous(),
        cu_keys=cu_keys.to(torch.int32).contiguous(),
        num_segments=cu_queries.numel() - 1,
        max_queries=max_q,
        max_keys=max_k,
        query_extent=query.shape[2],
        key_extent=key.shape[2],
        keys_unique=_keys_unique_code(flags),
        segment_layout=flags & 15,
        q_units=q_units,
        k_units=k_units,
        ds_offsets=ds_offsets,
        ds_elements=ds_elements,
    )


@torch.library.custom_op("white_matter::strict_varlen_fwd", mutates_args=())
def strict_varlen_fwd(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    query_indices: torch.Tensor,
    key_indices: torch.Tensor,
    cu_queries: torch.Tensor,
    cu_keys: torch.Tensor,
    max_queries: int,
    max_keys: int,
    schedule_flags: int,
    scale: float,
    out_gaps: torch.Tensor,
    dq_gaps: torch.Tensor,
    dkv_gaps: torch.Tensor,
    q_units: torch.Tensor,
    k_units: torch.Tensor,
    ds_offsets: torch.Tensor,
    ds_elements: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Packed-segment attention read straight from (B, H, T, D) storage;
    output (B, T, H, D) with zeros for the queries outside every segment
    (`out_gaps`: rows of the (B*T, H*D) view). `dq_gaps` and `dkv_gaps`
    (see _schedule_gaps) are kept for the backward; `q_units`, `k_units`,
    `ds_offsets` and `ds_elements` are the kernels' work lists and the
    backward's dS layout (see _work_units)."""
    return _varlen_forward(
        query, key, value, query_indices, key_indices, cu_queries, cu_keys, max_queries, max_keys, schedule_flags,
        scale, out_gaps, q_units, k_units,
    )


def _varlen_forward(
    query, key, value, query_indices, key_indices, cu_queries, cu_keys, max_queries, max_keys, schedule_flags, scale,
    out_gaps, q_units, k_units,
):
    q, k, v = (_kernels.operand(t) for t in (query, key, value))
    batch, heads, length, dim = q.shape
    out = torch.empty(batch, length, heads, dim, device=q.device, dtype=torch.bfloat16)
    if out_gaps.numel():
        out.view(batch * length, heads * dim).index_fill_(0, out_gaps, 0)
    lse = torch.empty(batch, heads, length, device=q.device, dtype=torch.float32)
    vis = _kernels.Visibility(
        varlen=_varlen(
            q, k, query_indices, key_indices, cu_queries, cu_keys, max_queries, max_keys, schedule_flags, q_units, k_units
        )
    )
    _kernels.forward(q, k, v, out.transpose(1, 2), lse, scale, vis)
    return out, lse


@strict_varlen_fwd.register_fake
def _(query, key, value, *args):
    batch, heads, length, dim = query.shape
    return (
        query.new_empty(batch, length, heads, dim, dtype=torch.bfloat16),
        query.new_empty(batch, heads, length, dtype=torch.float32),
    )


@torch.library.custom_op("white_matter::strict_varlen_bwd", mutates_args=())
def strict_varlen_bwd(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    out: torch.Tensor,
    lse: torch.Tensor,
    dout: torch.Tensor,
    query_indices: torch.Tensor,
    key_indices: torch.Tensor,
    cu_queries: torch.Tensor,
    cu_keys: torch.Tensor,
    max_queries: int,
    max_keys: int,
    schedule_flags: int,
    scale: float,
    dq_gaps: torch.Tensor,
    dkv_gaps: torch.Tensor,
    q_units: torch.Tensor,
    k_units: torch.Tensor,
    ds_offsets: torch.Tensor,
    ds_elements: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gradients of strict_varlen_fwd; the rows no segment writes (`dq_gaps`
    of the (B*H*T, D) view of dQ, `dkv_gaps` of the (B*Hkv*N, D) views of dK
    and dV) are zero."""
    return _varlen_backward_kernels(
        query, key, value, out, lse, dout, query_indices, key_indices, cu_queries, cu_keys, max_queries, max_keys,
        schedule_flags, scale, dq_gaps, dkv_gaps, q_units, k_units, ds_offsets, ds_elements,
    )


def _varlen_backward_kernels(
    query, key, value, out, lse, dout, query_indices, key_indices, cu_queries, cu_keys, max_queries, max_keys,
    schedule_flags, scale, dq_gaps, dkv_gaps, q_units, k_units, ds_offsets, ds_elements,
):
    q, k, v = (_kernels.operand(t) for t in (query, key, value))
    o = _kernels.operand(out.transpose(1, 2))
    g = _kernels.operand(dout.transpose(1, 2))
    dim = q.shape[3]
    dq = torch.empty(q.shape, device=q.device, dtype=torch.bfloat16)
    dk = torch.empty(k.shape, device=q.device, dtype=torch.bfloat16)
    dv = torch.empty(v.shape, device=q.device, dtype=torch.bfloat16)
    if dq_gaps.numel():
        dq.view(-1, dim).index_fill_(0, dq_gaps, 0)
    if dkv_gaps.numel():
        dk.view(-1, dim).index_fill_(0, dkv_gaps, 0)
        dv.view(-1, dim).index_fill_(0, dkv_gaps, 0)
    vis = _kernels.Visibility(
        varlen=_varlen(
            q, k, query_indices, key_indices, cu_queries, cu_keys, max_queries, max_keys, schedule_flags, q_units, k_units,
            ds_offsets, ds_elements,
        )
    )
    _kernels.backward(q, k, v, o, lse, g, dq, dk, dv, scale, vis)
    return dq, dk, dv


@strict_varlen_bwd.register_fake
def _(query, key, value, *args):
    return (
        query.new_empty(query.shape, dtype=torch.bfloat16),
        key.new_empty(key.shape, dtype=torch.bfloat16),
        value.new_empty(value.shape, dtype=torch.bfloat16),
    )


def _varlen_setup(ctx, inputs, output):
    query, key, value, qi, ki, cq, ck, ctx.max_q, ctx.max_k, ctx.flags, ctx.scale, _, dq_gaps, dkv_gaps, qu, ku, dso = inputs[:17]
    ctx.ds_elements = inputs[17]
    ctx.dtypes = (query.dtype, key.dtype, value.dtype)
    ctx.save_for_backward(query, key, value, *output, qi, ki, cq, ck, dq_gaps, dkv_gaps, qu, ku, dso)
    ctx.set_materialize_grads(False)  # the LSE output has no gradient: no zero fill for it


def _varlen_backward(ctx, dout, dlse):
    query, key, value, out, lse, qi, ki, cq, ck, dq_gaps, dkv_gaps, qu, ku, dso = ctx.saved_tensors
    if dout is None:
        dout = torch.zeros_like(out)
    dq, dk, dv = strict_varlen_bwd(
        query, key, value, out, lse, dout, qi, ki, cq, ck, ctx.max_q, ctx.max_k, ctx.flags, ctx.scale,
        dq_gaps, dkv_gaps, qu, ku, dso, ctx.ds_elements,
    )
    return (dq.to(ctx.dtypes[0]), dk.to(ctx.dtypes[1]), dv.to(ctx.dtypes[2])) + (None,) * 15


strict_varlen_fwd.register_autograd(_varlen_backward, setup_context=_varlen_setup)


# ------------------------------------------------- packed-document plans ----
@torch.library.custom_op("white_matter::_packed_plan", mutates_args=())
def _packed_plan(
    query_indices: torch.Tensor,
    key_indices: torch.Tensor,
    cu_queries: torch.Tensor,
    cu_keys: torch.Tensor,
    max_queries: int,
    max_keys: int,
    batch: int,
    length: int,
    key_slots: int,
    heads: int,
    kv_heads: int,
) -> list[torch.Tensor]:
    """The plan of a packed-document schedule for one call shape, built when
    the C++ packed operators miss their plan cache (which holds it until one
    of the schedule's tensors is freed or changed in place): a CPU int64 facts
    tensor {num_segments, max_queries, max_keys, segment_layout, keys_unique,
    ds_elements, covered, key_tile}, the covering schedule's query_indices, key_indices,
    cu_queries and cu_keys (empty when it is the schedule itself: covered 0),
    the rows no segment writes (out_gaps, dq_gaps, dkv_gaps, see
    _schedule_gaps) and the work lists q_units, k_units, ds_offsets (see
    _work_units)."""
    _kernels.guard_capture("planning a packed-document schedule")
    metadata = StrictCausalMetadata(query_indices, key_indices, cu_queries, cu_keys, max_queries, max_keys, key_slots)
    top_q, top_k = _schedule_facts(metadata)[3:5]
    if max_queries != length or top_q >= batch * length or top_k >= batch * key_slots:
        raise ValueError("metadata was prepared for other query/key shapes")
    cover = _covering_schedule(metadata, batch, length, key_slots)
    max_q, max_k, flags = _schedule_flags(cover)
    gaps = _schedule_gaps(cover, batch, length, heads, key_slots, kv_heads)
    key_tile = _key_tile(cover)
    q_units, k_units, ds_offsets, ds_elements = _work_units(cover, query_extent=length, key_tile=key_tile)
    covered = cover is not metadata
    facts = torch.tensor(
        [cover.cu_queries.numel() - 1, max_q, max_k, flags & 15, _keys_unique_code(flags), ds_elements, int(covered),
         key_tile],
        dtype=torch.int64,
    )
    device = query_indices.device

    def fresh(t: torch.Tensor) -> torch.Tensor:
        # outputs of an operator may not alias its inputs or each other
        return t.clone() if t.numel() == 0 else t

    schedule = (
        [cover.query_indices, cover.key_indices, cover.cu_queries, cover.cu_keys]
        if covered
        else [torch.empty(0, dtype=torch.int64, device=device) for _ in range(4)]
    )
    return [facts, *schedule, *(fresh(g) for g in gaps), q_units, k_units, ds_offsets]


def _fake_packed_fwd(query, key, value, *args):
    batch, heads, length, dim = query.shape
    return (
        query.new_empty(batch, length, heads, dim, dtype=torch.bfloat16),
        query.new_empty(batch, heads, length, dtype=torch.float32),
    )


def _fake_grads(query, key, value, *args):
    return (
        query.new_empty(query.shape, dtype=torch.bfloat16),
        key.new_empty(key.shape, dtype=torch.bfloat16),
        value.new_empty(value.shape, dtype=torch.bfloat16),
    )


def _fake_decode(query, *args):
    batch, heads, _, dim = query.shape
    return query.new_empty(batch, 1, heads, dim, dtype=torch.bfloat16)


def _fake_decode_out(out, query, *args):
    return None


for _name, _fake in (
    ("strict_packed_fwd", _fake_packed_fwd),
    ("strict_packed_bwd", _fake_grads),
    ("strict_dense_fwd", _fake_packed_fwd),
    ("strict_dense_bwd", _fake_grads),
    ("strict_decode", _fake_decode),
    ("strict_decode_out", _fake_decode_out),
):
    torch.library.register_fake(f"white_matter::{_name}", _fake)

# strict_packed_fwd(query, key, value, query_indices, key_indices, cu_queries,
#     cu_keys, max_queries, max_keys, scale) -> (out (B, T, H, D) bf16, lse)
#     attention over a packed-document schedule given as its own tensors
#     (StrictCausalMetadata's fields), differentiable; the plan is built inside
#     the operator, so a compiled graph holds this call and nothing data-dependent
strict_packed_fwd = torch.ops.white_matter.strict_packed_fwd
strict_packed_bwd = torch.ops.white_matter.strict_packed_bwd
# strict_dense_fwd(query, key, value, query_offset, row_offset, row_limit,
#     key_mask, keep_slot0, scale) -> (out, lse): key slot j is visible to query
#     i of row b iff j <= min(offset_b + i, limit_b), or j == 0 with keep_slot0,
#     and key_mask[b, j] when given; differentiable
strict_dense_fwd = torch.ops.white_matter.strict_dense_fwd
strict_dense_bwd = torch.ops.white_matter.strict_dense_bwd
# strict_decode(query, key, value, query_start, query_start_value, kv_lengths,
#     key_mask, use_dummy, scale, num_splits) -> (B, 1, H, D) bf16: one query
#     token per row over the KV pool (no gradient)
strict_decode = torch.ops.white_matter.strict_decode
# strict_decode_out(out, query, key, value, ...same as strict_decode) -> ():
#     the same into out (B, 1, H, D) bf16 with a unit head_dim stride
strict_decode_out = torch.ops.white_matter.strict_decode_out


# ------------------------------------------------------------ public API ----
def _zeros_linked(query, key, value, batch, length, heads, dim):
    zero = (query[..., :0, :].sum() + key[..., :0, :].sum() + value[..., :0, :].sum()).to(query.dtype)
    return query.new_zeros(batch, length, heads, dim) + zero


def _unsupported(dim: int) -> RuntimeError:
    return RuntimeError(f"the gfx950 attention kernels: this path does not support head_dim {dim} (maximum 128)")


def _hip_attention(query, key, value, query_start, kv_lengths, use_dummy_token, metadata, key_mask, scale, num_splits):
    batch, heads, length, dim = query.shape
    padded = _kernels.kernel_head_dim(dim)
    if padded is None:
        raise _unsupported(dim)
    if not scale > 0:
        raise RuntimeError(f"the gfx950 attention kernels: this path does not support softmax_scale {scale}")
    dtype = query.dtype
    q, k, v = (_kernels.pad_head_dim(t, padded) for t in (query, key, value))
    offset = int(use_dummy_token)
    differentiable = torch.is_grad_enabled() and any(t.requires_grad for t in (query, key, value))
    if metadata is None and length == 1 and not differentiable:
        tensor_start = query_start if isinstance(query_start, torch.Tensor) else None
        out = strict_decode(
            q, k, v, tensor_start, 0 if tensor_start is not None else int(query_start), kv_lengths,
            key_mask, use_dummy_token, scale, num_splits,
        )
    elif metadata is not None:
        if metadata.query_indices.numel() == 0:
            return _zeros_linked(query, key, value, batch, length, heads, dim)
        if metadata.max_queries != length:
            raise ValueError("metadata was prepared for other query/key shapes")
        out, _ = strict_packed_fwd(
            q, k, v, metadata.query_indices, metadata.key_indices, metadata.cu_queries, metadata.cu_keys,
            metadata.max_queries, metadata.max_keys, scale,
        )
    else:
        row_offset = row_limit = None
        if isinstance(query_start, torch.Tensor):
            row_offset = (query_start.to(query.device).expand(batch) + (offset - 1)).to(torch.int32)
            query_offset = 0
        else:
            query_offset = int(query_start) + offset - 1
        if kv_lengths is not None:
            row_limit = (kv_lengths.to(query.device) + (offset - 1)).to(torch.int32)
        out, _ = strict_dense_fwd(q, k, v, query_offset, row_offset, row_limit, key_mask, use_dummy_token, scale)
    return out[..., :dim].to(dtype)


def strict_causal_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    query_start: int | torch.Tensor = 0,
    kv_lengths: torch.Tensor | None = None,
    use_dummy_token: bool = False,
    metadata: StrictCausalMetadata | None = None,
    key_mask: torch.Tensor | None = None,
    softmax_scale: float | None = None,
    backend: Literal["auto", "reference", "torch_flash", "flash_attention_2"] = "auto",
    num_splits: int = 0,
    static_cache: bool = False,
) -> torch.Tensor:
    """Attend only to earlier real tokens, plus an optional leading dummy
    (reference strict_causal_attention.py:158-322).

    Q/K/V use (B,H,T,D); output uses (B,T,H,D). query_start and kv_lengths
    count real tokens, excluding the dummy slot. K/V may hold current tokens
    or unused cache capacity (even NaN); neither is read outside the
    strict-past bound. Inputs are never mutated. Rows with nothing visible
    return zero. key_mask is boolean (B,N). On ROCm devices "auto",
    "torch_flash" and "flash_attention_2" run the HIP kernels; num_splits sets
    the decode split count; static_cache is accepted for compatibility.
    """
    if backend not in _BACKENDS:
        raise ValueError(f"unsupported strict causal backend: {backend!r}")
    if type(use_dummy_token) is not bool:
        raise ValueError("use_dummy_token must be boolean")
    if any(t.ndim != 4 for t in (query, key, value)) or key.shape != value.shape:
        raise ValueError("Q/K/V require (B,H,T,D) tensors with matching K/V")
    batch, heads, length, dim = query.shape
    if key.shape[0] != batch or key.shape[-1] != dim or heads % key.shape[1]:
        raise ValueError("Q/K/V require matching batch/head_dim and divisible heads")
    if any(t.device != query.device for t in (key, value)):
        raise ValueError("Q/K/V must share a device")
    offset = int(use_dummy_token)
    if key.shape[-2] - offset < 0:
        raise ValueError("dummy-enabled K/V must contain the leading dummy slot")
    if kv_lengths is not None and (kv_lengths.shape != (batch,) or kv_lengths.dtype not in (torch.int32, torch.int64)):
        raise ValueError("kv_lengths must be integer (B,)")
    if isinstance(query_start, torch.Tensor) and (
        query_start.shape != (batch,) or query_start.dtype not in (torch.int32, torch.int64)
    ):
        raise ValueError("query_start must be an integer or integer (B,) tensor")
    if metadata is not None and key_mask is not None:
        raise ValueError("metadata and key_mask are mutually exclusive")
    if key_mask is not None and (key_mask.shape != (batch, key.shape[-2]) or key_mask.dtype != torch.bool):
        raise ValueError("key_mask must be boolean (B,N)")
    if metadata is not None:
        metadata = metadata.with_key_extent(key.shape[-2])
    scale = dim**-0.5 if softmax_scale is None else softmax_scale
    if not length or not key.shape[-2]:
        return _zeros_linked(query, key, value, batch, length, heads, dim)
    if backend == "auto":
        backend = "hip" if query.is_cuda else "reference"
    if backend == "reference":
        return portable.strict_causal_attention_portable(
            query, key, value, query_start=query_start, kv_lengths=kv_lengths, use_dummy_token=use_dummy_token,
            metadata=metadata, key_mask=key_mask, scale=scale,
        )
    if not query.is_cuda:
        raise ValueError("FlashAttention requires CUDA")
    if key_mask is not None and length != 1:
        raise ValueError("FlashAttention key_mask requires a single query; use document metadata for prefill")
    return _hip_attention(query, key, value, query_start, kv_lengths, use_dummy_token, metadata, key_mask, scale, num_splits)
