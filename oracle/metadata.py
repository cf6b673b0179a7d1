"""numpy restatements of the reference's metadata builders (test oracle).

Each function follows the reference definition step by step but is written
as explicit per-row scans, independent of the product's tensor formulation.
Inputs are numpy int arrays; outputs numpy arrays with the reference's dtypes.
"""

from __future__ import annotations

import numpy as np


def cyclic_metadata(query_ids: np.ndarray, key_ids: np.ndarray, use_dummy_token: bool = True):
    """prepare_cyclic_attention_metadata (src/white_matter/ops/cyclic_attention/metadata.py:17-56):
    start[b, i] = number of keys with id < q[b, i] (left search);
    end[b, j]   = number of queries with id <= k[b, j] (right search);
    the dummy key's end is the query count. All int32."""
    q = np.asarray(query_ids).astype(np.int32)
    k = np.asarray(key_ids).astype(np.int32)
    batch, q_len = q.shape
    start = np.zeros_like(q)
    end = np.zeros_like(k)
    for b in range(batch):
        start[b] = np.searchsorted(k[b], q[b], side="left")
        end[b] = np.searchsorted(q[b], k[b], side="right")
    if use_dummy_token:
        end[:, 0] = q_len
    return q, k, start.astype(np.int32), end.astype(np.int32)


def _runs(row: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """First token and exclusive end of the equal-id run holding each token
    (src/white_matter/modules/documents.py:24-27 boundaries)."""
    n = row.shape[0]
    first = np.zeros(n, dtype=np.int64)
    end = np.zeros(n, dtype=np.int64)
    s = 0
    while s < n:
        e = s + 1
        while e < n and row[e] == row[s]:
            e += 1
        first[s:e] = s
        end[s:e] = e
        s = e
    return first, end


def feedback_metadata(document_ids: np.ndarray, query_positions, key_length: int, use_dummy_token: bool = True):
    """prepare_feedback_metadata (src/white_matter/blocks/_execution/metadata.py:11-55)."""
    docs = np.asarray(document_ids)
    batch, length = docs.shape
    offset = int(use_dummy_token)
    groups = len(query_positions)
    ids = np.where(docs < 0, -2, docs).astype(np.int32)
    keys = np.concatenate([np.full((batch, offset), -1, np.int32), ids], axis=1)[:, :key_length]
    result = []
    for residue, slots in enumerate(query_positions):
        slots = np.asarray(slots)
        count = slots.shape[0]
        qid = np.zeros((batch, count), np.int32)
        qstart = np.zeros((batch, count), np.int32)
        kend = np.zeros((batch, length), np.int32)
        for b in range(batch):
            first, end = _runs(docs[b])
            qid[b] = ids[b, slots]
            qstart[b] = first[slots] + offset
            for t in range(length):
                # queries r + groups * i with i < count that lie before the run end
                visible = sum(1 for i in range(count) if residue + groups * i < end[t])
                kend[b, t] = visible
        kqend = np.concatenate([np.full((batch, offset), count, np.int32), kend], axis=1)[:, :key_length]
        result.append((qid, keys.copy(), qstart, kqend.astype(np.int32)))
    return tuple(result)


def strict_metadata(
    document_ids: np.ndarray,
    query_length: int,
    query_start=0,
    kv_lengths: np.ndarray | None = None,
    use_dummy_token: bool = False,
):
    """prepare_strict_causal_metadata (src/white_matter/ops/strict_causal_attention.py:75-155).

    Returns dict(query_indices int64, key_indices int64, cu_queries int32,
    cu_keys int32, max_queries, max_keys, key_extent), following the
    reference's definition with per-row scans:
      run: maximal present (id >= 0) slots with equal id, padding slots do
           not break it (strict_causal_attention.py:97-104);
      query at p: first = rank of its run's first slot, visible_end =
           present slots before min(p, kv_len) (:105-108); valid if its id is
           present and visible_end > first or a dummy exists (:109);
      segments split on run change or visible_end != previous + 1 (:110-116);
      keys of a segment: ranks [first, visible_end) of its last query, dummy
           first, as row * (extent + dummy) + slot + dummy (:128-142).
    """
    docs = np.asarray(document_ids)
    batch, extent = docs.shape
    offset = int(use_dummy_token)
    starts = np.broadcast_to(np.asarray(query_start, dtype=np.int64), (batch,))
    for b in range(batch):
        for i in range(query_length):
            p = int(starts[b]) + i
            if p < 0 or p >= extent:
                raise ValueError("document_ids must label every query position")
    key_extent = extent + offset
    records = []  # (flat query index, row, run id, first, visible_end)
    run_counter = 0
    for b in range(batch):
        present_slots = [s for s in range(extent) if docs[b, s] >= 0]
        rank_before = np.zeros(extent + 1, dtype=np.int64)
        for s in range(extent):
            rank_before[s + 1] = rank_before[s] + (docs[b, s] >= 0)
        run_of = np.full(extent, -1, dtype=np.int64)
        run_first_rank = np.zeros(extent, dtype=np.int64)
        prev_id, current_run, current_first = None, -1, 0
        for s in range(extent):
            if docs[b, s] >= 0:
                if prev_id is None or docs[b, s] != prev_id:
                    run_counter += 1
                    current_run, current_first = run_counter, int(rank_before[s])
                prev_id = docs[b, s]
            run_of[s] = current_run
            run_first_rank[s] = current_first
        for i in range(query_length):
            p = int(starts[b]) + i
            reach = p if kv_lengths is None else min(p, int(kv_lengths[b]))
            reach = min(max(reach, 0), extent)
            vend = int(rank_before[reach])
            first = int(run_first_rank[p])
            if docs[b, p] >= 0 and (vend > first or use_dummy_token):
                records.append((b * query_length + i, b, int(run_of[p]), first, vend, present_slots))
    query_indices = np.array([r[0] for r in records], dtype=np.int64)
    cu_q = []
    for n, r in enumerate(records):
        if n == 0 or r[2] != records[n - 1][2] or r[4] != records[n - 1][4] + 1:
            cu_q.append(n)
    cu_q.append(len(records))
    if not records:
        return dict(
            query_indices=query_indices,
            key_indices=query_indices.copy(),
            cu_queries=np.array([0], np.int32),
            cu_keys=np.array([0], np.int32),
            max_queries=query_length,
            max_keys=key_extent,
            key_extent=key_extent,
        )
    key_indices, cu_k = [], [0]
    for s in range(len(cu_q) - 1):
        _, row, _, first, vend, present_slots = records[cu_q[s + 1] - 1]
        if use_dummy_token:
            key_indices.append(row * key_extent)
        for rank in range(first, max(vend, first)):
            key_indices.append(row * key_extent + present_slots[rank] + offset)
        cu_k.append(len(key_indices))
    return dict(
        query_indices=query_indices,
        key_indices=np.array(key_indices, dtype=np.int64),
        cu_queries=np.array(cu_q, dtype=np.int32),
        cu_keys=np.array(cu_k, dtype=np.int32),
        max_queries=query_length,
        max_keys=key_extent,
        key_extent=key_extent,
    )


def with_key_extent(key_indices: np.ndarray, old_extent: int, new_extent: int) -> np.ndarray:
    """StrictCausalMetadata.with_key_extent (strict_causal_attention.py:57-72):
    the same (row, slot) in rows of another width."""
    key_indices = np.asarray(key_indices, dtype=np.int64)
    return (key_indices // old_extent) * new_extent + key_indices % old_extent
