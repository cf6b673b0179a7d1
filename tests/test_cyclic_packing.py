"""Packing cyclic document metadata into strided varlen segments (CPU).

Whenever the builder returns a schedule, the visibility it implies (segment
s: local key j visible to local query i iff j <= nk - 1 - stride *
(nq - 1 - i)) must equal the reference's per-pair rule
(ops/cyclic_attention/reference.py:20-30, restated as oracle.cyclic_keep)
exactly; metadata built by prepare_feedback_metadata /
prepare_cyclic_attention_metadata must always pack; arbitrary metadata may
be refused (None) but never packed wrongly."""

import numpy as np
import pytest
import torch

from oracle import attention as ref
from white_matter_amd import prepare_cyclic_attention_metadata, prepare_feedback_metadata
from white_matter_amd.cyclic_attention import _build_packed_schedule


def _implied_keep(schedule, batch, q_len, k_len, stride):
    keep = torch.zeros(batch, q_len, k_len, dtype=torch.bool)
    if schedule == "empty":
        return keep
    qi, ki = schedule.query_indices, schedule.key_indices
    for qs, qe, ks, ke in schedule.segments:
        nq, nk = qe - qs, ke - ks
        for li in range(nq):
            b, i = divmod(int(qi[qs + li]), q_len)
            bound = nk - 1 - stride * (nq - 1 - li)
            for lj in range(max(0, min(nk, bound + 1))):
                kb, j = divmod(int(ki[ks + lj]), k_len)
                assert kb == b, "a segment's keys stay in its query's row"
                keep[b, i, j] = True
    return keep


def _check(meta, q_len, k_len, stride, offset, must_pack):
    schedule = _build_packed_schedule(*meta, q_len, k_len, stride, offset)
    if schedule is None:
        assert not must_pack, "run-structured metadata was refused"
        return None
    batch = meta[0].shape[0]
    expected = ref.cyclic_keep(q_len, k_len, stride, offset, meta)[:, 0]
    assert torch.equal(_implied_keep(schedule, batch, q_len, k_len, stride), expected)
    if schedule != "empty":
        # every query row once, every key row at least once (dummies repeat): the
        # kernels then write all outputs and gradients themselves
        assert torch.equal(schedule.query_indices.sort().values, torch.arange(batch * q_len))
        assert torch.equal(schedule.key_indices.unique(), torch.arange(batch * k_len))
    return schedule


def _documents(rng, batch, length, mean):
    rows = []
    for _ in range(batch):
        sizes = []
        while sum(sizes) < length:
            sizes.append(int(rng.integers(1, 2 * mean)))
        sizes[-1] -= sum(sizes) - length
        rows.append(np.repeat(np.arange(len(sizes)), sizes))
    return torch.from_numpy(np.stack(rows))


@pytest.mark.parametrize("dummy", [False, True])
def test_feedback_metadata_always_packs_exactly(dummy):
    rng = np.random.default_rng(3 + dummy)
    for trial in range(24):
        batch, length = int(rng.integers(1, 4)), int(rng.integers(4, 60))
        stride = int(rng.integers(1, 6))
        docs = _documents(rng, batch, length, int(rng.integers(1, 12)))
        groups = [torch.arange(r, length, stride) for r in range(stride)]
        metas = prepare_feedback_metadata(docs, groups, length + int(dummy), use_dummy_token=dummy)
        for r in range(stride):
            q_len = groups[r].numel()
            if q_len == 0:
                continue
            # the model's calls: strict below each query's own slot without the
            # dummy, inclusive of it (the dummy shifts key slots by one) with it
            offset = r if dummy else r - 1
            _check(metas[r], q_len, length + int(dummy), stride, offset, must_pack=True)


def test_cyclic_metadata_packs_and_dummy_only_queries():
    ids = torch.tensor([[0, 0, 0, 1, 1, 2, 2, 2, 2, 3]])
    keys = torch.cat((torch.full((1, 1), -1), ids), dim=1)
    for stride in (1, 2, 3):
        for r in range(stride):
            q = ids[:, r::stride]
            meta = prepare_cyclic_attention_metadata(q, keys)
            # offset r is the model's call with a dummy; at r - 1 a query two
            # slots before its document start sees the dummy alone, which the
            # strided bound cannot express: refused (document-mode kernels)
            for offset, must_pack in ((r, True), (r - 1, False)):
                if offset + stride * (q.shape[1] - 1) < keys.shape[1]:
                    _check(meta, q.shape[1], keys.shape[1], stride, offset, must_pack=must_pack)


def test_arbitrary_metadata_is_refused_or_exact():
    rng = np.random.default_rng(11)
    packed = refused = 0
    for trial in range(150):
        batch, q_len, stride = int(rng.integers(1, 3)), int(rng.integers(1, 10)), int(rng.integers(1, 4))
        k_len = stride * q_len + int(rng.integers(0, 3))
        offset = int(rng.integers(-1, stride))
        if offset + stride * (q_len - 1) >= k_len:
            continue
        qseg = torch.from_numpy(rng.integers(-1, 3, size=(batch, q_len)))
        kseg = torch.from_numpy(rng.integers(-1, 3, size=(batch, k_len)))
        if trial % 3 == 0:  # mostly run-structured, with perturbed starts/ends
            kseg = torch.from_numpy(np.sort(rng.integers(0, 3, size=(batch, k_len)), axis=1))
            qseg = kseg[:, (offset + stride * torch.arange(q_len)).clamp_min(0)]
        qstart = torch.from_numpy(rng.integers(0, k_len, size=(batch, q_len)))
        kqend = torch.from_numpy(rng.integers(0, q_len + 2, size=(batch, k_len)))
        if _check((qseg, kseg, qstart, kqend), q_len, k_len, stride, offset, must_pack=False) is None:
            refused += 1
        else:
            packed += 1
    assert refused > 0 and packed > 0


@pytest.mark.parametrize("dummy", [False, True])
def test_fused_backward_lists_partition_the_segments(dummy):
    """The fused backward takes every segment of 1 to 128 queries and at least
    one key, heaviest first, with the segment's own work-list fields; the
    tiled dQ and dK/dV lists keep exactly their entries for the other
    segments, so each query and key tile has one owner."""
    from white_matter_amd.strict_causal_attention import _FUSED_ROWS, _fused_units, _segment_fields, _work_units

    rng = np.random.default_rng(11 + dummy)
    for trial in range(6):
        stride = int(rng.integers(1, 9))
        batch, length = 2, int(rng.integers(300, 1400))
        docs = _documents(rng, batch, length, int(rng.integers(20, 400)))
        groups = [torch.arange(r, length, stride) for r in range(stride)]
        metas = prepare_feedback_metadata(docs, groups, length + int(dummy), use_dummy_token=dummy)
        r = int(rng.integers(0, stride))
        q_len = groups[r].numel()
        offset = r if dummy else r - 1
        schedule = _check(metas[r], q_len, length + int(dummy), stride, offset, must_pack=True)
        if schedule == "empty":
            continue
        key_tile = 64 if stride >= 2 else 128
        q_units, k_units, ds_offsets, _ = _work_units(schedule, stride, query_extent=q_len, key_tile=key_tile)
        f_units, bq_units, bk_units = _fused_units(schedule, stride, q_len, key_tile)
        sizes = [(qe - qs, ke - ks) for qs, qe, ks, ke in schedule.segments]
        fused = [int(s) for s in f_units[:, 0]]
        assert sorted(fused) == [s for s, (nq, nk) in enumerate(sizes) if 1 <= nq <= _FUSED_ROWS and nk >= 1]
        tiles = [-(-sizes[s][1] // 64) for s in fused]
        assert tiles == sorted(tiles, reverse=True), "heaviest first"
        fields = _segment_fields(schedule, q_len, ds_offsets.cpu())
        expected = fields.index_select(0, torch.tensor(fused, dtype=torch.long))
        expected[:, 1] = 0
        assert torch.equal(f_units.cpu(), expected)
        for full, rest in ((q_units, bq_units), (k_units, bk_units)):
            keep = [row for row in full.tolist() if row[0] not in set(fused)]
            assert rest.tolist() == keep
