"""The HIP schedule builder (wmx_strict_meta_count / _fill, reached through
prepare_strict_causal_metadata with document ids on the GPU) against the
oracle, bit for bit: random schedules over several 1024-slot and 1024-query
chunks, padding and repeated labels, per-row query starts and kv lengths,
the dummy slot, the reference's known answers, the C2 schedule, and the
position check (reference ops/strict_causal_attention.py:75-155;
tests/unit/test_jacobi_flash_packing.py:15-16)."""

import numpy as np
import pytest
import torch

import bench
from oracle import metadata as meta
from white_matter_amd import prepare_strict_causal_metadata

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _assert_schedule_equal(actual, expected):
    for name in ("query_indices", "key_indices"):
        a = getattr(actual, name)
        assert a.is_cuda and a.dtype == torch.int64, name
        assert np.array_equal(a.cpu().numpy(), expected[name]), name
    for name in ("cu_queries", "cu_keys"):
        a = getattr(actual, name)
        assert a.is_cuda and a.dtype == torch.int32, name
        assert np.array_equal(a.cpu().numpy(), expected[name]), name
    assert actual.max_queries == expected["max_queries"]
    assert actual.max_keys == expected["max_keys"] and actual.key_extent == expected["key_extent"]
    cq, ck = expected["cu_queries"].tolist(), expected["cu_keys"].tolist()
    assert actual.segments == tuple((cq[s], cq[s + 1], ck[s], ck[s + 1]) for s in range(len(cq) - 1))


@pytest.mark.parametrize("dummy", [False, True])
def test_random_schedules_match_oracle(dummy):
    rng = np.random.default_rng(11 + dummy)
    for trial in range(40):
        batch = int(rng.integers(1, 5))
        extent = int(rng.integers(1, 40)) if trial % 2 else int(rng.integers(900, 2600))
        docs = np.sort(rng.integers(0, max(2, extent // 60), size=(batch, extent)), axis=1)
        docs = np.where(rng.random((batch, extent)) < 0.1, rng.choice([-1, -3], size=(batch, extent)), docs)
        if trial % 5 == 0:
            docs = rng.integers(-2, 3, size=(batch, extent))  # unsorted ids and repeated labels
        length = int(rng.integers(1, extent + 1))
        starts = rng.integers(0, extent - length + 1, size=batch)
        kv = None if trial % 3 else rng.integers(0, extent + 2, size=batch)
        query_start = int(starts[0]) if trial % 4 == 0 else torch.from_numpy(starts).to(DEV)
        if trial % 4 == 0:
            starts = np.full(batch, starts[0])
        dtype = torch.int32 if trial % 2 else torch.int64
        actual = prepare_strict_causal_metadata(
            torch.from_numpy(docs).to(DEV, dtype), length, query_start=query_start,
            kv_lengths=None if kv is None else torch.from_numpy(kv).to(DEV), use_dummy_token=dummy,
        )
        print(f"trial {trial} batch {batch} extent {extent} length {length}", flush=True)
        _assert_schedule_equal(actual, meta.strict_metadata(docs, length, starts, kv, dummy))


def test_known_answers_and_empty():
    documents = torch.tensor([[0, 0, 1, 1, 1, 2], [0, 1, 1, 2, 3, 3]], device=DEV)
    schedule = prepare_strict_causal_metadata(documents, 6, use_dummy_token=True)
    assert schedule.cu_queries.tolist() == [0, 2, 5, 6, 7, 9, 10, 12]
    empty = prepare_strict_causal_metadata(torch.empty(2, 0, dtype=torch.long, device=DEV), 0)
    assert empty.query_indices.numel() == empty.key_indices.numel() == 0
    assert empty.cu_queries.tolist() == empty.cu_keys.tolist() == [0]
    # every query is a document's first token: nothing is visible without the dummy
    firsts = prepare_strict_causal_metadata(torch.arange(6, device=DEV)[None], 6)
    assert firsts.query_indices.numel() == 0 and firsts.cu_queries.tolist() == [0]


def test_c2_schedule_matches_torch_builder_and_oracle():
    docs = bench.geometric_documents(8, 2048, 0)
    expected = meta.strict_metadata(docs.numpy(), 2048, np.zeros(8, dtype=np.int64), None, False)
    _assert_schedule_equal(prepare_strict_causal_metadata(docs.to(DEV), 2048), expected)
    on_cpu = prepare_strict_causal_metadata(docs, 2048)
    on_gpu = prepare_strict_causal_metadata(docs.to(DEV), 2048)
    for name in ("query_indices", "key_indices", "cu_queries", "cu_keys"):
        assert torch.equal(getattr(on_gpu, name).cpu(), getattr(on_cpu, name)), name


def test_expanded_and_strided_ids():
    row = torch.tensor([0, 0, 0, 1, 1, -1, 1, 2, 2, 2], device=DEV)
    wide = torch.zeros(3, 16, dtype=torch.long, device=DEV)
    wide[:, :10] = row
    for docs in (row.expand(3, 10), wide[:, :10]):
        actual = prepare_strict_causal_metadata(docs, 10, use_dummy_token=True)
        expected = meta.strict_metadata(np.tile(row.cpu().numpy(), (3, 1)), 10, np.zeros(3, dtype=np.int64), None, True)
        _assert_schedule_equal(actual, expected)


def test_rejects_positions_outside_the_ids():
    docs = torch.zeros(2, 8, dtype=torch.long, device=DEV)
    with pytest.raises(ValueError, match="document_ids must label every query position"):
        prepare_strict_causal_metadata(docs, 4, query_start=torch.tensor([0, 5], device=DEV))
    with pytest.raises(ValueError, match="document_ids must label every query position"):
        prepare_strict_causal_metadata(docs, 9)
