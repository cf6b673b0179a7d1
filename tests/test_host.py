"""Host-side logic of the drop-in on the CPU: metadata builders bit-exact
against the oracle, the reference's validation messages, and the portable
backend against the oracle (the reference's CPU unit tests,
tests/unit/test_ops.py, test_metadata.py, test_jacobi_flash_packing.py,
test_strict_causal_attention.py)."""

import subprocess
import sys

import numpy as np
import pytest
import torch

from oracle import attention as ref
from oracle import metadata as meta
from white_matter_amd import (
    cyclic_attention,
    prepare_cyclic_attention_metadata,
    prepare_feedback_metadata,
    prepare_strict_causal_metadata,
    strict_causal_attention,
)


def _np(t):
    return t.cpu().numpy()


# -------------------------------------------------------------- metadata ----
@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_cyclic_metadata_matches_oracle(dtype):
    rng = np.random.default_rng(0)
    for _ in range(30):
        qids = np.sort(rng.integers(0, 9, size=(3, 13)), axis=1)
        kids = np.sort(rng.integers(0, 9, size=(3, 29)), axis=1)
        kids[:, 0] = -1
        actual = prepare_cyclic_attention_metadata(torch.from_numpy(qids).to(dtype), torch.from_numpy(kids).to(dtype))
        for a, e in zip(actual, meta.cyclic_metadata(qids, kids)):
            assert a.dtype == torch.int32 and a.is_contiguous() and (_np(a) == e).all()


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_cyclic_metadata_known_answer_at_int32_max(dtype):
    maximum = torch.iinfo(torch.int32).max
    actual = prepare_cyclic_attention_metadata(
        torch.tensor([[0, maximum]], dtype=dtype), torch.tensor([[-1, 0, maximum]], dtype=dtype)
    )
    expected = ([[0, maximum]], [[-1, 0, maximum]], [[1, 2]], [[2, 1, 2]])
    for a, e in zip(actual, expected):
        torch.testing.assert_close(a, torch.tensor(e, dtype=torch.int32))


@pytest.mark.parametrize("overflow_input", ["query", "key"])
def test_cyclic_metadata_rejects_int32_overflow(overflow_input):
    query_ids = torch.tensor([[0]], dtype=torch.int64)
    key_ids = torch.tensor([[-1, 0]], dtype=torch.int64)
    ids = query_ids if overflow_input == "query" else key_ids
    ids[:, -1] = torch.iinfo(torch.int32).max + 1
    with pytest.raises(ValueError, match="segment IDs must fit int32"):
        prepare_cyclic_attention_metadata(query_ids, key_ids)


def test_validation_messages():
    q = torch.randn(1, 2, 3, 8)
    with pytest.raises(ValueError, match="CUDA BF16"):
        cyclic_attention(q, q, q, backend="tilelang")
    with pytest.raises(ValueError, match="query_offset"):
        cyclic_attention(q, q, q, query_offset=-1)
    with pytest.raises(ValueError, match="dummy"):
        prepare_cyclic_attention_metadata(torch.zeros(1, 3, dtype=torch.long), torch.zeros(1, 3, dtype=torch.long))
    with pytest.raises(ValueError, match="nondecreasing"):
        prepare_cyclic_attention_metadata(torch.tensor([[1, 0]]), torch.tensor([[-1, 0, 1]]))
    with pytest.raises(ValueError, match="requires CUDA"):
        strict_causal_attention(q, q, q, backend="torch_flash")
    with pytest.raises(ValueError, match="unsupported strict causal backend"):
        strict_causal_attention(q, q, q, backend="tilelang")
    with pytest.raises(ValueError, match="mutually exclusive"):
        md = prepare_strict_causal_metadata(torch.zeros(1, 3, dtype=torch.long), 3)
        strict_causal_attention(q, q, q, metadata=md, key_mask=torch.ones(1, 3, dtype=torch.bool))
    with pytest.raises(ValueError, match="nonempty"):
        prepare_feedback_metadata(torch.zeros(1, 8, dtype=torch.long), [], 8)
    with pytest.raises(ValueError, match="label every query position"):
        prepare_strict_causal_metadata(torch.zeros(1, 3, dtype=torch.long), 2, query_start=2)


@pytest.mark.parametrize("stride", [1, 2, 4])
@pytest.mark.parametrize("length", [17, 33])
@pytest.mark.parametrize("dummy", [False, True])
def test_feedback_metadata_matches_oracle(stride, length, dummy):
    torch.manual_seed(length)
    segments = torch.randint(0, 2, (2, length)).cumsum(1)
    segments[0] = torch.arange(length)
    segments[1, 3:6] = -1
    positions = [torch.arange(r, length, stride) for r in range(stride)]
    actual = prepare_feedback_metadata(segments, positions, length, use_dummy_token=dummy)
    expected = meta.feedback_metadata(_np(segments), [_np(p) for p in positions], length, dummy)
    for a, e in zip(actual, expected):
        for ta, te in zip(a, e):
            assert ta.dtype == torch.int32 and (_np(ta) == te).all()


def test_feedback_metadata_matches_segment_search():
    # reference tests/unit/test_metadata.py:10-23 on the product builders
    for stride in (1, 2, 4):
        for length in (17, 33):
            torch.manual_seed(length)
            segments = torch.randint(0, 2, (2, length)).cumsum(1)
            segments[0] = torch.arange(length)
            positions = [torch.arange(r, length, stride) for r in range(stride)]
            actual = prepare_feedback_metadata(segments, positions, length)
            keys = torch.cat((segments.new_full((2, 1), -1), segments[:, :-1]), dim=1)
            for slots, residue in zip(positions, range(stride)):
                expected = prepare_cyclic_attention_metadata(segments[:, slots], keys)
                torch.testing.assert_close(actual[residue], expected, rtol=0, atol=0)


def _assert_schedule_equal(actual, expected):
    for name in ("query_indices", "key_indices"):
        a = getattr(actual, name)
        assert a.dtype == torch.int64 and (_np(a) == expected[name]).all(), name
    for name in ("cu_queries", "cu_keys"):
        a = getattr(actual, name)
        assert a.dtype == torch.int32 and (_np(a) == expected[name]).all(), name
    assert actual.max_queries == expected["max_queries"]
    assert actual.max_keys == expected["max_keys"] and actual.key_extent == expected["key_extent"]
    cq, ck = expected["cu_queries"].tolist(), expected["cu_keys"].tolist()
    assert actual.segments == tuple((cq[s], cq[s + 1], ck[s], ck[s + 1]) for s in range(len(cq) - 1))


@pytest.mark.parametrize("dummy", [False, True])
def test_strict_metadata_bit_exact_random(dummy):
    rng = np.random.default_rng(5)
    for trial in range(60):
        batch, extent = int(rng.integers(1, 4)), int(rng.integers(1, 40))
        docs = np.sort(rng.integers(0, 5, size=(batch, extent)), axis=1)
        docs = np.where(rng.random((batch, extent)) < 0.15, rng.choice([-1, -2], size=(batch, extent)), docs)
        if trial % 5 == 0:
            docs = rng.integers(-2, 3, size=(batch, extent))  # unsorted ids and repeated labels
        length = int(rng.integers(1, extent + 1))
        starts = rng.integers(0, extent - length + 1, size=batch)
        kv = None if trial % 3 else rng.integers(0, extent + 2, size=batch)
        query_start = int(starts[0]) if trial % 4 == 0 else torch.from_numpy(starts)
        if trial % 4 == 0:
            starts = np.full(batch, starts[0])
        actual = prepare_strict_causal_metadata(
            torch.from_numpy(docs), length, query_start=query_start,
            kv_lengths=None if kv is None else torch.from_numpy(kv), use_dummy_token=dummy,
        )
        _assert_schedule_equal(actual, meta.strict_metadata(docs, length, starts, kv, dummy))


def test_strict_metadata_known_answers():
    documents = torch.tensor([[0, 0, 1, 1, 1, 2], [0, 1, 1, 2, 3, 3]])
    schedule = prepare_strict_causal_metadata(documents, 6, use_dummy_token=True)
    assert schedule.cu_queries.tolist() == [0, 2, 5, 6, 7, 9, 10, 12]
    empty = prepare_strict_causal_metadata(torch.empty(2, 0, dtype=torch.long), 0)
    assert empty.query_indices.numel() == empty.key_indices.numel() == 0
    assert empty.cu_queries.tolist() == empty.cu_keys.tolist() == [0]


def test_with_key_extent_closed_form():
    docs = torch.tensor([[0, 0, 1, 1], [0, 0, 0, 1]])
    schedule = prepare_strict_causal_metadata(docs, 4)
    wide = schedule.with_key_extent(9)
    assert wide.key_extent == 9
    assert (_np(wide.key_indices) == meta.with_key_extent(_np(schedule.key_indices), 4, 9)).all()
    assert schedule.with_key_extent(4) is schedule


# ------------------------------------------------------ portable backend ----
@pytest.mark.parametrize("document_masked", [False, True])
@pytest.mark.parametrize("offset", [0, 1])
def test_portable_cyclic_matches_oracle(document_masked, offset):
    # reference tests/unit/test_ops.py:31-54 (fp64, 1e-12)
    torch.manual_seed(42)
    q = torch.randn(2, 4, 5, 8, dtype=torch.float64, requires_grad=True)
    k = torch.randn(2, 2, 11, 8, dtype=torch.float64, requires_grad=True)
    v = torch.randn_like(k, requires_grad=True)
    slots = offset + 2 * torch.arange(5)
    metadata = None
    if document_masked:
        segments = torch.tensor([[0, 0, 0, 1, 1, 2, 2, 2, 3, 3, 3], [0, 1, 1, 1, 2, 2, 2, 3, 3, 3, 3]])
        metadata = prepare_cyclic_attention_metadata(segments[:, slots], torch.cat((torch.full((2, 1), -1), segments[:, :-1]), 1))
    actual = cyclic_attention(q, k, v, query_stride=2, query_offset=offset, metadata=metadata)
    expected = ref.cyclic_attention(q, k, v, query_stride=2, query_offset=offset, metadata=metadata)
    torch.testing.assert_close(actual, expected, rtol=1e-12, atol=1e-12)
    probe = torch.randn_like(actual)
    torch.testing.assert_close(
        torch.autograd.grad(actual, (q, k, v), probe), torch.autograd.grad(expected, (q, k, v), probe),
        rtol=1e-12, atol=1e-12,
    )


def test_config_c1_cpu_fp32_cyclic():
    """The C1 case: fp32 (1,4,64,64) queries over 2 KV heads of 256 keys,
    stride 4, one document; output and gradients of sum(output) within 1e-5
    relative of the float64 oracle."""
    gen = torch.Generator().manual_seed(0)
    q = torch.randn(1, 4, 64, 64, generator=gen, requires_grad=True)
    k = torch.randn(1, 2, 256, 64, generator=gen, requires_grad=True)
    v = torch.randn(1, 2, 256, 64, generator=gen, requires_grad=True)
    out = cyclic_attention(q, k, v, query_stride=4)
    grads = torch.autograd.grad(out.sum(), (q, k, v))
    leaves = [t.detach().double().requires_grad_() for t in (q, k, v)]
    expected = ref.cyclic_attention(*leaves, query_stride=4)
    ref_grads = torch.autograd.grad(expected.sum(), leaves)
    for a, e in zip((out, *grads), (expected, *ref_grads)):
        assert a.dtype == torch.float32
        assert ((a.double() - e).norm() / e.norm()).item() < 1e-5


def test_packed_jacobi_equals_cyclic_stride_one():
    # reference tests/unit/test_jacobi_flash_packing.py:9-28
    torch.manual_seed(1827)
    documents = torch.tensor([[0, 0, 1, 1, 1, 2], [0, 1, 1, 2, 3, 3]])
    query = torch.randn(2, 4, 6, 8, requires_grad=True)
    key = torch.randn(2, 2, 7, 8, requires_grad=True)
    value = torch.randn(2, 2, 7, 8, requires_grad=True)
    schedule = prepare_strict_causal_metadata(documents, 6, use_dummy_token=True)
    packed = strict_causal_attention(query, key, value, use_dummy_token=True, metadata=schedule, backend="reference")
    packed = packed.transpose(1, 2)
    metadata = prepare_feedback_metadata(documents, [torch.arange(6)], 6)[0]
    reference = cyclic_attention(query, key[..., :6, :], value[..., :6, :], query_stride=1, metadata=metadata)
    torch.testing.assert_close(packed, reference, rtol=1e-5, atol=1e-6)
    probe = torch.randn_like(reference)
    ga = torch.autograd.grad((packed * probe).sum(), (query, key, value), retain_graph=True)
    ge = torch.autograd.grad((reference * probe).sum(), (query, key, value))
    for a, e in zip(ga, ge):
        torch.testing.assert_close(a, e, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dummy", [False, True])
@pytest.mark.parametrize(("prefix", "count"), [(0, 1), (0, 7), (3, 5), (4, 1)])
@pytest.mark.parametrize("packed", [False, True])
def test_portable_strict_matches_per_query_oracle(dummy, prefix, count, packed):
    # reference tests/unit/test_strict_causal_attention.py:42-77 (CPU, fp64, 2e-6)
    torch.manual_seed(29)
    q = torch.randn(2, 4, count, 64, dtype=torch.float64, requires_grad=True)
    k = torch.randn(2, 2, prefix + count + int(dummy), 64, dtype=torch.float64, requires_grad=True)
    v = torch.randn_like(k, requires_grad=True)
    docs = None
    if packed:
        docs = torch.arange(prefix + count)[None].expand(2, -1).clone() // 3
        docs[1] = torch.arange(prefix + count) // 2
    metadata = None if docs is None else prepare_strict_causal_metadata(docs, count, query_start=prefix, use_dummy_token=dummy)
    actual = strict_causal_attention(q, k, v, query_start=prefix, use_dummy_token=dummy, metadata=metadata)
    expected = ref.per_query_strict(q, k, v, torch.full((2,), prefix), dummy, docs)
    torch.testing.assert_close(actual, expected, rtol=2e-6, atol=2e-6)
    probe = torch.randn_like(actual)
    ga = torch.autograd.grad((actual * probe).sum(), (q, k, v), retain_graph=True)
    ge = torch.autograd.grad((expected * probe).sum(), (q, k, v))
    for a, e in zip(ga, ge):
        assert torch.isfinite(a).all()
        torch.testing.assert_close(a, e, rtol=2e-6, atol=2e-6)


def test_portable_current_and_future_keys_have_zero_gradient():
    q = torch.randn(1, 2, 1, 8, requires_grad=True)
    k = torch.randn(1, 1, 7, 8, requires_grad=True)
    v = torch.randn_like(k, requires_grad=True)
    strict_causal_attention(q, k, v, query_start=3).sum().backward()
    assert k.grad[..., 3:, :].count_nonzero() == v.grad[..., 3:, :].count_nonzero() == 0


def test_portable_ragged_decode_ignores_nan_capacity():
    q = torch.randn(3, 4, 1, 16)
    k = torch.randn(3, 2, 10, 16)
    v = torch.randn_like(k)
    lengths = torch.tensor([0, 3, 7], dtype=torch.int32)
    for b, n in enumerate(lengths.tolist()):
        k[b, :, n + 1 :] = float("nan")
        v[b, :, n + 1 :] = float("nan")
    actual = strict_causal_attention(q, k, v, query_start=lengths, kv_lengths=lengths, use_dummy_token=True)
    expected = ref.per_query_strict(q, k, v, lengths, True)
    torch.testing.assert_close(actual.double(), expected, rtol=1e-5, atol=1e-5)


def test_empty_inputs_keep_gradient_linkage():
    q = torch.randn(1, 2, 0, 8, requires_grad=True)
    k = torch.randn(1, 1, 4, 8, requires_grad=True)
    out = strict_causal_attention(q, k, k)
    assert out.shape == (1, 0, 2, 8) and out.requires_grad


def test_core_import_needs_no_optional_packages():
    # reference tests/unit/test_ops.py:10-28
    code = """
import sys
from importlib.abc import MetaPathFinder
class Block(MetaPathFinder):
    def find_spec(self, fullname, *args):
        if fullname.split('.')[0] in {'transformers', 'tilelang', 'flash_attn'}:
            raise AssertionError('unexpected optional import: ' + fullname)
sys.meta_path.insert(0, Block())
from white_matter_amd import cyclic_attention, strict_causal_attention
assert callable(cyclic_attention) and callable(strict_causal_attention)
"""
    subprocess.run([sys.executable, "-c", code], check=True, cwd=str(__import__("pathlib").Path(__file__).parents[1]))


@pytest.mark.parametrize("dummy", [False, True])
def test_covering_schedule_adds_rows_not_pairs(dummy):
    """The schedule the kernels run covers every query and key row (idle query
    runs as segments without keys, idle key runs as segments without queries)
    and implies exactly the user schedule's visible pairs."""
    from white_matter_amd.strict_causal_attention import _covering_schedule

    docs = torch.tensor([[0, 0, 0, 1, 1, -1, 2, 2, 2, 2], [5, 5, 6, 6, 6, 6, 6, 7, -1, -1]])
    length, extent = 10, 10 + int(dummy)
    schedule = prepare_strict_causal_metadata(docs, length, use_dummy_token=dummy)
    cover = _covering_schedule(schedule, 2, length, extent)
    as_dict = lambda m: {k: _np(getattr(m, k)) for k in ("query_indices", "key_indices", "cu_queries", "cu_keys")} | {  # noqa: E731
        "key_extent": extent
    }
    assert torch.equal(ref.schedule_keep(as_dict(cover), 2, length, extent), ref.schedule_keep(as_dict(schedule), 2, length, extent))
    assert sorted(_np(cover.query_indices).tolist()) == list(range(2 * length))
    assert set(_np(cover.key_indices).tolist()) == set(range(2 * extent))
    assert _covering_schedule(schedule, 2, length, extent) is cover  # cached per call shape


@pytest.mark.parametrize("dummy", [False, True])
def test_work_list_entries_carry_segment_fields(dummy):
    """The work-list entries with segment fields (wmx_attn_args unit_fields
    16): each entry's segment and tile match the pair form's, and its fields
    equal what the kernels would read from cu_queries, cu_keys, the index
    arrays and ds_offsets (rows and slots of index elements 0 and 1)."""
    from white_matter_amd import prepare_strict_causal_metadata
    from white_matter_amd.strict_causal_attention import _work_units

    gen = torch.Generator().manual_seed(17 + dummy)
    length = 700
    docs = torch.cumsum(torch.rand(3, length, generator=gen) < 0.01, 1)
    md = prepare_strict_causal_metadata(docs, length, use_dummy_token=dummy)
    pairs = _work_units(md)
    full = _work_units(md, query_extent=length)
    assert full[0].shape[1] == full[1].shape[1] == 16
    for p, f in zip(pairs[:2], full[:2]):
        assert torch.equal(p, f[:, :2])
    assert torch.equal(pairs[2], full[2]) and pairs[3] == full[3]
    cq, ck = md.cu_queries.tolist(), md.cu_keys.tolist()
    qi, ki = md.query_indices.tolist(), md.key_indices.tolist()
    offsets = full[2].tolist()
    for entry in torch.cat(full[:2]).tolist():
        s = entry[0]
        qs, nq, ks, nk = cq[s], cq[s + 1] - cq[s], ck[s], ck[s + 1] - ck[s]
        assert entry[2:6] == [qs, nq, ks, nk]
        for base, start, n, index, extent in ((6, qs, nq, qi, length), (9, ks, nk, ki, md.key_extent)):
            if n:
                row, slot0 = divmod(index[start], extent)
                slot1 = index[start + 1] - row * extent if n > 1 else slot0 + 1
                assert entry[base : base + 3] == [row, slot0, slot1]
        assert (entry[12] & 0xFFFFFFFF) | (entry[13] << 32) == offsets[s]
