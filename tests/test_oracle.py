"""Pin the oracle: known answers from the reference's tests, brute force on tiny
inputs, the reference's own math-SDPA call, and invariants. Each check is
chosen so that a plausible slip in the oracle (a dropped rule, an off-by-one
bound, a wrong search side) fails it; test_planted_mistakes_are_caught plants
such slips in copies of the oracle and shows they are caught."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from oracle import attention as ref
from oracle import metadata as meta


# ------------------------------------------------------------- metadata ----
def test_cyclic_metadata_known_answer_at_int32_max():
    # reference tests/unit/test_ops.py:77-86
    m = 2**31 - 1
    q, k, start, end = meta.cyclic_metadata(np.array([[0, m]]), np.array([[-1, 0, m]]))
    assert q.tolist() == [[0, m]] and k.tolist() == [[-1, 0, m]]
    assert start.tolist() == [[1, 2]] and end.tolist() == [[2, 1, 2]]
    assert start.dtype == end.dtype == np.int32


@pytest.mark.parametrize("dummy", [False, True])
def test_cyclic_metadata_brute_force(dummy):
    rng = np.random.default_rng(3)
    for _ in range(20):
        qids = np.sort(rng.integers(0, 6, size=(2, 7)), axis=1)
        kids = np.sort(rng.integers(0, 6, size=(2, 11)), axis=1)
        if dummy:
            kids[:, 0] = -1
        _, _, start, end = meta.cyclic_metadata(qids, kids, dummy)
        for b in range(2):
            for i in range(7):
                assert start[b, i] == sum(1 for j in range(11) if kids[b, j] < qids[b, i])
            for j in range(11):
                expected = 7 if (dummy and j == 0) else sum(1 for i in range(7) if qids[b, i] <= kids[b, j])
                assert end[b, j] == expected


@pytest.mark.parametrize("stride", [1, 2, 4])
@pytest.mark.parametrize("length", [17, 33])
def test_feedback_metadata_equals_segment_search(stride, length):
    # reference tests/unit/test_metadata.py:10-23
    rng = np.random.default_rng(length)
    segments = rng.integers(0, 2, size=(2, length)).cumsum(1)
    segments[0] = np.arange(length)
    positions = [np.arange(r, length, stride) for r in range(stride)]
    actual = meta.feedback_metadata(segments, positions, length)
    keys = np.concatenate([np.full((2, 1), -1), segments[:, :-1]], axis=1)
    for r, slots in enumerate(positions):
        expected = meta.cyclic_metadata(segments[:, slots], keys)
        for a, e in zip(actual[r], expected):
            assert a.dtype == np.int32 and (a == e).all()


def test_feedback_metadata_padding_runs():
    docs = np.array([[0, 0, -1, -1, 1, 1, 1, -1]])
    qid, kid, qstart, kend = meta.feedback_metadata(docs, [np.arange(0, 8, 2), np.arange(1, 8, 2)], 9)[0]
    assert kid.tolist() == [[-1, 0, 0, -2, -2, 1, 1, 1, -2]]
    assert qid.tolist() == [[0, -2, 1, 1]]
    # run starts 0, 2, 4, 4 shifted by the dummy
    assert qstart.tolist() == [[1, 3, 5, 5]]
    # group 0 holds tokens 0,2,4,6: tokens of run [4,7) end at 7 -> 4 queries before it
    assert kend.tolist() == [[4, 1, 1, 2, 2, 4, 4, 4, 4]]


def test_strict_metadata_known_answers():
    # reference tests/unit/test_jacobi_flash_packing.py:15-16
    docs = np.array([[0, 0, 1, 1, 1, 2], [0, 1, 1, 2, 3, 3]])
    out = meta.strict_metadata(docs, 6, use_dummy_token=True)
    assert out["cu_queries"].tolist() == [0, 2, 5, 6, 7, 9, 10, 12]
    # reference tests/unit/test_strict_causal_attention.py:177-180
    empty = meta.strict_metadata(np.zeros((2, 0), dtype=np.int64), 0)
    assert empty["query_indices"].size == empty["key_indices"].size == 0
    assert empty["cu_queries"].tolist() == empty["cu_keys"].tolist() == [0]


def test_strict_metadata_hand_worked_example():
    # one row, docs [5,5,-1,5,7,7], no dummy, queries at slots 0..5:
    # runs (present ranks): {5: ranks 0,1,2 at slots 0,1,3}, {7: ranks 3,4 at slots 4,5}
    docs = np.array([[5, 5, -1, 5, 7, 7]])
    out = meta.strict_metadata(docs, 6)
    # valid: slot 1 (sees slot 0), slot 3 (sees 0,1), slot 5 (sees 4); slots 0 and 4 see nothing, 2 is padding
    assert out["query_indices"].tolist() == [1, 3, 5]
    # slot 1 ends at rank 1, slot 3 at rank 2 (consecutive) -> one segment; slot 5 another run
    assert out["cu_queries"].tolist() == [0, 2, 3]
    assert out["key_indices"].tolist() == [0, 1, 4]
    assert out["cu_keys"].tolist() == [0, 2, 3]
    dummy = meta.strict_metadata(docs, 6, use_dummy_token=True)
    # with a dummy every present slot is a query; the dummy key is slot 0 of the 7-wide row
    assert dummy["query_indices"].tolist() == [0, 1, 3, 4, 5]
    assert dummy["cu_queries"].tolist() == [0, 3, 5]
    assert dummy["key_indices"].tolist() == [0, 1, 2, 0, 5]
    assert dummy["cu_keys"].tolist() == [0, 3, 5]


def _query_run_and_end(docs, b, pos, kv_lengths):
    """For the query at slot `pos` of row b: its run (the slot where walking back
    over padding and its own id stops: one value per run, padding inside a run
    not breaking it) and its visible end (present slots before min(pos, kv_len)),
    the two quantities that decide segment membership."""
    first = pos
    while first and (docs[b, first - 1] < 0 or docs[b, first - 1] == docs[b, pos]):
        first -= 1
    cap = pos if kv_lengths is None else min(pos, int(kv_lengths[b]))
    return (b, first), int((docs[b, :cap] >= 0).sum())


def _schedule_invariants(out, docs, query_length, starts, kv_lengths, dummy):
    qi, ki = out["query_indices"], out["key_indices"]
    cq, ck = out["cu_queries"], out["cu_keys"]
    extent = docs.shape[1]
    assert cq[0] == 0 and ck[0] == 0 and cq[-1] == qi.size and ck[-1] == ki.size
    assert (np.diff(cq) > 0).all() and (np.diff(ck) >= 0).all()
    assert (np.diff(qi) > 0).all()
    facts = []
    for i in qi:
        b, t = divmod(int(i), query_length)
        facts.append(_query_run_and_end(docs, b, int(starts[b]) + t, kv_lengths))
    for s in range(len(cq) - 1):
        # inside a segment consecutive queries share a run and see one more key each
        for a in range(int(cq[s]), int(cq[s + 1]) - 1):
            assert facts[a + 1][0] == facts[a][0], "a segment spans two runs"
            assert facts[a + 1][1] == facts[a][1] + 1, "visible ends inside a segment are not +1 apart"
        # segments are maximal: the next segment's first query could not have joined this one
        if s + 2 < len(cq):
            last, nxt = facts[int(cq[s + 1]) - 1], facts[int(cq[s + 1])]
            assert not (nxt[0] == last[0] and nxt[1] == last[1] + 1), "segment is not maximal"
    for s in range(len(cq) - 1):
        rows = {int(i) // query_length for i in qi[cq[s] : cq[s + 1]]}
        assert len(rows) == 1
        (b,) = rows
        keys = ki[ck[s] : ck[s + 1]]
        assert (keys // (extent + int(dummy)) == b).all()
        last = int(qi[cq[s + 1] - 1]) % query_length
        pos = int(starts[b]) + last
        # the segment's keys are exactly the visible set of its last query
        visible = [t for t in range(min(pos, extent if kv_lengths is None else int(kv_lengths[b]))) if docs[b, t] >= 0]
        first = pos
        while first and (docs[b, first - 1] < 0 or docs[b, first - 1] == docs[b, pos]):
            first -= 1
        visible = [t + int(dummy) for t in visible if t >= first]
        expected = ([0] if dummy else []) + visible
        assert [int(x) % (extent + int(dummy)) for x in keys] == expected


@pytest.mark.parametrize("dummy", [False, True])
def test_strict_metadata_invariants_random(dummy):
    rng = np.random.default_rng(11)
    for trial in range(40):
        batch, extent = 2, int(rng.integers(4, 24))
        docs = np.sort(rng.integers(0, 4, size=(batch, extent)), axis=1)
        pad = rng.random((batch, extent)) < 0.2
        docs = np.where(pad, rng.choice([-1, -2], size=(batch, extent)), docs)
        length = int(rng.integers(1, extent + 1))
        starts = rng.integers(0, extent - length + 1, size=batch)
        kv = None if trial % 3 else rng.integers(0, extent + 1, size=batch)
        out = meta.strict_metadata(docs, length, starts, kv, dummy)
        _schedule_invariants(out, docs, length, starts, kv, dummy)


def test_planted_over_split_fails_invariants():
    """A schedule with one segment cut in two (each part keyed by its last
    query's visible set) implies the same attention, so only maximality and
    the +1 rule catch it; both fail it."""
    docs = np.array([[0, 0, 0, 0, 0, 0, 1, 1]])
    starts = np.array([0])
    good = meta.strict_metadata(docs, 8, starts, None, False)
    _schedule_invariants(good, docs, 8, starts, None, False)
    assert good["cu_queries"].tolist() == [0, 5, 6]  # queries 1..5 of document 0, then query 7
    qi, ki, cq = good["query_indices"], good["key_indices"], good["cu_queries"]
    # split segment 0 after its second query: part one ends at query 2 (keys 0, 1)
    bad = dict(good)
    bad["cu_queries"] = np.array([0, 2, 5, 6], dtype=np.int32)
    bad["key_indices"] = np.concatenate((ki[:2], ki))
    bad["cu_keys"] = np.array([0, 2, 2 + good["cu_keys"][1], 2 + good["cu_keys"][2]], dtype=np.int32)
    q = torch.randn(1, 2, 8, 8, dtype=torch.float64)
    k = torch.randn(1, 2, 8, 8, dtype=torch.float64)
    v = torch.randn_like(k)
    same = ref.strict_attention(q, k, v, metadata=bad)
    torch.testing.assert_close(same, ref.strict_attention(q, k, v, metadata=good), rtol=1e-12, atol=1e-12)
    with pytest.raises(AssertionError, match="not maximal"):
        _schedule_invariants(bad, docs, 8, starts, None, False)
    # a merge across the document boundary breaks the run rule instead
    merged = dict(good)
    merged["cu_queries"] = np.array([0, 6], dtype=np.int32)
    merged["key_indices"] = ki[good["cu_keys"][1] :]
    merged["cu_keys"] = np.array([0, merged["key_indices"].size], dtype=np.int32)
    with pytest.raises(AssertionError, match="two runs"):
        _schedule_invariants(merged, docs, 8, starts, None, False)
    assert qi.tolist() == [1, 2, 3, 4, 5, 7]


def test_with_key_extent_closed_form():
    idx = np.array([0, 5, 9, 10, 17])
    assert meta.with_key_extent(idx, 9, 12).tolist() == [0, 5, 12, 13, 20 + 0]


# ------------------------------------------------------------ attention ----
def _math_sdpa(q, k, v, keep, scale):
    with sdpa_kernel([SDPBackend.MATH]):
        return F.scaled_dot_product_attention(q, k, v, attn_mask=keep, scale=scale, enable_gqa=True)


@pytest.mark.parametrize("offset", [0, 1, -1])
@pytest.mark.parametrize("documents", [False, True])
def test_cyclic_oracle_matches_reference_sdpa_call(offset, documents):
    # reference.py:32-42 is math SDPA under the dense mask; rows that see nothing are 0
    torch.manual_seed(42)
    q = torch.randn(2, 4, 5, 8, dtype=torch.float64, requires_grad=True)
    k = torch.randn(2, 2, 11, 8, dtype=torch.float64, requires_grad=True)
    v = torch.randn_like(k, requires_grad=True)
    metadata = None
    if documents:
        segments = np.array([[0, 0, 0, 1, 1, 2, 2, 2, 3, 3, 3], [0, 1, 1, 1, 2, 2, 2, 3, 3, 3, 3]])
        slots = max(offset, 0) + 2 * np.arange(5)
        kseg = np.concatenate([np.full((2, 1), -1), segments[:, :-1]], axis=1)
        metadata = tuple(torch.from_numpy(t) for t in meta.cyclic_metadata(segments[:, slots], kseg))
    out = ref.cyclic_attention(q, k, v, query_stride=2, query_offset=offset, metadata=metadata)
    keep = ref.cyclic_keep(5, 11, 2, offset, metadata)
    expected = _math_sdpa(q, k, v, keep, 8**-0.5)
    torch.testing.assert_close(out, expected, rtol=1e-12, atol=1e-12)
    probe = torch.randn_like(out)
    ga = torch.autograd.grad(out, (q, k, v), probe)
    ge = torch.autograd.grad(expected, (q, k, v), probe)
    torch.testing.assert_close(ga, ge, rtol=1e-12, atol=1e-12)


def test_cyclic_oracle_matches_explicit_softmax_formula():
    # reference tests/unit/test_ops.py:31-54 (explicit masked softmax, fp64, 1e-12)
    torch.manual_seed(42)
    q = torch.randn(2, 4, 5, 8, dtype=torch.float64)
    k = torch.randn(2, 2, 11, 8, dtype=torch.float64)
    v = torch.randn_like(k)
    slots = 1 + 2 * torch.arange(5)
    keep = (slots[:, None] >= torch.arange(11)[None, :]).expand(2, 5, 11)
    scores = q @ k.repeat_interleave(2, dim=1).transpose(-1, -2) / 8**0.5
    expected = scores.masked_fill(~keep[:, None], -torch.inf).softmax(-1) @ v.repeat_interleave(2, dim=1)
    out = ref.cyclic_attention(q, k, v, query_stride=2, query_offset=1)
    torch.testing.assert_close(out, expected, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("dummy", [False, True])
@pytest.mark.parametrize(("prefix", "count"), [(0, 1), (0, 7), (3, 5), (4, 1)])
@pytest.mark.parametrize("packed", [False, True])
def test_strict_oracle_through_schedule_matches_per_query_loop(dummy, prefix, count, packed):
    # reference tests/unit/test_strict_causal_attention.py:42-77 (CPU, fp64)
    torch.manual_seed(29)
    q = torch.randn(2, 4, count, 16, dtype=torch.float64, requires_grad=True)
    k = torch.randn(2, 2, prefix + count + int(dummy), 16, dtype=torch.float64, requires_grad=True)
    v = torch.randn_like(k, requires_grad=True)
    docs = None
    if packed:
        docs = np.stack([np.arange(prefix + count) // 3, np.arange(prefix + count) // 2])
        schedule = meta.strict_metadata(docs, count, prefix, None, dummy)
        schedule["key_extent"] = k.shape[2]
        schedule["key_indices"] = meta.with_key_extent(schedule["key_indices"], docs.shape[1] + int(dummy), k.shape[2])
        out = ref.strict_attention(q, k, v, use_dummy_token=dummy, metadata=schedule)
    else:
        out = ref.strict_attention(q, k, v, query_start=prefix, use_dummy_token=dummy)
    expected = ref.per_query_strict(q, k, v, torch.full((2,), prefix), dummy, None if docs is None else torch.from_numpy(docs))
    torch.testing.assert_close(out, expected, rtol=1e-12, atol=1e-12)
    probe = torch.randn_like(out)
    ga = torch.autograd.grad(out, (q, k, v), probe)
    ge = torch.autograd.grad(expected, (q, k, v), probe)
    torch.testing.assert_close(ga, ge, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("dummy", [False, True])
def test_strict_oracle_padding_and_ragged_schedules(dummy):
    # reference tests/unit/test_strict_causal_attention.py:97-106 and 143-156
    torch.manual_seed(5)
    for docs, starts, length in (
        (np.array([[0, 0, 1, -1, -1, -1, -1], [0, 0, 0, 0, 1, 1, -1]]), np.array([0, 3]), 4),
        (np.array([[0, 0, -2, -2, 0, 0, -2, 0], [0, -2, 1, -2, 1, 0, 0, -2]]), np.array([4, 4]), 4),
    ):
        q = torch.randn(2, 4, length, 8, dtype=torch.float64)
        k = torch.randn(2, 2, docs.shape[1] + int(dummy), 8, dtype=torch.float64)
        v = torch.randn_like(k)
        schedule = meta.strict_metadata(docs, length, starts, None, dummy)
        out = ref.strict_attention(q, k, v, use_dummy_token=dummy, metadata=schedule)
        expected = ref.per_query_strict(q, k, v, torch.from_numpy(starts), dummy, torch.from_numpy(docs))
        torch.testing.assert_close(out, expected, rtol=1e-12, atol=1e-12)


def test_strict_dense_oracle_matches_reference_sdpa_with_lengths_and_mask():
    torch.manual_seed(9)
    q = torch.randn(3, 4, 1, 8, dtype=torch.float64)
    k = torch.randn(3, 2, 11, 8, dtype=torch.float64)
    v = torch.randn_like(k)
    lengths = torch.tensor([0, 6, 9])
    mask = torch.tensor([[False] * 11, [True, False] * 5 + [True], [True] * 11])
    for dummy in (False, True):
        keep = ref.strict_keep(3, 1, 11, lengths + 1, lengths, dummy, mask)
        out = ref.strict_attention(q, k, v, query_start=lengths + 1, kv_lengths=lengths, use_dummy_token=dummy, key_mask=mask)
        expected = _math_sdpa(q, k, v, keep[:, None], 8**-0.5).transpose(1, 2)
        torch.testing.assert_close(out, expected, rtol=1e-12, atol=1e-12)
        # the per-query loop agrees where it applies (no key_mask)
        out2 = ref.strict_attention(q, k, v, query_start=lengths + 1, kv_lengths=lengths, use_dummy_token=dummy)
        torch.testing.assert_close(out2, ref.per_query_strict(q, k, v, lengths + 1, dummy, lengths=lengths), rtol=1e-12, atol=1e-12)


def test_nan_in_unread_capacity_never_leaks():
    # reference tests/unit/test_strict_causal_attention.py:80-94
    q = torch.randn(3, 4, 1, 8, dtype=torch.float64)
    k = torch.randn(3, 2, 10, 8, dtype=torch.float64)
    v = torch.randn_like(k)
    lengths = torch.tensor([0, 3, 7])
    for b, n in enumerate(lengths.tolist()):
        k[b, :, n + 1 :] = float("nan")
        v[b, :, n + 1 :] = float("nan")
    out = ref.strict_attention(q, k, v, query_start=lengths, kv_lengths=lengths, use_dummy_token=True)
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out, ref.per_query_strict(q, k, v, lengths, True, lengths=lengths), rtol=1e-12, atol=1e-12)


def test_equal_scores_average_exactly_and_empty_rows_are_zero():
    q = torch.full((1, 2, 1, 8), 1.0, dtype=torch.float64)
    k = torch.full((1, 1, 64, 8), 2.0, dtype=torch.float64)
    v = torch.ones_like(k)
    v[:, :, 32:] = -1
    out = ref.cyclic_attention(q, k, v, query_stride=64, query_offset=63)
    assert torch.equal(out, torch.zeros_like(out))
    empty = ref.cyclic_attention(q, k, v, query_stride=1, query_offset=0, strict_past=True)
    assert torch.equal(empty, torch.zeros_like(empty))


def test_bf16_pipeline_is_within_bf16_rounding_of_the_oracle():
    torch.manual_seed(2)
    q, k, v = (torch.randn(1, 2, 9, 16).bfloat16() for _ in range(3))
    dout = torch.randn(1, 2, 9, 16).bfloat16()
    keep = ref.cyclic_keep(9, 9, 1, 0)
    out, dq, dk, dv = ref.bf16_pipeline(q, k, v, dout, keep, 0.25)
    leaves = [t.double().requires_grad_() for t in (q, k, v)]
    exact = ref.masked_attention(*leaves, keep, 0.25)
    grads = torch.autograd.grad(exact, leaves, dout.double())
    for a, e in zip((out, dq, dk, dv), (exact, *grads)):
        assert ((a - e).norm() / e.norm()).item() < 1.5e-2
        assert a.to(torch.bfloat16).double().equal(a)


# -------------------------------------------------------- planted slips ----
def test_planted_mistakes_are_caught():
    """Slips planted in copies of the oracle's outputs fail the checks above."""
    # (1) segments split on run change only (the visible-end rule dropped):
    # a kv cap makes visible ends repeat, so queries 1..5 of one document form
    # three segments; merging them gives the early queries the wrong keys.
    docs = np.zeros((1, 6), dtype=np.int64)
    good = meta.strict_metadata(docs, 6, 0, np.array([3]))
    assert good["cu_queries"].tolist() == [0, 3, 4, 5]
    bad = dict(good)
    bad["cu_queries"] = np.array([0, 5], dtype=np.int32)
    bad["key_indices"] = good["key_indices"][good["cu_keys"][2] :]
    bad["cu_keys"] = np.array([0, bad["key_indices"].size], dtype=np.int32)
    torch.manual_seed(1)
    q = torch.randn(1, 2, 6, 8, dtype=torch.float64)
    k = torch.randn(1, 2, 6, 8, dtype=torch.float64)
    v = torch.randn_like(k)
    expected = ref.per_query_strict(q, k, v, torch.tensor([0]), False, lengths=torch.tensor([3]))
    torch.testing.assert_close(ref.strict_attention(q, k, v, metadata=good), expected, rtol=1e-12, atol=1e-12)
    assert not torch.allclose(ref.strict_attention(q, k, v, metadata=bad), expected)
    # (2) an off-by-one causal bound (j < slot instead of j <= slot)
    assert not torch.equal(ref.cyclic_keep(5, 11, 2, 0), ref.cyclic_keep(5, 11, 2, 1))
    # (3) a left search for key_query_end misses the known answer
    m = 2**31 - 1
    q_ids, k_ids = np.array([[0, m]]), np.array([[-1, 0, m]])
    assert np.searchsorted(q_ids[0], k_ids[0], side="left").tolist() != [2, 1, 2]
    assert meta.cyclic_metadata(q_ids, k_ids)[3].tolist() == [[2, 1, 2]]
    # (4) dropping the document-start rule changes visibility on non-monotonic ids
    metadata = (np.array([[0, 0]]), np.array([[-1, 0, 1, 0]]), np.array([[3, 3]]), np.array([[2, 2, 2, 2]]))
    keep_full = ref.cyclic_keep(2, 4, 1, 2, metadata)
    qs, ks, _, ke = (torch.from_numpy(t) for t in metadata)
    keep_without_start = (
        (torch.arange(4)[None, :] <= 2 + torch.arange(2)[:, None])[None]
        & ((qs[:, :, None] == ks[:, None, :]) | (ks[:, None, :] == -1))
        & (torch.arange(2)[None, :, None] < ke[:, None, :])
    )
    assert not torch.equal(keep_full[:, 0], keep_without_start)
