"""prepare_feedback_metadata on device tensors runs one HIP kernel
(wmx_feedback_meta). Its outputs must equal the reference's bit for bit
(blocks/_execution/metadata.py:11-55):

  - against the oracle (per-row run scans and a brute-force count of the
    visible queries of every key) for strides 1, 2, 4 and 8, with and without
    the dummy, int32 and int64 ids, padding runs (negative ids), a key length
    short of the full extent and odd lengths;
  - against the product's CPU formulation (itself pinned by the oracle in
    tests/test_host.py) for arbitrary, unordered query slots, slots past the
    row, more groups than one launch takes (64) and the full C3 shape;
  - against prepare_cyclic_attention_metadata on the derived ids, the
    reference's own check (tests/unit/test_metadata.py:10-23), at C3 size.
"""

import numpy as np
import pytest
import torch

from bench import geometric_documents
from oracle import metadata as ref_meta
from white_matter_amd import prepare_cyclic_attention_metadata, prepare_feedback_metadata

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _docs(gen: torch.Generator, batch: int, length: int, padding: bool) -> torch.Tensor:
    """Nondecreasing document ids with runs of 1..12 tokens; with padding,
    some runs become negative ids (-1, or -5 in row 0)."""
    rows = []
    for b in range(batch):
        ids, d = [], 0
        while len(ids) < length:
            n = int(torch.randint(1, 13, (1,), generator=gen))
            pad = padding and bool(torch.rand(1, generator=gen) < 0.25)
            ids += [(-5 if b == 0 else -1) if pad else d] * n
            d += 1
        rows.append(ids[:length])
    return torch.tensor(rows, dtype=torch.long)


def _assert_equal(actual, expected):
    for a, e in zip(actual, expected, strict=True):
        for ta, te in zip(a, e, strict=True):
            te = torch.as_tensor(np.asarray(te)) if not isinstance(te, torch.Tensor) else te
            assert ta.dtype == torch.int32 and ta.is_contiguous()
            assert ta.shape == te.shape
            assert torch.equal(ta.cpu(), te.cpu().to(torch.int32))


@pytest.mark.parametrize("stride", [1, 2, 4, 8])
@pytest.mark.parametrize("dummy", [False, True])
@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_matches_oracle(stride, dummy, dtype):
    gen = torch.Generator().manual_seed(100 * stride + 10 * int(dummy) + (dtype == torch.int32))
    length = 97
    docs = _docs(gen, 3, length, padding=True).to(dtype)
    positions = [torch.arange(r, length, stride) for r in range(stride)]
    for key_length in (length + int(dummy), length - 13):
        actual = prepare_feedback_metadata(
            docs.to(DEV), [p.to(DEV) for p in positions], key_length, use_dummy_token=dummy
        )
        expected = ref_meta.feedback_metadata(docs.numpy(), [p.numpy() for p in positions], key_length, dummy)
        _assert_equal(actual, expected)


def test_arbitrary_slots_and_many_groups():
    """Unordered slots, repeated slots, slots past the row (read as padding on
    the device, where the CPU path would raise, so those are compared on their
    own) and 70 groups, which take two launches."""
    gen = torch.Generator().manual_seed(5)
    length = 150
    docs = _docs(gen, 2, length, padding=True)
    positions = [torch.randperm(length, generator=gen)[: 1 + (r * 7) % 40] for r in range(70)]
    positions[3] = torch.tensor([5, 5, 0, 149])
    for dummy in (False, True):
        key_length = length + int(dummy)
        actual = prepare_feedback_metadata(docs.to(DEV), [p.to(DEV) for p in positions], key_length, use_dummy_token=dummy)
        expected = prepare_feedback_metadata(docs, positions, key_length, use_dummy_token=dummy)
        _assert_equal(actual, expected)
    outside = prepare_feedback_metadata(docs.to(DEV), [torch.tensor([0, length, -1], device=DEV)], length)
    assert outside[0].query_document_ids[:, 1:].eq(-2).all() and outside[0].query_key_start[:, 1:].eq(0).all()


@pytest.mark.parametrize("stride", [2, 4, 8])
def test_c3_shape(stride):
    """The C3 configuration (8 rows x 2048 tokens of geometric documents):
    equal to the CPU formulation with and without the dummy, and, without
    padding, to the cyclic builder's searches over the derived ids."""
    length = 2048
    docs = geometric_documents(8, length, seed=3).long()
    positions = [torch.arange(r, length, stride) for r in range(stride)]
    for dummy in (False, True):
        key_length = length + int(dummy)
        actual = prepare_feedback_metadata(docs.to(DEV), [p.to(DEV) for p in positions], key_length, use_dummy_token=dummy)
        expected = prepare_feedback_metadata(docs, positions, key_length, use_dummy_token=dummy)
        _assert_equal(actual, expected)
    # reference tests/unit/test_metadata.py:10-23: with the dummy, the keys are
    # the dummy then tokens 0 .. T-2 (key_length T), and every residue's
    # metadata is the cyclic builder's on those ids
    docs_dev = docs.to(DEV)
    actual = prepare_feedback_metadata(docs_dev, [p.to(DEV) for p in positions], length)
    keys = torch.cat((docs_dev.new_full((8, 1), -1), docs_dev[:, :-1]), dim=1)
    for residue, slots in enumerate(positions):
        expected = prepare_cyclic_attention_metadata(docs_dev[:, slots.to(DEV)], keys)
        for ta, te in zip(actual[residue], expected, strict=True):
            assert torch.equal(ta, te)


def test_degenerate_shapes():
    """A key length inside the dummy, one-token rows and a one-slot group."""
    docs = torch.tensor([[4], [-3]], device=DEV)
    meta = prepare_feedback_metadata(docs, [torch.tensor([0], device=DEV)], 1, use_dummy_token=True)[0]
    assert meta.key_document_ids.tolist() == [[-1], [-1]] and meta.key_query_end.tolist() == [[1], [1]]
    assert meta.query_document_ids.tolist() == [[4], [-2]] and meta.query_key_start.tolist() == [[1], [1]]
    meta = prepare_feedback_metadata(docs, [torch.tensor([0], device=DEV)], 1, use_dummy_token=False)[0]
    assert meta.key_document_ids.tolist() == [[4], [-2]] and meta.key_query_end.tolist() == [[1], [1]]
    assert meta.query_key_start.tolist() == [[0], [0]]
