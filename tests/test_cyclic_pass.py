"""The cyclic pass driver and greedy decoding on the CPU: a float64 model with
the oracle's attention and KV store.

Pinned property: with G = T - 1 groups and one pass, every group but the
first holds one token, and token t (t < T - 1) reads the dummy and exactly
the refreshed keys of tokens 0 .. t - 1 of its document
(blocks/_execution/cyclic.py:357-431: groups publish in order, strict past
with the dummy shift). That is token-by-token decoding from a pool holding
only the dummy (blocks/white_matter.py:165-186, documents.py:57-61), so the
pool slots of tokens 0 .. T - 2 must agree to float64 rounding between the
two drivers. A wrong group order, slot shift, stride/offset or document
rule breaks that agreement."""

import pytest
import torch

from oracle import attention as ref
from oracle import kv_pool as ref_pool
from white_matter_amd.cyclic_pass import (
    FeedbackConfig,
    FeedbackModel,
    GreedyDecoder,
    document_positions,
    forward_cyclic,
    write_sources,
)


class OracleKernels:
    """The driver's kernel set on the float64 oracle (CPU), casting results to
    the model's dtype and device."""

    @staticmethod
    def cyclic(q, k, v, *, query_stride, query_offset, strict_past, metadata):
        meta = None if metadata is None else tuple(t.cpu() for t in metadata)
        out = ref.cyclic_attention(
            q.cpu(), k.cpu(), v.cpu(), query_stride=query_stride, query_offset=query_offset,
            strict_past=strict_past, metadata=meta,
        )
        return out.to(q.device, q.dtype).transpose(1, 2)

    @staticmethod
    def decode(q, k, v, *, lengths, use_dummy_token, key_mask):
        out = ref.strict_attention(
            q.cpu(), k.cpu(), v.cpu(), query_start=lengths.cpu(), kv_lengths=lengths.cpu(),
            use_dummy_token=use_dummy_token, key_mask=key_mask.cpu(),
        )
        return out.to(q.device, q.dtype)

    @staticmethod
    def store(key, value, weight, cos, sin, keys, values, slots, *, eps):
        k, v = ref_pool.write_pool(
            key.cpu(), value.cpu(), weight.cpu(), cos.cpu(), sin.cpu(), keys.cpu(), values.cpu(), slots.cpu(), eps
        )
        keys.copy_(k)
        values.copy_(v)


def _model(length, **overrides):
    config = FeedbackConfig(
        vocab_size=50, hidden_size=32, intermediate_size=64, num_layers=3, num_heads=4, num_kv_heads=2,
        head_dim=16, num_kv_channels=2, cyclic_groups=length - 1, num_passes=1, **overrides,
    )
    return FeedbackModel(config, device="cpu", dtype=torch.float64, residual_dtype=torch.float64, seed=3)


def _decode_tokens(model, ids, docs):
    """Teacher-forced decoding of every token from a pool holding only the
    dummy, resetting the visible slots and the position at document starts."""
    batch, length = ids.shape
    keys, values = model.new_pool(batch, length + 1)
    stacked = model.dummy.expand(batch, 1, model.config.num_sources, -1)
    write_sources(model, stacked, keys, values, torch.tensor([0]), model.rope(torch.zeros(batch, 1)), OracleKernels)
    keep = torch.zeros(batch, length + 1, dtype=torch.bool)
    keep[:, 0] = True
    decoder = GreedyDecoder(model, keys, values, 1, torch.zeros(batch, 1), ids[:, :1], keep,
                            kernels=OracleKernels, capture=False)
    for t in range(length - 1):
        for b in range(batch):
            if t > 0 and docs is not None and docs[b, t] != docs[b, t - 1]:
                decoder.key_mask[b, 1:] = False
                decoder.position[b] = 0
        decoder.token.copy_(ids[:, t : t + 1])
        decoder()
    return keys, values


@pytest.mark.parametrize("documents", [False, True])
def test_single_token_groups_match_decoding(documents):
    torch.manual_seed(0)
    length = 12
    model = _model(length)
    ids = torch.randint(0, 50, (2, length))
    docs = torch.tensor([[0, 0, 0, 1, 1, 1, 1, 2, 2, 2, 2, 2], [0, 0, 0, 0, 0, 1, 1, 2, 3, 3, 3, 3]]) if documents else None
    _, keys, values, positions = forward_cyclic(model, ids, docs, kernels=OracleKernels)
    dk, dv = _decode_tokens(model, ids, docs)
    # slot 0 the dummy, slots 1 .. T - 1 tokens 0 .. T - 2 (token T - 1 ran in group 0)
    for got, want in ((keys, dk), (values, dv)):
        assert torch.allclose(got[..., : length, :], want[..., : length, :], rtol=1e-9, atol=1e-12)


def test_passes_refresh_the_pool():
    """A second pass reads the pool the first one published: the last token
    (group 0, which first saw only the embedding-initialised pool) changes,
    while with one group per token tokens 0 .. T - 2 are already final."""
    torch.manual_seed(1)
    length = 10
    model = _model(length)
    ids = torch.randint(0, 50, (1, length))
    h1, k1, _, _ = forward_cyclic(model, ids, passes=1, kernels=OracleKernels)
    h2, k2, _, _ = forward_cyclic(model, ids, passes=2, kernels=OracleKernels)
    assert torch.allclose(h1[:, 1 : length - 1], h2[:, 1 : length - 1], rtol=1e-9, atol=1e-12)
    assert not torch.allclose(h1[:, length - 1], h2[:, length - 1], rtol=1e-6, atol=1e-9)


def test_document_positions_known_answer():
    """documents.py:24's example: [0,0,0,1,1,2] -> [0,1,2,0,1,0]."""
    ids = torch.tensor([[0, 0, 0, 1, 1, 2]])
    assert document_positions(ids).tolist() == [[0, 1, 2, 0, 1, 0]]


def test_router_prior_and_sources():
    """routing.py:18-25 with rows < cols: channel c mixes sources c, c + k, ..."""
    model = _model(8)
    k, s = model.config.num_kv_channels, model.config.num_sources
    bias = model.router["k"][1].view(k, s)
    for row in range(k):
        for col in range(s):
            assert bias[row, col] == (0.25 if col % k == row else 0.0)
    assert s == model.config.num_layers + 1
