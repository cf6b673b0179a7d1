"""Cyclic attention with packed documents through the strided varlen kernels
(document metadata packed into per-document segments) against the float64
oracle and against the document-mode kernels on the same inputs; the packed
route is the one taken for builder metadata, a query that sees no key gets a
zero row and an infinite LSE, and an in-place change of the metadata builds a
new schedule (the C++ operators' schedule cache sees the version counter)."""

import importlib

import pytest
import torch

import bench
from oracle import attention as ref
from tests.numerics import assert_bf16_close
from white_matter_amd import cyclic_attention, prepare_feedback_metadata

# the module (the package exports a function of the same name)
cyclic_module = importlib.import_module("white_matter_amd.cyclic_attention")

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(q, k, v, options, probe):
    leaves = [t.detach().clone().requires_grad_() for t in (q, k, v)]
    out = cyclic_attention(*leaves, backend="tilelang", **options)
    return out, torch.autograd.grad(out, leaves, probe)


@pytest.mark.parametrize("dummy", [False, True])
@pytest.mark.parametrize("stride", [2, 4, 8])
def test_packed_matches_document_kernels_and_oracle(stride, dummy, monkeypatch):
    torch.manual_seed(stride + 10 * dummy)
    batch, heads, kv_heads, length, dim = 2, 4, 2, 512, 128
    docs = bench.geometric_documents(batch, length, stride, mean=96, lo=4, hi=400).to(DEV)
    groups = [torch.arange(r, length, stride, device=DEV) for r in range(stride)]
    keys = length + int(dummy)
    metas = prepare_feedback_metadata(docs, groups, keys, use_dummy_token=dummy)
    k = torch.randn(batch, kv_heads, keys, dim, device=DEV, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    for residue in (0, stride - 1):
        print(f"stride {stride} dummy {dummy} residue {residue}", flush=True)
        q = torch.randn(batch, heads, groups[residue].numel(), dim, device=DEV, dtype=torch.bfloat16)
        options = dict(query_stride=stride, query_offset=residue, strict_past=not dummy, metadata=metas[residue])
        probe = torch.randn(q.shape, device=DEV, dtype=torch.bfloat16)
        packed_out, packed_grads = _run(q, k, v, options, probe)
        facts = torch.ops.white_matter._cyclic_schedule(*metas[residue], q.shape[2], keys, stride,
                                                         residue - int(not dummy))[0]
        assert int(facts[0]) == 2, "builder metadata takes the packed route"
        # the document-mode kernels on the same inputs: a packer that refuses
        with monkeypatch.context() as m:
            m.setattr(cyclic_module, "_build_packed_schedule", lambda *a, **kw: None)
            torch.ops.white_matter._cyclic_schedule_cache_clear()
            doc_out, doc_grads = _run(q, k, v, options, probe)
        torch.ops.white_matter._cyclic_schedule_cache_clear()
        leaves = [t.double().cpu().requires_grad_() for t in (q, k, v)]
        expected = ref.cyclic_attention(*leaves, query_stride=stride, query_offset=residue, strict_past=not dummy,
                                        metadata=tuple(t.cpu() for t in metas[residue]))
        expected_grads = torch.autograd.grad(expected, leaves, probe.double().cpu())
        for name, a, d, e in zip(("out", "dq", "dk", "dv"), (packed_out, *packed_grads), (doc_out, *doc_grads),
                                 (expected, *expected_grads)):
            assert_bf16_close(a, e, what=f"packed {name}")
            assert_bf16_close(d, e, what=f"document-mode {name}")


def test_unseen_queries_and_metadata_changes():
    torch.manual_seed(3)
    length, stride = 64, 4
    docs = (torch.arange(length, device=DEV) // 8)[None].expand(2, -1).contiguous()
    groups = [torch.arange(r, length, stride, device=DEV) for r in range(stride)]
    meta = prepare_feedback_metadata(docs, groups, length, use_dummy_token=False)[0]
    q = torch.randn(2, 2, 16, 64, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(2, 2, length, 64, device=DEV, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    out, lse = cyclic_module.cyclic_attn_doc_fwd(q, k, v, *meta, stride, -1, 64)
    # residue 0, strict: every document's first query (slot 8 d) sees no key
    first = torch.arange(0, 16, 2)
    assert (out[:, :, first] == 0).all() and torch.isinf(lse[:, :, first]).all()
    assert torch.isfinite(lse[:, :, 1::2]).all()
    cached = torch.ops.white_matter._cyclic_schedule_cache_size()
    cyclic_module.cyclic_attn_doc_fwd(q, k, v, *meta, stride, -1, 64)
    assert torch.ops.white_matter._cyclic_schedule_cache_size() == cached  # a cache hit
    meta.key_query_end.add_(0)  # an in-place write bumps the version: the schedule is rebuilt
    again, _ = cyclic_module.cyclic_attn_doc_fwd(q, k, v, *meta, stride, -1, 64)
    assert torch.ops.white_matter._cyclic_schedule_cache_size() == min(cached + 1, 256)
    assert torch.equal(again, out)
