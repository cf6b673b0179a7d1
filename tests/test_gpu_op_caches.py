"""Lifetimes of the C++ operators' caches (csrc/torch_ops.cpp): the packed
strict plans and the cyclic schedules hold their metadata tensors weakly, so
a cache entry is dropped once its metadata is freed (training builds new
metadata every step), a repeat call is a hit, and an in-place change of the
metadata builds a new entry."""

import gc

import pytest
import torch

import bench
from white_matter_amd import (
    prepare_feedback_metadata,
    prepare_strict_causal_metadata,
    strict_causal_attention,
)
from white_matter_amd.cyclic_attention import cyclic_attn_doc_fwd

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _plans() -> int:
    return torch.ops.white_matter._packed_plan_cache_size()


def _schedules() -> int:
    return torch.ops.white_matter._cyclic_schedule_cache_size()


def test_packed_plans_follow_their_metadata():
    torch.manual_seed(2)
    q, k, v = (torch.randn(2, 4, 256, 64, device=DEV, dtype=torch.bfloat16) for _ in range(3))
    base = _plans()
    for step in range(3):
        docs = bench.geometric_documents(2, 256, seed=step, mean=64, lo=8, hi=256).to(DEV)
        metadata = prepare_strict_causal_metadata(docs, 256)
        leaves = [t.clone().requires_grad_() for t in (q, k, v)]
        out = strict_causal_attention(*leaves, metadata=metadata)
        torch.autograd.grad(out.float().sum(), leaves)
        assert _plans() == base + 1, "one plan per live schedule and call shape"
        out = strict_causal_attention(q, k, v, metadata=metadata)
        assert _plans() == base + 1, "a repeat call is a hit"
        metadata.cu_keys.add_(0)  # an in-place write bumps the version: a new plan
        again = strict_causal_attention(q, k, v, metadata=metadata)
        assert torch.equal(again, out)
        assert _plans() == base + 2
        del metadata, docs, out, again, leaves
        gc.collect()
        assert _plans() == base, "the plans of a freed schedule are dropped"


def test_cyclic_schedules_follow_their_metadata():
    torch.manual_seed(4)
    length, stride = 256, 4
    q = torch.randn(2, 4, length // stride, 64, device=DEV, dtype=torch.bfloat16)
    k, v = (torch.randn(2, 2, length, 64, device=DEV, dtype=torch.bfloat16) for _ in range(2))
    groups = [torch.arange(r, length, stride, device=DEV) for r in range(stride)]
    base = _schedules()
    docs = bench.geometric_documents(2, length, seed=5, mean=48, lo=4, hi=200).to(DEV)
    metas = prepare_feedback_metadata(docs, groups, length, use_dummy_token=False)
    first, _ = cyclic_attn_doc_fwd(q, k, v, *metas[1], stride, 0, 64)
    assert _schedules() == base + 1
    again, _ = cyclic_attn_doc_fwd(q, k, v, *metas[1], stride, 0, 64)
    assert _schedules() == base + 1 and torch.equal(again, first)
    del metas
    gc.collect()
    assert _schedules() == base, "the schedule of freed metadata is dropped"
