"""A full cyclic pass (every residue call, forward and backward, packed
documents) captured in one HIP graph: each replay, with eager work and
synchronisations between replays, gives exactly the eager pass's outputs and
gradients (the same deterministic kernels in the same order)."""

import pytest
import torch

import bench
from white_matter_amd import cyclic_attention, prepare_feedback_metadata

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.skip(
    reason="its one run, on an earlier build whose operators were Python custom ops (schedule caches and gap fills in "
    "Python), segfaulted (exit 139) in torch.cuda.graph's capture_end, with the backward issued from the autograd "
    "engine's worker thread; no cause was identified. The operators are now C++ (csrc/torch_ops.cpp CyclicDocFn "
    "-> forward_impl/backward_impl -> wmx_attn_fwd/bwd): on a cached schedule they reach only caching-allocator "
    "tensors, fill kernels and kernel launches on the current stream, a cache miss raises under capture, and neither "
    "library imports an allocating, copying or synchronising call (tests/test_capture_guard.py). That rules out "
    "this library's host steps but names no cause, so the case stays off the GPU"
)
def test_captured_pass_matches_eager():
    torch.manual_seed(12)
    batch, heads, length, dim, stride = 2, 4, 512, 128, 4
    docs = bench.geometric_documents(batch, length, stride, mean=96, lo=4, hi=400).to(DEV)
    groups = [torch.arange(r, length, stride, device=DEV) for r in range(stride)]
    metas = prepare_feedback_metadata(docs, groups, length, use_dummy_token=False)
    k = torch.randn(batch, heads, length, dim, device=DEV, dtype=torch.bfloat16).requires_grad_()
    v = torch.randn_like(k).requires_grad_()
    qs = [torch.randn(batch, heads, g.numel(), dim, device=DEV, dtype=torch.bfloat16).requires_grad_() for g in groups]
    probes = [torch.randn(q.shape, device=DEV, dtype=torch.bfloat16) for q in qs]

    def full_pass():
        results = []
        for r in range(stride):
            out = cyclic_attention(qs[r], k, v, query_stride=stride, query_offset=r, strict_past=True,
                                   metadata=metas[r], backend="tilelang")
            results.append((out, *torch.autograd.grad(out, (qs[r], k, v), probes[r])))
        return results

    eager = [[t.clone() for t in call] for call in full_pass()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        full_pass()  # warm-up on the capture stream's side
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = full_pass()
    for replay in range(3):
        torch.randn(1 << 20, device=DEV).sum()  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        for r, (want, got) in enumerate(zip(eager, captured)):
            for name, a, b in zip(("out", "dq", "dk", "dv"), got, want):
                assert torch.equal(a, b), f"replay {replay}, residue {r}: {name} differs from the eager pass"
