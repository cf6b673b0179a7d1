"""The torch.compile contract of the HIP path, as the reference's tests state
it for its accelerated backends:

  - tests/unit/test_strict_causal_attention.py:247-275: strict prefill and
    Jacobi (dense and packed documents, a cached prefix, a padded head_dim)
    compiled with fullgraph=True, outputs and gradients against the oracle;
  - tests/unit/test_strict_causal_attention.py:278-331: single-query decode
    over per-row device lengths compiled with fullgraph=True, captured in a
    HIP graph, replayed after the lengths and the cache change, with
    recompilation forbidden (the lengths are data, not guards);
  - tests/unit/test_ops.py:89-103 and blocks/_execution/cyclic.py:445: the
    cyclic operators traced whole (fullgraph) with documents, forward and
    backward.

Tolerances are the reference's own for these tests (0.03 outputs, 0.04
gradients, bf16 against the float64 oracle)."""

import pytest
import torch

from oracle import attention as ref
from white_matter_amd import (
    cyclic_attention,
    prepare_cyclic_attention_metadata,
    prepare_strict_causal_metadata,
    strict_causal_attention,
)

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("prefix", [0, 5])
@pytest.mark.parametrize("dim", [63, 64])
def test_fullgraph_prefill(packed, prefix, dim):
    torch._dynamo.reset()
    torch.manual_seed(7 + prefix + dim)
    q = torch.randn(2, 4, 12, dim, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    k = torch.randn(2, 2, prefix + 13, dim, device=DEV, dtype=q.dtype, requires_grad=True)
    v = torch.randn_like(k, requires_grad=True)
    docs = (torch.arange(prefix + 12, device=DEV) // 7).expand(2, -1)
    metadata = prepare_strict_causal_metadata(docs, 12, query_start=prefix, use_dummy_token=True) if packed else None

    def run(q, k, v):
        return strict_causal_attention(
            q, k, v, query_start=prefix, use_dummy_token=True, metadata=metadata, backend="torch_flash"
        )

    actual = torch.compile(run, fullgraph=True)(q, k, v)
    leaves = [t.detach().cpu().double().requires_grad_() for t in (q, k, v)]
    expected = ref.per_query_strict(*leaves, torch.full((2,), prefix), True, docs.cpu() if packed else None)
    torch.testing.assert_close(actual.double().cpu(), expected, atol=0.03, rtol=0.03)
    probe = torch.randn_like(actual)
    ga = torch.autograd.grad(actual, (q, k, v), probe)
    ge = torch.autograd.grad(expected, leaves, probe.double().cpu())
    for a, e in zip(ga, ge, strict=True):
        torch.testing.assert_close(a.double().cpu(), e, atol=0.04, rtol=0.04)


@pytest.mark.parametrize("dummy", [False, True])
@pytest.mark.parametrize("strided", [False, True])
@pytest.mark.parametrize("batch", [1, 3])
@torch.no_grad()
def test_fullgraph_decode_graph_replay(dummy, strided, batch):
    torch._dynamo.reset()
    torch.manual_seed(11 + batch)
    q = torch.randn(batch, 4, 1, 64, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(batch, 4 if strided else 2, 33 + int(dummy), 64, device=DEV, dtype=q.dtype)
    v = torch.randn_like(k)
    if strided:  # a pool view: the batch stride spans heads this call does not read
        k, v = k[:, :2], v[:, :2]
    lengths = torch.tensor([0, 7, 16][:batch], device=DEV, dtype=torch.int32)

    def run(q, k, v, lengths):
        return strict_causal_attention(
            q, k, v, query_start=lengths, use_dummy_token=dummy, backend="torch_flash", static_cache=True
        )

    compiled = torch.compile(run, fullgraph=True)
    compiled(q, k, v, lengths)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = compiled(q, k, v, lengths)
    for values in ([0, 7, 16][:batch], [3, 12, 32][:batch]):
        lengths.copy_(torch.tensor(values, device=DEV, dtype=torch.int32))
        for row, count in enumerate(values):
            k[row, :, : count + int(dummy)].normal_()
            v[row, :, : count + int(dummy)].normal_()
            k[row, :, count + int(dummy) :] = float("nan")
            v[row, :, count + int(dummy) :] = float("nan")
        with torch.compiler.set_stance("fail_on_recompile"):
            actual = compiled(q, k, v, lengths)
        graph.replay()
        torch.cuda.synchronize()
        expected = ref.per_query_strict(q.cpu(), k.cpu(), v.cpu(), lengths.cpu(), dummy)
        torch.testing.assert_close(actual.double().cpu(), expected, atol=0.03, rtol=0.03)
        torch.testing.assert_close(captured.double().cpu(), expected, atol=0.03, rtol=0.03)


@pytest.mark.parametrize("dummy", [False, True])
def test_fullgraph_cyclic_with_documents(dummy):
    """A residue call of the cyclic pass traced whole: the registered cyclic
    operators (forward and backward) and the document metadata."""
    torch._dynamo.reset()
    torch.manual_seed(19 + int(dummy))
    stride, length = 4, 96
    docs = torch.cat([torch.full((n,), d) for d, n in enumerate((30, 41, 25))])[None].expand(2, -1).to(DEV)
    residue = 1
    qseg = docs[:, residue::stride].contiguous()
    kseg = torch.cat((docs.new_full((2, 1), -1), docs[:, :-1]), 1) if dummy else docs
    meta = prepare_cyclic_attention_metadata(qseg, kseg, use_dummy_token=dummy)
    keys = kseg.shape[1]
    q = (torch.randn(2, 4, qseg.shape[1], 64) * 0.125).to(DEV, torch.bfloat16).requires_grad_()
    k = (torch.randn(2, 2, keys, 64) * 0.125).to(DEV, torch.bfloat16).requires_grad_()
    v = (torch.randn(2, 2, keys, 64) * 0.125).to(DEV, torch.bfloat16).requires_grad_()

    def run(q, k, v):
        return cyclic_attention(
            q, k, v, query_stride=stride, query_offset=residue, metadata=meta, strict_past=not dummy, backend="tilelang"
        )

    actual = torch.compile(run, fullgraph=True)(q, k, v)
    eager = run(q, k, v)
    torch.testing.assert_close(actual, eager, atol=0, rtol=0)
    probe = torch.randn_like(actual)
    ga = torch.autograd.grad(actual, (q, k, v), probe)
    ge = torch.autograd.grad(eager, (q, k, v), probe)
    for a, e in zip(ga, ge, strict=True):
        torch.testing.assert_close(a, e, atol=0, rtol=0)
    expected = ref.cyclic_attention(
        q.detach().cpu(), k.detach().cpu(), v.detach().cpu(), query_stride=stride, query_offset=residue,
        strict_past=not dummy, metadata=tuple(t.cpu() for t in meta),
    )
    torch.testing.assert_close(actual.double().cpu(), expected, atol=0.03, rtol=0.03)


def test_fullgraph_k_norm_rope_forward_and_backward():
    """The store's key transform as the registered operator
    (white_matter::k_norm_rope) traced whole, forward and backward, equal to
    eager bit for bit (training projects keys through it,
    modules/kv_pool.py:213-216)."""
    from white_matter_amd import kv_pool

    torch._dynamo.reset()
    gen = torch.Generator().manual_seed(4)
    key = torch.randn(2, 3, 2, 40, 64, generator=gen).to(DEV).requires_grad_()
    weight = (1 + 0.1 * torch.randn(3, 64, generator=gen)).to(DEV).requires_grad_()
    angle = torch.rand(2, 40, 32, generator=gen).to(DEV) * 7.0
    angle = torch.cat((angle, angle), -1)
    cos, sin = angle.cos(), angle.sin()

    def run(key, weight):
        return kv_pool.k_norm_rope(key, weight, cos, sin)

    actual = torch.compile(run, fullgraph=True)(key, weight)
    eager = run(key, weight)
    torch.testing.assert_close(actual, eager, atol=0, rtol=0)
    probe = torch.randn(actual.shape, generator=gen).to(DEV, torch.bfloat16)
    ga = torch.autograd.grad(actual, (key, weight), probe)
    ge = torch.autograd.grad(eager, (key, weight), probe)
    for a, e in zip(ga, ge, strict=True):
        torch.testing.assert_close(a, e, atol=0, rtol=0)


@torch.no_grad()
def test_fullgraph_kv_producer():
    """kv_pool.projection_inputs (the HIP producer around the router GEMM:
    the operators white_matter::kv_premix and white_matter::kv_mix) traced
    whole, equal to eager bit for bit."""
    from white_matter_amd import kv_pool

    torch._dynamo.reset()
    gen = torch.Generator().manual_seed(8)
    batch, tokens, sources, hidden, channels = 2, 5, 7, 256, 3
    stacked = torch.randn(batch, tokens, sources, hidden, generator=gen).to(DEV)
    pre_mix = tuple((1 + 0.2 * torch.randn(sources, hidden, generator=gen)).bfloat16().to(DEV) for _ in range(2))
    router = tuple(
        ((torch.randn(channels * sources, sources * hidden, generator=gen) * 0.01).bfloat16().to(DEV),
         (torch.randn(channels * sources, generator=gen) * 0.25).bfloat16().to(DEV))
        for _ in range(2)
    )
    gain = tuple((1 + 0.2 * torch.randn(channels, hidden, generator=gen)).bfloat16().to(DEV) for _ in range(2))

    def run(x):
        return kv_pool.projection_inputs(x, pre_mix, router, gain, eps=1e-6, mix_eps=1e-4)

    compiled = torch.compile(run, fullgraph=True)(stacked)
    eager = run(stacked)
    for c, e in zip(compiled, eager, strict=True):
        assert c.shape == (channels, batch * tokens, hidden)
        torch.testing.assert_close(c, e, atol=0, rtol=0)


@pytest.mark.parametrize("batch", [1, 3])
@pytest.mark.parametrize("strided", [False, True])
@pytest.mark.parametrize("static_cache", [False, True])
@pytest.mark.parametrize("dim", [8, 63])
@torch.inference_mode()
def test_torch_flash_decode_cache_reuses_graphs(batch, strided, static_cache, dim):
    """reference tests/unit/test_compilation_policy.py:35-89: torch_flash_decode
    compiled with fullgraph=True and dynamic=True over caches of growing
    capacity (5..16 slots, or a fixed 20 with static_cache) compiles at most two
    graphs, the outputs match math SDPA under the lengths mask, and the graphs
    build no offsets on the device (no arange node: the decode kernel reads the
    cache through its strides)."""
    from white_matter_amd.flash_attention import torch_flash_decode

    torch.compiler.reset()
    graphs = []

    def backend(graph, inputs):
        graphs.append(graph)
        return graph.forward

    compiled = torch.compile(torch_flash_decode, backend=backend, dynamic=True, fullgraph=True)
    torch.manual_seed(5 + batch + dim)
    q = torch.randn(batch, 4, 1, dim, device=DEV, dtype=torch.bfloat16)
    for length in range(5, 17):
        capacity = 20 if static_cache else length
        k, v = (torch.randn(batch, 4 if strided else 2, capacity, dim, device=DEV, dtype=q.dtype) for _ in range(2))
        if strided:  # a pool view: the batch stride spans heads this call does not read
            k, v = k[:, :2], v[:, :2]
        lengths = length - torch.arange(batch, device=DEV, dtype=torch.int32)
        keep = torch.arange(capacity, device=DEV)[None, :] < lengths[:, None]
        expected = torch.nn.functional.scaled_dot_product_attention(
            q.float(), k.float(), v.float(), attn_mask=keep[:, None, None, :], scale=0.5, enable_gqa=True
        ).transpose(1, 2)
        actual = compiled(q, k, v, lengths, 0.5, static_cache=static_cache)
        assert actual.shape == (batch, 1, 4, dim) and actual.dtype == q.dtype
        torch.testing.assert_close(actual.float(), expected, atol=0.03, rtol=0.03)
    assert 1 <= len(graphs) <= 2
    for graph in graphs:
        assert sum(node.target is torch.arange for node in graph.graph.nodes) == 0
    torch.compiler.reset()
