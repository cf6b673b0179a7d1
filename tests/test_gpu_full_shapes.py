"""The benchmarked configurations at their full sizes, through the public
operators, and the kernel instantiations the bench lines run:

  C2  strict Jacobi, (8, 16, 2048, 128) bf16, geometric documents, fwd+bwd;
  C3  a full cyclic pass at stride 8 (eight residue calls), fwd+bwd;
  C4  prefill of 256 queries after ragged prefixes of 512..8192 keys, which
      runs the 256-row (8-wave) forward workgroups at head_dim 128.

A float64 oracle over a whole C2 batch is slow, so at full size two sampled
(row, head) slices are checked against the oracle at the north-star tolerance
(bf16 vs float64: max-abs <= 1e-2 * max(1, max|ref|), rel-L2 <= 5e-3), and
every other element through size-independent properties: everything finite,
the first token of every document outputs exactly zero with zero dQ (it sees
no key), and the last key of every document gets exactly zero dK/dV (no query
sees it). The 256-row prefill is also checked in full at a mid size."""

import numpy as np
import pytest
import torch

from bench import geometric_documents
from oracle import attention as ref
from tests.numerics import assert_bf16_close
from white_matter_amd import (
    cyclic_attention,
    prepare_feedback_metadata,
    prepare_strict_causal_metadata,
    strict_causal_attention,
)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _runs(row: torch.Tensor) -> list[tuple[int, int]]:
    """(first, end) of each document run of a 1-D id row."""
    ids = row.cpu().numpy()
    cuts = np.flatnonzero(np.diff(ids)) + 1
    starts = np.concatenate(([0], cuts))
    ends = np.concatenate((cuts, [ids.shape[0]]))
    return list(zip(starts.tolist(), ends.tolist()))


def _strict_doc_keep(row: torch.Tensor) -> torch.Tensor:
    """(1, 1, T, T) keep of the strict document rule on one row: key s is
    visible to query t iff both lie in one document run and s < t."""
    length = row.shape[0]
    doc = torch.zeros(length, dtype=torch.long)
    for n, (first, end) in enumerate(_runs(row)):
        doc[first:end] = n
    t = torch.arange(length)
    return ((doc[:, None] == doc[None, :]) & (t[None, :] < t[:, None]))[None, None]


def _normal(shape, gen, dim):
    return (torch.randn(shape, generator=gen) * dim**-0.5).to(DEV, torch.bfloat16)


def test_c2_full_shape_forward_backward():
    batch, heads, length, dim = 8, 16, 2048, 128
    print("C2 full shape: (8, 16, 2048, 128), geometric documents, fwd+bwd", flush=True)
    gen = torch.Generator().manual_seed(0)
    docs = geometric_documents(batch, length, 0)
    q, k, v = (_normal((batch, heads, length, dim), gen, dim) for _ in range(3))
    metadata = prepare_strict_causal_metadata(docs.to(DEV), length)
    leaves = [t.clone().requires_grad_() for t in (q, k, v)]
    out = strict_causal_attention(*leaves, metadata=metadata)
    probe = torch.randn(out.shape, generator=gen).to(DEV, torch.bfloat16)
    dq, dk, dv = torch.autograd.grad(out, leaves, probe)
    torch.cuda.synchronize()
    for name, t in (("out", out), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert torch.isfinite(t.float()).all(), name
    for b in range(batch):
        runs = _runs(docs[b])
        first = torch.tensor([s for s, _ in runs], device=DEV)
        last = torch.tensor([e - 1 for _, e in runs], device=DEV)
        assert out[b].index_select(0, first).count_nonzero() == 0
        assert dq[b].index_select(1, first).count_nonzero() == 0
        assert dk[b].index_select(1, last).count_nonzero() == 0
        assert dv[b].index_select(1, last).count_nonzero() == 0
    for b, h in ((2, 3), (7, 15)):
        keep = _strict_doc_keep(docs[b])
        slices = [t[b : b + 1, h : h + 1].cpu().double().requires_grad_() for t in (q, k, v)]
        expected = ref.masked_attention(*slices, keep, dim**-0.5)  # (1, 1, T, D)
        grads = torch.autograd.grad(expected, slices, probe[b : b + 1, :, h : h + 1].transpose(1, 2).cpu().double())
        assert_bf16_close(out[b, :, h], expected[0, 0], what=f"C2 out row {b} head {h}")
        for name, a, e in zip("qkv", (dq, dk, dv), grads):
            assert_bf16_close(a[b, h], e[0, 0], what=f"C2 d{name} row {b} head {h}")


def test_c3_full_stride8_pass():
    batch, heads, length, dim, stride = 8, 16, 2048, 128, 8
    print("C3 full stride-8 pass: 8 residue calls of (8, 16, 256, 128) over (8, 16, 2048, 128)", flush=True)
    gen = torch.Generator().manual_seed(3)
    docs = geometric_documents(batch, length, 3).to(DEV)
    groups = [torch.arange(r, length, stride, device=DEV) for r in range(stride)]
    metas = prepare_feedback_metadata(docs, groups, length, use_dummy_token=False)
    k, v = (_normal((batch, heads, length, dim), gen, dim) for _ in range(2))
    kl, vl = k.clone().requires_grad_(), v.clone().requires_grad_()
    for r in range(stride):
        q = _normal((batch, heads, length // stride, dim), gen, dim)
        ql = q.clone().requires_grad_()
        out = cyclic_attention(ql, kl, vl, query_stride=stride, query_offset=r, strict_past=True,
                               metadata=metas[r], backend="tilelang")
        probe = torch.randn(out.shape, generator=gen).to(DEV, torch.bfloat16)
        dq, dk, dv = torch.autograd.grad(out, (ql, kl, vl), probe)
        torch.cuda.synchronize()
        for name, t in (("out", out), ("dq", dq), ("dk", dk), ("dv", dv)):
            assert torch.isfinite(t.float()).all(), f"residue {r} {name}"
        # a query on the first token of its document sees nothing (strict past)
        for b in range(batch):
            firsts = [s for s, _ in _runs(docs[b]) if s % stride == r]
            if firsts:
                rows = torch.tensor([s // stride for s in firsts], device=DEV)
                assert out[b].index_select(1, rows).count_nonzero() == 0
                assert dq[b].index_select(1, rows).count_nonzero() == 0
        b, h = r % batch, (5 * r + 1) % heads
        meta = tuple(t[b : b + 1].cpu() for t in metas[r])
        slices = [t[b : b + 1, h : h + 1].cpu().double().requires_grad_() for t in (q, k, v)]
        expected = ref.cyclic_attention(*slices, query_stride=stride, query_offset=r, strict_past=True, metadata=meta)
        grads = torch.autograd.grad(expected, slices, probe[b : b + 1, h : h + 1].cpu().double())
        assert_bf16_close(out[b, h], expected[0, 0], what=f"C3 residue {r} out row {b} head {h}")
        for name, a, e in zip("qkv", (dq, dk, dv), grads):
            assert_bf16_close(a[b, h], e[0, 0], what=f"C3 residue {r} d{name} row {b} head {h}")


@pytest.mark.parametrize("kv_heads", [8, 4])
def test_prefill_256_row_workgroups_head_dim_128(kv_heads):
    """256 queries after ragged prefixes of 512 keys or more select the 8-wave
    (256-row) forward at head_dim 128; the whole output against the oracle."""
    heads, chunk, dim = 8, 256, 128
    prefix = torch.tensor([512, 1300, 2600])
    batch = prefix.numel()
    capacity = int(prefix.max()) + chunk
    print(f"C4-style prefill: 256 queries after prefixes {prefix.tolist()}, Hkv={kv_heads}", flush=True)
    gen = torch.Generator().manual_seed(41)
    q = _normal((batch, heads, chunk, dim), gen, dim)
    k, v = (_normal((batch, kv_heads, capacity, dim), gen, dim) for _ in range(2))
    lengths = prefix + chunk
    for b in range(batch):  # unused capacity may hold anything
        k[b, :, int(lengths[b]) :] = float("nan")
        v[b, :, int(lengths[b]) :] = float("nan")
    with torch.no_grad():
        out = strict_causal_attention(q, k, v, query_start=prefix.to(DEV), kv_lengths=lengths.to(DEV))
    expected = ref.strict_attention(q.cpu(), k.cpu(), v.cpu(), query_start=prefix, kv_lengths=lengths)
    assert_bf16_close(out, expected, what=f"256-row prefill Hkv={kv_heads}")


def test_c4_prefill_full_shape():
    batch, heads, chunk, dim = 32, 16, 256, 128
    print("C4 prefill full shape: B=32 H=16, 256 queries after prefixes ~U[512,8192]", flush=True)
    prefix = torch.from_numpy(np.random.default_rng(1).integers(512, 8192, size=batch, endpoint=True))
    capacity = int(prefix.max()) + chunk
    gen = torch.Generator().manual_seed(1)
    q = _normal((batch, heads, chunk, dim), gen, dim)
    k = torch.empty(batch, heads, capacity, dim, device=DEV, dtype=torch.bfloat16).normal_(0, dim**-0.5)
    v = torch.empty_like(k).normal_(0, dim**-0.5)
    lengths = prefix + chunk
    with torch.no_grad():
        out = strict_causal_attention(q, k, v, query_start=prefix.to(DEV), kv_lengths=lengths.to(DEV))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    for b, h in ((0, 0), (int(prefix.argmax()), 9), (int(prefix.argmin()), 15)):
        expected = ref.strict_attention(
            q[b : b + 1, h : h + 1].cpu(), k[b : b + 1, h : h + 1].cpu(), v[b : b + 1, h : h + 1].cpu(),
            query_start=prefix[b : b + 1], kv_lengths=lengths[b : b + 1],
        )
        assert_bf16_close(out[b, :, h], expected[0, :, 0], what=f"C4 prefill row {b} head {h}")
