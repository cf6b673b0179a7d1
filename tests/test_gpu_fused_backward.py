"""The fused backward of short packed segments (csrc/attn_bwd_seg.hip: one
workgroup holds a segment's queries, at most 128, and computes its dQ, dK and
dV in one pass over its keys) against the float64 oracle and against the
tiled backward kernels on the same inputs. Cyclic calls with as many query
heads as KV heads take it for short segments (the list's limit is raised
here to the kernel's 128 queries); the documents below put segments at the list's edges (1, 32, 33, 64, 65, 127, 128
and 129 queries, key counts that are not multiples of 64) beside longer ones
that stay on the tiled kernels, with and without the dummy slot."""

import importlib

import pytest
import torch

import bench
from oracle import attention as ref
from tests.numerics import assert_bf16_close
from white_matter_amd import cyclic_attention, prepare_feedback_metadata

# the module (the package exports a function of the same name)
strict_module = importlib.import_module("white_matter_amd.strict_causal_attention")

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _documents(lengths_per_row):
    rows = [torch.repeat_interleave(torch.arange(len(ls)), torch.tensor(ls)) for ls in lengths_per_row]
    return torch.stack(rows).to(DEV)


def _run(q, k, v, options, probe):
    leaves = [t.detach().clone().requires_grad_() for t in (q, k, v)]
    out = cyclic_attention(*leaves, backend="tilelang", **options)
    return (out, *torch.autograd.grad(out, leaves, probe))


def _check(docs, stride, dummy, dim, residues, heads=2, monkeypatch=None):
    batch, length = docs.shape
    keys = length + int(dummy)
    groups = [torch.arange(r, length, stride, device=DEV) for r in range(stride)]
    metas = prepare_feedback_metadata(docs, groups, keys, use_dummy_token=dummy)
    k = torch.randn(batch, heads, keys, dim, device=DEV, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    fused_seen = 0
    for residue in residues:
        print(f"stride {stride} dummy {dummy} dim {dim} residue {residue}", flush=True)
        q = torch.randn(batch, heads, groups[residue].numel(), dim, device=DEV, dtype=torch.bfloat16)
        options = dict(query_stride=stride, query_offset=residue, strict_past=not dummy, metadata=metas[residue])
        probe = torch.randn(q.shape, device=DEV, dtype=torch.bfloat16)
        # the kernel's whole range (1 to 128 queries), beyond the list's default limit
        monkeypatch.setattr(strict_module, "_FUSED_ROWS", strict_module._FUSED_ROWS_MAX)
        torch.ops.white_matter._cyclic_schedule_cache_clear()
        built = torch.ops.white_matter._cyclic_schedule(*metas[residue], q.shape[2], keys, stride,
                                                        residue - int(not dummy))
        assert int(built[0][0]) == 2 and len(built) == 11
        fused_seen += built[8].shape[0]
        fused = _run(q, k, v, options, probe)
        # the tiled kernels on the same inputs: an empty fused list (outputs
        # of the schedule operator must not alias one another: copies)
        def tiled_only(md, s, qe, kt=128):
            q_units, k_units = strict_module._work_units(md, s, query_extent=qe, key_tile=kt)[:2]
            return torch.zeros(1, 16, dtype=torch.int32, device=DEV)[:0], q_units.clone(), k_units.clone()

        with monkeypatch.context() as m:
            m.setattr(strict_module, "_fused_units", tiled_only)
            torch.ops.white_matter._cyclic_schedule_cache_clear()
            tiled = _run(q, k, v, options, probe)
        torch.ops.white_matter._cyclic_schedule_cache_clear()
        leaves = [t.double().cpu().requires_grad_() for t in (q, k, v)]
        expected = ref.cyclic_attention(*leaves, query_stride=stride, query_offset=residue, strict_past=not dummy,
                                        metadata=tuple(t.cpu() for t in metas[residue]))
        expected = (expected, *torch.autograd.grad(expected, leaves, probe.double().cpu()))
        for name, f, t, e in zip(("out", "dq", "dk", "dv"), fused, tiled, expected):
            assert_bf16_close(f, e, what=f"fused {name}")
            assert_bf16_close(t, e, what=f"tiled {name}")
    assert fused_seen > 0, "no segment took the fused backward"


@pytest.mark.parametrize("dummy", [False, True])
@pytest.mark.parametrize("dim", [128, 64, 96])
def test_edge_segment_sizes_stride_8(dim, dummy, monkeypatch):
    torch.manual_seed(dim + dummy)
    # at stride 8 a document of L tokens gives about L / 8 queries per residue
    docs = _documents([
        [8, 256, 264, 515, 1005],
        [1024, 1024],
        [1032, 1016],
    ])
    _check(docs, 8, dummy, dim, residues=(0, 3, 7), monkeypatch=monkeypatch)


@pytest.mark.parametrize("dummy", [False, True])
@pytest.mark.parametrize("stride", [1, 2, 4])
def test_geometric_documents(stride, dummy, monkeypatch):
    torch.manual_seed(stride + 10 * dummy)
    docs = bench.geometric_documents(2, 1024, stride, mean=96, lo=4, hi=600).to(DEV)
    _check(docs, stride, dummy, 128, residues=(0, stride - 1), heads=4, monkeypatch=monkeypatch)


def test_repeated_calls_are_identical():
    """No atomics: the fused kernel's gradients are the same on every run."""
    torch.manual_seed(5)
    docs = bench.geometric_documents(2, 1024, 8, mean=256, lo=16, hi=1024).to(DEV)
    stride, length = 8, docs.shape[1]
    groups = [torch.arange(r, length, stride, device=DEV) for r in range(stride)]
    metas = prepare_feedback_metadata(docs, groups, length + 1, use_dummy_token=True)
    q = torch.randn(2, 4, groups[2].numel(), 128, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(2, 4, length + 1, 128, device=DEV, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    probe = torch.randn(q.shape, device=DEV, dtype=torch.bfloat16)
    options = dict(query_stride=stride, query_offset=2, strict_past=False, metadata=metas[2])
    first = _run(q, k, v, options, probe)
    for _ in range(3):
        again = _run(q, k, v, options, probe)
        for a, b in zip(first, again):
            assert torch.equal(a, b)
