"""The two dQ paths of the backward on the gfx950 kernels: with the dS buffer
(the dK/dV kernel stores bf16 dS^T, the dQ kernel reads it) and without it
(the dQ kernel recomputes S and dP). Both run through the C ABI on the same
inputs; dK/dV come from the same kernel and must match bit for bit, dQ to the
bf16 tolerance, and both dQ results against the float64 oracle."""

import ctypes

import pytest
import torch

from oracle import attention as ref
from tests.numerics import assert_bf16_close
from white_matter_amd import _kernels, _native, prepare_strict_causal_metadata
from white_matter_amd.strict_causal_attention import _keys_unique_code, _schedule_flags, _work_units

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(q, k, v, dout, vis, scale, full_workspace):
    batch, heads, length, dim = q.shape
    o = torch.empty(batch, length, heads, dim, device=DEV, dtype=torch.bfloat16).transpose(1, 2)
    lse = torch.empty(batch, heads, length, device=DEV, dtype=torch.float32)
    dq, dk, dv = (torch.zeros_like(t) for t in (q, k, v))
    delta = torch.empty_like(lse)
    args = _kernels._base_args(q, k, v, o, lse, scale, vis, length)
    _native.attn_fwd(args, q.device)
    args.dout, args.delta = dout.data_ptr(), delta.data_ptr()
    args.do_stride = _kernels._strides(dout)
    args.dq, args.dk, args.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    args.dq_stride, args.dk_stride, args.dv_stride = (_kernels._strides(t) for t in (dq, dk, dv))
    lib = _native.load()
    full = lib.wmx_attn_bwd_workspace_size(ctypes.byref(args))
    least = lib.wmx_attn_bwd_min_workspace_size(ctypes.byref(args))
    need = full if full_workspace else least
    if full_workspace:
        assert full > least, "this shape should have a dS buffer"
    workspace = torch.empty(max(need, 16), device=DEV, dtype=torch.uint8).fill_(0xFF)  # NaN bit patterns
    args.workspace, args.workspace_bytes = workspace.data_ptr(), need
    _native.attn_bwd(args, q.device)
    torch.cuda.synchronize()
    return o, dq, dk, dv


def _inputs(batch, heads, kv_heads, length, dim, seed):
    gen = torch.Generator().manual_seed(seed)
    q = (torch.randn(batch, heads, length, dim, generator=gen) * dim**-0.5).bfloat16().to(DEV)
    k = (torch.randn(batch, kv_heads, length, dim, generator=gen) * dim**-0.5).bfloat16().to(DEV)
    v = torch.randn(batch, kv_heads, length, dim, generator=gen).bfloat16().to(DEV)
    dout = torch.randn(batch, heads, length, dim, generator=gen).bfloat16().to(DEV)
    return q, k, v, dout


def _compare(q, k, v, dout, vis, keep, repeats=0):
    scale = q.shape[-1] ** -0.5
    o1, dq1, dk1, dv1 = _run(q, k, v, dout, vis, scale, True)
    o2, dq2, dk2, dv2 = _run(q, k, v, dout, vis, scale, False)
    assert torch.equal(dk1, dk2) and torch.equal(dv1, dv2)
    for _ in range(repeats):  # the same gradients, bit for bit, on every run
        _, dq3, dk3, dv3 = _run(q, k, v, dout, vis, scale, True)
        assert torch.equal(dq3, dq1) and torch.equal(dk3, dk1) and torch.equal(dv3, dv1)
    assert torch.isfinite(dq1.float()).all()
    qr, kr, vr = (t.double().cpu().requires_grad_() for t in (q, k, v))
    expected = ref.masked_attention(qr, kr, vr, keep.cpu(), scale)
    eq, ek, ev = torch.autograd.grad(expected, (qr, kr, vr), dout.double().cpu())
    for name, a, e in (("dq with dS", dq1, eq), ("dq recomputed", dq2, eq), ("dk", dk1, ek), ("dv", dv1, ev)):
        assert_bf16_close(a, e, what=name)


@pytest.mark.parametrize(("length", "stride", "offset", "dim"), [(256, 1, 0, 128), (200, 2, 3, 64), (333, 1, -1, 96)])
def test_dense_paths_agree(length, stride, offset, dim):
    q, k, v, dout = _inputs(2, 4, 2, length, dim, seed=length)
    vis = _kernels.Visibility(query_stride=stride, query_offset=offset)
    i = torch.arange(length)[:, None]
    j = torch.arange(length)[None, :]
    keep = (j <= offset + stride * i)[None, None]
    _compare(q, k, v, dout, vis, keep)


@pytest.mark.parametrize("length", [300, 1024])
def test_varlen_paths_agree(length):
    batch, heads, dim = 2, 4, 128
    q, k, v, dout = _inputs(batch, heads, heads, length, dim, seed=7)
    docs = torch.cumsum(torch.rand(batch, length, generator=torch.Generator().manual_seed(1)) < 0.01, 1).to(DEV)
    md = prepare_strict_causal_metadata(docs, length)
    max_q, max_k, flags = _schedule_flags(md)
    varlen = _kernels.Varlen(
        md.query_indices, md.key_indices, md.cu_queries, md.cu_keys, md.cu_queries.numel() - 1, max_q, max_k,
        length, length, bool(flags & 16), flags & 15, *_work_units(md),
    )
    meta = {
        "query_indices": md.query_indices.cpu().numpy(),
        "key_indices": md.key_indices.cpu().numpy(),
        "cu_queries": md.cu_queries.cpu().numpy(),
        "cu_keys": md.cu_keys.cpu().numpy(),
        "key_extent": md.key_extent,
    }
    keep = ref.schedule_keep(meta, batch, length, length)[:, None]
    _compare(q, k, v, dout, _kernels.Visibility(varlen=varlen), keep)


@pytest.mark.parametrize(("length", "kv_heads"), [(300, 2), (1024, 4)])
def test_dummy_slot_parts(length, kv_heads):
    """A packed schedule with the leading dummy (only slot 0 repeats across
    segments, keys_unique 2): every segment stores its part of the dummy's
    dK/dV and a second kernel adds them in segment order. Both dQ paths
    against the oracle, the workspace filled with NaN patterns beforehand,
    and the same gradients bit for bit over repeated runs."""
    batch, heads, dim = 3, 4, 128
    gen = torch.Generator().manual_seed(length)
    q = (torch.randn(batch, heads, length, dim, generator=gen) * dim**-0.5).bfloat16().to(DEV)
    k = (torch.randn(batch, kv_heads, length + 1, dim, generator=gen) * dim**-0.5).bfloat16().to(DEV)
    v = torch.randn(batch, kv_heads, length + 1, dim, generator=gen).bfloat16().to(DEV)
    dout = torch.randn(batch, heads, length, dim, generator=gen).bfloat16().to(DEV)
    docs = torch.cumsum(torch.rand(batch, length, generator=gen) < 0.01, 1).to(DEV)
    md = prepare_strict_causal_metadata(docs, length, use_dummy_token=True)
    max_q, max_k, flags = _schedule_flags(md)
    assert _keys_unique_code(flags) == 2 and md.cu_queries.numel() - 1 > batch
    varlen = _kernels.Varlen(
        md.query_indices, md.key_indices, md.cu_queries, md.cu_keys, md.cu_queries.numel() - 1, max_q, max_k,
        length, length + 1, 2, flags & 15, *_work_units(md),
    )
    meta = {
        "query_indices": md.query_indices.cpu().numpy(),
        "key_indices": md.key_indices.cpu().numpy(),
        "cu_queries": md.cu_queries.cpu().numpy(),
        "cu_keys": md.cu_keys.cpu().numpy(),
        "key_extent": md.key_extent,
    }
    keep = ref.schedule_keep(meta, batch, length, length + 1)[:, None]
    assert keep[..., 0].all()
    _compare(q, k, v, dout, _kernels.Visibility(varlen=varlen), keep, repeats=2)


def test_work_list_entries_with_segment_fields_match_pairs():
    """The same packed schedule through work lists of (segment, tile) pairs
    and of entries that carry the segment's bounds (unit_fields 16): the
    kernels take the same values from the entry instead of reading cu_* and
    the index arrays, so every output and gradient is bit-identical."""
    batch, heads, dim, length = 2, 4, 128, 700
    q, k, v, dout = _inputs(batch, heads, 2, length, dim, seed=23)
    docs = torch.cumsum(torch.rand(batch, length, generator=torch.Generator().manual_seed(2)) < 0.01, 1).to(DEV)
    md = prepare_strict_causal_metadata(docs, length)
    max_q, max_k, flags = _schedule_flags(md)
    results = []
    for extent in (None, length):
        units = _work_units(md, query_extent=extent)
        assert units[0].shape[1] == (2 if extent is None else 16)
        varlen = _kernels.Varlen(
            md.query_indices, md.key_indices, md.cu_queries, md.cu_keys, md.cu_queries.numel() - 1, max_q, max_k,
            length, length, bool(flags & 16), flags & 15, *units,
        )
        results.append(_run(q, k, v, dout, _kernels.Visibility(varlen=varlen), dim**-0.5, True))
    # O rows of queries outside every segment are not written by the kernel
    # (the operators zero them): compare the rows the schedule holds
    rows = md.query_indices.long()
    written = [o.transpose(1, 2).reshape(batch * length, heads * dim).index_select(0, rows) for o, *_ in results]
    assert torch.equal(written[0], written[1])
    for a, b in zip(results[0][1:], results[1][1:]):
        assert torch.equal(a, b)
