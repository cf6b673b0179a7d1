"""Decode over the KV pool at GQA ratios 1-8, 12 and 16 and at the C4 shape,
and the reference's FlashAttention-layout entry points, against the float64
oracle (bf16 vs float64: max-abs <= 1e-2 * max(1, max|ref|), rel-L2 <= 5e-3).

C4 decode runs decode_split_kernel at G = Hq/Hkv = 1 (Hkv = 16) and 2
(Hkv = 8); the split count is the heuristic's (several splits and the
combine kernel) or forced to one (the split kernel writes the output)."""

import numpy as np
import pytest
import torch

from oracle import attention as ref
from tests.numerics import assert_bf16_close
from white_matter_amd import strict_causal_attention
from white_matter_amd.flash_attention import (
    TorchFlashDense,
    TorchFlashVarlen,
    flash_attention_decode,
    torch_flash_decode,
)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _normal(shape, gen, dim=None):
    x = torch.randn(shape, generator=gen)
    return (x * dim**-0.5 if dim else x).to(DEV, torch.bfloat16)


@pytest.mark.parametrize("num_splits", [1, 0])
@pytest.mark.parametrize("group", [1, 2, 4, 8])
@torch.no_grad()
def test_decode_group_sizes(group, num_splits):
    gen = torch.Generator().manual_seed(100 + group)
    batch, heads, capacity, dim = 4, 16, 3000, 128
    q = _normal((batch, heads, 1, dim), gen)
    k = _normal((batch, heads // group, capacity, dim), gen)
    v = _normal((batch, heads // group, capacity, dim), gen)
    lengths = torch.tensor([0, 1, 1777, 3000])
    for b in range(batch):
        k[b, :, int(lengths[b]) :] = float("nan")
        v[b, :, int(lengths[b]) :] = float("nan")
    out = strict_causal_attention(q, k, v, query_start=lengths.to(DEV), kv_lengths=lengths.to(DEV), num_splits=num_splits)
    expected = ref.strict_attention(q.cpu(), k.cpu(), v.cpu(), query_start=lengths, kv_lengths=lengths)
    assert_bf16_close(out, expected, what=f"decode G={group} splits={num_splits}")
    assert out[0].count_nonzero() == 0


@pytest.mark.parametrize("num_splits", [1, 0])
@pytest.mark.parametrize("group", [3, 5, 6, 7, 12, 16])
@torch.no_grad()
def test_decode_any_group_size(group, num_splits):
    """GQA ratios beyond powers of two (one workgroup serves up to 8 query
    heads of a KV head; 12 and 16 heads take two launches over the same rows),
    with head_dim 64 and 96 as well."""
    gen = torch.Generator().manual_seed(200 + group)
    for dim in (128, 64, 96):
        batch, kv_heads, capacity = 3, 2, 700
        q = _normal((batch, kv_heads * group, 1, dim), gen)
        k = _normal((batch, kv_heads, capacity, dim), gen)
        v = _normal((batch, kv_heads, capacity, dim), gen)
        lengths = torch.tensor([5, 700, 333])
        for b in range(batch):
            k[b, :, int(lengths[b]) :] = float("nan")
            v[b, :, int(lengths[b]) :] = float("nan")
        out = strict_causal_attention(q, k, v, query_start=lengths.to(DEV), num_splits=num_splits)
        expected = ref.strict_attention(q.cpu(), k.cpu(), v.cpu(), query_start=lengths)
        assert_bf16_close(out, expected, what=f"decode G={group} D={dim} splits={num_splits}")


@pytest.mark.parametrize("kv_heads", [16, 8])
@torch.no_grad()
def test_c4_decode_full_shape(kv_heads):
    batch, heads, dim = 32, 16, 128
    print(f"C4 decode full shape: B=32 Hq=16 Hkv={kv_heads} D=128, lengths ~U[512,8192]", flush=True)
    lengths = torch.from_numpy(np.random.default_rng(1).integers(512, 8192, size=batch, endpoint=True))
    capacity = 8192
    gen = torch.Generator().manual_seed(1)
    q = _normal((batch, heads, 1, dim), gen, dim)
    k = torch.empty(batch, kv_heads, capacity, dim, device=DEV, dtype=torch.bfloat16).normal_(0, dim**-0.5)
    v = torch.empty_like(k).normal_(0, dim**-0.5)
    out = strict_causal_attention(q, k, v, query_start=lengths.to(DEV), kv_lengths=lengths.to(DEV))
    expected = ref.strict_attention(q.cpu(), k.cpu(), v.cpu(), query_start=lengths, kv_lengths=lengths)
    assert_bf16_close(out, expected, what=f"C4 decode Hkv={kv_heads}")


def _fa_keep(lengths, count, slots, causal):
    """(B, 1, Sq, N): slot j visible to query s iff j < len (and, causal,
    j <= len - Sq + s), flash_attn_with_kvcache's cache_seqlens contract."""
    j = torch.arange(slots)[None, None, :]
    length = lengths[:, None, None]
    keep = j < length
    if causal:
        keep = keep & (j <= length - count + torch.arange(count)[None, :, None])
    return keep[:, None]


@pytest.mark.parametrize("dim", [64, 80, 128])
@pytest.mark.parametrize(("count", "causal"), [(1, True), (1, False), (5, True), (5, False), (300, True)])
@torch.no_grad()
def test_flash_attention_decode_layout(count, causal, dim):
    """white_matter::flash_attention_decode in its own layout: query
    (B, Sq, H, D), caches (B, N, Hkv, D), lengths (B,) int32."""
    gen = torch.Generator().manual_seed(count + dim)
    batch, heads, kv_heads, slots = 3, 8, 2, 700
    query = _normal((batch, count, heads, dim), gen)
    key = _normal((batch, slots, kv_heads, dim), gen)
    value = _normal((batch, slots, kv_heads, dim), gen)
    lengths = torch.tensor([0, 301, 700], dtype=torch.int32)
    out = flash_attention_decode(query, key, value, lengths.to(DEV), dim**-0.5, causal)
    assert out.shape == query.shape and out.dtype == query.dtype
    keep = _fa_keep(lengths.long(), count, slots, causal)
    expected = ref.masked_attention(
        query.transpose(1, 2).cpu(), key.transpose(1, 2).cpu(), value.transpose(1, 2).cpu(), keep, dim**-0.5
    ).transpose(1, 2)
    assert_bf16_close(out, expected, what=f"flash_attention_decode Sq={count} causal={causal} D={dim}")
    # the op is also reachable by its registered name
    again = torch.ops.white_matter.flash_attention_decode(query, key, value, lengths.to(DEV), dim**-0.5, causal, 0)
    assert torch.equal(again, out)


@torch.no_grad()
def test_torch_flash_decode_channel_view():
    gen = torch.Generator().manual_seed(7)
    batch, heads, dim = 3, 8, 64
    pool = _normal((batch, 8, 500, dim), gen)
    k, v = pool[:, :2], pool[:, 4:6]
    q = _normal((batch, heads, 1, dim), gen)
    lengths = torch.tensor([5, 0, 500], dtype=torch.int32)
    out = torch_flash_decode(q, k, v, lengths.to(DEV), 0.3)
    assert out.shape == (batch, 1, heads, dim)
    keep = (torch.arange(500)[None, :] < lengths[:, None].long())[:, None, None]
    expected = ref.masked_attention(q.cpu(), k.cpu(), v.cpu(), keep, 0.3).transpose(1, 2)
    assert_bf16_close(out, expected, what="torch_flash_decode")


@pytest.mark.parametrize("causal", [True, False])
def test_torch_flash_dense_bottom_right(causal):
    gen = torch.Generator().manual_seed(9)
    q = _normal((2, 4, 40, 64), gen).requires_grad_()
    k = _normal((2, 2, 100, 64), gen).requires_grad_()
    v = _normal((2, 2, 100, 64), gen).requires_grad_()
    out = TorchFlashDense.apply(q, k, v, 0.125, causal)
    assert out.shape == (2, 40, 4, 64) and out.is_contiguous()
    i, j = torch.arange(40)[:, None], torch.arange(100)[None, :]
    keep = (j <= i + 60) if causal else torch.ones(40, 100, dtype=torch.bool)
    leaves = [t.detach().cpu().double().requires_grad_() for t in (q, k, v)]
    expected = ref.masked_attention(*leaves, keep[None, None], 0.125).transpose(1, 2)
    assert_bf16_close(out, expected, what="TorchFlashDense out")
    probe = _normal(out.shape, gen)
    ga = torch.autograd.grad(out, (q, k, v), probe)
    ge = torch.autograd.grad(expected, leaves, probe.cpu().double())
    for name, a, e in zip("qkv", ga, ge):
        assert_bf16_close(a, e, what=f"TorchFlashDense d{name}")


def test_torch_flash_varlen_packed_segments():
    gen = torch.Generator().manual_seed(10)
    cu_q = torch.tensor([0, 3, 3, 40, 41], dtype=torch.int32)
    cu_k = torch.tensor([0, 5, 9, 70, 71], dtype=torch.int32)
    q = _normal((41, 4, 64), gen).requires_grad_()
    k = _normal((71, 2, 64), gen).requires_grad_()
    v = _normal((71, 2, 64), gen).requires_grad_()
    out = TorchFlashVarlen.apply(q, k, v, cu_q.to(DEV), cu_k.to(DEV), 37, 61, 0.125)
    keep = torch.zeros(41, 71, dtype=torch.bool)
    for s in range(4):
        qs, qe, ks, ke = int(cu_q[s]), int(cu_q[s + 1]), int(cu_k[s]), int(cu_k[s + 1])
        for a in range(qe - qs):
            keep[qs + a, ks : ks + (ke - ks) - (qe - qs) + a + 1] = True
    leaves = [t.detach().cpu().double().requires_grad_() for t in (q, k, v)]
    expected = ref.masked_attention(*(t.transpose(0, 1)[None] for t in leaves), keep[None, None], 0.125)[0].transpose(0, 1)
    assert_bf16_close(out, expected, what="TorchFlashVarlen out")
    probe = _normal(out.shape, gen)
    ga = torch.autograd.grad(out, (q, k, v), probe)
    ge = torch.autograd.grad(expected, leaves, probe.cpu().double())
    for name, a, e in zip("qkv", ga, ge):
        assert_bf16_close(a, e, what=f"TorchFlashVarlen d{name}")


@pytest.mark.parametrize(("batch", "kv_heads", "group", "dim"), [(3, 5, 1, 128), (4, 2, 12, 64), (32, 16, 1, 128), (7, 3, 2, 96)])
@torch.no_grad()
def test_merge_by_last_split_matches_combine_kernel(batch, kv_heads, group, dim):
    """The operator's decode merges the splits in the last split to finish
    (counters kept per stream); the C ABI call without counters runs the
    separate combine kernel. Same terms in the same order: bit-identical, on
    repeated calls (each launch leaves its counters zero), for row and KV-head
    counts that spread one row's splits over several XCDs (batch * kv_heads
    not a multiple of 8) and for groups of more than 8 heads (two launches
    sharing the counters)."""
    from white_matter_amd import _kernels

    gen = torch.Generator().manual_seed(batch * 100 + kv_heads * 10 + group)
    heads, capacity = kv_heads * group, 5000
    q = _normal((batch, heads, 1, dim), gen, dim)
    k = _normal((batch, kv_heads, capacity, dim), gen, dim)
    v = _normal((batch, kv_heads, capacity, dim), gen, dim)
    lengths = torch.randint(0, capacity + 1, (batch,), generator=gen).to(DEV)
    for call in range(3):
        print(f"last-split merge B={batch} Hkv={kv_heads} G={group} D={dim} call {call}", flush=True)
        merged = strict_causal_attention(q, k, v, query_start=lengths, kv_lengths=lengths)
        combined = torch.empty(batch, heads, dim, device=DEV, dtype=torch.bfloat16)
        _kernels.decode(q, k, v, combined, query_start=lengths, kv_lengths=lengths, key_mask=None, use_dummy=False,
                        scale=dim**-0.5)
        assert torch.equal(merged[:, 0], combined)
    expected = ref.strict_attention(q.cpu(), k.cpu(), v.cpu(), query_start=lengths.cpu(), kv_lengths=lengths.cpu())
    assert_bf16_close(merged, expected, what="last-split merge")


@pytest.mark.parametrize(("batch", "kv_heads", "group", "dim"), [(8, 8, 2, 64), (5, 3, 4, 128), (1, 2, 1, 96)])
@torch.no_grad()
def test_shared_length_and_decode_out(batch, kv_heads, group, dim):
    """A one-element length tensor serves every row in place (the operator
    passes it to wmx_decode with lengths_broadcast instead of copying it per
    row) and strict_decode_out writes into a caller's buffer: both give the
    per-row call's bits; a length tensor of another size is refused."""
    from white_matter_amd.strict_causal_attention import strict_decode, strict_decode_out

    gen = torch.Generator().manual_seed(batch + 10 * kv_heads + dim)
    heads, capacity = kv_heads * group, 1153
    q = _normal((batch, heads, 1, dim), gen, dim)
    k = _normal((batch, kv_heads, capacity, dim), gen, dim)
    v = _normal((batch, kv_heads, capacity, dim), gen, dim)
    for length in (1, 700, capacity):
        print(f"shared length B={batch} Hkv={kv_heads} G={group} D={dim} length {length}", flush=True)
        one = torch.tensor([length], device=DEV)
        rows = one.expand(batch).contiguous()
        want = strict_decode(q, k, v, rows, 0, rows, None, False, dim**-0.5, 0)
        got = strict_decode(q, k, v, one, 0, one, None, False, dim**-0.5, 0)
        assert torch.equal(got, want), f"length {length}: shared length differs from per-row lengths"
        out = torch.full((2, batch, 1, heads, dim), float("nan"), device=DEV, dtype=torch.bfloat16)
        strict_decode_out(out[1], q, k, v, one, 0, one, None, False, dim**-0.5, 0)
        assert torch.equal(out[1], want) and bool(out[0].isnan().all())
        # the dummy-slot form of the same visible length: length - 1 real keys plus the dummy
        dummy = strict_decode(q, k, v, rows - 1, 0, rows - 1, None, True, dim**-0.5, 0)
        assert torch.equal(dummy, want)
    if batch > 1:
        with pytest.raises(ValueError, match="kv_lengths"):
            strict_decode(q, k, v, rows, 0, one, None, False, dim**-0.5, 0)
