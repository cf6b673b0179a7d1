"""HIP cyclic attention against the oracle (the reference's GPU test matrix,
tests/gpu/test_cyclic_attention.py and test_cyclic_strict_past.py, re-pointed
at the gfx950 kernels). Tolerance: bf16 vs float64 oracle on identical bf16
inputs, rel-L2 <= 5e-3 and max-abs <= 1e-2 * max(1, max|ref|)."""

import pytest
import torch

from oracle import attention as ref
from oracle import metadata as ref_meta
from tests.numerics import assert_bf16_close
from white_matter_amd import cyclic_attention, prepare_cyclic_attention_metadata, prepare_feedback_metadata

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _leaves(*tensors):
    return [t.detach().clone().requires_grad_() for t in tensors]


def _check(q, k, v, options, probe=None, what=""):
    """HIP output and Q/K/V gradients against the float64 oracle."""
    qh, kh, vh = _leaves(q, k, v)
    actual = cyclic_attention(qh, kh, vh, backend="tilelang", **options)
    qr, kr, vr = _leaves(q.double().cpu(), k.double().cpu(), v.double().cpu())
    meta = options.get("metadata")
    meta = None if meta is None else tuple(t.cpu() for t in meta)
    expected = ref.cyclic_attention(
        qr, kr, vr, query_stride=options.get("query_stride", 1), query_offset=options.get("query_offset", 0),
        strict_past=options.get("strict_past", False), metadata=meta,
    )
    if probe is None:
        probe = torch.randn(actual.shape, generator=torch.Generator().manual_seed(5)).to(DEV, torch.bfloat16)
    ga = torch.autograd.grad(actual, (qh, kh, vh), probe)
    ge = torch.autograd.grad(expected, (qr, kr, vr), probe.double().cpu())
    assert_bf16_close(actual, expected, what=f"{what} out")
    for name, a, e in zip("qkv", ga, ge):
        assert_bf16_close(a, e, what=f"{what} d{name}")
    return actual, ga


@pytest.mark.parametrize("gqa_ratio", [1, 2, 3])
@pytest.mark.parametrize("documents", [False, True])
@pytest.mark.parametrize("head_dim", [64, 96, 128])
def test_outputs_and_gradients(documents, head_dim, gqa_ratio):
    torch.manual_seed(23)
    q = torch.randn(2, 2 * gqa_ratio, 33, head_dim, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(2, 2, 132, head_dim, device=DEV, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    metadata = None
    if documents:
        seg = torch.stack((torch.arange(132, device=DEV) // 19, torch.arange(132, device=DEV) // 31))
        metadata = prepare_cyclic_attention_metadata(seg[:, 1::4], torch.cat((seg.new_full((2, 1), -1), seg[:, :-1]), 1))
    actual, _ = _check(q, k, v, {"query_stride": 4, "query_offset": 1, "metadata": metadata}, what="cyclic")
    # (B, Tq, H, D) storage under the (B, H, Tq, D) view
    assert actual.transpose(1, 2).is_contiguous()


@pytest.mark.parametrize("documents", [False, True])
def test_equal_scores_average_exactly(documents):
    q = torch.full((1, 2, 1, 128), 13.0, device=DEV, dtype=torch.bfloat16)
    k = torch.full((1, 1, 4096, 128), 29.0, device=DEV, dtype=torch.bfloat16)
    v = torch.ones_like(k)
    v[:, :, 2048:].neg_()
    metadata = None
    if documents:
        qseg = torch.zeros((1, 1), device=DEV, dtype=torch.long)
        kseg = torch.zeros((1, 4096), device=DEV, dtype=torch.long)
        kseg[:, 0] = -1
        metadata = prepare_cyclic_attention_metadata(qseg, kseg)
    out = cyclic_attention(q, k, v, query_stride=4096, query_offset=4095, metadata=metadata, backend="tilelang")
    assert torch.equal(out, torch.zeros_like(out))


@pytest.mark.parametrize("element_stride", [1, 2])
def test_native_cache_views_match_contiguous(element_stride):
    torch.manual_seed(29)
    q = torch.randn(2, 4, 33, 128, device=DEV, dtype=torch.bfloat16)
    storage = [torch.randn(4, 3, 2, 145, 128 * element_stride, device=DEV, dtype=torch.bfloat16) for _ in range(2)]
    k, v = [t[1:3, 1, :, :132, ::element_stride] for t in storage]
    assert not k.is_contiguous()
    options = {"query_stride": 4, "query_offset": 1, "backend": "tilelang"}
    probe = torch.randn(2, 4, 33, 128, device=DEV, dtype=torch.bfloat16)
    grads = []
    for kk, vv in ((k.contiguous(), v.contiguous()), (k, v)):
        qh, kh, vh = _leaves(q, kk, vv)
        out = cyclic_attention(qh, kh, vh, **options)
        grads.append((out, *torch.autograd.grad(out, (qh, kh, vh), probe)))
    for a, b in zip(*grads):
        assert torch.equal(a, b)


@pytest.mark.parametrize("documents", [False, True])
def test_runtime_shapes(documents):
    torch.manual_seed(47)
    for batch, qlen, kvlen, padding, offset in ((2, 17, 71, 5, 1), (3, 65, 268, 19, 2), (2, 19, 83, 7, 0)):
        q = torch.randn(batch, 4, qlen, 64, device=DEV, dtype=torch.bfloat16)
        k, v = [
            torch.randn(batch, 2, kvlen + extra, 64, device=DEV, dtype=q.dtype)[:, :, :kvlen] for extra in (padding, padding + 3)
        ]
        metadata = None
        if documents:
            qseg = ((offset + 4 * torch.arange(qlen, device=DEV)) // 23).expand(batch, -1).contiguous()
            kseg = ((torch.arange(kvlen, device=DEV) - 1) // 23).expand(batch, -1).contiguous()
            metadata = prepare_cyclic_attention_metadata(qseg, kseg)
        _check(q, k, v, {"query_stride": 4, "query_offset": offset, "metadata": metadata}, what=f"shape {qlen}x{kvlen}")


@pytest.mark.parametrize("documents", [False, True])
def test_invisible_trailing_key_tiles_have_zero_gradients(documents):
    torch.manual_seed(127)
    q = torch.randn(1, 4, 1, 128, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(1, 2, 513, 128, device=DEV, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    metadata = None
    if documents:
        qseg = torch.zeros((1, 1), device=DEV, dtype=torch.int32)
        kseg = torch.zeros((1, 513), device=DEV, dtype=torch.int32)
        kseg[:, 0] = -1
        metadata = prepare_cyclic_attention_metadata(qseg, kseg)
    _, grads = _check(q, k, v, {"query_stride": 4, "query_offset": 0, "metadata": metadata}, what="trailing")
    for g in grads[1:]:
        assert torch.count_nonzero(g[:, :, 1:]) == 0


@pytest.mark.parametrize("misaligned_key", [False, True])
def test_misaligned_cache_pointer(misaligned_key):
    torch.manual_seed(61)
    q = torch.randn(2, 4, 17, 128, device=DEV, dtype=torch.bfloat16)
    shape = (2, 2, 71, 128)
    aligned = torch.randn(shape, device=DEV, dtype=q.dtype)
    misaligned = torch.randn(2 * 2 * 71 * 128 + 1, device=DEV, dtype=q.dtype)[1:].view(shape)
    assert misaligned.data_ptr() % 16 != 0
    k, v = (misaligned, aligned) if misaligned_key else (aligned, misaligned)
    _check(q, k, v, {"query_stride": 4, "query_offset": 1}, what="misaligned")


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("future_documents", [False, True])
def test_document_tile_skipping_keeps_dummy(head_dim, future_documents):
    torch.manual_seed(193)
    batch, query_length, key_length, stride = 2, 129, 1033, 8
    q = torch.randn(batch, 4, query_length, head_dim, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(batch, 2, key_length, head_dim, device=DEV, dtype=q.dtype)
    v = torch.randn_like(k)
    key_ids = torch.stack((torch.arange(key_length, device=DEV) // 257, torch.arange(key_length, device=DEV) // 321))
    key_ids[:, 0] = -1
    query_ids = key_ids[:, : query_length * stride : stride].clamp_min(0)
    if future_documents:
        query_ids = query_ids + 2
    metadata = prepare_cyclic_attention_metadata(query_ids, key_ids)
    actual, grads = _check(q, k, v, {"query_stride": stride, "metadata": metadata}, what="doc skip")
    if future_documents:
        dummy = v[:, :, :1].repeat_interleave(2, dim=1).expand_as(q)
        assert torch.equal(actual, dummy)
        assert torch.count_nonzero(grads[2][:, :, 1:]) == 0


@pytest.mark.parametrize("documents", [False, True])
@pytest.mark.parametrize("query_length", [1, 17, 33])
def test_short_queries_ignore_future_cache(documents, query_length):
    torch.manual_seed(107)
    stride, offset, kv_length = 8, 3, 2048
    q = torch.randn(2, 4, query_length, 128, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(2, 2, kv_length, 128, device=DEV, dtype=q.dtype)
    v = torch.randn_like(k)
    metadata = None
    if documents:
        pos = torch.arange(kv_length, device=DEV)
        key_ids = torch.stack((pos // 97, pos // 113)).to(torch.int32)
        key_ids[:, 0] = -1
        qpos = torch.arange(query_length, device=DEV) * stride + offset
        metadata = prepare_cyclic_attention_metadata(key_ids[:, qpos], key_ids)
    _, grads = _check(q, k, v, {"query_stride": stride, "query_offset": offset, "metadata": metadata}, what="short")
    first_future = offset + stride * (query_length - 1) + 1
    for g in grads[1:]:
        assert torch.count_nonzero(g[:, :, first_future:]) == 0


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("stride", [1, 4])
@pytest.mark.parametrize("dummy", [False, True])
def test_strict_past_residues(packed, stride, dummy):
    torch.manual_seed(71)
    length = 137
    docs = torch.arange(length, device=DEV)[None].expand(2, -1).clone() // 11
    docs[1] = torch.arange(length, device=DEV) // 3
    groups = [torch.arange(r, length, stride, device=DEV) for r in range(stride)]
    metadata = prepare_feedback_metadata(docs, groups, length, use_dummy_token=dummy) if packed else None
    for residue, slots in enumerate(groups):
        q = torch.randn(2, 4, slots.numel(), 64, device=DEV, dtype=torch.bfloat16)
        k = torch.randn(2, 2, length, 64, device=DEV, dtype=torch.bfloat16)
        v = torch.randn_like(k)
        options = {
            "query_stride": stride,
            "query_offset": residue,
            "strict_past": not dummy,
            "metadata": None if metadata is None else metadata[residue],
        }
        _check(q, k, v, options, what=f"strict residue {residue}")


def test_backward_preprocess_matches_fp64():
    from white_matter_amd import _kernels

    torch.manual_seed(81)
    for transposed in (False, True):
        for head_dim in (64, 96, 128):
            shape = (2, 3, 33, head_dim)
            dout = torch.randn(shape, device=DEV, dtype=torch.bfloat16)
            out = torch.randn((2, 33, 3, head_dim) if transposed else shape, device=DEV, dtype=torch.bfloat16)
            if transposed:
                out = out.transpose(1, 2)
            actual = _kernels.row_dot(dout, out)
            prod = dout.double() * out.double()
            bound = torch.finfo(torch.float32).eps * head_dim * prod.abs().sum(-1)
            assert torch.all((actual.double() - prod.sum(-1)).abs() <= bound)


def test_feedback_metadata_matches_oracle_on_gpu():
    torch.manual_seed(17)
    segments = torch.randint(0, 2, (2, 33)).cumsum(1).to(DEV)
    positions = [torch.arange(r, 33, 4, device=DEV) for r in range(4)]
    actual = prepare_feedback_metadata(segments, positions, 33)
    expected = ref_meta.feedback_metadata(segments.cpu().numpy(), [p.cpu().numpy() for p in positions], 33)
    for a, e in zip(actual, expected):
        for ta, te in zip(a, e):
            assert ta.dtype == torch.int32 and (ta.cpu().numpy() == te).all()


@pytest.mark.parametrize("dummy", [False, True])
def test_cyclic_metadata_matches_oracle_on_gpu(dummy):
    """prepare_cyclic_attention_metadata on device tensors, bit for bit against
    the oracle's row-wise searches (reference metadata.py:17-56), int32 and
    int64 ids, ragged id runs and repeated ids."""
    gen = torch.Generator().manual_seed(23 + int(dummy))
    for trial in range(16):
        batch = 1 + trial % 3
        q_len = int(torch.randint(1, 300, (1,), generator=gen))
        k_len = int(torch.randint(2, 700, (1,), generator=gen))
        q_ids = torch.randint(0, 3, (batch, q_len), generator=gen).cumsum(1)
        k_ids = torch.randint(0, 2, (batch, k_len), generator=gen).cumsum(1)
        if dummy:
            k_ids[:, 0] = -1
        dtype = torch.int32 if trial % 2 else torch.int64
        actual = prepare_cyclic_attention_metadata(q_ids.to(DEV, dtype), k_ids.to(DEV, dtype), use_dummy_token=dummy)
        expected = ref_meta.cyclic_metadata(q_ids.numpy(), k_ids.numpy(), use_dummy_token=dummy)
        for a, e in zip(actual, expected):
            assert a.device.type == "cuda" and a.dtype == torch.int32
            assert (a.cpu().numpy() == e).all(), f"trial {trial}"
