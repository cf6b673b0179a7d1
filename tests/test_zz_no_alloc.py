"""wmx_decode_noalloc (the allocation-free decode entry point) through the C
ABI: on two calls in a row, the second with a smaller input, its output is
bit-identical to wmx_decode's with a caller-allocated workspace (both run the
same kernels; only where the split-K partials live differs), and where the
split count wmx_decode would use needs more partials than the static scratch
holds, it runs the largest count that fits: bit-identical to wmx_decode at
that count, within the bf16 bar of wmx_decode at its own."""

import ctypes

import pytest
import torch

from white_matter_amd import _native

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _args(q, k, v, out, lengths, num_splits):
    a = _native.DecodeArgs()
    a.q, a.k, a.v, a.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    a.q_stride = (q.stride(0), q.stride(1))
    a.k_stride = (k.stride(0), k.stride(1), k.stride(2))
    a.v_stride = (v.stride(0), v.stride(1), v.stride(2))
    a.o_stride = (out.stride(0), out.stride(1))
    a.query_start = lengths.data_ptr()
    a.batch, a.q_heads, a.kv_heads = q.shape[0], q.shape[1], k.shape[1]
    a.capacity, a.head_dim = k.shape[2], q.shape[3]
    a.num_splits = num_splits
    a.softmax_scale = q.shape[3] ** -0.5
    return a


def _case(batch, heads, kv_heads, capacity, dim, num_splits, seed):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, heads, 1, dim, generator=gen).to(DEV, torch.bfloat16)
    pool_k = torch.randn(batch, 2 * kv_heads, capacity, dim, generator=gen).to(DEV, torch.bfloat16)
    pool_v = torch.randn(batch, 2 * kv_heads, capacity, dim, generator=gen).to(DEV, torch.bfloat16)
    k, v = pool_k[:, kv_heads:], pool_v[:, kv_heads:]  # a channel view of a pool, read in place
    lengths = torch.randint(0, capacity + 1, (batch,), generator=gen).to(DEV)
    return q, k, v, lengths, num_splits


def _both(q, k, v, lengths, num_splits):
    lib = _native.load()
    stream = torch.cuda.current_stream().cuda_stream
    ref = torch.full((q.shape[0], q.shape[1], q.shape[3]), float("nan"), device=DEV, dtype=torch.bfloat16)
    a = _args(q, k, v, ref, lengths, num_splits)
    need = int(lib.wmx_decode_workspace_size(ctypes.byref(a)))
    workspace = torch.empty(max(need, 16), device=DEV, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = workspace.data_ptr(), need
    assert lib.wmx_decode(ctypes.byref(a), stream) == 0, lib.wmx_last_error()
    out = torch.full_like(ref, float("nan"))
    b = _args(q, k, v, out, lengths, num_splits)
    assert lib.wmx_decode_noalloc(ctypes.byref(b), stream) == 0, lib.wmx_last_error()
    torch.cuda.synchronize()
    return ref, out, int(lib.wmx_decode_num_splits(ctypes.byref(a)))


def test_noalloc_matches_wmx_decode_on_two_calls():
    cases = [
        _case(batch=6, heads=16, kv_heads=4, capacity=5000, dim=128, num_splits=0, seed=1),
        _case(batch=2, heads=8, kv_heads=8, capacity=700, dim=64, num_splits=3, seed=2),  # smaller
    ]
    for i, case in enumerate(cases):
        print(f"no-alloc decode call {i}: q {tuple(case[0].shape)} kv {tuple(case[1].shape)}", flush=True)
        ref, out, splits = _both(*case)
        assert splits > 1, "the case must run the split-K partials through the scratch"
        assert torch.isfinite(ref.float()).all()
        assert torch.equal(out, ref), f"call {i}: wmx_decode_noalloc differs from wmx_decode"


def _decode(q, k, v, lengths, num_splits, noalloc):
    lib = _native.load()
    out = torch.full((q.shape[0], q.shape[1], q.shape[3]), float("nan"), device=DEV, dtype=torch.bfloat16)
    a = _args(q, k, v, out, lengths, num_splits)
    workspace = None
    if not noalloc:
        need = int(lib.wmx_decode_workspace_size(ctypes.byref(a)))
        workspace = torch.empty(max(need, 16), device=DEV, dtype=torch.uint8)
        a.workspace, a.workspace_bytes = workspace.data_ptr(), need
    entry = lib.wmx_decode_noalloc if noalloc else lib.wmx_decode
    assert entry(ctypes.byref(a), torch.cuda.current_stream().cuda_stream) == 0, lib.wmx_last_error()
    torch.cuda.synchronize()
    return out, a


@pytest.mark.parametrize("requested", [0, 2000])
def test_noalloc_clamps_splits_to_the_scratch(requested):
    # 8 rows x 64 query heads x (128 + 2) floats = 266,240 bytes per split:
    # 31 splits fit the 8 MiB scratch; a 33,792-slot cache asks for 33 splits
    # by default (1024 keys a split), and 2000 are asked for explicitly
    print(f"no-alloc clamp case: requested splits {requested}", flush=True)
    gen = torch.Generator().manual_seed(4)
    batch, heads, kv_heads, capacity, dim = 8, 64, 8, 33 * 1024, 128
    q = torch.randn(batch, heads, 1, dim, generator=gen).to(DEV, torch.bfloat16)
    k = torch.empty(batch, kv_heads, capacity, dim, device=DEV, dtype=torch.bfloat16).normal_(0, 1)
    v = torch.empty_like(k).normal_(0, 1)
    lengths = torch.randint(capacity // 2, capacity + 1, (batch,), generator=gen).to(DEV)
    lib = _native.load()
    per_split = batch * heads * (dim + 2) * 4
    fit = _native.DECODE_NOALLOC_MAX_BYTES // per_split
    out, a = _decode(q, k, v, lengths, requested, noalloc=True)
    natural = int(lib.wmx_decode_num_splits(ctypes.byref(a)))
    assert natural > fit == 31, "the case must ask for more partials than the scratch holds"
    same, _ = _decode(q, k, v, lengths, fit, noalloc=False)
    assert torch.equal(out, same), "the clamped call must equal wmx_decode at the clamped split count"
    full, _ = _decode(q, k, v, lengths, requested, noalloc=False)
    assert torch.isfinite(out.float()).all()
    assert (out.float() - full.float()).abs().max().item() < 1e-2
