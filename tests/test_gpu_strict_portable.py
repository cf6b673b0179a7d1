"""strict_causal_attention(backend="reference") in the GPU session: the
portable path (reference strict_causal_attention.py:279-322,362-373: the dense
strict mask or the varlen per-segment schedule, then math SDPA) in fp32 on
the GPU box's host cores and on the device, against the per-query float64
oracle (which builds no schedule) at 1e-5 relative L2, for the output and the
gradients of a random probe. Cases: a cached prefix, the dummy slot, packed
documents (with padding ids), kv_lengths caps, GQA."""

import pytest
import torch

from oracle import attention as ref
from white_matter_amd import prepare_strict_causal_metadata, strict_causal_attention

pytestmark = pytest.mark.gpu

CASES = [
    # (prefix, count, dummy, documents, capped)
    (0, 48, False, False, False),
    (0, 48, True, False, False),
    (17, 32, False, False, False),
    (17, 32, True, False, True),
    (0, 64, False, True, False),
    (0, 64, True, True, False),
    (9, 40, False, True, True),
    (9, 40, True, True, True),
]


def _documents(batch, slots, gen):
    docs = torch.empty(batch, slots, dtype=torch.long)
    for b in range(batch):
        cuts = sorted(torch.randperm(slots - 1, generator=gen)[:3].add(1).tolist())
        ids = torch.zeros(slots, dtype=torch.long)
        for c in cuts:
            ids[c:] += 1
        docs[b] = ids
    docs[1, 5:7] = -1  # padding slots inside a run do not break it
    return docs


@pytest.mark.parametrize("device", ["cpu", "cuda"])
@pytest.mark.parametrize(("prefix", "count", "dummy", "documents", "capped"), CASES)
def test_portable_strict_fp32_matches_per_query_oracle(device, prefix, count, dummy, documents, capped):
    gen = torch.Generator().manual_seed(1000 + 37 * prefix + count + 3 * dummy + 5 * documents + 7 * capped)
    batch, heads, kv_heads, dim = 2, 4, 2, 64
    slots = prefix + count
    base = [
        torch.randn(batch, heads, count, dim, generator=gen),
        torch.randn(batch, kv_heads, slots + int(dummy), dim, generator=gen),
        torch.randn(batch, kv_heads, slots + int(dummy), dim, generator=gen),
    ]
    starts = torch.full((batch,), prefix)
    lengths = torch.tensor([slots - 5, slots - 11]) if capped else None
    docs = _documents(batch, slots, gen) if documents else None
    leaves = [t.to(device).requires_grad_() for t in base]
    metadata = None
    if docs is not None:
        metadata = prepare_strict_causal_metadata(
            docs.to(device), count, query_start=prefix, use_dummy_token=dummy,
            kv_lengths=None if lengths is None else lengths.to(device),
        )
    out = strict_causal_attention(
        *leaves, query_start=prefix, kv_lengths=None if (lengths is None or metadata is not None) else lengths.to(device),
        use_dummy_token=dummy, metadata=metadata, backend="reference",
    )
    probe = torch.randn(out.shape, generator=gen)
    grads = torch.autograd.grad(out, leaves, probe.to(device))
    ref_leaves = [t.double().requires_grad_() for t in base]
    expected = ref.per_query_strict(*ref_leaves, starts, dummy, docs, lengths)
    ref_grads = torch.autograd.grad(expected, ref_leaves, probe.double())
    for name, a, e in zip(("out", "dq", "dk", "dv"), (out, *grads), (expected, *ref_grads)):
        assert a.dtype == torch.float32 and a.device.type == device, name
        err = ((a.double().cpu() - e).norm() / e.norm().clamp_min(1e-30)).item()
        assert err < 1e-5, f"{name}: rel-L2 {err:.3e}"
