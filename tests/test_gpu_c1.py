"""The C1 case (the reference's CPU-runnable configuration) in the GPU session: fp32 cyclic_attention on the
portable backend, (1, 4, 64, 64) queries over 2 KV heads of 256 keys at
query_stride 4, one document; output and gradients of sum(output) within
1e-5 relative L2 of the float64 oracle, on the GPU box's host cores and on
the device (the portable path is plain PyTorch math SDPA on either)."""

import pytest
import torch

from oracle import attention as ref
from white_matter_amd import cyclic_attention

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("device", ["cpu", "cuda"])
def test_config_c1_fp32_cyclic(device):
    gen = torch.Generator().manual_seed(0)
    base = [torch.randn(shape, generator=gen) for shape in ((1, 4, 64, 64), (1, 2, 256, 64), (1, 2, 256, 64))]
    leaves = [t.to(device).requires_grad_() for t in base]
    out = cyclic_attention(*leaves, query_stride=4)
    grads = torch.autograd.grad(out.sum(), leaves)
    ref_leaves = [t.double().requires_grad_() for t in base]
    expected = ref.cyclic_attention(*ref_leaves, query_stride=4)
    ref_grads = torch.autograd.grad(expected.sum(), ref_leaves)
    for a, e in zip((out, *grads), (expected, *ref_grads)):
        assert a.dtype == torch.float32 and a.device.type == device
        assert ((a.double().cpu() - e).norm() / e.norm()).item() < 1e-5
