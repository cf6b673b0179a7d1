"""Reference ops/cyclic_attention/_tilelang/backward_preprocess.py: the
backward's row reduction delta = sum(dout * out, -1) in fp32, here the
HIP delta kernel (wmx_attn_bwd_preprocess)."""

import torch

from white_matter_amd._kernels import row_dot


def backward_preprocess(dout: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """(B, H, Q) fp32 row sums of dout * out for (B, H, Q, D) operands."""
    return row_dot(dout, out)


__all__ = ["backward_preprocess"]
