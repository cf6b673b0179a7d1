"""white_matter.ops.flash_attention on the gfx950 HIP kernels (reference
src/white_matter/ops/flash_attention.py): the decode operator, the dense
forward operator and the autograd functions the model's readers import."""

from white_matter_amd.flash_attention import (
    TorchFlashDense,
    TorchFlashVarlen,
    can_use_torch_flash,
    flash_attention_decode,
    torch_flash_decode,
)
from white_matter_amd.flash_attention import torch_flash_dense_forward as _torch_flash_dense_forward

__all__ = [
    "TorchFlashDense",
    "TorchFlashVarlen",
    "_torch_flash_dense_forward",
    "can_use_torch_flash",
    "flash_attention_decode",
    "torch_flash_decode",
]
