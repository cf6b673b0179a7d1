"""white_matter.ops.strict_causal_attention on the gfx950 HIP kernels
(reference src/white_matter/ops/strict_causal_attention.py), with the
module-level names its callers and tests reach."""

from white_matter_amd.flash_attention import (
    TorchFlashDense,
    TorchFlashVarlen,
    can_use_torch_flash,
    flash_attention_decode,
    torch_flash_decode,
)
from white_matter_amd.strict_causal_attention import (
    StrictCausalMetadata,
    _standalone_flash_available,
    prepare_strict_causal_metadata,
    strict_causal_attention,
)

__all__ = [
    "StrictCausalMetadata",
    "TorchFlashDense",
    "TorchFlashVarlen",
    "_standalone_flash_available",
    "can_use_torch_flash",
    "flash_attention_decode",
    "prepare_strict_causal_metadata",
    "strict_causal_attention",
    "torch_flash_decode",
]
