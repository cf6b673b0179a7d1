"""white_matter.ops on the gfx950 HIP kernels (reference src/white_matter/ops/__init__.py:3-13)."""

from white_matter_amd import (
    CyclicAttentionMetadata,
    StrictCausalMetadata,
    cyclic_attention,
    prepare_cyclic_attention_metadata,
    prepare_strict_causal_metadata,
    strict_causal_attention,
)

__all__ = [
    "StrictCausalMetadata",
    "prepare_strict_causal_metadata",
    "strict_causal_attention",
    "CyclicAttentionMetadata",
    "cyclic_attention",
    "prepare_cyclic_attention_metadata",
]
