"""white_matter.ops.cyclic_attention on the gfx950 HIP kernels (reference
src/white_matter/ops/cyclic_attention/__init__.py)."""

from white_matter_amd.cyclic_attention import cyclic_attention
from white_matter_amd.metadata import CyclicAttentionMetadata, prepare_cyclic_attention_metadata

__all__ = ["CyclicAttentionMetadata", "cyclic_attention", "prepare_cyclic_attention_metadata"]
