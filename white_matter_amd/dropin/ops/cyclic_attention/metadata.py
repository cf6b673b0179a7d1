"""Reference ops/cyclic_attention/metadata.py: the document metadata contract."""

from white_matter_amd.metadata import CyclicAttentionMetadata, prepare_cyclic_attention_metadata

__all__ = ["CyclicAttentionMetadata", "prepare_cyclic_attention_metadata"]
