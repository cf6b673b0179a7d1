"""Reference ops/cyclic_attention/functional.py: the public operator."""

from white_matter_amd.cyclic_attention import cyclic_attention

__all__ = ["cyclic_attention"]
