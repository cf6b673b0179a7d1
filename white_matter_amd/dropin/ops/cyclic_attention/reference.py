"""Reference ops/cyclic_attention/reference.py: the portable math backend."""

from white_matter_amd.portable import cyclic_attention_portable as cyclic_attention_reference

__all__ = ["cyclic_attention_reference"]
