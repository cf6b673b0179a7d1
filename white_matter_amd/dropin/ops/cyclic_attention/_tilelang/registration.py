"""Reference ops/cyclic_attention/_tilelang/registration.py: the four
registered cyclic operators (names and argument names kept), here on the
gfx950 HIP kernels of libwmx_attn.so."""

from white_matter_amd.cyclic_attention import cyclic_attn_bwd, cyclic_attn_doc_bwd, cyclic_attn_doc_fwd, cyclic_attn_fwd

__all__ = ["cyclic_attn_bwd", "cyclic_attn_doc_bwd", "cyclic_attn_doc_fwd", "cyclic_attn_fwd"]
