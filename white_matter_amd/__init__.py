"""WhiteMatter's attention hot path on MI355X (gfx950).

Drop-in replacement for ``white_matter.ops`` (src/white_matter/ops/__init__.py:3-13):
the same six public names with the same signatures, the FlashAttention entry
points of ``white_matter.ops.flash_attention`` (``flash_attention``), plus the model-side
``prepare_feedback_metadata``, the fused KV-pool store (``kv_pool``) and the
captured decode step (``DecodeLoop``). GPU work runs in hand-written HIP kernels
loaded from ``lib/libwmx_attn.so`` through a C ABI (include/wmx_attn.h).
"""

from . import flash_attention, kv_pool
from .cyclic_attention import cyclic_attention
from .decode_loop import DecodeLoop
from .metadata import CyclicAttentionMetadata, prepare_cyclic_attention_metadata, prepare_feedback_metadata
from .strict_causal_attention import StrictCausalMetadata, prepare_strict_causal_metadata, strict_causal_attention

__all__ = [
    "StrictCausalMetadata",
    "prepare_strict_causal_metadata",
    "strict_causal_attention",
    "CyclicAttentionMetadata",
    "cyclic_attention",
    "prepare_cyclic_attention_metadata",
    "prepare_feedback_metadata",
    "DecodeLoop",
    "flash_attention",
    "kv_pool",
]
