"""ctypes binding of libwmx_attn.so (the C ABI in include/wmx_attn.h).

The structures below mirror ``wmx_attn_args`` and ``wmx_decode_args`` field by
field; ``load()`` checks their sizes against the library's own ``sizeof`` so a
header/binding mismatch fails at load time instead of corrupting a launch.
Nothing here falls back to another implementation: when the library is
missing or fails to load, every entry point raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import functools
import os
from pathlib import Path

import torch

LIBRARY = Path(__file__).resolve().parent / "lib" / "libwmx_attn.so"
# the operators registered from C++ (csrc/torch_ops.cpp), linked against LIBRARY
OPS_LIBRARY = Path(__file__).resolve().parent / "lib" / "libwmx_torch.so"
ABI_VERSION = 13

_c_i64_3 = ctypes.c_int64 * 3
_c_i64_2 = ctypes.c_int64 * 2
_vp = ctypes.c_void_p


class AttnArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp),
        ("k", _vp),
        ("v", _vp),
        ("o", _vp),
        ("lse", _vp),
        ("dout", _vp),
        ("delta", _vp),
        ("dq", _vp),
        ("dk", _vp),
        ("dv", _vp),
        ("workspace", _vp),
        ("workspace_bytes", ctypes.c_int64),
        ("q_stride", _c_i64_3),
        ("k_stride", _c_i64_3),
        ("v_stride", _c_i64_3),
        ("o_stride", _c_i64_3),
        ("do_stride", _c_i64_3),
        ("dq_stride", _c_i64_3),
        ("dk_stride", _c_i64_3),
        ("dv_stride", _c_i64_3),
        ("batch", ctypes.c_int32),
        ("q_heads", ctypes.c_int32),
        ("kv_heads", ctypes.c_int32),
        ("q_len", ctypes.c_int32),
        ("kv_len", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("query_stride", ctypes.c_int32),
        ("query_offset", ctypes.c_int32),
        ("row_offset", _vp),
        ("row_limit", _vp),
        ("key_mask", _vp),
        ("key_mask_stride", ctypes.c_int64),
        ("keep_slot0", ctypes.c_int32),
        ("keys_unique", ctypes.c_int32),
        ("q_seg", _vp),
        ("k_seg", _vp),
        ("q_start", _vp),
        ("k_qend", _vp),
        ("query_indices", _vp),
        ("key_indices", _vp),
        ("cu_queries", _vp),
        ("cu_keys", _vp),
        ("num_segments", ctypes.c_int32),
        ("max_queries", ctypes.c_int32),
        ("max_keys", ctypes.c_int32),
        ("query_extent", ctypes.c_int32),
        ("key_extent", ctypes.c_int32),
        ("segment_layout", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("q_units", _vp),
        ("k_units", _vp),
        ("num_q_units", ctypes.c_int32),
        ("num_k_units", ctypes.c_int32),
        ("ds_offsets", _vp),
        ("ds_elements", ctypes.c_int64),
        ("query_tile", ctypes.c_int32),
        ("unit_fields", ctypes.c_int32),
        ("key_tile", ctypes.c_int32),
        ("f_units", _vp),
        ("num_f_units", ctypes.c_int32),
    ]


UNIT_FIELDS = 16  # WMX_UNIT_FIELDS: ints per varlen work-list entry with the segment's bounds


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp),
        ("k", _vp),
        ("v", _vp),
        ("o", _vp),
        ("query_start", _vp),
        ("kv_lengths", _vp),
        ("key_mask", _vp),
        ("key_mask_stride", ctypes.c_int64),
        ("workspace", _vp),
        ("workspace_bytes", ctypes.c_int64),
        ("q_stride", _c_i64_2),
        ("k_stride", _c_i64_3),
        ("v_stride", _c_i64_3),
        ("o_stride", _c_i64_2),
        ("query_start_scalar", ctypes.c_int64),
        ("batch", ctypes.c_int32),
        ("q_heads", ctypes.c_int32),
        ("kv_heads", ctypes.c_int32),
        ("capacity", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("use_dummy", ctypes.c_int32),
        ("num_splits", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("counters", _vp),
        ("lengths_broadcast", ctypes.c_int32),
    ]


_c_i64_4 = ctypes.c_int64 * 4
DTYPE_F32, DTYPE_BF16 = 0, 1


_vp2 = _vp * 2


class KvMixArgs(ctypes.Structure):
    """Mirror of wmx_kv_mix_args (index 0 of each pair: the K side, 1: V)."""

    _fields_ = [
        ("sources", _vp),
        ("source_stride", _c_i64_3),
        ("pre_mix", _vp2),
        ("premixed", _vp2),
        ("alpha", _vp2),
        ("alpha_stride", ctypes.c_int64),
        ("gain", _vp2),
        ("mixed", _vp2),
        ("source_dtype", ctypes.c_int32),
        ("weight_dtype", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("tokens", ctypes.c_int32),
        ("num_sources", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("eps", ctypes.c_float),
        ("mix_eps", ctypes.c_float),
    ]


class KvRouterArgs(ctypes.Structure):
    """Mirror of wmx_kv_router_args (index 0 of each pair: the K side, 1: V)."""

    _fields_ = [
        ("premixed", _vp2),
        ("weight", _vp2),
        ("bias", _vp2),
        ("alpha", _vp2),
        ("workspace", _vp),
        ("workspace_bytes", ctypes.c_int64),
        ("rows", ctypes.c_int32),
        ("inputs", ctypes.c_int32),
        ("logits", ctypes.c_int32),
        ("row_stride", ctypes.c_int32),
        ("source_width", ctypes.c_int32),
        ("source_start", ctypes.c_int32),
        ("source_stride", ctypes.c_int32),
    ]


class KvStoreBwdArgs(ctypes.Structure):
    """Mirror of wmx_kv_store_bwd_args."""

    _fields_ = [
        ("key", _vp),
        ("grad_out", _vp),
        ("k_norm_weight", _vp),
        ("cos", _vp),
        ("sin", _vp),
        ("grad_key", _vp),
        ("grad_weight", _vp),
        ("workspace", _vp),
        ("workspace_bytes", ctypes.c_int64),
        ("key_stride", ctypes.c_int64 * 4),
        ("grad_out_stride", ctypes.c_int64 * 4),
        ("grad_key_stride", ctypes.c_int64 * 4),
        ("rope_stride", _c_i64_2),
        ("key_dtype", ctypes.c_int32),
        ("weight_dtype", ctypes.c_int32),
        ("rope_dtype", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("tokens", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("eps", ctypes.c_float),
    ]


KV_MIX_MAX_SOURCES = 512
KV_MIX_MAX_HIDDEN = 4096
KV_ROUTER_MAX_LOGITS = 256  # WMX_KV_ROUTER_MAX_LOGITS


class KvStoreArgs(ctypes.Structure):
    """Mirror of wmx_kv_store_args."""

    _fields_ = [
        ("key", _vp),
        ("value", _vp),
        ("k_norm_weight", _vp),
        ("cos", _vp),
        ("sin", _vp),
        ("key_pool", _vp),
        ("value_pool", _vp),
        ("slots", _vp),
        ("key_stride", _c_i64_4),
        ("value_stride", _c_i64_4),
        ("key_pool_stride", _c_i64_4),
        ("value_pool_stride", _c_i64_4),
        ("rope_stride", _c_i64_2),
        ("key_dtype", ctypes.c_int32),
        ("value_dtype", ctypes.c_int32),
        ("weight_dtype", ctypes.c_int32),
        ("rope_dtype", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("tokens", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("pool_slots", ctypes.c_int32),
        ("eps", ctypes.c_float),
        ("rope_by_slot", ctypes.c_int32),
    ]


DTYPE_I32, DTYPE_I64 = 2, 3


class StrictMetaArgs(ctypes.Structure):
    """Mirror of wmx_strict_meta_args."""

    _fields_ = [
        ("document_ids", _vp),
        ("query_start", _vp),
        ("kv_lengths", _vp),
        ("workspace", _vp),
        ("counts", _vp),
        ("query_indices", _vp),
        ("key_indices", _vp),
        ("cu_queries", _vp),
        ("cu_keys", _vp),
        ("doc_stride", ctypes.c_int64),
        ("query_start_scalar", ctypes.c_int64),
        ("workspace_bytes", ctypes.c_int64),
        ("doc_dtype", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("extent", ctypes.c_int32),
        ("query_length", ctypes.c_int32),
        ("use_dummy", ctypes.c_int32),
    ]


FEEDBACK_MAX_GROUPS = 64


class FeedbackMetaArgs(ctypes.Structure):
    """Mirror of wmx_feedback_meta_args."""

    _fields_ = [
        ("document_ids", _vp),
        ("slots", _vp),
        ("workspace", _vp),
        ("key_ids", _vp),
        ("key_query_end", _vp),
        ("query_ids", _vp),
        ("query_key_start", _vp),
        ("doc_stride", ctypes.c_int64),
        ("workspace_bytes", ctypes.c_int64),
        ("group_offsets", ctypes.c_int64 * (FEEDBACK_MAX_GROUPS + 1)),
        ("doc_dtype", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("length", ctypes.c_int32),
        ("key_length", ctypes.c_int32),
        ("groups", ctypes.c_int32),
        ("group_base", ctypes.c_int32),
        ("group_count", ctypes.c_int32),
        ("use_dummy", ctypes.c_int32),
    ]


EXPORTS = (
    "wmx_abi_version",
    "wmx_attn_args_size",
    "wmx_decode_args_size",
    "wmx_last_error",
    "wmx_attn_fwd",
    "wmx_attn_bwd_preprocess",
    "wmx_attn_bwd_workspace_size",
    "wmx_attn_bwd_min_workspace_size",
    "wmx_attn_bwd",
    "wmx_attn_bwd_dq",
    "wmx_attn_bwd_dkv",
    "wmx_decode_workspace_size",
    "wmx_decode_num_splits",
    "wmx_decode",
    "wmx_decode_noalloc",
    "wmx_kv_store_args_size",
    "wmx_kv_pool_store",
    "wmx_kv_mix_args_size",
    "wmx_kv_router_args_size",
    "wmx_kv_router_workspace_size",
    "wmx_kv_router",
    "wmx_kv_store_bwd_args_size",
    "wmx_kv_store_bwd_workspace_size",
    "wmx_kv_store_bwd",
    "wmx_kv_premix",
    "wmx_kv_mix",
    "wmx_strict_meta_args_size",
    "wmx_strict_meta_workspace_size",
    "wmx_strict_meta_count",
    "wmx_strict_meta_fill",
    "wmx_dense_units",
    "wmx_feedback_meta_args_size",
    "wmx_feedback_meta_workspace_size",
    "wmx_feedback_meta",
)


@functools.cache
def load() -> ctypes.CDLL:
    """Load the gfx950 library once; raise RuntimeError if it is absent or stale."""
    path = Path(os.environ.get("WMX_ATTN_LIBRARY", LIBRARY))
    if not path.exists():
        raise RuntimeError(
            f"libwmx_attn.so not found at {path}; build it with `python -c \"import __graft_entry__ as g; g.build()\"`"
        )
    lib = ctypes.CDLL(str(path))
    for name in EXPORTS:
        if not hasattr(lib, name):
            raise RuntimeError(f"{path} does not export {name}")
    lib.wmx_abi_version.restype = ctypes.c_int
    lib.wmx_attn_args_size.restype = ctypes.c_size_t
    lib.wmx_decode_args_size.restype = ctypes.c_size_t
    lib.wmx_last_error.restype = ctypes.c_char_p
    for name in ("wmx_attn_fwd", "wmx_attn_bwd_preprocess", "wmx_attn_bwd", "wmx_attn_bwd_dq", "wmx_attn_bwd_dkv"):
        getattr(lib, name).argtypes = [ctypes.POINTER(AttnArgs), _vp]
        getattr(lib, name).restype = ctypes.c_int
    for name in ("wmx_attn_bwd_workspace_size", "wmx_attn_bwd_min_workspace_size"):
        getattr(lib, name).argtypes = [ctypes.POINTER(AttnArgs)]
        getattr(lib, name).restype = ctypes.c_int64
    for name in ("wmx_decode", "wmx_decode_noalloc"):
        getattr(lib, name).argtypes = [ctypes.POINTER(DecodeArgs), _vp]
        getattr(lib, name).restype = ctypes.c_int
    lib.wmx_decode_workspace_size.argtypes = [ctypes.POINTER(DecodeArgs)]
    lib.wmx_decode_workspace_size.restype = ctypes.c_int64
    lib.wmx_decode_num_splits.argtypes = [ctypes.POINTER(DecodeArgs)]
    lib.wmx_decode_num_splits.restype = ctypes.c_int32
    lib.wmx_kv_store_args_size.restype = ctypes.c_size_t
    lib.wmx_kv_pool_store.argtypes = [ctypes.POINTER(KvStoreArgs), _vp]
    lib.wmx_kv_pool_store.restype = ctypes.c_int
    lib.wmx_kv_mix_args_size.restype = ctypes.c_size_t
    lib.wmx_kv_store_bwd_args_size.restype = ctypes.c_size_t
    lib.wmx_kv_store_bwd_workspace_size.argtypes = [ctypes.POINTER(KvStoreBwdArgs)]
    lib.wmx_kv_store_bwd_workspace_size.restype = ctypes.c_int64
    lib.wmx_kv_store_bwd.argtypes = [ctypes.POINTER(KvStoreBwdArgs), _vp]
    lib.wmx_kv_store_bwd.restype = ctypes.c_int
    for name in ("wmx_kv_premix", "wmx_kv_mix"):
        getattr(lib, name).argtypes = [ctypes.POINTER(KvMixArgs), _vp]
        getattr(lib, name).restype = ctypes.c_int
    lib.wmx_kv_router_args_size.restype = ctypes.c_size_t
    lib.wmx_kv_router_workspace_size.argtypes = [ctypes.POINTER(KvRouterArgs)]
    lib.wmx_kv_router_workspace_size.restype = ctypes.c_int64
    lib.wmx_kv_router.argtypes = [ctypes.POINTER(KvRouterArgs), _vp]
    lib.wmx_kv_router.restype = ctypes.c_int
    lib.wmx_strict_meta_args_size.restype = ctypes.c_size_t
    lib.wmx_strict_meta_workspace_size.argtypes = [ctypes.POINTER(StrictMetaArgs)]
    lib.wmx_strict_meta_workspace_size.restype = ctypes.c_int64
    for name in ("wmx_strict_meta_count", "wmx_strict_meta_fill"):
        getattr(lib, name).argtypes = [ctypes.POINTER(StrictMetaArgs), _vp]
        getattr(lib, name).restype = ctypes.c_int
    lib.wmx_dense_units.argtypes = [ctypes.POINTER(AttnArgs), _vp, _vp]
    lib.wmx_dense_units.restype = ctypes.c_int
    lib.wmx_feedback_meta_args_size.restype = ctypes.c_size_t
    lib.wmx_feedback_meta_workspace_size.argtypes = [ctypes.POINTER(FeedbackMetaArgs)]
    lib.wmx_feedback_meta_workspace_size.restype = ctypes.c_int64
    lib.wmx_feedback_meta.argtypes = [ctypes.POINTER(FeedbackMetaArgs), _vp]
    lib.wmx_feedback_meta.restype = ctypes.c_int
    if lib.wmx_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI {lib.wmx_abi_version()}, expected {ABI_VERSION}")
    if lib.wmx_attn_args_size() != ctypes.sizeof(AttnArgs):
        raise RuntimeError("wmx_attn_args layout differs between the library and the binding")
    if lib.wmx_decode_args_size() != ctypes.sizeof(DecodeArgs):
        raise RuntimeError("wmx_decode_args layout differs between the library and the binding")
    if lib.wmx_kv_store_args_size() != ctypes.sizeof(KvStoreArgs):
        raise RuntimeError("wmx_kv_store_args layout differs between the library and the binding")
    if lib.wmx_kv_store_bwd_args_size() != ctypes.sizeof(KvStoreBwdArgs):
        raise RuntimeError("wmx_kv_store_bwd_args layout differs between the library and the binding")
    if lib.wmx_kv_mix_args_size() != ctypes.sizeof(KvMixArgs):
        raise RuntimeError("wmx_kv_mix_args layout differs between the library and the binding")
    if lib.wmx_kv_router_args_size() != ctypes.sizeof(KvRouterArgs):
        raise RuntimeError("wmx_kv_router_args layout differs between the library and the binding")
    if lib.wmx_feedback_meta_args_size() != ctypes.sizeof(FeedbackMetaArgs):
        raise RuntimeError("wmx_feedback_meta_args layout differs between the library and the binding")
    if lib.wmx_strict_meta_args_size() != ctypes.sizeof(StrictMetaArgs):
        raise RuntimeError("wmx_strict_meta_args layout differs between the library and the binding")
    return lib


@functools.cache
def load_ops() -> None:
    """Register the C++ operators (white_matter::cyclic_attn_*) once; raise
    RuntimeError if their library is absent (there is no other implementation)."""
    if not OPS_LIBRARY.exists():
        raise RuntimeError(
            f"libwmx_torch.so not found at {OPS_LIBRARY}; build it with `python -c \"import __graft_entry__ as g; g.build()\"`"
        )
    torch.ops.load_library(str(OPS_LIBRARY))


def _check(lib: ctypes.CDLL, rc: int, what: str) -> None:
    if rc != 0:
        message = lib.wmx_last_error().decode(errors="replace")
        kind = ValueError if rc == -1 else RuntimeError
        raise kind(f"{what} failed ({rc}): {message}")


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def strides3(t: torch.Tensor | None) -> tuple[int, int, int]:
    """Element strides [batch, head, token] of a (B, H, T, D) tensor."""
    if t is None:
        return (0, 0, 0)
    return (t.stride(0), t.stride(1), t.stride(2))


def attn_fwd(args: AttnArgs, device: torch.device) -> None:
    lib = load()
    _check(lib, lib.wmx_attn_fwd(ctypes.byref(args), _stream(device)), "wmx_attn_fwd")


def attn_bwd_preprocess(args: AttnArgs, device: torch.device) -> None:
    lib = load()
    _check(lib, lib.wmx_attn_bwd_preprocess(ctypes.byref(args), _stream(device)), "wmx_attn_bwd_preprocess")


def attn_bwd_workspace_size(args: AttnArgs) -> int:
    return int(load().wmx_attn_bwd_workspace_size(ctypes.byref(args)))


def attn_bwd(args: AttnArgs, device: torch.device) -> None:
    lib = load()
    _check(lib, lib.wmx_attn_bwd(ctypes.byref(args), _stream(device)), "wmx_attn_bwd")


def attn_bwd_dq(args: AttnArgs, device: torch.device) -> None:
    lib = load()
    _check(lib, lib.wmx_attn_bwd_dq(ctypes.byref(args), _stream(device)), "wmx_attn_bwd_dq")


def attn_bwd_dkv(args: AttnArgs, device: torch.device) -> None:
    lib = load()
    _check(lib, lib.wmx_attn_bwd_dkv(ctypes.byref(args), _stream(device)), "wmx_attn_bwd_dkv")


def decode_workspace_size(args: DecodeArgs) -> int:
    return int(load().wmx_decode_workspace_size(ctypes.byref(args)))


def decode(args: DecodeArgs, device: torch.device) -> None:
    lib = load()
    _check(lib, lib.wmx_decode(ctypes.byref(args), _stream(device)), "wmx_decode")


# wmx_decode_noalloc's static scratch per GPU (WMX_DECODE_NOALLOC_MAX_BYTES)
DECODE_NOALLOC_MAX_BYTES = 8 << 20


def decode_noalloc(args: DecodeArgs, device: torch.device) -> None:
    """wmx_decode with the partials in the library's static device scratch
    (args.workspace is ignored); no device memory is allocated."""
    lib = load()
    _check(lib, lib.wmx_decode_noalloc(ctypes.byref(args), _stream(device)), "wmx_decode_noalloc")


def kv_pool_store(args: KvStoreArgs, device: torch.device) -> None:
    lib = load()
    _check(lib, lib.wmx_kv_pool_store(ctypes.byref(args), _stream(device)), "wmx_kv_pool_store")


def kv_store_bwd_workspace_size(args: KvStoreBwdArgs) -> int:
    return int(load().wmx_kv_store_bwd_workspace_size(ctypes.byref(args)))


def kv_store_bwd(args: KvStoreBwdArgs, device: torch.device) -> None:
    lib = load()
    _check(lib, lib.wmx_kv_store_bwd(ctypes.byref(args), _stream(device)), "wmx_kv_store_bwd")


def kv_premix(args: KvMixArgs, device: torch.device) -> None:
    lib = load()
    _check(lib, lib.wmx_kv_premix(ctypes.byref(args), _stream(device)), "wmx_kv_premix")


def kv_mix(args: KvMixArgs, device: torch.device) -> None:
    lib = load()
    _check(lib, lib.wmx_kv_mix(ctypes.byref(args), _stream(device)), "wmx_kv_mix")


def kv_router_workspace_size(args: KvRouterArgs) -> int:
    return int(load().wmx_kv_router_workspace_size(ctypes.byref(args)))


def kv_router(args: KvRouterArgs, device: torch.device) -> None:
    lib = load()
    _check(lib, lib.wmx_kv_router(ctypes.byref(args), _stream(device)), "wmx_kv_router")


def strict_meta_workspace_size(args: StrictMetaArgs) -> int:
    return int(load().wmx_strict_meta_workspace_size(ctypes.byref(args)))


def strict_meta_count(args: StrictMetaArgs, device: torch.device) -> None:
    lib = load()
    _check(lib, lib.wmx_strict_meta_count(ctypes.byref(args), _stream(device)), "wmx_strict_meta_count")


def strict_meta_fill(args: StrictMetaArgs, device: torch.device) -> None:
    lib = load()
    _check(lib, lib.wmx_strict_meta_fill(ctypes.byref(args), _stream(device)), "wmx_strict_meta_fill")


def feedback_meta_workspace_size(args: FeedbackMetaArgs) -> int:
    return int(load().wmx_feedback_meta_workspace_size(ctypes.byref(args)))


def feedback_meta(args: FeedbackMetaArgs, device: torch.device) -> None:
    lib = load()
    _check(lib, lib.wmx_feedback_meta(ctypes.byref(args), _stream(device)), "wmx_feedback_meta")


def dense_units(args: AttnArgs, units: torch.Tensor, device: torch.device) -> None:
    lib = load()
    _check(lib, lib.wmx_dense_units(ctypes.byref(args), units.data_ptr(), _stream(device)), "wmx_dense_units")
