"""The C-ABI library on the CPU: it loads, exports every function that
include/wmx_attn.h declares, its argument structs match the ctypes binding,
and argument checks fail with error codes before anything reaches a GPU."""

import ctypes
import re
from pathlib import Path

import pytest

from white_matter_amd import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "wmx_attn.h"


def _declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|int32_t|int64_t|size_t|const char\*)\s+(wmx_\w+)\s*\(", text, re.M)))


def test_header_declares_the_exported_entry_points():
    declared = _declared_functions()
    assert set(declared) == set(_native.EXPORTS)


def test_library_loads_and_exports_every_declared_symbol():
    lib = _native.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.wmx_abi_version() == _native.ABI_VERSION
    assert lib.wmx_attn_args_size() == ctypes.sizeof(_native.AttnArgs)
    assert lib.wmx_decode_args_size() == ctypes.sizeof(_native.DecodeArgs)
    assert lib.wmx_kv_mix_args_size() == ctypes.sizeof(_native.KvMixArgs)
    assert lib.wmx_kv_store_bwd_args_size() == ctypes.sizeof(_native.KvStoreBwdArgs)
    assert lib.wmx_kv_router_args_size() == ctypes.sizeof(_native.KvRouterArgs)


def test_argument_checks_return_errors_without_launching():
    lib = _native.load()
    assert lib.wmx_attn_fwd(None, None) == -1
    assert b"NULL" in lib.wmx_last_error()
    args = _native.AttnArgs()
    args.head_dim = 80
    assert lib.wmx_attn_fwd(ctypes.byref(args), None) == -2
    assert b"head_dim" in lib.wmx_last_error()
    args.head_dim, args.batch, args.q_heads, args.kv_heads, args.query_stride = 128, 1, 3, 2, 1
    assert lib.wmx_attn_fwd(ctypes.byref(args), None) == -1
    assert b"kv_heads" in lib.wmx_last_error()
    args.q_heads = 4
    args.key_tile = 32  # dK/dV workgroups take 64 or 128 keys
    assert lib.wmx_attn_fwd(ctypes.byref(args), None) == -1
    assert b"key_tile" in lib.wmx_last_error()
    args.key_tile = 64
    assert lib.wmx_attn_fwd(ctypes.byref(args), None) == -2
    assert b"softmax_scale" in lib.wmx_last_error()
    args.softmax_scale = 0.125
    args.q = args.k = args.v = args.o = args.lse = 0x1008  # misaligned pointer is rejected before use
    assert lib.wmx_attn_fwd(ctypes.byref(args), None) == -1
    assert b"aligned" in lib.wmx_last_error()
    dec = _native.DecodeArgs()
    dec.head_dim, dec.batch, dec.q_heads, dec.kv_heads = 128, 1, 6, 4
    assert lib.wmx_decode(ctypes.byref(dec), None) == -1
    assert b"kv_heads" in lib.wmx_last_error()
    dec.head_dim = 80
    assert lib.wmx_decode(ctypes.byref(dec), None) == -2
    assert b"head_dim" in lib.wmx_last_error()
    dec.head_dim, dec.kv_heads = 128, 2
    # the allocation-free decode checks its arguments before it touches a
    # device (partials beyond its static scratch take fewer splits instead)
    dec.q_heads, dec.capacity, dec.num_splits, dec.softmax_scale = 2, 4096, 20000, 0.1
    dec.q = dec.k = dec.v = dec.o = 0x1000
    dec.use_dummy = 2
    assert lib.wmx_decode_noalloc(ctypes.byref(dec), None) == -1
    assert b"use_dummy" in lib.wmx_last_error()
    bwd = _native.KvStoreBwdArgs()
    bwd.head_dim, bwd.batch, bwd.channels, bwd.heads, bwd.tokens = 80, 1, 1, 1, 1
    assert lib.wmx_kv_store_bwd(ctypes.byref(bwd), None) == -2
    assert b"head_dim" in lib.wmx_last_error()
    bwd.head_dim, bwd.k_norm_weight, bwd.grad_weight = 64, 0x1000, 0x1000
    assert lib.wmx_kv_store_bwd_workspace_size(ctypes.byref(bwd)) == 64 * 4
    assert lib.wmx_kv_store_bwd(ctypes.byref(bwd), None) == -1
    assert b"NULL" in lib.wmx_last_error()
    bwd.key = bwd.grad_out = bwd.cos = bwd.sin = bwd.grad_key = bwd.workspace = 0x1000
    bwd.workspace_bytes = 64
    assert lib.wmx_kv_store_bwd(ctypes.byref(bwd), None) == -3
    mix = _native.KvMixArgs()
    mix.batch, mix.tokens, mix.num_sources, mix.hidden, mix.channels = 1, 1, 25, 1028, 8
    assert lib.wmx_kv_premix(ctypes.byref(mix), None) == -2
    assert b"hidden" in lib.wmx_last_error()
    mix.hidden, mix.num_sources = 1024, _native.KV_MIX_MAX_SOURCES + 1
    assert lib.wmx_kv_mix(ctypes.byref(mix), None) == -2
    assert b"num_sources" in lib.wmx_last_error()
    mix.num_sources = 25
    assert lib.wmx_kv_mix(ctypes.byref(mix), None) == -1
    assert b"NULL" in lib.wmx_last_error()
    for side in range(2):
        mix.premixed[side] = mix.alpha[side] = mix.gain[side] = mix.mixed[side] = 0x1000
    mix.alpha_stride = 8 * 25 - 1
    assert lib.wmx_kv_mix(ctypes.byref(mix), None) == -1
    assert b"alpha_stride" in lib.wmx_last_error()
    mix.pre_mix[0] = mix.pre_mix[1] = 0x1000
    mix.sources, mix.source_stride = 0x1000, (25 * 1024, 1024, 1028)
    assert lib.wmx_kv_premix(ctypes.byref(mix), None) == -1
    assert b"strides" in lib.wmx_last_error()
    router = _native.KvRouterArgs()
    router.rows, router.inputs, router.logits = 2048, 25 * 1024 + 8, 200
    assert lib.wmx_kv_router(ctypes.byref(router), None) == -2
    assert b"multiple of 64" in lib.wmx_last_error()
    router.inputs, router.logits = 25 * 1024, _native.KV_ROUTER_MAX_LOGITS + 1
    assert lib.wmx_kv_router(ctypes.byref(router), None) == -2
    assert b"logits" in lib.wmx_last_error()
    router.logits = 200
    # the strided source view: widths that split a 64-input stage, a start
    # before the row, rows too short for the selected sources
    router.inputs, router.source_width, router.source_stride = 13 * 1024, 96, 2
    assert lib.wmx_kv_router(ctypes.byref(router), None) == -2
    assert b"source_width" in lib.wmx_last_error()
    router.source_width, router.source_start = 1024, -1
    assert lib.wmx_kv_router(ctypes.byref(router), None) == -1
    assert b"start" in lib.wmx_last_error()
    router.source_start, router.row_stride = 0, 24 * 1024  # sources 0, 2, .., 24 need 25 blocks
    assert lib.wmx_kv_router(ctypes.byref(router), None) == -1
    assert b"row_stride" in lib.wmx_last_error()
    router.row_stride = 25 * 1024
    assert lib.wmx_kv_router(ctypes.byref(router), None) == -1
    assert b"NULL" in lib.wmx_last_error()
    router.inputs, router.source_width = 25 * 1024, 0  # every source
    for side in range(2):
        router.premixed[side] = router.weight[side] = router.alpha[side] = 0x1000
    # 2 sides x 25 chunks of 1024 inputs x 2048 rows x 200 logits, fp32
    assert lib.wmx_kv_router_workspace_size(ctypes.byref(router)) == 2 * 25 * 2048 * 200 * 4
    router.workspace, router.workspace_bytes = 0x1000, 2 * 25 * 2048 * 200 * 4 - 1
    assert lib.wmx_kv_router(ctypes.byref(router), None) == -3
    assert b"workspace" in lib.wmx_last_error()


def test_workspace_sizes():
    lib = _native.load()
    args = _native.AttnArgs()
    args.head_dim, args.batch, args.kv_heads, args.key_extent = 128, 2, 4, 100
    assert lib.wmx_attn_bwd_workspace_size(ctypes.byref(args)) == 0
    # dense: a bf16 dS^T block of kv_len x (q_len rounded up to 128) per (batch row, query head)
    args.q_heads, args.q_len, args.kv_len = 8, 130, 300
    assert lib.wmx_attn_bwd_workspace_size(ctypes.byref(args)) == 2 * 8 * 300 * 256 * 2
    assert lib.wmx_attn_bwd_min_workspace_size(ctypes.byref(args)) == 0
    args.query_indices = 0x1000
    args.keys_unique = 0
    acc = 2 * 2 * 100 * 4 * 128 * 4
    assert lib.wmx_attn_bwd_workspace_size(ctypes.byref(args)) == acc  # no dS layout given
    assert lib.wmx_attn_bwd_min_workspace_size(ctypes.byref(args)) == acc
    args.ds_offsets, args.ds_elements = 0x2000, 1000
    assert lib.wmx_attn_bwd_workspace_size(ctypes.byref(args)) == acc + 8 * 1000 * 2
    dec = _native.DecodeArgs()
    dec.batch, dec.q_heads, dec.kv_heads, dec.capacity, dec.head_dim, dec.num_splits = 2, 4, 4, 1000, 64, 3
    assert lib.wmx_decode_num_splits(ctypes.byref(dec)) == 3
    assert lib.wmx_decode_workspace_size(ctypes.byref(dec)) == 2 * 4 * 3 * (64 + 2) * 4


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setenv("WMX_ATTN_LIBRARY", str(tmp_path / "absent.so"))
    _native.load.cache_clear()
    try:
        with pytest.raises(RuntimeError, match="not found"):
            _native.load()
    finally:
        monkeypatch.delenv("WMX_ATTN_LIBRARY")
        _native.load.cache_clear()


def test_fused_segment_list_checks():
    """wmx_attn_bwd refuses a fused segment list (f_units) the kernel cannot take,
    before anything is launched."""
    lib = _native.load()
    a = _native.AttnArgs()
    a.head_dim, a.batch, a.q_heads, a.kv_heads, a.q_len, a.kv_len = 128, 1, 2, 2, 64, 64
    a.query_stride, a.softmax_scale = 8, 0.125
    a.q = a.k = a.v = a.o = a.lse = a.dout = a.delta = a.dq = a.dk = a.dv = 0x1000
    for name in ("q_stride", "k_stride", "v_stride", "o_stride", "do_stride", "dq_stride", "dk_stride", "dv_stride"):
        setattr(a, name, (2 * 64 * 128, 64 * 128, 128))
    a.query_indices = a.key_indices = a.cu_queries = a.cu_keys = 0x1000
    a.num_segments, a.query_extent, a.key_extent, a.keys_unique = 1, 64, 64, 1
    a.f_units, a.num_f_units = 0x1000, 1
    assert lib.wmx_attn_bwd(ctypes.byref(a), None) == -1
    assert b"k_units and q_units" in lib.wmx_last_error()
    a.q_units = a.k_units = 0x1000
    assert lib.wmx_attn_bwd(ctypes.byref(a), None) == -1
    assert b"WMX_UNIT_FIELDS" in lib.wmx_last_error()
    a.unit_fields = _native.UNIT_FIELDS
    a.q_heads = 4
    assert lib.wmx_attn_bwd(ctypes.byref(a), None) == -1
    assert b"q_heads == kv_heads" in lib.wmx_last_error()
    a.q_heads = 2
    a.keys_unique = 0
    assert lib.wmx_attn_bwd(ctypes.byref(a), None) == -1
    assert b"keys_unique" in lib.wmx_last_error()
    a.keys_unique = 1
    assert lib.wmx_attn_bwd(ctypes.byref(a), None) == -1
    assert b"consecutive" in lib.wmx_last_error()
    a.segment_layout = 3
    a.k_stride = (2 * 64 * 2048, 64 * 2048, 1 << 23)  # beyond the strided tile loads' 32-bit offsets
    assert lib.wmx_attn_bwd(ctypes.byref(a), None) == -1
    assert b"token strides" in lib.wmx_last_error()
    a.f_units, a.query_indices = 0x1000, None
    assert lib.wmx_attn_bwd(ctypes.byref(a), None) == -1
    assert b"varlen schedule" in lib.wmx_last_error()
