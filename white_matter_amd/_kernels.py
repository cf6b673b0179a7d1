"""Tensor preparation and launches of the gfx950 kernels through the C ABI.

This layer turns PyTorch tensors into the plain pointers, element strides and
sizes of ``wmx_attn_args`` / ``wmx_decode_args`` and calls libwmx_attn.so on
the current HIP stream. It allocates outputs and workspaces with PyTorch; the
library itself allocates nothing. There is no alternative implementation
behind it: a missing library raises.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native

SUPPORTED_HEAD_DIMS = (64, 96, 128)


def guard_capture(what: str) -> None:
    """Raise before a host synchronisation or a schedule-cache build inside HIP
    graph capture: such a step would break the capture (or record a copy from
    host memory that is gone at replay). The call must run once eagerly on the
    same metadata first, so everything a captured call needs is cached."""
    if torch.cuda.is_initialized() and torch.cuda.is_current_stream_capturing():
        raise RuntimeError(
            f"{what} synchronises with the host, which HIP graph capture forbids; "
            "run the same call once before capturing so its schedule is cached"
        )


def kernel_head_dim(dim: int) -> int | None:
    """Smallest kernel head_dim that holds ``dim`` (zero padding), or None."""
    for size in SUPPORTED_HEAD_DIMS:
        if dim <= size:
            return size
    return None


def _vector_ready(x: torch.Tensor) -> bool:
    if x.stride(-1) != 1 and x.shape[-1] != 1:
        return False
    if x.data_ptr() % 16:
        return False
    return all(stride % 8 == 0 for stride, size in zip(x.stride()[:-1], x.shape[:-1]) if size > 1)


def operand(x: torch.Tensor) -> torch.Tensor:
    """bf16 with unit head_dim stride and 16-byte aligned rows; strided views
    (cache channels, capacity padding, BQHD storage) are kept without a copy."""
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    if _vector_ready(x):
        return x
    x = x.contiguous()
    return x if _vector_ready(x) else x.clone()


def pad_head_dim(x: torch.Tensor, size: int) -> torch.Tensor:
    return x if x.shape[-1] == size else torch.nn.functional.pad(x, (0, size - x.shape[-1]))


def _strides(x: torch.Tensor | None) -> tuple[int, int, int]:
    """[batch, head, token] element strides of a 4-D tensor; size-1 dims give 0."""
    if x is None:
        return (0, 0, 0)
    return tuple(s if n > 1 else 0 for s, n in zip(x.stride()[:3], x.shape[:3]))  # type: ignore[return-value]


@dataclass
class Varlen:
    """A packed-segment schedule in kernel form (see StrictCausalMetadata)."""

    query_indices: torch.Tensor  # int64, flat b * query_extent + t
    key_indices: torch.Tensor  # int64, flat b * key_extent + slot
    cu_queries: torch.Tensor  # int32 (num_segments + 1)
    cu_keys: torch.Tensor  # int32 (num_segments + 1)
    num_segments: int
    max_queries: int
    max_keys: int
    query_extent: int
    key_extent: int
    keys_unique: int  # wmx_attn_args.keys_unique: 1 unique, 2 only slot 0 repeats, 0 others repeat
    segment_layout: int = 0  # bit 0 consecutive queries, bit 1 consecutive keys from key 1
    # work lists, heaviest first: int32 (n, 2) (segment, tile) or (n, UNIT_FIELDS)
    # entries that also carry the segment's bounds (see _native.UNIT_FIELDS)
    q_units: torch.Tensor | None = None  # query tiles
    k_units: torch.Tensor | None = None  # key tiles
    ds_offsets: torch.Tensor | None = None  # int64 (num_segments + 1) dS block offsets (see wmx_attn.h)
    ds_elements: int = 0  # ds_offsets[-1]
    key_tile: int = 0  # keys per dK/dV workgroup: 0/128, or 64 (k_units then count 64-key tiles)


@dataclass
class Visibility:
    """Which key slots each query row reads (the mask of wmx_attn_args)."""

    query_stride: int = 1
    query_offset: int = 0
    row_offset: torch.Tensor | None = None  # int32 (B,)
    row_limit: torch.Tensor | None = None  # int32 (B,)
    keep_slot0: bool = False
    key_mask: torch.Tensor | None = None  # bool (B, Tk)
    documents: tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor] | None = None
    varlen: Varlen | None = None
    q_units: torch.Tensor | None = None  # int32 (n, 2) (batch row, query tile), heaviest first (dense)
    query_tile: int = 0  # forward rows per workgroup: 0/128, or 256 (q_units then count 256-row tiles)

    def fill(self, args: _native.AttnArgs) -> None:
        args.query_stride = self.query_stride
        args.query_offset = self.query_offset
        args.row_offset = _native.ptr(self.row_offset)
        args.row_limit = _native.ptr(self.row_limit)
        args.keep_slot0 = int(self.keep_slot0)
        if self.key_mask is not None:
            args.key_mask = self.key_mask.data_ptr()
            args.key_mask_stride = self.key_mask.stride(0)
        if self.documents is not None:
            args.q_seg, args.k_seg, args.q_start, args.k_qend = (t.data_ptr() for t in self.documents)
        args.query_tile = self.query_tile
        if self.q_units is not None:
            args.q_units, args.num_q_units = self.q_units.data_ptr(), self.q_units.shape[0]
        if self.varlen is not None:
            s = self.varlen
            args.query_indices = s.query_indices.data_ptr()
            args.key_indices = s.key_indices.data_ptr()
            args.cu_queries = s.cu_queries.data_ptr()
            args.cu_keys = s.cu_keys.data_ptr()
            args.num_segments = s.num_segments
            args.max_queries = s.max_queries
            args.max_keys = s.max_keys
            args.query_extent = s.query_extent
            args.key_extent = s.key_extent
            args.keys_unique = int(s.keys_unique)
            args.segment_layout = s.segment_layout
            if s.q_units is not None:
                args.q_units, args.num_q_units = s.q_units.data_ptr(), s.q_units.shape[0]
            if s.k_units is not None:
                args.k_units, args.num_k_units = s.k_units.data_ptr(), s.k_units.shape[0]
            widths = {t.shape[1] for t in (s.q_units, s.k_units) if t is not None}
            if len(widths) > 1:
                raise ValueError("q_units and k_units must have entries of one width")
            args.unit_fields = widths.pop() if widths else 0
            if s.ds_offsets is not None:
                args.ds_offsets, args.ds_elements = s.ds_offsets.data_ptr(), s.ds_elements
            args.key_tile = s.key_tile


QUERY_TILE = 128  # query rows per forward / dQ workgroup
KEY_STEP = 64  # key rows per step of their tile loops


def dense_units(
    batch: int, q_len: int, kv_len: int, query_offset: int, row_offset: torch.Tensor | None,
    row_limit: torch.Tensor | None, device: torch.device, tile: int = QUERY_TILE,
) -> torch.Tensor:
    """Work list of a dense problem with per-row bounds: the (batch row,
    `tile`-row query tile) pairs ordered by the number of 64-key tiles they
    visit, largest first, as an int32 (n, 2) tensor built by one HIP kernel
    (wmx_dense_units; no host synchronisation). Query i of row b sees key
    slots j <= min(offset_b + i, limit_b)."""
    tiles = -(-q_len // tile)
    units = torch.empty(batch * tiles, 2, device=device, dtype=torch.int32)
    args = _native.AttnArgs()
    args.batch, args.q_len, args.kv_len = batch, q_len, kv_len
    args.query_stride, args.query_offset = 1, query_offset
    args.row_offset, args.row_limit = _native.ptr(row_offset), _native.ptr(row_limit)
    args.query_tile = tile if tile == 256 else 0
    _native.dense_units(args, units, device)
    return units


def _base_args(q, k, v, o, lse, scale: float, vis: Visibility, q_len: int) -> _native.AttnArgs:
    args = _native.AttnArgs()
    args.q, args.k, args.v, args.o, args.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr()
    args.q_stride, args.k_stride, args.v_stride = _strides(q), _strides(k), _strides(v)
    args.o_stride = _strides(o)
    args.batch, args.q_heads, args.kv_heads = q.shape[0], q.shape[1], k.shape[1]
    args.q_len, args.kv_len, args.head_dim = q_len, k.shape[2], q.shape[3]
    args.softmax_scale = scale
    vis.fill(args)
    return args


def forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    o: torch.Tensor,
    lse: torch.Tensor,
    scale: float,
    vis: Visibility,
) -> None:
    """o, lse <- attention(q, k, v) under ``vis``. q/k/v/o are (B, H, T, D)
    views of any layout accepted by ``operand``; lse is (B, Hq, Tq) fp32."""
    args = _base_args(q, k, v, o, lse, scale, vis, q.shape[2])
    _native.attn_fwd(args, q.device)


def backward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    o: torch.Tensor,
    lse: torch.Tensor,
    dout: torch.Tensor,
    dq: torch.Tensor,
    dk: torch.Tensor,
    dv: torch.Tensor,
    scale: float,
    vis: Visibility,
) -> None:
    """dq, dk, dv <- gradients of attention(q, k, v) for output gradient dout."""
    args = _base_args(q, k, v, o, lse, scale, vis, q.shape[2])
    delta = torch.empty(lse.shape, device=q.device, dtype=torch.float32)
    args.dout, args.delta = dout.data_ptr(), delta.data_ptr()
    args.do_stride = _strides(dout)
    args.dq, args.dk, args.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    args.dq_stride, args.dk_stride, args.dv_stride = _strides(dq), _strides(dk), _strides(dv)
    need = _native.attn_bwd_workspace_size(args)
    workspace = None
    if need > 0:
        workspace = torch.empty(need, device=q.device, dtype=torch.uint8)
        args.workspace, args.workspace_bytes = workspace.data_ptr(), need
    _native.attn_bwd(args, q.device)


def row_dot(dout: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """delta = sum(dout * out, -1) in fp32 for (B, H, T, D) bf16 views."""
    dout, out = operand(dout), operand(out)
    batch, heads, length, dim = dout.shape
    delta = torch.empty(batch, heads, length, device=dout.device, dtype=torch.float32)
    args = _native.AttnArgs()
    args.o, args.dout, args.delta = out.data_ptr(), dout.data_ptr(), delta.data_ptr()
    args.o_stride, args.do_stride = _strides(out), _strides(dout)
    args.batch, args.q_heads, args.q_len, args.head_dim = batch, heads, length, dim
    _native.attn_bwd_preprocess(args, dout.device)
    return delta


def decode(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    *,
    query_start: int | torch.Tensor,
    kv_lengths: torch.Tensor | None,
    key_mask: torch.Tensor | None,
    use_dummy: bool,
    scale: float,
    num_splits: int = 0,
) -> None:
    """out[b, h] <- single-query attention of q[b, h, 0] over slots of k/v[b, h / G].

    q is (B, Hq, 1, D), k/v are (B, Hkv, N, D) with any strides, out is (B, Hq, D).
    """
    args = _native.DecodeArgs()
    args.q, args.k, args.v, args.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    args.q_stride = (q.stride(0), q.stride(1))
    args.k_stride, args.v_stride = _strides(k), _strides(v)
    args.o_stride = (out.stride(0), out.stride(1))
    keep = []
    if isinstance(query_start, torch.Tensor):
        starts = query_start.to(device=q.device, dtype=torch.int64).expand(q.shape[0]).contiguous()
        keep.append(starts)
        args.query_start = starts.data_ptr()
    else:
        args.query_start_scalar = int(query_start)
    if kv_lengths is not None:
        lengths = kv_lengths.to(device=q.device, dtype=torch.int64).contiguous()
        keep.append(lengths)
        args.kv_lengths = lengths.data_ptr()
    if key_mask is not None:
        args.key_mask = key_mask.data_ptr()
        args.key_mask_stride = key_mask.stride(0)
    args.batch, args.q_heads, args.kv_heads = q.shape[0], q.shape[1], k.shape[1]
    args.capacity, args.head_dim = k.shape[2], q.shape[3]
    args.use_dummy = int(use_dummy)
    args.num_splits = num_splits
    args.softmax_scale = scale
    need = _native.decode_workspace_size(args)
    workspace = torch.empty(max(need, 16), device=q.device, dtype=torch.uint8)
    args.workspace, args.workspace_bytes = workspace.data_ptr(), need
    _native.decode(args, q.device)
