"""Cached decoding of the attention hot path, one token per HIP-graph replay.

The reference replays a captured one-token model forward
(src/white_matter/models/generation.py:38-100, `DecodeGraph`) over the static
`DecoderCache` (models/cache.py:13-273). Its attention side per token is:

  * every layer attends, strictly causally, from its query to one KV-pool
    channel: the pool stores the k channels folded into the head axis as
    (B, k * Hkv, N, D), and the visible length comes from the pool's
    `cumulative_length` (cache.py:184-190; layers/white_matter.py:120-146,
    with the leading dummy slot);
  * the token's keys and values (modules/kv_pool.py:219-226 `project_token`:
    K-norm, RoPE, bf16) are written into slot `cumulative_length`, which then
    advances by one.

`DecodeLoop` captures exactly that step: the layers' split-K decode kernels,
the fused K-norm/RoPE store and the counter update, with the RoPE rows
gathered on the device from the slot, so a replay needs nothing from the host.
Like `DecodeGraph`, a replay returns borrowed outputs that the next call
overwrites, and moving or replacing the pool storage requires a new capture.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

from . import _kernels, kv_pool
from .strict_causal_attention import strict_causal_attention, strict_decode_out


class DecodeLoop:
    """One decode token: L layer attentions over pool channels, the store of the
    token's keys and values, and the length update, captured in a HIP graph.

    keys, values: bf16 pool (B, k * Hkv, N, D), channels folded into heads,
        slot 0 the dummy when `use_dummy_token`.
    cumulative_length: int64 (1,) device tensor, the slots in use (dummy
        included); the next token is written there.
    layer_channels: the pool channel each layer reads.
    k_norm_weight: (k, D) per-channel key-norm weight.
    cos_table, sin_table: (N, D) RoPE rows by slot (the store reads the
        token's row at its slot).
    Inputs per call (static buffers, copied in by `__call__`): `query`
    (L, B, Hq, 1, D) bf16, `new_key` / `new_value` (B, k, Hkv, 1, D) raw
    projections. Output: `output` (L, B, 1, Hq, D) bf16.
    """

    @torch.no_grad()
    def __init__(
        self,
        keys: torch.Tensor,
        values: torch.Tensor,
        cumulative_length: torch.Tensor,
        layer_channels: Sequence[int],
        k_norm_weight: torch.Tensor,
        cos_table: torch.Tensor,
        sin_table: torch.Tensor,
        *,
        query_heads: int,
        use_dummy_token: bool = True,
        softmax_scale: float | None = None,
        eps: float = 1e-6,
        warmup: int = 2,
    ) -> None:
        if not keys.is_cuda or keys.shape != values.shape or keys.dtype != torch.bfloat16 or values.dtype != torch.bfloat16:
            raise ValueError("decode capture requires bf16 CUDA pool keys/values of one shape")
        batch, folded, capacity, dim = keys.shape
        channels = k_norm_weight.shape[0]
        if folded % channels or k_norm_weight.shape != (channels, dim):
            raise ValueError("pool heads must fold k_norm_weight's channels: (B, k * Hkv, N, D) with weight (k, D)")
        if cos_table.shape != (capacity, dim) or sin_table.shape != cos_table.shape:
            raise ValueError("cos_table/sin_table must be (N, D)")
        if any(not 0 <= c < channels for c in layer_channels) or not layer_channels:
            raise ValueError("layer_channels must name pool channels")
        if cumulative_length.shape != (1,) or cumulative_length.dtype != torch.long or not cumulative_length.is_cuda:
            raise ValueError("cumulative_length must be an int64 (1,) CUDA tensor")
        kv_heads = folded // channels
        if query_heads % kv_heads:
            raise ValueError("query heads must be a multiple of the pool's KV heads")
        self.keys, self.values, self.cumulative_length = keys, values, cumulative_length
        self.layer_channels = tuple(int(c) for c in layer_channels)
        self.k_norm_weight, self.cos_table, self.sin_table = k_norm_weight, cos_table, sin_table
        self.use_dummy_token, self.eps = bool(use_dummy_token), float(eps)
        self.scale = softmax_scale if softmax_scale is not None else dim**-0.5
        self.capacity, self._kv_heads, self._channels = capacity, kv_heads, channels
        self.seen = int(cumulative_length.item())  # host copy of the counter, as DecodeGraph keeps seen_tokens
        if not int(self.use_dummy_token) < self.seen < capacity:
            raise ValueError("prefill must leave room for a decoding token")
        device = keys.device
        layers = len(self.layer_channels)
        self.query = torch.zeros(layers, batch, query_heads, 1, dim, device=device, dtype=torch.bfloat16)
        self.new_key = torch.zeros(batch, channels, kv_heads, 1, dim, device=device, dtype=torch.bfloat16)
        self.new_value = torch.zeros_like(self.new_key)
        self._storage = (keys.data_ptr(), values.data_ptr(), cumulative_length.data_ptr())
        # the layers write their outputs here directly where the kernels take
        # this head_dim (no stacking copy); otherwise through the public API
        self._direct = _kernels.kernel_head_dim(dim) == dim
        self._out = torch.empty(layers, batch, 1, query_heads, dim, device=device, dtype=torch.bfloat16)

        snapshot = cumulative_length.clone()
        # warm-up and capture on one stream the loop keeps: the decode
        # operator's split-merge counters belong to a stream, so the graph
        # then records no counter initialisation
        stream = self._stream = torch.cuda.Stream(device=device)
        stream.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(stream):
            for _ in range(warmup):
                self.step()
                cumulative_length.copy_(snapshot)
        torch.cuda.current_stream(device).wait_stream(stream)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=stream):
            self.output = self.step()
        cumulative_length.copy_(snapshot)
        torch.cuda.current_stream(device).synchronize()

    def step(self) -> torch.Tensor:
        """The token's work as eager launches on the current stream (what the
        graph holds): returns (L, B, 1, Hq, D)."""
        batch, _, _, dim = self.keys.shape
        offset = int(self.use_dummy_token)
        outs = []
        h = self._kv_heads
        if not self._direct:
            # real keys before this token, per the reference's lengths; one (B,) tensor shared by all layers
            lengths = self.cumulative_length.expand(batch) - offset
        for layer, channel in enumerate(self.layer_channels):
            k = self.keys[:, channel * h : (channel + 1) * h]
            v = self.values[:, channel * h : (channel + 1) * h]
            if self._direct:
                # the decode sees slots [0, length) with length = real keys +
                # the dummy: the counter itself, read in place by every row
                # (the dummy then needs no separate term)
                strict_decode_out(
                    self._out[layer], self.query[layer], k, v, self.cumulative_length, 0, self.cumulative_length,
                    None, False, self.scale, 0,
                )
            else:
                outs.append(
                    strict_causal_attention(
                        self.query[layer], k, v, query_start=lengths, kv_lengths=lengths,
                        use_dummy_token=self.use_dummy_token, softmax_scale=self.scale,
                    )
                )
        slot = self.cumulative_length
        pool = (self.keys.unflatten(1, (self._channels, h)), self.values.unflatten(1, (self._channels, h)))
        kv_pool.write_pool(
            self.new_key, self.new_value, self.k_norm_weight, self.cos_table, self.sin_table, pool[0], pool[1], slot,
            eps=self.eps, rope_by_slot=True,
        )
        self.cumulative_length.add_(1)
        return self._out if self._direct else torch.stack(outs)

    @torch.no_grad()
    def __call__(
        self,
        query: torch.Tensor | None = None,
        new_key: torch.Tensor | None = None,
        new_value: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Copy the given inputs into the static buffers, replay one token and
        return the borrowed (L, B, 1, Hq, D) output."""
        if self.seen >= self.capacity:
            raise ValueError("the pool is full: no slot left for a decoding token")
        if self._storage != (self.keys.data_ptr(), self.values.data_ptr(), self.cumulative_length.data_ptr()):
            raise ValueError("pool storage changed; capture decoding again")
        for source, target in ((query, self.query), (new_key, self.new_key), (new_value, self.new_value)):
            if source is not None:
                if source.shape != target.shape:
                    raise ValueError(f"decode input must be {tuple(target.shape)}, got {tuple(source.shape)}")
                target.copy_(source)
        self.graph.replay()
        self.seen += 1
        return self.output
