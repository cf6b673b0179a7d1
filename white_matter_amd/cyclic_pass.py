"""Cyclic prefill passes and cached decoding of a minimal WhiteMatter model
over the HIP kernels: the end-to-end harness of the attention path.

Inference restatement of the reference's feedback block:

  * `forward_cyclic` (src/white_matter/blocks/_execution/cyclic.py:119-275,
    the bounded inference schedule): the pool starts from the embeddings
    written for every source (and the leading dummy slot), then `passes`
    passes run the strided token groups over the same block input;
  * `cyclic_pass` (cyclic.py:276-431 `run_pass`, the pool_chunk_size branch;
    `_group_layers` :461-489): group c's tokens c, c+G, ... run through every
    layer, layer l reading pool channel l % k with `cyclic_attention`
    (query_stride G, query_offset c), and the group's layer inputs plus the
    top output are projected and written into the pool before group c+1;
  * the layer (blocks/decoder_layer.py:33-72 `FeedbackDecoderLayer`,
    layers/white_matter.py:98-199 `WhiteMatterAttention`): pre-norm
    attention with a local Q projection, q-norm and RoPE, and a gated MLP;
  * the pool projection (modules/kv_pool.py:97-217 `KVPool._project`,
    `project_sequence`; modules/routing.py:46-124 `Router`, `_RoutedMixer`):
    RMS norm, per-source premix, content routers over every second of the
    L+1 sources (router_layer_stride 2, the reference configuration's
    default), mix norm, gains and the per-channel projection: the norms, premix, routed
    sum and gains run as two HIP kernels around the router GEMM
    (`kv_pool.projection_inputs`), the K-norm, RoPE, bf16 cast and pool write
    as one (`kv_pool.write_pool`);
  * cached decoding (models/generation.py:38-100 `DecodeGraph`,
    blocks/white_matter.py:165-186 `_run_token_layers`): one token through
    every layer with the split-K decode kernel over the pool, the token's
    keys and values stored at the next slot, captured in a HIP graph.

The model is random-initialised (no checkpoints): projections N(0, 0.02),
norms and gains one, routers at the reference's "cyclic:0.25" prior with zero
weights (routing.py:9-42, 77-80), dummy token zero. Out of scope: training
passes (compact histories, checkpointing, gradient passes), padding masks,
the LCKV fixed-source mixer and sampling other than greedy.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import kv_pool
from .cyclic_attention import cyclic_attention
from .metadata import prepare_feedback_metadata
from .strict_causal_attention import strict_causal_attention


@dataclass(frozen=True)
class FeedbackConfig:
    """Dimensions of the model (defaults: the C5 workload, Hq/Hkv = 2 as in the
    reference's recipes; intermediate size 3 x hidden as in its Qwen3 shapes)."""

    vocab_size: int = 151936
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_layers: int = 24
    num_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 64
    num_kv_channels: int = 8
    cyclic_groups: int = 8
    num_passes: int = 3
    use_dummy_token: bool = True
    rope_theta: float = 1.0e6
    rms_norm_eps: float = 1.0e-6
    mix_norm_eps: float = 1.0e-4  # kv_pool.py:58
    router_peak: float = 0.25  # the "cyclic:0.25" prior
    # sources the router reads: every router_layer_stride-th from the top
    # (configuration_white_matter.py:16, modules/routing.py:66-72)
    router_layer_stride: int = 2

    @property
    def num_sources(self) -> int:  # the block input and every layer output
        return self.num_layers + 1


class HipKernels:
    """The attention-path operations of the pass and of decoding, on the HIP
    kernels. q is (B, Hq, T, D); the pool views are (B, Hkv, N, D)."""

    @staticmethod
    def cyclic(q, k, v, *, query_stride, query_offset, strict_past, metadata):
        """(B, Hq, T, D) -> (B, T, Hq, D), as layers/white_matter.py:168-184."""
        out = cyclic_attention(
            q, k, v, query_stride=query_stride, query_offset=query_offset, strict_past=strict_past,
            metadata=metadata, backend="tilelang",
        )
        return out.transpose(1, 2)

    @staticmethod
    def decode(q, k, v, *, lengths, use_dummy_token, key_mask):
        """One query per row over the pool's committed slots -> (B, 1, Hq, D)."""
        return strict_causal_attention(
            q, k, v, query_start=lengths, kv_lengths=lengths, use_dummy_token=use_dummy_token, key_mask=key_mask
        )

    @staticmethod
    def store(key, value, k_norm_weight, cos, sin, keys, values, slots, *, eps):
        kv_pool.write_pool(key, value, k_norm_weight, cos, sin, keys, values, slots, eps=eps)

    @staticmethod
    def mix(model: "FeedbackModel", stacked):
        """The projection inputs (k, B T, d) per side on the HIP kernels."""
        c = model.config
        return kv_pool.projection_inputs(
            stacked, (model.pre_mix["k"], model.pre_mix["v"]), (model.router["k"], model.router["v"]),
            (model.gain["k"], model.gain["v"]), eps=c.rms_norm_eps, mix_eps=c.mix_norm_eps,
            router_layer_stride=c.router_layer_stride,
        )


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def document_positions(document_ids: torch.Tensor) -> torch.Tensor:
    """Positions restarting at every document (modules/documents.py:23-27)."""
    length = document_ids.shape[1]
    positions = torch.arange(length, device=document_ids.device).expand_as(document_ids)
    starts = torch.ones_like(document_ids, dtype=torch.bool)
    starts[:, 1:] = document_ids[:, 1:] != document_ids[:, :-1]
    return positions - torch.where(starts, positions, 0).cummax(dim=1).values


class FeedbackModel:
    """Weights and the token-local parts of the model (embedding, layers,
    pool projection, head). `dtype` is the activation and weight type (bf16
    on the GPU), `residual_dtype` that of the residual stream and of the
    norms' arithmetic (the reference's default "fp32" residual policy)."""

    def __init__(
        self,
        config: FeedbackConfig,
        *,
        device: torch.device | str = "cuda",
        dtype: torch.dtype = torch.bfloat16,
        residual_dtype: torch.dtype = torch.float32,
        seed: int = 0,
    ) -> None:
        c = config
        if c.num_heads % c.num_kv_heads or not 1 <= c.num_kv_channels <= c.num_sources:
            raise ValueError("num_heads must be a multiple of num_kv_heads and 1 <= num_kv_channels <= L + 1")
        self.config, self.device, self.dtype, self.residual_dtype = c, torch.device(device), dtype, residual_dtype
        gen = torch.Generator(device=self.device).manual_seed(seed)

        def normal(*shape):
            return (torch.randn(*shape, generator=gen, device=self.device) * 0.02).to(dtype)

        def ones(*shape):
            return torch.ones(*shape, device=self.device, dtype=dtype)

        d, hd, kvd = c.hidden_size, c.num_heads * c.head_dim, c.num_kv_heads * c.head_dim
        k, s = c.num_kv_channels, c.num_sources
        self.embed = normal(c.vocab_size, d)  # tied with the output head
        self.layers = [
            dict(
                input_norm=ones(d), q_proj=normal(hd, d), q_norm=ones(c.head_dim), o_proj=normal(d, hd),
                post_norm=ones(d), gate=normal(c.intermediate_size, d), up=normal(c.intermediate_size, d),
                down=normal(d, c.intermediate_size),
            )
            for _ in range(c.num_layers)
        ]
        self.final_norm = ones(d)
        self.dummy = torch.zeros(d, device=self.device, dtype=dtype)
        self.pre_mix = {side: ones(s, d) for side in "kv"}
        prior = torch.zeros(k, s)
        for col in range(s):  # routing.py:18-25, rows < cols
            prior[col % k, col] = c.router_peak
        self.router_read = kv_pool.router_sources(s, c.router_layer_stride)
        self.router = {
            side: (
                torch.zeros(k * s, len(self.router_read) * d, device=self.device, dtype=dtype),
                prior.reshape(-1).to(self.device, dtype),
            )
            for side in "kv"
        }
        self.gain = {side: ones(k, d) for side in "kv"}
        # per-channel projections stored as (k, d, Hkv * D): the batched product's
        # right operand is then contiguous
        self.proj = {side: normal(k, kvd, d).transpose(1, 2).contiguous() for side in "kv"}
        self.k_norm = ones(k, c.head_dim)
        self.inv_freq = 1.0 / (c.rope_theta ** (torch.arange(0, c.head_dim, 2, dtype=torch.float64) / c.head_dim))
        self.inv_freq = self.inv_freq.float().to(self.device)

    # -- token-local pieces ---------------------------------------------------
    def rope(self, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """cos, sin (B, T, D) in the residual dtype (modules/rotary.py:66-78)."""
        freqs = positions.float()[..., None] * self.inv_freq
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(self.residual_dtype), emb.sin().to(self.residual_dtype)

    def _norm(self, x: torch.Tensor, weight: torch.Tensor, eps: float | None = None) -> torch.Tensor:
        eps = self.config.rms_norm_eps if eps is None else eps
        x = F.rms_norm(x.to(self.residual_dtype), (x.shape[-1],), None, eps)
        return (x * weight.to(self.residual_dtype)).to(self.dtype)

    def layer(self, index: int, x: torch.Tensor, attend, rope) -> torch.Tensor:
        """decoder_layer.py:51-72 with layers/white_matter.py:109-116, 199:
        x (B, T, d) residual; attend(q (B, Hq, T, D)) -> (B, T, Hq, D)."""
        c, p = self.config, self.layers[index]
        batch, length, _ = x.shape
        h = self._norm(x, p["input_norm"])
        q = (h @ p["q_proj"].t()).view(batch, length, c.num_heads, c.head_dim)
        q = self._norm(q, p["q_norm"]).transpose(1, 2).to(self.residual_dtype)
        cos, sin = (t[:, None] for t in rope)
        q = (q * cos + _rotate_half(q) * sin).to(self.dtype)
        out = attend(q).reshape(batch, length, c.num_heads * c.head_dim)
        x = x + (out @ p["o_proj"].t()).to(self.residual_dtype)
        h = self._norm(x, p["post_norm"])
        mlp = (F.silu(h @ p["gate"].t()) * (h @ p["up"].t())) @ p["down"].t()
        return x + mlp.to(self.residual_dtype)

    def layers_forward(self, x: torch.Tensor, attend_layer, rope) -> tuple[torch.Tensor, list[torch.Tensor]]:
        """run_feedback_layers (decoder_layer.py:75-94) with the top output kept:
        returns the output and the L + 1 pool sources."""
        states = []
        for index in range(self.config.num_layers):
            states.append(x)
            x = self.layer(index, x, lambda q, i=index: attend_layer(i, q), rope)
        states.append(x)
        return x, states

    def projection_inputs(self, stacked: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """KVPool._project up to the projection (kv_pool.py:97-136, routing.py:
        108-124) as torch operations: (B, T, S, d) sources -> the K and V
        projection inputs (k, B T, d) in the activation dtype."""
        c = self.config
        batch, length, sources, d = stacked.shape
        normed = F.rms_norm(stacked.to(self.residual_dtype), (d,), None, c.rms_norm_eps)
        out = []
        for side in "kv":
            premixed = (normed * self.pre_mix[side].to(self.residual_dtype)).to(self.dtype)  # (B, T, S, d)
            weight, bias = self.router[side]
            read = self.router_read
            context = premixed[:, :, read.start :: read.step].reshape(batch, length, len(read) * d)
            alpha = F.linear(context, weight, bias)
            alpha = alpha.view(batch, length, c.num_kv_channels, sources)
            mixed = torch.matmul(alpha, premixed)  # (B, T, k, d): sum over sources
            mixed = F.rms_norm(mixed.to(self.residual_dtype), (d,), None, c.mix_norm_eps)
            mixed = (mixed * self.gain[side].to(self.residual_dtype)).to(self.dtype)
            out.append(mixed.permute(2, 0, 1, 3).reshape(c.num_kv_channels, batch * length, d))
        return out[0], out[1]

    def project(self, stacked: torch.Tensor, kernels=None) -> tuple[torch.Tensor, torch.Tensor]:
        """KVPool._project (kv_pool.py:97-160): (B, T, S, d) sources -> raw keys
        and values (B, k, Hkv, T, D) in the activation dtype (views). The
        projection inputs come from `kernels.mix` where the kernel set has one
        (the HIP producer), else from the torch operations."""
        c = self.config
        batch, length = stacked.shape[:2]
        mix = getattr(kernels, "mix", None)
        rows = mix(self, stacked) if mix is not None else self.projection_inputs(stacked)
        out = []
        for side, r in zip("kv", rows, strict=True):
            proj = torch.bmm(r, self.proj[side])  # (k, B T, Hkv D)
            out.append(
                proj.view(c.num_kv_channels, batch, length, c.num_kv_heads, c.head_dim).permute(1, 0, 3, 2, 4)
            )
        return out[0], out[1]

    def logits(self, x: torch.Tensor) -> torch.Tensor:
        """Tied output head on the final norm."""
        return self._norm(x, self.final_norm) @ self.embed.t()

    def new_pool(self, batch: int, capacity: int) -> tuple[torch.Tensor, torch.Tensor]:
        c = self.config
        shape = (batch, c.num_kv_channels, c.num_kv_heads, capacity, c.head_dim)
        keys = torch.zeros(shape, device=self.device, dtype=self.dtype)
        return keys, torch.zeros_like(keys)


@torch.no_grad()
def write_sources(model: FeedbackModel, stacked, keys, values, slots, rope, kernels=HipKernels, chunk: int = 512):
    """Project (B, T, S, d) sources and write them into pool slots `slots`
    (cyclic.py:435-446 `_write_pool`), in token chunks that bound the
    temporaries (kv_pool.py:189-211)."""
    cos, sin = rope
    for start in range(0, stacked.shape[1], chunk):
        stop = min(start + chunk, stacked.shape[1])
        key, value = model.project(stacked[:, start:stop], kernels)
        kernels.store(
            key, value, model.k_norm, cos[:, start:stop], sin[:, start:stop], keys, values, slots[start:stop],
            eps=model.config.rms_norm_eps,
        )


@torch.no_grad()
def cyclic_pass(model: FeedbackModel, x, keys, values, groups, rope, metadata=None, kernels=HipKernels):
    """One pass over the token groups (cyclic.py:357-431, pool_chunk_size branch).

    x (B, T, d) the block input (residual dtype); keys/values the pool
    (B, k, Hkv, N, D), slot s + dummy holding token s; groups[c] the token
    slots c, c + G, ...; rope = (cos, sin) (B, T, D) of the query positions
    (a token's key uses its query position: cyclic.py:41-44); metadata the
    per-group cyclic metadata or None. Returns the pass output (B, T, d); the
    pool is updated in place, group by group."""
    c = model.config
    offset, length = int(c.use_dummy_token), x.shape[1]
    out = torch.empty_like(x)
    readers = [(keys[:, ch, :, :length], values[:, ch, :, :length]) for ch in range(c.num_kv_channels)]
    for g, positions in enumerate(groups):
        group_rope = tuple(t.index_select(1, positions) for t in rope)

        def attend(index, q, g=g):
            k, v = readers[index % c.num_kv_channels]
            return kernels.cyclic(
                q, k, v, query_stride=len(groups), query_offset=g, strict_past=not c.use_dummy_token,
                metadata=None if metadata is None else metadata[g],
            )

        h, states = model.layers_forward(x.index_select(1, positions), attend, group_rope)
        out.index_copy_(1, positions, h)
        write_sources(model, torch.stack(states, dim=2), keys, values, positions + offset, group_rope, kernels)
    return out


@torch.no_grad()
def forward_cyclic(
    model: FeedbackModel,
    input_ids: torch.Tensor,
    document_ids: torch.Tensor | None = None,
    *,
    capacity: int | None = None,
    passes: int | None = None,
    kernels=HipKernels,
):
    """The block's cyclic forward for inference (cyclic.py:119-275): returns
    the last pass's output (B, T, d), the pool (keys, values) with `capacity`
    slots (default T + dummy) and the query positions (B, T)."""
    c = model.config
    batch, length = input_ids.shape
    offset, groups_n = int(c.use_dummy_token), c.cyclic_groups
    if length <= groups_n:
        raise ValueError("the harness needs more tokens than cyclic groups (no padding path)")
    capacity = length + offset if capacity is None else capacity
    if capacity < length + offset:
        raise ValueError("capacity must hold every token and the dummy slot")
    device = input_ids.device
    x = model.embed[input_ids].to(model.residual_dtype)
    if document_ids is None:
        positions = torch.arange(length, device=device).expand(batch, length)
    else:
        positions = document_positions(document_ids)
    rope = model.rope(positions + offset)  # real positions follow the dummy (white_matter.py:59-73)
    keys, values = model.new_pool(batch, capacity)

    # the pool starts from the embeddings of every source (cyclic.py:221-229)
    initial = x
    key_rope = rope
    if offset:  # the dummy slot sits at position 0 (white_matter.py:70-71)
        initial = torch.cat((model.dummy.to(x.dtype).expand(batch, 1, -1), x), dim=1)
        dummy_rope = model.rope(torch.zeros(batch, 1, device=device))
        key_rope = tuple(torch.cat((d, t), dim=1) for d, t in zip(dummy_rope, rope))
    stacked = initial[:, :, None].expand(-1, -1, c.num_sources, -1)
    write_sources(model, stacked, keys, values, torch.arange(length + offset, device=device), key_rope, kernels)

    groups = [torch.arange(g, length, groups_n, device=device) for g in range(groups_n)]
    metadata = None
    if document_ids is not None:
        metadata = prepare_feedback_metadata(document_ids, groups, length, use_dummy_token=c.use_dummy_token)
    hidden = x
    for _ in range(c.num_passes if passes is None else passes):
        hidden = cyclic_pass(model, x, keys, values, groups, rope, metadata, kernels)
    return hidden, keys, values, positions


class GreedyDecoder:
    """Greedy decoding after a cyclic prefill, one token per HIP-graph replay
    (generation.py:38-100 `DecodeGraph`; white_matter.py:165-186): the token
    runs through every layer, layer l attending from its query to pool channel
    l % k over the committed slots (the dummy and the row's last document,
    then every decoded token), and its keys and values are written at the next
    slot. Static buffers, readable and writable between calls: `token` (B, 1)
    the next input token, `position` (B, 1) its position (before the dummy
    shift), `length` (1,) the slots in use (dummy included; the token is
    written there), `key_mask` (B, N) the slots it may read."""

    @torch.no_grad()
    def __init__(self, model: FeedbackModel, keys, values, length: int, position, token, key_mask, *,
                 kernels=HipKernels, capture: bool = True) -> None:
        self.model, self.keys, self.values, self.kernels = model, keys, values, kernels
        self.capacity = keys.shape[3]
        device = keys.device
        if key_mask.shape != (keys.shape[0], self.capacity) or key_mask.dtype != torch.bool:
            raise ValueError("key_mask must be boolean (B, N)")
        self.length = torch.full((1,), length, device=device, dtype=torch.long)
        self.position = position.to(device=device, dtype=torch.long).reshape(-1, 1).clone()
        self.token = token.to(device=device, dtype=torch.long).reshape(-1, 1).clone()
        self.key_mask = key_mask.clone()
        self.graph = None
        if capture:
            snapshot = (self.length.clone(), self.position.clone(), self.token.clone(), self.key_mask.clone())
            stream = torch.cuda.Stream(device=device)
            stream.wait_stream(torch.cuda.current_stream(device))
            with torch.cuda.stream(stream):
                self.step()  # warm-up launch outside the capture
            torch.cuda.current_stream(device).wait_stream(stream)
            for t, s in zip((self.length, self.position, self.token, self.key_mask), snapshot):
                t.copy_(s)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph):
                self.step()
            for t, s in zip((self.length, self.position, self.token, self.key_mask), snapshot):
                t.copy_(s)
            torch.cuda.current_stream(device).synchronize()
        self.seen = length

    @classmethod
    @torch.no_grad()
    def after_prefill(cls, model: FeedbackModel, hidden, keys, values, positions, document_ids=None, **kwargs):
        """Continue the row's last document after `forward_cyclic`: the first
        input is the greedy token of the last position; it reads the dummy and
        its document's slots (documents.py:57-61 `feedback_document_mask`)."""
        batch, length = positions.shape
        offset = int(model.config.use_dummy_token)
        keep = torch.zeros(batch, keys.shape[3], device=keys.device, dtype=torch.bool)
        same = torch.ones(batch, length, device=keys.device, dtype=torch.bool)
        if document_ids is not None:
            same = document_ids == document_ids[:, -1:]
        keep[:, offset : length + offset] = same
        if offset:
            keep[:, 0] = True
        token = model.logits(hidden[:, -1:]).argmax(-1)
        return cls(model, keys, values, length + offset, positions[:, -1:] + 1, token, keep, **kwargs)

    def step(self) -> None:
        """One token as eager launches on the current stream (what the graph holds)."""
        model, c = self.model, self.model.config
        batch = self.token.shape[0]
        offset = int(c.use_dummy_token)
        x = model.embed[self.token].to(model.residual_dtype)  # (B, 1, d)
        rope = model.rope(self.position + offset)
        lengths = (self.length - offset).expand(batch).contiguous()

        def attend(index, q):
            ch = index % c.num_kv_channels
            return self.kernels.decode(
                q, self.keys[:, ch], self.values[:, ch], lengths=lengths, use_dummy_token=c.use_dummy_token,
                key_mask=self.key_mask,
            )

        x, states = model.layers_forward(x, attend, rope)
        slot = self.length
        key, value = model.project(torch.stack(states, dim=2), self.kernels)
        self.kernels.store(key, value, model.k_norm, rope[0], rope[1], self.keys, self.values, slot,
                           eps=c.rms_norm_eps)
        self.key_mask.index_fill_(1, slot, True)
        self.length.add_(1)
        self.position.add_(1)
        self.token.copy_(model.logits(x).argmax(-1))

    @torch.no_grad()
    def __call__(self) -> torch.Tensor:
        """Decode one token; returns the (B, 1) greedy token (a borrowed buffer)."""
        if self.seen >= self.capacity:
            raise ValueError("the pool is full: no slot left for a decoding token")
        if self.graph is not None:
            self.graph.replay()
        else:
            self.step()
        self.seen += 1
        return self.token
