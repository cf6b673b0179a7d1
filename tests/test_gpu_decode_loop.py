"""The captured decode step (DecodeLoop): every replay equals the same work
launched eagerly on a copy of the pool, bit for bit, over several tokens
with new inputs each time; the attention outputs match the float64 oracle
over the pool as it stood; the stored keys match the KV-store oracle; and
the slot counter advances on the device (the attention side of reference
models/generation.py:38-100 over models/cache.py:13-273)."""

import pytest
import torch

from oracle import attention as ref
from oracle import kv_pool as kv_ref
from tests.numerics import assert_bf16_close
from white_matter_amd import DecodeLoop, kv_pool, strict_causal_attention

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _setup(batch=3, channels=2, kv_heads=2, dim=64, capacity=40, prefix=11, seed=0):
    gen = torch.Generator().manual_seed(seed)
    keys = torch.full((batch, channels * kv_heads, capacity, dim), float("nan"), dtype=torch.bfloat16)
    values = keys.clone()
    used = prefix + 1  # the dummy slot and the prefix
    keys[:, :, :used] = torch.randn(batch, channels * kv_heads, used, dim, generator=gen).bfloat16()
    values[:, :, :used] = torch.randn(batch, channels * kv_heads, used, dim, generator=gen).bfloat16()
    weight = (1 + 0.1 * torch.randn(channels, dim, generator=gen)).float()
    angle = torch.arange(capacity)[:, None].float() * torch.logspace(0, -3, dim // 2)[None]
    angle = torch.cat((angle, angle), -1)
    return keys.to(DEV), values.to(DEV), torch.tensor([used], device=DEV), weight.to(DEV), angle.cos().to(DEV), angle.sin().to(DEV)


def _eager_step(keys, values, length, channels_of_layer, weight, cos, sin, query, new_key, new_value, kv_heads):
    batch, _, _, dim = keys.shape
    lengths = (length - 1).expand(batch)
    outs = []
    for layer, c in enumerate(channels_of_layer):
        k, v = keys[:, c * kv_heads : (c + 1) * kv_heads], values[:, c * kv_heads : (c + 1) * kv_heads]
        outs.append(strict_causal_attention(query[layer], k, v, query_start=lengths, kv_lengths=lengths, use_dummy_token=True))
    pool_k = keys.unflatten(1, (weight.shape[0], kv_heads))
    pool_v = values.unflatten(1, (weight.shape[0], kv_heads))
    kv_pool.write_pool(new_key, new_value, weight, cos[length].expand(batch, 1, dim), sin[length].expand(batch, 1, dim),
                       pool_k, pool_v, length)
    length.add_(1)
    return torch.stack(outs)


@torch.inference_mode()
def test_replays_equal_eager_and_oracle():
    keys, values, length, weight, cos, sin = _setup()
    layer_channels = (0, 1, 0)
    heads, kv_heads = 4, 2
    loop = DecodeLoop(keys, values, length, layer_channels, weight, cos, sin, query_heads=heads)
    e_keys, e_values, e_length = keys.clone(), values.clone(), length.clone()
    gen = torch.Generator().manual_seed(5)
    for step in range(6):
        print(f"decode step {step}", flush=True)
        query = torch.randn(3, 3, heads, 1, 64, generator=gen).bfloat16().to(DEV)
        new_key = (2 * torch.randn(3, 2, kv_heads, 1, 64, generator=gen)).bfloat16().to(DEV)
        new_value = torch.randn(3, 2, kv_heads, 1, 64, generator=gen).bfloat16().to(DEV)
        before_k, before_v, used = keys.clone(), values.clone(), int(length.item())
        out = loop(query, new_key, new_value)
        torch.cuda.synchronize()
        expected = _eager_step(e_keys, e_values, e_length, layer_channels, weight, cos, sin, query, new_key, new_value, kv_heads)
        torch.cuda.synchronize()
        assert torch.equal(out, expected), f"step {step}: replay differs from eager launches"
        same_bits = lambda a, b: torch.equal(a.view(torch.int16), b.view(torch.int16))  # noqa: E731 (NaN slots)
        assert same_bits(keys, e_keys) and same_bits(values, e_values), f"step {step}: pool differs"
        assert int(length.item()) == used + 1 == loop.seen
        for layer, c in enumerate(layer_channels):
            kk = before_k[:, c * kv_heads : (c + 1) * kv_heads].cpu()
            vv = before_v[:, c * kv_heads : (c + 1) * kv_heads].cpu()
            starts = torch.full((3,), used - 1)
            want = ref.per_query_strict(query[layer].cpu(), kk, vv, starts, True, lengths=starts)
            assert_bf16_close(out[layer].double().cpu(), want, what=f"step {step} layer {layer}")
        stored = keys[:, :, used].unflatten(1, (2, kv_heads)).cpu()  # (B, C, H, D)
        want_k = kv_ref.k_norm_rope(new_key.cpu(), weight.cpu(), cos[used].expand(3, 1, 64).cpu(),
                                    sin[used].expand(3, 1, 64).cpu(), 1e-6).bfloat16()[:, :, :, 0]
        assert (stored.double() == want_k.double()).double().mean() >= 0.99
        assert torch.equal(values[:, :, used].cpu(), new_value[:, :, :, 0].flatten(1, 2).cpu())


@torch.inference_mode()
def test_full_pool_and_moved_storage_are_rejected():
    keys, values, length, weight, cos, sin = _setup(capacity=14, prefix=11)  # 12 slots used, 2 free
    loop = DecodeLoop(keys, values, length, (0,), weight, cos, sin, query_heads=2)
    loop()
    loop()
    with pytest.raises(ValueError, match="pool is full"):
        loop()
    keys2, values2, length2, weight2, cos2, sin2 = _setup(capacity=20)
    loop2 = DecodeLoop(keys2, values2, length2, (1,), weight2, cos2, sin2, query_heads=2)
    loop2.keys = keys2.clone()
    with pytest.raises(ValueError, match="storage changed"):
        loop2()
