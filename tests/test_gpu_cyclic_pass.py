"""The cyclic pass driver and captured greedy decoding on the HIP kernels, for
a small bf16 model with C5's head_dim (64), packed documents, the dummy slot
and two passes.

Three runs share the weights: the bf16 model on the HIP kernels, the bf16
model on the float64 oracle's attention and KV store (results rounded to
bf16), and the same weights as a float32 model on the oracle. Every bf16 cast
of the model (norm outputs, projections, keys and values) adds rounding noise
of its own, so two bf16 runs drift apart by more than one operation's bf16
bar over layers, passes and the pool's feedback. The bar here: against the
float32 run, the HIP run's relative L2 error is at most 1.5x that of the
oracle-kernel bf16 run (the kernels add no more error than bf16 arithmetic
does), and its max-abs error is within the bf16 bar. Decoding is
teacher-forced: the other runs are given the tokens the HIP run chose, and
the pool slots each token writes are compared the same way."""

import pytest
import torch

from tests.test_cyclic_pass import OracleKernels
from white_matter_amd.cyclic_pass import FeedbackConfig, FeedbackModel, GreedyDecoder, HipKernels, forward_cyclic

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _setup(dummy=True):
    config = FeedbackConfig(
        vocab_size=96, hidden_size=128, intermediate_size=256, num_layers=3, num_heads=4, num_kv_heads=2,
        head_dim=64, num_kv_channels=2, cyclic_groups=4, num_passes=2, use_dummy_token=dummy,
    )
    model = FeedbackModel(config, device=DEV, seed=5)
    exact = FeedbackModel(config, device=DEV, dtype=torch.float32, seed=5)
    # the float32 model holds the bf16 model's weights exactly
    exact.embed, exact.final_norm, exact.dummy, exact.k_norm = (
        t.float() for t in (model.embed, model.final_norm, model.dummy, model.k_norm)
    )
    exact.layers = [{name: t.float() for name, t in layer.items()} for layer in model.layers]
    for side in "kv":
        exact.pre_mix[side], exact.gain[side], exact.proj[side] = (
            t.float() for t in (model.pre_mix[side], model.gain[side], model.proj[side])
        )
        exact.router[side] = tuple(t.float() for t in model.router[side])
    gen = torch.Generator().manual_seed(7)
    ids = torch.randint(0, 96, (2, 64), generator=gen).to(DEV)
    docs = torch.tensor([[0] * 20 + [1] * 30 + [2] * 14, [0] * 7 + [1] * 41 + [2] * 16]).to(DEV)
    return model, exact, ids, docs


def _rel_l2(a, e):
    a, e = a.double().cpu(), e.double().cpu()
    return float((a - e).norm() / e.norm()), float((a - e).abs().max()), float(e.abs().max())


def _check(hip, ref, exact, what):
    r_hip, m_hip, scale = _rel_l2(hip, exact)
    r_ref, _, _ = _rel_l2(ref, exact)
    print(f"{what}: rel_l2 hip {r_hip:.3e} bf16-oracle {r_ref:.3e}, max_abs hip {m_hip:.3e}", flush=True)
    assert r_hip <= 1.5 * r_ref + 1e-6, f"{what}: HIP rel_l2 {r_hip:.3e} vs bf16 oracle run {r_ref:.3e}"
    assert m_hip <= 1e-2 * max(1.0, scale), f"{what}: max_abs {m_hip:.3e}"


@pytest.mark.parametrize("dummy", [True, False])
def test_prefill_matches_oracle_kernels(dummy):
    model, exact, ids, docs = _setup(dummy)
    print(f"cyclic pass prefill, dummy {dummy}", flush=True)
    hip = forward_cyclic(model, ids, docs, kernels=HipKernels)
    ref = forward_cyclic(model, ids, docs, kernels=OracleKernels)
    full = forward_cyclic(exact, ids, docs, kernels=OracleKernels)
    torch.cuda.synchronize()
    for index, name in enumerate(("pass output", "pool keys", "pool values")):
        _check(hip[index], ref[index], full[index], name)


def test_captured_decoding_matches_oracle_kernels():
    model, exact, ids, docs = _setup()
    steps = 4
    capacity = ids.shape[1] + 1 + steps
    print("cyclic pass decode", flush=True)
    runs = []
    for m, kernels in ((model, HipKernels), (model, OracleKernels), (exact, OracleKernels)):
        runs.append(forward_cyclic(m, ids, docs, capacity=capacity, kernels=kernels))
    h, k, v, pos = runs[0]
    hip = GreedyDecoder.after_prefill(model, h, k, v, pos, docs)  # captured
    eager = GreedyDecoder.after_prefill(model, h, k.clone(), v.clone(), pos, docs, capture=False)
    ref = GreedyDecoder.after_prefill(model, *runs[1], docs, kernels=OracleKernels, capture=False)
    full = GreedyDecoder.after_prefill(exact, *runs[2], docs, kernels=OracleKernels, capture=False)
    for step in range(steps):
        slot = ids.shape[1] + 1 + step
        for other in (eager, ref, full):
            other.token.copy_(hip.token)
        for decoder in (hip, eager, ref, full):
            decoder()
        torch.cuda.synchronize()
        for name in ("keys", "values"):
            got, want, exp = (getattr(d, name)[..., slot, :] for d in (hip, ref, full))
            _check(got, want, exp, f"decode step {step} {name}")
            assert torch.equal(got, getattr(eager, name)[..., slot, :]), \
                "graph replay and eager launches must store the same token"
    assert int(hip.length) == capacity and bool(hip.key_mask[:, -steps:].all())
