"""The host path refuses to synchronise with the host or build a schedule
cache while a HIP graph is being captured (on the CPU, with capture
simulated): such a step inside capture breaks the capture or records a copy
from host memory that is gone at replay. Once a schedule is cached, the same
calls go through without raising, and what they reach beyond that (the two
native libraries) imports nothing that allocates or synchronises."""

import importlib
import shutil
import subprocess

import pytest
import torch

from white_matter_amd import _native, prepare_cyclic_attention_metadata, prepare_strict_causal_metadata
from white_matter_amd.strict_causal_attention import (
    _covering_schedule,
    _schedule_facts,
    _schedule_gaps,
    _work_units,
)

cyclic_module = importlib.import_module("white_matter_amd.cyclic_attention")


@pytest.fixture
def capturing(monkeypatch):
    state = {"on": False}
    monkeypatch.setattr(torch.cuda, "is_initialized", lambda: True)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: state["on"])
    return state


def test_strict_schedule_steps_refuse_capture_until_cached(capturing):
    docs = torch.tensor([[0, 0, 0, 1, 1, 2], [0, 1, 1, 1, 1, 1]])
    capturing["on"] = True
    with pytest.raises(RuntimeError, match="graph capture"):
        prepare_strict_causal_metadata(docs, 6)
    capturing["on"] = False
    meta = prepare_strict_causal_metadata(docs, 6)
    steps = (
        lambda: _schedule_facts(meta),
        lambda: _covering_schedule(meta, 2, 6, 6),
        lambda: _schedule_gaps(meta, 2, 6, 4, 6, 2),
        lambda: _work_units(meta),
    )
    for step in steps:
        capturing["on"] = True
        with pytest.raises(RuntimeError, match="graph capture"):
            step()
        capturing["on"] = False
        first = step()
        capturing["on"] = True
        assert step() is first  # cached: no host work inside capture
        capturing["on"] = False


def test_cyclic_packer_refuses_capture(capturing):
    ids = torch.tensor([[0, 0, 1, 1, 1, 2, 2, 2]])
    keys = torch.cat((torch.full((1, 1), -1), ids), 1)
    meta = prepare_cyclic_attention_metadata(ids[:, ::2].contiguous(), keys)
    capturing["on"] = True
    with pytest.raises(RuntimeError, match="graph capture"):
        cyclic_module._cyclic_schedule(*meta, 4, 9, 2, 0)
    capturing["on"] = False
    facts = cyclic_module._cyclic_schedule(*meta, 4, 9, 2, 0)[0]
    assert facts.dtype == torch.int64 and int(facts[0]) == 2


def _imported_symbols(library):
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm (binutils) is not installed")
    if not library.exists():
        pytest.skip(f"{library.name} is not built")
    listing = subprocess.run([nm, "-D", "--undefined-only", "-C", str(library)], capture_output=True, text=True, check=True)
    return {line.split(None, 1)[1].split("@")[0] for line in listing.stdout.splitlines() if line.strip()}


def test_libraries_cannot_allocate_copy_or_synchronise():
    """What a captured call can reach once its schedule is cached: the C-ABI
    library imports only kernel launch and registration, error queries and
    device lookups from the HIP runtime (no allocation, copy, fill, event or
    synchronisation), and the C++ operator library only the current stream,
    with no scalar read of a device tensor (`_local_scalar_dense`, which
    .item() and host conversions go through): its memory comes from torch's
    caching allocator, which serves a capture from the graph's pool."""
    attn = {s for s in _imported_symbols(_native.LIBRARY) if s.startswith(("hip", "__hip"))}
    assert attn <= {
        "__hipPopCallConfiguration", "__hipPushCallConfiguration", "__hipRegisterFatBinary", "__hipRegisterFunction",
        "__hipRegisterVar", "__hipUnregisterFatBinary", "hipLaunchKernel", "hipGetLastError", "hipGetErrorString",
        "hipGetDevice", "hipStreamGetDevice", "hipGetSymbolAddress",
    }, attn
    ops = _imported_symbols(_native.OPS_LIBRARY)
    assert not {s for s in ops if s.startswith(("hip", "__hip"))}, "libwmx_torch.so calls the HIP runtime directly"
    assert not [s for s in ops if "_local_scalar_dense" in s or "synchronize" in s.lower()]
    assert {s for s in ops if "c10::hip::" in s} <= {
        "c10::hip::getCurrentHIPStream(signed char)", "c10::hip::HIPStream::stream() const"
    }
