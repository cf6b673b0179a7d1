"""The drop-in white_matter/ops tree (white_matter_amd/dropin/ops) on the CPU:
placed where the reference's src/white_matter/ops/ was and imported in the
order the reference's own modules import it, every module path and name those
importers use exists, and every registered white_matter:: operator resolves
to this package's implementation with the reference's schema. torch accepts
a second custom_op registration of a name silently and the last one wins, so
the swap must leave no module that registers these names with other kernels."""

import importlib
import shutil
import sys
from pathlib import Path

import pytest
import torch

DROPIN = Path(__file__).resolve().parents[1] / "white_matter_amd" / "dropin" / "ops"

# (module, names) as the reference's callers import them (grep of
# `from white_matter.ops...` over src/, benchmarks/ and tests/)
IMPORTS = [
    # layers/white_matter.py:16-22
    ("white_matter.ops", ["CyclicAttentionMetadata", "StrictCausalMetadata", "cyclic_attention",
                          "prepare_strict_causal_metadata", "strict_causal_attention",
                          "prepare_cyclic_attention_metadata"]),
    # layers/backends.py:22,61
    ("white_matter.ops.flash_attention", ["TorchFlashDense", "can_use_torch_flash", "torch_flash_decode",
                                          "flash_attention_decode", "TorchFlashVarlen"]),
    # benchmarks/_flop_counter.py:88-90
    ("white_matter.ops.cyclic_attention._tilelang.registration", ["cyclic_attn_fwd", "cyclic_attn_bwd",
                                                                  "cyclic_attn_doc_fwd", "cyclic_attn_doc_bwd"]),
    ("white_matter.ops.strict_causal_attention", ["_standalone_flash_available", "strict_causal_attention",
                                                   "prepare_strict_causal_metadata", "StrictCausalMetadata",
                                                   "can_use_torch_flash", "torch_flash_decode",
                                                   "flash_attention_decode", "TorchFlashDense"]),
    # blocks/_execution/cyclic.py, metadata.py; tests/unit/test_metadata.py
    ("white_matter.ops.cyclic_attention", ["CyclicAttentionMetadata", "cyclic_attention",
                                           "prepare_cyclic_attention_metadata"]),
    ("white_matter.ops.cyclic_attention.functional", ["cyclic_attention"]),
    ("white_matter.ops.cyclic_attention.metadata", ["CyclicAttentionMetadata", "prepare_cyclic_attention_metadata"]),
    ("white_matter.ops.cyclic_attention.reference", ["cyclic_attention_reference"]),
    # tests/gpu/test_cyclic_attention.py
    ("white_matter.ops.cyclic_attention._tilelang.backward_preprocess", ["backward_preprocess"]),
]

# reference schemas: registration.py:164-173,184-196,261-274,280-296; flash_attention.py:15-24,170-173
SCHEMAS = {
    "cyclic_attn_fwd": ["Q", "K", "V", "K_stride", "residue", "block_M"],
    "cyclic_attn_bwd": ["Q", "K", "V", "Out", "Lse", "dOut", "K_stride", "residue", "block_M"],
    "cyclic_attn_doc_fwd": ["Q", "K", "V", "QSeg", "KSeg", "QStart", "KQEnd", "K_stride", "residue", "block_M"],
    "cyclic_attn_doc_bwd": ["Q", "K", "V", "QSeg", "KSeg", "QStart", "KQEnd", "Out", "Lse", "dOut", "K_stride",
                            "residue", "block_M"],
    "flash_attention_decode": ["query", "key", "value", "lengths", "scale", "causal", "num_splits"],
    "torch_flash_dense_forward": ["query", "key", "value", "scale", "causal"],
}


@pytest.fixture
def swapped_tree(tmp_path, monkeypatch):
    root = tmp_path / "src"
    package = root / "white_matter"
    package.mkdir(parents=True)
    # stands in for the reference's package root, which imports models lazily
    (package / "__init__.py").write_text('"""white_matter package root (test stand-in)."""\n')
    shutil.copytree(DROPIN, package / "ops", ignore=shutil.ignore_patterns("__pycache__"))
    monkeypatch.syspath_prepend(str(root))
    yield
    for name in [m for m in sys.modules if m == "white_matter" or m.startswith("white_matter.")]:
        del sys.modules[name]


def test_reference_import_order_resolves_to_this_package(swapped_tree):
    from torch._library.custom_ops import OPDEFS

    for module, names in IMPORTS:
        loaded = importlib.import_module(module)
        for name in names:
            assert hasattr(loaded, name), f"{module} lacks {name}"
    python_ops = {name.split("::")[1] for name in OPDEFS if name.startswith("white_matter::")}
    for name in python_ops:
        implementation = OPDEFS[f"white_matter::{name}"]._init_fn
        assert implementation.__module__.startswith("white_matter_amd."), (name, implementation.__module__)
    for name in set(SCHEMAS) - python_ops:
        # registered from C++: every kernel of the operator comes from this package's library
        dump = torch._C._dispatch_dump(f"white_matter::{name}")
        kernels = [line for line in dump.splitlines() if line.startswith(("CUDA:", "Autograd", "debug:"))]
        assert kernels and all("white_matter_amd/csrc/torch_ops.cpp" in line for line in kernels), (name, dump)
    for name, arguments in SCHEMAS.items():
        schema = getattr(torch.ops.white_matter, name).default._schema
        assert [a.name for a in schema.arguments] == arguments, name


def test_dropin_names_are_this_packages_objects(swapped_tree):
    import white_matter_amd
    from white_matter_amd import flash_attention

    ops = importlib.import_module("white_matter.ops")
    assert ops.strict_causal_attention is white_matter_amd.strict_causal_attention
    assert ops.cyclic_attention is white_matter_amd.cyclic_attention
    fa = importlib.import_module("white_matter.ops.flash_attention")
    assert fa.flash_attention_decode is flash_attention.flash_attention_decode
    assert fa.TorchFlashDense is flash_attention.TorchFlashDense
    sca = importlib.import_module("white_matter.ops.strict_causal_attention")
    assert sca._standalone_flash_available() is False


def test_can_use_torch_flash_on_the_cpu():
    """The capability check is shape/dtype logic that a compiled region can
    trace (reference tests/unit/test_compilation_policy.py:15-31): CPU
    operands are never taken by the HIP kernels."""
    from white_matter_amd.flash_attention import can_use_torch_flash

    x = torch.randn(2, 1, 2, 8)
    assert can_use_torch_flash(x, x, x) is False

    @torch.compiler.nested_compile_region
    def region(x):
        query = x.sin()
        return query + int(can_use_torch_flash(query, query, query))

    def forward(x):
        return region(x.cos())

    compiled = torch.compile(forward, backend="aot_eager", fullgraph=True)
    torch.testing.assert_close(compiled(x), forward(x))
