"""The per-block LocalTHC and TriangularLazy models (flowmatching_lthc/models/local_thc.py:759-1153, :1434-1535) on
the CPU: registry, parameter layout against tests/golden/lthc_triangular_layouts.json (written from the reference
by tests/golden/make_triangular_fixture.py), initial values, and the refusals.  Their forward runs on the GPU
only (tests/test_gpu_model_triangular.py).
"""

import json
import os

import pytest
import torch

from flowmatching_lthc_amd import model as M
from flowmatching_lthc_amd import model_triangular as MT

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "lthc_triangular_layouts.json")


@pytest.fixture(scope="module")
def layouts():
    with open(FIXTURE) as f:
        return json.load(f)


def small(cls, **kw):
    """A small model of cls: 64x64 pixels, patch 4, 4x4 workspace, hidden 32, 2 heads."""
    args = dict(input_size=64, patch_size=4, hidden_size=32, depth=12, num_heads=2, bottleneck_dim=8,
                workspace_grid=4, num_classes=10)  # fmt: skip
    args.update(kw)
    return cls(**args)


def test_registry_classes_and_parameter_layout(layouts):
    """build_model builds every recorded name as the reference's class, with its parameter names, order and shapes,
    so a reference state dict loads strictly."""
    assert set(layouts["models"]) == set(MT.PerBlock_JiT_models)
    for name, info in layouts["models"].items():
        model = M.build_model(name)
        assert type(model).__name__ == info["class"], name
        layout = [[k, list(v.shape)] for k, v in model.state_dict().items()]
        assert layout == layouts["layouts"][info["layout"]], name
    state = {k: torch.randn(s) for k, s in layouts["layouts"][layouts["models"][name]["layout"]]}
    model.load_state_dict(state, strict=True)
    assert torch.equal(model.blocks[4].hyper.read_logits, state["blocks.4.hyper.read_logits"])


def test_initial_values():
    """The reference's initialisation: zero read logits (uniform softmax), unit write weights, zeroed AdaLN heads and
    decoder, zero patch-embedding bias."""
    model = M.build_model("TriangularLazy-FusedFinal12-LocalTHC-DirectTriton-SharedAdaLN-JiT-B/4")
    for blk in model.blocks:
        assert torch.all(blk.hyper.read_logits == 0) and torch.all(blk.hyper.write_weight == 1)
    for head in (model.shared_adaLN_modulation[-1], model.shared_final_modulation[-1], model.final_layer.linear):
        assert head.weight.abs().max() == 0 and head.bias.abs().max() == 0
    assert model.x_embedder.proj.bias.abs().max() == 0
    assert model.x_embedder.proj.weight.abs().max() > 0
    alpha = model._expanded_alpha(model.blocks[0], torch.float32)
    assert torch.allclose(alpha, torch.full((768, 16), 1.0 / 16))
    assert torch.equal(model._expanded_beta(model.blocks[0], torch.bfloat16), torch.ones((768, 16), dtype=torch.bfloat16))


def test_old_checkpoint_key_names_load():
    """Old hyper-connection key names (write_logits for the read, read_weight for the write) load into the current
    ones (local_thc.py:41-61)."""
    model = small(MT.LocalTHCDirectTritonTraceableSharedAdaLNJiT)
    state = model.state_dict()
    old = {}
    for k, v in state.items():
        k = k.replace(".read_logits", ".write_logits") if k.endswith(".read_logits") else k
        k = k.replace(".write_weight", ".read_weight") if k.endswith(".write_weight") else k
        old[k] = torch.randn_like(v)
    assert "blocks.3.hyper.write_logits" in old
    model.load_state_dict(old, strict=True)
    assert torch.equal(model.blocks[3].hyper.read_logits, old["blocks.3.hyper.write_logits"])
    assert torch.equal(model.blocks[3].hyper.write_weight, old["blocks.3.hyper.read_weight"])


def test_refusals():
    """The lazy forward keeps the reference's depth of 12; the hyper-connections take only cell side 4 and one
    pool group per channel; there is no CPU fallback."""
    with pytest.raises(ValueError, match="requires depth=12"):
        small(MT.TriangularLazyFusedFinal12LocalTHCDirectTritonSharedAdaLNJiT, depth=6).forward_lazy(
            torch.zeros(1, 3, 64, 64), torch.zeros(1), torch.zeros(1, dtype=torch.long)
        )
    with pytest.raises(ValueError, match="cell side 4"):
        small(MT.LocalTHCTritonSharedAdaLNJiT, workspace_grid=8)
    with pytest.raises(ValueError, match="pool_groups == hidden_size"):
        small(MT.LocalTHCTritonSharedAdaLNJiT, pool_groups=16)
    model = small(MT.TriangularLazyFusedFinal12LocalTHCDirectTritonSharedAdaLNJiT)
    x, t, y = torch.randn(1, 3, 64, 64), torch.rand(1), torch.zeros(1, dtype=torch.long)
    for lazy in (True, False):
        with torch.no_grad(), pytest.raises(ValueError, match="no CPU fallback"):
            model(x, t, y, use_lazy=lazy)
    with pytest.raises(ValueError, match="unknown model"):
        M.build_model("TriangularLazy-FusedFinal24-LocalTHC-B/4")
