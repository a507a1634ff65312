"""The v2 models (flowmatching_lthc/models/lthc_v2/model.py) on the CPU: registry, parameter layout and the three
modules v2 adds, against tests/golden/lthc_v2_fixture.pt (written from the reference by
tests/golden/make_v2_fixture.py).  The v2 forward runs on the GPU only (tests/test_gpu_model_v2.py).
"""

import os

import pytest
import torch

from flowmatching_lthc_amd import model as M
from flowmatching_lthc_amd import model_v2 as V

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "lthc_v2_fixture.pt")
V2_NAMES = {
    "local_thc_v2_fused_final12_shared_adaln_b4": "LocalTHCv2-FusedFinal12-SharedAdaLN-JiT-B/4",
    "local_thc_v2_fused_final12_adaln_b4": "LocalTHCv2-FusedFinal12-AdaLN-JiT-B/4",
    "local_thc_v2_direct_fused_final12_shared_adaln_b4": "LocalTHCv2-Direct-FusedFinal12-SharedAdaLN-JiT-B/4",
    "local_thc_v2_direct_fused_final12_adaln_b4": "LocalTHCv2-Direct-FusedFinal12-AdaLN-JiT-B/4",
}


@pytest.fixture(scope="module")
def fixture():
    return torch.load(FIXTURE, weights_only=True)


def close(got, ref, tol=1e-5):
    err = (got - ref).abs().max().item() / max(ref.abs().max().item(), 1e-30)
    assert err <= tol, f"max|d|/max|ref| = {err:.3e}"


@pytest.mark.parametrize("name", list(V2_NAMES))
def test_v2_registry_and_parameter_layout(fixture, name):
    """build_model builds each v2 name with the reference's parameter names, order and shapes, so a reference
    state dict loads strictly."""
    model = M.build_model(name)
    assert isinstance(model, V._LocalTHCV2Base)
    layout = [(k, tuple(v.shape)) for k, v in model.state_dict().items()]
    assert layout == [(k, tuple(s)) for k, s in fixture["layouts"][V2_NAMES[name]]]
    state = {k: torch.randn(s) for k, s in layout}
    model.load_state_dict(state, strict=True)
    # the reference's initialisation: zeroed decoder, AdaLN heads and unit write weights
    fresh = M.build_model(name)
    assert fresh.final_layer.linear.weight.abs().max() == 0
    assert torch.all(fresh.blocks[3].pool.write_weight == 1.0)
    assert torch.allclose(fresh.blocks[3].pool.read_weight, torch.full((768, 16), 1.0 / 16))
    heads = [m for n, m in fresh.named_modules() if n.endswith("adaLN_modulation") or n.endswith("_modulation")]
    assert heads and all(h[-1].weight.abs().max() == 0 for h in heads)


def test_v2_rejects_other_geometries():
    with pytest.raises(ValueError, match="only B/4"):
        V.LocalTHCV2FusedFinal12AdaLNJiT(input_size=128)
    with pytest.raises(ValueError, match="per-channel pools"):
        V.LocalTHCV2FusedFinal12AdaLNJiT(pool_groups=16)
    with pytest.raises(ValueError, match="high_grid=64"):
        V.LinearChannelwisePool(32, 16, 8)
    with pytest.raises(ValueError, match="unknown model"):
        M.build_model("local_thc_v3")


def test_jit_branch_matches_reference(fixture):
    f = fixture["branch"]
    branch = M.WorkspaceJiTBranch(f["hidden"], f["heads"], attn_backend="math").eval()
    branch.load_state_dict(f["state"], strict=True)
    rope = M.VisionRotaryEmbeddingFast(f["hidden"] // f["heads"] // 2, f["grid"])
    with torch.no_grad():
        close(branch(f["z"], f["c"], rope), f["out"])


def test_final_layer_matches_reference(fixture):
    f = fixture["final"]
    final = M.FinalLayer(f["hidden"], 4, 3).eval()
    final.load_state_dict(f["state"], strict=True)
    with torch.no_grad():
        close(final(f["x"], f["c"]), f["out"])


def test_direct_patch_embed_matches_reference(fixture):
    f = fixture["embed"]
    embed = M.DirectPatchEmbedNHWC(32, 4, 3, 8, f["hidden"]).eval()
    embed.load_state_dict(f["state"], strict=True)
    with torch.no_grad():
        out = embed(f["x"])
    assert out.shape == f["out"].shape and out.is_contiguous()
    close(out, f["out"])
    with pytest.raises(ValueError, match="expected image size"):
        embed(torch.zeros(1, 3, 16, 16))


def test_v2_checkpoint_round_trip(tmp_path):
    """A v2 checkpoint ({model, optimizer, ema, step, args, meta}) loads back, model and EMA: its pool.read_weight
    keys are the model's own names and are not migrated onto pool.write_weight (the reference's loader folds
    them together)."""
    from flowmatching_lthc_amd import checkpoint as CK

    src = M.randomize_parameters(M.build_model("local_thc_v2_fused_final12_adaln_b4"), seed=3)
    opt = torch.optim.SGD(src.parameters(), lr=0.0)
    ema = [p.detach() * 0.5 for p in src.parameters()]
    path = tmp_path / "v2.pt"
    CK.save_checkpoint(path, src, opt, ema, 7, {"model": "local_thc_v2_fused_final12_adaln_b4"})
    ck = CK.load_checkpoint(path)
    dst = M.build_model("local_thc_v2_fused_final12_adaln_b4")
    assert CK.load_model_state(dst, ck, key="model") == []
    for k, v in src.state_dict().items():
        assert torch.equal(dst.state_dict()[k], v), k
    assert not torch.equal(dst.blocks[0].pool.read_weight, dst.blocks[0].pool.write_weight)
    dst2 = M.build_model("local_thc_v2_fused_final12_adaln_b4")
    CK.load_model_state(dst2, ck, key="ema")
    for (n, p), e in zip(dst2.named_parameters(), ema):
        assert torch.equal(p.detach(), e), n
