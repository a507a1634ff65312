"""Full LTHC model: structure and transformer parity on the CPU (no HIP op runs here).

The golden fixture tests/golden/lthc_tiny_model.pt holds the reference model's
outputs on a tiny configuration (written by tests/golden/make_model_fixture.py).
On the CPU the interface hooks are supplied by library convolutions
(depthwise conv2d / conv_transpose2d, the equivalences the reference states at
local_thc.py:620-692), so these tests pin the restated transformer, embedders
and decoder; tests/test_gpu_model.py runs the same fixture through the HIP ops.
"""

import os
import re

import pytest
import torch
import torch.nn.functional as F

from flowmatching_lthc_amd import model as M

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "lthc_tiny_model.pt")
CONFIG = dict(input_size=32, patch_size=4, hidden_size=32, depth=2, num_heads=2, num_classes=10, bottleneck_dim=8, workspace_grid=2, attn_backend="math")


def load_fixture():
    return torch.load(FIXTURE, weights_only=True)


def conv_interface(model, form="conv"):
    """Replace the HIP interface hooks with torch forms of the same maps.

    form="conv": depthwise conv2d / conv_transpose2d (library routines, used on the CPU);
    form="reshape": the cell view [B,G,4,G,4,C] times the weights (no MIOpen search, used on the GPU).
    """
    s = model.high_grid // model.workspace_grid
    c = model.hidden_size
    g = model.workspace_grid

    def read(x):
        a = model.shared_read.alpha(dtype=x.dtype)
        if form == "conv":
            z = F.conv2d(x.permute(0, 3, 1, 2), a.reshape(c, 1, s, s), stride=s, groups=c)
            return z.permute(0, 2, 3, 1).reshape(x.shape[0], -1, c)
        cells = x.reshape(x.shape[0], g, s, g, s, c).permute(0, 1, 3, 2, 4, 5).reshape(x.shape[0], g * g, s * s, c)
        return (cells * a.t()[None, None]).sum(2)

    def write(dz, w):
        if form == "conv":
            out = F.conv_transpose2d(dz.reshape(dz.shape[0], g, g, c).permute(0, 3, 1, 2), w.reshape(c, 1, s, s), stride=s, groups=c)
            return out.permute(0, 2, 3, 1)
        cells = dz[:, :, None, :] * w.t()[None, None]
        return cells.reshape(dz.shape[0], g, g, s, s, c).permute(0, 1, 3, 2, 4, 5).reshape(dz.shape[0], g * s, g * s, c)

    model.shared_read.read = read
    model.shared_read.read_with_residual = lambda x: (x, read(x))
    for blk in model.blocks:
        blk.write.write_add = lambda x_hi, dz, b=blk: x_hi + write(dz, b.write.beta(dtype=dz.dtype))

        def lazy(z, dz, shared_read, b=blk):
            return z + b.write.gamma_from_alpha(shared_read.alpha(dtype=dz.dtype))[None, None, :] * dz

        blk.lazy_workspace_update = lazy
        blk.lazy_workspace_step = lambda z, dz, shared_read, f=lazy: (f(z, dz, shared_read), dz)

    def final(x0, dz_list):
        x = x0
        for blk, dz in zip(model.blocks, dz_list, strict=True):
            x = x + write(dz, blk.write.beta(dtype=dz.dtype))
        return x

    model.final_accumulate_reference = final
    return model


def rel(a, b):
    return float((a - b).abs().max() / b.abs().max())


def test_fixture_loads_safely_and_keys_match():
    fx = load_fixture()
    ours = M.SharedReadLocalTHCSharedAdaLNJiT(**CONFIG)
    sd = ours.state_dict()
    assert set(sd) == set(fx["state_dict"])
    for k, v in fx["state_dict"].items():
        assert sd[k].shape == v.shape, k
    ours.load_state_dict(fx["state_dict"])


def test_transformer_matches_reference_fixture_on_cpu():
    fx = load_fixture()
    ours = M.SharedReadLocalTHCSharedAdaLNJiT(**CONFIG).eval()
    ours.load_state_dict(fx["state_dict"])
    conv_interface(ours)
    with torch.no_grad():
        x0 = ours.x_embedder(fx["x"])
        assert rel(x0, fx["x0"]) <= 1e-6
        assert rel(ours.shared_read.read(x0), fx["z0"]) <= 1e-6
        assert rel(ours(fx["x"], fx["t"], fx["y"], use_lazy=True), fx["out_lazy"]) <= 1e-5
        assert rel(ours(fx["x"], fx["t"], fx["y"], use_lazy=False), fx["out_naive"]) <= 1e-5


def test_reshape_form_equals_conv_form():
    """The GPU tests' torch reference (cell reshape) is pinned to the library convolutions here."""
    fx = load_fixture()
    a = M.SharedReadLocalTHCSharedAdaLNJiT(**CONFIG).eval()
    a.load_state_dict(fx["state_dict"])
    b = M.SharedReadLocalTHCSharedAdaLNJiT(**CONFIG).eval()
    b.load_state_dict(fx["state_dict"])
    conv_interface(a, "conv")
    conv_interface(b, "reshape")
    with torch.no_grad():
        for lazy in (True, False):
            assert rel(b(fx["x"], fx["t"], fx["y"], use_lazy=lazy), a(fx["x"], fx["t"], fx["y"], use_lazy=lazy)) <= 1e-5


def test_mutated_rope_layout_is_caught():
    """Transposing the token grid of the RoPE table (rows for columns) must break fixture parity."""
    fx = load_fixture()
    ours = M.SharedReadLocalTHCSharedAdaLNJiT(**CONFIG).eval()
    ours.load_state_dict(fx["state_dict"])
    conv_interface(ours)
    rope = ours.workspace_rope
    g = ours.workspace_grid
    perm = torch.arange(g * g).reshape(g, g).t().reshape(-1)
    rope.freqs_cos = rope.freqs_cos[perm]
    rope.freqs_sin = rope.freqs_sin[perm]
    with torch.no_grad():
        out = ours(fx["x"], fx["t"], fx["y"], use_lazy=True)
    assert rel(out, fx["out_lazy"]) > 1e-3


def test_released_model_shape_and_names():
    m = M.build_model("lthc_b4_velocity")
    assert sum(p.numel() for p in m.parameters()) == 91_633_968  # README.md:138 (91.63 M)
    names = dict(m.named_parameters())
    assert names["shared_read.read_logits"].shape == (768, 16)
    for i in range(12):
        assert names[f"blocks.{i}.write.write_weight"].shape == (768, 16)
    assert isinstance(m, M.SharedReadFusedFinal12LocalTHCSharedAdaLNJiT)
    with pytest.raises(ValueError, match="unknown model"):
        M.build_model("nope")


def test_legacy_checkpoint_keys_migrate():
    old = {
        "shared_write.write_logits": torch.zeros(768, 16),
        "blocks.3.read.read_weight": torch.ones(768, 16),
        "blocks.3.branch.norm1.weight": torch.ones(768),
    }
    new = M.migrate_lthc_state_dict_keys(old)
    assert set(new) == {"shared_read.read_logits", "blocks.3.write.write_weight", "blocks.3.branch.norm1.weight"}


def test_wrong_image_size_raises():
    m = M.SharedReadLocalTHCSharedAdaLNJiT(**CONFIG)
    with pytest.raises(ValueError, match="expected image size"):
        m.x_embedder(torch.zeros(1, 3, 16, 16))


# ---------------------------------------------------------------------------
# checkpoint format (scripts/train_imagenet256.py:79-94, flowmatching_lthc/checkpoint.py)
# ---------------------------------------------------------------------------
def _legacy(sd):
    """The same state with the old research key names (the inverse of the migration)."""
    out = {}
    for k, v in sd.items():
        k = k.replace("shared_read.", "shared_write.").replace(".read_logits", ".write_logits")
        k = re.sub(r"blocks\.(\d+)\.write\.", r"blocks.\1.read.", k).replace(".write_weight", ".read_weight")
        out[k] = v
    return out


def test_checkpoint_round_trip_with_legacy_keys(tmp_path):
    from flowmatching_lthc_amd import checkpoint as CK

    fx = load_fixture()
    src = M.SharedReadLocalTHCSharedAdaLNJiT(**CONFIG)
    src.load_state_dict(fx["state_dict"])
    opt = torch.optim.AdamW(src.parameters(), lr=1e-4)
    ema = [p.detach() * 0.5 for p in src.parameters()]
    path = tmp_path / "ckpt.pt"
    CK.save_checkpoint(path, src, opt, ema, 1234, {"model": "tiny", "prediction": "velocity"})
    ck = CK.load_checkpoint(path)
    assert set(ck) == set(CK.CHECKPOINT_KEYS) and ck["step"] == 1234
    assert ck["meta"]["model"] == "tiny" and ck["meta"]["image_size"] == CONFIG["input_size"]

    # the full state, written with the old key names, loads strictly after migration
    dst = M.SharedReadLocalTHCSharedAdaLNJiT(**CONFIG)
    ck_old = dict(ck, model=_legacy(ck["model"]), ema=_legacy(ck["ema"]))
    assert "shared_write.write_logits" in ck_old["model"]
    assert CK.load_model_state(dst, ck_old, key="model") == []
    for k, v in src.state_dict().items():
        assert torch.equal(dst.state_dict()[k], v), k

    # EMA: parameters come from the EMA, buffers stay the model's own
    kept = CK.load_model_state(dst, ck_old, key="ema")
    params = dict(src.named_parameters())
    assert set(kept) == set(dst.state_dict()) - set(params)
    for (n, p), e in zip(dst.named_parameters(), ema):
        assert torch.equal(p.detach(), e), n
    with pytest.raises(ValueError):
        CK.load_model_state(dst, ck, key="optimizer")
    with pytest.raises(KeyError):
        CK.load_model_state(dst, {"model": ck["model"]}, key="ema")


def test_checkpoint_loader_refuses_pickled_objects(tmp_path):
    """Checkpoints load with the weights-only loader: an arbitrary pickled object is refused, not run."""
    from flowmatching_lthc_amd import checkpoint as CK

    path = tmp_path / "bad.pt"
    torch.save({"model": {}, "obj": _Opaque()}, path)
    with pytest.raises(Exception):
        CK.load_checkpoint(path)


class _Opaque:
    pass


def test_legacy_hyper_connection_modules_on_cpu():
    """Parameter names and initial values follow local_thc.py:511-551; the HIP ops refuse CPU tensors."""
    from flowmatching_lthc_amd import local_thc as LT

    m = LT.ChannelwiseLocalTokenHyperConnectionTritonReadAdd(64, 16, 32, 32)
    assert [n for n, _ in m.named_parameters()] == ["read_logits", "write_weight"]
    assert not m.read_logits.any() and bool((m.write_weight == 1).all())
    with pytest.raises(ValueError):
        LT.ChannelwiseLocalTokenHyperConnectionTriton(64, 16, 32, 16)
    with pytest.raises(ValueError):
        LT.ChannelwiseLocalTokenHyperConnectionTriton(64, 16, 32, 32, use_softmax_write=False)
    with pytest.raises(ValueError, match="no CPU fallback"):
        m.read(torch.zeros(1, 64, 64, 32))


def conv_read(model, x):
    s, c = model.high_grid // model.workspace_grid, model.hidden_size
    a = model.shared_read.alpha(dtype=x.dtype)
    z = F.conv2d(x.permute(0, 3, 1, 2), a.reshape(c, 1, s, s), stride=s, groups=c)
    return z.permute(0, 2, 3, 1).reshape(x.shape[0], -1, c)


def conv_final(model, x0, dz_list):
    s, c, g = model.high_grid // model.workspace_grid, model.hidden_size, model.workspace_grid
    x = x0
    for blk, dz in zip(model.blocks, dz_list, strict=True):
        w = blk.write.beta(dtype=dz.dtype)
        out = F.conv_transpose2d(dz.reshape(dz.shape[0], g, g, c).permute(0, 3, 1, 2), w.reshape(c, 1, s, s), stride=s, groups=c)
        x = x + out.permute(0, 2, 3, 1)
    return x


def test_forward_lazy_calls_an_overridden_lazy_workspace_update():
    """A reference-style instance override of lazy_workspace_update (local_thc.py:1325, called at :1384) and of
    shared_read.read alone defines forward_lazy's recurrence and read: the fixture is reproduced through them, and
    a changed update changes the output."""
    fx = load_fixture()
    calls = []
    m = M.SharedReadLocalTHCSharedAdaLNJiT(**CONFIG).eval()
    m.load_state_dict(fx["state_dict"])
    m.shared_read.read = lambda x: conv_read(m, x)
    m.final_accumulate_reference = lambda x0, dzs: conv_final(m, x0, dzs)
    for i, blk in enumerate(m.blocks):

        def upd(z, dz, shared_read, b=blk, i=i, scale=1.0):
            calls.append(i)
            return z + scale * b.write.gamma_from_alpha(shared_read.alpha(dtype=dz.dtype))[None, None, :] * dz

        blk.lazy_workspace_update = upd
    with torch.no_grad():
        out = m(fx["x"], fx["t"], fx["y"], use_lazy=True)
    assert calls == list(range(CONFIG["depth"]))
    assert rel(out, fx["out_lazy"]) <= 1e-5
    for blk in m.blocks:  # a different recurrence must show in the output
        f = blk.lazy_workspace_update
        blk.lazy_workspace_update = lambda z, dz, sr, f=f: f(z, 2.0 * dz, sr)
    with torch.no_grad():
        assert rel(m(fx["x"], fx["t"], fx["y"], use_lazy=True), fx["out_lazy"]) > 1e-4


def test_overridden_gamma_or_alpha_hooks_disable_the_one_launch_gammas():
    """_all_gammas (one launch for every block's gamma) stands aside whenever a hook it would bypass is replaced."""
    m = M.SharedReadLocalTHCSharedAdaLNJiT(**CONFIG)
    from flowmatching_lthc_amd.local_thc import LayerLocalWrite, SharedLocalRead, overridden

    std = M.SharedReadLocalTHCSharedAdaLNJiTBlock
    blk = m.blocks[0]
    assert not overridden(blk, "lazy_workspace_update", std)
    assert not overridden(blk.write, "gamma_from_alpha", LayerLocalWrite)
    blk.write.gamma_from_alpha = lambda a: a.sum(-1)
    assert overridden(blk.write, "gamma_from_alpha", LayerLocalWrite)

    class Sub(SharedLocalRead):
        def alpha(self, dtype=None):
            return super().alpha(dtype)

    sr = Sub(8, 2, CONFIG["hidden_size"], CONFIG["hidden_size"])
    assert overridden(sr, "alpha", SharedLocalRead)
    assert not overridden(m.shared_read, "alpha", SharedLocalRead)


def test_fused_decoder_only_where_autograd_does_not_record_it():
    """The one-pass decoder head's backward replays the eager sequence (slower than the eager decoder's forward and
    backward), so the models take it only where autograd records nothing: no-grad, or nothing that needs a gradient."""
    fl = M.FinalLayerSharedAdaLN(32, 4, 3)
    x = torch.randn(2, 64, 32)
    t2 = torch.randn(2, 64)
    assert M.decoder_records_grad(fl, x, t2)  # the decoder's parameters need gradients
    with torch.no_grad():
        assert not M.decoder_records_grad(fl, x, t2)
    for p in fl.parameters():
        p.requires_grad_(False)
    assert not M.decoder_records_grad(fl, x, t2)
    assert M.decoder_records_grad(fl, x.requires_grad_(), t2)
    assert M.decoder_records_grad(fl, x.detach(), t2.requires_grad_())
    # the per-block-AdaLN decoder counts its own AdaLN head
    fa = M.FinalLayer(32, 4, 3)
    for p in fa.parameters():
        p.requires_grad_(False)
    fa.adaLN_modulation[-1].weight.requires_grad_(True)
    assert M.decoder_records_grad(fa, x.detach(), t2.detach())
