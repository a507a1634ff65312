"""Writes tests/golden/lthc_tiny_model.pt: outputs of the reference model on a tiny config.

Run in the build container only (the reference tree is not present on the GPU
box); the fixture it writes is data.  The full-model forward (the workspace
transformer around the interface: RoPE layout, SwiGLU split, AdaLN chunk
order, unpatchify permutation) has no library routine or invariant that pins
it, so its parity is anchored on these vectors.

Model: flowmatching_lthc.models.local_thc.SharedReadLocalTHCSharedAdaLNJiT at
input 32, patch 4 (8x8 high-res grid), 2x2 workspace (cell side 4), hidden 32,
2 heads, depth 2, bottleneck 8, 10 classes, SDPA math backend, fp32 on CPU.
Every parameter is re-drawn (the default init zeroes the AdaLN heads and the
decoder, which would make the output identically 0).

Usage: python tests/golden/make_model_fixture.py [/root/reference]
"""

import os
import sys

import torch

CONFIG = dict(input_size=32, patch_size=4, hidden_size=32, depth=2, num_heads=2, num_classes=10, bottleneck_dim=8, workspace_grid=2, attn_backend="math")
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lthc_tiny_model.pt")


def redraw(model, seed):
    gen = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            r = torch.randn(p.shape, generator=gen)
            leaf = name.split(".")[-2] if "." in name else name
            if "norm" in leaf:
                p.copy_(1.0 + 0.1 * r)
            elif name.endswith("write_weight"):
                p.copy_(1.0 + 0.5 * r)
            elif name.endswith("read_logits"):
                p.copy_(0.5 * r)
            else:
                p.copy_(0.2 * r)


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, ref)
    from flowmatching_lthc.models.local_thc import SharedReadLocalTHCSharedAdaLNJiT

    torch.manual_seed(0)
    model = SharedReadLocalTHCSharedAdaLNJiT(**CONFIG).eval()
    redraw(model, seed=1)
    gen = torch.Generator().manual_seed(2)
    x = torch.randn((2, 3, 32, 32), generator=gen)
    t = torch.rand((2,), generator=gen)
    y = torch.tensor([3, 10])  # 10 = the null label
    with torch.no_grad():
        x0 = model.x_embedder(x)
        z0 = model.shared_read.read(x0)
        out_lazy = model(x, t, y, use_lazy=True)
        out_naive = model(x, t, y, use_lazy=False)
    fixture = {
        "state_dict": {k: v.clone() for k, v in model.state_dict().items()},
        "x": x, "t": t, "y": y, "x0": x0, "z0": z0, "out_lazy": out_lazy, "out_naive": out_naive,
    }
    torch.save(fixture, OUT)
    print(f"wrote {OUT}: |out_lazy| max {out_lazy.abs().max():.4f}, lazy-naive max diff {(out_lazy - out_naive).abs().max():.2e}")


if __name__ == "__main__":
    main()
