"""Writes tests/golden/lthc_v2_fixture.pt: vectors of the reference's v2 model parts on the CPU.

Run in the build container only (the reference tree is not present on the GPU box); what it writes is data.
The v2 models (flowmatching_lthc/models/lthc_v2/model.py) are built from three modules that no library routine
or invariant pins: the per-block AdaLN branch WorkspaceJiTBranch (local_thc.py:270-297), the per-block AdaLN
decoder FinalLayer (:853-862) and the one-GEMM patch embedding DirectPatchEmbedNHWC (:92-119).  Their forward on
seeded inputs, fp32, with every parameter re-drawn, is recorded here; so is the parameter layout (names and
shapes) of the four v2 models, which a checkpoint of the reference must load into.  The v2 interface itself
(per-layer reads, the triangular sums, the materialisation) is pinned by the oracle's closed forms; its Triton
kernels cannot run on the CPU, so the whole v2 forward is not recorded.

Usage: python tests/golden/make_v2_fixture.py [/root/reference]
"""

import os
import sys

import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lthc_v2_fixture.pt")


def redraw(module, seed):
    gen = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in module.named_parameters():
            r = torch.randn(p.shape, generator=gen)
            p.copy_(1.0 + 0.1 * r if "norm" in name else 0.2 * r)


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, ref)
    from flowmatching_lthc.models import lthc_v2
    from flowmatching_lthc.models.local_thc import (
        DirectPatchEmbedNHWC,
        FinalLayer,
        VisionRotaryEmbeddingFast,
        WorkspaceJiTBranch,
    )

    torch.manual_seed(0)
    fixture = {"layouts": {}}
    for name, ctor in lthc_v2.LocalTHCV2_JiT_models.items():
        model = ctor()
        fixture["layouts"][name] = [(k, tuple(v.shape)) for k, v in model.state_dict().items()]

    gen = torch.Generator().manual_seed(5)
    hidden, heads, grid = 32, 2, 4
    branch = WorkspaceJiTBranch(hidden, heads, attn_backend="math").eval()
    redraw(branch, 6)
    rope = VisionRotaryEmbeddingFast(hidden // heads // 2, grid, num_prefix_tokens=0)
    z = torch.randn((2, grid * grid, hidden), generator=gen)
    c = torch.randn((2, hidden), generator=gen)
    final = FinalLayer(hidden, 4, 3).eval()
    redraw(final, 7)
    xf = torch.randn((2, 64, hidden), generator=gen)
    embed = DirectPatchEmbedNHWC(32, 4, 3, 8, hidden).eval()
    redraw(embed, 8)
    img = torch.randn((2, 3, 32, 32), generator=gen)
    with torch.no_grad():
        fixture["branch"] = {"state": branch.state_dict(), "z": z, "c": c, "out": branch(z, c, rope),
                             "hidden": hidden, "heads": heads, "grid": grid}  # fmt: skip
        fixture["final"] = {"state": final.state_dict(), "x": xf, "c": c, "out": final(xf, c), "hidden": hidden}
        fixture["embed"] = {"state": embed.state_dict(), "x": img, "out": embed(img), "hidden": hidden}
    torch.save(fixture, OUT)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
