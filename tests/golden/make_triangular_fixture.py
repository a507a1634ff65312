"""Writes tests/golden/lthc_triangular_layouts.json: the parameter layout of the reference's per-block LocalTHC
models with the Triton interface modules and of the two TriangularLazy models.

Run in the build container only (the reference tree is not present on the GPU box); what it writes is data.
The models are LocalTHCSharedAdaLNJiT subclasses (flowmatching_lthc/models/local_thc.py:992-1018, :1108-1153)
and TriangularLazyFusedFinal12... (:1434-1535).  Their forward runs Triton kernels that cannot run on the
CPU, so only the layout is recorded: every state-dict key with its shape, in order, which a checkpoint of the
reference must load into.  The interface math these models use (per-layer reads, the triangular sums, the
materialisation) is pinned by the oracle's closed forms, their branch, embedders and decoder by
tests/golden/lthc_v2_fixture.pt and tests/golden/lthc_tiny_model.pt.

Usage: python tests/golden/make_triangular_fixture.py [/root/reference]
"""

import json
import os
import sys

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lthc_triangular_layouts.json")
NAMES = (
    "LocalTHC-Triton-SharedAdaLN-JiT-B/4",
    "LocalTHC-Direct-Triton-SharedAdaLN-JiT-B/4",
    "LocalTHC-Direct-Triton-ReadAdd-SharedAdaLN-JiT-B/4",
    "LocalTHC-Direct-Triton-Frozen-SharedAdaLN-JiT-B/4",
    "LocalTHC-Direct-Triton-Traceable-SharedAdaLN-JiT-B/4",
    "TriangularLazy-FusedFinal12-LocalTHC-DirectTriton-SharedAdaLN-JiT-B/4",
    "TriangularLazy-FusedFinal12-LocalTHC-TritonTraceable-SharedAdaLN-JiT-B/4",
)


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, ref)
    from flowmatching_lthc.models.local_thc import LocalTHC_JiT_models

    layouts, models = [], {}
    for name in NAMES:
        model = LocalTHC_JiT_models[name]()
        layout = [[k, list(v.shape)] for k, v in model.state_dict().items()]
        if layout not in layouts:
            layouts.append(layout)
        models[name] = {"layout": layouts.index(layout), "class": type(model).__name__}
    with open(OUT, "w") as f:
        json.dump({"layouts": layouts, "models": models}, f, separators=(",", ":"))
        f.write("\n")
    print(f"wrote {OUT}: {len(models)} models, {len(layouts)} layouts")


if __name__ == "__main__":
    main()
