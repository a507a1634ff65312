"""The per-block LocalTHC and TriangularLazy models on the GPU (MI355X only): the HIP interface against the same
model with the interface written as plain torch in fp32.

Per-block (local_thc.py:759-787, :1009-1018): z_l = R_l(x_l), x_{l+1} = x_l + P_l(branch_l(z_l)), with
R_l(x)[m, c] = sum_k alpha_l[c, k] x[m, k, c] over the 16 taps of cell m, alpha_l = softmax(read_logits_l), and
P_l(dz)[m, k, c] = beta_l[c, k] dz[m, c], beta_l = write_weight_l.  TriangularLazy (local_thc.py:1434-1515) computes
the same x_L as z_l = R_l(x0) + sum_{j<l} gamma[l, j] dz_j, gamma[l, j, c] = sum_k alpha_l[c, k] beta_j[c, k], then
x_L = x0 + sum_l P_l(dz_l).  The references evaluate these definitions with einsum on the cell view and call the
model's own embedders, branches and decoder (pinned on the CPU by the tests/golden fixtures), so the tests isolate
the interface ops.  Bounds: fp32 to 1e-4 of max|ref|; bf16 autocast to 2e-2 of max|ref|.
"""

import pytest
import torch

from flowmatching_lthc_amd import model as M

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
LAZY = [
    "TriangularLazy-FusedFinal12-LocalTHC-DirectTriton-SharedAdaLN-JiT-B/4",
    "TriangularLazy-FusedFinal12-LocalTHC-TritonTraceable-SharedAdaLN-JiT-B/4",
]
PER_BLOCK = [
    "LocalTHC-Triton-SharedAdaLN-JiT-B/4",
    "LocalTHC-Direct-Triton-SharedAdaLN-JiT-B/4",
    "LocalTHC-Direct-Triton-ReadAdd-SharedAdaLN-JiT-B/4",
    "LocalTHC-Direct-Triton-Frozen-SharedAdaLN-JiT-B/4",
    "LocalTHC-Direct-Triton-Traceable-SharedAdaLN-JiT-B/4",
]


def to_cells(xh, g):
    b, h, _, ch = xh.shape
    return xh.view(b, g, 4, g, 4, ch).permute(0, 1, 3, 2, 4, 5).reshape(b, g * g, 16, ch)


def from_cells(cells, g):
    b, _, _, ch = cells.shape
    return cells.view(b, g, g, 4, 4, ch).permute(0, 1, 3, 2, 4, 5).reshape(b, 4 * g, 4 * g, ch)


def weights(m):
    alphas = [torch.softmax(blk.hyper.read_logits.float(), dim=-1) for blk in m.blocks]
    betas = [blk.hyper.write_weight.float() for blk in m.blocks]
    return alphas, betas


def torch_per_block(m, x, t, y):
    t6, t2 = m._conditioning(t, y)
    g = m.workspace_grid
    cells = to_cells(m.x_embedder(x).float(), g)
    alphas, betas = weights(m)
    for l, blk in enumerate(m.blocks):
        z = torch.einsum("bmkc,ck->bmc", cells, alphas[l])
        dz = blk.branch(z, t6, m.workspace_rope).float()
        cells = cells + betas[l].t()[None, None] * dz[:, :, None, :]
    return m._dense_output(from_cells(cells, g), t2)


def torch_lazy(m, x, t, y):
    t6, t2 = m._conditioning(t, y)
    g = m.workspace_grid
    cells = to_cells(m.x_embedder(x).float(), g)
    alphas, betas = weights(m)
    dzs = []
    for l, blk in enumerate(m.blocks):
        z = torch.einsum("bmkc,ck->bmc", cells, alphas[l])
        for j in range(l):
            z = z + (alphas[l] * betas[j]).sum(-1) * dzs[j]
        dzs.append(blk.branch(z, t6, m.workspace_rope).float())
    for l in range(len(dzs)):
        cells = cells + betas[l].t()[None, None] * dzs[l][:, :, None, :]
    return m._dense_output(from_cells(cells, g), t2)


def inputs(seed, b=2):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((b, 3, 256, 256), generator=gen, device=DEV)
    t = torch.rand((b,), generator=gen, device=DEV)
    y = torch.randint(0, 1000, (b,), generator=gen, device=DEV)
    return x, t, y, gen


def rel(a, b):
    return (a.float() - b.float()).abs().max().item() / max(b.abs().max().item(), 1e-30)


@pytest.mark.parametrize("name", LAZY)
def test_lazy_forward_matches_torch_interface(name):
    print(f"case triangular lazy forward {name} B=2 fp32 and bf16 autocast", flush=True)
    model = M.randomize_parameters(M.build_model(name), seed=21).to(DEV).eval()
    x, t, y, _ = inputs(22)
    with torch.no_grad():
        ref = torch_lazy(model, x, t, y)
        assert ref.abs().max().item() > 0
        out = model(x, t, y)
        assert out.shape == (2, 3, 256, 256)
        assert rel(out, ref) <= 1e-4, f"lazy fp32: {rel(out, ref):.3e}"
        # the per-block recurrence: other HIP ops (one read and one write-add per block), the same x_L
        naive = model(x, t, y, use_lazy=False)
        assert rel(naive, ref) <= 1e-4, f"naive fp32: {rel(naive, ref):.3e}"
        assert rel(torch_per_block(model, x, t, y), ref) <= 1e-5
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out16 = model(x, t, y)
            naive16 = model(x, t, y, use_lazy=False)
        assert rel(out16, ref) <= 2e-2, f"lazy bf16: {rel(out16, ref):.3e}"
        assert rel(naive16, ref) <= 2e-2, f"naive bf16: {rel(naive16, ref):.3e}"


@pytest.mark.parametrize("name", PER_BLOCK)
def test_per_block_forward_matches_torch_interface(name):
    print(f"case per-block forward {name} B=2 fp32", flush=True)
    model = M.randomize_parameters(M.build_model(name), seed=23).to(DEV).eval()
    x, t, y, _ = inputs(24)
    with torch.no_grad():
        ref = torch_per_block(model, x, t, y)
        out = model(x, t, y)
        assert rel(out, ref) <= 1e-4, f"fp32: {rel(out, ref):.3e}"


@pytest.mark.parametrize("name,lazy", [(LAZY[0], True), (LAZY[1], True), (LAZY[0], False), (PER_BLOCK[0], False)])
def test_gradients_match_torch_interface(name, lazy):
    """Parameter gradients through the HIP interface's autograd (the bases' read-weight and x0 gradients, the
    triangular sums' dz and gamma gradients and the materialisation's in the lazy form; each read's and write's
    in the per-block form) equal those of the torch definition, fp32."""
    print(f"case gradients {name} lazy={lazy} B=1 fp32", flush=True)
    model = M.randomize_parameters(M.build_model(name), seed=25).to(DEV).train()
    x, t, y, gen = inputs(26, b=1)
    w = torch.randn((1, 3, 256, 256), generator=gen, device=DEV)
    params = {
        "read_0": model.blocks[0].hyper.read_logits,
        "read_7": model.blocks[7].hyper.read_logits,
        "write_2": model.blocks[2].hyper.write_weight,
        "write_11": model.blocks[11].hyper.write_weight,
        "branch_5_w3": model.blocks[5].branch.mlp.w3.weight,
        "embed": next(model.x_embedder.parameters()),
    }
    out = model(x, t, y, use_lazy=lazy) if name in LAZY else model(x, t, y)
    got = torch.autograd.grad((out * w).sum(), list(params.values()))
    ref = torch.autograd.grad((torch_per_block(model, x, t, y) * w).sum(), list(params.values()))
    for key, a, b in zip(params, got, ref):
        assert rel(a, b) <= 1e-4, f"{key}: {rel(a, b):.3e}"


def test_frozen_weights_get_no_gradient():
    """The frozen hyper-connections pass gradients to the stream and the branches but none to their own weights."""
    print("case frozen per-block gradients B=1 fp32", flush=True)
    model = M.randomize_parameters(M.build_model(PER_BLOCK[3]), seed=27).to(DEV).train()
    x, t, y, gen = inputs(28, b=1)
    w = torch.randn((1, 3, 256, 256), generator=gen, device=DEV)
    frozen = [model.blocks[3].hyper.read_logits, model.blocks[3].hyper.write_weight]
    live = [model.blocks[5].branch.mlp.w3.weight, next(model.x_embedder.parameters())]
    got = torch.autograd.grad((model(x, t, y) * w).sum(), frozen + live, allow_unused=True)
    assert got[0] is None and got[1] is None
    for p in frozen:
        p.requires_grad_(False)
    ref = torch.autograd.grad((torch_per_block(model, x, t, y) * w).sum(), live)
    for a, b in zip(got[2:], ref):
        assert rel(a, b) <= 1e-4, f"{rel(a, b):.3e}"


def test_lazy_forward_graph_replay_equals_eager():
    """The TriangularLazy forward captured as one HIP graph replays to the eager output bit for bit, several times
    with eager work in between."""
    print("case triangular lazy graph replay B=2 bf16 autocast", flush=True)
    model = M.randomize_parameters(M.build_model(LAZY[0]), seed=29).to(DEV).eval()
    x, t, y, _ = inputs(30)

    def fwd():
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            return model(x, t, y)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fwd()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fwd()
    eager = fwd().clone()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        fwd()
        torch.cuda.synchronize()


@pytest.mark.parametrize(
    "name",
    [LAZY[0], LAZY[1], PER_BLOCK[0], "local_thc_v2_fused_final12_shared_adaln_b4", "local_thc_v2_direct_fused_final12_adaln_b4"],
)
def test_inference_fusions_match_plain_forward(name):
    """Inference under bf16 autocast: the one-launch weight conversion changes no bit of the output, and the fused
    decoder (with X_L formed inside it, for the lazy and v2 schedules) stays within 1e-2 of max|out| of the plain
    materialise-then-decode forward.  The fused pass keeps X_L unrounded and leaves out the eager sequence's
    intermediate roundings of the norm and modulation, so the two differ by a few bf16 steps of the output."""
    print(f"case inference fusions {name} B=2 bf16 autocast", flush=True)
    model = M.randomize_parameters(M.build_model(name), seed=31).to(DEV).eval()
    x, t, y, _ = inputs(32)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        fused = model(x, t, y)
        assert "_batched_cast" in model.__dict__, "the one-launch conversion did not run"
        model.fused_decoder = False
        plain_cast = model(x, t, y)
        model.batched_weight_cast = False
        plain = model(x, t, y)
    assert torch.equal(plain_cast, plain)
    assert all("_cast" not in mod.__dict__ for mod in model.modules()), "converted weights left attached"
    assert fused.dtype == plain.dtype == torch.bfloat16 and fused.shape == plain.shape
    assert rel(fused, plain) <= 1e-2, f"{rel(fused, plain):.3e}"
