"""The v2 models' forward on the GPU (MI355X only): the HIP interface schedule against the same model with the
interface written as plain torch in fp32.

v2 (lthc_v2/model.py:1-12, 253-268): z_l = R_l(x0) + sum_{j<l} gamma[l, j] dz_j with R_l(x)[m, c] =
sum_k alpha_l[c, k] x[m, k, c] over the 16 taps of cell m, gamma[l, j, c] = sum_k alpha_l[c, k] beta_j[c, k],
dz_l = branch_l(z_l), and X_L = x0 + sum_l beta_l[c, k] dz_l[m, c] ahead of the decoder.  The reference here is
that definition evaluated with einsum on the cell view of the same x0, calling the model's own embedders,
branches and decoder (pinned on the CPU by tests/golden/lthc_v2_fixture.pt), so the test isolates the
interface ops: bases, active-prefix triangular sums, materialisation.  Bounds: fp32 to 1e-4 of max|ref|; bf16
autocast to 2e-2 of max|ref| (the stated bf16 bound at the output's scale).
"""

import pytest
import torch

from flowmatching_lthc_amd import model as M

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
NAMES = [
    "local_thc_v2_fused_final12_shared_adaln_b4",
    "local_thc_v2_fused_final12_adaln_b4",
    "local_thc_v2_direct_fused_final12_shared_adaln_b4",
    "local_thc_v2_direct_fused_final12_adaln_b4",
]


def torch_v2_forward(m, x, t, y):
    c = m.t_embedder(t) + m.y_embedder(y)
    shared = hasattr(m, "shared_adaLN_modulation")
    cond = m.shared_adaLN_modulation(c) if shared else c
    final_cond = m.shared_final_modulation(c) if shared else c
    x0 = m.x_embedder(x).float()
    b, h, _, ch = x0.shape
    g = m.workspace_grid
    cells = x0.view(b, g, 4, g, 4, ch).permute(0, 1, 3, 2, 4, 5).reshape(b, g * g, 16, ch)
    alphas = [blk.pool.read_weight.float() for blk in m.blocks]
    betas = [blk.pool.write_weight.float() for blk in m.blocks]
    dzs = []
    for l, blk in enumerate(m.blocks):
        z = torch.einsum("bmkc,ck->bmc", cells, alphas[l])
        for j in range(l):
            z = z + (alphas[l] * betas[j]).sum(-1) * dzs[j]
        dzs.append(blk.branch_update(z, cond, m.workspace_rope).float())
    xl = cells.clone()
    for l in range(len(dzs)):
        xl = xl + betas[l].t()[None, None] * dzs[l][:, :, None, :]
    x_hi = xl.view(b, g, g, 4, 4, ch).permute(0, 1, 3, 2, 4, 5).reshape(b, h, h, ch)
    return m._dense_output(x_hi, final_cond)


@pytest.mark.parametrize("name", NAMES)
def test_v2_forward_matches_torch_interface(name):
    print(f"case v2 model {name} B=2 fp32 and bf16 autocast", flush=True)
    model = M.randomize_parameters(M.build_model(name), seed=11).to(DEV).eval()
    gen = torch.Generator(device=DEV).manual_seed(12)
    x = torch.randn((2, 3, 256, 256), generator=gen, device=DEV)
    t = torch.rand((2,), generator=gen, device=DEV)
    y = torch.randint(0, 1000, (2,), generator=gen, device=DEV)
    with torch.no_grad():
        out = model(x, t, y)
        ref = torch_v2_forward(model, x, t, y)
        assert out.shape == (2, 3, 256, 256)
        scale = ref.abs().max().item()
        assert scale > 0
        err = (out - ref).abs().max().item() / scale
        assert err <= 1e-4, f"fp32: max|d|/max|ref| = {err:.3e}"
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out16 = model(x, t, y)
        err16 = (out16.float() - ref).abs().max().item() / scale
        assert err16 <= 2e-2, f"bf16 autocast: max|d|/max|ref| = {err16:.3e}"


@pytest.mark.parametrize("name", NAMES[:2])
def test_v2_gradients_match_torch_interface(name):
    """Parameter gradients through the v2 schedule's autograd (the bases' read-weight and x0 gradients, the
    triangular sums' dz and gamma gradients, the materialisation's) equal those of the torch definition, fp32."""
    print(f"case v2 gradients {name} B=1 fp32", flush=True)
    model = M.randomize_parameters(M.build_model(name), seed=13).to(DEV).train()
    gen = torch.Generator(device=DEV).manual_seed(14)
    x = torch.randn((1, 3, 256, 256), generator=gen, device=DEV)
    t = torch.rand((1,), generator=gen, device=DEV)
    y = torch.randint(0, 1000, (1,), generator=gen, device=DEV)
    w = torch.randn((1, 3, 256, 256), generator=gen, device=DEV)
    params = {
        "read_0": model.blocks[0].pool.read_weight,
        "read_7": model.blocks[7].pool.read_weight,
        "write_2": model.blocks[2].pool.write_weight,
        "write_11": model.blocks[11].pool.write_weight,
        "branch_5_w3": model.blocks[5].branch.mlp.w3.weight,
        "embed": next(model.x_embedder.parameters()),
    }
    got = torch.autograd.grad((model(x, t, y) * w).sum(), list(params.values()))
    ref = torch.autograd.grad((torch_v2_forward(model, x, t, y) * w).sum(), list(params.values()))
    for key, a, b in zip(params, got, ref):
        err = (a - b).abs().max().item() / max(b.abs().max().item(), 1e-30)
        assert err <= 1e-4, f"{key}: max|d|/max|ref| = {err:.3e}"


def test_v2_forward_graph_replay_equals_eager():
    """The v2 forward captured as one HIP graph (bases, active-prefix sums, materialisation, branch) replays to the
    eager output bit for bit, several times with eager work in between."""
    print("case v2 graph replay B=2 bf16 autocast", flush=True)
    model = M.randomize_parameters(M.build_model(NAMES[0]), seed=15).to(DEV).eval()
    gen = torch.Generator(device=DEV).manual_seed(16)
    x = torch.randn((2, 3, 256, 256), generator=gen, device=DEV)
    t = torch.rand((2,), generator=gen, device=DEV)
    y = torch.randint(0, 1000, (2,), generator=gen, device=DEV)

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
