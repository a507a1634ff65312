"""The op boundary on the GPU: torch.library.opcheck of the jit_thc ops (schema, fake-tensor and autograd
registration, the checks torch.compile relies on; local_thc_triton_kernels.py:17,1669-1919 registers the
reference's ops as traceable), and the reference checkpoint format loaded into the HIP model.
"""

import pytest
import torch

from flowmatching_lthc_amd import checkpoint as CK
from flowmatching_lthc_amd import model as M
from flowmatching_lthc_amd import ops
from tests.test_model import CONFIG, _legacy, load_fixture, rel

pytestmark = pytest.mark.gpu
DEV = "cuda"
# schema, fake tensor and autograd registration; the AOT-dispatch check traces through autograd.Function and is
# left to torch.compile users (the ops do not mutate and have no aliasing outputs, which the schema check covers)
UTILS = ("test_schema", "test_autograd_registration", "test_faketensor")


def _inputs(dtype, B=2, G=2, C=64, L=12, seed=0):
    gen = torch.Generator().manual_seed(seed)
    H = 4 * G
    x0 = torch.randn(B, H, H, C, generator=gen).to(DEV, dtype).requires_grad_()
    alpha = (torch.randn(C, 16, generator=gen) * 0.01 + 1 / 16).to(DEV).requires_grad_()
    betas = [(torch.randn(C, 16, generator=gen) * 0.02).to(DEV).requires_grad_() for _ in range(L)]
    dzs = [(torch.randn(B, G * G, C, generator=gen) * 0.02).to(DEV, dtype).requires_grad_() for _ in range(L)]
    z = torch.randn(B, G * G, C, generator=gen).to(DEV, dtype).requires_grad_()
    gamma = (torch.randn(C, generator=gen) * 0.1).to(DEV, dtype).requires_grad_()
    return x0, alpha, betas, dzs, z, gamma


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_opcheck_interface_ops(dtype):
    print(f"case opcheck dtype={dtype}", flush=True)
    x0, alpha, betas, dzs, z, gamma = _inputs(dtype)
    cases = [
        (ops.local_write_traceable, (x0, alpha)),
        (ops.local_read_traceable, (dzs[0], betas[0])),
        (ops.local_read_add_traceable, (dzs[0], betas[0], x0)),
        (ops.local_weight_grad_traceable, (x0.detach(), dzs[0].detach())),
        (ops.final_accumulate_b4_12_traceable, (x0, *dzs, *betas)),
        (ops.final_accumulate_b4_12_grad_dz_ptr_traceable, (x0.detach(), *[b.detach() for b in betas])),
        (ops.final_accumulate_b4_12_grad_beta_ptr_traceable, (x0.detach(), *[d.detach() for d in dzs])),
        (ops.final_accumulate_list, (x0, dzs[:5], betas[:5])),
        (ops.final_accumulate_b4_traceable, (x0, torch.stack(dzs[:3]).detach(), torch.stack(betas[:3]).detach())),
        (ops.lazy_workspace_update, (z, dzs[0], gamma)),
        (ops.lazy_gamma_stack, (alpha.detach(), torch.stack(betas).detach())),
    ]
    for op, args in cases:
        print(f"  opcheck {op}", flush=True)
        torch.library.opcheck(op, args, test_utils=UTILS)


def test_legacy_checkpoint_runs_the_fixture_on_the_gpu(tmp_path):
    """A {model, optimizer, ema, step, args, meta} file with the old key names (shared_write., blocks.N.read.,
    write_logits, read_weight) and the fixture's weights in `ema` (scripts/train_imagenet256.py:79-94,
    flowmatching_lthc/checkpoint.py:12-41, local_thc.py:41-61), loaded with load_checkpoint and
    load_model_state(..., "ema") into a fresh model whose `model` entry holds other weights, runs the HIP path to the
    reference fixture's outputs (fp32, 1e-4)."""
    fx = load_fixture()
    src = M.SharedReadLocalTHCSharedAdaLNJiT(**CONFIG)
    other = M.randomize_parameters(M.SharedReadLocalTHCSharedAdaLNJiT(**CONFIG), seed=99)
    names = [n for n, _ in src.named_parameters()]
    ema = {n: fx["state_dict"][n].clone() for n in names}
    ckpt = {
        "model": _legacy(other.state_dict()),
        "optimizer": torch.optim.AdamW(other.parameters(), lr=1e-4).state_dict(),
        "ema": _legacy(ema),
        "step": 777,
        "args": {"model": "tiny", "prediction": "velocity"},
        "meta": {"model": "tiny", "prediction": "velocity", "num_classes": 10, "image_size": 32, "patch_size": 4},
    }
    assert "shared_write.write_logits" in ckpt["ema"] and "blocks.1.read.read_weight" in ckpt["ema"]
    path = tmp_path / "legacy.pt"
    torch.save(ckpt, path)
    loaded = CK.load_checkpoint(path)
    m = M.SharedReadLocalTHCSharedAdaLNJiT(**CONFIG)
    CK.load_model_state(m, loaded, key="model")  # the non-EMA weights first: the EMA must replace every parameter
    kept = CK.load_model_state(m, loaded, key="ema")
    assert set(kept) == set(m.state_dict()) - set(names)
    m = m.to(DEV).eval()
    x, t, y = fx["x"].to(DEV), fx["t"].to(DEV), fx["y"].to(DEV)
    with torch.no_grad():
        assert rel(m(x, t, y, use_lazy=True).cpu(), fx["out_lazy"]) <= 1e-4
        assert rel(m(x, t, y, use_lazy=False).cpu(), fx["out_naive"]) <= 1e-4


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_recurrence_rounding_against_eager(dtype):
    """jit_thc::lazy_workspace_update computes fma(gamma, dz, z) in fp32 and rounds once to the 16-bit dtype; the
    reference's eager `z + gamma[None, None, :] * dz` (local_thc.py:1328) rounds the product and then the sum.
    Pinned here: ours is the correctly rounded result of the exact value (|ours - exact| <= u |exact|, u the unit
    roundoff), eager is within its two roundings (u |gamma dz| + u |eager|), the two agree on most elements and
    never differ by more than those two bounds, and ours is on average no further from exact."""
    print(f"case recurrence rounding dtype={dtype}", flush=True)
    u = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11
    gen = torch.Generator().manual_seed(31)
    B, M, C = 8, 256, 768
    z = torch.randn(B, M, C, generator=gen).to(DEV, dtype)
    dz = (torch.randn(B, M, C, generator=gen) * 0.3).to(DEV, dtype)
    gamma = (torch.randn(C, generator=gen) * 0.5).to(DEV, dtype)
    ours = ops.lazy_workspace_update(z, dz, gamma)
    eager = z + gamma[None, None, :] * dz
    exact = z.double() + gamma.double()[None, None, :] * dz.double()
    prod = (gamma.double()[None, None, :] * dz.double()).abs()
    tiny = 2.0**-24 if dtype == torch.float16 else 2.0**-133
    e_ours = (ours.double() - exact).abs()
    e_eager = (eager.double() - exact).abs()
    assert (e_ours <= u * (1 + 2.0**-12) * exact.abs() + tiny).all()  # fp32 fma, then one rounding
    assert (e_eager <= u * prod + u * eager.double().abs() + tiny).all()
    assert (ours != eager).double().mean().item() <= 0.25  # about 10 % here, where gamma dz is ~0.15 z
    assert e_ours.mean().item() <= e_eager.mean().item()
