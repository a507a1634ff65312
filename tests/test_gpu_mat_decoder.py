"""jit_thc::final_accumulate_decoder_head (lthc_materialise_decoder_fwd): the final materialisation with the decoder's
RMSNorm, modulation and linear layer in its epilogue (local_thc.py:1368-1372, 865-873, 972-980), X_L never written.

Reference: the exact function in float64 of the X_L that the materialisation writes (ops.final_accumulate_list,
whose rounding the fused kernel applies per token before the decoder front):
    o[t, j] = sum_c y[t,c] r(W[j,c]) + r(b[j]),   y = x inv nw r(1 + scale) + shift,   inv = 1/sqrt(mean x^2 + eps)
r() the rounding to the activation dtype (autocast's casts).  The kernel rounds M = nw r(1 + scale) r(W) to the
activation dtype, sums in fp32 on the matrix cores and rounds o once, so each pixel must be within
    |d| <= u |o| + 2u sum_c |x_c inv M_jc| + 2^-20 (max|o| + 1),   u = 2^-8 (bf16) or 2^-11 (fp16)
(one output rounding, one rounding of every M term, fp32 sums).  The eager sequence (decoder_head_eager on the
written X_L) rounds the normalised and modulated rows as well; the fused result is no further from the exact function
than eager is, in the maximum over the image, within a factor 1.5.
"""

from __future__ import annotations

from unittest import mock

import pytest
import torch

from flowmatching_lthc_amd import model as M
from flowmatching_lthc_amd import ops

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _unpatchify(o: torch.Tensor, h: int, p: int = 4, co: int = 3) -> torch.Tensor:
    b = o.shape[0]
    return o.reshape(b, h, h, p, p, co).permute(0, 5, 1, 3, 2, 4).reshape(b, co, h * p, h * p)


def _inputs(B, G, C, L, dtype, pdt, seed):
    gen = torch.Generator().manual_seed(seed)
    H = 4 * G
    x0 = torch.randn((B, H, H, C), generator=gen).to(DEV, dtype)
    dzs = [(torch.randn((B, G * G, C), generator=gen) * 0.5).to(DEV, dtype) for _ in range(L)]
    betas = [(torch.rand((C, 16), generator=gen) * 0.25).to(DEV) for _ in range(L)]
    t2 = (torch.randn((B, 2 * C), generator=gen) * 0.3).to(DEV, dtype)
    nw = (torch.randn(C, generator=gen) * 0.2 + 1).to(DEV, pdt)
    lw = (torch.randn((48, C), generator=gen) * 0.05).to(DEV, pdt)
    lb = (torch.randn(48, generator=gen) * 0.1).to(DEV, pdt)
    return x0, dzs, betas, t2, nw, lw, lb


@pytest.mark.parametrize(
    "B,G,C,L,dtype,pdt",
    [
        (2, 16, 768, 12, torch.bfloat16, torch.float32),  # the model's width and depth
        (2, 16, 256, 5, torch.bfloat16, torch.bfloat16),  # padded depth bucket, 16-bit decoder weights
        (1, 32, 512, 3, torch.float16, torch.float32),    # fp16, a 32 x 32 workspace grid
        (3, 16, 256, 12, torch.float16, torch.float16),
    ],
)
def test_materialise_decoder_matches_exact(B, G, C, L, dtype, pdt):
    print(f"case B={B} G={G} C={C} L={L} dtype={dtype} params={pdt}", flush=True)
    x0, dzs, betas, t2, nw, lw, lb = _inputs(B, G, C, L, dtype, pdt, seed=100 + L + C)
    shift, scale = t2.chunk(2, dim=1)
    eps, H = 1e-6, 4 * G
    img = ops.final_accumulate_decoder_head(x0, dzs, betas, nw, shift, scale, lw, lb, eps, 4)
    assert img.shape == (B, 3, 4 * H, 4 * H) and img.dtype == dtype
    xl = ops.final_accumulate_list(x0, dzs, betas)  # the X_L the kernel forms per token
    x = xl.double().cpu().reshape(B, H * H, C)
    inv = torch.rsqrt((x * x).mean(dim=-1, keepdim=True) + eps)
    u_mod = (1 + scale.double().cpu()).to(dtype).double()  # r(1 + scale), as autocast's bf16 add rounds it
    W = lw.to(dtype).double().cpu()
    bias = lb.to(dtype).double().cpu()
    nwd = nw.double().cpu()
    y = x * inv * nwd * u_mod[:, None, :] + shift.double().cpu()[:, None, :]
    o = y @ W.T + bias
    u = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11
    mag = torch.einsum("btc,bc,jc->btj", (x * inv).abs(), (nwd * u_mod).abs(), W.abs())
    ref = _unpatchify(o, H)
    bound = _unpatchify(u * o.abs() + 2 * u * mag, H) + 2.0**-20 * (o.abs().max().item() + 1)
    d = (img.double().cpu() - ref).abs()
    assert (d <= bound).all(), f"max excess {(d - bound).max().item():.3e} (max |d| {d.max().item():.3e})"
    eager = ops.decoder_head_eager(xl.reshape(B, H * H, C), nw, shift, scale, lw, lb, eps, H, 4)
    e_ours, e_eager = d.max().item(), (eager.double().cpu() - ref).abs().max().item()
    print(f"  max |fused - exact| {e_ours:.3e}, max |eager - exact| {e_eager:.3e}")
    assert e_ours <= 1.5 * e_eager + 1e-6


def test_materialise_decoder_rejects_unsupported_shapes():
    print("case unsupported shapes", flush=True)
    x0, dzs, betas, t2, nw, lw, lb = _inputs(1, 16, 256, 2, torch.bfloat16, torch.float32, seed=5)
    shift, scale = t2.chunk(2, dim=1)
    with pytest.raises(ValueError):  # C not a multiple of 256
        ops.final_accumulate_decoder_head(x0[..., :192].contiguous(), [d[..., :192].contiguous() for d in dzs],
                                          [b[:192].contiguous() for b in betas], nw[:192], shift[:, :192],
                                          scale[:, :192], lw[:, :192], lb, 1e-6, 4)  # fmt: skip
    with pytest.raises(ValueError):  # fp32 activations
        ops.final_accumulate_decoder_head(x0.float(), [d.float() for d in dzs], betas, nw, shift.float(),
                                          scale.float(), lw, lb, 1e-6, 4)  # fmt: skip
    assert not ops.materialise_decoder_supported(x0[:, :32, :32].contiguous(), dzs, lw, 4)  # G = 8


def test_model_fused_materialise_decoder_matches_unfused():
    """LTHC-B/4 (random-init weights) at B=2, bf16 autocast, no grad: the fused materialise + decoder against the
    model with X_L written and the decoder head applied, both against the fp32 model; the fused form no further from
    fp32 than the unfused one (x 1.5) and within 2e-2 of its scale."""
    print("case model fused materialise + decoder", flush=True)
    torch.manual_seed(0)
    m = M.randomize_parameters(M.build_model("lthc_b4_velocity"), seed=21).to(DEV).eval()
    gen = torch.Generator().manual_seed(22)
    B = 2
    x = torch.randn(B, 3, 256, 256, generator=gen).to(DEV)
    t = torch.rand(B, generator=gen).to(DEV)
    y = torch.randint(0, 1000, (B,), generator=gen).to(DEV)
    with torch.no_grad():
        exact = m(x, t, y).float()
        with torch.autocast("cuda", dtype=torch.bfloat16):
            with mock.patch.object(ops, "final_accumulate_decoder_head", wraps=ops.final_accumulate_decoder_head) as op:
                fused = m(x, t, y).float()
            assert op.call_count == 1, "the model did not take the fused materialise + decoder path"
            m.fused_materialise_decoder = False
            with mock.patch.object(ops, "final_accumulate_decoder_head", wraps=ops.final_accumulate_decoder_head) as op:
                unfused = m(x, t, y).float()
            assert op.call_count == 0
            m.fused_materialise_decoder = True
    scale = exact.abs().max().item()
    e_f = (fused - exact).abs().max().item() / scale
    e_u = (unfused - exact).abs().max().item() / scale
    print(f"  fused {e_f:.3e} unfused {e_u:.3e} of max|exact| {scale:.3f}")
    assert e_f <= 2e-2 and e_f <= max(1.5 * e_u, 1e-3)


def test_materialise_decoder_graph_replay_equals_eager():
    """The op under HIP-graph capture (its workspace from the graph's pool): every replay, with eager work and
    synchronisations between replays, equals the eager result bit for bit."""
    print("case graph replay", flush=True)
    x0, dzs, betas, t2, nw, lw, lb = _inputs(2, 16, 768, 12, torch.bfloat16, torch.float32, seed=77)
    shift, scale = t2.chunk(2, dim=1)
    run = lambda: ops.final_accumulate_decoder_head(x0, dzs, betas, nw, shift, scale, lw, lb, 1e-6, 4)  # noqa: E731
    eager = run()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = run()
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        other = ops.final_accumulate_decoder_head(x0 * 0.5, dzs, betas, nw, shift, scale, lw, lb, 1e-6, 4)  # eager work
        torch.cuda.synchronize()
        assert not torch.equal(other, eager)


def test_fused_final12_other_depth_raises_under_no_grad():
    """SharedReadFusedFinal12LocalTHCSharedAdaLNJiT requires depth 12 (local_thc.py:1416-1418).  A model of another
    depth must raise that ValueError under no-grad too, where the fused materialise + decoder path would otherwise
    run without calling the hook; the same model class at depth 12 takes the fused path."""
    print("case FusedFinal12 depth 2", flush=True)
    kw = dict(input_size=256, patch_size=4, hidden_size=256, num_heads=4, bottleneck_dim=16, workspace_grid=16)
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(1, 3, 256, 256, generator=gen).to(DEV)
    t = torch.rand(1, generator=gen).to(DEV)
    y = torch.randint(0, 1000, (1,), generator=gen).to(DEV)
    for depth, fused_calls in ((2, None), (12, 1)):
        m = M.SharedReadFusedFinal12LocalTHCSharedAdaLNJiT(depth=depth, **kw).to(DEV).eval()
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            with mock.patch.object(ops, "final_accumulate_decoder_head", wraps=ops.final_accumulate_decoder_head) as op:
                if fused_calls is None:
                    with pytest.raises(ValueError, match="depth=12"):
                        m(x, t, y)
                    assert op.call_count == 0
                else:
                    m(x, t, y)
                    assert op.call_count == fused_calls
