"""GPU parity of the fused branch ops (jit_thc::qk_norm_rope, jit_thc::qk_norm_rope_attention, jit_thc::swiglu,
the gated residuals) against the eager sequences they replace (MI355X only).

The eager sequences are the model's own modules (RMSNorm, VisionRotaryEmbeddingFast on the permuted q/k
views of the projection; chunk + F.silu + mul), so the check covers the exact op chain the kernels stand in
for.  fp32: max|d| / max|ref| <= 1e-6.  16-bit: the kernels reproduce every eager rounding, so at least
99 % of the elements are bit-identical and none differs by more than one unit in the last place
(|d| <= 2^-7 |ref| for bf16, 2^-10 |ref| for fp16) -- a reduction-order difference in the fp32 mean can
move one rounding.  Gradients (recomputed through the eager sequence) equal the eager model's.
"""

from __future__ import annotations

import pytest
import torch

from flowmatching_lthc_amd import model as M
from flowmatching_lthc_amd import ops_branch as OB

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
ULP = {torch.bfloat16: 2.0**-7, torch.float16: 2.0**-10}


def check_close(got, ref, dtype, what):
    got, ref = got.detach().double().cpu(), ref.detach().double().cpu()
    if dtype == torch.float32:
        err = ((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()
        assert err <= 1e-6, f"{what}: {err:.3e}"
        return
    d = (got - ref).abs()
    same = (d == 0).double().mean().item()
    assert same >= 0.99, f"{what}: only {same:.4f} of the elements are bit-identical"
    # one ulp of the operands of the last eager op: where that op cancels (RoPE's add), an intermediate's
    # one-ulp move is many ulps of the small result, so the bound uses the tensor's RMS as the operand scale
    rms = ref.pow(2).mean().sqrt().item()
    bad = (d > ULP[dtype] * (ref.abs() + rms)).sum().item()
    assert bad == 0, f"{what}: {bad} elements differ by more than one operand ulp"


def eager_qk(qkv5, q_norm, k_norm, rope):
    """The model's eager path: permuted views -> RMSNorm module -> RoPE module, back to [B, N, H, D]."""
    q, k, _ = qkv5.permute(2, 0, 3, 1, 4).unbind(0)
    return rope(q_norm(q)).transpose(1, 2), rope(k_norm(k)).transpose(1, 2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_qk_norm_rope_matches_eager(dtype):
    print(f"case dtype={dtype}", flush=True)
    B, G, H, D = 2, 16, 12, 64
    N = G * G
    gen = torch.Generator().manual_seed(0)
    qkv = (torch.randn((B, N, 3, H, D), generator=gen) * 2.0).to(DEV, dtype)
    q_norm, k_norm = M.RMSNorm(D), M.RMSNorm(D)
    with torch.no_grad():
        q_norm.weight.copy_(torch.randn(D, generator=gen) * 0.2 + 1)
        k_norm.weight.copy_(torch.randn(D, generator=gen) * 0.2 + 1)
    rope = M.VisionRotaryEmbeddingFast(D // 2, G)
    q_norm, k_norm, rope = q_norm.to(DEV), k_norm.to(DEV), rope.to(DEV)

    q, k = OB.qk_norm_rope(qkv, q_norm.weight, k_norm.weight, rope.freqs_cos, rope.freqs_sin, q_norm.eps)
    assert q.shape == (B, N, H, D) and q.dtype == dtype and q.is_contiguous()
    rq, rk = eager_qk(qkv, q_norm, k_norm, rope)
    check_close(q, rq, dtype, "q")
    check_close(k, rk, dtype, "k")
    # the op's own eager restatement is the model's sequence
    eq, ek = OB.qk_norm_rope_eager(qkv, q_norm.weight, k_norm.weight, rope.freqs_cos, rope.freqs_sin, q_norm.eps)
    assert torch.equal(eq, rq) and torch.equal(ek, rk)
    # against the exact function in float64 (no intermediate roundings)
    x = qkv.double()
    c, s = rope.freqs_cos.double()[:, None], rope.freqs_sin.double()[:, None]
    for got, part, w in ((q, 0, q_norm.weight), (k, 1, k_norm.weight)):
        v = x[:, :, part]
        n = v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + 1e-6) * w.double()
        rot = torch.stack((-n[..., 1::2], n[..., 0::2]), dim=-1).flatten(-2)
        exact = n * c + rot * s
        tol = 1e-5 if dtype == torch.float32 else 4 * ULP[dtype]
        err = ((got.double() - exact).abs().max() / exact.abs().max()).item()
        assert err <= tol, f"part {part}: {err:.3e} vs exact"

    # gradients equal the eager model's
    g = torch.Generator().manual_seed(1)
    gq = torch.randn(q.shape, generator=g).to(DEV, dtype)
    gk = torch.randn(k.shape, generator=g).to(DEV, dtype)
    leaves = [qkv.clone().requires_grad_(), q_norm.weight.detach().clone().requires_grad_(), k_norm.weight.detach().clone().requires_grad_()]
    fq, fk = OB.qk_norm_rope(leaves[0], leaves[1], leaves[2], rope.freqs_cos, rope.freqs_sin, 1e-6)
    torch.autograd.backward((fq, fk), (gq, gk))
    eleaves = [qkv.clone().requires_grad_()]
    q_norm.weight.grad = k_norm.weight.grad = None
    rq, rk = eager_qk(eleaves[0].view(B, N, 3, H, D), q_norm, k_norm, rope)
    torch.autograd.backward((rq, rk), (gq, gk))
    check_close(leaves[0].grad, eleaves[0].grad, dtype, "grad qkv")
    for got, ref, what in ((leaves[1].grad, q_norm.weight.grad, "grad q weight"), (leaves[2].grad, k_norm.weight.grad, "grad k weight")):
        err = ((got.double() - ref.double()).abs().max() / ref.double().abs().max()).item()
        assert err <= 1e-4, f"{what}: {err:.3e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_swiglu_matches_eager(dtype):
    print(f"case dtype={dtype}", flush=True)
    gen = torch.Generator().manual_seed(2)
    x = (torch.randn((4, 256, 2 * 2048), generator=gen) * 3).to(DEV, dtype)
    out = OB.swiglu(x)
    assert out.shape == (4, 256, 2048) and out.dtype == dtype
    ref = OB.swiglu_eager(x)
    check_close(out, ref, dtype, "swiglu")
    a, v = x.double().chunk(2, -1)
    exact = a * torch.sigmoid(a) * v
    tol = 1e-6 if dtype == torch.float32 else 2 * ULP[dtype]
    assert ((out.double() - exact).abs().max() / exact.abs().max()).item() <= tol
    xl = x.clone().requires_grad_()
    g = torch.randn(out.shape, generator=gen).to(DEV, dtype)
    OB.swiglu(xl).backward(g)
    xe = x.clone().requires_grad_()
    OB.swiglu_eager(xe).backward(g)
    assert torch.equal(xl.grad, xe.grad)
    with pytest.raises(ValueError):
        OB.swiglu(x[..., :24])


def test_model_with_fused_branch_equals_eager_branch(monkeypatch):
    """A model whose heads are 64 wide (the fused path) gives the eager branch's output and gradients (fp32);
    the eager run replaces every fused branch op by its eager sequence."""
    # heads of 64 channels and a SwiGLU width (int(4 * 192 * 2 / 3) = 512) that the fused ops take
    cfg = dict(input_size=32, patch_size=4, hidden_size=192, depth=2, num_heads=3, num_classes=10, bottleneck_dim=16,
               workspace_grid=2, attn_backend="math")
    torch.manual_seed(0)
    m = M.randomize_parameters(M.SharedReadLocalTHCSharedAdaLNJiT(**cfg), seed=3).to(DEV)
    gen = torch.Generator().manual_seed(4)
    x = torch.randn((2, 3, 32, 32), generator=gen).to(DEV)
    t = torch.rand((2,), generator=gen).to(DEV)
    y = torch.randint(0, 10, (2,), generator=gen).to(DEV)
    calls = {"qk": 0, "swiglu": 0}
    real_qk, real_sw = OB.qk_norm_rope, OB.swiglu

    def count_qk(*a):
        calls["qk"] += 1
        return real_qk(*a)

    def count_sw(*a):
        calls["swiglu"] += 1
        return real_sw(*a)

    monkeypatch.setattr(OB, "qk_norm_rope", count_qk)
    monkeypatch.setattr(OB, "swiglu", count_sw)
    out = m(x, t, y)
    out.square().mean().backward()
    grads = {n: p.grad.clone() for n, p in m.named_parameters() if p.grad is not None}
    assert calls == {"qk": 2, "swiglu": 2}, calls
    m.zero_grad()
    monkeypatch.setattr(OB, "qk_norm_rope", OB.qk_norm_rope_eager)
    monkeypatch.setattr(OB, "swiglu", OB.swiglu_eager)
    monkeypatch.setattr(OB, "gate_add_norm_modulate", OB.gate_add_norm_modulate_eager)
    monkeypatch.setattr(OB, "gate_residual", OB.gate_residual_eager)
    ref = m(x, t, y)
    ref.square().mean().backward()
    assert ((out - ref).abs().max() / ref.abs().max()).item() <= 1e-5
    for n, p in m.named_parameters():
        if n in grads:
            scale = p.grad.abs().max().clamp_min(1e-12)
            assert ((grads[n] - p.grad).abs().max() / scale).item() <= 1e-4, n


@pytest.mark.parametrize("N", [256, 9])  # 256: the block-shared kernel; 9: the per-wavefront one
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gated_residual_ops_match_eager(dtype, N):
    print(f"case dtype={dtype} N={N}", flush=True)
    B, C = 4, 768
    gen = torch.Generator().manual_seed(5)
    z, a, m = (torch.randn((B, N, C), generator=gen).to(DEV, dtype) for _ in range(3))
    gate, shift, scale = ((torch.randn((B, 6 * C), generator=gen) * 0.3).to(DEV, dtype)[:, :C] for _ in range(3))
    w = (torch.randn(C, generator=gen) * 0.1 + 1).to(DEV)
    d, y = OB.gate_add_norm_modulate(z, a, gate, w, shift, scale, 1e-6)
    rd, ry = OB.gate_add_norm_modulate_eager(z, a, gate, w, shift, scale, 1e-6)
    assert torch.equal(d, rd), "d = gate * a is one rounded multiply"
    check_close(y, ry, dtype, "y")
    # the eager restatement is the model's: modulate(RMSNorm module(z + d))
    norm = M.RMSNorm(C).to(DEV)
    with torch.no_grad():
        norm.weight.copy_(w)
    assert torch.equal(ry, M.modulate(norm(z + rd), shift, scale))
    out = OB.gate_residual(d, gate, m)
    assert torch.equal(out, OB.gate_residual_eager(d, gate, m)) or dtype == torch.float32
    check_close(out, OB.gate_residual_eager(d, gate, m), dtype, "gate_residual")
    # gradients through both ops equal the eager sequence's
    leaves = [t.clone().requires_grad_() for t in (z, a, gate, shift, scale, m)]
    wl = w.clone().requires_grad_()
    d1, y1 = OB.gate_add_norm_modulate(leaves[0], leaves[1], leaves[2], wl, leaves[3], leaves[4], 1e-6)
    (OB.gate_residual(d1, leaves[2], leaves[5]).float().sum() + y1.float().square().sum()).backward()
    eleaves = [t.clone().requires_grad_() for t in (z, a, gate, shift, scale, m)]
    we = w.clone().requires_grad_()
    d2, y2 = OB.gate_add_norm_modulate_eager(eleaves[0], eleaves[1], eleaves[2], we, eleaves[3], eleaves[4], 1e-6)
    (OB.gate_residual_eager(d2, eleaves[2], eleaves[5]).float().sum() + y2.float().square().sum()).backward()
    for name, p, q in zip(("z", "a", "gate", "shift", "scale", "m"), leaves, eleaves):
        err = ((p.grad.double() - q.grad.double()).abs().max() / q.grad.double().abs().max().clamp_min(1e-30)).item()
        assert err <= (1e-5 if dtype == torch.float32 else 2e-2), f"grad {name}: {err:.3e}"
    err = ((wl.grad - we.grad).abs().max() / we.grad.abs().max()).item()
    assert err <= 1e-4, f"grad weight: {err:.3e}"


# ---------------------------------------------------------------------------
# jit_thc::qk_norm_rope_attention
# ---------------------------------------------------------------------------
def attention_exact(q, k, v):
    """softmax(q k^T / sqrt(64)) v in float64 on the CPU; q, k, v and the result [B, N, H, 64]."""
    q, k, v = (t.detach().double().cpu().transpose(1, 2) for t in (q, k, v))
    s = q @ k.transpose(-1, -2).contiguous() / 8.0
    return (torch.softmax(s, dim=-1) @ v).transpose(1, 2)


def random_rope_tables(n, gen):
    theta = torch.rand((n, 64), generator=gen) * 6.2831853
    return torch.cos(theta).to(DEV), torch.sin(theta).to(DEV)


@pytest.mark.parametrize("dtype,N,H", [(torch.bfloat16, 256, 12), (torch.float16, 256, 4), (torch.bfloat16, 64, 3),
                                       (torch.bfloat16, 192, 2)])
def test_qk_norm_rope_attention_matches_exact(dtype, N, H):
    """Against softmax attention in float64 on the op's own normalised q and k (qk_norm_rope, which the kernel
    reproduces bit for bit) and v: every element within one rounding of the probabilities and one of the output,
    |d| <= u (max|v| + |ref|) with u = 2^-8 (bf16) or 2^-11 (fp16), and no further from the exact result than
    torch's scaled_dot_product_attention on the same q, k, v."""
    print(f"case dtype={dtype} N={N} H={H}", flush=True)
    B = 2
    gen = torch.Generator().manual_seed(7)
    qkv = (torch.randn((B, N, 3, H, 64), generator=gen) * 2.0).to(DEV, dtype)
    qw = (torch.randn(64, generator=gen) * 0.2 + 1).to(DEV)
    kw = (torch.randn(64, generator=gen) * 0.2 + 1).to(DEV)
    cos, sin = random_rope_tables(N, gen)
    o = OB.qk_norm_rope_attention(qkv, qw, kw, cos, sin, 1e-6)
    assert o.shape == (B, N, H, 64) and o.dtype == dtype and o.is_contiguous()
    q, k = OB.qk_norm_rope(qkv, qw, kw, cos, sin, 1e-6)
    v = qkv[:, :, 2]
    ref = attention_exact(q, k, v)
    d = (o.double().cpu() - ref).abs()
    u = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11
    vmax = v.double().abs().max().item()
    bad = (d > u * (vmax + ref.abs())).sum().item()
    assert bad == 0, f"{bad} elements beyond one rounding (max |d| {d.max().item():.3e})"
    sdpa = torch.nn.functional.scaled_dot_product_attention(*(t.transpose(1, 2).contiguous() for t in (q, k, v)))
    e_sdpa = (sdpa.transpose(1, 2).double().cpu() - ref).abs().max().item()
    assert d.max().item() <= max(1.5 * e_sdpa, u * vmax), (d.max().item(), e_sdpa)
    # the op's eager restatement is the path it replaces
    eager = OB.qk_norm_rope_attention_eager(qkv, qw, kw, cos, sin, 1e-6)
    assert (eager.double().cpu() - ref).abs().max().item() <= max(2 * e_sdpa, u * vmax)


def test_qk_norm_rope_attention_gradients_and_errors():
    """The backward (recomputed through the eager q/k norm + RoPE sequence, the attention itself in fp32 products)
    matches autograd of the eager sequence to 1e-2 of each gradient's scale; unsupported shapes and dtypes raise
    ValueError."""
    print("case attention gradients", flush=True)
    B, N, H = 2, 256, 4
    gen = torch.Generator().manual_seed(8)
    qkv = (torch.randn((B, N, 3, H, 64), generator=gen) * 2.0).to(DEV, torch.bfloat16)
    w0 = (torch.randn(64, generator=gen) * 0.2 + 1).to(DEV)
    w1 = (torch.randn(64, generator=gen) * 0.2 + 1).to(DEV)
    cos, sin = random_rope_tables(N, gen)
    g = (torch.randn((B, N, H, 64), generator=gen) * 0.1).to(DEV, torch.bfloat16)
    grads = []
    for fn in (OB.qk_norm_rope_attention, OB.qk_norm_rope_attention_eager):
        leaves = [t.clone().requires_grad_() for t in (qkv, w0, w1)]
        fn(*leaves, cos, sin, 1e-6).backward(g)
        grads.append([t.grad.double() for t in leaves])
    for name, a, b in zip(("qkv", "q_weight", "k_weight"), *grads):
        err = ((a - b).abs().max() / b.abs().max()).item()
        assert err <= 1e-2, f"grad {name}: {err:.3e}"
    with pytest.raises(ValueError):
        OB.qk_norm_rope_attention(qkv[:, :100], w0, w1, cos[:100], sin[:100], 1e-6)
    with pytest.raises(ValueError):
        OB.qk_norm_rope_attention(qkv.float(), w0, w1, cos, sin, 1e-6)


def test_model_fused_attention_matches_sdpa_bf16():
    """A model with 64-wide heads over an 8x8 workspace (N = 64) under bf16 autocast: the fused attention path
    stays as close to the fp32 result as the SDPA path does, and the math backend keeps SDPA."""
    cfg = dict(input_size=128, patch_size=4, hidden_size=192, depth=2, num_heads=3, num_classes=10,
               bottleneck_dim=16, workspace_grid=8)
    m = M.randomize_parameters(M.SharedReadLocalTHCSharedAdaLNJiT(**cfg), seed=5).to(DEV).eval()
    gen = torch.Generator().manual_seed(9)
    x = torch.randn((2, 3, 128, 128), generator=gen).to(DEV)
    t = torch.rand((2,), generator=gen).to(DEV)
    y = torch.randint(0, 10, (2,), generator=gen).to(DEV)
    calls = {"n": 0}
    real = OB.qk_norm_rope_attention

    def count(*a):
        calls["n"] += 1
        return real(*a)

    attns = [blk.branch.attn for blk in m.blocks]
    with torch.no_grad():
        exact = m(x, t, y).double()
        outs = {}
        for fused in (True, False):
            for a in attns:
                a.fused_attention = fused
            OB.qk_norm_rope_attention = count
            try:
                with torch.autocast("cuda", dtype=torch.bfloat16):
                    outs[fused] = m(x, t, y).double()
            finally:
                OB.qk_norm_rope_attention = real
        assert calls["n"] == 2, calls
        for a in attns:
            a.fused_attention, a.attn_backend = True, "math"
        with torch.autocast("cuda", dtype=torch.bfloat16):
            m(x, t, y)
        assert calls["n"] == 2, "the math backend must keep SDPA"

    def rel(a):
        return ((a - exact).abs().max() / exact.abs().max()).item()

    assert rel(outs[True]) <= max(1.5 * rel(outs[False]), 1e-3), (rel(outs[True]), rel(outs[False]))


# ---------------------------------------------------------------------------
# jit_thc::decoder_head (RMSNorm + modulate + linear + unpatchify)
# ---------------------------------------------------------------------------
def unpatchify(o, h, p=4, co=3):
    b, t, _ = o.shape
    w = t // h
    return o.reshape(b, h, w, p, p, co).permute(0, 5, 1, 3, 2, 4).reshape(b, co, h * p, w * p)


@pytest.mark.parametrize("dtype,pdt,C,h", [(torch.bfloat16, torch.float32, 768, 64), (torch.bfloat16, torch.bfloat16, 768, 16),
                                           (torch.float16, torch.float32, 192, 8)])
def test_decoder_head_matches_exact(dtype, pdt, C, h):
    """Against y W^T + b in float64, y being the norm_modulate op's output (the kernel's rounding sequence) and W, b
    rounded to the activation dtype: each pixel within one output rounding plus two ulps of every y element (a
    different reduction order for the inverse RMS can move a y rounding):
    |d| <= u |o| + 4u sum_c |y_c W_jc|,  u = 2^-8 (bf16) or 2^-11 (fp16)."""
    from flowmatching_lthc_amd import ops

    print(f"case dtype={dtype} params={pdt} C={C} h={h}", flush=True)
    B, T = 2, h * h
    gen = torch.Generator().manual_seed(11)
    x = (torch.randn((B, T, C), generator=gen) * 2.0).to(DEV, dtype)
    t2 = (torch.randn((B, 2 * C), generator=gen) * 0.3).to(DEV, dtype)
    shift, scale = t2.chunk(2, dim=1)
    nw = (torch.randn(C, generator=gen) * 0.2 + 1).to(DEV, pdt)
    lw = (torch.randn((48, C), generator=gen) * 0.05).to(DEV, pdt)
    lb = (torch.randn(48, generator=gen) * 0.1).to(DEV, pdt)
    img = ops.decoder_head(x, nw, shift, scale, lw, lb, 1e-6, h, 4)
    assert img.shape == (B, 3, 4 * h, 4 * h) and img.dtype == dtype
    y = ops.norm_modulate(x, nw, shift, scale, 1e-6)[0].double().cpu()
    W, bb = lw.to(dtype).double().cpu(), lb.to(dtype).double().cpu()
    o = y @ W.T + bb
    mag = y.abs() @ W.abs().T
    u = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11
    ref, bound = unpatchify(o, h), unpatchify(u * o.abs() + 4 * u * mag, h)
    d = (img.double().cpu() - ref).abs()
    assert (d <= bound).all(), f"max excess {(d - bound).max().item():.3e}"
    eager = ops.decoder_head_eager(x, nw, shift, scale, lw, lb, 1e-6, h, 4)
    assert ((eager.double().cpu() - ref).abs() <= bound).all(), "the eager restatement is the same function"
    with pytest.raises(ValueError):
        ops.decoder_head(x.float(), nw, shift.float(), scale.float(), lw, lb, 1e-6, h, 4)


def test_decoder_head_gradients():
    """The backward (recomputed through the eager sequence) gives the eager sequence's gradients."""
    from flowmatching_lthc_amd import ops

    print("case decoder gradients", flush=True)
    B, C, h = 2, 192, 8
    gen = torch.Generator().manual_seed(12)
    x = (torch.randn((B, h * h, C), generator=gen) * 2.0).to(DEV, torch.bfloat16)
    t2 = (torch.randn((B, 2 * C), generator=gen) * 0.3).to(DEV, torch.bfloat16)
    nw = (torch.randn(C, generator=gen) * 0.2 + 1).to(DEV)
    lw = (torch.randn((48, C), generator=gen) * 0.05).to(DEV)
    lb = (torch.randn(48, generator=gen) * 0.1).to(DEV)
    g = torch.randn((B, 3, 4 * h, 4 * h), generator=gen).to(DEV, torch.bfloat16)
    grads = []
    for fn in (ops.decoder_head, ops.decoder_head_eager):
        xl, tl = x.clone().requires_grad_(), t2.clone().requires_grad_()
        ws = [t.clone().requires_grad_() for t in (nw, lw, lb)]
        sh, sc = tl.chunk(2, dim=1)
        fn(xl, ws[0], sh, sc, ws[1], ws[2], 1e-6, h, 4).backward(g)
        grads.append([xl.grad.double(), tl.grad.double()] + [w.grad.double() for w in ws])
    for name, a, b in zip(("x", "t2", "norm_weight", "lin_weight", "lin_bias"), *grads):
        err = ((a - b).abs().max() / b.abs().max()).item()
        assert err <= 1e-3, f"grad {name}: {err:.3e}"


def test_model_fused_decoder_matches_unfused_bf16():
    """Under bf16 autocast the fused decoder head stays as close to the fp32 model as the unfused head does."""
    cfg = dict(input_size=128, patch_size=4, hidden_size=192, depth=2, num_heads=3, num_classes=10,
               bottleneck_dim=16, workspace_grid=8)
    m = M.randomize_parameters(M.SharedReadLocalTHCSharedAdaLNJiT(**cfg), seed=6).to(DEV).eval()
    gen = torch.Generator().manual_seed(13)
    x = torch.randn((2, 3, 128, 128), generator=gen).to(DEV)
    t = torch.rand((2,), generator=gen).to(DEV)
    y = torch.randint(0, 10, (2,), generator=gen).to(DEV)
    with torch.no_grad():
        exact = m(x, t, y).double()
        outs = {}
        for fused in (True, False):
            m.fused_decoder = fused
            with torch.autocast("cuda", dtype=torch.bfloat16):
                outs[fused] = m(x, t, y).double()

    def rel(a, b=exact):
        return ((a - b).abs().max() / b.abs().max()).item()

    assert rel(outs[True], outs[False]) <= 2e-2, rel(outs[True], outs[False])
    assert rel(outs[True]) <= max(1.5 * rel(outs[False]), 1e-3), (rel(outs[True]), rel(outs[False]))


# ---------------------------------------------------------------------------
# jit_thc::block_tail (inference: gate_residual + recurrence step + next pre-norm)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype,gdt", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                       (torch.float16, torch.float16), (torch.float32, torch.float32)])
@pytest.mark.parametrize("C,N", [(768, 256), (1024, 256), (136, 256), (768, 7)])
def test_block_tail_equals_the_three_ops(dtype, gdt, C, N):
    """block_tail gives dz, Z_{l+1} and the next pre-norm bit for bit as gate_residual, lazy_workspace_update and
    norm_modulate do in sequence (the AdaLN rows as strided chunks of one [B, 6C] buffer, as in the model).
    N = 256 runs the block-shared kernel, N = 7 the per-wavefront one."""
    from flowmatching_lthc_amd import ops

    print(f"case dtype={dtype} gamma={gdt} C={C} N={N}", flush=True)
    B = 3
    gen = torch.Generator().manual_seed(C)
    z, a, m = ((torch.randn((B, N, C), generator=gen) * s).to(DEV, dtype) for s in (1.0, 0.1, 0.5))
    t6 = (torch.randn((B, 6 * C), generator=gen) * 0.3).to(DEV, dtype)
    sh_a, sc_a, _, _, _, g_m = t6.chunk(6, dim=-1)
    gamma = (torch.randn(C, generator=gen) * 0.05).to(DEV, gdt)
    w = (torch.randn(C, generator=gen) * 0.1 + 1).to(DEV)
    with torch.no_grad():
        dz, zn, y = OB.block_tail(z, a, g_m, m, gamma, w, sh_a, sc_a, 1e-6)
        rdz = OB.gate_residual(a, g_m, m)
        rzn = ops.lazy_workspace_update(z, rdz, gamma)
        ry = ops.norm_modulate(rzn, w, sh_a, sc_a, 1e-6)[0]
    assert torch.equal(dz, rdz), "dz"
    assert torch.equal(zn, rzn), "z_next"
    assert torch.equal(y, ry), "next pre-norm"


def test_model_fused_block_tail_equals_hook_path():
    """LTHC-B/4 forward under no-grad bf16 autocast: the fused block tails give the hook path's output bit for bit,
    also captured in a HIP graph and replayed; with gradients enabled the model keeps the hook path."""
    m = M.randomize_parameters(M.build_model("lthc_b4_velocity"), seed=12).to(DEV).eval()
    gen = torch.Generator().manual_seed(14)
    x = torch.randn((2, 3, 256, 256), generator=gen).to(DEV)
    t = torch.rand((2,), generator=gen).to(DEV)
    y = torch.tensor([7, 512], device=DEV)
    calls = []
    orig = OB.block_tail

    def spy(*args):
        calls.append(1)
        return orig(*args)

    OB.block_tail = spy
    try:
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            m.fused_block_tail = True
            a = m(x, t, y)
            assert len(calls) == len(m.blocks) - 1, "the fused tail path did not run"
            m.fused_block_tail = False
            b = m(x, t, y)
            m.fused_block_tail = True
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                m(x, t, y)
            torch.cuda.current_stream().wait_stream(s)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                c = m(x, t, y)
        for _ in range(3):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(c, a)
        assert torch.equal(a, b)
        calls.clear()
        with torch.autocast("cuda", dtype=torch.bfloat16):
            m(x, t, y).float().sum().backward()
        assert not calls, "the training forward must keep the hook path"
    finally:
        OB.block_tail = orig
