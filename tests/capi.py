"""Direct C-ABI calls for the GPU parity tests (torch only allocates memory)."""

from __future__ import annotations

import ctypes

import torch

from flowmatching_lthc_amd import _abi

S = 4


def _lib():
    return _abi.load()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def read(x: torch.Tensor, alpha: torch.Tensor) -> torch.Tensor:
    b, h, _, c = x.shape
    g = h // S
    z = torch.empty((b, g * g, c), device=x.device, dtype=x.dtype)
    rc = _lib().lthc_read_fwd(x.data_ptr(), _abi.code(x), alpha.data_ptr(), _abi.code(alpha), z.data_ptr(), b, g, S, c, _stream())
    _abi.check(rc, "lthc_read_fwd")
    return z


def materialise(base, dzs, betas, h=None) -> torch.Tensor:
    b, m, c = dzs[0].shape
    g = int(round(m**0.5))
    h = g * S
    out = torch.empty((b, h, h, c), device=dzs[0].device, dtype=dzs[0].dtype)
    rc = _lib().lthc_materialise_fwd(
        _abi.ptr(base), _abi.ptr_array(dzs), _abi.code(dzs[0]), _abi.ptr_array(betas), _abi.code(betas[0]),
        out.data_ptr(), b, g, S, c, len(dzs), _stream(),
    )  # fmt: skip
    _abi.check(rc, "lthc_materialise_fwd")
    return out


def read_multi(gr: torch.Tensor, ws) -> list[torch.Tensor]:
    b, h, _, c = gr.shape
    g = h // S
    outs = [torch.empty((b, g * g, c), device=gr.device, dtype=gr.dtype) for _ in ws]
    rc = _lib().lthc_read_multi_fwd(
        gr.data_ptr(), _abi.code(gr), _abi.ptr_array(ws), _abi.code(ws[0]), _abi.ptr_array(outs), b, g, S, c, len(ws), _stream()
    )
    _abi.check(rc, "lthc_read_multi_fwd")
    return outs


def weight_grad(high: torch.Tensor, lows) -> torch.Tensor:
    b, h, _, c = high.shape
    g = h // S
    L = len(lows)
    out = torch.empty((L, c, S * S), device=high.device, dtype=torch.float32)
    nbytes = _abi.weight_grad_workspace_bytes(b, g, S, c, L)
    ws = torch.empty((max(nbytes, 16),), device=high.device, dtype=torch.uint8)
    rc = _lib().lthc_weight_grad(
        high.data_ptr(), _abi.ptr_array(lows), _abi.code(high), out.data_ptr(), b, g, S, c, L, ws.data_ptr(), ws.numel(), _stream()
    )
    _abi.check(rc, "lthc_weight_grad")
    return out


def materialise_bwd(gr: torch.Tensor, dzs, betas) -> tuple[list[torch.Tensor], torch.Tensor]:
    b, h, _, c = gr.shape
    g = h // S
    L = len(dzs)
    outs = [torch.empty((b, g * g, c), device=gr.device, dtype=gr.dtype) for _ in dzs]
    gb = torch.empty((L, c, S * S), device=gr.device, dtype=torch.float32)
    nbytes = _abi.materialise_bwd_workspace_bytes(b, g, S, c, L)
    ws = torch.empty((max(nbytes, 16),), device=gr.device, dtype=torch.uint8)
    rc = _lib().lthc_materialise_bwd(
        gr.data_ptr(), _abi.code(gr), _abi.ptr_array(dzs), _abi.ptr_array(betas), _abi.code(betas[0]),
        _abi.ptr_array(outs), gb.data_ptr(), b, g, S, c, L, ws.data_ptr(), ws.numel(), _stream(),
    )  # fmt: skip
    _abi.check(rc, "lthc_materialise_bwd")
    return outs, gb


def gamma(alpha: torch.Tensor, betas, out_dtype=torch.float32) -> torch.Tensor:
    c, k = alpha.shape
    out = torch.empty((len(betas), c), device=alpha.device, dtype=out_dtype)
    rc = _lib().lthc_gamma(
        alpha.data_ptr(), _abi.ptr_array(betas), _abi.code(alpha), out.data_ptr(), _abi.DTYPE_CODE[out_dtype], c, k, len(betas), _stream()
    )
    _abi.check(rc, "lthc_gamma")
    return out


def recur(z: torch.Tensor, dz: torch.Tensor, gam: torch.Tensor) -> torch.Tensor:
    return recur_into(z, dz, gam, torch.empty_like(z))


def recur_into(z: torch.Tensor, dz: torch.Tensor, gam: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    c = z.shape[-1]
    rc = _lib().lthc_recur_fwd(z.data_ptr(), dz.data_ptr(), _abi.code(z), gam.data_ptr(), _abi.code(gam), out.data_ptr(), z.numel() // c, c, _stream())
    _abi.check(rc, "lthc_recur_fwd")
    return out


def recur_bwd(gr: torch.Tensor, dz: torch.Tensor, gam: torch.Tensor, add: torch.Tensor | None = None):
    c = gr.shape[-1]
    rows = gr.numel() // c
    gdz = torch.empty_like(gr)
    gg = torch.empty((c,), device=gr.device, dtype=torch.float32)
    ws = torch.empty((max(_abi.recur_bwd_workspace_bytes(rows, c), 16),), device=gr.device, dtype=torch.uint8)
    rc = _lib().lthc_recur_bwd(
        gr.data_ptr(), dz.data_ptr(), _abi.ptr(add), _abi.code(gr), gam.data_ptr(), _abi.code(gam), gdz.data_ptr(),
        gg.data_ptr(), rows, c, ws.data_ptr(), ws.numel(), _stream(),
    )  # fmt: skip
    _abi.check(rc, "lthc_recur_bwd")
    return gdz, gg


def recur_bwd_sum(
    gr: torch.Tensor, gb: torch.Tensor, dz: torch.Tensor, gam: torch.Tensor, add: torch.Tensor | None = None,
    gg_dtype: torch.dtype = torch.float32,
):
    c = gr.shape[-1]
    rows = gr.numel() // c
    gsum, gdz = torch.empty_like(gr), torch.empty_like(gr)
    gg = torch.empty((c,), device=gr.device, dtype=gg_dtype)
    ws = torch.empty((max(_abi.recur_bwd_workspace_bytes(rows, c), 16),), device=gr.device, dtype=torch.uint8)
    rc = _lib().lthc_recur_bwd_sum(
        gr.data_ptr(), gb.data_ptr(), dz.data_ptr(), _abi.ptr(add), _abi.code(gr), gam.data_ptr(), _abi.code(gam),
        gsum.data_ptr(), gdz.data_ptr(), gg.data_ptr(), _abi.code(gg), rows, c, ws.data_ptr(), ws.numel(), _stream(),
    )  # fmt: skip
    _abi.check(rc, "lthc_recur_bwd_sum")
    return gsum, gdz, gg


def recur_prefix(z0: torch.Tensor, dzs, gam: torch.Tensor) -> list[torch.Tensor]:
    """Z_1..Z_L from lthc_recur_fwd_prefix; gam [L, C]."""
    c = z0.shape[-1]
    outs = [torch.empty_like(z0) for _ in dzs]
    rc = _lib().lthc_recur_fwd_prefix(
        z0.data_ptr(), _abi.ptr_array(dzs), _abi.code(z0), gam.data_ptr(), _abi.code(gam), _abi.ptr_array(outs),
        z0.numel() // c, c, len(dzs), _stream(),
    )  # fmt: skip
    _abi.check(rc, "lthc_recur_fwd_prefix")
    return outs


def read_bwd(gz: torch.Tensor, x: torch.Tensor, alpha: torch.Tensor, g_base: torch.Tensor | None = None):
    b, h, _, c = x.shape
    g = h // S
    dx = torch.empty_like(x)
    da = torch.empty((c, S * S), device=x.device, dtype=torch.float32)
    nbytes = int(_lib().lthc_read_bwd_workspace_bytes(b, g, S, c))
    ws = torch.empty((max(nbytes, 16),), device=x.device, dtype=torch.uint8)
    rc = _lib().lthc_read_bwd(
        gz.data_ptr(), x.data_ptr(), _abi.code(x), alpha.data_ptr(), _abi.code(alpha), _abi.ptr(g_base),
        dx.data_ptr(), da.data_ptr(), b, g, S, c, ws.data_ptr(), ws.numel(), _stream(),
    )  # fmt: skip
    _abi.check(rc, "lthc_read_bwd")
    return dx, da


def _iface_ws(b, g, c, L, dev):
    nbytes = int(_lib().lthc_interface_workspace_bytes(b, g, S, c, L))
    return torch.empty((max(nbytes, 16),), device=dev, dtype=torch.uint8)


def interface_fwd(x0: torch.Tensor, alpha: torch.Tensor, betas, dzs):
    b, h, _, c = x0.shape
    g, L = h // S, len(dzs)
    zs = [torch.empty((b, g * g, c), device=x0.device, dtype=x0.dtype) for _ in range(L + 1)]
    xl = torch.empty_like(x0)
    ws = _iface_ws(b, g, c, L, x0.device)
    rc = _lib().lthc_interface_fwd(
        x0.data_ptr(), _abi.code(x0), alpha.data_ptr(), _abi.ptr_array(betas), _abi.code(betas[0]),
        _abi.ptr_array(dzs), _abi.ptr_array(zs), xl.data_ptr(), b, g, S, c, L, ws.data_ptr(), ws.numel(), _stream(),
    )  # fmt: skip
    _abi.check(rc, "lthc_interface_fwd")
    return zs, xl


def interface_bwd(gx: torch.Tensor, gzs, x0: torch.Tensor, dzs, alpha: torch.Tensor, betas):
    """gzs: L entries (None = zero).  Returns (dx0, [ddz_l], dalpha fp32 [C,16], dbeta fp32 [L,C,16])."""
    b, h, _, c = x0.shape
    g, L = h // S, len(dzs)
    dx0 = torch.empty_like(x0)
    ddz = [torch.empty_like(d) for d in dzs]
    da = torch.empty((c, S * S), device=x0.device, dtype=torch.float32)
    db = torch.empty((L, c, S * S), device=x0.device, dtype=torch.float32)
    ws = _iface_ws(b, g, c, L, x0.device)
    gz_ptrs = (ctypes.c_void_p * L)(*[None if t is None else t.data_ptr() for t in gzs])
    rc = _lib().lthc_interface_bwd(
        gx.data_ptr(), gz_ptrs, _abi.code(x0), x0.data_ptr(), _abi.ptr_array(dzs), alpha.data_ptr(),
        _abi.ptr_array(betas), _abi.code(betas[0]), dx0.data_ptr(), _abi.ptr_array(ddz), da.data_ptr(), db.data_ptr(),
        b, g, S, c, L, ws.data_ptr(), ws.numel(), _stream(),
    )  # fmt: skip
    _abi.check(rc, "lthc_interface_bwd")
    return dx0, ddz, da, db
