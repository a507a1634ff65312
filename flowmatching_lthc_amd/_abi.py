"""ctypes binding of liblthc_hip.so (the C ABI declared in include/lthc.h).

torch is imported first so that its HIP runtime is the one the library binds
to: both name ``libamdhip64.so.7`` as their SONAME, and loading torch first
makes the dynamic linker reuse that copy, so streams and device pointers
handed over from torch are valid inside the library.
"""

from __future__ import annotations

import ctypes
import os
from typing import Sequence

import torch

from ._build import LIB_PATH

F32, BF16, F16 = 0, 1, 2
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP = 0, 1, 2, 3
MAX_LAYERS = 48

DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

# Every symbol include/lthc.h declares (tests check the library exports them).
EXPORTS = (
    "lthc_last_error",
    "lthc_abi_version",
    "lthc_read_fwd",
    "lthc_read_multi_fwd",
    "lthc_materialise_fwd",
    "lthc_weight_grad_workspace_bytes",
    "lthc_weight_grad",
    "lthc_materialise_bwd_workspace_bytes",
    "lthc_materialise_bwd",
    "lthc_noalloc_scratch_bytes",
    "lthc_materialise_bwd_noalloc",
    "lthc_gamma",
    "lthc_gamma_rounded",
    "lthc_gamma_rounded_bwd",
    "lthc_recur_fwd",
    "lthc_recur_bwd_workspace_bytes",
    "lthc_recur_bwd",
    "lthc_recur_bwd_sum",
    "lthc_ws_accumulate_fwd",
    "lthc_ws_accumulate_bwd_workspace_bytes",
    "lthc_ws_accumulate_bwd",
    "lthc_norm_modulate_fwd",
    "lthc_norm_modulate_bwd_workspace_bytes",
    "lthc_norm_modulate_bwd",
    "lthc_qk_norm_rope",
    "lthc_qk_norm_rope_attention",
    "lthc_decoder_fwd",
    "lthc_materialise_decoder_workspace_bytes",
    "lthc_materialise_decoder_fwd",
    "lthc_cast_many",
    "lthc_swiglu",
    "lthc_gate_add_norm_modulate_fwd",
    "lthc_gate_residual",
    "lthc_block_tail_fwd",
    "lthc_recur_fwd_prefix",
    "lthc_read_bwd_workspace_bytes",
    "lthc_read_bwd",
    "lthc_interface_workspace_bytes",
    "lthc_interface_fwd",
    "lthc_interface_bwd",
)

_lib = None


class LthcError(RuntimeError):
    """A HIP runtime failure reported by liblthc_hip.so."""


def load() -> ctypes.CDLL:
    """Load and declare the library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: the LTHC HIP library must be built "
            "(python -m flowmatching_lthc_amd._build); there is no CPU fallback"
        )
    lib = ctypes.CDLL(LIB_PATH)
    vp, ci, i64, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
    pp = ctypes.POINTER(ctypes.c_void_p)
    lib.lthc_last_error.restype = ctypes.c_char_p
    lib.lthc_last_error.argtypes = []
    lib.lthc_abi_version.restype = ci
    lib.lthc_abi_version.argtypes = []
    sig = {
        "lthc_read_fwd": [vp, ci, vp, ci, vp, i64, i64, i64, i64, vp],
        "lthc_read_multi_fwd": [vp, ci, pp, ci, pp, i64, i64, i64, i64, ci, vp],
        "lthc_materialise_fwd": [vp, pp, ci, pp, ci, vp, i64, i64, i64, i64, ci, vp],
        "lthc_weight_grad": [vp, pp, ci, vp, i64, i64, i64, i64, ci, vp, sz, vp],
        "lthc_materialise_bwd": [vp, ci, pp, pp, ci, pp, vp, i64, i64, i64, i64, ci, vp, sz, vp],
        "lthc_materialise_bwd_noalloc": [vp, ci, pp, pp, ci, pp, vp, i64, i64, i64, i64, ci, vp],
        "lthc_gamma": [vp, pp, ci, vp, ci, i64, i64, ci, vp],
        "lthc_gamma_rounded": [vp, ci, pp, ci, vp, ci, i64, i64, ci, vp],
        "lthc_gamma_rounded_bwd": [vp, vp, ci, pp, ci, vp, pp, ci, i64, i64, ci, vp],
        "lthc_recur_fwd": [vp, vp, ci, vp, ci, vp, i64, i64, vp],
        "lthc_recur_bwd": [vp, vp, vp, ci, vp, ci, vp, vp, i64, i64, vp, sz, vp],
        "lthc_recur_bwd_sum": [vp, vp, vp, vp, ci, vp, ci, vp, vp, vp, ci, i64, i64, vp, sz, vp],
        "lthc_ws_accumulate_fwd": [vp, pp, ci, vp, ci, vp, i64, i64, ci, vp],
        "lthc_ws_accumulate_bwd": [vp, pp, ci, vp, ci, pp, vp, i64, i64, ci, vp, sz, vp],
        "lthc_norm_modulate_fwd": [vp, ci, vp, ci, vp, vp, i64, vp, vp, i64, i64, i64, ctypes.c_float, vp],
        "lthc_qk_norm_rope": [vp, ci, vp, vp, ci, vp, vp, ci, vp, vp, i64, i64, i64, i64, ctypes.c_float, vp],
        "lthc_qk_norm_rope_attention": [
            vp, ci, vp, vp, ci, vp, vp, ci, vp, i64, i64, i64, i64, ctypes.c_float, ctypes.c_float, vp,
        ],  # fmt: skip
        "lthc_decoder_fwd": [
            vp, ci, vp, ci, vp, vp, i64, vp, ci, vp, ci, vp, i64, i64, i64, i64, i64, i64, ctypes.c_float, vp,
        ],  # fmt: skip
        "lthc_materialise_decoder_fwd": [
            vp, ci, pp, pp, ci, vp, ci, vp, vp, i64, vp, ci, vp, ci, vp, i64, i64, i64, i64, ci, i64, i64,
            ctypes.c_float, vp, sz, vp,
        ],  # fmt: skip
        "lthc_cast_many": [vp, vp, i64, vp, ci, vp],
        "lthc_swiglu": [vp, ci, vp, i64, i64, vp],
        "lthc_gate_add_norm_modulate_fwd": [
            vp, vp, vp, ci, vp, ci, vp, vp, i64, vp, vp, vp, i64, i64, i64, ctypes.c_float, vp,
        ],  # fmt: skip
        "lthc_gate_residual": [vp, vp, i64, vp, ci, vp, i64, i64, i64, vp],
        "lthc_recur_fwd_prefix": [vp, pp, ci, vp, ci, pp, i64, i64, ci, vp],
        "lthc_read_bwd": [vp, vp, ci, vp, ci, vp, vp, vp, i64, i64, i64, i64, vp, sz, vp],
        "lthc_interface_fwd": [vp, ci, vp, pp, ci, pp, pp, vp, i64, i64, i64, i64, ci, vp, sz, vp],
        "lthc_interface_bwd": [
            vp, pp, ci, vp, pp, vp, pp, ci, vp, pp, vp, vp, i64, i64, i64, i64, ci, vp, sz, vp,
        ],  # fmt: skip
        "lthc_block_tail_fwd": [
            vp, vp, vp, vp, ci, vp, ci, vp, ci, vp, vp, i64, vp, vp, vp, i64, i64, i64, ctypes.c_float, vp,
        ],  # fmt: skip
        "lthc_norm_modulate_bwd": [vp, vp, ci, vp, ci, vp, i64, vp, vp, vp, vp, vp, i64, i64, i64, vp, sz, vp],
    }
    for name, args in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ci
    lib.lthc_weight_grad_workspace_bytes.argtypes = [i64, i64, i64, i64, ci]
    lib.lthc_weight_grad_workspace_bytes.restype = sz
    lib.lthc_materialise_bwd_workspace_bytes.argtypes = [i64, i64, i64, i64, ci]
    lib.lthc_materialise_bwd_workspace_bytes.restype = sz
    lib.lthc_noalloc_scratch_bytes.argtypes = []
    lib.lthc_noalloc_scratch_bytes.restype = sz
    lib.lthc_materialise_decoder_workspace_bytes.argtypes = [i64, i64, i64, i64]
    lib.lthc_materialise_decoder_workspace_bytes.restype = sz
    lib.lthc_read_bwd_workspace_bytes.argtypes = [i64, i64, i64, i64]
    lib.lthc_read_bwd_workspace_bytes.restype = sz
    lib.lthc_interface_workspace_bytes.argtypes = [i64, i64, i64, i64, ci]
    lib.lthc_interface_workspace_bytes.restype = sz
    lib.lthc_recur_bwd_workspace_bytes.argtypes = [i64, i64]
    lib.lthc_recur_bwd_workspace_bytes.restype = sz
    lib.lthc_ws_accumulate_bwd_workspace_bytes.argtypes = [i64, i64, ci]
    lib.lthc_ws_accumulate_bwd_workspace_bytes.restype = sz
    lib.lthc_norm_modulate_bwd_workspace_bytes.argtypes = [i64, i64, i64]
    lib.lthc_norm_modulate_bwd_workspace_bytes.restype = sz
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc == OK:
        return
    msg = load().lthc_last_error().decode(errors="replace") or what
    if rc in (ERR_INVALID, ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise LthcError(msg)


def code(t: torch.Tensor) -> int:
    try:
        return DTYPE_CODE[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}; expected float32, bfloat16 or float16") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def ptr_array(ts: Sequence[torch.Tensor]):
    return (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """The raw hipStream_t of torch's current stream on t's device."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def weight_grad_workspace_bytes(B: int, G: int, S: int, C: int, L: int) -> int:
    return int(load().lthc_weight_grad_workspace_bytes(B, G, S, C, L))


def materialise_bwd_workspace_bytes(B: int, G: int, S: int, C: int, L: int) -> int:
    return int(load().lthc_materialise_bwd_workspace_bytes(B, G, S, C, L))


def materialise_decoder_workspace_bytes(B: int, G: int, S: int, C: int) -> int:
    return int(load().lthc_materialise_decoder_workspace_bytes(B, G, S, C))


def recur_bwd_workspace_bytes(rows: int, C: int) -> int:
    return int(load().lthc_recur_bwd_workspace_bytes(rows, C))


def norm_modulate_bwd_workspace_bytes(B: int, N: int, C: int) -> int:
    return int(load().lthc_norm_modulate_bwd_workspace_bytes(B, N, C))


def ws_accumulate_bwd_workspace_bytes(rows: int, C: int, L: int) -> int:
    return int(load().lthc_ws_accumulate_bwd_workspace_bytes(rows, C, L))
