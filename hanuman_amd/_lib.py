"""ctypes binding of ``libhanuman_moe.so`` (declared in ``include/hanuman_moe.h``).

The library is loaded after ``torch`` so that it binds to the HIP runtime
torch already mapped (both carry the soname ``libamdhip64.so.7``): one runtime,
one set of streams.  There is no fallback: if the library is missing or does
not export a declared symbol, :func:`lib` raises.
"""
from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libhanuman_moe.so"
HEADER = PKG.parent / "include" / "hanuman_moe.h"

# hmoe status codes and enums (hanuman_moe.h)
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP, ERR_WORKSPACE = 0, 1, 2, 3, 4
F32, BF16, FP8_E4M3 = 0, 1, 2
ROUTE_SIGMOID_BIAS, ROUTE_SOFTMAX = 0, 1
GEMM_TILE_M = 256

_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes)
SIGNATURES = {
    "hmoe_last_error": (ctypes.c_char_p, []),
    "hmoe_abi_version": (_i32, []),
    "hmoe_capacity": (_i64, [_i64, _i32, _i32, ctypes.c_double]),
    "hmoe_rows_cap": (_i64, [_i64, _i32, _i32, _i64]),
    "hmoe_plan_workspace_bytes": (_sz, [_i64, _i32, _i32]),
    "hmoe_router": (_i32, [_vp, _i32, _vp, _i32, _vp, _i64, _i32, _i32, _i32, _i32, _f32,
                           _vp, _vp, _vp, _vp]),
    "hmoe_router_quant_fp8": (_i32, [_vp, _i32, _vp, _i32, _vp, _i64, _i32, _i32, _i32, _i32,
                                     _f32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "hmoe_router_from_logits": (_i32, [_vp, _vp, _i64, _i32, _i32, _i32, _f32, _vp, _vp, _vp]),
    "hmoe_dispatch_plan": (_i32, [_vp, _i64, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp,
                                  _sz, _vp]),
    "hmoe_dispatch_plan_noalloc": (_i32, [_vp, _i64, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _vp,
                                          _vp]),
    "hmoe_permute_rows": (_i32, [_vp, _i32, _i64, _i32, _i32, _vp, _vp, _i32, _vp]),
    "hmoe_packed_gate_up_bytes": (_sz, [_i32, _i32, _i32]),
    "hmoe_pack_gate_up": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    "hmoe_packed_down_bytes": (_sz, [_i32, _i32, _i32]),
    "hmoe_pack_down": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    "hmoe_grouped_gate_up": (_i32, [_vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp]),
    "hmoe_grouped_gate_up_gather": (_i32, [_vp, _i64, _i32, _vp, _vp, _i32, _i64, _i32, _i32, _vp,
                                           _vp, _vp]),
    "hmoe_grouped_down": (_i32, [_vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp]),
    "hmoe_grouped_swiglu_fused_workspace_bytes": (_sz, [_i64, _i32]),
    "hmoe_zero_fill": (_i32, [_vp, _sz, _vp]),
    "hmoe_grouped_swiglu_fused": (_i32, [_vp, _i64, _i32, _vp, _vp, _i32, _i64, _i32, _i32, _vp,
                                         _vp, _vp, _vp, _vp, _sz, _i64, _i32, _vp]),
    "hmoe_combine": (_i32, [_vp, _i32, _vp, _vp, _vp, _i32, _i64, _i32, _i32, _vp, _i32, _vp]),
    "hmoe_permute_rows_fp8": (_i32, [_vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp, _vp]),
    "hmoe_quantize_rows_fp8": (_i32, [_vp, _i64, _i32, _vp, _i32, _vp, _vp, _vp]),
    "hmoe_packed_fp8_gate_up_bytes": (_sz, [_i32, _i32, _i32]),
    "hmoe_pack_fp8_gate_up": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "hmoe_packed_fp8_down_bytes": (_sz, [_i32, _i32, _i32]),
    "hmoe_pack_fp8_down": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "hmoe_grouped_gate_up_fp8": (_i32, [_vp, _vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp, _vp]),
    "hmoe_grouped_gate_up_fp8_gather": (_i32, [_vp, _vp, _i64, _i32, _vp, _vp, _i32, _i64, _i32,
                                               _i32, _vp, _vp, _vp, _vp]),
    "hmoe_grouped_down_fp8": (_i32, [_vp, _vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp, _vp]),
    "hmoe_grouped_gate_up_fp8_qh": (_i32, [_vp, _vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp,
                                           _vp, _vp]),
    "hmoe_grouped_gate_up_fp8_gather_qh": (_i32, [_vp, _vp, _i64, _i32, _vp, _vp, _i32, _i64,
                                                  _i32, _i32, _vp, _vp, _vp, _vp, _vp]),
    "hmoe_grouped_down_fp8_mx": (_i32, [_vp, _vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp,
                                        _vp]),
    "hmoe_aux_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "hmoe_router_aux": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _sz, _vp]),
    "hmoe_combine_bwd": (_i32, [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _vp, _vp, _vp, _f32, _vp]),
    "hmoe_grouped_gate_up_raw_gather": (_i32, [_vp, _i64, _i32, _vp, _vp, _i32, _i64, _i32, _i32,
                                               _vp, _vp, _vp]),
    "hmoe_grouped_gate_up_raw": (_i32, [_vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp]),
    "hmoe_grouped_gate_up_swiglu_bwd_gather": (_i32, [_vp, _i64, _i32, _vp, _vp, _i32, _i64, _i32,
                                                      _i32, _vp, _vp, _vp, _vp]),
    "hmoe_grouped_gate_up_swiglu_bwd": (_i32, [_vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp, _vp]),
    "hmoe_swiglu_bwd": (_i32, [_vp, _vp, _vp, _i32, _i64, _i32, _vp, _vp]),
    "hmoe_pack_down_dgrad": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    "hmoe_pack_gate_up_dgrad": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    "hmoe_grouped_dgrad_down": (_i32, [_vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp]),
    "hmoe_grouped_dgrad_gate_up": (_i32, [_vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp]),
    "hmoe_gather_bwd": (_i32, [_vp, _i32, _vp, _vp, _i32, _i64, _i32, _i32, _vp, _i32, _vp]),
    "hmoe_router_bwd": (_i32, [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _f32, _vp, _vp]),
    "hmoe_aux_bwd_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "hmoe_router_aux_bwd": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _i32, _vp, _sz, _vp]),
    "hmoe_grouped_gate_up_f32": (_i32, [_vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp, _vp]),
    "hmoe_grouped_down_f32": (_i32, [_vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp]),
    "hmoe_combine_bwd_f32": (_i32, [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _vp, _vp, _vp, _f32, _vp]),
    "hmoe_grouped_dgrad_down_f32": (_i32, [_vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp]),
    "hmoe_grouped_gate_up_swiglu_bwd_f32": (_i32, [_vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp,
                                                   _vp, _vp, _vp]),
    "hmoe_grouped_dgrad_gate_up_f32": (_i32, [_vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp,
                                              _vp]),
    "hmoe_grouped_wgrad_gate_up_f32": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp]),
    "hmoe_grouped_wgrad_down_f32": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp]),
    "hmoe_router_dx": (_i32, [_vp, _vp, _i32, _i64, _i32, _i32, _vp, _i32, _vp]),
    "hmoe_grouped_wgrad_down": (_i32, [_vp, _vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp]),
    "hmoe_grouped_wgrad_gate_up": (_i32, [_vp, _vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp, _vp]),
    "hmoe_router_dw_workspace_bytes": (_sz, [_i64, _i32, _i32]),
    "hmoe_router_dw": (_i32, [_vp, _i32, _vp, _i64, _i32, _i32, _vp, _vp, _sz, _vp]),
}


class HmoeError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.fn, self.code, self.msg = fn, code, msg


_LIB = None


def header_symbols() -> list[str]:
    """Function names declared in ``include/hanuman_moe.h``."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hmoe_[a-z0-9_]+)\s*\(", text)))


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it is missing or incomplete)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -m hanuman_amd.build` (there is no CPU fallback)")
    try:
        import torch  # noqa: F401  -- map torch's HIP runtime first
    except ImportError:
        pass
    so = ctypes.CDLL(str(LIB_PATH), mode=getattr(os, "RTLD_LOCAL", 0))
    missing = [n for n in header_symbols() if not hasattr(so, n)]
    if missing:
        raise RuntimeError(f"{LIB_PATH} does not export {missing}")
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(so, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = so
    return so


def call(name: str, *args) -> None:
    """Calls a status-returning entry point and raises :class:`HmoeError` on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != OK:
        msg = lib().hmoe_last_error().decode(errors="replace")
        raise HmoeError(name, rc, msg)
