"""Per-stage wrappers over the C ABI on torch device tensors.

torch provides device memory and the current stream; every computation runs in
``libhanuman_moe.so``.  Each wrapper validates shapes/dtypes/devices on the
host (so no kernel ever sees an inconsistent launch), allocates outputs with
``torch.empty`` and enqueues the kernel on ``torch.cuda.current_stream()``.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from ._lib import call

_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32 or bfloat16") from None


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _check(t: torch.Tensor, name: str, ndim: int | None = None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be on a GPU device (got {t.device})")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must have {ndim} dims (got shape {tuple(t.shape)})")


def capacity(tokens: int, top_k: int, n_experts: int, capacity_factor) -> int:
    """Capacity per expert (``ceil(CF*T*K/N)``; ``None`` = dropless)."""
    cf = 0.0 if capacity_factor is None else float(capacity_factor)
    return int(_lib.lib().hmoe_capacity(tokens, top_k, n_experts, cf))


def rows_cap(tokens: int, top_k: int, n_experts: int, cap: int) -> int:
    return int(_lib.lib().hmoe_rows_cap(tokens, top_k, n_experts, cap))


# ---------------------------------------------------------------- router --

def router(x: torch.Tensor, router_w: torch.Tensor, bias: torch.Tensor | None, top_k: int,
           mode: int = _lib.ROUTE_SIGMOID_BIAS, routed_scaling_factor: float = 1.0):
    """Router logits, top-k indices and gates (``moe.py:175-192``).

    ``x [T,D]``, ``router_w [D,N]``, ``bias [N]`` float32 or None.
    Returns (logits f32 [T,N], top_idx i32 [T,K], gates f32 [T,K]).
    """
    _check(x, "x", 2)
    _check(router_w, "router_w", 2)
    T, D = x.shape
    if router_w.shape[0] != D:
        raise ValueError(f"router_w has {router_w.shape[0]} rows, x has d_model {D}")
    N = router_w.shape[1]
    if bias is not None:
        _check(bias, "bias", 1)
        if bias.dtype != torch.float32 or bias.shape[0] != N:
            raise ValueError("bias must be float32 [n_experts]")
    dev = x.device
    logits = torch.empty((T, N), dtype=torch.float32, device=dev)
    top_idx = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    gates = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    call("hmoe_router", _ptr(x), _dtype_code(x), _ptr(router_w), _dtype_code(router_w),
         _ptr(bias), T, D, N, top_k, mode, float(routed_scaling_factor), _ptr(logits),
         _ptr(top_idx), _ptr(gates), _stream())
    return logits, top_idx, gates


def router_quant_fp8(x: torch.Tensor, router_w: torch.Tensor, bias: torch.Tensor | None,
                     top_k: int, mode: int = _lib.ROUTE_SIGMOID_BIAS,
                     routed_scaling_factor: float = 1.0):
    """:func:`router` and :func:`quantize_rows_fp8` of ``x`` in one launch
    (``hmoe_router_quant_fp8``): the per-token e4m3 quantisation runs in
    workgroups beside the router's.  ``x`` is bf16 ``[T,D]``.  Returns
    (logits, top_idx, gates, x_q uint8 [T,D], x_scale f32 [T]), bit-identical
    to the two calls."""
    _check(x, "x", 2)
    _check(router_w, "router_w", 2)
    if x.dtype != torch.bfloat16:
        raise TypeError("router_quant_fp8 takes bf16 tokens")
    T, D = x.shape
    if router_w.shape[0] != D:
        raise ValueError(f"router_w has {router_w.shape[0]} rows, x has d_model {D}")
    N = router_w.shape[1]
    if bias is not None:
        _check(bias, "bias", 1)
        if bias.dtype != torch.float32 or bias.shape[0] != N:
            raise ValueError("bias must be float32 [n_experts]")
    dev = x.device
    logits = torch.empty((T, N), dtype=torch.float32, device=dev)
    top_idx = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    gates = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    x_q = torch.empty((T, D), dtype=torch.uint8, device=dev)
    x_s = torch.empty(T, dtype=torch.float32, device=dev)
    call("hmoe_router_quant_fp8", _ptr(x), _dtype_code(x), _ptr(router_w), _dtype_code(router_w),
         _ptr(bias), T, D, N, top_k, mode, float(routed_scaling_factor), _ptr(logits),
         _ptr(top_idx), _ptr(gates), _ptr(x_q), _ptr(x_s), _stream())
    return logits, top_idx, gates, x_q, x_s


def router_from_logits(logits: torch.Tensor, bias: torch.Tensor | None, top_k: int,
                       mode: int = _lib.ROUTE_SOFTMAX, routed_scaling_factor: float = 1.0):
    """Top-k indices and gates from given float32 logits [T,N]."""
    _check(logits, "logits", 2)
    if logits.dtype != torch.float32:
        raise TypeError("logits must be float32")
    T, N = logits.shape
    if bias is not None:
        _check(bias, "bias", 1)
        if bias.dtype != torch.float32 or bias.shape[0] != N:
            raise ValueError("bias must be float32 [n_experts]")
    top_idx = torch.empty((T, top_k), dtype=torch.int32, device=logits.device)
    gates = torch.empty((T, top_k), dtype=torch.float32, device=logits.device)
    call("hmoe_router_from_logits", _ptr(logits), _ptr(bias), T, N, top_k, mode,
         float(routed_scaling_factor), _ptr(top_idx), _ptr(gates), _stream())
    return top_idx, gates


# ---------------------------------------------------------- dispatch plan --

@dataclass
class Plan:
    """Dispatch plan of one call (see ``hmoe_dispatch_plan``)."""
    counts: torch.Tensor    # [N] int32, pre-drop histogram (bincount)
    offsets: torch.Tensor   # [N+1] int32, kept-row segment starts
    slot_pos: torch.Tensor  # [T*K] int32, dispatched row of slot i or -1
    perm_src: torch.Tensor  # [rows_cap] int32, slot of row j or -1
    keep: torch.Tensor      # [T*K] uint8
    capacity: int
    rows_cap: int
    n_experts: int
    top_k: int


def dispatch_plan(top_idx: torch.Tensor, n_experts: int, cap: int,
                  workspace: torch.Tensor | None = None) -> Plan:
    """Stable expert-grouped permutation with capacity drops (``moe.py:54-57,80``)."""
    _check(top_idx, "top_idx", 2)
    if top_idx.dtype != torch.int32:
        raise TypeError("top_idx must be int32")
    T, K = top_idx.shape
    dev = top_idx.device
    rc = rows_cap(T, K, n_experts, cap)
    ws_bytes = int(_lib.lib().hmoe_plan_workspace_bytes(T, K, n_experts))
    if workspace is None or workspace.numel() < ws_bytes:
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    counts = torch.empty(n_experts, dtype=torch.int32, device=dev)
    offsets = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    slot_pos = torch.empty(T * K, dtype=torch.int32, device=dev)
    perm_src = torch.empty(rc, dtype=torch.int32, device=dev)
    keep = torch.empty(T * K, dtype=torch.uint8, device=dev)
    call("hmoe_dispatch_plan", _ptr(top_idx), T, K, n_experts, cap, _ptr(counts), _ptr(offsets),
         _ptr(slot_pos), _ptr(perm_src), _ptr(keep), _ptr(workspace), workspace.numel(),
         _stream())
    return Plan(counts, offsets, slot_pos, perm_src, keep, cap, rc, n_experts, K)


def permute_rows(x: torch.Tensor, plan: Plan, out_dtype: torch.dtype = torch.bfloat16):
    """Dispatched rows ``xs [rows_cap, D]`` (``moe.py:56,198``); token-centric."""
    _check(x, "x", 2)
    T, D = x.shape
    if plan.slot_pos.numel() != T * plan.top_k:
        raise ValueError("plan does not match x's token count")
    xs = torch.empty((plan.rows_cap, D), dtype=out_dtype, device=x.device)
    call("hmoe_permute_rows", _ptr(x), _dtype_code(x), T, D, plan.top_k, _ptr(plan.slot_pos),
         _ptr(xs), _DT[out_dtype], _stream())
    return xs


def permute_rows_fp8(x: torch.Tensor, plan: Plan):
    """Dispatched e4m3 rows and their per-token scales (fp8 workload rule):
    ``(xs_q uint8 [rows_cap, D], xs_scale f32 [rows_cap])``."""
    _check(x, "x", 2)
    T, D = x.shape
    if plan.slot_pos.numel() != T * plan.top_k:
        raise ValueError("plan does not match x's token count")
    xs_q = torch.empty((plan.rows_cap, D), dtype=torch.uint8, device=x.device)
    xs_s = torch.empty(plan.rows_cap, dtype=torch.float32, device=x.device)
    call("hmoe_permute_rows_fp8", _ptr(x), _dtype_code(x), T, D, plan.top_k, _ptr(plan.slot_pos),
         _ptr(xs_q), _ptr(xs_s), _stream())
    return xs_q, xs_s


def quantize_rows_fp8(a: torch.Tensor, offsets: torch.Tensor | None = None):
    """Per-row e4m3 codes and scales of a bf16 matrix ``[rows, cols]``; rows at
    or past ``offsets[-1]`` are not read when offsets are given (codes left as
    allocated, scale 1)."""
    _check(a, "a", 2)
    if a.dtype != torch.bfloat16:
        raise TypeError("quantize_rows_fp8 takes a bf16 matrix")
    rows, cols = a.shape
    q = torch.empty((rows, cols), dtype=torch.uint8, device=a.device)
    sc = torch.empty(rows, dtype=torch.float32, device=a.device)
    n = 0
    if offsets is not None:
        _check(offsets, "offsets", 1)
        n = offsets.numel() - 1
    call("hmoe_quantize_rows_fp8", _ptr(a), rows, cols, _ptr(offsets), n, _ptr(q), _ptr(sc),
         _stream())
    return q, sc


# ---------------------------------------------------------------- weights --

def pack_gate_up(w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """bf16 gate/up operand [N, 2F, D] from ``[N,D,F]`` masters (``moe.py:204-205``)."""
    _check(w_gate, "w_gate", 3)
    _check(w_up, "w_up", 3)
    if w_gate.shape != w_up.shape or w_gate.dtype != w_up.dtype:
        raise ValueError("w_gate and w_up must have the same shape and dtype")
    N, D, F = w_gate.shape
    out = torch.empty((N, 2 * F, D), dtype=torch.bfloat16, device=w_gate.device)
    call("hmoe_pack_gate_up", _ptr(w_gate), _ptr(w_up), _dtype_code(w_gate), N, D, F, _ptr(out),
         _stream())
    return out


def pack_down(w_down: torch.Tensor) -> torch.Tensor:
    """bf16 down operand [N, D, F] from the ``[N,F,D]`` master (``moe.py:206``)."""
    _check(w_down, "w_down", 3)
    N, F, D = w_down.shape
    out = torch.empty((N, D, F), dtype=torch.bfloat16, device=w_down.device)
    call("hmoe_pack_down", _ptr(w_down), _dtype_code(w_down), N, F, D, _ptr(out), _stream())
    return out


def pack_fp8_gate_up(w_gate: torch.Tensor, w_up: torch.Tensor):
    """e4m3 gate/up operand [N, 2F, D] (uint8) and its scales [N, 2F]."""
    _check(w_gate, "w_gate", 3)
    _check(w_up, "w_up", 3)
    if w_gate.shape != w_up.shape or w_gate.dtype != w_up.dtype:
        raise ValueError("w_gate and w_up must have the same shape and dtype")
    N, D, F = w_gate.shape
    out = torch.empty((N, 2 * F, D), dtype=torch.uint8, device=w_gate.device)
    sc = torch.empty((N, 2 * F), dtype=torch.float32, device=w_gate.device)
    call("hmoe_pack_fp8_gate_up", _ptr(w_gate), _ptr(w_up), _dtype_code(w_gate), N, D, F,
         _ptr(out), _ptr(sc), _stream())
    return out, sc


def pack_fp8_down(w_down: torch.Tensor):
    """e4m3 down operand [N, D, F] (uint8) and its scales [N, D]."""
    _check(w_down, "w_down", 3)
    N, F, D = w_down.shape
    out = torch.empty((N, D, F), dtype=torch.uint8, device=w_down.device)
    sc = torch.empty((N, D), dtype=torch.float32, device=w_down.device)
    call("hmoe_pack_fp8_down", _ptr(w_down), _dtype_code(w_down), N, F, D, _ptr(out), _ptr(sc),
         _stream())
    return out, sc


# ------------------------------------------------------------ grouped GEMM --

def grouped_gate_up(xs: torch.Tensor, offsets: torch.Tensor, w_gate_up: torch.Tensor,
                    rows: int | None = None) -> torch.Tensor:
    """``h = bf16(silu(xs Wg) * (xs Wu))`` per expert segment (``moe.py:70-72``)."""
    _check(xs, "xs", 2)
    _check(offsets, "offsets", 1)
    _check(w_gate_up, "w_gate_up", 3)
    if xs.dtype != torch.bfloat16 or w_gate_up.dtype != torch.bfloat16:
        raise TypeError("grouped_gate_up takes bf16 operands")
    N, F2, D = w_gate_up.shape
    if xs.shape[1] != D or offsets.numel() != N + 1 or offsets.dtype != torch.int32:
        raise ValueError("grouped_gate_up: inconsistent shapes")
    R = xs.shape[0] if rows is None else rows
    h = torch.empty((xs.shape[0], F2 // 2), dtype=torch.bfloat16, device=xs.device)
    call("hmoe_grouped_gate_up", _ptr(xs), _ptr(offsets), N, R, D, F2 // 2, _ptr(w_gate_up),
         _ptr(h), _stream())
    return h


def grouped_gate_up_gather(x: torch.Tensor, plan: Plan, w_gate_up: torch.Tensor) -> torch.Tensor:
    """``h`` of :func:`grouped_gate_up` on the dispatched rows of ``x`` without
    materialising them: the GEMM loads row ``r`` from ``x[perm_src[r] // K]``
    (``moe.py:56`` fused into ``moe.py:70-72``)."""
    _check(x, "x", 2)
    _check(w_gate_up, "w_gate_up", 3)
    if x.dtype != torch.bfloat16 or w_gate_up.dtype != torch.bfloat16:
        raise TypeError("grouped_gate_up_gather takes bf16 operands")
    T, D = x.shape
    N, F2, D2 = w_gate_up.shape
    if D2 != D or plan.n_experts != N or plan.slot_pos.numel() != T * plan.top_k:
        raise ValueError("grouped_gate_up_gather: inconsistent shapes")
    h = torch.empty((plan.rows_cap, F2 // 2), dtype=torch.bfloat16, device=x.device)
    call("hmoe_grouped_gate_up_gather", _ptr(x), T, plan.top_k, _ptr(plan.perm_src),
         _ptr(plan.offsets), N, plan.rows_cap, D, F2 // 2, _ptr(w_gate_up), _ptr(h), _stream())
    return h


def grouped_down(h: torch.Tensor, offsets: torch.Tensor, w_down: torch.Tensor,
                 rows: int | None = None) -> torch.Tensor:
    """``ys = bf16(h Wd)`` per expert segment (``moe.py:73-74``)."""
    _check(h, "h", 2)
    _check(offsets, "offsets", 1)
    _check(w_down, "w_down", 3)
    if h.dtype != torch.bfloat16 or w_down.dtype != torch.bfloat16:
        raise TypeError("grouped_down takes bf16 operands")
    N, D, F = w_down.shape
    if h.shape[1] != F or offsets.numel() != N + 1 or offsets.dtype != torch.int32:
        raise ValueError("grouped_down: inconsistent shapes")
    R = h.shape[0] if rows is None else rows
    ys = torch.empty((h.shape[0], D), dtype=torch.bfloat16, device=h.device)
    call("hmoe_grouped_down", _ptr(h), _ptr(offsets), N, R, F, D, _ptr(w_down), _ptr(ys),
         _stream())
    return ys


FUSED_STATUS_WORD = 8   # uint32 word of the fused launch's workspace: bit 0 = a wait gave up


def grouped_swiglu_fused_workspace(plan: Plan) -> torch.Tensor:
    """Workspace of :func:`grouped_swiglu_fused` for plans of this shape."""
    n = int(_lib.lib().hmoe_grouped_swiglu_fused_workspace_bytes(plan.rows_cap, plan.n_experts))
    # zero before the first call; every call leaves it zeroed again
    return torch.zeros(max(n, 4 * (FUSED_STATUS_WORD + 1)), dtype=torch.uint8,
                       device=plan.offsets.device)


def grouped_swiglu_fused(x: torch.Tensor, plan: Plan, w_gate_up: torch.Tensor,
                         w_down: torch.Tensor, workspace: torch.Tensor | None = None,
                         wait_timeout_us: int = 0, extra_ready_needed: int = 0):
    """``h`` and ``ys`` of :func:`grouped_gate_up_gather` then :func:`grouped_down`
    in one persistent launch (``moe.py:56,70-74``), bit-identical.  Returns
    ``(h, ys, workspace)``; word :data:`FUSED_STATUS_WORD` of the workspace
    (uint32) is 0 when every down tile's wait for its gate/up tiles was met.
    A workspace passed in must have been zero before its first call (as
    :func:`grouped_swiglu_fused_workspace` makes it); each call leaves it so."""
    _check(x, "x", 2)
    _check(w_gate_up, "w_gate_up", 3)
    _check(w_down, "w_down", 3)
    if x.dtype != torch.bfloat16 or w_gate_up.dtype != torch.bfloat16 or w_down.dtype != torch.bfloat16:
        raise TypeError("grouped_swiglu_fused takes bf16 operands")
    T, D = x.shape
    N, F2, D2 = w_gate_up.shape
    if (D2 != D or plan.n_experts != N or plan.slot_pos.numel() != T * plan.top_k
            or tuple(w_down.shape) != (N, D, F2 // 2)):
        raise ValueError("grouped_swiglu_fused: inconsistent shapes")
    if workspace is None:
        workspace = grouped_swiglu_fused_workspace(plan)
    _check(workspace, "workspace", 1)
    h = torch.empty((plan.rows_cap, F2 // 2), dtype=torch.bfloat16, device=x.device)
    ys = torch.empty((plan.rows_cap, D), dtype=torch.bfloat16, device=x.device)
    call("hmoe_grouped_swiglu_fused", _ptr(x), T, plan.top_k, _ptr(plan.perm_src),
         _ptr(plan.offsets), N, plan.rows_cap, D, F2 // 2, _ptr(w_gate_up), _ptr(w_down), _ptr(h),
         _ptr(ys), _ptr(workspace), workspace.numel() * workspace.element_size(),
         int(wait_timeout_us), int(extra_ready_needed), _stream())
    return h, ys, workspace


def fused_status(workspace: torch.Tensor) -> int:
    """Status word of a fused launch's workspace (synchronises with the device)."""
    return int(workspace[4 * FUSED_STATUS_WORD:4 * FUSED_STATUS_WORD + 4].view(torch.int32).item())


def grouped_gate_up_f32(xs: torch.Tensor, offsets: torch.Tensor, w_gate: torch.Tensor,
                        w_up: torch.Tensor) -> torch.Tensor:
    """Float32 ``h = silu(xs Wg[e]) * (xs Wu[e])`` per expert segment
    (``moe.py:70-72`` with dtype float32), masters ``[N, D, F]`` as they are."""
    for t, n in ((xs, "xs"), (offsets, "offsets"), (w_gate, "w_gate"), (w_up, "w_up")):
        _check(t, n)
    if xs.dtype != torch.float32 or w_gate.dtype != torch.float32 or w_up.dtype != torch.float32:
        raise TypeError("grouped_gate_up_f32 takes float32 operands")
    R, D = xs.shape
    N, D2, F = w_gate.shape
    if D2 != D or tuple(w_up.shape) != (N, D, F) or offsets.numel() != N + 1:
        raise ValueError("grouped_gate_up_f32: inconsistent shapes")
    h = torch.empty((R, F), dtype=torch.float32, device=xs.device)
    call("hmoe_grouped_gate_up_f32", _ptr(xs), _ptr(offsets), N, R, D, F, _ptr(w_gate), _ptr(w_up),
         _ptr(h), _stream())
    return h


def combine_bwd_f32(dy: torch.Tensor, ys: torch.Tensor, plan: Plan, gates: torch.Tensor,
                    n_shared: int = 0):
    """VJP of :func:`combine` for float32 rows (compute dtype float32):
    ``(d_ys f32 [rows, D], d_gates f32 [T, K], d_shared)`` with ``d_shared =
    dy / n_shared`` ``[T, D]`` when ``n_shared > 0``, else None."""
    for t, n in ((dy, "dy"), (ys, "ys"), (gates, "gates")):
        _check(t, n, 2)
    T, D = dy.shape
    K = plan.top_k
    if (dy.dtype != torch.float32 or ys.dtype != torch.float32 or ys.shape[1] != D
            or tuple(gates.shape) != (T, K) or gates.dtype != torch.float32
            or plan.slot_pos.numel() != T * K):
        raise ValueError("combine_bwd_f32: inconsistent shapes or dtypes")
    d_ys = torch.empty_like(ys)
    d_g = torch.empty((T, K), dtype=torch.float32, device=dy.device)
    d_sh = torch.empty((T, D), dtype=torch.float32, device=dy.device) if n_shared > 0 else None
    call("hmoe_combine_bwd_f32", _ptr(dy), _ptr(ys), _ptr(plan.slot_pos), _ptr(gates), T, K, D,
         _ptr(d_ys), _ptr(d_g), _ptr(d_sh), float(max(n_shared, 1)), _stream())
    return d_ys, d_g, d_sh


def _f32_operands(name: str, *ts):
    for t in ts:
        _check(t, name)
        if t.dtype != torch.float32:
            raise TypeError(f"{name} takes float32 operands")


def grouped_dgrad_down_f32(d_ys: torch.Tensor, offsets: torch.Tensor,
                           w_down: torch.Tensor) -> torch.Tensor:
    """Float32 ``dh = d_ys Wd[e]^T`` per expert segment, ``[rows, F]``."""
    _f32_operands("grouped_dgrad_down_f32", d_ys, w_down)
    _check(offsets, "offsets", 1)
    R, D = d_ys.shape
    N, F, D2 = w_down.shape
    if D2 != D or offsets.numel() != N + 1:
        raise ValueError("grouped_dgrad_down_f32: inconsistent shapes")
    dh = torch.empty((R, F), dtype=torch.float32, device=d_ys.device)
    call("hmoe_grouped_dgrad_down_f32", _ptr(d_ys), _ptr(offsets), N, R, D, F, _ptr(w_down),
         _ptr(dh), _stream())
    return dh


def grouped_gate_up_swiglu_bwd_f32(xs: torch.Tensor, offsets: torch.Tensor, w_gate: torch.Tensor,
                                   w_up: torch.Tensor, dh: torch.Tensor) -> torch.Tensor:
    """g, u recomputed from ``xs`` and the VJP of ``h = silu(g) * u``:
    float32 ``[rows, 2F]`` = ``[dg | du]``."""
    _f32_operands("grouped_gate_up_swiglu_bwd_f32", xs, w_gate, w_up, dh)
    _check(offsets, "offsets", 1)
    R, D = xs.shape
    N, D2, F = w_gate.shape
    if (D2 != D or tuple(w_up.shape) != (N, D, F) or tuple(dh.shape) != (R, F)
            or offsets.numel() != N + 1):
        raise ValueError("grouped_gate_up_swiglu_bwd_f32: inconsistent shapes")
    dgu = torch.empty((R, 2 * F), dtype=torch.float32, device=xs.device)
    call("hmoe_grouped_gate_up_swiglu_bwd_f32", _ptr(xs), _ptr(offsets), N, R, D, F, _ptr(w_gate),
         _ptr(w_up), _ptr(dh), _ptr(dgu), _stream())
    return dgu


def grouped_dgrad_gate_up_f32(dgu: torch.Tensor, offsets: torch.Tensor, w_gate: torch.Tensor,
                              w_up: torch.Tensor) -> torch.Tensor:
    """Float32 ``d_xs = dg Wg[e]^T + du Wu[e]^T`` per segment, ``[rows, D]``."""
    _f32_operands("grouped_dgrad_gate_up_f32", dgu, w_gate, w_up)
    _check(offsets, "offsets", 1)
    R, F2 = dgu.shape
    N, D, F = w_gate.shape
    if F2 != 2 * F or tuple(w_up.shape) != (N, D, F) or offsets.numel() != N + 1:
        raise ValueError("grouped_dgrad_gate_up_f32: inconsistent shapes")
    d_xs = torch.empty((R, D), dtype=torch.float32, device=dgu.device)
    call("hmoe_grouped_dgrad_gate_up_f32", _ptr(dgu), _ptr(offsets), N, R, D, F, _ptr(w_gate),
         _ptr(w_up), _ptr(d_xs), _stream())
    return d_xs


def grouped_wgrad_gate_up_f32(xs: torch.Tensor, dgu: torch.Tensor, offsets: torch.Tensor):
    """Float32 ``(dWg, dWu)`` ``[N, D, F]`` = ``xs^T dg``, ``xs^T du`` per segment."""
    _f32_operands("grouped_wgrad_gate_up_f32", xs, dgu)
    _check(offsets, "offsets", 1)
    R, D = xs.shape
    F = dgu.shape[1] // 2
    if dgu.shape[0] != R or dgu.shape[1] != 2 * F:
        raise ValueError("grouped_wgrad_gate_up_f32: inconsistent shapes")
    N = offsets.numel() - 1
    dwg = torch.empty((N, D, F), dtype=torch.float32, device=xs.device)
    dwu = torch.empty((N, D, F), dtype=torch.float32, device=xs.device)
    call("hmoe_grouped_wgrad_gate_up_f32", _ptr(xs), _ptr(dgu), _ptr(offsets), N, D, F, _ptr(dwg),
         _ptr(dwu), _stream())
    return dwg, dwu


def grouped_wgrad_down_f32(h: torch.Tensor, d_ys: torch.Tensor, offsets: torch.Tensor) -> torch.Tensor:
    """Float32 ``dWd[e] = h^T d_ys`` per segment, ``[N, F, D]``."""
    _f32_operands("grouped_wgrad_down_f32", h, d_ys)
    _check(offsets, "offsets", 1)
    R, F = h.shape
    D = d_ys.shape[1]
    if d_ys.shape[0] != R:
        raise ValueError("grouped_wgrad_down_f32: h and d_ys must have the same rows")
    N = offsets.numel() - 1
    dwd = torch.empty((N, F, D), dtype=torch.float32, device=h.device)
    call("hmoe_grouped_wgrad_down_f32", _ptr(h), _ptr(d_ys), _ptr(offsets), N, F, D, _ptr(dwd),
         _stream())
    return dwd


def grouped_down_f32(h: torch.Tensor, offsets: torch.Tensor, w_down: torch.Tensor) -> torch.Tensor:
    """Float32 ``ys = h Wd[e]`` per expert segment (``moe.py:73``), master
    ``[N, F, D]`` as it is."""
    for t, n in ((h, "h"), (offsets, "offsets"), (w_down, "w_down")):
        _check(t, n)
    if h.dtype != torch.float32 or w_down.dtype != torch.float32:
        raise TypeError("grouped_down_f32 takes float32 operands")
    R, F = h.shape
    N, F2, D = w_down.shape
    if F2 != F or offsets.numel() != N + 1:
        raise ValueError("grouped_down_f32: inconsistent shapes")
    ys = torch.empty((R, D), dtype=torch.float32, device=h.device)
    call("hmoe_grouped_down_f32", _ptr(h), _ptr(offsets), N, R, F, D, _ptr(w_down), _ptr(ys),
         _stream())
    return ys


def grouped_gate_up_fp8(xs_q: torch.Tensor, xs_scale: torch.Tensor, offsets: torch.Tensor,
                        w_packed: torch.Tensor, w_scales: torch.Tensor) -> torch.Tensor:
    """bf16 ``h`` of the fp8 gate/up GEMM (dequantised, SwiGLU applied)."""
    for t, n in ((xs_q, "xs_q"), (xs_scale, "xs_scale"), (offsets, "offsets"),
                 (w_packed, "w_packed"), (w_scales, "w_scales")):
        _check(t, n)
    N, F2, D = w_packed.shape
    if (xs_q.dtype != torch.uint8 or w_packed.dtype != torch.uint8 or xs_q.shape[1] != D
            or xs_scale.numel() != xs_q.shape[0] or tuple(w_scales.shape) != (N, F2)
            or offsets.numel() != N + 1 or offsets.dtype != torch.int32):
        raise ValueError("grouped_gate_up_fp8: inconsistent shapes or dtypes")
    h = torch.empty((xs_q.shape[0], F2 // 2), dtype=torch.bfloat16, device=xs_q.device)
    call("hmoe_grouped_gate_up_fp8", _ptr(xs_q), _ptr(xs_scale), _ptr(offsets), N, xs_q.shape[0],
         D, F2 // 2, _ptr(w_packed), _ptr(w_scales), _ptr(h), _stream())
    return h


def grouped_gate_up_fp8_gather(x_q: torch.Tensor, x_scale: torch.Tensor, plan: Plan,
                               w_packed: torch.Tensor, w_scales: torch.Tensor) -> torch.Tensor:
    """``h`` of :func:`grouped_gate_up_fp8` with the row permutation done by the
    GEMM's loads: ``x_q, x_scale`` are the per-token codes and scales of ``x``
    (:func:`quantize_rows_fp8` of ``x``) and row ``r`` of the dispatched operand
    is token ``perm_src[r] // K`` (bit-identical to the permuted path)."""
    for t, n in ((x_q, "x_q"), (x_scale, "x_scale"), (w_packed, "w_packed"),
                 (w_scales, "w_scales")):
        _check(t, n)
    N, F2, D = w_packed.shape
    T = x_q.shape[0]
    if (x_q.dtype != torch.uint8 or w_packed.dtype != torch.uint8 or x_q.shape[1] != D
            or x_scale.numel() != T or tuple(w_scales.shape) != (N, F2)
            or plan.n_experts != N or plan.slot_pos.numel() != T * plan.top_k):
        raise ValueError("grouped_gate_up_fp8_gather: inconsistent shapes or dtypes")
    h = torch.empty((plan.rows_cap, F2 // 2), dtype=torch.bfloat16, device=x_q.device)
    call("hmoe_grouped_gate_up_fp8_gather", _ptr(x_q), _ptr(x_scale), T, plan.top_k,
         _ptr(plan.perm_src), _ptr(plan.offsets), N, plan.rows_cap, D, F2 // 2, _ptr(w_packed),
         _ptr(w_scales), _ptr(h), _stream())
    return h


def grouped_down_fp8(h_q: torch.Tensor, h_scale: torch.Tensor, offsets: torch.Tensor,
                     w_packed: torch.Tensor, w_scales: torch.Tensor) -> torch.Tensor:
    """bf16 ``ys`` of the fp8 down GEMM (dequantised)."""
    for t, n in ((h_q, "h_q"), (h_scale, "h_scale"), (offsets, "offsets"),
                 (w_packed, "w_packed"), (w_scales, "w_scales")):
        _check(t, n)
    N, D, F = w_packed.shape
    if (h_q.dtype != torch.uint8 or w_packed.dtype != torch.uint8 or h_q.shape[1] != F
            or h_scale.numel() != h_q.shape[0] or tuple(w_scales.shape) != (N, D)
            or offsets.numel() != N + 1 or offsets.dtype != torch.int32):
        raise ValueError("grouped_down_fp8: inconsistent shapes or dtypes")
    ys = torch.empty((h_q.shape[0], D), dtype=torch.bfloat16, device=h_q.device)
    call("hmoe_grouped_down_fp8", _ptr(h_q), _ptr(h_scale), _ptr(offsets), N, h_q.shape[0], F, D,
         _ptr(w_packed), _ptr(w_scales), _ptr(ys), _stream())
    return ys


def grouped_gate_up_fp8_qh(xs_q: torch.Tensor, xs_scale: torch.Tensor, offsets: torch.Tensor,
                           w_packed: torch.Tensor, w_scales: torch.Tensor):
    """Block-scaled e4m3 ``h`` of the fp8 gate/up GEMM, quantised in its
    epilogue: codes ``[rows, F]`` (uint8) and biased exponents ``[rows, F/32]``
    (uint8, ``e + 127``; every 32 columns of a row share ``2**e``)."""
    for t, n in ((xs_q, "xs_q"), (xs_scale, "xs_scale"), (offsets, "offsets"),
                 (w_packed, "w_packed"), (w_scales, "w_scales")):
        _check(t, n)
    N, F2, D = w_packed.shape
    if (xs_q.dtype != torch.uint8 or w_packed.dtype != torch.uint8 or xs_q.shape[1] != D
            or xs_scale.numel() != xs_q.shape[0] or tuple(w_scales.shape) != (N, F2)
            or offsets.numel() != N + 1 or offsets.dtype != torch.int32):
        raise ValueError("grouped_gate_up_fp8_qh: inconsistent shapes or dtypes")
    R, F = xs_q.shape[0], F2 // 2
    h_q = torch.empty((R, F), dtype=torch.uint8, device=xs_q.device)
    h_exp = torch.empty((R, F // 32), dtype=torch.uint8, device=xs_q.device)
    call("hmoe_grouped_gate_up_fp8_qh", _ptr(xs_q), _ptr(xs_scale), _ptr(offsets), N, R, D, F,
         _ptr(w_packed), _ptr(w_scales), _ptr(h_q), _ptr(h_exp), _stream())
    return h_q, h_exp


def grouped_gate_up_fp8_gather_qh(x_q: torch.Tensor, x_scale: torch.Tensor, plan: Plan,
                                  w_packed: torch.Tensor, w_scales: torch.Tensor):
    """:func:`grouped_gate_up_fp8_qh` gathering its rows from the per-token
    codes of ``x`` through ``perm_src`` (as :func:`grouped_gate_up_fp8_gather`)."""
    for t, n in ((x_q, "x_q"), (x_scale, "x_scale"), (w_packed, "w_packed"),
                 (w_scales, "w_scales")):
        _check(t, n)
    N, F2, D = w_packed.shape
    T = x_q.shape[0]
    if (x_q.dtype != torch.uint8 or w_packed.dtype != torch.uint8 or x_q.shape[1] != D
            or x_scale.numel() != T or tuple(w_scales.shape) != (N, F2)
            or plan.n_experts != N or plan.slot_pos.numel() != T * plan.top_k):
        raise ValueError("grouped_gate_up_fp8_gather_qh: inconsistent shapes or dtypes")
    F = F2 // 2
    h_q = torch.empty((plan.rows_cap, F), dtype=torch.uint8, device=x_q.device)
    h_exp = torch.empty((plan.rows_cap, F // 32), dtype=torch.uint8, device=x_q.device)
    call("hmoe_grouped_gate_up_fp8_gather_qh", _ptr(x_q), _ptr(x_scale), T, plan.top_k,
         _ptr(plan.perm_src), _ptr(plan.offsets), N, plan.rows_cap, D, F, _ptr(w_packed),
         _ptr(w_scales), _ptr(h_q), _ptr(h_exp), _stream())
    return h_q, h_exp


def grouped_down_fp8_mx(h_q: torch.Tensor, h_exp: torch.Tensor, offsets: torch.Tensor,
                        w_packed: torch.Tensor, w_scales: torch.Tensor) -> torch.Tensor:
    """bf16 ``ys`` of the fp8 down GEMM on block-scaled ``h`` (the MFMA applies
    ``h_exp``; the accumulators are dequantised by the column scales)."""
    for t, n in ((h_q, "h_q"), (h_exp, "h_exp"), (offsets, "offsets"), (w_packed, "w_packed"),
                 (w_scales, "w_scales")):
        _check(t, n)
    N, D, F = w_packed.shape
    if (h_q.dtype != torch.uint8 or h_exp.dtype != torch.uint8 or w_packed.dtype != torch.uint8
            or h_q.shape[1] != F or tuple(h_exp.shape) != (h_q.shape[0], F // 32)
            or tuple(w_scales.shape) != (N, D) or offsets.numel() != N + 1
            or offsets.dtype != torch.int32):
        raise ValueError("grouped_down_fp8_mx: inconsistent shapes or dtypes")
    ys = torch.empty((h_q.shape[0], D), dtype=torch.bfloat16, device=h_q.device)
    call("hmoe_grouped_down_fp8_mx", _ptr(h_q), _ptr(h_exp), _ptr(offsets), N, h_q.shape[0], F, D,
         _ptr(w_packed), _ptr(w_scales), _ptr(ys), _stream())
    return ys


# ---------------------------------------------------------------- combine --

def combine(ys: torch.Tensor, plan: Plan, gates: torch.Tensor,
            residual: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float32):
    """``y[t] = sum_k bf16(g[t,k]) ys[slot_pos[t,k]] (+ residual)`` (``moe.py:80-85``)."""
    _check(ys, "ys", 2)
    _check(gates, "gates", 2)
    T, K = gates.shape
    if gates.dtype != torch.float32 or K != plan.top_k or plan.slot_pos.numel() != T * K:
        raise ValueError("combine: gates must be float32 [T, K] matching the plan")
    D = ys.shape[1]
    if residual is not None:
        _check(residual, "residual", 2)
        if tuple(residual.shape) != (T, D):
            raise ValueError("combine: residual must be [T, D]")
    out = torch.empty((T, D), dtype=out_dtype, device=ys.device)
    call("hmoe_combine", _ptr(ys), _dtype_code(ys), _ptr(plan.slot_pos), _ptr(gates),
         _ptr(residual), _DT[residual.dtype] if residual is not None else _lib.F32, T, K, D,
         _ptr(out), _DT[out_dtype], _stream())
    return out


# -------------------------------------------------------------------- aux --

def router_aux(logits: torch.Tensor, top_idx: torch.Tensor, batch: int, seq: int):
    """Aux outputs (``moe.py:253-292``): (losses f32 [3] = z, balance, entropy;
    expert_counts f32 [N])."""
    _check(logits, "logits", 2)
    _check(top_idx, "top_idx", 2)
    T, N = logits.shape
    if T != batch * seq or top_idx.shape[0] != T:
        raise ValueError("router_aux: logits/top_idx must hold batch*seq tokens")
    dev = logits.device
    ws = int(_lib.lib().hmoe_aux_workspace_bytes(batch, seq, N))
    work = torch.empty(max(ws, 1), dtype=torch.uint8, device=dev)
    losses = torch.empty(3, dtype=torch.float32, device=dev)
    counts = torch.empty(N, dtype=torch.float32, device=dev)
    call("hmoe_router_aux", _ptr(logits), _ptr(top_idx), batch, seq, N, top_idx.shape[1],
         _ptr(losses), _ptr(counts), _ptr(work), work.numel(), _stream())
    return losses, counts


# ---------------------------------------------------------------- backward --
# Data gradients of the layer (the VJP of moe.py:170-246 with the routing held
# fixed); see hanuman_amd.backward for the composed pass.

def combine_bwd(dy: torch.Tensor, ys: torch.Tensor, plan: Plan, gates: torch.Tensor,
                n_shared: int = 0):
    """VJP of :func:`combine`: ``(d_ys bf16 [rows, D], d_gates f32 [T, K],
    d_shared)``; rows of ``d_ys`` no kept slot maps to are left as allocated.
    ``d_shared`` is ``bf16(dy / n_shared)`` ``[T, D]`` (the cotangent of each
    shared expert's output, ``moe.py:249-251``) when ``n_shared > 0``, else
    None."""
    _check(dy, "dy", 2)
    _check(ys, "ys", 2)
    _check(gates, "gates", 2)
    T, D = dy.shape
    K = plan.top_k
    if (dy.dtype != torch.float32 or ys.dtype != torch.bfloat16 or ys.shape[1] != D
            or tuple(gates.shape) != (T, K) or gates.dtype != torch.float32
            or plan.slot_pos.numel() != T * K):
        raise ValueError("combine_bwd: inconsistent shapes or dtypes")
    d_ys = torch.empty_like(ys)
    d_g = torch.empty((T, K), dtype=torch.float32, device=dy.device)
    d_sh = torch.empty((T, D), dtype=torch.bfloat16, device=dy.device) if n_shared > 0 else None
    call("hmoe_combine_bwd", _ptr(dy), _ptr(ys), _ptr(plan.slot_pos), _ptr(gates), T, K, D,
         _ptr(d_ys), _ptr(d_g), _ptr(d_sh), float(max(n_shared, 1)), _stream())
    return d_ys, d_g, d_sh


def grouped_gate_up_raw_gather(x: torch.Tensor, plan: Plan, w_gate_up: torch.Tensor) -> torch.Tensor:
    """g and u (``moe.py:70-71``) of the dispatched rows of ``x``, bf16
    ``[rows_cap, 2F]`` in the packed gate/up column order."""
    _check(x, "x", 2)
    _check(w_gate_up, "w_gate_up", 3)
    if x.dtype != torch.bfloat16 or w_gate_up.dtype != torch.bfloat16:
        raise TypeError("grouped_gate_up_raw_gather takes bf16 operands")
    T, D = x.shape
    N, F2, D2 = w_gate_up.shape
    if D2 != D or plan.n_experts != N or plan.slot_pos.numel() != T * plan.top_k:
        raise ValueError("grouped_gate_up_raw_gather: inconsistent shapes")
    gu = torch.empty((plan.rows_cap, F2), dtype=torch.bfloat16, device=x.device)
    call("hmoe_grouped_gate_up_raw_gather", _ptr(x), T, plan.top_k, _ptr(plan.perm_src),
         _ptr(plan.offsets), N, plan.rows_cap, D, F2 // 2, _ptr(w_gate_up), _ptr(gu), _stream())
    return gu


def grouped_gate_up_swiglu_bwd_gather(x: torch.Tensor, plan: Plan, w_gate_up: torch.Tensor,
                                      dh: torch.Tensor) -> torch.Tensor:
    """The g, u recompute (``moe.py:70-71``) with the SwiGLU VJP (``:72``) in
    its epilogue: ``dgu`` bf16 ``[rows_cap, 2F]`` in the gate/up column order
    from ``dh`` ``[rows_cap, F]``; g and u never reach HBM.  Bit-identical to
    :func:`grouped_gate_up_raw_gather` followed by :func:`swiglu_bwd`."""
    _check(x, "x", 2)
    _check(w_gate_up, "w_gate_up", 3)
    _check(dh, "dh", 2)
    if x.dtype != torch.bfloat16 or w_gate_up.dtype != torch.bfloat16 or dh.dtype != torch.bfloat16:
        raise TypeError("grouped_gate_up_swiglu_bwd_gather takes bf16 operands")
    T, D = x.shape
    N, F2, D2 = w_gate_up.shape
    if (D2 != D or plan.n_experts != N or plan.slot_pos.numel() != T * plan.top_k
            or tuple(dh.shape) != (plan.rows_cap, F2 // 2)):
        raise ValueError("grouped_gate_up_swiglu_bwd_gather: inconsistent shapes")
    dgu = torch.empty((plan.rows_cap, F2), dtype=torch.bfloat16, device=x.device)
    call("hmoe_grouped_gate_up_swiglu_bwd_gather", _ptr(x), T, plan.top_k, _ptr(plan.perm_src),
         _ptr(plan.offsets), N, plan.rows_cap, D, F2 // 2, _ptr(w_gate_up), _ptr(dh), _ptr(dgu),
         _stream())
    return dgu


def grouped_gate_up_swiglu_bwd(xs: torch.Tensor, offsets: torch.Tensor, w_gate_up: torch.Tensor,
                               dh: torch.Tensor) -> torch.Tensor:
    """:func:`grouped_gate_up_swiglu_bwd_gather` on rows given in order (the
    shared expert)."""
    _check(xs, "xs", 2)
    _check(offsets, "offsets", 1)
    _check(w_gate_up, "w_gate_up", 3)
    _check(dh, "dh", 2)
    if xs.dtype != torch.bfloat16 or w_gate_up.dtype != torch.bfloat16 or dh.dtype != torch.bfloat16:
        raise TypeError("grouped_gate_up_swiglu_bwd takes bf16 operands")
    R, D = xs.shape
    N, F2, D2 = w_gate_up.shape
    if D2 != D or offsets.numel() != N + 1 or tuple(dh.shape) != (R, F2 // 2):
        raise ValueError("grouped_gate_up_swiglu_bwd: inconsistent shapes")
    dgu = torch.empty((R, F2), dtype=torch.bfloat16, device=xs.device)
    call("hmoe_grouped_gate_up_swiglu_bwd", _ptr(xs), _ptr(offsets), N, R, D, F2 // 2,
         _ptr(w_gate_up), _ptr(dh), _ptr(dgu), _stream())
    return dgu


def grouped_gate_up_raw(xs: torch.Tensor, offsets: torch.Tensor, w_gate_up: torch.Tensor) -> torch.Tensor:
    """g and u of rows given in order (the shared expert, ``moe.py:23-29``),
    bf16 ``[rows, 2F]`` in the packed gate/up column order."""
    _check(xs, "xs", 2)
    _check(offsets, "offsets", 1)
    _check(w_gate_up, "w_gate_up", 3)
    if xs.dtype != torch.bfloat16 or w_gate_up.dtype != torch.bfloat16:
        raise TypeError("grouped_gate_up_raw takes bf16 operands")
    R, D = xs.shape
    N, F2, D2 = w_gate_up.shape
    if D2 != D or offsets.numel() != N + 1:
        raise ValueError("grouped_gate_up_raw: inconsistent shapes")
    gu = torch.empty((R, F2), dtype=torch.bfloat16, device=xs.device)
    call("hmoe_grouped_gate_up_raw", _ptr(xs), _ptr(offsets), N, R, D, F2 // 2, _ptr(w_gate_up),
         _ptr(gu), _stream())
    return gu


def swiglu_bwd(dh: torch.Tensor, gu: torch.Tensor, offsets: torch.Tensor | None) -> torch.Tensor:
    """VJP of ``h = silu(g) * u`` (``moe.py:72``): ``dgu`` bf16 ``[rows, 2F]`` in
    ``gu``'s column order; rows at or past ``offsets[-1]`` left as allocated."""
    _check(dh, "dh", 2)
    _check(gu, "gu", 2)
    rows, F = dh.shape
    if (dh.dtype != torch.bfloat16 or gu.dtype != torch.bfloat16
            or tuple(gu.shape) != (rows, 2 * F)):
        raise ValueError("swiglu_bwd: inconsistent shapes or dtypes")
    n = 1
    if offsets is not None:
        _check(offsets, "offsets", 1)
        n = offsets.numel() - 1
    dgu = torch.empty_like(gu)
    call("hmoe_swiglu_bwd", _ptr(dh), _ptr(gu), _ptr(offsets), n, rows, F, _ptr(dgu), _stream())
    return dgu


def pack_down_dgrad(w_down: torch.Tensor) -> torch.Tensor:
    """bf16 ``[N, F, D]`` operand of :func:`grouped_dgrad_down` from the ``[N,F,D]`` master."""
    _check(w_down, "w_down", 3)
    N, F, D = w_down.shape
    out = torch.empty((N, F, D), dtype=torch.bfloat16, device=w_down.device)
    call("hmoe_pack_down_dgrad", _ptr(w_down), _dtype_code(w_down), N, F, D, _ptr(out), _stream())
    return out


def pack_gate_up_dgrad(w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """bf16 ``[N, D, 2F]`` operand of :func:`grouped_dgrad_gate_up` from the
    ``[N,D,F]`` masters (columns in the packed gate/up order)."""
    _check(w_gate, "w_gate", 3)
    _check(w_up, "w_up", 3)
    if w_gate.shape != w_up.shape or w_gate.dtype != w_up.dtype:
        raise ValueError("w_gate and w_up must have the same shape and dtype")
    N, D, F = w_gate.shape
    out = torch.empty((N, D, 2 * F), dtype=torch.bfloat16, device=w_gate.device)
    call("hmoe_pack_gate_up_dgrad", _ptr(w_gate), _ptr(w_up), _dtype_code(w_gate), N, D, F,
         _ptr(out), _stream())
    return out


def grouped_dgrad_down(d_ys: torch.Tensor, offsets: torch.Tensor, w_down_dgrad: torch.Tensor) -> torch.Tensor:
    """``dh = bf16(d_ys Wd[e]^T)`` per expert segment (VJP of ``moe.py:73``)."""
    _check(d_ys, "d_ys", 2)
    _check(offsets, "offsets", 1)
    _check(w_down_dgrad, "w_down_dgrad", 3)
    N, F, D = w_down_dgrad.shape
    if (d_ys.dtype != torch.bfloat16 or w_down_dgrad.dtype != torch.bfloat16
            or d_ys.shape[1] != D or offsets.numel() != N + 1):
        raise ValueError("grouped_dgrad_down: inconsistent shapes or dtypes")
    R = d_ys.shape[0]
    dh = torch.empty((R, F), dtype=torch.bfloat16, device=d_ys.device)
    call("hmoe_grouped_dgrad_down", _ptr(d_ys), _ptr(offsets), N, R, D, F, _ptr(w_down_dgrad),
         _ptr(dh), _stream())
    return dh


def grouped_dgrad_gate_up(dgu: torch.Tensor, offsets: torch.Tensor, w_gate_up_dgrad: torch.Tensor) -> torch.Tensor:
    """``d_xs = bf16(dg Wg[e]^T + du Wu[e]^T)`` per expert segment (VJP of
    ``moe.py:70-71``)."""
    _check(dgu, "dgu", 2)
    _check(offsets, "offsets", 1)
    _check(w_gate_up_dgrad, "w_gate_up_dgrad", 3)
    N, D, F2 = w_gate_up_dgrad.shape
    if (dgu.dtype != torch.bfloat16 or w_gate_up_dgrad.dtype != torch.bfloat16
            or dgu.shape[1] != F2 or offsets.numel() != N + 1):
        raise ValueError("grouped_dgrad_gate_up: inconsistent shapes or dtypes")
    R = dgu.shape[0]
    d_xs = torch.empty((R, D), dtype=torch.bfloat16, device=dgu.device)
    call("hmoe_grouped_dgrad_gate_up", _ptr(dgu), _ptr(offsets), N, R, D, F2 // 2,
         _ptr(w_gate_up_dgrad), _ptr(d_xs), _stream())
    return d_xs


def gather_bwd(d_xs: torch.Tensor, plan: Plan, out_dtype: torch.dtype = torch.float32,
               residual: torch.Tensor | None = None) -> torch.Tensor:
    """VJP of the row gather (``moe.py:56``): ``dx[t] = sum_k d_xs[slot_pos[t,k]]``
    (+ ``residual[t]``, the shared expert's input gradient, added last)."""
    _check(d_xs, "d_xs", 2)
    T = plan.slot_pos.numel() // plan.top_k
    D = d_xs.shape[1]
    res_dt = _lib.F32
    if residual is not None:
        _check(residual, "residual", 2)
        if tuple(residual.shape) != (T, D):
            raise ValueError("gather_bwd: residual must be [T, D]")
        res_dt = _dtype_code(residual)
    dx = torch.empty((T, D), dtype=out_dtype, device=d_xs.device)
    call("hmoe_gather_bwd", _ptr(d_xs), _dtype_code(d_xs), _ptr(plan.slot_pos), _ptr(residual),
         res_dt, T, plan.top_k, D, _ptr(dx), _DT[out_dtype], _stream())
    return dx


def router_bwd(logits: torch.Tensor | None, top_idx: torch.Tensor, gates: torch.Tensor,
               d_gates: torch.Tensor, n_experts: int, mode: int = _lib.ROUTE_SOFTMAX,
               routed_scaling_factor: float = 1.0) -> torch.Tensor:
    """``d_logits`` f32 ``[T, N]`` from ``d_gates`` (VJP of ``moe.py:179-192``)."""
    _check(top_idx, "top_idx", 2)
    _check(d_gates, "d_gates", 2)
    T, K = top_idx.shape
    if logits is not None:
        _check(logits, "logits", 2)
    dl = torch.empty((T, n_experts), dtype=torch.float32, device=top_idx.device)
    call("hmoe_router_bwd", _ptr(logits), _ptr(top_idx), _ptr(gates), _ptr(d_gates), T,
         n_experts, K, mode, routed_scaling_factor, _ptr(dl), _stream())
    return dl


def router_aux_bwd(logits: torch.Tensor, top_idx: torch.Tensor, batch: int, seq: int,
                   d_losses: torch.Tensor, d_logits: torch.Tensor | None = None,
                   workspace: torch.Tensor | None = None) -> torch.Tensor:
    """VJP of the aux losses (``moe.py:253-283``) with respect to the logits
    for ``d_losses`` f32 ``[3]`` (cotangents of router_z_loss, balance_loss,
    mean_entropy): added into ``d_logits`` when given, else a new f32
    ``[T, N]``.  The per-sequence expert counts of ``top_idx`` are held fixed."""
    _check(logits, "logits", 2)
    _check(top_idx, "top_idx", 2)
    _check(d_losses, "d_losses", 1)
    T, N = logits.shape
    if T != batch * seq or top_idx.shape[0] != T or d_losses.numel() != 3 \
            or d_losses.dtype != torch.float32:
        raise ValueError("router_aux_bwd: logits/top_idx must hold batch*seq tokens, d_losses f32 [3]")
    acc = d_logits is not None
    if acc:
        _check(d_logits, "d_logits", 2)
        if tuple(d_logits.shape) != (T, N) or d_logits.dtype != torch.float32:
            raise ValueError("router_aux_bwd: d_logits must be f32 [T, N]")
    else:
        d_logits = torch.empty((T, N), dtype=torch.float32, device=logits.device)
    ws = int(_lib.lib().hmoe_aux_bwd_workspace_bytes(batch, seq, N))
    if workspace is None or workspace.numel() < ws:
        workspace = torch.empty(max(ws, 1), dtype=torch.uint8, device=logits.device)
    call("hmoe_router_aux_bwd", _ptr(logits), _ptr(top_idx), batch, seq, N, top_idx.shape[1],
         _ptr(d_losses), _ptr(d_logits), int(acc), _ptr(workspace), workspace.numel(), _stream())
    return d_logits


def router_dx(d_logits: torch.Tensor, router_w: torch.Tensor, dx: torch.Tensor | None = None) -> torch.Tensor:
    """``dx (+)= d_logits @ router_w^T`` (VJP of ``moe.py:178`` w.r.t. x), f32 ``[T, D]``."""
    _check(d_logits, "d_logits", 2)
    _check(router_w, "router_w", 2)
    T, N = d_logits.shape
    D = router_w.shape[0]
    acc = dx is not None
    if dx is None:
        dx = torch.empty((T, D), dtype=torch.float32, device=d_logits.device)
    elif dx.dtype != torch.float32 or tuple(dx.shape) != (T, D):
        raise ValueError("router_dx: dx must be float32 [T, D]")
    call("hmoe_router_dx", _ptr(d_logits), _ptr(router_w), _dtype_code(router_w), T, D, N,
         _ptr(dx), 1 if acc else 0, _stream())
    return dx


def grouped_wgrad_down(h: torch.Tensor, d_ys: torch.Tensor, offsets: torch.Tensor) -> torch.Tensor:
    """``dWd[e] = h^T d_ys`` over each expert's segment, f32 ``[N, F, D]``."""
    _check(h, "h", 2)
    _check(d_ys, "d_ys", 2)
    _check(offsets, "offsets", 1)
    R, F = h.shape
    D = d_ys.shape[1]
    if h.dtype != torch.bfloat16 or d_ys.dtype != torch.bfloat16 or d_ys.shape[0] != R:
        raise ValueError("grouped_wgrad_down: h and d_ys must be bf16 with the same rows")
    N = offsets.numel() - 1
    dw = torch.empty((N, F, D), dtype=torch.float32, device=h.device)
    call("hmoe_grouped_wgrad_down", _ptr(h), _ptr(d_ys), _ptr(offsets), N, R, F, D, _ptr(dw),
         _stream())
    return dw


def grouped_wgrad_gate_up(xs: torch.Tensor, dgu: torch.Tensor, offsets: torch.Tensor):
    """``(dWg, dWu)[e] = xs^T (dg, du)`` over each expert's segment, f32 ``[N, D, F]`` each."""
    _check(xs, "xs", 2)
    _check(dgu, "dgu", 2)
    _check(offsets, "offsets", 1)
    R, D = xs.shape
    F = dgu.shape[1] // 2
    if xs.dtype != torch.bfloat16 or dgu.dtype != torch.bfloat16 or dgu.shape[0] != R:
        raise ValueError("grouped_wgrad_gate_up: xs and dgu must be bf16 with the same rows")
    N = offsets.numel() - 1
    dwg = torch.empty((N, D, F), dtype=torch.float32, device=xs.device)
    dwu = torch.empty_like(dwg)
    call("hmoe_grouped_wgrad_gate_up", _ptr(xs), _ptr(dgu), _ptr(offsets), N, R, D, F, _ptr(dwg),
         _ptr(dwu), _stream())
    return dwg, dwu


def router_dw(x: torch.Tensor, d_logits: torch.Tensor, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """``d_router = x^T d_logits`` f32 ``[D, N]`` (VJP of ``moe.py:178`` w.r.t. the router)."""
    _check(x, "x", 2)
    _check(d_logits, "d_logits", 2)
    T, D = x.shape
    N = d_logits.shape[1]
    ws = int(_lib.lib().hmoe_router_dw_workspace_bytes(T, D, N))
    if workspace is None or workspace.numel() < ws:
        workspace = torch.empty(max(ws, 1), dtype=torch.uint8, device=x.device)
    out = torch.empty((D, N), dtype=torch.float32, device=x.device)
    call("hmoe_router_dw", _ptr(x), _dtype_code(x), _ptr(d_logits), T, D, N, _ptr(out),
         _ptr(workspace), workspace.numel(), _stream())
    return out
