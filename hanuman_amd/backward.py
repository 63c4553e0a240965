"""Backward of the MoE layer on the HIP library.

``jax.value_and_grad`` (``train.py:266``) differentiates ``MoE.__call__``
(``model/moe.py:170-294``) inside the loss of ``train.py:191-200`` (output
plus ``z_loss_weight * router_z_loss + balance_loss_weight * balance_loss``);
this is that VJP, with the routing decisions (top-k indices, capacity drops,
the dispatch plan, the expert counts) held fixed, as JAX does for
integer-valued operations:

    combine  (moe.py:80-85)   d_ys, d_gates      hmoe_combine_bwd
    experts  (moe.py:70-73)   g, u recomputed    hmoe_grouped_gate_up_raw_gather
                              dh = d_ys Wd^T     hmoe_grouped_dgrad_down
                              dg, du             hmoe_swiglu_bwd
                              d_xs               hmoe_grouped_dgrad_gate_up
    gather   (moe.py:56)      dx_experts         hmoe_gather_bwd
    gates    (moe.py:179-192) d_logits           hmoe_router_bwd
    router   (moe.py:178)     dx += d_l W^T      hmoe_router_dx

and the weight gradients (:func:`moe_backward_weights`):

    experts  (moe.py:70-73)   dWd = h^T d_ys,    hmoe_grouped_wgrad_down
                              dWg|dWu = xs^T dg|du  hmoe_grouped_wgrad_gate_up
    router   (moe.py:178)     d_router = x^T d_l hmoe_router_dw

(:func:`moe_backward_data` keeps these steps apart and returns their
intermediates; :func:`moe_backward` runs the recompute and the SwiGLU VJP as
one GEMM, ``hmoe_grouped_gate_up_swiglu_bwd_gather``, so that g and u never
reach HBM) and, in :func:`moe_backward` (the whole module), the shared expert
(``moe.py:161-168, 249-251``: the same grouped kernels with one segment of
all tokens, its output cotangent ``bf16(dy / n_shared)`` from
``hmoe_combine_bwd``) and the aux losses (``moe.py:253-283``,
``hmoe_router_aux_bwd`` into ``d_logits``).

For the float32 compute dtype, :func:`moe_backward_f32` is the same VJP on
the float32 kernels (``hmoe_combine_bwd_f32``, ``hmoe_grouped_*_f32``) with
the masters as they are and no rounding points.

Every step runs in the library on the current stream; there is no CPU
fallback.
"""
from __future__ import annotations

import torch

from . import _lib
from . import kernels as K


class BackwardOperands:
    """The backward's packed expert weights, built once from the masters."""

    def __init__(self, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor):
        self.w_gate_up_dgrad = K.pack_gate_up_dgrad(w_gate, w_up)
        self.w_down_dgrad = K.pack_down_dgrad(w_down)


class SharedOperands:
    """Packed operands of the shared expert(s) (``moe.py:152-159``): 2-D
    masters for one shared expert, stacked ``[n, ...]`` for several.  Per
    expert: the forward gate/up pack (for the g, u recompute) and the two
    backward packs."""

    def __init__(self, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor,
                 n_shared: int, forward_packs=None):
        if n_shared < 1:
            raise ValueError("the shared-expert backward needs n_shared >= 1")
        self.n_shared = n_shared
        if n_shared == 1:
            w_gate, w_up, w_down = (w.unsqueeze(0) for w in (w_gate, w_up, w_down))
        self.experts = []
        for i in range(n_shared):
            wg, wu, wd = (w[i:i + 1].contiguous() for w in (w_gate, w_up, w_down))
            fwd_gu = forward_packs[i][0] if forward_packs is not None else K.pack_gate_up(wg, wu)
            self.experts.append((fwd_gu, K.pack_gate_up_dgrad(wg, wu), K.pack_down_dgrad(wd)))


def moe_backward_data(x: torch.Tensor, router_w: torch.Tensor, fwd: dict,
                      w_gate_up: torch.Tensor, ops: BackwardOperands, dy: torch.Tensor,
                      mode: int = _lib.ROUTE_SOFTMAX,
                      routed_scaling_factor: float = 1.0) -> dict:
    """Data gradients of the routed layer for the cotangent ``dy`` (f32
    ``[T, D]``) of its output.

    ``x`` bf16 ``[T, D]``; ``fwd`` the forward's ``logits``, ``top_idx``,
    ``gates``, ``plan`` and ``ys``; ``w_gate_up`` the forward's packed gate/up
    operand.  Returns ``dx`` (f32 ``[T, D]``, experts plus router),
    ``d_gates``, ``d_logits`` and the intermediates ``d_ys``, ``gu``, ``dh``,
    ``dgu``, ``d_xs``.
    """
    plan = fwd["plan"]
    N = plan.n_experts
    d_ys, d_gates, _ = K.combine_bwd(dy, fwd["ys"], plan, fwd["gates"])
    gu = K.grouped_gate_up_raw_gather(x, plan, w_gate_up)
    dh = K.grouped_dgrad_down(d_ys, plan.offsets, ops.w_down_dgrad)
    dgu = K.swiglu_bwd(dh, gu, plan.offsets)
    d_xs = K.grouped_dgrad_gate_up(dgu, plan.offsets, ops.w_gate_up_dgrad)
    dx = K.gather_bwd(d_xs, plan)
    d_logits = K.router_bwd(fwd["logits"], fwd["top_idx"], fwd["gates"], d_gates, N, mode,
                            routed_scaling_factor)
    K.router_dx(d_logits, router_w, dx)
    return {"dx": dx, "d_gates": d_gates, "d_logits": d_logits, "d_ys": d_ys, "gu": gu,
            "dh": dh, "dgu": dgu, "d_xs": d_xs}


def moe_backward_weights(x: torch.Tensor, fwd: dict, data: dict) -> dict:
    """Weight gradients of the routed layer from the forward's ``plan`` and
    ``h`` and :func:`moe_backward_data`'s result: ``dWg``, ``dWu`` f32
    ``[N, D, F]``, ``dWd`` f32 ``[N, F, D]``, ``d_router`` f32 ``[D, N]``
    (the dispatched rows ``xs`` are gathered once for the gate/up gradient)."""
    plan = fwd["plan"]
    xs = K.permute_rows(x, plan, torch.bfloat16)
    dwg, dwu = K.grouped_wgrad_gate_up(xs, data["dgu"], plan.offsets)
    dwd = K.grouped_wgrad_down(fwd["h"], data["d_ys"], plan.offsets)
    d_router = K.router_dw(x, data["d_logits"])
    return {"dWg": dwg, "dWu": dwu, "dWd": dwd, "d_router": d_router}


def shared_backward(xc: torch.Tensor, d_shared: torch.Tensor, h_shared, ops: SharedOperands,
                    weights: bool = True) -> dict:
    """VJP of the shared expert(s) for the output cotangent ``d_shared``
    (``bf16(dy / n_shared)`` from :func:`kernels.combine_bwd`): each SwiGLU
    (``moe.py:23-29``) is one segment of all ``T`` rows on the grouped
    kernels.  ``xc`` bf16 ``[T, D]``; ``h_shared`` the forward's ``h`` per
    shared expert.  Returns ``dx`` (bf16 ``[T, D]`` for one shared expert,
    float32 sum for several) and ``dWg``, ``dWu``, ``dWd`` in the parameter
    shapes."""
    T = xc.shape[0]
    off = torch.tensor([0, T], dtype=torch.int32, device=xc.device)
    dxs, dwg, dwu, dwd = [], [], [], []
    for (fwd_gu, gu_dgrad, down_dgrad), h in zip(ops.experts, h_shared):
        dh = K.grouped_dgrad_down(d_shared, off, down_dgrad)
        dgu = K.grouped_gate_up_swiglu_bwd(xc, off, fwd_gu, dh)
        dxs.append(K.grouped_dgrad_gate_up(dgu, off, gu_dgrad))
        if weights:
            g_, u_ = K.grouped_wgrad_gate_up(xc, dgu, off)
            dwg.append(g_)
            dwu.append(u_)
            dwd.append(K.grouped_wgrad_down(h, d_shared, off))
    if not weights:
        dx = dxs[0] if ops.n_shared == 1 else sum(d.float() for d in dxs)
        return {"dx": dx, "dWg": None, "dWu": None, "dWd": None}
    if ops.n_shared == 1:
        return {"dx": dxs[0], "dWg": dwg[0][0], "dWu": dwu[0][0], "dWd": dwd[0][0]}
    # several shared experts: their input gradients add in float32
    dx = dxs[0].float()
    for d in dxs[1:]:
        dx += d.float()
    return {"dx": dx, "dWg": torch.cat(dwg), "dWu": torch.cat(dwu), "dWd": torch.cat(dwd)}


def moe_backward(x: torch.Tensor, router_w: torch.Tensor | None, fwd: dict,
                 w_gate_up: torch.Tensor, ops: BackwardOperands, dy: torch.Tensor, *,
                 mode: int = _lib.ROUTE_SOFTMAX, routed_scaling_factor: float = 1.0,
                 shared: SharedOperands | None = None, h_shared=None,
                 aux: tuple | None = None, need: dict | None = None,
                 shared_promoted: tuple | None = None) -> dict:
    """The whole module's VJP (``moe.py:170-294``): every input and weight
    gradient for the cotangent ``dy`` (f32 ``[T, D]``) of ``out`` and, with
    ``aux = (batch, seq, d_losses)``, the cotangents ``d_losses`` (f32 ``[3]``:
    router_z_loss, balance_loss, mean_entropy) of the aux losses.

    ``x`` ``[T, D]`` (bf16 or f32); ``fwd`` the forward's ``logits``,
    ``top_idx``, ``gates``, ``plan``, ``h``, ``ys``; ``shared``/``h_shared``
    the shared expert's operands and forward ``h`` (None: no shared expert).
    Returns ``dx`` f32 ``[T, D]``, ``d_router`` f32 ``[D, N]`` (None without a
    router weight), ``dWg``, ``dWu`` ``[N, D, F]``, ``dWd`` ``[N, F, D]`` and
    ``dWg_shared``, ``dWu_shared``, ``dWd_shared`` when there is a shared
    expert.  ``need`` (``{"router", "experts", "shared"}`` -> bool, default
    all) skips the weight gradients not asked for; those entries are None.
    ``shared_promoted = (w_gate, w_up, w_down, n_shared)`` (bf16-rounded
    masters as float32) in place of ``shared``: float32 ``x``, whose shared
    expert ran promoted to float32 (``moe.py:249``); its VJP runs on the
    float32 kernels and the master gradients pass through bf16 (the VJP of
    ``w.astype(bf16)``).
    """
    need = {"router": True, "experts": True, "shared": True, **(need or {})}
    plan = fwd["plan"]
    N = plan.n_experts
    xc = x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16)   # x.astype(dtype), moe.py:198
    n_sh = shared.n_shared if shared is not None else 0
    d_ys, d_gates, d_sh = K.combine_bwd(dy, fwd["ys"], plan, fwd["gates"], n_sh)
    if shared_promoted is not None and shared is not None:
        raise ValueError("moe_backward: shared and shared_promoted are exclusive")
    dh = K.grouped_dgrad_down(d_ys, plan.offsets, ops.w_down_dgrad)
    dgu = K.grouped_gate_up_swiglu_bwd_gather(xc, plan, w_gate_up, dh)
    del dh
    d_xs = K.grouped_dgrad_gate_up(dgu, plan.offsets, ops.w_gate_up_dgrad)
    res = {}
    residual = None
    if shared is not None:
        sh = shared_backward(xc, d_sh, h_shared, shared, weights=need["shared"])
        residual = sh["dx"]
        res.update(dWg_shared=sh["dWg"], dWu_shared=sh["dWu"], dWd_shared=sh["dWd"])
    elif shared_promoted is not None:
        n_p = shared_promoted[3]
        # each float32 SwiGLU's output cotangent is dy / n_shared (no bf16 cast)
        d_sh32 = dy if n_p == 1 else dy / n_p
        sh = _shared_backward_f32(x.float().contiguous(), d_sh32, h_shared, shared_promoted)
        residual = sh["dx"]
        if need["shared"]:
            dws = [sh[k].to(torch.bfloat16).float() for k in ("dWg", "dWu", "dWd")]
            if n_p == 1:
                dws = [w[0] for w in dws]
            res.update(dWg_shared=dws[0], dWu_shared=dws[1], dWd_shared=dws[2])
        else:
            res.update(dWg_shared=None, dWu_shared=None, dWd_shared=None)
    dx = K.gather_bwd(d_xs, plan, residual=residual)
    del d_xs, residual
    d_logits = K.router_bwd(fwd["logits"], fwd["top_idx"], fwd["gates"], d_gates, N, mode,
                            routed_scaling_factor)
    if aux is not None:
        batch, seq, d_losses = aux
        K.router_aux_bwd(fwd["logits"], fwd["top_idx"], batch, seq, d_losses, d_logits)
    if router_w is not None:
        K.router_dx(d_logits, router_w, dx)
    dwg = dwu = dwd = None
    if need["experts"]:
        xs = K.permute_rows(x, plan, torch.bfloat16)
        dwg, dwu = K.grouped_wgrad_gate_up(xs, dgu, plan.offsets)
        del xs
        dwd = K.grouped_wgrad_down(fwd["h"], d_ys, plan.offsets)
    del dgu
    d_router = K.router_dw(x, d_logits) if router_w is not None and need["router"] else None
    res.update(dx=dx, d_router=d_router, dWg=dwg, dWu=dwu, dWd=dwd, d_logits=d_logits,
               d_gates=d_gates)
    return res


def _shared_backward_f32(x32: torch.Tensor, d_shared: torch.Tensor, h_shared, masters) -> dict:
    """Float32 VJP of the shared expert(s): ``masters = (w_gate, w_up, w_down,
    n_shared)`` (2-D for one shared expert, stacked for several), ``d_shared =
    dy / n_shared``, ``h_shared`` the forward's ``h`` per shared expert."""
    w_gate, w_up, w_down, n_shared = masters
    if n_shared == 1:
        w_gate, w_up, w_down = (w.unsqueeze(0) for w in (w_gate, w_up, w_down))
    T = x32.shape[0]
    off = torch.tensor([0, T], dtype=torch.int32, device=x32.device)
    dx, dwg, dwu, dwd = None, [], [], []
    for i, h in enumerate(h_shared):
        wg, wu, wd = (w[i:i + 1].contiguous() for w in (w_gate, w_up, w_down))
        dh = K.grouped_dgrad_down_f32(d_shared, off, wd)
        dgu = K.grouped_gate_up_swiglu_bwd_f32(x32, off, wg, wu, dh)
        d = K.grouped_dgrad_gate_up_f32(dgu, off, wg, wu)
        dx = d if dx is None else dx.add_(d)
        g_, u_ = K.grouped_wgrad_gate_up_f32(x32, dgu, off)
        dwg.append(g_)
        dwu.append(u_)
        dwd.append(K.grouped_wgrad_down_f32(h, d_shared, off))
    return {"dx": dx, "dWg": torch.cat(dwg), "dWu": torch.cat(dwu), "dWd": torch.cat(dwd)}


def moe_backward_f32(x: torch.Tensor, router_w: torch.Tensor | None, fwd: dict, masters, dy,
                     *, mode: int = _lib.ROUTE_SOFTMAX, routed_scaling_factor: float = 1.0,
                     shared=None, h_shared=None, aux: tuple | None = None,
                     need: dict | None = None) -> dict:
    """:func:`moe_backward` for the float32 compute dtype: ``masters =
    (w_gate, w_up, w_down)`` float32 as they are, ``fwd`` adds the forward's
    dispatched rows ``xs`` (float32), ``shared = (w_gate, w_up, w_down,
    n_shared)`` or None.  Same results dict and ``need``."""
    need = {"router": True, "experts": True, "shared": True, **(need or {})}
    plan = fwd["plan"]
    N = plan.n_experts
    wg, wu, wd = masters
    n_sh = shared[3] if shared is not None else 0
    d_ys, d_gates, d_sh = K.combine_bwd_f32(dy, fwd["ys"], plan, fwd["gates"], n_sh)
    xs = fwd["xs"]
    dh = K.grouped_dgrad_down_f32(d_ys, plan.offsets, wd)
    dgu = K.grouped_gate_up_swiglu_bwd_f32(xs, plan.offsets, wg, wu, dh)
    del dh
    d_xs = K.grouped_dgrad_gate_up_f32(dgu, plan.offsets, wg, wu)
    res = {}
    residual = None
    if shared is not None:
        x32 = x if x.dtype == torch.float32 else x.float()   # x.astype(dtype), moe.py:198
        sh = _shared_backward_f32(x32.contiguous(), d_sh, h_shared, shared)
        residual = sh["dx"]
        dws = [sh[k] for k in ("dWg", "dWu", "dWd")]
        if n_sh == 1:
            dws = [w[0] for w in dws]
        res.update(dWg_shared=dws[0], dWu_shared=dws[1], dWd_shared=dws[2])
    dx = K.gather_bwd(d_xs, plan, residual=residual)
    del d_xs, residual
    d_logits = K.router_bwd(fwd["logits"], fwd["top_idx"], fwd["gates"], d_gates, N, mode,
                            routed_scaling_factor)
    if aux is not None:
        batch, seq, d_losses = aux
        K.router_aux_bwd(fwd["logits"], fwd["top_idx"], batch, seq, d_losses, d_logits)
    if router_w is not None:
        K.router_dx(d_logits, router_w, dx)
    dwg = dwu = dwd = None
    if need["experts"]:
        dwg, dwu = K.grouped_wgrad_gate_up_f32(xs, dgu, plan.offsets)
        dwd = K.grouped_wgrad_down_f32(fwd["h"], d_ys, plan.offsets)
    del dgu
    d_router = K.router_dw(x, d_logits) if router_w is not None and need["router"] else None
    res.update(dx=dx, d_router=d_router, dWg=dwg, dWu=dwu, dWd=dwd, d_logits=d_logits,
               d_gates=d_gates)
    return res
