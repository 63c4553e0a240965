"""Data-gradient backward of the MoE layer on the HIP library.

``jax.value_and_grad`` (``train.py:266``) differentiates ``MoE.__call__``
(``model/moe.py:170-246``); this is that VJP for the routed bf16 path, with
the routing decisions (top-k indices, capacity drops, the dispatch plan) held
fixed, as JAX does for integer-valued operations:

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
    d_ys, d_gates = K.combine_bwd(dy, fwd["ys"], plan, fwd["gates"])
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
