"""JAX host side of the XLA FFI boundary: ``model/moe.py``'s ``MoE.__call__``
(``moe.py:170-294``) with its forward and its VJP on ``libhanuman_moe.so``.

A JAX maintainer keeps the reference's ``MoE`` module (constructor, parameter
pytree, ``transformer.py:71-73,92-95`` call sites) and replaces the body of
``__call__`` with::

    from hanuman_amd.xla_ffi import moe_jax
    moe_jax.register()                                  # once per process
    def __call__(self, x):
        return moe_jax.moe_call(self, x)

``moe_call`` reads the module's parameters (``router``, ``bias``,
``expert_w_gate/up/down``, ``shared_w_gate/up/down``) and returns ``(out
[B,S,D] float32, aux)`` with the four aux entries of ``moe.py:286-291``.  It
is a ``jax.custom_vjp``: ``jax.value_and_grad`` (``train.py:266``) takes the
library's VJP (``moe.py:37-85,161-294`` differentiated with the routing held
fixed, as JAX does for the integer top-k, argsort and bincount), so the
reference's ``loss_fn`` (``train.py:191-217``) trains through it unchanged.
The router bias gets a zero gradient (it only selects, ``moe.py:181-183``);
``expert_counts`` has none.

Every step is one custom call (``jax.ffi.ffi_call``) to a handler of
``hmoe_xla_ffi.cc``; all shapes are static (``hmoe_rows_cap``, the
workspace-size functions of the C ABI, evaluated at trace time).  bf16
compute (the reference's default ``dtype``); sigmoid routing with the
reference's ``routed_scaling_factor``, or the workload rules (softmax
routing, capacity factor) through :class:`MoEConfig`.

Neither this module nor the handler library can be exercised in this
repository's image (JAX is not installed and its FFI headers ship with it);
the C ABI below them is the one the GPU tests drive through ``ctypes``.
"""
from __future__ import annotations

import ctypes
import dataclasses
import functools
from pathlib import Path

import jax
import jax.numpy as jnp
import numpy as np

_HERE = Path(__file__).resolve().parent
CORE_LIB = _HERE.parent / "libhanuman_moe.so"
FFI_LIB = _HERE / "libhanuman_moe_xla.so"

ROUTE_SIGMOID_BIAS, ROUTE_SOFTMAX = 0, 1

# custom-call target -> handler symbol in libhanuman_moe_xla.so
TARGETS = {
    # forward
    "hmoe_router": "HmoeRouter",
    "hmoe_router_quant_fp8": "HmoeRouterQuantFp8",
    "hmoe_router_from_logits": "HmoeRouterFromLogits",
    "hmoe_dispatch_plan": "HmoeDispatchPlan",
    "hmoe_permute_rows": "HmoePermuteRows",
    "hmoe_permute_rows_fp8": "HmoePermuteRowsFp8",
    "hmoe_quantize_rows_fp8": "HmoeQuantizeRowsFp8",
    "hmoe_pack_gate_up": "HmoePackGateUp",
    "hmoe_pack_down": "HmoePackDown",
    "hmoe_pack_fp8_gate_up": "HmoePackFp8GateUp",
    "hmoe_pack_fp8_down": "HmoePackFp8Down",
    "hmoe_grouped_gate_up": "HmoeGroupedGateUp",
    "hmoe_grouped_gate_up_gather": "HmoeGroupedGateUpGather",
    "hmoe_grouped_down": "HmoeGroupedDown",
    "hmoe_grouped_swiglu_fused": "HmoeGroupedSwigluFused",
    "hmoe_grouped_gate_up_fp8": "HmoeGroupedGateUpFp8",
    "hmoe_grouped_gate_up_fp8_gather": "HmoeGroupedGateUpFp8Gather",
    "hmoe_grouped_down_fp8": "HmoeGroupedDownFp8",
    "hmoe_grouped_gate_up_fp8_qh": "HmoeGroupedGateUpFp8Qh",
    "hmoe_grouped_gate_up_fp8_gather_qh": "HmoeGroupedGateUpFp8GatherQh",
    "hmoe_grouped_down_fp8_mx": "HmoeGroupedDownFp8Mx",
    "hmoe_grouped_gate_up_f32": "HmoeGroupedGateUpF32",
    "hmoe_grouped_down_f32": "HmoeGroupedDownF32",
    "hmoe_combine": "HmoeCombine",
    "hmoe_router_aux": "HmoeRouterAux",
    # backward
    "hmoe_combine_bwd": "HmoeCombineBwd",
    "hmoe_grouped_gate_up_raw_gather": "HmoeGroupedGateUpRawGather",
    "hmoe_grouped_gate_up_raw": "HmoeGroupedGateUpRaw",
    "hmoe_grouped_gate_up_swiglu_bwd_gather": "HmoeGroupedGateUpSwigluBwdGather",
    "hmoe_grouped_gate_up_swiglu_bwd": "HmoeGroupedGateUpSwigluBwd",
    "hmoe_swiglu_bwd": "HmoeSwigluBwd",
    "hmoe_pack_down_dgrad": "HmoePackDownDgrad",
    "hmoe_pack_gate_up_dgrad": "HmoePackGateUpDgrad",
    "hmoe_grouped_dgrad_down": "HmoeGroupedDgradDown",
    "hmoe_grouped_dgrad_gate_up": "HmoeGroupedDgradGateUp",
    "hmoe_gather_bwd": "HmoeGatherBwd",
    "hmoe_router_bwd": "HmoeRouterBwd",
    "hmoe_router_aux_bwd": "HmoeRouterAuxBwd",
    "hmoe_router_dx": "HmoeRouterDx",
    "hmoe_grouped_wgrad_down": "HmoeGroupedWgradDown",
    "hmoe_grouped_wgrad_gate_up": "HmoeGroupedWgradGateUp",
    "hmoe_router_dw": "HmoeRouterDw",
    "hmoe_combine_bwd_f32": "HmoeCombineBwdF32",
    "hmoe_grouped_dgrad_down_f32": "HmoeGroupedDgradDownF32",
    "hmoe_grouped_gate_up_swiglu_bwd_f32": "HmoeGroupedGateUpSwigluBwdF32",
    "hmoe_grouped_dgrad_gate_up_f32": "HmoeGroupedDgradGateUpF32",
    "hmoe_grouped_wgrad_gate_up_f32": "HmoeGroupedWgradGateUpF32",
    "hmoe_grouped_wgrad_down_f32": "HmoeGroupedWgradDownF32",
}


@functools.lru_cache(maxsize=None)
def _core():
    lib = ctypes.CDLL(str(CORE_LIB))
    i32, i64, sz, dbl = ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_double
    for name, res, args in (
            ("hmoe_capacity", i64, [i64, i32, i32, dbl]),
            ("hmoe_rows_cap", i64, [i64, i32, i32, i64]),
            ("hmoe_plan_workspace_bytes", sz, [i64, i32, i32]),
            ("hmoe_aux_workspace_bytes", sz, [i32, i32, i32]),
            ("hmoe_aux_bwd_workspace_bytes", sz, [i32, i32, i32]),
            ("hmoe_router_dw_workspace_bytes", sz, [i64, i32, i32]),
            ("hmoe_packed_gate_up_bytes", sz, [i32, i32, i32]),
            ("hmoe_packed_down_bytes", sz, [i32, i32, i32]),
            ("hmoe_grouped_swiglu_fused_workspace_bytes", sz, [i64, i32])):
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    return lib


def register(platform: str = "ROCM") -> None:
    """Registers every handler of ``libhanuman_moe_xla.so`` as an XLA FFI
    target (once per process)."""
    lib = ctypes.CDLL(str(FFI_LIB))
    for name, sym in TARGETS.items():
        jax.ffi.register_ffi_target(name, jax.ffi.pycapsule(getattr(lib, sym)), platform=platform)


def _sds(shape, dtype):
    return jax.ShapeDtypeStruct(tuple(int(s) for s in shape), dtype)


def _call(target, outs, *args, aliases=None, **attrs):
    return jax.ffi.ffi_call(target, outs, input_output_aliases=aliases or {})(*args, **attrs)


@dataclasses.dataclass(frozen=True)
class MoEConfig:
    """Static configuration of one layer (the reference module's hyper-
    parameters plus the workload rules that have no reference code)."""
    n_experts: int
    top_k: int
    n_shared: int
    routed_scaling_factor: float = 1.0
    routing: str = "sigmoid"          # "sigmoid" (moe.py:179-192) or "softmax"
    capacity_factor: float | None = None
    # fused: gate/up and down in one persistent launch where the shapes allow.
    # Off by default, as in the torch layer: the two launches measure within
    # noise of it, and its bounded wait reports a give-up only in the status
    # word (uint32 8 of its workspace result), which this module does not read.
    fused: bool = False

    @property
    def mode(self) -> int:
        return ROUTE_SIGMOID_BIAS if self.routing == "sigmoid" else ROUTE_SOFTMAX


# ---- forward steps ---------------------------------------------------------------

def _router(cfg, x, router_w, bias):
    T, N, K = x.shape[0], cfg.n_experts, cfg.top_k
    return _call("hmoe_router", (_sds((T, N), jnp.float32), _sds((T, K), jnp.int32),
                                 _sds((T, K), jnp.float32)),
                 x, router_w, bias, mode=np.int64(cfg.mode),
                 routed_scaling_factor=np.float32(cfg.routed_scaling_factor))


def _plan(cfg, top_idx):
    T, K, N = top_idx.shape[0], cfg.top_k, cfg.n_experts
    lib = _core()
    cap = int(lib.hmoe_capacity(T, K, N, float(cfg.capacity_factor or 0.0)))
    rows = int(lib.hmoe_rows_cap(T, K, N, cap))
    ws = int(lib.hmoe_plan_workspace_bytes(T, K, N))
    counts, offsets, slot_pos, perm_src, keep, _ = _call(
        "hmoe_dispatch_plan",
        (_sds((N,), jnp.int32), _sds((N + 1,), jnp.int32), _sds((T * K,), jnp.int32),
         _sds((rows,), jnp.int32), _sds((T * K,), jnp.uint8), _sds((max(ws, 1),), jnp.uint8)),
        top_idx, capacity=np.int64(cap))
    return {"counts": counts, "offsets": offsets, "slot_pos": slot_pos, "perm_src": perm_src,
            "keep": keep}


def _pack(wg, wu, wd):
    N, D, F = wg.shape
    lib = _core()
    gu_bytes = int(lib.hmoe_packed_gate_up_bytes(N, D, F))
    dn_bytes = int(lib.hmoe_packed_down_bytes(N, F, D))
    wgu = _call("hmoe_pack_gate_up", (_sds((gu_bytes,), jnp.uint8),), wg, wu)[0]
    wdn = _call("hmoe_pack_down", (_sds((dn_bytes,), jnp.uint8),), wd)[0]
    return wgu, wdn


def _experts(cfg, xb, plan, wgu, wdn, D, F):
    rows, N = plan["perm_src"].shape[0], cfg.n_experts
    if cfg.fused and D % 256 == 0 and F % 128 == 0 and F >= 256:
        ws = int(_core().hmoe_grouped_swiglu_fused_workspace_bytes(rows, N))
        h, ys, _ = _call("hmoe_grouped_swiglu_fused",
                         (_sds((rows, F), jnp.bfloat16), _sds((rows, D), jnp.bfloat16),
                          _sds((max(ws, 64),), jnp.uint8)),
                         xb, plan["perm_src"], plan["offsets"], wgu, wdn, top_k=np.int64(cfg.top_k))
        return h, ys
    h = _call("hmoe_grouped_gate_up_gather", (_sds((rows, F), jnp.bfloat16),),
              xb, plan["perm_src"], plan["offsets"], wgu, top_k=np.int64(cfg.top_k))[0]
    ys = _call("hmoe_grouped_down", (_sds((rows, D), jnp.bfloat16),), h, plan["offsets"], wdn)[0]
    return h, ys


def _one_segment(T):
    return jnp.array([0, T], dtype=jnp.int32)


def _shared_weights(module_or_params, n_shared):
    ws = [module_or_params["shared_w_gate"], module_or_params["shared_w_up"],
          module_or_params["shared_w_down"]]
    if n_shared == 1:
        return [tuple(w[None] for w in ws)]
    return [tuple(w[i:i + 1] for w in ws) for i in range(n_shared)]


def _shared_forward(cfg, xb, params):
    """Shared expert(s) (moe.py:161-168, 23-29): one segment of all tokens on
    the grouped kernels; bf16 output, the float32 mean over several."""
    T = xb.shape[0]
    off = _one_segment(T)
    outs, hs = [], []
    for wg, wu, wd in _shared_weights(params, cfg.n_shared):
        wgu, wdn = _pack(wg, wu, wd)
        F, D = wg.shape[2], wg.shape[1]
        h = _call("hmoe_grouped_gate_up", (_sds((T, F), jnp.bfloat16),), xb, off, wgu)[0]
        y = _call("hmoe_grouped_down", (_sds((T, D), jnp.bfloat16),), h, off, wdn)[0]
        outs.append(y)
        hs.append(h)
    if len(outs) == 1:
        return outs[0], hs
    return sum(o.astype(jnp.float32) for o in outs) / cfg.n_shared, hs


def _aux(cfg, logits, top_idx, B, S):
    N = cfg.n_experts
    ws = int(_core().hmoe_aux_workspace_bytes(B, S, N))
    losses, counts, _ = _call("hmoe_router_aux",
                              (_sds((3,), jnp.float32), _sds((N,), jnp.float32),
                               _sds((max(ws, 1),), jnp.uint8)),
                              logits, top_idx, batch=np.int64(B))
    return losses, counts


def _forward(cfg, params, x):
    B, S, D = x.shape
    T = B * S
    xb = x.astype(jnp.bfloat16).reshape(T, D)                       # moe.py:198
    logits, top_idx, gates = _router(cfg, x.reshape(T, D), params["router"],
                                     params["bias"].astype(jnp.float32))
    plan = _plan(cfg, top_idx)
    wg, wu, wd = (params[k].astype(jnp.bfloat16)                    # moe.py:204-206
                  for k in ("expert_w_gate", "expert_w_up", "expert_w_down"))
    F = wg.shape[2]
    wgu, wdn = _pack(wg, wu, wd)
    h, ys = _experts(cfg, xb, plan, wgu, wdn, D, F)
    shared, h_sh = _shared_forward(cfg, x.reshape(T, D).astype(jnp.bfloat16), params)
    out = _call("hmoe_combine", (_sds((T, D), jnp.float32),), ys, plan["slot_pos"], gates,
                shared)[0]
    losses, counts = _aux(cfg, logits, top_idx, B, S)
    aux = {"router_z_loss": losses[0], "balance_loss": losses[1], "mean_entropy": losses[2],
           "expert_counts": counts}
    saved = (x, logits, top_idx, gates, plan, h, ys, h_sh, wgu)
    return (out.reshape(B, S, D), aux), saved


# ---- backward steps ----------------------------------------------------------------

def _backward(cfg, params, saved, cts):
    x, logits, top_idx, gates, plan, h, ys, h_sh, wgu = saved
    d_out, d_aux = cts
    B, S, D = x.shape
    T, N, K = B * S, cfg.n_experts, cfg.top_k
    rows = plan["perm_src"].shape[0]    # static: hmoe_rows_cap at trace time
    xb = x.astype(jnp.bfloat16).reshape(T, D)
    dy = d_out.reshape(T, D).astype(jnp.float32)
    F = params["expert_w_gate"].shape[2]
    # 1. combine VJP (moe.py:80-85) and the shared experts' output cotangent
    d_ys, d_gates, d_sh = _call(
        "hmoe_combine_bwd",
        (_sds((rows, D), jnp.bfloat16), _sds((T, K), jnp.float32), _sds((T, D), jnp.bfloat16)),
        dy, ys, plan["slot_pos"], gates, shared_div=np.float32(cfg.n_shared))
    # 2-4. expert data gradients (moe.py:70-73)
    wg, wu, wd = (params[k].astype(jnp.bfloat16)
                  for k in ("expert_w_gate", "expert_w_up", "expert_w_down"))
    wd_dgrad = _call("hmoe_pack_down_dgrad", (_sds((N, F, D), jnp.bfloat16),), wd)[0]
    wgu_dgrad = _call("hmoe_pack_gate_up_dgrad", (_sds((N, D, 2 * F), jnp.bfloat16),), wg, wu)[0]
    dh = _call("hmoe_grouped_dgrad_down", (_sds((rows, F), jnp.bfloat16),),
               d_ys, plan["offsets"], wd_dgrad)[0]
    dgu = _call("hmoe_grouped_gate_up_swiglu_bwd_gather", (_sds((rows, 2 * F), jnp.bfloat16),),
                xb, plan["perm_src"], plan["offsets"], wgu, dh, top_k=np.int64(K))[0]
    d_xs = _call("hmoe_grouped_dgrad_gate_up", (_sds((rows, D), jnp.bfloat16),),
                 dgu, plan["offsets"], wgu_dgrad)[0]
    # 5. shared experts (moe.py:23-29, 161-168): one segment of all tokens
    off1 = _one_segment(T)
    dx_sh = None
    sh_grads = []
    for (swg, swu, swd), hs in zip(_shared_weights(params, cfg.n_shared), h_sh):
        Fs = swg.shape[2]
        swg_b, swu_b, swd_b = (w.astype(jnp.bfloat16) for w in (swg, swu, swd))
        s_gu, _ = _pack(swg_b, swu_b, swd_b)
        s_dn_dgrad = _call("hmoe_pack_down_dgrad", (_sds((1, Fs, D), jnp.bfloat16),), swd_b)[0]
        s_gu_dgrad = _call("hmoe_pack_gate_up_dgrad", (_sds((1, D, 2 * Fs), jnp.bfloat16),),
                           swg_b, swu_b)[0]
        s_dh = _call("hmoe_grouped_dgrad_down", (_sds((T, Fs), jnp.bfloat16),), d_sh, off1,
                     s_dn_dgrad)[0]
        s_dgu = _call("hmoe_grouped_gate_up_swiglu_bwd", (_sds((T, 2 * Fs), jnp.bfloat16),),
                      xb, off1, s_gu, s_dh)[0]
        s_dx = _call("hmoe_grouped_dgrad_gate_up", (_sds((T, D), jnp.bfloat16),), s_dgu, off1,
                     s_gu_dgrad)[0]
        s_dwg, s_dwu = _call("hmoe_grouped_wgrad_gate_up",
                             (_sds((1, D, Fs), jnp.float32), _sds((1, D, Fs), jnp.float32)),
                             xb, s_dgu, off1)
        s_dwd = _call("hmoe_grouped_wgrad_down", (_sds((1, Fs, D), jnp.float32),), hs, d_sh,
                      off1)[0]
        dx_sh = s_dx.astype(jnp.float32) if dx_sh is None else dx_sh + s_dx.astype(jnp.float32)
        sh_grads.append((s_dwg, s_dwu, s_dwd))
    # 6. gather VJP (moe.py:56), the shared experts' input gradient as the residual
    dx = _call("hmoe_gather_bwd", (_sds((T, D), jnp.float32),), d_xs, plan["slot_pos"],
               dx_sh if dx_sh is not None else jnp.zeros((0, D), jnp.float32))[0]
    # 7. gates and aux losses into d_logits (moe.py:179-192, 253-283)
    d_logits = _call("hmoe_router_bwd", (_sds((T, N), jnp.float32),), logits, top_idx, gates,
                     d_gates, mode=np.int64(cfg.mode),
                     routed_scaling_factor=np.float32(cfg.routed_scaling_factor))[0]
    d_losses = jnp.stack([d_aux["router_z_loss"], d_aux["balance_loss"],
                          d_aux["mean_entropy"]]).astype(jnp.float32)
    aux_ws = int(_core().hmoe_aux_bwd_workspace_bytes(B, S, N))
    d_logits, _ = _call("hmoe_router_aux_bwd",
                        (_sds((T, N), jnp.float32), _sds((max(aux_ws, 1),), jnp.uint8)),
                        logits, top_idx, d_losses, d_logits, aliases={3: 0}, batch=np.int64(B))
    # 8. dx += d_logits router^T (moe.py:175,178)
    dx = _call("hmoe_router_dx", (_sds((T, D), jnp.float32),), d_logits, params["router"], dx,
               aliases={2: 0})[0]
    # 9. weight gradients
    xs = _call("hmoe_permute_rows", (_sds((rows, D), jnp.bfloat16),), xb, plan["slot_pos"])[0]
    dwg, dwu = _call("hmoe_grouped_wgrad_gate_up",
                     (_sds((N, D, F), jnp.float32), _sds((N, D, F), jnp.float32)),
                     xs, dgu, plan["offsets"])
    dwd = _call("hmoe_grouped_wgrad_down", (_sds((N, F, D), jnp.float32),), h, d_ys,
                plan["offsets"])[0]
    dw_ws = int(_core().hmoe_router_dw_workspace_bytes(T, D, N))
    d_router, _ = _call("hmoe_router_dw",
                        (_sds((D, N), jnp.float32), _sds((max(dw_ws, 1),), jnp.uint8)),
                        x.reshape(T, D), d_logits)
    grads = {
        "router": d_router.astype(params["router"].dtype),
        "bias": jnp.zeros_like(params["bias"]),
        "expert_w_gate": dwg.astype(params["expert_w_gate"].dtype),
        "expert_w_up": dwu.astype(params["expert_w_up"].dtype),
        "expert_w_down": dwd.astype(params["expert_w_down"].dtype),
    }
    if cfg.n_shared == 1:
        g, u, d = sh_grads[0]
        grads.update(shared_w_gate=g[0], shared_w_up=u[0], shared_w_down=d[0])
    else:
        grads.update(shared_w_gate=jnp.concatenate([g for g, _, _ in sh_grads]),
                     shared_w_up=jnp.concatenate([u for _, u, _ in sh_grads]),
                     shared_w_down=jnp.concatenate([d for _, _, d in sh_grads]))
    for k in ("shared_w_gate", "shared_w_up", "shared_w_down"):
        grads[k] = grads[k].astype(params[k].dtype)
    return grads, dx.reshape(B, S, D).astype(x.dtype)


@functools.partial(jax.custom_vjp, nondiff_argnums=(0,))
def moe_layer(cfg: MoEConfig, params: dict, x):
    """``MoE.__call__`` on the library: ``(out [B,S,D] f32, aux)``."""
    return _forward(cfg, params, x)[0]


def _moe_layer_fwd(cfg, params, x):
    out, saved = _forward(cfg, params, x)
    return out, (params, saved)


def _moe_layer_bwd(cfg, res, cts):
    params, saved = res
    return _backward(cfg, params, saved, cts)


moe_layer.defvjp(_moe_layer_fwd, _moe_layer_bwd)

PARAM_NAMES = ("router", "bias", "expert_w_gate", "expert_w_up", "expert_w_down",
               "shared_w_gate", "shared_w_up", "shared_w_down")


def moe_call(module, x, *, routing: str = "sigmoid", capacity_factor=None, fused: bool = False):
    """Drop-in body of the reference ``MoE.__call__``: reads the module's
    parameters by their pytree names and runs :func:`moe_layer`."""
    params = {k: getattr(module, k).value for k in PARAM_NAMES}
    cfg = MoEConfig(n_experts=module.n_experts, top_k=module.n_active,
                    n_shared=module.n_shared_experts,
                    routed_scaling_factor=float(module.routed_scaling_factor),
                    routing=routing, capacity_factor=capacity_factor, fused=fused)
    return moe_layer(cfg, params, x)
