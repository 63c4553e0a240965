"""Drop-in MoE layer for one MI355X (reference: ``model/moe.py`` of theorionic/hanuman).

``MoE`` keeps the reference constructor signature (``moe.py:126-128``), its
parameter names -- ``router``, ``bias``, ``expert_w_gate``, ``expert_w_up``,
``expert_w_down``, ``shared_w_gate``, ``shared_w_up``, ``shared_w_down`` --
with the same shapes, and its call contract ``x [B,S,D] -> (out [B,S,D] f32,
aux)`` (``moe.py:170-294``).  Parameters are torch tensors held in ``Param``
objects (``.value``, like ``nnx.Param``).  Every stage runs in
``libhanuman_moe.so``; torch only allocates and supplies the stream.

Only the single-device branch exists (``moe.py:216-218``): all experts are
resident in one GPU's HBM, so ``mesh`` must be None or hold one device.
"""
from __future__ import annotations

import weakref

import numpy as np
import torch

from . import _lib
from . import kernels as K


class Param:
    """Parameter holder with a ``.value`` tensor (the ``nnx.Param`` role)."""

    __slots__ = ("value",)

    def __init__(self, value: torch.Tensor):
        self.value = value

    def __repr__(self):
        v = self.value
        return f"Param(shape={tuple(v.shape)}, dtype={v.dtype}, device={v.device})"


def _torch_dtype(dtype) -> torch.dtype:
    if isinstance(dtype, torch.dtype):
        return dtype
    name = getattr(dtype, "name", None) or getattr(dtype, "__name__", None) or str(dtype)
    name = name.lower().replace("jnp.", "").replace("numpy.", "")
    if name in ("bfloat16", "bf16"):
        return torch.bfloat16
    if name in ("float32", "f32", "fp32"):
        return torch.float32
    raise TypeError(f"unsupported compute dtype {dtype!r}")


def _generator(rngs, device) -> torch.Generator:
    if isinstance(rngs, torch.Generator):
        return rngs
    if isinstance(rngs, np.random.Generator):
        seed = int(rngs.integers(0, 2**63 - 1))
    elif rngs is None:
        seed = 0
    else:
        seed = int(rngs)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _require_bf16_compute(dtype: torch.dtype):
    if dtype not in (torch.bfloat16, torch.float32):
        raise NotImplementedError(
            "the grouped expert GEMMs compute in bfloat16 (fp32 accumulation) or float32; "
            f"compute dtype {dtype} is not built")


def _f32_swiglu_one(x32: torch.Tensor, wg, wu, wd, hs: list | None = None) -> torch.Tensor:
    """One float32 SwiGLU (``moe.py:23-29`` with dtype float32): one segment
    of all rows on the float32 grouped GEMMs, masters as they are.  ``hs``
    collects ``h`` for the backward."""
    off = _offsets_one_group(x32.shape[0], x32.device)
    h = K.grouped_gate_up_f32(x32, off, wg.float().unsqueeze(0).contiguous(),
                              wu.float().unsqueeze(0).contiguous())
    if hs is not None:
        hs.append(h)
    return K.grouped_down_f32(h, off, wd.float().unsqueeze(0).contiguous())


class _PackCache:
    """Packed bf16 operands of fp32 master weights, rebuilt when a master
    changes: a different tensor object (held by weak reference and compared
    by identity, so a new tensor at a freed address is not mistaken for the
    old one), an in-place update (the tensor's version counter), or new
    storage under the same object (``t.data = other``, which keeps both the
    identity and the version counter: caught by the data pointer, shape,
    stride and dtype)."""

    def __init__(self):
        self._refs = None
        self._keys = None
        self._val = None

    @staticmethod
    def _key(t):
        return (t._version, t.data_ptr(), tuple(t.shape), t.stride(), t.dtype, t.device)

    def get(self, tensors, build):
        same = (self._refs is not None and len(self._refs) == len(tensors)
                and all(r() is t for r, t in zip(self._refs, tensors))
                and all(self._key(t) == k for t, k in zip(tensors, self._keys)))
        if not same:
            self._val = build()
            self._refs = tuple(weakref.ref(t) for t in tensors)
            self._keys = tuple(self._key(t) for t in tensors)
        return self._val


def _offsets_one_group(rows: int, device) -> torch.Tensor:
    return torch.tensor([0, rows], dtype=torch.int32, device=device)


def swiglu(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor,
           dtype) -> torch.Tensor:
    """Dense SwiGLU ``down(silu(x@gate) * (x@up))`` -> float32 (``moe.py:23-29``).

    Runs the grouped GEMMs with one group.  ``x [T,D]``; weights ``[D,F]``,
    ``[D,F]``, ``[F,D]``.  The output of the down matmul is rounded to the
    compute dtype and returned as float32, as the reference does.
    """
    dt = _torch_dtype(dtype)
    _require_bf16_compute(dt)
    if dt == torch.float32:
        return _f32_swiglu_one(x.float().contiguous(), w_gate, w_up, w_down)
    xb = x.to(dt).contiguous()
    T = xb.shape[0]
    off = _offsets_one_group(T, x.device)
    wgu = K.pack_gate_up(w_gate.unsqueeze(0).contiguous(), w_up.unsqueeze(0).contiguous())
    wd = K.pack_down(w_down.unsqueeze(0).contiguous())
    h = K.grouped_gate_up(xb, off, wgu)
    return K.grouped_down(h, off, wd).float()


def ragged_dispatch(x_flat: torch.Tensor, top_idx: torch.Tensor, weights: torch.Tensor,
                    w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor,
                    dtype) -> torch.Tensor:
    """Route each token to its top-k experts and run SwiGLU (``moe.py:37-85``).

    ``x_flat [T,D]`` (compute dtype), ``top_idx [T,K]`` int32, ``weights [T,K]``
    float32, stacked expert weights ``[N,D,F]``/``[N,F,D]``.  Dropless, stable
    expert grouping, float32 result ``[T,D]``.
    """
    dt = _torch_dtype(dtype)
    _require_bf16_compute(dt)
    T, Kk = top_idx.shape
    N = w_gate.shape[0]
    plan = K.dispatch_plan(top_idx.to(torch.int32).contiguous(), N, T * Kk)
    if dt == torch.float32:
        xs = K.permute_rows(x_flat.contiguous(), plan, torch.float32)
        h = K.grouped_gate_up_f32(xs, plan.offsets, w_gate.float().contiguous(),
                                  w_up.float().contiguous())
        ys = K.grouped_down_f32(h, plan.offsets, w_down.float().contiguous())
        return K.combine(ys, plan, weights.float().contiguous(), None, torch.float32)
    wgu = K.pack_gate_up(w_gate, w_up)
    if x_flat.dtype == torch.bfloat16:
        # the gate/up GEMM gathers its rows from x (moe.py:56 fused)
        h = K.grouped_gate_up_gather(x_flat.contiguous(), plan, wgu)
    else:
        h = K.grouped_gate_up(K.permute_rows(x_flat.contiguous(), plan, dt), plan.offsets, wgu)
    ys = K.grouped_down(h, plan.offsets, K.pack_down(w_down))
    return K.combine(ys, plan, weights.float().contiguous(), None, torch.float32)


class MoE:
    """Mixture of Experts with aux-loss-free sigmoid routing (``moe.py:116-294``).

    Reference behaviour by default.  Keyword-only extensions (not in the
    reference): ``routing="softmax"`` (top-k of softmax, renormalised gates,
    no bias, no scaling) and ``capacity_factor`` (per-expert capacity
    ``ceil(CF*T*K/N)`` with token-order priority; ``None`` = dropless).
    """

    def __init__(self, d_model: int, d_ff: int, n_experts: int, n_active: int,
                 n_shared_experts: int, router_init_std: float, routed_scaling_factor: float,
                 dtype, rngs, mesh=None, d_ff_shared: int | None = None, *,
                 routing: str = "sigmoid", capacity_factor: float | None = None,
                 device: str | torch.device | None = None):
        if mesh is not None:
            size = getattr(getattr(mesh, "devices", None), "size", 1)
            if size > 1:
                raise NotImplementedError("one GPU holds every expert; a multi-device mesh is not built")
        if routing not in ("sigmoid", "softmax"):
            raise ValueError(f"routing must be 'sigmoid' or 'softmax' (got {routing!r})")
        dev = torch.device(device) if device is not None else torch.device("cuda")
        self.mesh = mesh
        self.expert_axis_name = None
        self.n_experts = n_experts
        self.n_active = n_active
        self.n_shared_experts = n_shared_experts
        self.routed_scaling_factor = routed_scaling_factor
        self.dtype = _torch_dtype(dtype)
        self.routing = routing
        self.capacity_factor = capacity_factor
        g = _generator(rngs, dev)

        def normal(shape, std):
            return torch.randn(shape, generator=g, device=dev, dtype=torch.float32) * std

        self.router = Param(normal((d_model, n_experts), router_init_std))
        self.bias = Param(torch.zeros(n_experts, dtype=torch.float32, device=dev))
        std = (1.0 / d_model) ** 0.5
        self.expert_w_gate = Param(normal((n_experts, d_model, d_ff), std))
        self.expert_w_up = Param(normal((n_experts, d_model, d_ff), std))
        self.expert_w_down = Param(normal((n_experts, d_ff, d_model), std))
        dfs = d_ff if d_ff_shared is None else d_ff_shared
        if n_shared_experts == 1:
            self.shared_w_gate = Param(normal((d_model, dfs), std))
            self.shared_w_up = Param(normal((d_model, dfs), std))
            self.shared_w_down = Param(normal((dfs, d_model), std))
        else:
            self.shared_w_gate = Param(normal((n_shared_experts, d_model, dfs), std))
            self.shared_w_up = Param(normal((n_shared_experts, d_model, dfs), std))
            self.shared_w_down = Param(normal((n_shared_experts, dfs, d_model), std))
        self._routed_pack = _PackCache()
        self._shared_pack = _PackCache()

    # ---- parameters ------------------------------------------------------
    def named_params(self) -> dict:
        """Parameter pytree paths -> Param, in reference attribute order."""
        names = ("router", "bias", "expert_w_gate", "expert_w_up", "expert_w_down",
                 "shared_w_gate", "shared_w_up", "shared_w_down")
        return {n: getattr(self, n) for n in names}

    def state(self) -> dict:
        """The parameters as a pure dict of float32 NumPy arrays under the
        reference's attribute names (the MoE subtree of the nnx state that
        ``train.py:326-334`` checkpoints)."""
        return {n: p.value.detach().float().cpu().numpy() for n, p in self.named_params().items()}

    def load_state(self, tree) -> None:
        """Loads parameters from a mapping in the reference's layout: each
        name of :meth:`named_params` maps to an array (NumPy, torch or
        anything ``np.asarray`` takes) or to an nnx-style ``{"value": array}``
        node.  Every name must be present with the parameter's shape; values
        are copied in place (float32), so packed operands rebuild on the next
        call."""
        for name, param in self.named_params().items():
            if name not in tree:
                raise KeyError(f"checkpoint has no {name!r}")
            leaf = tree[name]
            if isinstance(leaf, dict):
                if "value" not in leaf:
                    raise KeyError(f"checkpoint node {name!r} has no 'value'")
                leaf = leaf["value"]
            arr = leaf if isinstance(leaf, torch.Tensor) else torch.from_numpy(
                np.ascontiguousarray(np.asarray(leaf, dtype=np.float32)))
            if tuple(arr.shape) != tuple(param.value.shape):
                raise ValueError(f"{name}: checkpoint shape {tuple(arr.shape)} != "
                                 f"parameter shape {tuple(param.value.shape)}")
            with torch.no_grad():
                param.value.copy_(arr.to(device=param.value.device, dtype=param.value.dtype))

    def save_safetensors(self, path) -> None:
        """Writes :meth:`state` to a safetensors file (reference names)."""
        from safetensors.numpy import save_file
        save_file(self.state(), str(path))

    def load_safetensors(self, path) -> None:
        """Loads a file written by :meth:`save_safetensors` (or any
        safetensors file with the reference names and shapes)."""
        from safetensors.numpy import load_file
        self.load_state(load_file(str(path)))

    def _packed_routed(self, masters=None):
        """Packed routed-expert operands of ``masters`` (default: the current
        parameters)."""
        wg, wu, wd = masters if masters is not None else (
            self.expert_w_gate.value, self.expert_w_up.value, self.expert_w_down.value)
        return self._routed_pack.get((wg, wu, wd), lambda: (K.pack_gate_up(wg, wu), K.pack_down(wd)))

    def _packed_shared(self, masters=None):
        wg, wu, wd = masters if masters is not None else (
            self.shared_w_gate.value, self.shared_w_up.value, self.shared_w_down.value)

        def build():
            if self.n_shared_experts == 1:
                return [(K.pack_gate_up(wg.unsqueeze(0).contiguous(), wu.unsqueeze(0).contiguous()),
                         K.pack_down(wd.unsqueeze(0).contiguous()))]
            return [(K.pack_gate_up(wg[i:i + 1].contiguous(), wu[i:i + 1].contiguous()),
                     K.pack_down(wd[i:i + 1].contiguous())) for i in range(self.n_shared_experts)]
        return self._shared_pack.get((wg, wu, wd), build)

    # ---- forward -----------------------------------------------------------
    def _shared_ffn(self, x_flat: torch.Tensor, hs: list | None = None) -> torch.Tensor:
        """Shared expert(s) (``moe.py:161-168``): bf16 output of one expert, or
        the float32 mean over ``n_shared_experts``.  ``hs`` collects each
        expert's ``h`` for the backward."""
        if self.n_shared_experts == 0:
            return 0.0 / self.n_shared_experts  # ZeroDivisionError, as the reference
        T = x_flat.shape[0]
        off = _offsets_one_group(T, x_flat.device)
        outs = []
        if self.dtype == torch.float32:
            wg, wu, wdn = self.shared_w_gate.value, self.shared_w_up.value, self.shared_w_down.value
            if self.n_shared_experts == 1:
                return _f32_swiglu_one(x_flat, wg, wu, wdn, hs)
            acc = torch.zeros((T, wdn.shape[-1]), dtype=torch.float32, device=x_flat.device)
            for i in range(self.n_shared_experts):
                acc += _f32_swiglu_one(x_flat, wg[i], wu[i], wdn[i], hs)
            return acc / self.n_shared_experts
        for wgu, wd in self._packed_shared():
            h = K.grouped_gate_up(x_flat, off, wgu)
            if hs is not None:
                hs.append(h)
            outs.append(K.grouped_down(h, off, wd))
        if len(outs) == 1:
            return outs[0]
        acc = torch.zeros_like(outs[0], dtype=torch.float32)
        for o in outs:
            acc += o.float()
        return acc / self.n_shared_experts

    def _shared_ffn_promoted(self, x32: torch.Tensor, hs: list | None = None) -> torch.Tensor:
        """Shared expert(s) for a float32 ``x`` under bf16 compute: ``moe.py:249``
        passes ``x`` as given, so each SwiGLU's ``x @ w.astype(bf16)``
        (``moe.py:23-29``) promotes to float32: a float32 SwiGLU on the
        bf16-rounded weights, on the float32 grouped GEMMs, float32 output
        (the mean over several)."""
        wg, wu, wd = (w.to(torch.bfloat16).float()
                      for w in (self.shared_w_gate.value, self.shared_w_up.value,
                                self.shared_w_down.value))
        if self.n_shared_experts == 1:
            return _f32_swiglu_one(x32, wg, wu, wd, hs)
        acc = torch.zeros((x32.shape[0], wd.shape[-1]), dtype=torch.float32, device=x32.device)
        for i in range(self.n_shared_experts):
            acc += _f32_swiglu_one(x32, wg[i], wu[i], wd[i], hs)
        return acc / self.n_shared_experts

    def _params(self):
        return (self.router.value, self.expert_w_gate.value, self.expert_w_up.value,
                self.expert_w_down.value, self.shared_w_gate.value, self.shared_w_up.value,
                self.shared_w_down.value)

    def __call__(self, x: torch.Tensor):
        """``x [B,S,D]`` -> (``out [B,S,D]`` float32, aux dict).

        When autograd is on and ``x`` or a parameter requires grad, the call
        is recorded as one autograd node whose backward is the library's VJP
        of the whole module (:func:`hanuman_amd.backward.moe_backward`):
        ``out``, ``router_z_loss``, ``balance_loss`` and ``mean_entropy``
        are differentiable, ``expert_counts`` is not (``train.py:191-200``
        differentiates the same outputs)."""
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self._params())):
            out, z, bal, ent, counts = _MoEFunction.apply(self, x, *self._params())
            return out, {"router_z_loss": z, "balance_loss": bal, "mean_entropy": ent,
                         "expert_counts": counts}
        out, losses, counts, _ = self._forward(x, save=False)
        aux = {
            "router_z_loss": losses[0],
            "balance_loss": losses[1],
            "mean_entropy": losses[2],
            "expert_counts": counts,
        }
        return out, aux

    def _forward(self, x: torch.Tensor, save: bool):
        """The forward; returns ``(out [B,S,D], losses [3], counts [N], saved)``
        with ``saved`` the backward's residuals when ``save``."""
        _require_bf16_compute(self.dtype)
        if x.dim() != 3:
            raise ValueError(f"x must be [B, S, d_model] (got {tuple(x.shape)})")
        B, S, D = x.shape
        N, Kk = self.n_experts, self.n_active
        T = B * S
        x2 = x.reshape(T, D).contiguous()
        mode = _lib.ROUTE_SIGMOID_BIAS if self.routing == "sigmoid" else _lib.ROUTE_SOFTMAX
        rsf = self.routed_scaling_factor if self.routing == "sigmoid" else 1.0
        bias = self.bias.value if self.routing == "sigmoid" else None
        logits, top_idx, gates = K.router(x2, self.router.value.float().contiguous(),
                                          bias, Kk, mode, rsf)
        cap = K.capacity(T, Kk, N, self.capacity_factor)
        plan = K.dispatch_plan(top_idx, N, cap)
        if self.dtype == torch.float32:
            # float32 compute dtype: the experts on the float32 matrix cores
            xs = K.permute_rows(x2, plan, torch.float32)
            h = K.grouped_gate_up_f32(xs, plan.offsets, self.expert_w_gate.value.float().contiguous(),
                                      self.expert_w_up.value.float().contiguous())
            ys = K.grouped_down_f32(h, plan.offsets, self.expert_w_down.value.float().contiguous())
            hs = [] if save else None
            shared = self._shared_ffn(x2.float().contiguous(), hs)
            out = K.combine(ys, plan, gates, shared, torch.float32)
            losses, counts = K.router_aux(logits, top_idx, B, S)
            saved = None
            if save:
                saved = {"x": x2, "logits": logits, "top_idx": top_idx, "gates": gates,
                         "plan": plan, "xs": xs, "h": h, "ys": ys, "h_shared": hs, "mode": mode,
                         "rsf": rsf, "batch": B, "seq": S}
            return out.reshape(B, S, D), losses, counts, saved
        wgu, wd = self._packed_routed()
        if x2.dtype == torch.bfloat16:
            # the gate/up GEMM gathers its rows from x (moe.py:56 fused)
            h = K.grouped_gate_up_gather(x2, plan, wgu)
        else:
            h = K.grouped_gate_up(K.permute_rows(x2, plan, self.dtype), plan.offsets, wgu)
        ys = K.grouped_down(h, plan.offsets, wd)
        hs = [] if save else None
        promoted = x2.dtype == torch.float32 and self.n_shared_experts > 0
        if promoted:
            shared = self._shared_ffn_promoted(x2, hs)
        else:
            shared = self._shared_ffn(x2 if x2.dtype == self.dtype else x2.to(self.dtype), hs)
        out = K.combine(ys, plan, gates, shared, torch.float32)
        losses, counts = K.router_aux(logits, top_idx, B, S)
        saved = None
        if save:
            saved = {"x": x2, "logits": logits, "top_idx": top_idx, "gates": gates, "plan": plan,
                     "h": h, "ys": ys, "h_shared": hs, "mode": mode, "rsf": rsf,
                     "batch": B, "seq": S, "shared_promoted": promoted}
        return out.reshape(B, S, D), losses, counts, saved

    def _backward_operands(self, masters):
        """Packed backward operands of the routed and shared experts for the
        masters ``(wg, wu, wd, swg, swu, swd)`` the forward used, cached like
        the forward's packs (rebuilt when a master changes)."""
        if not hasattr(self, "_bwd_pack"):
            self._bwd_pack = _PackCache()
        wg, wu, wd, swg, swu, swd = masters
        from .backward import BackwardOperands, SharedOperands

        def build():
            return (BackwardOperands(wg, wu, wd),
                    SharedOperands(swg, swu, swd, self.n_shared_experts,
                                   self._packed_shared((swg, swu, swd))))
        return self._bwd_pack.get((wg, wu, wd, swg, swu, swd), build)


class _MoEFunction(torch.autograd.Function):
    """``MoE.__call__`` as one autograd node: forward on the library, backward
    the library's VJP of the whole module (routing held fixed).  Every
    residual, and every parameter tensor the forward read, goes through
    ``save_for_backward``: a second backward through a retained graph works,
    and an in-place change of a parameter between forward and backward raises
    (torch's saved-tensor version check) instead of giving gradients of
    other weights."""

    _PLAN = ("counts", "offsets", "slot_pos", "perm_src", "keep")

    @staticmethod
    def forward(ctx, layer, x, router, wg, wu, wd, swg, swu, swd):
        out, losses, counts, saved = layer._forward(x, save=True)
        plan = saved["plan"]
        hs = list(saved["h_shared"] or [])
        ctx.layer = layer
        ctx.meta = {"capacity": plan.capacity, "rows_cap": plan.rows_cap,
                    "n_experts": plan.n_experts, "top_k": plan.top_k, "mode": saved["mode"],
                    "rsf": saved["rsf"], "batch": saved["batch"], "seq": saved["seq"],
                    "n_hs": len(hs), "f32": "xs" in saved,
                    "shared_promoted": saved.get("shared_promoted", False)}
        ctx.x_shape, ctx.x_dtype = x.shape, x.dtype
        ctx.save_for_backward(saved["x"], saved["logits"], saved["top_idx"], saved["gates"],
                              *(getattr(plan, k) for k in _MoEFunction._PLAN),
                              saved["h"], saved["ys"], saved.get("xs"), *hs,
                              router, wg, wu, wd, swg, swu, swd)
        ctx.mark_non_differentiable(counts)
        z, bal, ent = (v.clone() for v in losses.unbind())
        return out, z, bal, ent, counts

    @staticmethod
    def backward(ctx, d_out, d_z, d_bal, d_ent, d_counts):
        from .backward import moe_backward, moe_backward_f32
        layer, m = ctx.layer, ctx.meta
        st = list(ctx.saved_tensors)
        x2, logits, top_idx, gates = st[0:4]
        plan = K.Plan(*st[4:9], m["capacity"], m["rows_cap"], m["n_experts"], m["top_k"])
        h, ys, xs = st[9:12]
        hs = st[12:12 + m["n_hs"]]
        router, wg, wu, wd, swg, swu, swd = st[12 + m["n_hs"]:]
        fwd = {"logits": logits, "top_idx": top_idx, "gates": gates, "plan": plan, "h": h,
               "ys": ys}
        T, D = x2.shape
        dev = x2.device
        dy = (d_out.reshape(T, D).float().contiguous() if d_out is not None
              else torch.zeros((T, D), dtype=torch.float32, device=dev))
        zero = torch.zeros((), dtype=torch.float32, device=dev)
        d_losses = torch.stack([(g.float() if g is not None else zero)
                                for g in (d_z, d_bal, d_ent)]).contiguous()
        router_w = router.float().contiguous()
        aux = (m["batch"], m["seq"], d_losses)
        ng = ctx.needs_input_grad  # (layer, x, router, wg, wu, wd, swg, swu, swd)
        need = {"router": ng[2], "experts": any(ng[3:6]), "shared": any(ng[6:9])}
        if m["f32"]:
            fwd["xs"] = xs
            masters = tuple(t.float().contiguous() for t in (wg, wu, wd))
            shared = None
            if layer.n_shared_experts > 0:
                shared = tuple(t.float().contiguous() for t in (swg, swu, swd))
                shared = shared + (layer.n_shared_experts,)
            g = moe_backward_f32(x2, router_w, fwd, masters, dy, mode=m["mode"],
                                 routed_scaling_factor=m["rsf"], shared=shared, h_shared=hs,
                                 aux=aux, need=need)
        else:
            ops, shared = layer._backward_operands((wg, wu, wd, swg, swu, swd))
            wgu, _ = layer._packed_routed((wg, wu, wd))
            promoted = None
            if m["shared_promoted"]:
                # float32 x: the shared expert ran promoted to float32 on bf16(w)
                shared = None
                promoted = tuple(t.to(torch.bfloat16).float() for t in (swg, swu, swd)) + (
                    layer.n_shared_experts,)
            g = moe_backward(x2, router_w, fwd, wgu, ops, dy, mode=m["mode"],
                             routed_scaling_factor=m["rsf"], shared=shared, h_shared=hs,
                             aux=aux, need=need, shared_promoted=promoted)
        dx = g["dx"].reshape(ctx.x_shape).to(ctx.x_dtype) if ng[1] else None

        def shaped(key, like, wanted):
            return g[key].reshape(like.shape) if wanted and g.get(key) is not None else None
        return (None, dx, g["d_router"] if ng[2] else None,
                g["dWg"] if ng[3] else None, g["dWu"] if ng[4] else None,
                g["dWd"] if ng[5] else None,
                shaped("dWg_shared", swg, ng[6]), shaped("dWu_shared", swu, ng[7]),
                shaped("dWd_shared", swd, ng[8]))
