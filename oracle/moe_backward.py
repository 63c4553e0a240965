"""NumPy restatement of the MoE-layer backward: the vector-Jacobian product of
the routed forward that ``moe_oracle`` restates.

TEST INFRASTRUCTURE ONLY -- imported by ``tests/`` as the checker of the HIP
backward path, never by the product.

The reference has no hand-written backward: ``train.py:266`` differentiates
``MoE.__call__`` (``model/moe.py:170-294``) with ``jax.value_and_grad``.  Each
function below is the VJP of the forward lines it cites, with the routing
decisions (top-k indices, capacity drops, the dispatch plan) held fixed: they
are integer-valued and have no derivative.  Two precisions:

* ``"fp64"`` -- every operation in float64 on the given values (no bf16
  rounding): the reference value the finite-difference tests pin;
* ``"bf16"`` -- the rounding points of the compute-dtype path: bf16 weights
  (``moe.py:204-206``), the cotangents of bf16 tensors (``ys``, ``h``, ``g``,
  ``u``, ``xs``) rounded to bf16 where the forward rounded the primal, float32
  accumulation of sums over tokens and slots.

Pinning: ``tests/test_oracle_backward.py`` checks every function against
central finite differences of the float64 forward on tiny random problems
(the mathematics fixes the derivative; a dropped term, a wrong sign or a
transposed operand changes the result by O(1), far above the O(eps^2)
difference error), and the composed ``moe_backward`` against finite
differences of the whole routed layer.
"""
from __future__ import annotations

import numpy as np

from .moe_oracle import F32, F64, bf16_round

__all__ = [
    "silu64", "dsilu64", "combine_bwd", "swiglu_bwd", "expert_ffn_bwd", "gather_bwd",
    "route_softmax_bwd", "route_sigmoid_bwd", "router_bwd", "aux_bwd", "shared_bwd",
    "moe_backward", "routed_forward64", "aux_forward64", "shared_forward64",
]


def silu64(a):
    a = np.asarray(a, F64)
    return a / (1.0 + np.exp(-a))


def dsilu64(a):
    """d silu / d a = sigma(a) * (1 + a * (1 - sigma(a)))."""
    a = np.asarray(a, F64)
    s = 1.0 / (1.0 + np.exp(-a))
    return s * (1.0 + a * (1.0 - s))


def _r(a, precision):
    return bf16_round(np.asarray(a, F32)) if precision == "bf16" else np.asarray(a, F64)


# --------------------------------------------------------------------------
# combine (moe.py:80-85): y[t] = sum_k bf16(g[t,k]) * ys[pos(t,k)]
# --------------------------------------------------------------------------

def combine_bwd(dy, ys, slot_pos, gates, T: int, K: int, precision: str = "bf16"):
    """VJP of the weighted combine (``moe.py:80-85``).

    ``d_ys[pos(t,k)] = dy[t] * bf16(g[t,k])`` (the cotangent of the bf16 ``ys``:
    the float32 product rounded to bf16) and ``d_g[t,k] = sum_d dy[t,d] *
    ys[pos(t,k),d]`` (through the bf16 cast of the gates, ``:84``; rounded to
    bf16 and back, as the cast's transpose does).  Dropped slots get
    ``d_g = 0`` and no row.  Returns ``(d_ys [rows, D], d_gates [T, K])``;
    rows of ``d_ys`` that no slot maps to are zero.
    """
    dy = np.asarray(dy, F32)
    ys = np.asarray(ys, F32 if precision == "bf16" else F64)
    sp = np.asarray(slot_pos).reshape(T, K)
    g = np.asarray(gates, F32).reshape(T, K)
    g16 = bf16_round(g) if precision == "bf16" else g.astype(F64)
    d_ys = np.zeros(ys.shape, F32 if precision == "bf16" else F64)
    d_g = np.zeros((T, K), F32 if precision == "bf16" else F64)
    for k in range(K):
        p = sp[:, k]
        kept = p >= 0
        t = np.nonzero(kept)[0]
        rows = p[kept]
        if precision == "bf16":
            d_ys[rows] = bf16_round((dy[t] * g16[t, k:k + 1]).astype(F32))
            dot = (dy[t].astype(F64) * ys[rows].astype(F64)).sum(axis=1)
            d_g[t, k] = bf16_round(dot.astype(F32))
        else:
            d_ys[rows] = dy[t].astype(F64) * g16[t, k:k + 1]
            d_g[t, k] = (dy[t].astype(F64) * ys[rows]).sum(axis=1)
    return d_ys, d_g


# --------------------------------------------------------------------------
# experts (moe.py:67-74): g = xs Wg, u = xs Wu, h = silu(g) u, ys = h Wd
# --------------------------------------------------------------------------

def swiglu_bwd(dh, g, u, precision: str = "bf16"):
    """VJP of ``h = silu(g) * u`` (``moe.py:72``): ``dg = dh * u * silu'(g)``,
    ``du = dh * silu(g)``, each rounded to bf16 once in ``"bf16"`` mode."""
    dh = np.asarray(dh, F64)
    g = np.asarray(g, F64)
    u = np.asarray(u, F64)
    dg = dh * u * dsilu64(g)
    du = dh * silu64(g)
    return _r(dg, precision), _r(du, precision)


def expert_ffn_bwd(xs, offsets, wg, wu, wd, d_ys, precision: str = "bf16") -> dict:
    """VJP of the grouped SwiGLU (``moe.py:70-74``) per expert segment.

    Forward (recomputed): ``g = xs Wg[e]``, ``u = xs Wu[e]`` (bf16),
    ``h = bf16(silu(g) u)``.  Backward: ``dh = d_ys Wd[e]^T``,
    ``(dg, du) = swiglu_bwd``, ``d_xs = dg Wg[e]^T + du Wu[e]^T`` (one float32
    accumulation over the 2F columns, one rounding), ``dWd[e] = h^T d_ys``,
    ``dWg[e] = xs^T dg``, ``dWu[e] = xs^T du`` (float32 results).  Rows past
    ``offsets[-1]`` get ``d_xs = 0``.  Returns a dict with ``d_xs``, ``dh``,
    ``g``, ``u``, ``dg``, ``du``, ``h``, ``dWg``, ``dWu``, ``dWd``.
    """
    xs = np.asarray(xs, F64)
    d_ys = np.asarray(d_ys, F64)
    offsets = np.asarray(offsets, np.int64)
    N = len(offsets) - 1
    R, D = xs.shape
    F = wg.shape[2]
    cast = (lambda w: bf16_round(np.asarray(w, F32)).astype(F64)) if precision == "bf16" \
        else (lambda w: np.asarray(w, F64))
    out = {k: np.zeros((R, c), F64) for k, c in
           (("d_xs", D), ("dh", F), ("g", F), ("u", F), ("dg", F), ("du", F), ("h", F))}
    dWg = np.zeros((N, D, F), F64)
    dWu = np.zeros((N, D, F), F64)
    dWd = np.zeros((N, F, D), F64)
    for e in range(N):
        a, b = int(offsets[e]), int(offsets[e + 1])
        if b <= a:
            continue
        x = xs[a:b]
        Wg, Wu, Wd = cast(wg[e]), cast(wu[e]), cast(wd[e])
        g = _r(x @ Wg, precision).astype(F64)
        u = _r(x @ Wu, precision).astype(F64)
        h = _r(silu64(g) * u, precision).astype(F64)
        dy = d_ys[a:b]
        dh = _r(dy @ Wd.T, precision).astype(F64)
        dg, du = (v.astype(F64) for v in swiglu_bwd(dh, g, u, precision))
        dx = dg @ Wg.T + du @ Wu.T
        out["d_xs"][a:b] = _r(dx, precision)
        for k, v in (("dh", dh), ("g", g), ("u", u), ("dg", dg), ("du", du), ("h", h)):
            out[k][a:b] = v
        dWd[e] = h.T @ dy
        dWg[e] = x.T @ dg
        dWu[e] = x.T @ du
    dt = F32 if precision == "bf16" else F64
    res = {k: v.astype(dt) for k, v in out.items()}
    res.update(dWg=dWg.astype(dt), dWu=dWu.astype(dt), dWd=dWd.astype(dt))
    return res


# --------------------------------------------------------------------------
# gather (moe.py:56): xs[j] = x_flat[perm_src[j] // K]
# --------------------------------------------------------------------------

def gather_bwd(d_xs, slot_pos, T: int, K: int, precision: str = "bf16"):
    """VJP of the row gather (``moe.py:56``): ``dx[t] = sum_k d_xs[pos(t,k)]``
    over kept slots, ``k`` ascending in float32 (``"bf16"``) or float64."""
    d_xs = np.asarray(d_xs, F32 if precision == "bf16" else F64)
    sp = np.asarray(slot_pos).reshape(T, K)
    acc = np.zeros((T, d_xs.shape[1]), d_xs.dtype)
    for k in range(K):
        p = sp[:, k]
        kept = p >= 0
        rows = d_xs[np.where(kept, p, 0)]
        acc = np.where(kept[:, None], (acc + rows).astype(acc.dtype), acc)
    return acc


# --------------------------------------------------------------------------
# routing (moe.py:175-192) and the workload's softmax rule
# --------------------------------------------------------------------------

def route_softmax_bwd(logits, top_idx, gates, d_gates):
    """VJP of the softmax gates over the selected logits: ``g_k =
    exp(l_k) / sum_j exp(l_j)`` for the K selected experts, so
    ``d l_k = g_k (d g_k - sum_j g_j d g_j)``; unselected logits get 0.
    Returns ``d_logits [T, N]`` (float64)."""
    logits = np.asarray(logits, F64)
    idx = np.asarray(top_idx)
    g = np.asarray(gates, F64)
    dg = np.asarray(d_gates, F64)
    s = (g * dg).sum(axis=1, keepdims=True)
    dl_sel = g * (dg - s)
    dl = np.zeros(logits.shape, F64)
    np.put_along_axis(dl, idx, dl_sel, axis=1)
    return dl


def route_sigmoid_bwd(logits, top_idx, d_gates, rsf: float):
    """VJP of the reference gates ``g_k = rsf * s_k / (sum_j s_j + 1e-9)``,
    ``s = sigmoid(l)`` over the selected experts (``moe.py:179-192``; the bias
    only selects): ``d s_k = rsf * (d g_k / Z - sum_j d g_j s_j / Z^2)`` with
    ``Z = sum_j s_j + 1e-9``, ``d l_k = d s_k * s_k (1 - s_k)``.  Returns
    ``d_logits [T, N]`` (float64)."""
    logits = np.asarray(logits, F64)
    idx = np.asarray(top_idx)
    l_sel = np.take_along_axis(logits, idx, axis=1)
    s = 1.0 / (1.0 + np.exp(-l_sel))
    dg = np.asarray(d_gates, F64)
    Z = s.sum(axis=1, keepdims=True) + 1e-9
    ds = rsf * (dg / Z - (dg * s).sum(axis=1, keepdims=True) / Z ** 2)
    dl = np.zeros(logits.shape, F64)
    np.put_along_axis(dl, idx, ds * s * (1.0 - s), axis=1)
    return dl


def router_bwd(x, router_w, d_logits):
    """VJP of ``l = f32(x) @ router`` (``moe.py:175,178``): ``d_router =
    x^T d_l`` [D, N] and ``dx = d_l router^T`` [T, D], float64."""
    x = np.asarray(x, F64)
    w = np.asarray(router_w, F64)
    dl = np.asarray(d_logits, F64)
    return x.T @ dl, dl @ w.T


# --------------------------------------------------------------------------
# aux losses (moe.py:253-283) and the shared expert (moe.py:161-168, 249-251)
# --------------------------------------------------------------------------

def aux_forward64(logits, top_idx, B: int, S: int):
    """``(router_z_loss, balance_loss, mean_entropy)`` in float64 with the
    per-sequence expert counts taken from ``top_idx`` (``moe.py:253-283``;
    the same arithmetic as ``moe_oracle.aux_losses``, scores recomputed from
    the logits): the function :func:`aux_bwd` differentiates."""
    l = np.asarray(logits, F64)
    N = l.shape[-1]
    l = l.reshape(B, S, N)
    K = np.asarray(top_idx).shape[-1]
    m = l.max(axis=-1, keepdims=True)
    lse = (m + np.log(np.exp(l - m).sum(axis=-1, keepdims=True)))[..., 0]
    idx = np.asarray(top_idx).reshape(B, S * K)
    counts = np.stack([np.bincount(idx[b], minlength=N) for b in range(B)]).astype(F64)
    s = 1.0 / (1.0 + np.exp(-l))
    p = s / (s.sum(axis=-1, keepdims=True) + 1e-9)
    bal = np.mean(N * np.sum(counts / (S * K) * p.mean(axis=1), axis=-1))
    ent = np.mean(-np.sum(p * np.log(p + 1e-9), axis=-1))
    return float(np.mean(lse ** 2)), float(bal), float(ent)


def aux_bwd(logits, top_idx, B: int, S: int, d_z: float, d_bal: float, d_ent: float = 0.0):
    """VJP of the aux losses with respect to the router logits, for the
    cotangents ``d_z``, ``d_bal``, ``d_ent`` of ``router_z_loss``,
    ``balance_loss`` and ``mean_entropy`` (``moe.py:253-283``).  The expert
    counts come from the top-k indices and carry no derivative.  With
    ``T = B*S``, ``q = softmax(l)``, ``s = sigmoid(l)``, ``Z = sum s + 1e-9``,
    ``p = s / Z`` and ``f[b,n] = counts[b,n] / (S*K)``:

    * z-loss: ``dl += d_z * 2 lse / T * q``;
    * ``dp = d_bal * N f[b] / (B*S) - d_ent * (log(p + 1e-9) + p / (p + 1e-9)) / T``;
    * through ``p = s / Z``: ``ds = dp / Z - sum(dp s) / Z^2``, ``dl += ds s (1 - s)``.

    Returns ``d_logits [T, N]`` float64.
    """
    l = np.asarray(logits, F64)
    N = l.shape[-1]
    T = B * S
    l = l.reshape(B, S, N)
    K = np.asarray(top_idx).shape[-1]
    m = l.max(axis=-1, keepdims=True)
    e = np.exp(l - m)
    se = e.sum(axis=-1, keepdims=True)
    lse = m + np.log(se)
    dl = d_z * 2.0 * lse / T * (e / se)
    idx = np.asarray(top_idx).reshape(B, S * K)
    counts = np.stack([np.bincount(idx[b], minlength=N) for b in range(B)]).astype(F64)
    s = 1.0 / (1.0 + np.exp(-l))
    Z = s.sum(axis=-1, keepdims=True) + 1e-9
    p = s / Z
    dp = d_bal * N * (counts / (S * K))[:, None, :] / (B * S)
    dp = dp - d_ent * (np.log(p + 1e-9) + p / (p + 1e-9)) / T
    ds = dp / Z - (dp * s).sum(axis=-1, keepdims=True) / Z ** 2
    dl = dl + ds * s * (1.0 - s)
    return dl.reshape(T, N)


def shared_forward64(x, w_gate, w_up, w_down, n_shared: int):
    """``_shared_ffn`` (``moe.py:161-168``) in float64: one SwiGLU for 2-D
    weights, the mean of ``n_shared`` SwiGLUs for 3-D ones."""
    x = np.asarray(x, F64)
    if n_shared == 1:
        w_gate, w_up, w_down = (np.asarray(w, F64)[None] for w in (w_gate, w_up, w_down))
    out = 0.0
    for i in range(n_shared):
        g = x @ np.asarray(w_gate[i], F64)
        u = x @ np.asarray(w_up[i], F64)
        out = out + (silu64(g) * u) @ np.asarray(w_down[i], F64)
    return out / n_shared


def shared_bwd(x, w_gate, w_up, w_down, n_shared: int, dy, precision: str = "bf16",
               promoted: bool = False) -> dict:
    """VJP of the shared expert(s) (``moe.py:161-168``, added with weight 1 at
    ``:249-251``) for the float32 cotangent ``dy`` of the layer output.

    Each SwiGLU returns ``f32(bf16 out)`` (``moe.py:23-29``), so its output
    cotangent is ``bf16(dy / n_shared)``; the rest is :func:`expert_ffn_bwd`
    with one segment holding every token.  Returns ``dx [T, D]`` and
    ``dWg``, ``dWu``, ``dWd`` in the parameter shapes (2-D for one shared
    expert, stacked for several), plus ``d_out`` (the per-expert cotangent).

    ``promoted``: a float32 ``x`` under bf16 compute, whose SwiGLUs ran in
    float32 on the bf16-rounded weights (``moe.py:249`` passes ``x`` as
    given): the output cotangent is ``dy / n_shared`` (float32 outputs, no
    cast), the VJP is the float32 one on ``bf16(w)``, and the master
    gradients pass through bf16 (the VJP of ``w.astype(bf16)``).
    """
    x = np.asarray(x)
    T = x.shape[0]
    if promoted:
        d_out = np.asarray(dy, F32) / F32(n_shared)
        stack = n_shared > 1
        ws = [(w_gate[i], w_up[i], w_down[i]) for i in range(n_shared)] if stack \
            else [(w_gate, w_up, w_down)]
        dx = np.zeros(x.shape, F64)
        grads = {"dWg": [], "dWu": [], "dWd": []}
        for wg_, wu_, wd_ in ws:
            r = expert_ffn_bwd(x, np.array([0, T]), bf16_round(np.asarray(wg_, F32))[None],
                               bf16_round(np.asarray(wu_, F32))[None],
                               bf16_round(np.asarray(wd_, F32))[None], d_out, "fp32")
            dx = dx + r["d_xs"]
            for k in grads:
                grads[k].append(bf16_round(np.asarray(r[k][0], F32)))
        res = {k: (np.stack(v) if stack else v[0]).astype(F32) for k, v in grads.items()}
        res["dx"] = dx.astype(F32)
        res["d_out"] = d_out
        return res
    dy = np.asarray(dy, F32 if precision == "bf16" else F64)
    d_out = _r(dy / dy.dtype.type(n_shared), precision)
    stack = n_shared > 1
    ws = [(w_gate[i], w_up[i], w_down[i]) for i in range(n_shared)] if stack \
        else [(w_gate, w_up, w_down)]
    dx = np.zeros(x.shape, F64)
    grads = {"dWg": [], "dWu": [], "dWd": []}
    for wg_, wu_, wd_ in ws:
        r = expert_ffn_bwd(x, np.array([0, T]), np.asarray(wg_)[None], np.asarray(wu_)[None],
                           np.asarray(wd_)[None], d_out, precision)
        dx = dx + r["d_xs"]
        for k in grads:
            grads[k].append(r[k][0])
    dt = F32 if precision == "bf16" else F64
    res = {k: (np.stack(v) if stack else v[0]).astype(dt) for k, v in grads.items()}
    res["dx"] = dx.astype(dt)
    res["d_out"] = d_out
    return res


# --------------------------------------------------------------------------
# composed routed layer
# --------------------------------------------------------------------------

def routed_forward64(x, router_w, wg, wu, wd, top_idx, slot_pos, perm_src, offsets, *,
                     routing: str = "softmax", rsf: float = 1.0):
    """The routed layer output in float64 with the routing decisions given
    (``moe.py:175-192`` gates, ``:56`` gather, ``:70-74`` experts, ``:80-85``
    combine): the function :func:`moe_backward` differentiates, for the
    finite-difference checks."""
    x = np.asarray(x, F64)
    T = x.shape[0]
    K = np.asarray(top_idx).shape[1]
    logits = x @ np.asarray(router_w, F64)
    l_sel = np.take_along_axis(logits, np.asarray(top_idx), axis=1)
    if routing == "softmax":
        e = np.exp(l_sel - l_sel.max(axis=1, keepdims=True))
        gates = e / e.sum(axis=1, keepdims=True)
    else:
        s = 1.0 / (1.0 + np.exp(-l_sel))
        gates = rsf * s / (s.sum(axis=1, keepdims=True) + 1e-9)
    perm = np.asarray(perm_src)
    xs = np.zeros((perm.size, x.shape[1]), F64)
    valid = perm >= 0
    xs[valid] = x[perm[valid] // K]
    offsets = np.asarray(offsets, np.int64)
    ys = np.zeros((perm.size, np.asarray(wd).shape[2]), F64)
    for ex in range(len(offsets) - 1):
        a, b = int(offsets[ex]), int(offsets[ex + 1])
        if b > a:
            g = xs[a:b] @ np.asarray(wg[ex], F64)
            u = xs[a:b] @ np.asarray(wu[ex], F64)
            ys[a:b] = (silu64(g) * u) @ np.asarray(wd[ex], F64)
    sp = np.asarray(slot_pos).reshape(T, K)
    y = np.zeros((T, ys.shape[1]), F64)
    for k in range(K):
        kept = sp[:, k] >= 0
        y[kept] += gates[kept, k:k + 1] * ys[sp[kept, k]]
    return y


def moe_backward(x, params: dict, dy, fwd: dict, *, routing: str = "softmax",
                 rsf: float = 1.0, precision: str = "bf16", n_shared: int = 0,
                 batch_shape=None, d_aux=None, x_dtype: str | None = None) -> dict:
    """VJP of the MoE layer (``moe.py:170-294``) for the cotangent ``dy`` of
    ``out`` and, optionally, ``d_aux = (d_z, d_bal, d_ent)`` of the aux losses
    (with ``batch_shape = (B, S)``; ``:253-283``).

    ``fwd`` is :func:`moe_oracle.moe_forward`'s result (logits, top_idx,
    gates, plan, xs, ys).  ``n_shared > 0`` adds the shared expert's VJP
    (``params["shared_w_*"]``).  Returns ``dx [T, D]`` (experts + router +
    shared), ``d_router [D, N]``, ``dWg``, ``dWu [N, D, F]``, ``dWd [N, F, D]``,
    ``dWg_shared``/``dWu_shared``/``dWd_shared`` when there is a shared expert,
    and the intermediates ``d_ys``, ``d_gates``, ``d_logits``, ``d_xs``,
    ``dx_experts``, ``dx_router``.  ``x_dtype`` is the dtype ``x`` arrived in
    (``"f32"`` under bf16 compute promotes the shared expert, as in
    :func:`moe_oracle.moe_forward`; default: the compute dtype).
    """
    if x_dtype not in (None, "bf16", "f32"):
        raise ValueError(x_dtype)
    x = np.asarray(x, F32)
    T = x.shape[0]
    K = np.asarray(fwd["top_idx"]).shape[1]
    plan = fwd["plan"]
    ys = fwd["ys"]
    d_ys, d_g = combine_bwd(dy, ys, plan["slot_pos"], fwd["gates"], T, K, precision)
    ex = expert_ffn_bwd(fwd["xs"], plan["offsets"], params["expert_w_gate"],
                        params["expert_w_up"], params["expert_w_down"], d_ys, precision)
    dx_e = gather_bwd(ex["d_xs"], plan["slot_pos"], T, K, precision)
    if routing == "softmax":
        dl = route_softmax_bwd(fwd["logits"], fwd["top_idx"], fwd["gates"], d_g)
    else:
        dl = route_sigmoid_bwd(fwd["logits"], fwd["top_idx"], d_g, rsf)
    if d_aux is not None:
        B, S = batch_shape
        dl = dl + aux_bwd(fwd["logits"], fwd["top_idx"], B, S, *d_aux)
    d_router, dx_r = router_bwd(x, params["router"], dl)
    dt = F32 if precision == "bf16" else F64
    dx = np.asarray(dx_e, F64) + dx_r
    res = {}
    if n_shared > 0:
        xc = bf16_round(x) if precision == "bf16" else x
        # a float32 x under bf16 compute reaches the shared expert as given
        # (moe.py:249); decided by x's dtype, never by its values
        promoted = precision == "bf16" and x_dtype == "f32"
        sh = shared_bwd(x if promoted else xc, params["shared_w_gate"], params["shared_w_up"],
                        params["shared_w_down"], n_shared, dy, precision, promoted=promoted)
        dx = dx + sh["dx"]
        res = {"dWg_shared": sh["dWg"], "dWu_shared": sh["dWu"], "dWd_shared": sh["dWd"],
               "dx_shared": sh["dx"], "d_shared_out": sh["d_out"]}
    res.update({"dx": dx.astype(dt), "d_router": d_router.astype(dt),
                "dWg": ex["dWg"], "dWu": ex["dWu"], "dWd": ex["dWd"], "d_ys": d_ys,
                "d_gates": d_g, "d_logits": dl.astype(dt), "d_xs": ex["d_xs"],
                "dx_experts": dx_e, "dx_router": dx_r.astype(dt), "expert": ex})
    return res
