"""Pins the backward oracle (``oracle/moe_backward.py``) to the mathematics.

The reference has no backward code and JAX is absent, so every VJP is checked
against central finite differences of the float64 forward it differentiates,
on tiny random problems, along random directions: ``<grad, v>`` must equal
``(f(p + eps v) - f(p - eps v)) / (2 eps)`` to O(eps^2).  A dropped term, a
wrong sign or a transposed operand moves the directional derivative by O(1).
"""
import numpy as np
import pytest

import oracle as O
from oracle import moe_backward as B

EPS = 1e-5


def fd(f, p, v):
    return (f(p + EPS * v) - f(p - EPS * v)) / (2 * EPS)


def close(a, b, rtol=1e-6):
    a, b = float(a), float(b)
    assert abs(a - b) <= rtol * max(1.0, abs(a), abs(b)), (a, b)


def tiny_problem(seed, T=12, D=16, N=5, K=2, F=8, cf=None):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, D))
    w = 0.3 * rng.standard_normal((D, N))
    wg = 0.3 * rng.standard_normal((N, D, F))
    wu = 0.3 * rng.standard_normal((N, D, F))
    wd = 0.3 * rng.standard_normal((N, F, D))
    logits = x @ w
    idx = O.topk_desc(logits.astype(np.float32), K)
    C = O.capacity_of(T, K, N, cf)
    plan = O.dispatch_plan(idx, N, C)
    return rng, x, w, wg, wu, wd, idx, plan


def test_silu_derivative():
    a = np.linspace(-6, 6, 101)
    v = np.ones_like(a)
    np.testing.assert_allclose(B.dsilu64(a), fd(B.silu64, a, v), rtol=1e-8, atol=1e-10)


def test_swiglu_bwd():
    rng = np.random.default_rng(1)
    g, u, dh = rng.standard_normal((3, 7, 9))
    dg, du = B.swiglu_bwd(dh, g, u, "fp64")
    vg, vu = rng.standard_normal((2, 7, 9))
    close((dg * vg).sum(), fd(lambda p: (dh * B.silu64(p) * u).sum(), g, vg))
    close((du * vu).sum(), fd(lambda p: (dh * B.silu64(g) * p).sum(), u, vu))


def test_combine_bwd():
    rng, x, w, wg, wu, wd, idx, plan = tiny_problem(2, cf=0.8)   # with drops
    T, K = idx.shape
    R = plan["perm_src"].size
    ys = rng.standard_normal((R, 6))
    gates = rng.uniform(0.1, 1.0, (T, K))
    dy = rng.standard_normal((T, 6))
    sp = plan["slot_pos"].reshape(T, K)
    assert (sp < 0).any()

    def y(ys_, g_):
        out = np.zeros((T, 6))
        for k in range(K):
            kept = sp[:, k] >= 0
            out[kept] += g_[kept, k:k + 1] * ys_[sp[kept, k]]
        return out

    d_ys, d_g = B.combine_bwd(dy, ys, plan["slot_pos"], gates, T, K, "fp64")
    v = rng.standard_normal(ys.shape)
    close((d_ys * v).sum(), fd(lambda p: (dy * y(p, gates)).sum(), ys, v))
    vg = rng.standard_normal(gates.shape)
    close((d_g * vg).sum(), fd(lambda p: (dy * y(ys, p)).sum(), gates, vg))
    assert np.all(d_g[sp < 0] == 0)


def test_expert_ffn_bwd():
    rng, x, w, wg, wu, wd, idx, plan = tiny_problem(3)
    R = plan["perm_src"].size
    xs = O.permute_rows(x, plan["perm_src"], idx.shape[1])
    d_ys = rng.standard_normal((R, x.shape[1]))
    off = plan["offsets"]
    r = B.expert_ffn_bwd(xs, off, wg, wu, wd, d_ys, "fp64")

    def L(xs_, wg_, wu_, wd_):
        ys = np.zeros_like(d_ys)
        for e in range(len(off) - 1):
            a, b = off[e], off[e + 1]
            g = xs_[a:b] @ wg_[e]
            u = xs_[a:b] @ wu_[e]
            ys[a:b] = (B.silu64(g) * u) @ wd_[e]
        return (d_ys * ys).sum()

    v = rng.standard_normal(xs.shape)
    close((r["d_xs"] * v).sum(), fd(lambda p: L(p, wg, wu, wd), xs, v))
    for name, arr, pos in (("dWg", wg, 1), ("dWu", wu, 2), ("dWd", wd, 3)):
        v = rng.standard_normal(arr.shape)
        args = [xs, wg, wu, wd]

        def f(p, pos=pos):
            a = list(args)
            a[pos] = p
            return L(*a)

        close((r[name] * v).sum(), fd(f, arr, v))


def test_gather_bwd():
    rng, x, w, wg, wu, wd, idx, plan = tiny_problem(4, cf=0.8)
    T, K = idx.shape
    R = plan["perm_src"].size
    d_xs = rng.standard_normal((R, x.shape[1]))
    dx = B.gather_bwd(d_xs, plan["slot_pos"], T, K, "fp64")
    v = rng.standard_normal(x.shape)
    close((dx * v).sum(), fd(lambda p: (d_xs * O.permute_rows(p, plan["perm_src"], K)).sum(), x, v))


@pytest.mark.parametrize("routing", ["softmax", "sigmoid"])
def test_route_bwd(routing):
    rng = np.random.default_rng(5)
    T, N, K, rsf = 9, 7, 3, 2.5
    logits = rng.standard_normal((T, N))
    idx = O.topk_desc(logits.astype(np.float32), K)
    dg = rng.standard_normal((T, K))

    def gates(l):
        sel = np.take_along_axis(l, idx, axis=1)
        if routing == "softmax":
            e = np.exp(sel - sel.max(axis=1, keepdims=True))
            return e / e.sum(axis=1, keepdims=True)
        s = 1.0 / (1.0 + np.exp(-sel))
        return rsf * s / (s.sum(axis=1, keepdims=True) + 1e-9)

    if routing == "softmax":
        dl = B.route_softmax_bwd(logits, idx, gates(logits), dg)
    else:
        dl = B.route_sigmoid_bwd(logits, idx, dg, rsf)
    v = rng.standard_normal(logits.shape)
    close((dl * v).sum(), fd(lambda p: (dg * gates(p)).sum(), logits, v))
    unsel = np.ones((T, N), bool)
    np.put_along_axis(unsel, idx, False, axis=1)
    assert np.all(dl[unsel] == 0)


@pytest.mark.parametrize("routing,cf", [("softmax", None), ("softmax", 0.8), ("sigmoid", 1.0)])
def test_moe_backward_whole_layer(routing, cf):
    rng, x, w, wg, wu, wd, idx, plan = tiny_problem(6, cf=cf)
    T, K = idx.shape
    rsf = 2.5 if routing == "sigmoid" else 1.0
    args = dict(top_idx=idx, slot_pos=plan["slot_pos"], perm_src=plan["perm_src"],
                offsets=plan["offsets"], routing=routing, rsf=rsf)
    dy = rng.standard_normal((T, x.shape[1]))
    logits = x @ w
    sel = np.take_along_axis(logits, idx, axis=1)
    if routing == "softmax":
        e = np.exp(sel - sel.max(axis=1, keepdims=True))
        gates = e / e.sum(axis=1, keepdims=True)
    else:
        s = 1.0 / (1.0 + np.exp(-sel))
        gates = rsf * s / (s.sum(axis=1, keepdims=True) + 1e-9)
    xs = O.permute_rows(x, plan["perm_src"], K)
    ys = np.zeros((xs.shape[0], x.shape[1]))
    off = plan["offsets"]
    for ex in range(len(off) - 1):
        a, b = off[ex], off[ex + 1]
        ys[a:b] = (B.silu64(xs[a:b] @ wg[ex]) * (xs[a:b] @ wu[ex])) @ wd[ex]
    fwd = {"logits": logits, "top_idx": idx, "gates": gates, "plan": plan, "xs": xs, "ys": ys}
    params = {"router": w, "expert_w_gate": wg, "expert_w_up": wu, "expert_w_down": wd}
    g = B.moe_backward(x, params, dy, fwd, routing=routing, rsf=rsf, precision="fp64")
    # the differentiated function is the forward the fwd dict holds
    sp = plan["slot_pos"].reshape(T, K)
    y_ref = np.zeros((T, x.shape[1]))
    for k in range(K):
        kept = sp[:, k] >= 0
        y_ref[kept] += gates[kept, k:k + 1] * ys[sp[kept, k]]
    np.testing.assert_allclose(B.routed_forward64(x, w, wg, wu, wd, **args), y_ref, rtol=1e-12)

    def L(x_, w_, wg_, wu_, wd_):
        return (dy * B.routed_forward64(x_, w_, wg_, wu_, wd_, **args)).sum()

    base = [x, w, wg, wu, wd]
    for name, pos in (("dx", 0), ("d_router", 1), ("dWg", 2), ("dWu", 3), ("dWd", 4)):
        v = rng.standard_normal(base[pos].shape)

        def f(p, pos=pos):
            a = list(base)
            a[pos] = p
            return L(*a)

        close((g[name] * v).sum(), fd(f, base[pos], v), rtol=1e-5)


def test_bf16_mode_tracks_fp64():
    """The bf16-rounded backward stays within bf16 accuracy of the float64 one."""
    rng, x, w, wg, wu, wd, idx, plan = tiny_problem(7, T=64, D=64, N=4, K=2, F=32)
    T, K = idx.shape
    x = O.bf16_round(x.astype(np.float32))
    fwd = O.moe_forward(x, {"router": w.astype(np.float32), "expert_w_gate": wg.astype(np.float32),
                            "expert_w_up": wu.astype(np.float32),
                            "expert_w_down": wd.astype(np.float32)},
                        top_k=K, routing="softmax", dtype="bf16", precision="bf16")
    dy = rng.standard_normal((T, x.shape[1])).astype(np.float32)
    params = {"router": w, "expert_w_gate": wg, "expert_w_up": wu, "expert_w_down": wd}
    g16 = B.moe_backward(x, params, dy, fwd, routing="softmax", precision="bf16")
    g64 = B.moe_backward(x, params, dy, fwd, routing="softmax", precision="fp64")
    for k in ("dx", "d_router", "dWg", "dWu", "dWd", "d_gates"):
        assert O.normwise_rel_err(np.asarray(g16[k], np.float64), np.asarray(g64[k], np.float64)) < 2e-2, k


def test_aux_bwd():
    """All three aux terms, two sequences, counts from fixed top-k indices."""
    rng = np.random.default_rng(8)
    Bq, Sq, N, K = 2, 6, 7, 3
    logits = 1.5 * rng.standard_normal((Bq * Sq, N))
    idx = O.topk_desc(logits.astype(np.float32), K)
    d_z, d_bal, d_ent = 0.7, -1.3, 0.4
    dl = B.aux_bwd(logits, idx, Bq, Sq, d_z, d_bal, d_ent)

    def f(p):
        z, bal, ent = B.aux_forward64(p, idx, Bq, Sq)
        return d_z * z + d_bal * bal + d_ent * ent

    for _ in range(3):
        v = rng.standard_normal(logits.shape)
        close((dl * v).sum(), fd(f, logits, v))
    # each term alone (a dropped term shows here even if the others cancel it)
    for dz_, db_, de_ in ((1.0, 0.0, 0.0), (0.0, 1.0, 0.0), (0.0, 0.0, 1.0)):
        dl1 = B.aux_bwd(logits, idx, Bq, Sq, dz_, db_, de_)
        v = rng.standard_normal(logits.shape)

        def f1(p):
            z, bal, ent = B.aux_forward64(p, idx, Bq, Sq)
            return dz_ * z + db_ * bal + de_ * ent

        close((dl1 * v).sum(), fd(f1, logits, v))


def test_aux_forward64_matches_forward_oracle():
    rng = np.random.default_rng(9)
    Bq, Sq, N, K = 3, 5, 6, 2
    logits = rng.standard_normal((Bq * Sq, N)).astype(np.float32)
    idx = O.topk_desc(logits, K)
    scores = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    ref = O.aux_losses(logits, scores, idx, Bq, Sq, N)
    z, bal, ent = B.aux_forward64(logits, idx, Bq, Sq)
    np.testing.assert_allclose([z, bal, ent],
                               [ref["router_z_loss"], ref["balance_loss"], ref["mean_entropy"]],
                               rtol=1e-12)


@pytest.mark.parametrize("n_shared", [1, 3])
def test_shared_bwd(n_shared):
    rng = np.random.default_rng(10 + n_shared)
    T, D, F = 7, 12, 10
    x = rng.standard_normal((T, D))
    shape = (lambda *s: s) if n_shared == 1 else (lambda *s: (n_shared,) + s)
    wg = 0.3 * rng.standard_normal(shape(D, F))
    wu = 0.3 * rng.standard_normal(shape(D, F))
    wd = 0.3 * rng.standard_normal(shape(F, D))
    dy = rng.standard_normal((T, D))
    r = B.shared_bwd(x, wg, wu, wd, n_shared, dy, "fp64")
    base = [x, wg, wu, wd]
    for name, pos in (("dx", 0), ("dWg", 1), ("dWu", 2), ("dWd", 3)):
        assert r[name].shape == base[pos].shape
        v = rng.standard_normal(base[pos].shape)

        def f(p, pos=pos):
            a = list(base)
            a[pos] = p
            return (dy * B.shared_forward64(*a, n_shared)).sum()

        close((r[name] * v).sum(), fd(f, base[pos], v))


@pytest.mark.parametrize("n_shared", [1, 2])
def test_shared_bwd_promoted(n_shared):
    """The shared expert of a float32 x under bf16 compute (moe.py:249: a
    float32 SwiGLU on bf16(w)): dx against finite differences of the float64
    forward on the rounded weights; the master gradients against the same
    differences with respect to the rounded weights, to bf16 accuracy (they
    pass through bf16, the VJP of w.astype(bf16))."""
    rng = np.random.default_rng(30 + n_shared)
    T, D, F = 7, 12, 10
    x = rng.standard_normal((T, D)).astype(np.float32)
    shape = (lambda *s: s) if n_shared == 1 else (lambda *s: (n_shared,) + s)
    wg = (0.3 * rng.standard_normal(shape(D, F))).astype(np.float32)
    wu = (0.3 * rng.standard_normal(shape(D, F))).astype(np.float32)
    wd = (0.3 * rng.standard_normal(shape(F, D))).astype(np.float32)
    dy = rng.standard_normal((T, D)).astype(np.float32)
    r = B.shared_bwd(x, wg, wu, wd, n_shared, dy, "bf16", promoted=True)
    assert np.array_equal(r["d_out"], dy / np.float32(n_shared))
    base = [x.astype(np.float64)] + [O.bf16_round(w).astype(np.float64) for w in (wg, wu, wd)]
    for name, pos, rtol in (("dx", 0, 1e-5), ("dWg", 1, None), ("dWu", 2, None), ("dWd", 3, None)):
        assert r[name].shape == base[pos].shape
        if pos > 0:
            assert np.array_equal(O.bf16_round(r[name]), r[name])
        v = rng.standard_normal(base[pos].shape)

        def f(p, pos=pos):
            a = list(base)
            a[pos] = p
            return (dy * B.shared_forward64(*a, n_shared)).sum()

        terms = r[name].astype(np.float64) * v
        if pos == 0:
            close(terms.sum(), fd(f, base[pos], v), rtol)
        else:
            # bf16 rounding moves each term by at most 2^-8 of itself
            assert abs(terms.sum() - fd(f, base[pos], v)) <= 2.0 ** -8 * np.abs(terms).sum()


def test_shared_forward64_matches_forward_oracle():
    rng = np.random.default_rng(12)
    T, D, F = 5, 8, 6
    x = rng.standard_normal((T, D)).astype(np.float32)
    w = [0.3 * rng.standard_normal(s) for s in ((2, D, F), (2, D, F), (2, F, D))]
    np.testing.assert_allclose(B.shared_forward64(x, *w, 2),
                               O.shared_expert(x, *w, 2, precision="fp32"), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("n_shared", [1, 2])
def test_moe_backward_module_with_shared_and_aux(n_shared):
    """The whole module (routed + shared + aux losses, reference sigmoid
    routing, two sequences) against finite differences of its float64
    forward with the routing held fixed."""
    rng, x, w, wg, wu, wd, idx, plan = tiny_problem(13, T=12, cf=0.8)
    T, K = idx.shape
    D, F = x.shape[1], wg.shape[2]
    Bq, Sq = 2, 6
    rsf = 2.5
    shp = (lambda *s: s) if n_shared == 1 else (lambda *s: (n_shared,) + s)
    swg = 0.3 * rng.standard_normal(shp(D, F))
    swu = 0.3 * rng.standard_normal(shp(D, F))
    swd = 0.3 * rng.standard_normal(shp(F, D))
    args = dict(top_idx=idx, slot_pos=plan["slot_pos"], perm_src=plan["perm_src"],
                offsets=plan["offsets"], routing="sigmoid", rsf=rsf)
    dy = rng.standard_normal((T, D))
    d_aux = (0.3, 0.8, -0.5)
    logits = x @ w
    sel = np.take_along_axis(logits, idx, axis=1)
    s = 1.0 / (1.0 + np.exp(-sel))
    gates = rsf * s / (s.sum(axis=1, keepdims=True) + 1e-9)
    xs = O.permute_rows(x, plan["perm_src"], K)
    ys = np.zeros((xs.shape[0], D))
    off = plan["offsets"]
    for ex in range(len(off) - 1):
        a, b = off[ex], off[ex + 1]
        ys[a:b] = (B.silu64(xs[a:b] @ wg[ex]) * (xs[a:b] @ wu[ex])) @ wd[ex]
    fwd = {"logits": logits, "top_idx": idx, "gates": gates, "plan": plan, "xs": xs, "ys": ys}
    params = {"router": w, "expert_w_gate": wg, "expert_w_up": wu, "expert_w_down": wd,
              "shared_w_gate": swg, "shared_w_up": swu, "shared_w_down": swd}
    g = B.moe_backward(x, params, dy, fwd, routing="sigmoid", rsf=rsf, precision="fp64",
                       n_shared=n_shared, batch_shape=(Bq, Sq), d_aux=d_aux)

    def L(x_, w_, wg_, wu_, wd_, swg_, swu_, swd_):
        out = B.routed_forward64(x_, w_, wg_, wu_, wd_, **args) \
            + B.shared_forward64(x_, swg_, swu_, swd_, n_shared)
        z, bal, ent = B.aux_forward64(x_ @ w_, idx, Bq, Sq)
        return (dy * out).sum() + d_aux[0] * z + d_aux[1] * bal + d_aux[2] * ent

    base = [x, w, wg, wu, wd, swg, swu, swd]
    names = ("dx", "d_router", "dWg", "dWu", "dWd", "dWg_shared", "dWu_shared", "dWd_shared")
    for pos, name in enumerate(names):
        assert g[name].shape == base[pos].shape, name
        v = rng.standard_normal(base[pos].shape)

        def f(p, pos=pos):
            a = list(base)
            a[pos] = p
            return L(*a)

        close((g[name] * v).sum(), fd(f, base[pos], v), rtol=1e-5)


def test_moe_backward_promotion_follows_x_dtype():
    """moe_backward takes the shared expert's promoted VJP for a float32 x
    (x_dtype="f32") even when every value of x is bf16-exact, and the bf16
    VJP for the same values declared bf16 (the default): the choice follows
    the dtype moe.py:249 sees, not the values."""
    rng = np.random.default_rng(91)
    T, D, F, N, K = 24, 16, 12, 4, 2
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    params = {"router": (0.2 * rng.standard_normal((D, N))).astype(np.float32),
              "expert_w_gate": (0.2 * rng.standard_normal((N, D, F))).astype(np.float32),
              "expert_w_up": (0.2 * rng.standard_normal((N, D, F))).astype(np.float32),
              "expert_w_down": (0.2 * rng.standard_normal((N, F, D))).astype(np.float32),
              "shared_w_gate": (0.2 * rng.standard_normal((D, F))).astype(np.float32),
              "shared_w_up": (0.2 * rng.standard_normal((D, F))).astype(np.float32),
              "shared_w_down": (0.2 * rng.standard_normal((F, D))).astype(np.float32)}
    dy = rng.standard_normal((T, D)).astype(np.float32)
    fwd = O.moe_forward(x, params, top_k=K, routing="softmax", dtype="bf16", precision="bf16")
    sw = (params["shared_w_gate"], params["shared_w_up"], params["shared_w_down"], 1, dy, "bf16")
    want_p = B.shared_bwd(x, *sw, promoted=True)
    want_b = B.shared_bwd(x, *sw, promoted=False)
    assert not np.array_equal(want_p["dWd"], want_b["dWd"])
    got_p = B.moe_backward(x, params, dy, fwd, precision="bf16", n_shared=1, x_dtype="f32")
    got_b = B.moe_backward(x, params, dy, fwd, precision="bf16", n_shared=1)
    for k in ("dWg", "dWu", "dWd", "dx"):
        assert np.array_equal(got_p[k + "_shared"] if k != "dx" else got_p["dx_shared"], want_p[k])
        assert np.array_equal(got_b[k + "_shared"] if k != "dx" else got_b["dx_shared"], want_b[k])
    with pytest.raises(ValueError):
        B.moe_backward(x, params, dy, fwd, precision="bf16", n_shared=1, x_dtype="fp16")
