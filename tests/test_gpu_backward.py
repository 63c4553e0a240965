"""Parity of the HIP backward against the backward oracle (needs an MI355X).

The combine VJP's bf16 cotangent rows and the gather VJP are compared bit for
bit (their rounding points are fixed: one float32 product, one bf16
rounding; float32 sums over k ascending).  Values that come out of a dot
product and are then rounded to bf16 (d_gates) may sit on a bf16 rounding
boundary that a different float64 summation order crosses: at most one bf16
ulp apart, and nearly all equal.  The GEMMs are compared with float64 on the
same bf16 operands (normwise 1e-2: bf16 output rounding is 2^-9 relative);
elementwise float32 arithmetic (SwiGLU VJP, router VJP) against the float64
oracle to the stated tolerances.
"""
import numpy as np
import pytest
import torch

import oracle as O
from oracle import moe_backward as B
from hanuman_amd import _lib
from hanuman_amd import kernels as K
from hanuman_amd.backward import BackwardOperands, moe_backward_data, moe_backward_weights
from hanuman_amd.moe import MoE

pytestmark = pytest.mark.gpu


def dev_f32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def dev_bf16(a, dev):
    return dev_f32(a, dev).to(torch.bfloat16)


def host(t):
    return t.float().cpu().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()


def bf16_ulps(a, b):
    """Distance in bf16 ulps between bf16-valued float32 arrays (-0 == +0)."""
    def key(v):
        i = (np.ascontiguousarray(v, np.float32).view(np.int32) >> 16).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFF), i)
    return np.abs(key(a) - key(b))


def plan_on(gpu, rng, T, N, Kk, cf):
    logits = rng.standard_normal((T, N)).astype(np.float32)
    idx = O.topk_desc(logits, Kk)
    cap = O.capacity_of(T, Kk, N, cf)
    plan = K.dispatch_plan(torch.from_numpy(idx).to(gpu), N, cap)
    return idx, plan, O.dispatch_plan(idx, N, cap)


@pytest.mark.parametrize("T,D,N,Kk,cf", [(1000, 256, 8, 4, 1.0), (513, 2048, 64, 8, 1.25),
                                         (64, 64, 4, 1, None)])
def test_combine_bwd(gpu, T, D, N, Kk, cf):
    rng = np.random.default_rng(T + D)
    idx, plan, ref_plan = plan_on(gpu, rng, T, N, Kk, cf)
    R = plan.rows_cap
    ys = O.bf16_round(rng.standard_normal((R, D)).astype(np.float32))
    gates = rng.uniform(0.0, 1.0, (T, Kk)).astype(np.float32)
    dy = rng.standard_normal((T, D)).astype(np.float32)
    n_sh = 0 if Kk == 1 else (1 if Kk == 4 else 3)
    d_ys, d_g, d_sh = K.combine_bwd(dev_f32(dy, gpu), dev_bf16(ys, gpu), plan, dev_f32(gates, gpu),
                                    n_shared=n_sh)
    torch.cuda.synchronize()
    if n_sh == 0:
        assert d_sh is None
    else:
        # the shared expert's output cotangent, bf16(dy / n_shared), bit for bit
        ref_sh = O.bf16_round((dy / np.float32(n_sh)).astype(np.float32))
        assert np.array_equal(host(d_sh).view(np.uint32), ref_sh.view(np.uint32)), "d_shared"
    r_ys, r_g = B.combine_bwd(dy, ys, ref_plan["slot_pos"], gates, T, Kk, "bf16")
    kept = int(ref_plan["offsets"][-1])
    got = host(d_ys)[:kept]
    assert np.array_equal(got.view(np.uint32), r_ys[:kept].view(np.uint32)), "d_ys rows"
    g = host(d_g)
    dropped = ref_plan["slot_pos"].reshape(T, Kk) < 0
    assert np.all(g[dropped] == 0.0)
    ulps = bf16_ulps(g, r_g)
    assert ulps.max() <= 1 and (ulps > 0).mean() < 0.01, (ulps.max(), (ulps > 0).mean())


@pytest.mark.parametrize("rows,F,kept", [(300, 256, 250), (1024, 1024, 1024), (96, 32, 70)])
def test_swiglu_bwd(gpu, rows, F, kept):
    rng = np.random.default_rng(rows + F)
    dh = O.bf16_round((rng.standard_normal((rows, F)) * 0.5).astype(np.float32))
    gu = O.bf16_round((rng.standard_normal((rows, 2 * F)) * 2.0).astype(np.float32))
    offsets = torch.tensor([0, kept // 2, kept], dtype=torch.int32, device=gpu)
    dgu = host(K.swiglu_bwd(dev_bf16(dh, gpu), dev_bf16(gu, gpu), offsets))
    col = np.arange(F)
    gc = (col // 32) * 64 + col % 32
    g, u = gu[:, gc], gu[:, gc + 32]
    rdg, rdu = B.swiglu_bwd(dh, g, u, "bf16")
    for name, got, ref in (("dg", dgu[:kept, gc], rdg[:kept]), ("du", dgu[:kept, gc + 32], rdu[:kept])):
        scale = np.abs(ref).max()
        err = np.abs(got - ref)
        assert np.all(err <= 2 ** -7 * np.abs(ref) + 1e-6 * scale), name


def expert_problem(gpu, rng, T, D, N, Kk, F, cf):
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    w = (0.02 * rng.standard_normal((D, N))).astype(np.float32)
    wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
    wd = (0.02 * rng.standard_normal((N, F, D))).astype(np.float32)
    logits = O.router_logits(x, w)
    idx, gates = O.route_softmax(logits, Kk)
    cap = O.capacity_of(T, Kk, N, cf)
    ref_plan = O.dispatch_plan(idx, N, cap)
    plan = K.dispatch_plan(torch.from_numpy(idx).to(gpu), N, cap)
    return x, w, wg, wu, wd, logits, idx, gates, ref_plan, plan


@pytest.mark.parametrize("T,D,N,Kk,F", [(512, 512, 8, 2, 256), (777, 192, 16, 4, 128)])
def test_gate_up_raw_gather(gpu, T, D, N, Kk, F):
    rng = np.random.default_rng(T)
    x, w, wg, wu, wd, logits, idx, gates, ref_plan, plan = expert_problem(gpu, rng, T, D, N, Kk, F, 1.25)
    xd = dev_bf16(x, gpu)
    wgu = K.pack_gate_up(dev_f32(wg, gpu), dev_f32(wu, gpu))
    gu = host(K.grouped_gate_up_raw_gather(xd, plan, wgu))
    h = host(K.grouped_gate_up_gather(xd, plan, wgu))
    torch.cuda.synchronize()
    kept = int(ref_plan["offsets"][-1])
    xs = O.permute_rows(x, ref_plan["perm_src"], Kk).astype(np.float64)
    col = np.arange(F)
    gc = (col // 32) * 64 + col % 32
    off = ref_plan["offsets"]
    for e in range(N):
        a, b = off[e], off[e + 1]
        if b <= a:
            continue
        g = xs[a:b] @ O.bf16_round(wg[e]).astype(np.float64)
        u = xs[a:b] @ O.bf16_round(wu[e]).astype(np.float64)
        assert O.normwise_rel_err(gu[a:b, gc], g) < 1e-2
        assert O.normwise_rel_err(gu[a:b, gc + 32], u) < 1e-2
    # the SwiGLU of the recomputed g, u is the forward's h, which is formed
    # from the float32 accumulators (g and u unrounded): within 2 bf16 ulps
    g16, u16 = gu[:kept, gc], gu[:kept, gc + 32]
    h_re = O.bf16_round((O.silu(g16.astype(np.float64)) * u16).astype(np.float32))
    assert bf16_ulps(h_re, h[:kept]).max() <= 2


@pytest.mark.parametrize("T,D,N,Kk,F", [(512, 512, 8, 2, 256), (600, 256, 4, 3, 96)])
def test_dgrad_gemms(gpu, T, D, N, Kk, F):
    rng = np.random.default_rng(T + 7)
    x, w, wg, wu, wd, logits, idx, gates, ref_plan, plan = expert_problem(gpu, rng, T, D, N, Kk, F, 1.25)
    R = plan.rows_cap
    off = ref_plan["offsets"]
    ops = BackwardOperands(dev_f32(wg, gpu), dev_f32(wu, gpu), dev_f32(wd, gpu))
    if F % 256 == 0:
        d_ys = O.bf16_round(rng.standard_normal((R, D)).astype(np.float32))
        dh = host(K.grouped_dgrad_down(dev_bf16(d_ys, gpu), plan.offsets, ops.w_down_dgrad))
        for e in range(N):
            a, b = off[e], off[e + 1]
            if b > a:
                ref = d_ys[a:b].astype(np.float64) @ O.bf16_round(wd[e]).astype(np.float64).T
                assert O.normwise_rel_err(dh[a:b], ref) < 1e-2, e
    dgu = O.bf16_round(rng.standard_normal((R, 2 * F)).astype(np.float32))
    d_xs = host(K.grouped_dgrad_gate_up(dev_bf16(dgu, gpu), plan.offsets, ops.w_gate_up_dgrad))
    col = np.arange(F)
    gc = (col // 32) * 64 + col % 32
    for e in range(N):
        a, b = off[e], off[e + 1]
        if b > a:
            ref = (dgu[a:b, gc].astype(np.float64) @ O.bf16_round(wg[e]).astype(np.float64).T
                   + dgu[a:b, gc + 32].astype(np.float64) @ O.bf16_round(wu[e]).astype(np.float64).T)
            assert O.normwise_rel_err(d_xs[a:b], ref) < 1e-2, e


@pytest.mark.parametrize("T,D,N,Kk,cf", [(1000, 256, 8, 4, 1.0), (300, 2048, 64, 8, 1.25)])
def test_gather_bwd_bit_exact(gpu, T, D, N, Kk, cf):
    rng = np.random.default_rng(T + 3)
    idx, plan, ref_plan = plan_on(gpu, rng, T, N, Kk, cf)
    d_xs = O.bf16_round(rng.standard_normal((plan.rows_cap, D)).astype(np.float32))
    dx = host(K.gather_bwd(dev_bf16(d_xs, gpu), plan))
    ref = B.gather_bwd(d_xs, ref_plan["slot_pos"], T, Kk, "bf16")
    assert np.array_equal(dx.view(np.uint32), ref.view(np.uint32))
    # with the shared expert's input gradient added last (float32)
    res = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    dx2 = host(K.gather_bwd(dev_bf16(d_xs, gpu), plan, residual=dev_bf16(res, gpu)))
    assert np.array_equal(dx2.view(np.uint32), (ref + res).astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("mode", ["softmax", "sigmoid"])
# N % 64 < K puts selected experts in a partial last 64-expert chunk
@pytest.mark.parametrize("T,N,Kk", [(1000, 64, 8), (257, 200, 6), (64, 8, 2), (300, 66, 8),
                                    (300, 130, 4)])
def test_router_bwd(gpu, mode, T, N, Kk):
    rng = np.random.default_rng(T + N)
    logits = rng.standard_normal((T, N)).astype(np.float32)
    dg = rng.standard_normal((T, Kk)).astype(np.float32)
    if mode == "softmax":
        idx, gates = O.route_softmax(logits, Kk)
        ref = B.route_softmax_bwd(logits, idx, gates, dg)
        m, rsf = _lib.ROUTE_SOFTMAX, 1.0
    else:
        idx, gates, _ = O.route_sigmoid(logits, None, Kk, 2.5)
        ref = B.route_sigmoid_bwd(logits, idx, dg, 2.5)
        m, rsf = _lib.ROUTE_SIGMOID_BIAS, 2.5
    dl = host(K.router_bwd(dev_f32(logits, gpu), torch.from_numpy(idx).to(gpu),
                           dev_f32(gates, gpu), dev_f32(dg, gpu), N, m, rsf))
    unsel = np.ones((T, N), bool)
    np.put_along_axis(unsel, idx, False, axis=1)
    assert np.all(dl[unsel] == 0.0)
    np.testing.assert_allclose(dl, ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())


@pytest.mark.parametrize("N", [72, 64, 40, 20])
@pytest.mark.parametrize("w_dtype", ["f32", "bf16"])
def test_router_dx(gpu, w_dtype, N):
    """Expert counts around the 64-wide LDS chunks (one partial chunk,
    exactly one, a part of one, two with the second partial)."""
    rng = np.random.default_rng(11 + N)
    T, D = 777, 512
    dl = rng.standard_normal((T, N)).astype(np.float32)
    w = (0.02 * rng.standard_normal((D, N))).astype(np.float32)
    if w_dtype == "bf16":
        w = O.bf16_round(w)
        wd = dev_bf16(w, gpu)
    else:
        wd = dev_f32(w, gpu)
    base = rng.standard_normal((T, D)).astype(np.float32)
    ref = dl.astype(np.float64) @ w.astype(np.float64).T
    dx = host(K.router_dx(dev_f32(dl, gpu), wd))
    np.testing.assert_allclose(dx, ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())
    acc = host(K.router_dx(dev_f32(dl, gpu), wd, dev_f32(base, gpu)))
    np.testing.assert_allclose(acc, base + ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())


@pytest.mark.parametrize("T,D,N,Kk,F,cf", [(512, 512, 16, 4, 256, 1.25), (384, 256, 8, 2, 256, 0.9)])
def test_layer_backward_matches_oracle(gpu, T, D, N, Kk, F, cf):
    """The composed data-gradient pass against the oracle's bf16-mode VJP,
    fed with the GPU forward's own intermediates."""
    rng = np.random.default_rng(T * 3 + N)
    x, w, wg, wu, wd, logits, idx, gates, ref_plan, plan = expert_problem(gpu, rng, T, D, N, Kk, F, cf)
    print(f"layer backward T={T} D={D} N={N} K={Kk} F={F} cf={cf}", flush=True)
    xd = dev_bf16(x, gpu)
    wdv = dev_f32(w, gpu)
    lg, top_idx, g = K.router(xd, wdv, None, Kk, _lib.ROUTE_SOFTMAX)
    plan = K.dispatch_plan(top_idx, N, O.capacity_of(T, Kk, N, cf))
    wgu = K.pack_gate_up(dev_f32(wg, gpu), dev_f32(wu, gpu))
    h = K.grouped_gate_up_gather(xd, plan, wgu)
    ys = K.grouped_down(h, plan.offsets, K.pack_down(dev_f32(wd, gpu)))
    ops = BackwardOperands(dev_f32(wg, gpu), dev_f32(wu, gpu), dev_f32(wd, gpu))
    dy = rng.standard_normal((T, D)).astype(np.float32)
    fwd = {"logits": lg, "top_idx": top_idx, "gates": g, "plan": plan, "ys": ys}
    res = moe_backward_data(xd, wdv, fwd, wgu, ops, dev_f32(dy, gpu))
    torch.cuda.synchronize()
    assert np.array_equal(host(top_idx), idx)
    ref_fwd = {"logits": host(lg), "top_idx": idx, "gates": host(g), "plan": ref_plan,
               "xs": O.permute_rows(x, ref_plan["perm_src"], Kk), "ys": host(ys)}
    params = {"router": w, "expert_w_gate": wg, "expert_w_up": wu, "expert_w_down": wd}
    ref = B.moe_backward(x, params, dy, ref_fwd, routing="softmax", precision="bf16")
    kept = int(ref_plan["offsets"][-1])
    assert np.array_equal(host(res["d_ys"])[:kept].view(np.uint32),
                          ref["d_ys"][:kept].view(np.uint32)), "d_ys"
    ulps = bf16_ulps(host(res["d_gates"]), ref["d_gates"])
    assert ulps.max() <= 1, "d_gates"
    fwd["h"] = h
    wres = moe_backward_weights(xd, fwd, res)
    torch.cuda.synchronize()
    for name, got, want in (("d_xs", host(res["d_xs"])[:kept], ref["d_xs"][:kept]),
                            ("dx", host(res["dx"]), ref["dx"]),
                            ("d_logits", host(res["d_logits"]), ref["d_logits"]),
                            ("dWg", host(wres["dWg"]), ref["dWg"]),
                            ("dWu", host(wres["dWu"]), ref["dWu"]),
                            ("dWd", host(wres["dWd"]), ref["dWd"]),
                            ("d_router", host(wres["d_router"]), ref["d_router"])):
        err = O.normwise_rel_err(np.asarray(got, np.float64), np.asarray(want, np.float64))
        print(f"  {name}: normwise {err:.2e}", flush=True)
        assert err < 2e-2, (name, err)


@pytest.mark.parametrize("R,D,F,N", [(1500, 512, 256, 6), (700, 256, 384, 3)])
def test_wgrad_gemms(gpu, R, D, F, N):
    """Weight gradients per expert segment against float64 on the same bf16
    operands; the last expert has no rows (its gradient must be zero) and the
    segments end at arbitrary rows (partial 64-row steps)."""
    rng = np.random.default_rng(R + F)
    cuts = np.sort(rng.choice(np.arange(1, R - 4), N - 2, replace=False))
    offsets = np.concatenate([[0], cuts, [R - 3, R - 3]]).astype(np.int32)   # rows past R-3 unused
    off_d = torch.from_numpy(offsets).to(gpu)
    h = O.bf16_round(rng.standard_normal((R, F)).astype(np.float32))
    d_ys = O.bf16_round(rng.standard_normal((R, D)).astype(np.float32))
    xs = O.bf16_round(rng.standard_normal((R, D)).astype(np.float32))
    dgu = O.bf16_round(rng.standard_normal((R, 2 * F)).astype(np.float32))
    dwd = host(K.grouped_wgrad_down(dev_bf16(h, gpu), dev_bf16(d_ys, gpu), off_d)) if F % 256 == 0 else None
    dwg, dwu = (host(t) for t in K.grouped_wgrad_gate_up(dev_bf16(xs, gpu), dev_bf16(dgu, gpu), off_d))
    col = np.arange(F)
    gc = (col // 32) * 64 + col % 32
    for e in range(N):
        a, b = offsets[e], offsets[e + 1]
        x64 = xs[a:b].astype(np.float64)
        for name, got, ref in (("dWg", dwg[e], x64.T @ dgu[a:b, gc]), ("dWu", dwu[e], x64.T @ dgu[a:b, gc + 32])):
            if b == a:
                assert np.all(got == 0), (name, e)
            else:
                assert O.normwise_rel_err(got, ref) < 1e-5, (name, e, O.normwise_rel_err(got, ref))
        if dwd is not None:
            ref = h[a:b].astype(np.float64).T @ d_ys[a:b]
            if b == a:
                assert np.all(dwd[e] == 0)
            else:
                assert O.normwise_rel_err(dwd[e], ref) < 1e-5, ("dWd", e)


@pytest.mark.parametrize("x_dtype", ["bf16", "f32"])
def test_router_dw(gpu, x_dtype):
    rng = np.random.default_rng(5)
    T, D, N = 2500, 256, 72
    x = rng.standard_normal((T, D)).astype(np.float32)
    if x_dtype == "bf16":
        x = O.bf16_round(x)
    dl = rng.standard_normal((T, N)).astype(np.float32)
    xd = dev_bf16(x, gpu) if x_dtype == "bf16" else dev_f32(x, gpu)
    got = host(K.router_dw(xd, dev_f32(dl, gpu)))
    ref = x.astype(np.float64).T @ dl.astype(np.float64)
    assert O.normwise_rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("Bq,Sq,N,Kk", [(2, 300, 64, 8), (3, 70, 200, 6), (1, 64, 8, 2),
                                        (2, 150, 66, 8)])
def test_router_aux_bwd(gpu, Bq, Sq, N, Kk):
    rng = np.random.default_rng(Bq * Sq + N)
    T = Bq * Sq
    logits = (1.5 * rng.standard_normal((T, N))).astype(np.float32)
    idx = O.topk_desc(logits, Kk)
    d_losses = np.array([0.7, -1.3, 0.4], np.float32)
    ref = B.aux_bwd(logits, idx, Bq, Sq, *[float(v) for v in d_losses])
    lg, ix, dl = dev_f32(logits, gpu), torch.from_numpy(idx).to(gpu), dev_f32(d_losses, gpu)
    got = host(K.router_aux_bwd(lg, ix, Bq, Sq, dl))
    tol = dict(rtol=1e-4, atol=1e-5 * np.abs(ref).max())
    np.testing.assert_allclose(got, ref, **tol)
    base = rng.standard_normal((T, N)).astype(np.float32)
    acc = host(K.router_aux_bwd(lg, ix, Bq, Sq, dl, dev_f32(base, gpu)))
    np.testing.assert_allclose(acc, base + ref, **tol)


@pytest.mark.parametrize("T,D,N,Kk,F,cf", [(600, 512, 8, 2, 256, 1.25), (777, 192, 16, 4, 128, 0.8)])
def test_fused_swiglu_bwd_matches_unfused(gpu, T, D, N, Kk, F, cf):
    """The recompute with the SwiGLU VJP in its epilogue equals the raw
    recompute followed by hmoe_swiglu_bwd bit for bit, gathering from x and
    on rows given in order."""
    rng = np.random.default_rng(T + F)
    x, w, wg, wu, wd, logits, idx, gates, ref_plan, plan = expert_problem(gpu, rng, T, D, N, Kk, F, cf)
    xd = dev_bf16(x, gpu)
    wgu = K.pack_gate_up(dev_f32(wg, gpu), dev_f32(wu, gpu))
    dh = dev_bf16(rng.standard_normal((plan.rows_cap, F)).astype(np.float32), gpu)
    ref = K.swiglu_bwd(dh, K.grouped_gate_up_raw_gather(xd, plan, wgu), plan.offsets)
    fused = K.grouped_gate_up_swiglu_bwd_gather(xd, plan, wgu, dh)
    xs = K.permute_rows(xd, plan)
    fused2 = K.grouped_gate_up_swiglu_bwd(xs, plan.offsets, wgu, dh)
    torch.cuda.synchronize()
    kept = int(ref_plan["offsets"][-1])
    assert torch.equal(fused[:kept], ref[:kept])
    assert torch.equal(fused2[:kept], ref[:kept])


def test_gate_up_raw_matches_gather(gpu):
    """The non-gather recompute on the dispatched rows equals the gathering
    one bit for bit (same tiles, same accumulation order)."""
    rng = np.random.default_rng(21)
    T, D, N, Kk, F = 600, 512, 8, 2, 256
    x, w, wg, wu, wd, logits, idx, gates, ref_plan, plan = expert_problem(gpu, rng, T, D, N, Kk, F, 1.25)
    xd = dev_bf16(x, gpu)
    wgu = K.pack_gate_up(dev_f32(wg, gpu), dev_f32(wu, gpu))
    a = K.grouped_gate_up_raw_gather(xd, plan, wgu)
    b = K.grouped_gate_up_raw(K.permute_rows(xd, plan), plan.offsets, wgu)
    torch.cuda.synchronize()
    kept = int(ref_plan["offsets"][-1])
    assert torch.equal(a[:kept], b[:kept])


@pytest.mark.parametrize("n_shared,cf,x_dtype,N,Kk", [(1, None, "bf16", 8, 2), (2, 1.0, "bf16", 8, 2),
                                                      (1, 1.0, "f32", 8, 2), (2, None, "f32", 8, 2),
                                                      (1, None, "bf16", 66, 8)])
def test_module_autograd_matches_oracle(gpu, n_shared, cf, x_dtype, N, Kk):
    """MoE.__call__ under torch autograd: loss = <dy, out> + c_z z_loss +
    c_b balance_loss (train.py:191-200), backward through the library's VJP
    of the whole module, every gradient against the bf16-mode oracle fed
    with the forward's own routing."""
    Bq, Sq, D, F = 2, 160, 256, 256
    m = MoE(D, F, N, Kk, n_shared, 0.05, 2.5, torch.bfloat16, rngs=1, device=gpu,
            capacity_factor=cf)
    m.bias.value.copy_(torch.linspace(-0.02, 0.02, N, device=gpu))
    names = ("router", "expert_w_gate", "expert_w_up", "expert_w_down",
             "shared_w_gate", "shared_w_up", "shared_w_down")
    for n in names:
        getattr(m, n).value.requires_grad_(True)
    gen = torch.Generator(device=gpu).manual_seed(5)
    x = torch.randn(Bq, Sq, D, generator=gen, device=gpu)
    if x_dtype == "bf16":
        x = x.to(torch.bfloat16)
    x.requires_grad_(True)
    dy = torch.randn(Bq, Sq, D, generator=gen, device=gpu)
    c_z, c_b = 0.37, 0.81
    print(f"module autograd n_shared={n_shared} cf={cf} x {x_dtype} N={N} K={Kk}", flush=True)
    out, aux = m(x)
    loss = (out * dy).sum() + c_z * aux["router_z_loss"] + c_b * aux["balance_loss"]
    loss.backward()
    torch.cuda.synchronize()
    assert out.grad_fn is not None and x.grad is not None and x.grad.dtype == x.dtype
    with torch.no_grad():
        _, _, _, sv = m._forward(x.detach(), save=True)
    T = Bq * Sq
    idx = host(sv["top_idx"])
    cap = O.capacity_of(T, Kk, N, cf)
    ref_plan = O.dispatch_plan(idx, N, cap)
    xn = host(x.detach()).reshape(T, D)
    p = {n: getattr(m, n).value.detach().float().cpu().numpy() for n in names}
    # the experts see x in bf16 (moe.py:198); the router sees it as given
    ref_fwd = {"logits": host(sv["logits"]), "top_idx": idx, "gates": host(sv["gates"]),
               "plan": ref_plan, "xs": O.permute_rows(O.bf16_round(xn), ref_plan["perm_src"], Kk),
               "ys": host(sv["ys"])}
    ref = B.moe_backward(xn, p, host(dy).reshape(T, D), ref_fwd, routing="sigmoid", rsf=2.5,
                         precision="bf16", n_shared=n_shared, batch_shape=(Bq, Sq),
                         d_aux=(c_z, c_b, 0.0), x_dtype=x_dtype)
    pairs = [("dx", x.grad, ref["dx"]), ("d_router", m.router.value.grad, ref["d_router"]),
             ("dWg", m.expert_w_gate.value.grad, ref["dWg"]),
             ("dWu", m.expert_w_up.value.grad, ref["dWu"]),
             ("dWd", m.expert_w_down.value.grad, ref["dWd"]),
             ("dWg_shared", m.shared_w_gate.value.grad, ref["dWg_shared"]),
             ("dWu_shared", m.shared_w_up.value.grad, ref["dWu_shared"]),
             ("dWd_shared", m.shared_w_down.value.grad, ref["dWd_shared"])]
    for name, got, want in pairs:
        got = host(got).reshape(np.shape(want))
        err = O.normwise_rel_err(got, want)
        print(f"  {name}: normwise {err:.2e}", flush=True)
        assert err < 2e-2, (name, err)
    # the aux terms alone reach the router: a loss of only the aux losses
    for n in names:
        getattr(m, n).value.grad = None
    out, aux = m(x.detach())
    (c_z * aux["router_z_loss"] + c_b * aux["balance_loss"]).backward()
    torch.cuda.synchronize()
    ref_aux = B.router_bwd(xn, p["router"], B.aux_bwd(host(sv["logits"]), idx, Bq, Sq, c_z, c_b))[0]
    err = O.normwise_rel_err(host(m.router.value.grad), ref_aux)
    print(f"  d_router (aux only): normwise {err:.2e}", flush=True)
    assert err < 1e-4
    assert float(m.expert_w_gate.value.grad.abs().max()) == 0.0


def test_f32_expert_backward_kernels(gpu):
    """The float32 backward GEMMs per expert segment against float64 numpy
    products (a library routine): an empty segment (zero weight gradients),
    segments that end inside a 64-row tile, rows past the last segment."""
    rng = np.random.default_rng(31)
    D, F = 128, 192
    offs = np.array([0, 40, 40, 161, 230], np.int32)
    N, R = len(offs) - 1, 256
    xs = rng.standard_normal((R, D)).astype(np.float32)
    wg, wu = (0.1 * rng.standard_normal((N, D, F))).astype(np.float32), \
        (0.1 * rng.standard_normal((N, D, F))).astype(np.float32)
    wd = (0.1 * rng.standard_normal((N, F, D))).astype(np.float32)
    d_ys = rng.standard_normal((R, D)).astype(np.float32)
    dh = rng.standard_normal((R, F)).astype(np.float32)
    h = rng.standard_normal((R, F)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(gpu)
    off = t(offs)
    print("f32 backward kernels", flush=True)
    g_dh = host(K.grouped_dgrad_down_f32(t(d_ys), off, t(wd)))
    g_dgu = host(K.grouped_gate_up_swiglu_bwd_f32(t(xs), off, t(wg), t(wu), t(dh)))
    dgu_in = rng.standard_normal((R, 2 * F)).astype(np.float32)
    g_dxs = host(K.grouped_dgrad_gate_up_f32(t(dgu_in), off, t(wg), t(wu)))
    g_dwg, g_dwu = (host(a) for a in K.grouped_wgrad_gate_up_f32(t(xs), t(dgu_in), off))
    g_dwd = host(K.grouped_wgrad_down_f32(t(h), t(d_ys), off))
    torch.cuda.synchronize()
    f = lambda a: a.astype(np.float64)
    for e in range(N):
        lo, hi = offs[e], offs[e + 1]
        x_e, g_e, u_e = f(xs[lo:hi]), f(wg[e]), f(wu[e])
        rows = slice(lo, hi)
        checks = [("dh", g_dh[rows], f(d_ys[rows]) @ f(wd[e]).T)]
        gg, uu = x_e @ g_e, x_e @ u_e
        s = 1.0 / (1.0 + np.exp(-gg))
        d = f(dh[rows])
        checks += [("dg", g_dgu[rows, :F], d * uu * s * (1 + gg * (1 - s))),
                   ("du", g_dgu[rows, F:], d * gg * s),
                   ("d_xs", g_dxs[rows], f(dgu_in[rows, :F]) @ g_e.T + f(dgu_in[rows, F:]) @ u_e.T),
                   ("dWg", g_dwg[e], x_e.T @ f(dgu_in[rows, :F])),
                   ("dWu", g_dwu[e], x_e.T @ f(dgu_in[rows, F:])),
                   ("dWd", g_dwd[e], f(h[rows]).T @ f(d_ys[rows]))]
        for name, got, want in checks:
            if hi == lo and name.startswith("dW"):
                assert np.all(got == 0.0), (name, e)
                continue
            if hi == lo:
                continue
            err = O.normwise_rel_err(got, want)
            assert err < 1e-5, (name, e, err)


@pytest.mark.parametrize("n_shared,cf", [(1, None), (2, 1.0)])
def test_module_autograd_float32_matches_oracle(gpu, n_shared, cf):
    """dtype float32: the module's backward on the float32 kernels, every
    gradient against the oracle's float64 VJP on the forward's own routing
    (no rounding points; the float32 GEMM sums are the only difference)."""
    Bq, Sq, D, F, N, Kk = 2, 160, 256, 256, 8, 2
    m = MoE(D, F, N, Kk, n_shared, 0.05, 2.5, torch.float32, rngs=1, device=gpu,
            capacity_factor=cf)
    m.bias.value.copy_(torch.linspace(-0.02, 0.02, N, device=gpu))
    names = ("router", "expert_w_gate", "expert_w_up", "expert_w_down",
             "shared_w_gate", "shared_w_up", "shared_w_down")
    for n in names:
        getattr(m, n).value.requires_grad_(True)
    gen = torch.Generator(device=gpu).manual_seed(5)
    x = torch.randn(Bq, Sq, D, generator=gen, device=gpu).requires_grad_(True)
    dy = torch.randn(Bq, Sq, D, generator=gen, device=gpu)
    c_z, c_b = 0.37, 0.81
    print(f"module autograd float32 n_shared={n_shared} cf={cf}", flush=True)
    out, aux = m(x)
    loss = (out * dy).sum() + c_z * aux["router_z_loss"] + c_b * aux["balance_loss"]
    loss.backward()
    torch.cuda.synchronize()
    assert out.grad_fn is not None and x.grad is not None and x.grad.dtype == torch.float32
    with torch.no_grad():
        _, _, _, sv = m._forward(x.detach(), save=True)
    T = Bq * Sq
    idx = host(sv["top_idx"])
    cap = O.capacity_of(T, Kk, N, cf)
    ref_plan = O.dispatch_plan(idx, N, cap)
    xn = host(x.detach()).reshape(T, D)
    p = {n: getattr(m, n).value.detach().cpu().numpy() for n in names}
    ref_fwd = {"logits": host(sv["logits"]), "top_idx": idx, "gates": host(sv["gates"]),
               "plan": ref_plan, "xs": O.permute_rows(xn, ref_plan["perm_src"], Kk),
               "ys": host(sv["ys"])}
    ref = B.moe_backward(xn, p, host(dy).reshape(T, D), ref_fwd, routing="sigmoid", rsf=2.5,
                         precision="fp64", n_shared=n_shared, batch_shape=(Bq, Sq),
                         d_aux=(c_z, c_b, 0.0))
    pairs = [("dx", x.grad, ref["dx"]), ("d_router", m.router.value.grad, ref["d_router"]),
             ("dWg", m.expert_w_gate.value.grad, ref["dWg"]),
             ("dWu", m.expert_w_up.value.grad, ref["dWu"]),
             ("dWd", m.expert_w_down.value.grad, ref["dWd"]),
             ("dWg_shared", m.shared_w_gate.value.grad, ref["dWg_shared"]),
             ("dWu_shared", m.shared_w_up.value.grad, ref["dWu_shared"]),
             ("dWd_shared", m.shared_w_down.value.grad, ref["dWd_shared"])]
    for name, got, want in pairs:
        got = host(got).reshape(np.shape(want))
        err = O.normwise_rel_err(got, want)
        print(f"  {name}: normwise {err:.2e}", flush=True)
        assert err < 1e-5, (name, err)   # measured ~6e-7


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_module_trains(gpu, dtype):
    """End to end: the module as the reference's train step uses it
    (train.py:191-200: output loss plus weighted z and balance losses),
    Adam on every trainable parameter through torch autograd; a target made
    by a second MoE of the same shape is learnable, so the loss must fall
    (both compute dtypes, tokens in the compute dtype)."""
    torch.manual_seed(0)
    Bq, Sq, D, F, N, Kk = 2, 128, 256, 256, 8, 2
    student = MoE(D, F, N, Kk, 1, 0.05, 2.5, dtype, rngs=3, device=gpu)
    teacher = MoE(D, F, N, Kk, 1, 0.05, 2.5, dtype, rngs=4, device=gpu)
    x = torch.randn(Bq, Sq, D, generator=torch.Generator(device=gpu).manual_seed(6),
                    device=gpu).to(dtype)
    with torch.no_grad():
        target, _ = teacher(x)
    params = [p.value for n, p in student.named_params().items() if n != "bias"]
    for p in params:
        p.requires_grad_(True)
    opt = torch.optim.Adam(params, lr=3e-3)
    losses = []
    for step in range(40):
        opt.zero_grad(set_to_none=True)
        out, aux = student(x)
        loss = ((out - target) ** 2).mean() + 1e-3 * aux["router_z_loss"] \
            + 1e-2 * aux["balance_loss"]
        loss.backward()
        opt.step()
        losses.append(float(loss.detach()))
    print(f"module training ({dtype}): loss {losses[0]:.4e} -> {losses[-1]:.4e}", flush=True)
    assert all(np.isfinite(losses))
    assert losses[-1] < 0.5 * losses[0]


def test_module_autograd_saved_tensors(gpu):
    """The autograd node keeps its residuals and the forward's parameters as
    saved tensors: a second backward through a retained graph gives the same
    gradients, an in-place parameter update between forward and backward
    raises (torch's version check), and with only the input requiring grad
    the input gradient is unchanged and no weight gradient is produced."""
    Bq, Sq, D, F, N, Kk = 1, 128, 256, 256, 8, 2
    m = MoE(D, F, N, Kk, 1, 0.05, 2.5, torch.bfloat16, rngs=3, device=gpu)
    names = ("router", "expert_w_gate", "expert_w_up", "expert_w_down",
             "shared_w_gate", "shared_w_up", "shared_w_down")
    gen = torch.Generator(device=gpu).manual_seed(9)
    x = torch.randn(Bq, Sq, D, generator=gen, device=gpu).to(torch.bfloat16)
    dy = torch.randn(Bq, Sq, D, generator=gen, device=gpu)
    for n in names:
        getattr(m, n).value.requires_grad_(True)
    xg = x.clone().requires_grad_(True)
    out, aux = m(xg)
    loss = (out * dy).sum() + 0.3 * aux["router_z_loss"]
    loss.backward(retain_graph=True)
    first = {n: getattr(m, n).value.grad.clone() for n in names}
    dx_first = xg.grad.clone()
    for n in names:
        getattr(m, n).value.grad = None
    xg.grad = None
    loss.backward()
    torch.cuda.synchronize()
    for n in names:
        assert torch.equal(getattr(m, n).value.grad, first[n]), n
    assert torch.equal(xg.grad, dx_first)
    # an in-place update of a parameter the forward read
    out, aux = m(x)
    with torch.no_grad():
        m.expert_w_up.value.mul_(1.0)
    with pytest.raises(RuntimeError):
        out.sum().backward()
    # only the input requires grad
    for n in names:
        getattr(m, n).value.grad = None
        getattr(m, n).value.requires_grad_(False)
    xg2 = x.clone().requires_grad_(True)
    out, aux = m(xg2)
    ((out * dy).sum() + 0.3 * aux["router_z_loss"]).backward()
    torch.cuda.synchronize()
    assert torch.equal(xg2.grad, dx_first)
    assert all(getattr(m, n).value.grad is None for n in names)


def test_wgrad_gemms_past_2gib(gpu):
    """Weight gradients on dispatched buffers larger than 2 GiB (the skewed
    workload's backward: 65536 tokens x top-8 rows of d_model 2048 are 2 GiB
    of bf16): each K step's buffer resource starts at its own first row, so
    experts whose rows lie past byte 2^31 are computed like the first ones.
    Sampled experts (the first, one in the middle, the last two, an empty
    one) against float64 on the same bf16 operands."""
    D, F, N = 2048, 768, 128
    rng = np.random.default_rng(77)
    sizes = rng.integers(4000, 4800, N)
    sizes[5] = 0                                     # an empty expert
    offsets = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    R = int(offsets[-1])
    assert R * D * 2 > 2 ** 31 and int(offsets[-3]) * D * 2 > 2 ** 31
    print(f"wgrad past 2 GiB: R={R} D={D} F={F} N={N}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(3)
    xs = torch.randn(R, D, generator=g, device=gpu).to(torch.bfloat16)
    dgu = torch.randn(R, 2 * F, generator=g, device=gpu).to(torch.bfloat16)
    h = torch.randn(R, F, generator=g, device=gpu).to(torch.bfloat16)
    d_ys = torch.randn(R, D, generator=g, device=gpu).to(torch.bfloat16)
    off_d = torch.from_numpy(offsets).to(gpu)
    dwg, dwu = K.grouped_wgrad_gate_up(xs, dgu, off_d)
    dwd = K.grouped_wgrad_down(h, d_ys, off_d)
    torch.cuda.synchronize()
    col = np.arange(F)
    gc = (col // 32) * 64 + col % 32
    for e in (0, 5, N // 2, N - 2, N - 1):
        a, b = int(offsets[e]), int(offsets[e + 1])
        if b == a:
            assert torch.all(dwg[e] == 0) and torch.all(dwu[e] == 0) and torch.all(dwd[e] == 0)
            continue
        x64 = host(xs[a:b]).astype(np.float64)
        g64 = host(dgu[a:b]).astype(np.float64)
        for name, got, ref in (("dWg", dwg[e], x64.T @ g64[:, gc]),
                               ("dWu", dwu[e], x64.T @ g64[:, gc + 32]),
                               ("dWd", dwd[e], host(h[a:b]).astype(np.float64).T
                                @ host(d_ys[a:b]).astype(np.float64))):
            err = O.normwise_rel_err(host(got), ref)
            print(f"  expert {e} rows {a}-{b} {name}: {err:.2e}", flush=True)
            assert err < 1e-5, (name, e, err)


def test_wgrad_gate_up_segment_past_2gib(gpu):
    """One expert whose own segment is larger than 2 GiB (530000 rows of
    d_model 2048 bf16: the buffer resources are then rebased at every K
    step), beside a small one; dWg and dWu against float64, summed over
    65536-row chunks on the host."""
    D, F = 2048, 128
    sizes = np.array([530_000, 100])
    offsets = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    R = int(offsets[-1])
    assert int(sizes[0]) * D * 2 > 2 ** 31
    print(f"wgrad gate/up segment past 2 GiB: rows {sizes.tolist()}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(4)
    xs = torch.randn(R, D, generator=g, device=gpu).to(torch.bfloat16)
    dgu = torch.randn(R, 2 * F, generator=g, device=gpu).to(torch.bfloat16)
    dwg, dwu = K.grouped_wgrad_gate_up(xs, dgu, torch.from_numpy(offsets).to(gpu))
    torch.cuda.synchronize()
    col = np.arange(F)
    gc = (col // 32) * 64 + col % 32
    for e in range(2):
        a, b = int(offsets[e]), int(offsets[e + 1])
        ref_g = np.zeros((D, F))
        ref_u = np.zeros((D, F))
        for c in range(a, b, 65536):
            d = min(b, c + 65536)
            x64 = host(xs[c:d]).astype(np.float64)
            g64 = host(dgu[c:d]).astype(np.float64)
            ref_g += x64.T @ g64[:, gc]
            ref_u += x64.T @ g64[:, gc + 32]
        for name, got, ref in (("dWg", dwg[e], ref_g), ("dWu", dwu[e], ref_u)):
            err = O.normwise_rel_err(host(got), ref)
            print(f"  expert {e} rows {b - a} {name}: {err:.2e}", flush=True)
            # float32 accumulation over 8282 K steps: ~4e-7 x sqrt(530000 / 4500)
            assert err < 3e-5, (name, e, err)
