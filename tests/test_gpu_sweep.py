"""Seeded sweep of small random layer shapes through the C ABI (needs an MI355X).

Each case draws its own shape (tokens, d_model, experts, top-k, d_ff), routing
mode (softmax, or sigmoid with a bias and a scaling factor), capacity factor
(from heavy drops to none) and weight scale.  Routing (logits, indices, gates)
and the dispatch plan (counts, offsets, slot map, permutation, keep mask) must
be bit-exact against the oracle; the layer output of the bf16 path (router,
plan, gathering gate/up GEMM with the SwiGLU epilogue, down GEMM, combine)
must be within the bf16 tolerance of the oracle's float32 expert pass on the
oracle's plan.  The e4m3 expert path is swept the same way against the
oracle's e4m3 emulation.  Shapes stay small so that the oracle's float64
router runs in well under a second per case.
"""
import numpy as np
import pytest
import torch

import oracle as O
from hanuman_amd import _lib
from hanuman_amd import kernels as K

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2
N_CASES = 24


def host(t):
    return t.float().cpu().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()


def bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float32:
        a, b = a.view(np.uint32), np.asarray(b, np.float32).view(np.uint32)
    return a.shape == b.shape and np.array_equal(a, b)


def draw_case(i):
    rng = np.random.default_rng(1000 + i)
    T = int(rng.integers(1, 1200))
    D = 256 * int(rng.integers(1, 3))             # multiples of the 256-column output tile
    N = int(rng.choice([1, 3, 8, 17, 64, 70, 96]))
    Kk = int(rng.integers(1, min(N, 8) + 1))
    F = 128 * int(rng.integers(1, 5))
    mode = "softmax" if rng.random() < 0.5 else "sigmoid"
    cf = [None, 0.5, 1.0, 1.25, 2.0][int(rng.integers(0, 5))]
    wstd = float(rng.choice([0.02, 0.2]))
    return rng, T, D, N, Kk, F, mode, cf, wstd


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_layer_matches_oracle(gpu, i):
    rng, T, D, N, Kk, F, mode, cf, wstd = draw_case(i)
    print(f"sweep case {i}: T={T} D={D} N={N} K={Kk} F={F} {mode} cf={cf} wstd={wstd}", flush=True)
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    router_w = (wstd * rng.standard_normal((D, N))).astype(np.float32)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32) if mode == "sigmoid" else None
    rsf = 2.5 if mode == "sigmoid" else 1.0
    wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
    wd = (0.02 * rng.standard_normal((N, F, D))).astype(np.float32)

    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    xt = dev(x).to(torch.bfloat16)
    m = _lib.ROUTE_SOFTMAX if mode == "softmax" else _lib.ROUTE_SIGMOID_BIAS
    logits, idx, gates = K.router(xt, dev(router_w), dev(bias) if bias is not None else None, Kk,
                                  m, rsf)
    cap = K.capacity(T, Kk, N, cf)
    plan = K.dispatch_plan(idx, N, cap)
    h = K.grouped_gate_up_gather(xt, plan, K.pack_gate_up(dev(wg), dev(wu)))
    ys = K.grouped_down(h, plan.offsets, K.pack_down(dev(wd)))
    out = K.combine(ys, plan, gates, None, torch.float32)
    torch.cuda.synchronize()

    ref_logits = O.router_logits(x, router_w)
    if mode == "softmax":
        ref_idx, ref_gates = O.route_softmax(ref_logits, Kk)
    else:
        ref_idx, ref_gates, _ = O.route_sigmoid(ref_logits, bias, Kk, rsf)
    assert cap == O.capacity_of(T, Kk, N, cf)
    ref_plan = O.dispatch_plan(ref_idx, N, cap)
    assert bits_equal(host(logits), ref_logits), "logits"
    assert bits_equal(host(idx), ref_idx), "top_idx"
    assert bits_equal(host(gates), ref_gates), "gates"
    for k in ("counts", "offsets", "slot_pos", "perm_src", "keep"):
        assert np.array_equal(host(getattr(plan, k)), ref_plan[k]), k
    xs = O.permute_rows(x, ref_plan["perm_src"], Kk)
    ys_ref = O.expert_ffn(xs, ref_plan["offsets"], wg, wu, wd, precision="fp32")
    ref = O.combine(ys_ref, ref_plan["slot_pos"], ref_gates, T, Kk, ys_dtype="bf16")
    kept = int(ref_plan["offsets"][-1])
    if kept == 0:
        assert not np.any(host(out)), "a layer with every slot dropped returns zeros"
        return
    err = O.normwise_rel_err(host(out), ref)
    print(f"  kept {kept} of {T * Kk} slots, output normwise err {err:.2e}", flush=True)
    assert err < BF16_TOL


FP8_TOL = 5e-2
N_FP8_CASES = 12


@pytest.mark.parametrize("i", range(N_FP8_CASES))
def test_random_fp8_layer_matches_oracle(gpu, i):
    """The e4m3 expert path on random shapes: routing, plan and the per-token
    codes and scales of x bit-exact; the bf16 output within 1e-2 of the
    oracle's e4m3 emulation and within 5e-2 of the float32 layer on the
    dequantised weights."""
    rng, T, D, N, Kk, F, mode, cf, wstd = draw_case(500 + i)
    print(f"fp8 sweep case {i}: T={T} D={D} N={N} K={Kk} F={F} {mode} cf={cf} wstd={wstd}",
          flush=True)
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    router_w = (wstd * rng.standard_normal((D, N))).astype(np.float32)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32) if mode == "sigmoid" else None
    rsf = 2.5 if mode == "sigmoid" else 1.0
    wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
    wd = (0.02 * rng.standard_normal((N, F, D))).astype(np.float32)

    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    xt = dev(x).to(torch.bfloat16)
    m = _lib.ROUTE_SOFTMAX if mode == "softmax" else _lib.ROUTE_SIGMOID_BIAS
    logits, idx, gates = K.router(xt, dev(router_w), dev(bias) if bias is not None else None, Kk,
                                  m, rsf)
    plan = K.dispatch_plan(idx, N, K.capacity(T, Kk, N, cf))
    fgu, sgu = K.pack_fp8_gate_up(dev(wg), dev(wu))
    fd, sd = K.pack_fp8_down(dev(wd))
    x_q, x_s = K.quantize_rows_fp8(xt)
    h_q, h_e = K.grouped_gate_up_fp8_gather_qh(x_q, x_s, plan, fgu, sgu)
    ys8 = K.grouped_down_fp8_mx(h_q, h_e, plan.offsets, fd, sd)
    out = K.combine(ys8, plan, gates, None, torch.bfloat16)
    torch.cuda.synchronize()

    params = {"router": router_w, "expert_w_gate": wg, "expert_w_up": wu, "expert_w_down": wd}
    if bias is not None:
        params["bias"] = bias
    kw = dict(top_k=Kk, routing=mode, routed_scaling_factor=rsf, capacity_factor=cf)
    r8 = O.moe_forward(x, params, expert="swiglu_fp8", out_dtype="bf16", **kw)
    ref = O.moe_forward(x, {**params, **O.dequantized_weights(r8["fp8"])}, precision="fp32", **kw)
    assert bits_equal(host(logits), r8["logits"]), "logits"
    assert bits_equal(host(idx), r8["top_idx"]), "top_idx"
    assert bits_equal(host(gates), r8["gates"]), "gates"
    for k in ("counts", "offsets", "slot_pos", "perm_src", "keep"):
        assert np.array_equal(host(getattr(plan, k)), r8["plan"][k]), k
    assert np.array_equal(x_q.cpu().numpy(), r8["x_q"]), "x codes"
    assert bits_equal(host(x_s), r8["x_s"]), "x scales"
    got = host(out)
    err_emul = O.normwise_rel_err(got, r8["out"])
    err = O.normwise_rel_err(got, ref["out"])
    print(f"  output normwise err {err:.2e} (vs the e4m3 emulation {err_emul:.2e})", flush=True)
    assert err_emul < 1e-2
    assert err < FP8_TOL


N_BWD_CASES = 8


@pytest.mark.parametrize("i", range(N_BWD_CASES))
def test_random_module_backward_matches_oracle(gpu, i):
    """MoE.__call__ under torch autograd on random shapes (with 1-2 shared
    experts, the z and balance losses in the loss): every gradient against the
    bf16-mode VJP oracle fed with the forward's own routing, normwise 2e-2."""
    from hanuman_amd.moe import MoE
    from oracle import moe_backward as B

    rng = np.random.default_rng(2000 + i)
    Bq = int(rng.integers(1, 4))
    Sq = int(rng.integers(16, 300))
    D = 256 * int(rng.integers(1, 3))
    F = 256 * int(rng.integers(1, 3))    # the bf16 backward's dh GEMM takes whole 256-column tiles
    N = int(rng.choice([2, 8, 17, 64, 70]))
    Kk = int(rng.integers(1, min(N, 8) + 1))
    n_shared = int(rng.integers(1, 3))   # the reference divides by the count (moe.py:168)
    cf = [None, 0.75, 1.25][int(rng.integers(0, 3))]
    seed = int(rng.integers(0, 1 << 30))
    print(f"bwd sweep case {i}: B={Bq} S={Sq} D={D} F={F} N={N} K={Kk} shared={n_shared} cf={cf}",
          flush=True)
    m = MoE(D, F, N, Kk, n_shared, 0.05, 2.5, torch.bfloat16, rngs=seed, device=gpu,
            capacity_factor=cf)
    m.bias.value.copy_(torch.from_numpy((0.02 * rng.standard_normal(N)).astype(np.float32)))
    names = ["router", "expert_w_gate", "expert_w_up", "expert_w_down",
             "shared_w_gate", "shared_w_up", "shared_w_down"]
    for n in names:
        getattr(m, n).value.requires_grad_(True)
    x = torch.from_numpy(rng.standard_normal((Bq, Sq, D)).astype(np.float32)).to(gpu)
    x = x.to(torch.bfloat16).requires_grad_(True)
    dy = torch.from_numpy(rng.standard_normal((Bq, Sq, D)).astype(np.float32)).to(gpu)
    c_z, c_b = 0.37, 0.81
    out, aux = m(x)
    (((out * dy).sum()) + c_z * aux["router_z_loss"] + c_b * aux["balance_loss"]).backward()
    torch.cuda.synchronize()
    with torch.no_grad():
        _, _, _, sv = m._forward(x.detach(), save=True)
    T = Bq * Sq
    idx = host(sv["top_idx"])
    ref_plan = O.dispatch_plan(idx, N, O.capacity_of(T, Kk, N, cf))
    xn = host(x.detach()).reshape(T, D)
    p = {n: getattr(m, n).value.detach().float().cpu().numpy() for n in names}
    ref_fwd = {"logits": host(sv["logits"]), "top_idx": idx, "gates": host(sv["gates"]),
               "plan": ref_plan, "xs": O.permute_rows(xn, ref_plan["perm_src"], Kk),
               "ys": host(sv["ys"])}
    ref = B.moe_backward(xn, p, host(dy).reshape(T, D), ref_fwd, routing="sigmoid", rsf=2.5,
                         precision="bf16", n_shared=n_shared, batch_shape=(Bq, Sq),
                         d_aux=(c_z, c_b, 0.0))
    pairs = [("dx", x.grad, "dx"), ("d_router", m.router.value.grad, "d_router"),
             ("dWg", m.expert_w_gate.value.grad, "dWg"), ("dWu", m.expert_w_up.value.grad, "dWu"),
             ("dWd", m.expert_w_down.value.grad, "dWd"),
             ("dWg_shared", m.shared_w_gate.value.grad, "dWg_shared"),
             ("dWu_shared", m.shared_w_up.value.grad, "dWu_shared"),
             ("dWd_shared", m.shared_w_down.value.grad, "dWd_shared")]
    for name, got, key in pairs:
        want = ref[key]
        if not np.any(want):
            # an expert set that received no kept rows has an exactly zero gradient
            assert not torch.any(got), name
            continue
        err = O.normwise_rel_err(host(got).reshape(np.shape(want)), want)
        print(f"  {name}: normwise {err:.2e}", flush=True)
        assert err < 2e-2, (name, err)


def test_module_backward_needs_d_ff_multiple_of_256(gpu):
    """d_ff = 384 runs forward (gate/up columns come in 256-column tiles of
    the packed [gate | up] pairs, so d_ff % 128 suffices), and the backward
    refuses it with the library's error instead of computing on partial
    tiles (its dh = d_ys Wd^T GEMM has d_ff output columns)."""
    from hanuman_amd._lib import HmoeError
    from hanuman_amd.moe import MoE

    m = MoE(256, 384, 8, 2, 1, 0.05, 2.5, torch.bfloat16, rngs=3, device=gpu)
    m.expert_w_gate.value.requires_grad_(True)
    x = torch.randn(1, 64, 256, device=gpu).to(torch.bfloat16).requires_grad_(True)
    out, _ = m(x)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    with pytest.raises(HmoeError, match="multiple of 256"):
        out.sum().backward()


N_ROUTER_CASES = 20


@pytest.mark.parametrize("i", range(N_ROUTER_CASES))
def test_random_router_with_ties_matches_oracle(gpu, i):
    """Routing alone on tie-heavy inputs: the fused router on router weights
    whose columns repeat (every token then has equal logits on those experts),
    and the logits-given selection on small-integer logits.  Shapes span the
    eight-tokens-per-wave selection (up to 64 experts) and the one-token-per-
    wave one (beyond), partial groups of eight tokens and top-k up to 32."""
    rng = np.random.default_rng(5000 + i)
    T = int(rng.integers(1, 3000))
    D = 8 * int(rng.integers(1, 65))
    N = int(rng.choice([1, 2, 7, 8, 9, 31, 33, 50, 63, 64, 65, 100, 256]))
    Kk = int(rng.integers(1, min(N, 32) + 1))
    mode = "softmax" if rng.random() < 0.5 else "sigmoid"
    rsf = 2.5 if mode == "sigmoid" else 1.0
    m = _lib.ROUTE_SOFTMAX if mode == "softmax" else _lib.ROUTE_SIGMOID_BIAS
    print(f"router sweep case {i}: T={T} D={D} N={N} K={Kk} {mode}", flush=True)
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    w = (0.05 * rng.standard_normal((D, N))).astype(np.float32)
    for _ in range(min(N // 2, 6)):
        a, b = rng.choice(N, 2, replace=False)
        w[:, b] = w[:, a]
    bias = None
    if mode == "sigmoid":
        bias = (0.1 * rng.integers(-2, 3, size=N)).astype(np.float32)   # ties in the bias too
    logits_ref = O.router_logits(x, w)
    if mode == "softmax":
        idx_ref, g_ref = O.route_softmax(logits_ref, Kk)
    else:
        idx_ref, g_ref, _ = O.route_sigmoid(logits_ref, bias, Kk, rsf)
    dev_bias = torch.from_numpy(bias).to(gpu) if bias is not None else None
    logits, idx, g = K.router(torch.from_numpy(x).to(gpu).to(torch.bfloat16),
                              torch.from_numpy(w).to(gpu), dev_bias, Kk, m, rsf)
    torch.cuda.synchronize()
    assert bits_equal(host(logits), logits_ref), "fused router logits"
    assert bits_equal(host(idx), idx_ref), "fused router top_idx"
    assert bits_equal(host(g), g_ref), "fused router gates"

    lg = rng.integers(-3, 4, size=(T, N)).astype(np.float32)
    if mode == "softmax":
        idx_ref, g_ref = O.route_softmax(lg, Kk)
    else:
        idx_ref, g_ref, _ = O.route_sigmoid(lg, bias, Kk, rsf)
    idx, g = K.router_from_logits(torch.from_numpy(lg).to(gpu), dev_bias, Kk, m, rsf)
    torch.cuda.synchronize()
    assert bits_equal(host(idx), idx_ref), "logits-given top_idx"
    assert bits_equal(host(g), g_ref), "logits-given gates"
