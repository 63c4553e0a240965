"""Whole-layer parity of the HIP path against the oracle (needs an MI355X).

Routing, plan and drop mask must be bit-exact; the layer output must be within
2e-2 normwise relative error of the oracle's fp32 result (float64 arithmetic
on the fp32 master weights), the bf16 tolerance of the measured workloads.
"""
import numpy as np
import pytest
import torch

import oracle as O
from hanuman_amd import workloads as W
from hanuman_amd.layer import DeviceLayer
from hanuman_amd.moe import MoE

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2
# Worst single token (normwise over its d_model values) at the full-size
# workloads, against the float32 layer on the weights the kernels use.
WORST_TOKEN_TOL_BF16 = 1.5e-2   # measured 5.4e-3 (full_bf16), 6.0e-3 (skewed_bf16)
WORST_TOKEN_TOL_FP8 = 7e-2     # measured 5.4e-2 (fp8_experts)


def host(t):
    return t.float().cpu().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()


def check_routing_and_plan(res, ref_idx, ref_gates, ref_plan, ref_logits=None):
    if ref_logits is not None:
        assert np.array_equal(host(res["logits"]).view(np.uint32), ref_logits.view(np.uint32))
    assert np.array_equal(host(res["top_idx"]), ref_idx), "top_idx"
    assert np.array_equal(host(res["gates"]).view(np.uint32), ref_gates.view(np.uint32)), "gates"
    plan = res["plan"]
    for k in ("counts", "offsets", "slot_pos", "perm_src", "keep"):
        assert np.array_equal(host(getattr(plan, k)), ref_plan[k]), k


def oracle_routing(inp):
    wl = inp.wl
    logits = inp.logits if wl.router_from_logits else O.router_logits(inp.x, inp.router)
    idx, gates = O.route_softmax(logits, wl.top_k)
    plan = O.dispatch_plan(idx, wl.n_experts, wl.capacity)
    return logits, idx, gates, plan


@pytest.mark.parametrize("name,tokens", [("tiny_fp32", 2048), ("dispatch_identity", 4096),
                                         ("full_bf16", 2048), ("skewed_bf16", 4096)])
def test_workload_reduced_tokens(gpu, name, tokens):
    wl = W.WORKLOADS[name].scaled(tokens)
    print(f"layer {name} T={wl.tokens}", flush=True)
    inp = W.make_inputs(wl, seed=0)
    ref = O.moe_forward(inp.x, {"router": inp.router, "expert_w_gate": inp.w_gate,
                                "expert_w_up": inp.w_up, "expert_w_down": inp.w_down},
                        top_k=wl.top_k, routing="softmax", capacity_factor=wl.capacity_factor,
                        expert=wl.expert, dtype="f32" if wl.expert_dtype == "f32" else "bf16",
                        precision="fp32", logits=inp.logits if wl.router_from_logits else None)
    layer = DeviceLayer(inp, gpu)
    res = layer.forward()
    torch.cuda.synchronize()
    check_routing_and_plan(res, ref["top_idx"], ref["gates"], ref["plan"],
                           None if wl.router_from_logits else ref["logits"])
    out = host(res["out"])
    if wl.expert == "identity":
        assert np.array_equal(out.view(np.uint32), ref["out"].view(np.uint32)), "identity combine"
    else:
        err = O.normwise_rel_err(out, ref["out"])
        print(f"{name}: normwise rel err {err:.3e}", flush=True)
        assert err < (1e-5 if wl.expert_dtype == "f32" else BF16_TOL)


def full_output_ref(x, w_gate, w_up, w_down, gates, plan, K):
    """The whole [T, D] layer output in float32 arithmetic on the fp32
    weights given, on the plan given (the GPU's own routing, which the tests
    check bit-exact first): per expert, the kept rows' tokens go through the
    SwiGLU as float32 BLAS products, and each token gets bf16(gate) times its
    row (moe.py:80-85).  A token meets an expert at most once, so the
    scatter per expert has no repeated index."""
    from threadpoolctl import threadpool_limits
    import os
    T, D = x.shape
    out = np.zeros((T, D), np.float32)
    off = np.asarray(plan["offsets"])
    perm = np.asarray(plan["perm_src"])
    g16 = O.bf16_round(np.asarray(gates, np.float32)).reshape(-1)
    with threadpool_limits(min(16, len(os.sched_getaffinity(0)))):
        for e in range(len(off) - 1):
            a, b = int(off[e]), int(off[e + 1])
            if b <= a:
                continue
            slots = perm[a:b]
            toks = slots // K
            xe = x[toks]
            g = xe @ w_gate[e]
            u = xe @ w_up[e]
            ys = ((g / (1.0 + np.exp(-g))) * u).astype(np.float32) @ w_down[e]
            out[toks] += g16[slots][:, None] * ys
    return out


def _token_subplan(plan, K, T, tokens):
    """The plan restricted to the given tokens: their kept slots in
    dispatched order (grouped by expert) as rows of a plan of their own.
    Returns (offsets, source token of each row, slot -> row [len, K] with -1
    for dropped slots)."""
    offsets = np.asarray(plan["offsets"], np.int64)
    N = len(offsets) - 1
    slot_pos = np.asarray(plan["slot_pos"]).reshape(T, K)[tokens]
    pos = np.unique(slot_pos[slot_pos >= 0])
    expert = np.searchsorted(offsets, pos, side="right") - 1
    sub_off = np.concatenate([[0], np.cumsum(np.bincount(expert, minlength=N))]).astype(np.int32)
    src = np.asarray(plan["perm_src"])[pos] // K
    remap = np.full(int(offsets[-1]), -1, np.int64)
    remap[pos] = np.arange(pos.size)
    sub_slot = np.where(slot_pos >= 0, remap[np.maximum(slot_pos, 0)], -1)
    return sub_off, src, sub_slot


def fp8_emulated_tokens(x, wq, gates, plan, K, tokens):
    """The fp8 rule's layer output (``O.expert_ffn_fp8``: x per token and h per
    32-column block in e4m3, float64 dot products of the decoded codes, bf16
    rounding points as the kernels have them) for the given tokens only.
    Every row's quantisation depends on that row alone, so the tokens' kept
    slots form a plan of their own."""
    T = x.shape[0]
    sub_off, src, sub_slot = _token_subplan(plan, K, T, tokens)
    xq, xs = O.quantize_rows_e4m3(O.bf16_round(x[src]))
    ys, *_ = O.expert_ffn_fp8(xq, xs, sub_off, wq["wg_q"], wq["wg_s"], wq["wu_q"], wq["wu_s"],
                              wq["wd_q"], wq["wd_s"])
    g = np.asarray(gates, np.float32).reshape(T, K)[tokens]
    return O.bf16_round(O.combine(ys, sub_slot.reshape(-1), g, len(tokens), K))


def bf16_mode_tokens(x, w_gate, w_up, w_down, gates, plan, K, tokens, out_dtype):
    """The oracle's bf16 mode (``moe.py``'s rounding points: bf16 weights, g
    and u rounded to bf16, ``h = bf16(silu(g) u)``, ys bf16, bf16 gates in the
    float32 combine; float32 dot products) for the given tokens only."""
    T = x.shape[0]
    sub_off, src, sub_slot = _token_subplan(plan, K, T, tokens)
    ys = O.expert_ffn(O.bf16_round(x[src]), sub_off, w_gate, w_up, w_down, precision="bf16")
    g = np.asarray(gates, np.float32).reshape(T, K)[tokens]
    out = O.combine(ys, sub_slot.reshape(-1), g, len(tokens), K)
    return O.bf16_round(out) if out_dtype == "bf16" else out


@pytest.mark.parametrize("name", ["full_bf16", "skewed_bf16"])
def test_rounding_points_match_reference_bf16_mode(gpu, name):
    """The bf16 layer rounds where moe.py:70-85 rounds: g and u to bf16 (the
    ragged_dot outputs), h = bf16(silu(g) u), ys bf16, gates to bf16 in the
    combine.  Against the oracle's bf16 mode (the same rounding points,
    float32 dot products) the output agrees to 5e-3 normwise; a forward
    that skipped any of these roundings would sit near the 2e-2 distance
    to the float64 result instead."""
    wl = W.WORKLOADS[name].scaled(2048)
    inp = W.make_inputs(wl, seed=3)
    params = {"router": inp.router, "expert_w_gate": inp.w_gate, "expert_w_up": inp.w_up,
              "expert_w_down": inp.w_down}
    kw = dict(top_k=wl.top_k, routing="softmax", capacity_factor=wl.capacity_factor,
              logits=inp.logits if wl.router_from_logits else None)
    ref16 = O.moe_forward(inp.x, params, precision="bf16", **kw)
    ref64 = O.moe_forward(inp.x, params, precision="fp32", **kw)
    res = DeviceLayer(inp, gpu).forward()
    torch.cuda.synchronize()
    check_routing_and_plan(res, ref16["top_idx"], ref16["gates"], ref16["plan"])
    out = host(res["out"])
    e16 = O.normwise_rel_err(out, ref16["out"])
    e64 = O.normwise_rel_err(out, ref64["out"])
    print(f"{name} T={wl.tokens}: normwise err {e16:.3e} against the bf16-mode oracle, "
          f"{e64:.3e} against the float64 result", flush=True)
    assert e16 < 5e-3
    assert e64 < BF16_TOL


@pytest.mark.parametrize("name", ["full_bf16", "skewed_bf16"])
def test_workload_full_size(gpu, name):
    wl = W.WORKLOADS[name]
    print(f"layer {name} full size T={wl.tokens}", flush=True)
    inp = W.make_inputs(wl, seed=0)
    logits, idx, gates, plan = oracle_routing(inp)
    layer = DeviceLayer(inp, gpu)
    res = layer.forward()
    torch.cuda.synchronize()
    check_routing_and_plan(res, idx, gates, plan, None if wl.router_from_logits else logits)
    dropped = 1.0 - plan["keep"].mean()
    print(f"{name}: dropped fraction {dropped:.4f}, counts min/max "
          f"{plan['counts'].min()}/{plan['counts'].max()}", flush=True)
    out = host(res["out"])
    ref = full_output_ref(inp.x, inp.w_gate, inp.w_up, inp.w_down, gates, plan, wl.top_k)
    err = O.normwise_rel_err(out, ref)
    tok = np.linalg.norm(out - ref, axis=1) / np.maximum(np.linalg.norm(ref, axis=1), 1e-30)
    print(f"{name}: whole output [{wl.tokens}, {wl.d_model}] normwise rel err {err:.3e}, "
          f"worst token {tok.max():.3e}, max abs / max |ref| "
          f"{np.abs(out - ref).max() / np.abs(ref).max():.3e}", flush=True)
    assert err < BF16_TOL
    # every token, not only the whole output: one wrong K step in one of the
    # thousands of persistent tiles moves the normwise figure by ~1e-3 but
    # puts that tile's tokens far above this bound
    assert tok.max() < WORST_TOKEN_TOL_BF16, f"worst token {tok.max():.3e}"
    # against the oracle's bf16 mode (the reference's rounding points) on 256
    # evenly spaced tokens and the worst one above: what is left is the
    # summation order's bf16 rounding flips, well under the rounding points'
    # own distance to the float32 layer
    sample = np.unique(np.concatenate([np.linspace(0, wl.tokens - 1, 256).astype(np.int64),
                                       [int(tok.argmax())]]))
    b16 = bf16_mode_tokens(inp.x, inp.w_gate, inp.w_up, inp.w_down, gates, plan, wl.top_k,
                           sample, wl.out_dtype)
    err_b = O.normwise_rel_err(out[sample], b16)
    tok_b = (np.linalg.norm(out[sample] - b16, axis=1)
             / np.maximum(np.linalg.norm(b16, axis=1), 1e-30))
    print(f"{name}: {sample.size} sampled tokens against the bf16 mode: normwise err "
          f"{err_b:.3e}, worst token {tok_b.max():.3e}", flush=True)
    # measured 2.0e-4 / 7.0e-4 (full_bf16), 1.9e-4 / 1.2e-3 (skewed_bf16)
    assert err_b < 1e-3
    assert tok_b.max() < 5e-3, f"worst sampled token {tok_b.max():.3e}"
    # size-independent property: the fused gate/up (rows gathered from x by
    # the GEMM) equals the unfused permute + gate/up on the kept rows, bit for bit
    import hanuman_amd.kernels as K
    p = res["plan"]
    total = int(plan["offsets"][-1])
    xs = K.permute_rows(layer.x, p, torch.bfloat16)
    j = torch.from_numpy(np.nonzero(plan["perm_src"] >= 0)[0][::997]).to(gpu)
    src_tok = torch.from_numpy(plan["perm_src"]).to(gpu)[j] // wl.top_k
    assert torch.equal(xs[j], layer.x[src_tok].to(torch.bfloat16))
    h_unfused = K.grouped_gate_up(xs, p.offsets, layer.w_gate_up)
    assert res["h"] is not None and torch.equal(res["h"][:total], h_unfused[:total]), "fused gate/up"



def test_dispatch_identity_full_size(gpu):
    wl = W.WORKLOADS["dispatch_identity"]
    inp = W.make_inputs(wl, seed=0)
    logits, idx, gates, plan = oracle_routing(inp)
    res = DeviceLayer(inp, gpu).forward()
    torch.cuda.synchronize()
    check_routing_and_plan(res, idx, gates, plan)
    ref = O.combine_identity(inp.x, plan["slot_pos"], gates, wl.tokens, wl.top_k)
    assert np.array_equal(host(res["out"]).view(np.uint32), ref.view(np.uint32))
    assert 0.0 < 1.0 - plan["keep"].mean() < 0.02


def _params_np(m: MoE) -> dict:
    return {k: p.value.float().cpu().numpy() for k, p in m.named_params().items()}


@pytest.mark.parametrize("n_shared", [1, 2])
def test_moe_module_reference_mode(gpu, n_shared):
    B, S, D, F, N, Kk = 2, 96, 256, 128, 8, 2
    m = MoE(D, F, N, Kk, n_shared, 0.05, 2.5, torch.bfloat16, rngs=0, device=gpu)
    m.bias.value.copy_(torch.linspace(-0.02, 0.02, N, device=gpu))
    x = torch.randn(B, S, D, generator=torch.Generator(device=gpu).manual_seed(3), device=gpu)
    x = x.to(torch.bfloat16)
    out, aux = m(x)
    torch.cuda.synchronize()
    p = _params_np(m)
    xn = x.float().cpu().numpy().reshape(B * S, D)
    ref = O.moe_forward(xn, p, top_k=Kk, routing="sigmoid", routed_scaling_factor=2.5,
                        n_shared=n_shared, dtype="bf16", precision="fp32", batch_shape=(B, S))
    assert out.dtype == torch.float32 and tuple(out.shape) == (B, S, D)
    err = O.normwise_rel_err(host(out).reshape(B * S, D), ref["out"])
    print(f"MoE reference mode n_shared={n_shared}: normwise rel err {err:.3e}", flush=True)
    assert err < BF16_TOL
    a = ref["aux"]
    assert np.allclose([float(aux["router_z_loss"]), float(aux["balance_loss"]),
                        float(aux["mean_entropy"])],
                       [a["router_z_loss"], a["balance_loss"], a["mean_entropy"]], rtol=2e-5)
    assert np.array_equal(host(aux["expert_counts"]), a["expert_counts"])


@pytest.mark.parametrize("n_shared", [1, 2])
def test_moe_module_float32_input_promotes_shared_expert(gpu, n_shared):
    """bf16 compute with a float32 x: the routed experts see bf16(x)
    (moe.py:198), the shared expert x as given (moe.py:249), so its SwiGLU
    runs in float32 on the bf16-rounded weights. The shared output matches
    the oracle's promoted SwiGLU to float32 accuracy (the bf16 path would be
    ~3e-3 away), the layer output the bf16-mode oracle."""
    B, S, D, F, N, Kk = 2, 192, 256, 256, 8, 2
    m = MoE(D, F, N, Kk, n_shared, 0.05, 2.5, torch.bfloat16, rngs=3, device=gpu)
    x = torch.randn(B, S, D, generator=torch.Generator(device=gpu).manual_seed(6), device=gpu)
    print(f"module float32 x, n_shared={n_shared}", flush=True)
    out, _ = m(x)
    sh = m._shared_ffn_promoted(x.reshape(B * S, D).contiguous())
    torch.cuda.synchronize()
    p = _params_np(m)
    xn = x.cpu().numpy().reshape(B * S, D)
    sh_ref = O.shared_expert(xn, p["shared_w_gate"], p["shared_w_up"], p["shared_w_down"],
                             n_shared, "bf16_promoted")
    err_sh = O.normwise_rel_err(host(sh), sh_ref)
    err_bf = O.normwise_rel_err(O.shared_expert(O.bf16_round(xn), p["shared_w_gate"],
                                                p["shared_w_up"], p["shared_w_down"], n_shared,
                                                "bf16"), sh_ref)
    ref = O.moe_forward(xn, p, top_k=Kk, routing="sigmoid", routed_scaling_factor=2.5,
                        n_shared=n_shared, dtype="bf16", precision="bf16", x_dtype="f32")
    err = O.normwise_rel_err(host(out).reshape(B * S, D), ref["out"])
    print(f"  shared vs promoted oracle {err_sh:.2e} (bf16 path {err_bf:.2e}); out {err:.2e}",
          flush=True)
    assert err_sh < 1e-5 and err_bf > 1e-3
    assert err < 5e-3


def test_moe_module_capacity_softmax(gpu):
    B, S, D, F, N, Kk = 1, 512, 512, 256, 16, 4
    m = MoE(D, F, N, Kk, 1, 0.5, 1.0, "bfloat16", rngs=7, device=gpu, routing="softmax",
            capacity_factor=0.5)
    x = torch.randn(B, S, D, generator=torch.Generator(device=gpu).manual_seed(4), device=gpu)
    out, aux = m(x.to(torch.bfloat16))
    torch.cuda.synchronize()
    p = _params_np(m)
    xn = x.to(torch.bfloat16).float().cpu().numpy().reshape(B * S, D)
    ref = O.moe_forward(xn, p, top_k=Kk, routing="softmax", capacity_factor=0.5, n_shared=1,
                        dtype="bf16", precision="fp32")
    assert (ref["plan"]["keep"] == 0).any()
    err = O.normwise_rel_err(host(out).reshape(B * S, D), ref["out"])
    assert err < BF16_TOL


FP8_TOL = 5e-2


def _fp8_refs(inp, wl):
    params = {"router": inp.router, "expert_w_gate": inp.w_gate, "expert_w_up": inp.w_up,
              "expert_w_down": inp.w_down}
    r8 = O.moe_forward(inp.x, params, top_k=wl.top_k, routing="softmax",
                       capacity_factor=wl.capacity_factor, expert="swiglu_fp8", out_dtype="bf16")
    ref = O.moe_forward(inp.x, {**params, **O.dequantized_weights(r8["fp8"])}, top_k=wl.top_k,
                        routing="softmax", capacity_factor=wl.capacity_factor, precision="fp32")
    return r8, ref


def test_fp8_workload_reduced_tokens(gpu):
    """fp8 experts (e4m3 activations per token, weights per output channel):
    routing, plan and dispatched codes bit-exact; output within 5e-2 normwise
    of the float32 layer on the dequantised weights."""
    wl = W.WORKLOADS["fp8_experts"].scaled(1024)
    print(f"layer fp8_experts T={wl.tokens}", flush=True)
    inp = W.make_inputs(wl, seed=0)
    r8, ref = _fp8_refs(inp, wl)
    res = DeviceLayer(inp, gpu).forward()
    torch.cuda.synchronize()
    check_routing_and_plan(res, r8["top_idx"], r8["gates"], r8["plan"], r8["logits"])
    total = int(r8["plan"]["offsets"][-1])
    xs_q, xs_s = res["xs"].cpu().numpy(), res["xs_scale"].cpu().numpy()
    if res["xs_per_token"]:
        # per-token codes, gathered by the gate/up GEMM through perm_src
        src = r8["plan"]["perm_src"][:total] // wl.top_k
        xs_q, xs_s = xs_q[src], xs_s[src]
    assert np.array_equal(xs_q[:total], r8["xs"][:total]), "xs codes"
    assert np.array_equal(xs_s[:total], r8["xs_s"][:total]), "xs scales"
    out = host(res["out"])
    assert res["out"].dtype == torch.bfloat16
    err = O.normwise_rel_err(out, ref["out"])
    err_emul = O.normwise_rel_err(out, r8["out"])
    print(f"fp8: normwise err vs fp32 on dequantised weights {err:.3e}, vs fp8 emulation {err_emul:.3e}",
          flush=True)
    assert err < FP8_TOL
    assert err_emul < 1e-2


def test_fp8_workload_full_size(gpu):
    wl = W.WORKLOADS["fp8_experts"]
    print(f"layer fp8_experts full size T={wl.tokens}", flush=True)
    inp = W.make_inputs(wl, seed=0)
    logits = O.router_logits(inp.x, inp.router)
    idx, gates = O.route_softmax(logits, wl.top_k)
    plan = O.dispatch_plan(idx, wl.n_experts, wl.capacity)
    layer = DeviceLayer(inp, gpu)
    res = layer.forward()
    torch.cuda.synchronize()
    check_routing_and_plan(res, idx, gates, plan, logits)
    # sampled tokens against the float32 layer on the dequantised weights
    wq = O.quantize_expert_weights({"expert_w_gate": inp.w_gate, "expert_w_up": inp.w_up,
                                    "expert_w_down": inp.w_down})
    deq = O.dequantized_weights(wq)
    out = host(res["out"])
    ref = full_output_ref(inp.x, deq["expert_w_gate"], deq["expert_w_up"], deq["expert_w_down"],
                          gates, plan, wl.top_k)
    err = O.normwise_rel_err(out, ref)
    tok = np.linalg.norm(out - ref, axis=1) / np.maximum(np.linalg.norm(ref, axis=1), 1e-30)
    # the same layer on the unquantised float32 weights: reported, not bounded
    # (the e4m3 rule's own error there is ~6.5 %)
    ref32 = full_output_ref(inp.x, inp.w_gate, inp.w_up, inp.w_down, gates, plan, wl.top_k)
    err32 = O.normwise_rel_err(out, ref32)
    print(f"fp8 full size: whole output normwise err {err:.3e} (worst token {tok.max():.3e}) "
          f"against the float32 layer on the dequantised weights; {err32:.3e} against the "
          f"unquantised float32 weights", flush=True)
    assert err < FP8_TOL
    assert tok.max() < WORST_TOKEN_TOL_FP8, f"worst token {tok.max():.3e}"
    # Against the fp8 rule itself (activations quantised as the kernels do),
    # on 256 evenly spaced tokens and the worst one above: the distance left
    # is the kernels' float32 accumulation (rare bf16 / e4m3 rounding flips),
    # not the e4m3 rule's own ~5 %.
    sample = np.unique(np.concatenate([np.linspace(0, wl.tokens - 1, 256).astype(np.int64),
                                       [int(tok.argmax())]]))
    emu = fp8_emulated_tokens(inp.x, wq, gates, plan, wl.top_k, sample)
    err_emu = O.normwise_rel_err(out[sample], emu)
    tok_emu = (np.linalg.norm(out[sample] - emu, axis=1)
               / np.maximum(np.linalg.norm(emu, axis=1), 1e-30))
    print(f"fp8 full size: {sample.size} sampled tokens against the fp8 emulation: normwise "
          f"err {err_emu:.3e}, worst token {tok_emu.max():.3e}", flush=True)
    assert err_emu < 1e-2
    assert tok_emu.max() < 2e-2, f"worst sampled token {tok_emu.max():.3e}"


@pytest.mark.parametrize("n_shared,routing,cf", [(1, "sigmoid", None), (2, "softmax", 1.25)])
def test_moe_module_float32_compute(gpu, n_shared, routing, cf):
    """dtype float32 (the tiny configuration's fp32): experts and shared
    expert on the float32 matrix cores, gates kept float32 in the combine
    (moe.py:84 casts them to the rows' dtype); against the oracle's float64
    arithmetic on the same values."""
    B, S, D, F, N, Kk = 4, 128, 256, 512, 8, 2
    m = MoE(D, F, N, Kk, n_shared, 0.05, 2.5, torch.float32, rngs=2, device=gpu,
            routing=routing, capacity_factor=cf)
    if routing == "sigmoid":
        m.bias.value.copy_(torch.linspace(-0.02, 0.02, N, device=gpu))
    x = torch.randn(B, S, D, generator=torch.Generator(device=gpu).manual_seed(4), device=gpu)
    out, aux = m(x)
    torch.cuda.synchronize()
    p = _params_np(m)
    xn = x.cpu().numpy().reshape(B * S, D)
    ref = O.moe_forward(xn, p, top_k=Kk, routing=routing, routed_scaling_factor=2.5,
                        capacity_factor=cf, n_shared=n_shared, dtype="f32", precision="fp32",
                        batch_shape=(B, S))
    err = O.normwise_rel_err(host(out).reshape(B * S, D), ref["out"])
    print(f"float32 MoE n_shared={n_shared} {routing}: normwise rel err {err:.3e}", flush=True)
    assert out.dtype == torch.float32 and err < 1e-5
