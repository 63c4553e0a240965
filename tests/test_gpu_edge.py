"""Empty and degenerate inputs through the C ABI (needs an MI355X).

* zero tokens: every stage of the bf16 and fp8 layer paths is a no-op that
  returns empty outputs (the plan's counts and offsets all zero);
* top_k equal to the expert count, a single expert, and every token's first
  choice on one expert far past its capacity (heavy drops): routing and plan
  bit-exact against the oracle, the layer output within the bf16 tolerance
  of the oracle's float32 result on the same plan.
"""
import numpy as np
import pytest
import torch

import oracle as O
from hanuman_amd import _lib
from hanuman_amd import kernels as K

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def host(t):
    return t.float().cpu().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()


def bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float32:
        a, b = a.view(np.uint32), np.asarray(b, np.float32).view(np.uint32)
    return a.shape == b.shape and np.array_equal(a, b)


def test_zero_tokens_is_a_no_op(gpu):
    D, N, Kk, F = 256, 8, 2, 128
    print("zero tokens", flush=True)
    rng = np.random.default_rng(3)
    x = torch.empty((0, D), dtype=torch.bfloat16, device=gpu)
    w = torch.from_numpy((0.02 * rng.standard_normal((D, N))).astype(np.float32)).to(gpu)
    logits, idx, gates = K.router(x, w, None, Kk, _lib.ROUTE_SOFTMAX)
    cap = K.capacity(0, Kk, N, 1.25)
    plan = K.dispatch_plan(idx, N, cap)
    wg, wu = (torch.from_numpy((0.02 * rng.standard_normal((N, D, F))).astype(np.float32)).to(gpu)
              for _ in range(2))
    wd = torch.from_numpy((0.02 * rng.standard_normal((N, F, D))).astype(np.float32)).to(gpu)
    wgu, wdp = K.pack_gate_up(wg, wu), K.pack_down(wd)
    h = K.grouped_gate_up_gather(x, plan, wgu)
    ys = K.grouped_down(h, plan.offsets, wdp)
    out = K.combine(ys, plan, gates, None, torch.float32)
    fgu, sgu = K.pack_fp8_gate_up(wg, wu)
    fd, sd = K.pack_fp8_down(wd)
    x_q, x_s = K.quantize_rows_fp8(x)
    h8 = K.grouped_gate_up_fp8_gather(x_q, x_s, plan, fgu, sgu)
    h_q, h_s = K.quantize_rows_fp8(h8, plan.offsets)
    ys8 = K.grouped_down_fp8(h_q, h_s, plan.offsets, fd, sd)
    out8 = K.combine(ys8, plan, gates, None, torch.bfloat16)
    hb_q, hb_e = K.grouped_gate_up_fp8_gather_qh(x_q, x_s, plan, fgu, sgu)
    ysb = K.grouped_down_fp8_mx(hb_q, hb_e, plan.offsets, fd, sd)
    torch.cuda.synchronize()
    assert hb_q.shape[0] == 0 and hb_e.shape[0] == 0 and ysb.shape[0] == 0
    assert tuple(logits.shape) == (0, N) and tuple(idx.shape) == (0, Kk)
    assert plan.rows_cap == 0
    assert host(plan.counts).tolist() == [0] * N and host(plan.offsets).tolist() == [0] * (N + 1)
    assert h.shape[0] == 0 and ys.shape[0] == 0 and tuple(out.shape) == (0, D)
    assert h8.shape[0] == 0 and ys8.shape[0] == 0 and tuple(out8.shape) == (0, D)


def _run_layer(gpu, x, router_w, logits_in, wg, wu, wd, Kk, cf):
    """The bf16 layer path (router or given logits, plan, gathered gate/up,
    down, combine) on the kernels, plus the oracle's routing, plan and
    float32 output."""
    T, D = x.shape
    N = wg.shape[0]
    xt = torch.from_numpy(x).to(gpu, torch.bfloat16)
    if logits_in is None:
        logits, idx, gates = K.router(xt, torch.from_numpy(router_w).to(gpu), None, Kk,
                                      _lib.ROUTE_SOFTMAX)
        ref_logits = O.router_logits(x, router_w)
    else:
        logits = torch.from_numpy(logits_in).to(gpu)
        idx, gates = K.router_from_logits(logits, None, Kk, _lib.ROUTE_SOFTMAX)
        ref_logits = logits_in
    cap = K.capacity(T, Kk, N, cf)
    plan = K.dispatch_plan(idx, N, cap)
    dev = lambda a: torch.from_numpy(a).to(gpu)
    h = K.grouped_gate_up_gather(xt, plan, K.pack_gate_up(dev(wg), dev(wu)))
    ys = K.grouped_down(h, plan.offsets, K.pack_down(dev(wd)))
    out = K.combine(ys, plan, gates, None, torch.float32)
    torch.cuda.synchronize()
    ref_idx, ref_gates = O.route_softmax(ref_logits, Kk)
    ref_plan = O.dispatch_plan(ref_idx, N, O.capacity_of(T, Kk, N, cf))
    assert bits_equal(host(logits), ref_logits), "logits"
    assert bits_equal(host(idx), ref_idx), "top_idx"
    assert bits_equal(host(gates), ref_gates), "gates"
    for k in ("counts", "offsets", "slot_pos", "perm_src", "keep"):
        assert np.array_equal(host(getattr(plan, k)), ref_plan[k]), k
    xs = O.permute_rows(x, ref_plan["perm_src"], Kk)
    ys_ref = O.expert_ffn(xs, ref_plan["offsets"], wg, wu, wd, precision="fp32")
    ref = O.combine(ys_ref, ref_plan["slot_pos"], ref_gates, T, Kk, ys_dtype="bf16")
    return host(out), ref, ref_plan


@pytest.mark.parametrize("case", ["top_k_equals_n_experts", "single_expert", "all_to_one_expert"])
def test_degenerate_routing(gpu, case):
    print(f"edge case {case}", flush=True)
    rng = np.random.default_rng({"top_k_equals_n_experts": 61, "single_expert": 62,
                                 "all_to_one_expert": 63}[case])
    D, F = 256, 256
    if case == "top_k_equals_n_experts":
        T, N, Kk, cf = 300, 8, 8, None
    elif case == "single_expert":
        T, N, Kk, cf = 500, 1, 1, None
    else:
        T, N, Kk, cf = 700, 8, 2, 1.0
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    router_w = (0.02 * rng.standard_normal((D, N))).astype(np.float32)
    wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
    wd = (0.02 * rng.standard_normal((N, F, D))).astype(np.float32)
    logits_in = None
    if case == "all_to_one_expert":
        # every token's first choice is expert 3: its capacity ceil(T K / N) = 175
        # keeps the first 175 tokens' slots there and drops the rest
        logits_in = rng.standard_normal((T, N)).astype(np.float32)
        logits_in[:, 3] += 10.0
    out, ref, plan = _run_layer(gpu, x, router_w, logits_in, wg, wu, wd, Kk, cf)
    if case == "all_to_one_expert":
        assert plan["counts"][3] == T and plan["offsets"][4] - plan["offsets"][3] == 175
        assert (plan["keep"] == 0).sum() == T - 175
    err = O.normwise_rel_err(out, ref)
    print(f"  output normwise err {err:.2e}", flush=True)
    assert err < BF16_TOL
