"""The fused gate/up + down launch (``hmoe_grouped_swiglu_fused``) against the
two launches it replaces (needs an MI355X).

The fused launch runs the same tile code as ``hmoe_grouped_gate_up_gather``
and ``hmoe_grouped_down``; only the schedule differs (per-XCD work lists,
claimed tiles, down tiles waiting for their m-tile's gate/up tiles), so h
and ys must be bit-identical to the two-launch path on every shape: many
tiles per workgroup, fewer m-tiles than XCDs (idle XCDs), empty experts,
capacity drops, one expert, and calls in a row on one workspace.  The give-up
path of the bounded wait is forced from the host (a ready count no gate/up
tile can reach, a short time limit): every launch still exits, the status
word says so, and h, which no wait guards, stays exact.
"""
import numpy as np
import pytest
import torch

import oracle as O
from hanuman_amd import kernels as K

pytestmark = pytest.mark.gpu


def _case(gpu, T, D, F, N, Kk, cap_factor, seed, skew=2.0):
    rng = np.random.default_rng(seed)
    p = np.exp(-skew * np.linspace(0.0, 1.0, N))
    if N > 4:
        p[N // 3] = 1e-12            # one expert never chosen
    p = p[rng.permutation(N)]
    p /= p.sum()
    keys = np.log(rng.random((T, N))) / p
    top = np.argsort(-keys, axis=1, kind="stable")[:, :Kk].astype(np.int32)
    cap = O.capacity_of(T, Kk, N, cap_factor)
    plan = K.dispatch_plan(torch.from_numpy(top).to(gpu), N, cap)
    x = torch.from_numpy(O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))).to(gpu)
    x = x.to(torch.bfloat16)
    wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
    wd = (0.02 * rng.standard_normal((N, F, D))).astype(np.float32)
    wgu = K.pack_gate_up(torch.from_numpy(wg).to(gpu), torch.from_numpy(wu).to(gpu))
    wdn = K.pack_down(torch.from_numpy(wd).to(gpu))
    return x, plan, wgu, wdn


CASES = [
    # T, D, F, N, K, capacity factor
    (4096, 2048, 1024, 64, 8, None),      # ~5 tiles per workgroup, ragged 0..1200 rows
    (2000, 512, 256, 16, 4, 0.75),        # capacity drops
    (300, 256, 256, 8, 2, None),          # few tiles: down tiles wait on gate/up tiles
    (100, 256, 512, 4, 2, None),          # at most 4 m-tiles: some XCDs have no work
    (700, 1024, 384, 1, 1, None),         # one expert
    (16384, 2048, 1024, 64, 8, 1.25),     # the full bf16 workload's shape
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "T{}_D{}_F{}_N{}_K{}_cf{}".format(*c))
def test_fused_matches_two_launches(gpu, case):
    T, D, F, N, Kk, cf = case
    print(f"fused case {case}", flush=True)
    x, plan, wgu, wdn = _case(gpu, T, D, F, N, Kk, cf, seed=T + D + N)
    h_ref = K.grouped_gate_up_gather(x, plan, wgu)
    ys_ref = K.grouped_down(h_ref, plan.offsets, wdn)
    h, ys, ws = K.grouped_swiglu_fused(x, plan, wgu, wdn)
    torch.cuda.synchronize()
    R = int(plan.offsets[-1].item())
    assert R > 0
    assert K.fused_status(ws) == 0
    assert torch.equal(h[:R], h_ref[:R]), "h differs from the gathered gate/up GEMM"
    assert torch.equal(ys[:R], ys_ref[:R]), "ys differs from the down GEMM"


def test_fused_calls_in_a_row_share_a_workspace(gpu):
    """Two routings through one workspace, the second smaller: both
    bit-identical to the two-launch path, and after each call every word of
    the workspace but the status is back at zero (the last workgroup clears
    the counters, so the next call needs no clearing)."""
    ws = None
    for T, seed in ((3000, 1), (1100, 2)):
        x, plan, wgu, wdn = _case(gpu, T, 512, 512, 32, 4, None, seed)
        if ws is None:
            ws = K.grouped_swiglu_fused_workspace(plan)
        h, ys, _ = K.grouped_swiglu_fused(x, plan, wgu, wdn, workspace=ws)
        h_ref = K.grouped_gate_up_gather(x, plan, wgu)
        ys_ref = K.grouped_down(h_ref, plan.offsets, wdn)
        torch.cuda.synchronize()
        R = int(plan.offsets[-1].item())
        print(f"fused in a row T={T}: status {K.fused_status(ws)}", flush=True)
        assert K.fused_status(ws) == 0
        words = ws.view(torch.int32)
        assert int(words.ne(0).sum().item()) == 0, "counters left set"
        assert torch.equal(h[:R], h_ref[:R]) and torch.equal(ys[:R], ys_ref[:R])


def test_fused_wait_gives_up_when_forced(gpu):
    """A ready count no gate/up tile reaches (extra_ready_needed=1) with a
    50 us limit: every down tile's wait gives up, the launch exits, the status
    bit is set, and h (computed before any wait) is still exact."""
    x, plan, wgu, wdn = _case(gpu, 600, 256, 256, 8, 2, None, seed=9)
    print("fused forced give-up", flush=True)
    h, ys, ws = K.grouped_swiglu_fused(x, plan, wgu, wdn, wait_timeout_us=50, extra_ready_needed=1)
    torch.cuda.synchronize()
    assert K.fused_status(ws) & 1 == 1
    h_ref = K.grouped_gate_up_gather(x, plan, wgu)
    torch.cuda.synchronize()
    R = int(plan.offsets[-1].item())
    assert torch.equal(h[:R], h_ref[:R])
    # the same workspace serves a normal call afterwards
    h2, ys2, _ = K.grouped_swiglu_fused(x, plan, wgu, wdn, workspace=ws)
    ys_ref = K.grouped_down(h_ref, plan.offsets, wdn)
    torch.cuda.synchronize()
    assert K.fused_status(ws) == 0 and torch.equal(ys2[:R], ys_ref[:R])


def test_fused_refuses_unsupported_shapes(gpu):
    x, plan, wgu, wdn = _case(gpu, 200, 256, 128, 4, 2, None, seed=3)
    with pytest.raises(Exception, match="d_ff"):
        K.grouped_swiglu_fused(x, plan, wgu, wdn)
    ws = torch.zeros(8, dtype=torch.uint8, device=gpu)
    x, plan, wgu, wdn = _case(gpu, 200, 256, 256, 4, 2, None, seed=3)
    with pytest.raises(Exception, match="workspace"):
        K.grouped_swiglu_fused(x, plan, wgu, wdn, workspace=ws)
