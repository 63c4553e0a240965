"""The bf16 layer forward captured into a HIP graph (needs an MI355X).

Every kernel of the path takes its stream from the caller and allocates
nothing itself (outputs and the plan's workspace come from torch's allocator,
which serves a capture from the graph's private pool), so the whole forward
-- router, plan, gathering gate/up GEMM, down GEMM, combine -- can be
captured once and replayed.  Each replay runs on new token values written
into the captured input and is compared bit for bit with an eager forward
on the same values, with that eager work between the replays.
"""
import numpy as np
import pytest
import torch

import oracle as O
from hanuman_amd import _lib
from hanuman_amd import kernels as K

pytestmark = pytest.mark.gpu


def forward(x, router_w, wgu, wdp, n_experts, top_k, cap):
    logits, idx, gates = K.router(x, router_w, None, top_k, _lib.ROUTE_SOFTMAX)
    plan = K.dispatch_plan(idx, n_experts, cap)
    h = K.grouped_gate_up_gather(x, plan, wgu)
    ys = K.grouped_down(h, plan.offsets, wdp)
    out = K.combine(ys, plan, gates, None, torch.float32)
    return {"logits": logits, "top_idx": idx, "gates": gates, "offsets": plan.offsets,
            "perm_src": plan.perm_src, "out": out}


def test_layer_forward_replays_from_a_hip_graph(gpu):
    T, D, N, Kk, F = 1024, 256, 8, 2, 256
    print(f"graph capture T={T} D={D} N={N} K={Kk} F={F}", flush=True)
    rng = np.random.default_rng(41)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    draw_x = lambda: dev(O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))).to(torch.bfloat16)
    router_w = dev((0.05 * rng.standard_normal((D, N))).astype(np.float32))
    wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
    wd = (0.02 * rng.standard_normal((N, F, D))).astype(np.float32)
    wgu, wdp = K.pack_gate_up(dev(wg), dev(wu)), K.pack_down(dev(wd))
    cap = K.capacity(T, Kk, N, 1.0)            # with drops
    x = draw_x()                               # the captured input
    args = (router_w, wgu, wdp, N, Kk, cap)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):              # warm-up outside the capture
        forward(x, *args)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = forward(x, *args)
    torch.cuda.synchronize()

    for r in range(4):
        x.copy_(draw_x())
        graph.replay()
        torch.cuda.synchronize()
        eager = forward(x.clone(), *args)
        torch.cuda.synchronize()
        for k, v in eager.items():
            assert torch.equal(captured[k], v), f"replay {r}: {k} differs from the eager forward"
        print(f"  replay {r}: kept {int(eager['offsets'][-1])} rows, bit-identical", flush=True)
