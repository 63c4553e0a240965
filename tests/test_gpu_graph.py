"""The layer forward under HIP graph capture (needs an MI355X).

A caller such as an XLA command buffer records the layer's launches once and
replays them.  The library enqueues kernels only (no host synchronisation, no
allocation, no memset, launch shapes fixed by the call's sizes), so a captured
forward must recompute everything from whatever the input buffers hold at
replay time.  Each test captures ``DeviceLayer.forward`` once, then replays it
on two different token matrices written into the captured input buffer, with
eager work and synchronisations between the replays, and checks every replay
bit for bit against the eager forward on the same input.
"""
import pytest
import torch

from hanuman_amd import workloads as W
from hanuman_amd.layer import DeviceLayer

pytestmark = pytest.mark.gpu

KEYS = ("top_idx", "gates", "ys", "out")
PLAN_KEYS = ("counts", "offsets", "slot_pos", "perm_src", "keep")


def snapshot(res):
    snap = {k: res[k].clone() for k in KEYS}
    # dispatched rows past the kept ones are never written (left as allocated)
    snap["ys"] = res["ys"][: int(res["plan"].offsets[-1].item())].clone()
    if res.get("logits") is not None:
        snap["logits"] = res["logits"].clone()
    for k in PLAN_KEYS:
        snap["plan." + k] = getattr(res["plan"], k).clone()
    return snap


def assert_same(got, want, what):
    for k, v in want.items():
        g = got[k]
        assert g.dtype == v.dtype and g.shape == v.shape, (what, k)
        assert torch.equal(g.view(torch.uint8) if g.dtype.is_floating_point else g,
                           v.view(torch.uint8) if v.dtype.is_floating_point else v), (what, k)


@pytest.mark.parametrize("name,tokens,fused_ffn", [("full_bf16", 2048, False),
                                                   ("fp8_experts", 1024, False),
                                                   ("dispatch_identity", 4096, False),
                                                   ("skewed_bf16", 4096, False),
                                                   # the one-launch gate/up + down: its
                                                   # counters clear themselves, no memset
                                                   ("full_bf16", 2048, True),
                                                   ("skewed_bf16", 4096, True)])
def test_forward_graph_replays(gpu, name, tokens, fused_ffn):
    wl = W.WORKLOADS[name].scaled(tokens)
    print(f"graph {name} T={wl.tokens} fused_ffn={fused_ffn}", flush=True)
    layer = DeviceLayer(W.make_inputs(wl, seed=0), gpu, fused_ffn=fused_ffn)
    assert layer.fused_ffn == fused_ffn
    src = layer.logits_in if wl.router_from_logits else layer.x
    other = W.make_inputs(wl, seed=1)
    src_b = torch.from_numpy(other.logits if wl.router_from_logits else other.x)
    src_b = src_b.to(src.device, src.dtype).contiguous()
    src_a = src.clone()

    def eager(value):
        src.copy_(value)
        out = snapshot(layer.forward())
        torch.cuda.synchronize()
        return out

    want_a = eager(src_a)
    want_b = eager(src_b)
    assert not torch.equal(want_a["top_idx"], want_b["top_idx"])

    # warm-up on a side stream, as torch requires before capture
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        layer.forward()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    src.copy_(src_a)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        captured = layer.forward()

    for value, want, what in ((src_a, want_a, "replay a"), (src_b, want_b, "replay b"),
                              (src_a, want_a, "replay a again")):
        src.copy_(value)
        graph.replay()
        torch.cuda.synchronize()
        assert_same(snapshot(captured), want, what)
        # eager work between replays, on other buffers of the same layer
        eager(src_b if value is src_a else src_a)
        src.copy_(value)
        torch.cuda.synchronize()
    graph.reset()
