"""hmoe_dispatch_plan_noalloc (the plan with its histogram in the library's
fixed device scratch) against hmoe_dispatch_plan with a caller workspace,
called through the C ABI: two calls in a row, the second with a smaller
input (the scratch then holds the first call's larger histogram), every
output bit-exact; a plan larger than the scratch is refused with
HMOE_ERR_WORKSPACE and nothing is launched.  Needs an MI355X."""
import ctypes

import numpy as np
import pytest
import torch

from hanuman_amd import _lib

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _outputs(T, K, N, rows_cap, dev):
    return {"counts": torch.full((N,), -7, dtype=torch.int32, device=dev),
            "offsets": torch.full((N + 1,), -7, dtype=torch.int32, device=dev),
            "slot_pos": torch.full((T * K,), -7, dtype=torch.int32, device=dev),
            "perm_src": torch.full((rows_cap,), -7, dtype=torch.int32, device=dev),
            "keep": torch.full((T * K,), 7, dtype=torch.uint8, device=dev)}


def _run(noalloc, idx, N, cap, dev):
    lib = _lib.lib()
    T, K = idx.shape
    rows_cap = int(lib.hmoe_rows_cap(T, K, N, cap))
    o = _outputs(T, K, N, rows_cap, dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [_ptr(idx), T, K, N, cap, _ptr(o["counts"]), _ptr(o["offsets"]), _ptr(o["slot_pos"]),
            _ptr(o["perm_src"]), _ptr(o["keep"])]
    if noalloc:
        rc = lib.hmoe_dispatch_plan_noalloc(*args, stream)
    else:
        ws_bytes = int(lib.hmoe_plan_workspace_bytes(T, K, N))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        rc = lib.hmoe_dispatch_plan(*args, _ptr(ws), ws.numel(), stream)
    assert rc == _lib.OK, lib.hmoe_last_error().decode()
    torch.cuda.synchronize()
    return {k: v.cpu() for k, v in o.items()}


def _skewed_idx(rng, T, K, N):
    """top-k expert ids with a skewed load, so capacity drops occur."""
    p = np.arange(1, N + 1, dtype=np.float64) ** -1.2
    logits = np.log(p)[None, :] + rng.gumbel(size=(T, N))
    return np.argsort(-logits, axis=1, kind="stable")[:, :K].astype(np.int32)


@pytest.mark.parametrize("cf", [1.25, None])
def test_noalloc_plan_matches_workspace_plan(gpu, cf):
    rng = np.random.default_rng(11)
    # the second call is smaller than the first, and the first fills half of
    # the scratch (ceil(T*K/1024) * N = 131072 of the 262144 int32 it holds)
    for T, K, N in [(65536, 8, 256), (3000, 4, 48)]:
        cap = int(_lib.lib().hmoe_capacity(T, K, N, cf if cf else 0.0))
        print(f"noalloc plan T={T} K={K} N={N} cap={cap}", flush=True)
        idx = torch.from_numpy(_skewed_idx(rng, T, K, N)).to(gpu)
        ref = _run(False, idx, N, cap, gpu)
        got = _run(True, idx, N, cap, gpu)
        for k in ref:
            assert torch.equal(got[k], ref[k]), (T, K, N, k)
        if cf:
            assert int(ref["keep"].sum()) < T * K  # drops happened


def test_noalloc_plan_rejects_oversized_plan(gpu):
    lib = _lib.lib()
    T, K, N = 1 << 19, 8, 128            # ceil(T*K/1024) * N = 524288 > 262144
    dummy = torch.zeros(1, dtype=torch.int32, device=gpu)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = _ptr(dummy)
    rc = lib.hmoe_dispatch_plan_noalloc(p, T, K, N, T * K, p, p, p, p, p, stream)
    assert rc == _lib.ERR_WORKSPACE
    assert "scratch" in lib.hmoe_last_error().decode()


def test_noalloc_plan_first_call_inside_graph_capture(gpu):
    """In a fresh process, the first hmoe_dispatch_plan_noalloc call (which
    looks the scratch array's address up) is made during a HIP graph capture;
    the graph's replays match hmoe_dispatch_plan bit for bit."""
    import subprocess
    import sys
    from pathlib import Path
    child = Path(__file__).with_name("noalloc_capture_child.py")
    r = subprocess.run([sys.executable, str(child)], capture_output=True, text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "noalloc capture ok" in r.stdout
