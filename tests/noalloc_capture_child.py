"""Child process of tests/test_zz_no_alloc.py (run with a GPU, never imported
by pytest): the process's first hmoe_dispatch_plan_noalloc call is made
inside a torch.cuda.graph capture, so the scratch array's address is looked
up for the first time during capture.  The graph is replayed on two
routings written into the captured input, with eager work in between, and
every replay is compared bit for bit with hmoe_dispatch_plan (caller
workspace) on the same input.  Prints "noalloc capture ok" on success."""
import ctypes
import os
import sys

import numpy as np
import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
from hanuman_amd import _lib  # noqa: E402


def main():
    dev = torch.device("cuda:0")
    lib = _lib.lib()
    T, K, N = 3000, 4, 48
    cap = int(lib.hmoe_capacity(T, K, N, 1.25))
    rows_cap = int(lib.hmoe_rows_cap(T, K, N, cap))
    rng = np.random.default_rng(5)

    def routing():
        p = np.arange(1, N + 1, dtype=np.float64) ** -1.2
        lg = np.log(p)[None, :] + rng.gumbel(size=(T, N))
        return torch.from_numpy(np.argsort(-lg, axis=1, kind="stable")[:, :K].astype(np.int32))

    def outs():
        return [torch.full((N,), -7, dtype=torch.int32, device=dev),
                torch.full((N + 1,), -7, dtype=torch.int32, device=dev),
                torch.full((T * K,), -7, dtype=torch.int32, device=dev),
                torch.full((rows_cap,), -7, dtype=torch.int32, device=dev),
                torch.full((T * K,), 7, dtype=torch.uint8, device=dev)]

    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    idx = routing().to(dev)
    got = outs()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = lib.hmoe_dispatch_plan_noalloc(P(idx), T, K, N, cap, *map(P, got), s)
    assert rc == _lib.OK, lib.hmoe_last_error().decode()
    ws = torch.empty(int(lib.hmoe_plan_workspace_bytes(T, K, N)), dtype=torch.uint8, device=dev)
    for rep in range(2):
        if rep:
            idx.copy_(routing().to(dev))
        g.replay()
        torch.cuda.synchronize()
        _ = (torch.randn(1000, device=dev) * 2).sum().item()   # eager work between replays
        ref = outs()
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        assert lib.hmoe_dispatch_plan(P(idx), T, K, N, cap, *map(P, ref), P(ws), ws.numel(), s) == 0
        torch.cuda.synchronize()
        for a, b in zip(got, ref):
            assert torch.equal(a, b), f"replay {rep} differs"
    print("noalloc capture ok", flush=True)


if __name__ == "__main__":
    main()
