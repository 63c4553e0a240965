"""Golden fixtures (``tests/golden/*.npz``, written by
``tests/golden/make_fixtures.py`` from the oracle).

CPU: the oracle reproduces every fixture bit for bit (a change to the oracle's
rules shows up here).  GPU: the HIP path matches the fixtures -- routing and
dispatch plan bit-exact, identity-expert output bit-exact, SwiGLU output
within the bf16 tolerance (2e-2 normwise).  Inputs are regenerated from the
workloads' seeded generators.
"""
import os

import numpy as np
import pytest

import oracle as O
from hanuman_amd import workloads as W

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")


def _load(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _make(name):
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_fixtures",
                                                  os.path.join(GOLDEN, "make_fixtures.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.FIXTURES[name]()


@pytest.mark.parametrize("name", ["tiny_fp32", "dispatch_identity_256", "reference_mode"])
def test_oracle_reproduces_fixture(name):
    want = _load(name)
    got = _make(name)
    assert sorted(got) == sorted(want)
    for k in want:
        a, b = np.asarray(got[k]), want[k]
        assert a.shape == b.shape and a.dtype == b.dtype, k
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), k


def test_fixture_invariants():
    """Size-independent facts the fixtures must satisfy."""
    f = _load("tiny_fp32")
    T, K = f["top_idx"].shape
    assert f["plan_counts"].sum() == T * K
    kept = f["plan_slot_pos"][f["plan_slot_pos"] >= 0]
    assert np.array_equal(np.sort(kept), np.arange(f["plan_offsets"][-1]))
    assert np.allclose(f["gates"].sum(axis=1), 1.0, atol=1e-6)
    r = _load("reference_mode")
    assert r["aux_expert_counts"].sum() == r["top_idx"].size


@pytest.mark.gpu
def test_gpu_matches_tiny_fixture(gpu):
    import torch
    from hanuman_amd.layer import DeviceLayer
    f = _load("tiny_fp32")
    wl = W.WORKLOADS["tiny_fp32"]
    res = DeviceLayer(W.make_inputs(wl, seed=0), gpu).forward()
    torch.cuda.synchronize()
    assert np.array_equal(res["logits"].cpu().numpy().view(np.uint32), f["logits"].view(np.uint32))
    assert np.array_equal(res["top_idx"].cpu().numpy(), f["top_idx"])
    assert np.array_equal(res["gates"].cpu().numpy().view(np.uint32), f["gates"].view(np.uint32))
    for k in ("counts", "offsets", "slot_pos", "perm_src", "keep"):
        assert np.array_equal(getattr(res["plan"], k).cpu().numpy(), f[f"plan_{k}"]), k
    out = res["out"].cpu().numpy()[: f["out"].shape[0]]
    assert O.normwise_rel_err(out, f["out"]) < 2e-2


@pytest.mark.gpu
def test_gpu_matches_identity_fixture(gpu):
    import torch
    from hanuman_amd.layer import DeviceLayer
    f = _load("dispatch_identity_256")
    wl = W.WORKLOADS["dispatch_identity"].scaled(256)
    res = DeviceLayer(W.make_inputs(wl, seed=0), gpu).forward()
    torch.cuda.synchronize()
    assert np.array_equal(res["top_idx"].cpu().numpy(), f["top_idx"])
    for k in ("counts", "offsets", "slot_pos", "perm_src", "keep"):
        assert np.array_equal(getattr(res["plan"], k).cpu().numpy(), f[f"plan_{k}"]), k
    out = res["out"].cpu().numpy()[: f["out"].shape[0]]
    assert np.array_equal(out.view(np.uint32), f["out"].view(np.uint32))
