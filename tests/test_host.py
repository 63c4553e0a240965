"""Host-side logic that needs no GPU: workload definitions, input generation,
and the drop-in module's constructor contract (parameter names and shapes of
``model/moe.py:126-159``)."""
import numpy as np
import pytest
import torch

import oracle as O
from hanuman_amd import workloads as W
from hanuman_amd.moe import MoE, Param


def test_workload_capacities():
    caps = {n: (w.capacity, w.rows_cap) for n, w in W.WORKLOADS.items()}
    assert caps["tiny_fp32"] == (640, 4096)
    assert caps["dispatch_identity"] == (4096, 262144)
    assert caps["full_bf16"] == (2560, 131072)
    assert caps["skewed_bf16"] == (5120, 524288)
    assert caps["fp8_experts"] == (1280, 32768)
    for w in W.WORKLOADS.values():
        assert w.capacity == O.capacity_of(w.tokens, w.top_k, w.n_experts, w.capacity_factor)


def test_inputs_are_seeded_and_bf16_rounded():
    wl = W.WORKLOADS["full_bf16"].scaled(64)
    a = W.make_inputs(wl, seed=0)
    b = W.make_inputs(wl, seed=0)
    c = W.make_inputs(wl, seed=1)
    assert np.array_equal(a.x, b.x) and np.array_equal(a.w_down, b.w_down)
    assert not np.array_equal(a.x, c.x)
    assert np.array_equal(a.x, O.bf16_round(a.x))
    assert a.router.shape == (2048, 64) and a.w_gate.shape == (64, 2048, 1024)
    assert abs(float(a.w_gate.std()) - 0.02) < 1e-3


def test_bf16_rounding_helper_matches_oracle():
    x = np.random.default_rng(0).standard_normal(100_000).astype(np.float32) * 1e3
    assert np.array_equal(W.bf16_round_np(x), O.bf16_round(x))


def test_zipf_bias_skews_load():
    wl = W.WORKLOADS["skewed_bf16"].scaled(4096)
    inp = W.make_inputs(wl, seed=0, with_weights=False)
    assert inp.bias.max() == pytest.approx(3.0) and inp.bias.min() > 0
    idx = O.topk_desc(inp.logits, wl.top_k)
    counts = np.bincount(idx.reshape(-1), minlength=wl.n_experts)
    assert counts.max() > 4 * counts.mean()
    plan = O.dispatch_plan(idx, wl.n_experts, wl.capacity)
    assert 0.05 < 1 - plan["keep"].mean() < 0.5      # real drops


def test_moe_constructor_contract():
    m = MoE(64, 32, 8, 2, 1, 0.01, 2.5, "bfloat16", rngs=0, device="cpu")
    shapes = {k: tuple(p.value.shape) for k, p in m.named_params().items()}
    assert shapes == {"router": (64, 8), "bias": (8,), "expert_w_gate": (8, 64, 32),
                      "expert_w_up": (8, 64, 32), "expert_w_down": (8, 32, 64),
                      "shared_w_gate": (64, 32), "shared_w_up": (64, 32),
                      "shared_w_down": (32, 64)}
    assert all(isinstance(p, Param) for p in m.named_params().values())
    assert m.bias.value.abs().sum() == 0
    assert abs(float(m.router.value.std()) - 0.01) < 3e-3
    m2 = MoE(64, 32, 8, 2, 3, 0.01, 2.5, torch.bfloat16, rngs=0, device="cpu", d_ff_shared=16)
    assert tuple(m2.shared_w_gate.value.shape) == (3, 64, 16)
    assert tuple(m2.shared_w_down.value.shape) == (3, 16, 64)


def test_moe_rejects_what_is_not_built():
    with pytest.raises(NotImplementedError):
        MoE(64, 32, 8, 2, 1, 0.01, 2.5, "bfloat16", rngs=0, device="cpu",
            mesh=type("M", (), {"devices": np.zeros(8)})())
    with pytest.raises(TypeError):
        MoE(64, 32, 8, 2, 1, 0.01, 2.5, "float16", rngs=0, device="cpu")
    m = MoE(64, 32, 8, 2, 1, 0.01, 2.5, "float32", rngs=0, device="cpu")
    with pytest.raises(ValueError, match="GPU"):   # float32 compute is built; CPU tensors are not
        m(torch.zeros(1, 4, 64))
    m.router.value.requires_grad_(True)
    with pytest.raises(ValueError, match="GPU"):   # so is its backward, on the GPU only
        m(torch.zeros(1, 4, 64))
    m = MoE(64, 32, 8, 2, 1, 0.01, 2.5, "bfloat16", rngs=0, device="cpu")
    with pytest.raises(ValueError, match="GPU"):   # no CPU path: kernels need device tensors
        m(torch.zeros(1, 4, 64, dtype=torch.bfloat16))


def test_moe_state_round_trip(tmp_path):
    """Reference-named parameter tree in and out: a safetensors file, nnx
    {"value": array} nodes, shape and name checks."""
    a = MoE(64, 32, 8, 2, 1, 0.01, 2.5, "bfloat16", rngs=0, device="cpu")
    b = MoE(64, 32, 8, 2, 1, 0.01, 2.5, "bfloat16", rngs=1, device="cpu")
    assert not np.array_equal(a.state()["router"], b.state()["router"])
    a.save_safetensors(tmp_path / "moe.safetensors")
    b.load_safetensors(tmp_path / "moe.safetensors")
    for k, v in a.state().items():
        assert np.array_equal(v, b.state()[k]), k
    c = MoE(64, 32, 8, 2, 1, 0.01, 2.5, "bfloat16", rngs=2, device="cpu")
    c.load_state({k: {"value": v} for k, v in a.state().items()})
    assert all(np.array_equal(v, c.state()[k]) for k, v in a.state().items())
    bad = a.state()
    bad["expert_w_up"] = bad["expert_w_up"][:, :, :16]
    with pytest.raises(ValueError, match="expert_w_up"):
        c.load_state(bad)
    missing = a.state()
    del missing["bias"]
    with pytest.raises(KeyError, match="bias"):
        c.load_state(missing)


def test_pack_cache_rebuilds_on_identity_or_version():
    """The packed-operand cache rebuilds for a different tensor object (even
    with equal contents), after an in-place update and after new storage is
    assigned under the same object (``t.data = other``, which keeps identity
    and version counter), and not otherwise."""
    import torch
    from hanuman_amd.moe import _PackCache
    builds = []
    c = _PackCache()
    a = torch.ones(4)
    b = torch.zeros(4)
    c.get((a, b), lambda: builds.append(1) or len(builds))
    c.get((a, b), lambda: builds.append(1) or len(builds))
    assert len(builds) == 1
    a.add_(1.0)
    c.get((a, b), lambda: builds.append(1) or len(builds))
    assert len(builds) == 2
    a2 = a.clone()
    c.get((a2, b), lambda: builds.append(1) or len(builds))
    assert len(builds) == 3
    c.get((a2, b), lambda: builds.append(1) or len(builds))
    assert len(builds) == 3
    v = a2._version
    a2.data = torch.full((6,), 5.0)          # new storage and shape, same object
    assert a2._version == v
    assert c.get((a2, b), lambda: builds.append(1) or len(builds)) == 4
    a2.data = torch.full((6,), 7.0)          # same shape, new storage
    assert c.get((a2, b), lambda: builds.append(1) or len(builds)) == 5
    assert c.get((a2, b), lambda: builds.append(1) or len(builds)) == 5


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; asking for more exits with a message instead
    of reporting a figure for a configuration it did not run."""
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], cwd=root,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)
    assert r.stdout.strip() == ""   # no JSON line


def test_bench_algorithmic_work_closed_forms():
    """The roofline denominators bench.py reports, from the closed forms:
    grouped GEMM 6 R D F FLOP (gate 2 R D F, up 2 R D F, down 2 R F D); the
    dispatch reads every token row once, writes every kept row and reads the
    slot map; the combine reads every kept row, writes every token row and
    reads the slot map and gates; the router's float64 dot products 2 T D N."""
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    import bench
    from hanuman_amd import workloads as W

    wl = W.WORKLOADS["full_bf16"]   # 16384 tokens, D 2048, 64 experts, top-8, F 1024
    T, D, N, K, F = 16384, 2048, 64, 8, 1024
    kept = T * K
    w = bench.algorithmic(wl, kept)
    assert w["gate_up"][1] + w["down"][1] == 6 * kept * D * F == w["ffn"][1]
    assert abs(w["ffn"][1] / 1e12 - 1.649) < 1e-3
    assert w["permute"][1] == T * D * 2 + kept * D * 2 + kept * 4
    assert w["combine"][1] == kept * D * 2 + T * D * 4 + kept * 8   # float32 output
    assert w["router"] == ("fp64", 2 * T * D * N, bench.FP64_PEAK_TFLOPS)
    assert w["gate_up"][2] == bench.BF16_PEAK_TFLOPS == 2500.0
    # fewer kept rows (capacity drops) lower the GEMM and row traffic only
    w2 = bench.algorithmic(wl, kept - 1000)
    assert w["ffn"][1] - w2["ffn"][1] == 6 * 1000 * D * F
    assert w["combine"][1] - w2["combine"][1] == 1000 * D * 2

    wl = W.WORKLOADS["fp8_experts"]  # 8192 tokens, D 4096, 32 experts, top-4, F 2048, e4m3
    T, D, N, K, F = 8192, 4096, 32, 4, 2048
    kept = T * K
    w = bench.algorithmic(wl, kept)
    assert w["ffn"][1] == 6 * kept * D * F and w["ffn"][2] == bench.FP8_PEAK_TFLOPS == 5000.0
    # codes and one float32 scale per dispatched row
    assert w["permute"][1] == T * D * 2 + kept * (D + 4) + kept * 4
    assert w["quant_x"][1] == T * D * 2 + T * D + T * 4
    assert w["combine"][1] == kept * D * 2 + T * D * 2 + kept * 8   # bf16 output

    wl = W.WORKLOADS["dispatch_identity"]  # logits given: the router is a read of them
    T, N, K = 32768, 64, 8
    w = bench.algorithmic(wl, T * K)
    assert w["router"] == ("hbm", T * N * 4 + T * K * 8, bench.HBM_PEAK_GBS)
    assert "gate_up" not in w
