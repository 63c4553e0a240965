"""Per-kernel parity of the HIP path against the oracle (needs an MI355X).

Integer outputs (top-k indices, counts, offsets, permutation, drop mask) and
every float32 value the contract fixes bit for bit (router logits, gates,
combine sums) are compared exactly; the grouped GEMM against float64 on the
same bf16 operands with a stated tolerance.
"""
import numpy as np
import pytest
import torch

import oracle as O
from hanuman_amd import _lib
from hanuman_amd import kernels as K

pytestmark = pytest.mark.gpu



def swiglu_ref(g, u):
    """h from float64 products at the kernels' rounding points: g and u
    rounded to bf16 first (the ragged_dot outputs, moe.py:70-71), then
    silu(g) * u (moe.py:72)."""
    g = O.bf16_round(np.asarray(g, np.float32)).astype(np.float64)
    u = O.bf16_round(np.asarray(u, np.float32)).astype(np.float64)
    return g / (1 + np.exp(-g)) * u

def dev_f32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def dev_bf16(a, dev):
    return dev_f32(a, dev).to(torch.bfloat16)


def host(t):
    if t.dtype == torch.bfloat16:
        return t.float().cpu().numpy()
    return t.cpu().numpy()


def assert_bits_equal(got, ref, what):
    got = np.ascontiguousarray(got)
    ref = np.ascontiguousarray(ref)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    if got.dtype == np.float32:
        bad = got.view(np.uint32) != ref.view(np.uint32)
    else:
        bad = got != ref
    n = int(bad.sum())
    assert n == 0, f"{what}: {n} of {bad.size} elements differ; first at {np.argwhere(bad)[:5].tolist()}"


# ------------------------------------------------------------------- router --

ROUTER_CASES = [
    # T, D, N, K, x_dtype, w_dtype, mode, rsf, bias
    (2048, 256, 8, 2, "f32", "f32", "softmax", 1.0, False),
    (1024, 2048, 64, 8, "bf16", "f32", "softmax", 1.0, False),
    (777, 2048, 128, 8, "bf16", "f32", "softmax", 1.0, False),
    (300, 512, 200, 6, "bf16", "f32", "sigmoid", 2.5, True),
    (256, 4096, 32, 4, "bf16", "bf16", "softmax", 1.0, False),
    (129, 1536, 80, 8, "bf16", "f32", "sigmoid", 2.5, True),
    # enough tokens for one 64-token workgroup per CU (8-wave router), last one partial
    (16450, 512, 66, 6, "bf16", "f32", "sigmoid", 2.5, True),
    (16400, 768, 64, 8, "bf16", "bf16", "softmax", 1.0, False),
    # 128-d LDS chunks with a partial last chunk: 8-wave, 4-wave up to 32
    # experts, and float32 x
    (16384, 1000, 64, 8, "bf16", "f32", "softmax", 1.0, False),
    (600, 520, 32, 4, "bf16", "f32", "sigmoid", 2.5, True),
    (700, 200, 20, 3, "f32", "f32", "softmax", 1.0, False),
    # 62 experts: W rows not a multiple of 16 bytes (scalar W staging, 64-d chunks)
    (16400, 648, 62, 8, "bf16", "f32", "sigmoid", 2.5, True),
]


@pytest.mark.parametrize("case", ROUTER_CASES, ids=lambda c: f"T{c[0]}_D{c[1]}_N{c[2]}_K{c[3]}_{c[6]}")
def test_router_bit_exact(gpu, case):
    T, D, N, Kk, xd, wd, mode, rsf, with_bias = case
    print(f"router case {case}", flush=True)
    rng = np.random.default_rng(T + D + N)
    x = rng.standard_normal((T, D)).astype(np.float32)
    if xd == "bf16":
        x = O.bf16_round(x)
    w = (0.02 * rng.standard_normal((D, N))).astype(np.float32)
    if wd == "bf16":
        w = O.bf16_round(w)
    bias = (0.05 * rng.standard_normal(N)).astype(np.float32) if with_bias else None
    logits_ref = O.router_logits(x, w)
    if mode == "softmax":
        idx_ref, g_ref = O.route_softmax(logits_ref, Kk)
    else:
        idx_ref, g_ref, _ = O.route_sigmoid(logits_ref, bias, Kk, rsf)
    xt = dev_bf16(x, gpu) if xd == "bf16" else dev_f32(x, gpu)
    wt = dev_bf16(w, gpu) if wd == "bf16" else dev_f32(w, gpu)
    bt = dev_f32(bias, gpu) if bias is not None else None
    m = _lib.ROUTE_SOFTMAX if mode == "softmax" else _lib.ROUTE_SIGMOID_BIAS
    logits, idx, g = K.router(xt, wt, bt, Kk, m, rsf)
    torch.cuda.synchronize()
    assert_bits_equal(host(logits), logits_ref, "logits")
    assert_bits_equal(host(idx), idx_ref, "top_idx")
    assert_bits_equal(host(g), g_ref, "gates")


# The router with x's per-token e4m3 quantisation in the same launch: every
# bf16-token router case above, plus rows past 4096 values (the two-pass
# quantisation), a single token and the 8-wave router configuration.
ROUTER_QUANT_CASES = [c for c in ROUTER_CASES if c[4] == "bf16"] + [
    (2048, 4096, 32, 4, "bf16", "bf16", "softmax", 1.0, False),
    (101, 4104, 16, 2, "bf16", "f32", "sigmoid", 2.5, True),
    (1, 512, 8, 2, "bf16", "bf16", "softmax", 1.0, False),
]


@pytest.mark.parametrize("case", ROUTER_QUANT_CASES,
                         ids=lambda c: f"T{c[0]}_D{c[1]}_N{c[2]}_K{c[3]}_{c[6]}")
def test_router_quant_fp8_bit_exact(gpu, case):
    """hmoe_router_quant_fp8 against the oracle's router and per-row e4m3
    rule, bit for bit (rows of zeros and a wide dynamic range included)."""
    T, D, N, Kk, _, wd, mode, rsf, with_bias = case
    print(f"router+quant case {case}", flush=True)
    rng = np.random.default_rng(T + D + N + 7)
    x = rng.standard_normal((T, D)) * np.exp(rng.uniform(-12, 6, (T, 1)))
    x = O.bf16_round(x.astype(np.float32))
    x[T // 3] = 0.0
    w = (0.02 * rng.standard_normal((D, N))).astype(np.float32)
    if wd == "bf16":
        w = O.bf16_round(w)
    bias = (0.05 * rng.standard_normal(N)).astype(np.float32) if with_bias else None
    logits_ref = O.router_logits(x, w)
    if mode == "softmax":
        idx_ref, g_ref = O.route_softmax(logits_ref, Kk)
    else:
        idx_ref, g_ref, _ = O.route_sigmoid(logits_ref, bias, Kk, rsf)
    q_ref, s_ref = O.quantize_rows_e4m3(x)
    wt = dev_bf16(w, gpu) if wd == "bf16" else dev_f32(w, gpu)
    bt = dev_f32(bias, gpu) if bias is not None else None
    m = _lib.ROUTE_SOFTMAX if mode == "softmax" else _lib.ROUTE_SIGMOID_BIAS
    logits, idx, g, x_q, x_s = K.router_quant_fp8(dev_bf16(x, gpu), wt, bt, Kk, m, rsf)
    torch.cuda.synchronize()
    assert_bits_equal(host(logits), logits_ref, "logits")
    assert_bits_equal(host(idx), idx_ref, "top_idx")
    assert_bits_equal(host(g), g_ref, "gates")
    assert_bits_equal(x_q.cpu().numpy(), q_ref, "x codes")
    assert_bits_equal(x_s.cpu().numpy(), s_ref, "x scales")


def test_router_quant_fp8_equals_separate_launches_at_fp8_workload(gpu):
    """At the fp8 experts workload's shape (8192 tokens, d_model 4096, 32
    experts, top-4, bf16 router weight) the one launch gives the bits of
    hmoe_router followed by hmoe_quantize_rows_fp8."""
    print("router+quant at 8192 x 4096, 32 experts", flush=True)
    g = torch.Generator(device="cpu").manual_seed(5)
    x = torch.randn(8192, 4096, generator=g).to(torch.bfloat16).to(gpu)
    w = (torch.randn(4096, 32, generator=g) * 4096 ** -0.5).to(torch.bfloat16).to(gpu)
    a = K.router(x, w, None, 4, _lib.ROUTE_SOFTMAX)
    q, s = K.quantize_rows_fp8(x)
    b = K.router_quant_fp8(x, w, None, 4, _lib.ROUTE_SOFTMAX)
    torch.cuda.synchronize()
    for name, u, v in zip(("logits", "top_idx", "gates", "x codes", "x scales"), (*a, q, s), b):
        assert torch.equal(u, v), name


def test_router_quant_fp8_refusals(gpu):
    x = torch.zeros(8, 64, dtype=torch.float32, device=gpu)
    w = torch.zeros(64, 8, dtype=torch.float32, device=gpu)
    with pytest.raises(TypeError):
        K.router_quant_fp8(x, w, None, 2)
    lib = _lib.lib()
    p = x.data_ptr()
    rc = lib.hmoe_router_quant_fp8(p, _lib.F32, p, _lib.F32, None, 8, 64, 8, 2, 0, 1.0, p, p, p,
                                   p, p, None)
    assert rc == _lib.ERR_INVALID and "BF16" in lib.hmoe_last_error().decode()
    rc = lib.hmoe_router_quant_fp8(p, _lib.BF16, p, _lib.F32, None, 8, 64, 8, 2, 0, 1.0, p, p, p,
                                   None, p, None)
    assert rc == _lib.ERR_INVALID and "null" in lib.hmoe_last_error().decode()


@pytest.mark.parametrize("T,N,Kk,mode", [(16400, 64, 8, "softmax"), (700, 64, 8, "sigmoid"),
                                         (333, 50, 6, "softmax"), (16390, 40, 4, "sigmoid")])
def test_router_ties_through_logits(gpu, T, N, Kk, mode):
    """Experts with identical router columns get identical logits for every
    token; the lower expert index must come first (within one lane, across
    lanes and across lane groups), and all-zero columns tie at exactly 0."""
    print(f"router ties T={T} N={N} K={Kk} {mode}", flush=True)
    rng = np.random.default_rng(T + 7 * N)
    D = 512
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    w = (0.02 * rng.standard_normal((D, N))).astype(np.float32)
    for a, b in [(5, 9), (0, N - 1), (32 % N, 33 % N), (7, 8), (3, 20)]:
        w[:, b] = w[:, a]
    w[:, [1, 2, N - 2]] = 0.0
    bias = None
    if mode == "sigmoid":
        bias = np.zeros(N, np.float32)
        bias[[5, 9, 0, N - 1]] = 0.25
    logits_ref = O.router_logits(x, w)
    if mode == "softmax":
        idx_ref, g_ref = O.route_softmax(logits_ref, Kk)
    else:
        idx_ref, g_ref, _ = O.route_sigmoid(logits_ref, bias, Kk, 2.5)
    m = _lib.ROUTE_SOFTMAX if mode == "softmax" else _lib.ROUTE_SIGMOID_BIAS
    logits, idx, g = K.router(dev_bf16(x, gpu), dev_f32(w, gpu),
                              dev_f32(bias, gpu) if bias is not None else None, Kk, m, 2.5)
    torch.cuda.synchronize()
    assert_bits_equal(host(logits), logits_ref, "logits")
    assert_bits_equal(host(idx), idx_ref, "top_idx")
    assert_bits_equal(host(g), g_ref, "gates")


def test_router_from_logits_ties_and_signed_zero(gpu):
    rng = np.random.default_rng(21)
    T, N, Kk = 512, 64, 8
    logits = rng.integers(-3, 4, size=(T, N)).astype(np.float32)   # many exact ties
    logits[0] = 0.0
    logits[0, 10:20] = -0.0
    logits[1] = 1.0
    for mode in (_lib.ROUTE_SOFTMAX, _lib.ROUTE_SIGMOID_BIAS):
        bias = np.zeros(N, np.float32) if mode == _lib.ROUTE_SIGMOID_BIAS else None
        if mode == _lib.ROUTE_SOFTMAX:
            idx_ref, g_ref = O.route_softmax(logits, Kk)
        else:
            idx_ref, g_ref, _ = O.route_sigmoid(logits, bias, Kk, 2.5)
        idx, g = K.router_from_logits(dev_f32(logits, gpu),
                                      dev_f32(bias, gpu) if bias is not None else None, Kk, mode, 2.5)
        torch.cuda.synchronize()
        assert_bits_equal(host(idx), idx_ref, f"top_idx mode {mode}")
        assert_bits_equal(host(g), g_ref, f"gates mode {mode}")
    assert host(idx)[1].tolist() == list(range(Kk))      # all equal -> lowest indices


@pytest.mark.parametrize("N", [20, 60, 100])
def test_router_from_logits_nan_and_infinities(gpu, N):
    """NaNs, infinities and signed zeros order by IEEE totalOrder; the
    negative NaN with every payload bit set has the lowest key of all, which
    must still rank above the padding past n_experts (top-k = N selects
    every expert)."""
    rng = np.random.default_rng(N + 1)
    T, Kk = 16, min(N, 32)
    bits = rng.standard_normal((T, N)).astype(np.float32).view(np.uint32)
    bits[0] = 0xFFFFFFFF                       # all the lowest key: index order
    bits[1, [3, 17, N - 1]] = 0xFFFFFFFF       # negative NaN, full payload
    bits[1, 5] = 0xFF800000                    # -inf
    bits[1, 6] = 0x7F800000                    # +inf
    bits[1, 7] = 0x7FC00000                    # +NaN: above +inf
    bits[1, 8] = 0x80000000                    # -0.0 below +0.0
    bits[1, 9] = 0x00000000
    bits[2:, ::7] = 0xFFFFFFFF
    logits = bits.view(np.float32)
    # softmax selects on the logits' own bits; the sigmoid keys are computed,
    # and a NaN's payload after arithmetic is not fixed, so that mode gets -inf
    # where the logits hold NaNs
    finite_or_inf = np.where(np.isnan(logits), np.float32(-np.inf), logits)
    for mode, lg in ((_lib.ROUTE_SOFTMAX, logits), (_lib.ROUTE_SIGMOID_BIAS, finite_or_inf)):
        bias = np.zeros(N, np.float32) if mode == _lib.ROUTE_SIGMOID_BIAS else None
        if mode == _lib.ROUTE_SOFTMAX:
            idx_ref, g_ref = O.route_softmax(lg, Kk)
        else:
            idx_ref, g_ref, _ = O.route_sigmoid(lg, bias, Kk, 2.5)
        idx, g = K.router_from_logits(dev_f32(lg, gpu),
                                      dev_f32(bias, gpu) if bias is not None else None, Kk, mode, 2.5)
        torch.cuda.synchronize()
        assert_bits_equal(host(idx), idx_ref, f"top_idx mode {mode}")
        g, g_ref = host(g), np.asarray(g_ref, np.float32)
        assert np.array_equal(np.isnan(g), np.isnan(g_ref)), f"gate NaNs mode {mode}"
        ok = ~np.isnan(g_ref)
        assert_bits_equal(g[ok], g_ref[ok], f"gates mode {mode}")
        assert host(idx)[0].tolist() == list(range(Kk)), f"row of equal keys, mode {mode}"


@pytest.mark.parametrize("N", [100, 200])
def test_router_from_logits_ties_across_lanes(gpu, N):
    """Experts past 64 share lanes with lower ones (lane = expert % 64): equal
    keys on two experts of one lane, or on a low expert of a high lane and a
    high expert of a low lane, must still go to the lower expert index."""
    rng = np.random.default_rng(N)
    T, Kk = 700, 8
    logits = rng.integers(-2, 3, size=(T, N)).astype(np.float32)   # many exact ties
    logits[0] = 0.0                        # all tied: the lowest K indices
    logits[1] = 0.0
    logits[1, [5, 69, 133 % N]] = 3.0      # one lane, several j
    logits[2] = 0.0
    logits[2, [70, 6]] = 2.0               # expert 6 (lane 6) before 70 (lane 6, j=1)
    logits[3] = -1.0
    logits[3, [N - 1, 63, 64]] = 1.0       # the last expert, lane 63 and lane 0 of j=1
    for mode in (_lib.ROUTE_SOFTMAX, _lib.ROUTE_SIGMOID_BIAS):
        bias = np.zeros(N, np.float32) if mode == _lib.ROUTE_SIGMOID_BIAS else None
        if mode == _lib.ROUTE_SOFTMAX:
            idx_ref, g_ref = O.route_softmax(logits, Kk)
        else:
            idx_ref, g_ref, _ = O.route_sigmoid(logits, bias, Kk, 2.5)
        idx, g = K.router_from_logits(dev_f32(logits, gpu),
                                      dev_f32(bias, gpu) if bias is not None else None, Kk, mode, 2.5)
        torch.cuda.synchronize()
        assert_bits_equal(host(idx), idx_ref, f"top_idx mode {mode}")
        assert_bits_equal(host(g), g_ref, f"gates mode {mode}")
    got = host(idx)
    assert got[0].tolist() == list(range(Kk))
    assert got[2][:2].tolist() == [6, 70]
    assert got[3][:3].tolist() == [63, 64, N - 1]


@pytest.mark.parametrize("T,N,Kk,mode", [(1003, 200, 6, "sigmoid"), (77, 100, 4, "softmax"),
                                         (18, 16, 2, "softmax")])
def test_router_from_logits_ragged(gpu, T, N, Kk, mode):
    """Token counts that leave the last wave's group of tokens partial."""
    rng = np.random.default_rng(T + N)
    logits = rng.standard_normal((T, N), dtype=np.float32)
    if mode == "softmax":
        idx_ref, g_ref = O.route_softmax(logits, Kk)
        bias = None
    else:
        bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
        idx_ref, g_ref, _ = O.route_sigmoid(logits, bias, Kk, 2.5)
    m = _lib.ROUTE_SOFTMAX if mode == "softmax" else _lib.ROUTE_SIGMOID_BIAS
    idx, g = K.router_from_logits(dev_f32(logits, gpu), dev_f32(bias, gpu) if bias is not None else None,
                                  Kk, m, 2.5)
    torch.cuda.synchronize()
    assert_bits_equal(host(idx), idx_ref, "top_idx")
    assert_bits_equal(host(g), g_ref, "gates")


def test_router_from_logits_dispatch_workload_full_size(gpu):
    rng = np.random.default_rng(0)
    T, N, Kk = 32768, 64, 8
    logits = rng.standard_normal((T, N), dtype=np.float32)
    idx_ref, g_ref = O.route_softmax(logits, Kk)
    idx, g = K.router_from_logits(dev_f32(logits, gpu), None, Kk, _lib.ROUTE_SOFTMAX)
    torch.cuda.synchronize()
    assert_bits_equal(host(idx), idx_ref, "top_idx")
    assert_bits_equal(host(g), g_ref, "gates")


# -------------------------------------------------------------------- plan --

def _skewed_top_idx(rng, T, K, N):
    logits = rng.standard_normal((T, N), dtype=np.float32)
    ranks = rng.permutation(N) + 1
    logits += (3.0 * ranks.astype(np.float64) ** -1.1).astype(np.float32)
    return O.topk_desc(logits, K)


PLAN_CASES = [
    # name, T, K, N, capacity factor (None = dropless)
    ("dispatch_full", 32768, 8, 64, 1.0),
    ("skewed_full", 65536, 8, 128, 1.25),
    ("dropless", 4096, 8, 64, None),
    ("tiny", 3, 2, 5, None),
    ("cap1", 1000, 4, 16, 0.001),
    ("one_expert", 700, 1, 1, 0.5),
    ("ragged_blocks", 4097, 3, 1000, 1.0),
    # 128 blocks x 1024 experts: past the fused rank's histogram limit, so
    # the three-pass plan (histogram, column scan, rank)
    ("wide_histogram", 16384, 8, 1024, 1.25),
]


@pytest.mark.parametrize("case", PLAN_CASES, ids=lambda c: c[0])
def test_dispatch_plan_bit_exact(gpu, case):
    name, T, Kk, N, cf = case
    print(f"plan case {case}", flush=True)
    rng = np.random.default_rng(T * 7 + N)
    if name == "skewed_full":
        top = _skewed_top_idx(rng, T, Kk, N)
    else:
        top = np.stack([rng.permutation(N)[:Kk] if N >= Kk else rng.integers(0, N, Kk)
                        for _ in range(T)]).astype(np.int32) if T <= 5000 else \
            O.topk_desc(rng.standard_normal((T, N), dtype=np.float32), Kk)
    C = O.capacity_of(T, Kk, N, cf)
    ref = O.dispatch_plan(top, N, C)
    cap = K.capacity(T, Kk, N, cf)
    assert cap == C
    plan = K.dispatch_plan(torch.from_numpy(top).to(gpu), N, cap)
    torch.cuda.synchronize()
    assert plan.rows_cap == O.rows_cap_of(T, Kk, N, C)
    for k in ("counts", "offsets", "slot_pos", "perm_src", "keep"):
        assert_bits_equal(host(getattr(plan, k)), ref[k], k)


def test_dispatch_plan_is_deterministic(gpu):
    rng = np.random.default_rng(5)
    top = torch.from_numpy(O.topk_desc(rng.standard_normal((16384, 64), dtype=np.float32), 8)).to(gpu)
    a = K.dispatch_plan(top, 64, 2560)
    b = K.dispatch_plan(top, 64, 2560)
    torch.cuda.synchronize()
    for k in ("counts", "offsets", "slot_pos", "perm_src", "keep"):
        assert torch.equal(getattr(a, k), getattr(b, k)), k


# ------------------------------------------------------------- permutation --

@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_permute_rows_bit_exact(gpu, xdt):
    rng = np.random.default_rng(30)
    T, D, N, Kk = 3000, 2048, 64, 8
    x = rng.standard_normal((T, D)).astype(np.float32)
    if xdt == "bf16":
        x = O.bf16_round(x)
    top = O.topk_desc(rng.standard_normal((T, N), dtype=np.float32), Kk)
    C = O.capacity_of(T, Kk, N, 1.0)
    ref = O.dispatch_plan(top, N, C)
    xs_ref = O.permute_rows(O.bf16_round(x), ref["perm_src"], Kk)
    xt = dev_bf16(x, gpu) if xdt == "bf16" else dev_f32(x, gpu)
    plan = K.dispatch_plan(torch.from_numpy(top).to(gpu), N, C)
    xs = K.permute_rows(xt, plan, torch.bfloat16)
    torch.cuda.synchronize()
    total = int(ref["offsets"][-1])
    assert_bits_equal(host(xs)[:total], xs_ref[:total], "xs")


# ----------------------------------------------------------------- combine --

@pytest.mark.parametrize("residual,ys_dtype", [(None, "bf16"), ("bf16", "bf16"), ("f32", "bf16"),
                                              (None, "f32")])
@pytest.mark.parametrize("out_dtype", ["f32", "bf16"])
def test_combine_bit_exact(gpu, residual, out_dtype, ys_dtype):
    rng = np.random.default_rng(40)
    T, D, N, Kk = 2000, 1024, 32, 4
    top = O.topk_desc(rng.standard_normal((T, N), dtype=np.float32), Kk)
    C = O.capacity_of(T, Kk, N, 1.0)
    ref = O.dispatch_plan(top, N, C)
    rows = int(ref["offsets"][-1])
    ys = rng.standard_normal((O.rows_cap_of(T, Kk, N, C), D)).astype(np.float32)
    if ys_dtype == "bf16":
        ys = O.bf16_round(ys)
    g = rng.random((T, Kk)).astype(np.float32)
    res = None
    if residual == "bf16":
        res = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    elif residual == "f32":
        res = rng.standard_normal((T, D)).astype(np.float32)
    out_ref = O.combine(ys[:max(rows, 1)], ref["slot_pos"], g, T, Kk, residual=res, ys_dtype=ys_dtype)
    plan = K.dispatch_plan(torch.from_numpy(top).to(gpu), N, C)
    rt = None if res is None else (dev_bf16(res, gpu) if residual == "bf16" else dev_f32(res, gpu))
    out = K.combine(dev_bf16(ys, gpu) if ys_dtype == "bf16" else dev_f32(ys, gpu), plan, dev_f32(g, gpu), rt,
                    torch.float32 if out_dtype == "f32" else torch.bfloat16)
    torch.cuda.synchronize()
    if out_dtype == "bf16":
        out_ref = O.bf16_round(out_ref)
    assert_bits_equal(host(out), out_ref, "combine")


# ------------------------------------------------------------- pack + GEMM --

def test_pack_layouts(gpu):
    rng = np.random.default_rng(50)
    N, D, F = 3, 256, 384
    wg, wu = rng.standard_normal((2, N, D, F)).astype(np.float32)
    wd = rng.standard_normal((N, F, D)).astype(np.float32)
    pgu = host(K.pack_gate_up(dev_f32(wg, gpu), dev_f32(wu, gpu)))
    pd = host(K.pack_down(dev_f32(wd, gpu)))
    torch.cuda.synchronize()
    p = np.arange(2 * F)
    col = (p // 64) * 32 + p % 32
    is_up = (p % 64) >= 32
    exp_gu = np.where(is_up[None, :, None], np.transpose(wu, (0, 2, 1))[:, col],
                      np.transpose(wg, (0, 2, 1))[:, col])
    assert_bits_equal(pgu, O.bf16_round(exp_gu), "packed gate/up")
    assert_bits_equal(pd, O.bf16_round(np.transpose(wd, (0, 2, 1))), "packed down")


GEMM_CASES = [
    # name, D, F, segment sizes
    ("ragged", 256, 128, [0, 1, 255, 256, 257, 600, 0, 31]),
    ("wide", 2048, 1024, [300, 2048, 513]),
    ("skinny_tail", 512, 768, [1, 1, 1, 700]),
]


@pytest.mark.parametrize("case", GEMM_CASES, ids=lambda c: c[0])
def test_grouped_gemm(gpu, case):
    name, D, F, sizes = case
    print(f"gemm case {case}", flush=True)
    rng = np.random.default_rng(60 + D)
    N = len(sizes)
    offsets = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    R = int(offsets[-1])
    xs = O.bf16_round(rng.standard_normal((R, D)).astype(np.float32))
    wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
    wd = (0.02 * rng.standard_normal((N, F, D))).astype(np.float32)
    off_t = torch.from_numpy(offsets).to(gpu)
    h = K.grouped_gate_up(dev_bf16(xs, gpu), off_t, K.pack_gate_up(dev_f32(wg, gpu), dev_f32(wu, gpu)))
    h_host = host(h)
    ys = K.grouped_down(h, off_t, K.pack_down(dev_f32(wd, gpu)))
    ys_host = host(ys)
    torch.cuda.synchronize()
    wgb, wub, wdb = (O.bf16_round(w).astype(np.float64) for w in (wg, wu, wd))
    for e in range(N):
        a, b = offsets[e], offsets[e + 1]
        if b == a:
            continue
        x64 = xs[a:b].astype(np.float64)
        g = x64 @ wgb[e]
        u = x64 @ wub[e]
        h_ref = swiglu_ref(g, u)
        err_h = np.abs(h_host[a:b] - h_ref)
        assert np.all(err_h <= 8e-3 * np.abs(h_ref) + 1e-3 * np.abs(h_ref).max()), \
            f"h expert {e}: max err {err_h.max()}"
        y_ref = h_host[a:b].astype(np.float64) @ wdb[e]
        err_y = np.abs(ys_host[a:b] - y_ref)
        assert np.all(err_y <= 8e-3 * np.abs(y_ref) + 1e-3 * np.abs(y_ref).max()), \
            f"ys expert {e}: max err {err_y.max()}"


ODD_K_CASES = [
    # name, D, F, segment sizes: gate/up reduces over D, down over F; an odd
    # number of 64-element K steps takes the zero-padded extra step per tile
    ("gate_up_k192", 192, 128, [0, 5, 300, 256, 1]),
    ("down_k192", 256, 192, [7, 0, 513, 64]),
    ("down_k64", 256, 64, [200, 1, 300]),
]


@pytest.mark.parametrize("case", ODD_K_CASES, ids=lambda c: c[0])
def test_grouped_gemm_odd_k_steps(gpu, case):
    name, D, F, sizes = case
    print(f"gemm odd-k case {case}", flush=True)
    rng = np.random.default_rng(90 + D + F)
    N = len(sizes)
    offsets = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    R = int(offsets[-1])
    off_t = torch.from_numpy(offsets).to(gpu)
    if name.startswith("gate_up"):
        xs = O.bf16_round(rng.standard_normal((R, D)).astype(np.float32))
        wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
        out = host(K.grouped_gate_up(dev_bf16(xs, gpu), off_t, K.pack_gate_up(dev_f32(wg, gpu), dev_f32(wu, gpu))))
        wgb, wub = (O.bf16_round(w).astype(np.float64) for w in (wg, wu))
        for e in range(N):
            a, b = offsets[e], offsets[e + 1]
            if b == a:
                continue
            x64 = xs[a:b].astype(np.float64)
            g, u = x64 @ wgb[e], x64 @ wub[e]
            ref = swiglu_ref(g, u)
            err = np.abs(out[a:b] - ref)
            assert np.all(err <= 8e-3 * np.abs(ref) + 1e-3 * np.abs(ref).max()), f"h expert {e}: {err.max()}"
    else:
        h = O.bf16_round(rng.standard_normal((R, F)).astype(np.float32))
        wd = (0.02 * rng.standard_normal((N, F, D))).astype(np.float32)
        out = host(K.grouped_down(dev_bf16(h, gpu), off_t, K.pack_down(dev_f32(wd, gpu))))
        wdb = O.bf16_round(wd).astype(np.float64)
        for e in range(N):
            a, b = offsets[e], offsets[e + 1]
            if b == a:
                continue
            ref = h[a:b].astype(np.float64) @ wdb[e]
            err = np.abs(out[a:b] - ref)
            assert np.all(err <= 8e-3 * np.abs(ref) + 1e-3 * np.abs(ref).max()), f"ys expert {e}: {err.max()}"


GATHER_CASES = [
    # T, D, N, K, F, capacity (rows per expert; small values drop slots)
    (700, 256, 8, 2, 128, 10**6),
    (1000, 192, 6, 4, 256, 300),
    (333, 512, 16, 8, 128, 90),
]


@pytest.mark.parametrize("case", GATHER_CASES, ids=lambda c: f"T{c[0]}_D{c[1]}_N{c[2]}_K{c[3]}_cap{c[5]}")
def test_grouped_gate_up_gather_matches_unfused(gpu, case):
    """The gate/up GEMM that gathers its rows from x through perm_src gives the
    same h, bit for bit, as the permutation followed by the plain GEMM."""
    T, D, N, Kk, F, cap = case
    print(f"gather case {case}", flush=True)
    rng = np.random.default_rng(7 + T)
    x = dev_bf16(O.bf16_round(rng.standard_normal((T, D)).astype(np.float32)), gpu)
    top = np.stack([rng.choice(N, Kk, replace=False) for _ in range(T)]).astype(np.int32)
    plan = K.dispatch_plan(torch.from_numpy(top).to(gpu), N, cap)
    wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
    w = K.pack_gate_up(dev_f32(wg, gpu), dev_f32(wu, gpu))
    h_fused = K.grouped_gate_up_gather(x, plan, w)
    h_ref = K.grouped_gate_up(K.permute_rows(x, plan, torch.bfloat16), plan.offsets, w)
    total = int(plan.offsets[-1].item())
    assert total > 0
    assert torch.equal(h_fused[:total], h_ref[:total])


# --------------------------------------------------------------------- aux --

def test_router_aux(gpu):
    rng = np.random.default_rng(70)
    B, S, N, Kk = 3, 200, 40, 6
    logits = (2 * rng.standard_normal((B * S, N))).astype(np.float32)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
    idx, _, scores = O.route_sigmoid(logits, bias, Kk, 2.5)
    ref = O.aux_losses(logits, scores, idx, B, S, N)
    losses, counts = K.router_aux(dev_f32(logits, gpu), torch.from_numpy(idx).to(gpu), B, S)
    torch.cuda.synchronize()
    got = host(losses)
    assert np.allclose(got, [ref["router_z_loss"], ref["balance_loss"], ref["mean_entropy"]],
                       rtol=2e-5, atol=0)
    assert_bits_equal(host(counts), ref["expert_counts"], "expert_counts")


# ------------------------------------------------------------------- fp8 --

@pytest.mark.parametrize("D,xdt", [(4096, "bf16"), (256, "bf16"), (8, "f32"), (1032, "f32")])
def test_permute_rows_fp8_bit_exact(gpu, D, xdt):
    print(f"permute fp8 D={D} {xdt}", flush=True)
    rng = np.random.default_rng(90 + D)
    T, N, Kk = 700, 32, 4
    x = (rng.standard_normal((T, D)) * np.exp(rng.uniform(-8, 4, (T, 1)))).astype(np.float32)
    x[5] = 0.0
    x[6, : min(D, 4)] = [-0.0, 1e-30, -1e-30, 0.0][: min(D, 4)]
    if xdt == "bf16":
        x = O.bf16_round(x)
    top = O.topk_desc(rng.standard_normal((T, N), dtype=np.float32), Kk)
    C = O.capacity_of(T, Kk, N, 1.0)
    ref = O.dispatch_plan(top, N, C)
    xq, xsc = O.quantize_rows_e4m3(x)
    total = int(ref["offsets"][-1])
    src = ref["perm_src"][:total] // Kk
    xt = dev_bf16(x, gpu) if xdt == "bf16" else dev_f32(x, gpu)
    plan = K.dispatch_plan(torch.from_numpy(top).to(gpu), N, C)
    xs_q, xs_s = K.permute_rows_fp8(xt, plan)
    torch.cuda.synchronize()
    assert_bits_equal(xs_q.cpu().numpy()[:total], xq[src], "xs_q")
    assert_bits_equal(xs_s.cpu().numpy()[:total], xsc[src], "xs_scale")


def test_quantize_rows_fp8_bit_exact_and_skips_past_offsets(gpu):
    rng = np.random.default_rng(91)
    R, F = 300, 2048
    h = O.bf16_round((rng.standard_normal((R, F)) * np.exp(rng.uniform(-20, 6, (R, 1)))).astype(np.float32))
    h[7] = 0.0
    q_ref, s_ref = O.quantize_rows_e4m3(h)
    q, s = K.quantize_rows_fp8(dev_bf16(h, gpu))
    torch.cuda.synchronize()
    assert_bits_equal(q.cpu().numpy(), q_ref, "codes")
    assert_bits_equal(s.cpu().numpy(), s_ref, "scales")
    offsets = torch.tensor([0, 100, 250], dtype=torch.int32, device=gpu)
    q2, s2 = K.quantize_rows_fp8(dev_bf16(h, gpu), offsets)
    torch.cuda.synchronize()
    assert_bits_equal(q2.cpu().numpy()[:250], q_ref[:250], "codes below offsets[-1]")
    assert np.all(s2.cpu().numpy()[250:] == 1.0)   # rows past the kept total: scale 1, not read


def test_pack_fp8_layouts(gpu):
    rng = np.random.default_rng(92)
    N, D, F = 3, 256, 384
    wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
    wd = (0.02 * rng.standard_normal((N, F, D))).astype(np.float32)
    pgu, sgu = K.pack_fp8_gate_up(dev_f32(wg, gpu), dev_f32(wu, gpu))
    pd, sd = K.pack_fp8_down(dev_f32(wd, gpu))
    torch.cuda.synchronize()
    wq = O.quantize_expert_weights({"expert_w_gate": wg, "expert_w_up": wu, "expert_w_down": wd})
    p = np.arange(2 * F)
    col = (p // 64) * 32 + p % 32
    is_up = (p % 64) >= 32
    exp_codes = np.where(is_up[None, :, None], np.transpose(wq["wu_q"], (0, 2, 1))[:, col],
                         np.transpose(wq["wg_q"], (0, 2, 1))[:, col])
    exp_scales = np.where(is_up[None, :], wq["wu_s"][:, col], wq["wg_s"][:, col])
    assert_bits_equal(pgu.cpu().numpy(), exp_codes, "packed fp8 gate/up")
    assert_bits_equal(sgu.cpu().numpy(), exp_scales, "gate/up scales")
    assert_bits_equal(pd.cpu().numpy(), np.transpose(wq["wd_q"], (0, 2, 1)), "packed fp8 down")
    assert_bits_equal(sd.cpu().numpy(), wq["wd_s"], "down scales")


FP8_GEMM_CASES = [
    # name, D, F, segment sizes
    ("ragged", 256, 128, [0, 1, 255, 256, 257, 600, 0, 31]),
    ("wide", 4096, 2048, [300, 1024, 513]),
]


FP8_GATHER_CASES = [
    # T, D, N, K, F, capacity (rows per expert; small values drop slots)
    (700, 256, 8, 2, 128, 10**6),
    (1000, 384, 6, 4, 256, 300),
    (333, 512, 16, 8, 128, 90),
]


@pytest.mark.parametrize("case", FP8_GATHER_CASES,
                         ids=lambda c: f"T{c[0]}_D{c[1]}_N{c[2]}_K{c[3]}_cap{c[5]}")
def test_grouped_gate_up_fp8_gather_matches_permuted(gpu, case):
    """The fp8 gate/up GEMM that gathers its rows from the per-token codes of x
    gives the same h, bit for bit, as the fp8 permutation followed by the
    plain fp8 GEMM (the per-token codes are the dispatched codes)."""
    T, D, N, Kk, F, cap = case
    print(f"fp8 gather case {case}", flush=True)
    rng = np.random.default_rng(17 + T)
    x = dev_bf16(O.bf16_round(rng.standard_normal((T, D)).astype(np.float32)), gpu)
    top = np.stack([rng.choice(N, Kk, replace=False) for _ in range(T)]).astype(np.int32)
    plan = K.dispatch_plan(torch.from_numpy(top).to(gpu), N, cap)
    wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
    w, ws = K.pack_fp8_gate_up(dev_f32(wg, gpu), dev_f32(wu, gpu))
    x_q, x_s = K.quantize_rows_fp8(x)
    h_fused = K.grouped_gate_up_fp8_gather(x_q, x_s, plan, w, ws)
    xs_q, xs_s = K.permute_rows_fp8(x, plan)
    h_ref = K.grouped_gate_up_fp8(xs_q, xs_s, plan.offsets, w, ws)
    total = int(plan.offsets[-1].item())
    assert total > 0
    src = plan.perm_src[:total].long() // Kk
    assert torch.equal(x_q[src], xs_q[:total]) and torch.equal(x_s[src], xs_s[:total])
    assert torch.equal(h_fused[:total], h_ref[:total])


@pytest.mark.parametrize("case", FP8_GEMM_CASES, ids=lambda c: c[0])
def test_grouped_gemm_fp8(gpu, case):
    """fp8 GEMMs against float64 dot products of the same decoded operands and
    scales: h = bf16(silu(g)*u) and ys = bf16(y), fp32 accumulation."""
    name, D, F, sizes = case
    print(f"fp8 gemm case {case}", flush=True)
    rng = np.random.default_rng(93 + D)
    N = len(sizes)
    offsets = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    R = int(offsets[-1])
    xq, xs = O.quantize_rows_e4m3(rng.standard_normal((R, D)).astype(np.float32))
    wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
    wd = (0.02 * rng.standard_normal((N, F, D))).astype(np.float32)
    off_t = torch.from_numpy(offsets).to(gpu)
    pgu, sgu = K.pack_fp8_gate_up(dev_f32(wg, gpu), dev_f32(wu, gpu))
    pd, sd = K.pack_fp8_down(dev_f32(wd, gpu))
    h = K.grouped_gate_up_fp8(torch.from_numpy(xq).to(gpu), torch.from_numpy(xs).to(gpu), off_t, pgu, sgu)
    h_host = host(h)
    hq, hs = O.quantize_rows_e4m3(h_host)
    ys = K.grouped_down_fp8(torch.from_numpy(hq).to(gpu), torch.from_numpy(hs).to(gpu), off_t, pd, sd)
    ys_host = host(ys)
    torch.cuda.synchronize()
    wq = O.quantize_expert_weights({"expert_w_gate": wg, "expert_w_up": wu, "expert_w_down": wd})
    x64 = O.e4m3_decode(xq).astype(np.float64) * xs[:, None]
    h64 = O.e4m3_decode(hq).astype(np.float64) * hs[:, None]
    for e in range(N):
        a, b = offsets[e], offsets[e + 1]
        if b == a:
            continue
        g = (x64[a:b] @ O.e4m3_decode(wq["wg_q"][e]).astype(np.float64)) * wq["wg_s"][e]
        u = (x64[a:b] @ O.e4m3_decode(wq["wu_q"][e]).astype(np.float64)) * wq["wu_s"][e]
        h_ref = swiglu_ref(g, u)
        err_h = np.abs(h_host[a:b] - h_ref)
        assert np.all(err_h <= 8e-3 * np.abs(h_ref) + 1e-3 * np.abs(h_ref).max()), \
            f"h expert {e}: max err {err_h.max()}"
        y_ref = (h64[a:b] @ O.e4m3_decode(wq["wd_q"][e]).astype(np.float64)) * wq["wd_s"][e]
        err_y = np.abs(ys_host[a:b] - y_ref)
        assert np.all(err_y <= 8e-3 * np.abs(y_ref) + 1e-3 * np.abs(y_ref).max()), \
            f"ys expert {e}: max err {err_y.max()}"
