"""Pins the CPU oracle (oracle/moe_oracle.py) without running the reference.

The reference (JAX/Flax) cannot run in this image and holds no golden vectors
for the MoE path, so each oracle function is checked against something that
fixes it independently: a library routine (numpy argsort/bincount/matmul,
torch dtype conversions), exact rational arithmetic, brute force on tiny
inputs, or a closed form the mathematics forces.
"""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle as O


# ------------------------------------------------------------------ dtypes --

def test_bf16_round_matches_torch():
    rng = np.random.default_rng(1)
    a = np.concatenate([
        (rng.standard_normal(200_000) * 10.0 ** rng.integers(-30, 30, 200_000)).astype(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 3.3895314e38, -3.3895314e38, 1e-45, 2**-126],
                 np.float32)])
    ours = O.bf16_bits(a)
    ref = torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    assert np.isnan(O.bf16_round(np.array([np.nan], np.float32)))[0]


def test_e4m3_matches_torch_after_clamp():
    rng = np.random.default_rng(2)
    a = np.concatenate([
        (rng.standard_normal(300_000) * 2.0 ** rng.integers(-12, 12, 300_000)).astype(np.float32),
        np.array([0.0, -0.0, 448, 449, 464, 465, 480, 1e6, -1e6, 2**-9, 2**-10, 3 * 2**-10,
                  -2**-10, 2**-6, 2**-7 * 1.0625, 1e-30], np.float32)])
    ours = O.e4m3_encode(a)
    ref = torch.from_numpy(np.clip(a, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)


def test_e4m3_decode_roundtrip_and_grid():
    codes = np.arange(256, dtype=np.uint8)
    v = O.e4m3_decode(codes)
    finite = ~np.isnan(v)
    assert finite.sum() == 254                       # 0x7F and 0xFF are NaN
    assert np.array_equal(O.e4m3_encode(v[finite]), codes[finite])
    assert v[0x7E] == 448.0 and v[0x01] == 2.0 ** -9  # max normal, min subnormal
    torch_v = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(v[finite], torch_v[finite])


# ------------------------------------------------------- deterministic exp --

def test_exp_det_accuracy():
    x = np.linspace(-87.0, 88.5, 3_000_001, dtype=np.float32)
    y = O.exp_det(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    assert np.max(np.abs(y / ref - 1.0)) < 3e-7


def test_exp_det_special_values():
    x = np.array([0.0, -0.0, 88.6, 1e30, -87.5, -1e30, np.nan, 1.0], np.float32)
    y = O.exp_det(x)
    assert y[0] == 1.0 and y[1] == 1.0
    assert np.isinf(y[2]) and np.isinf(y[3])
    assert y[4] == 0.0 and y[5] == 0.0
    assert np.isnan(y[6])
    assert abs(float(y[7]) - math.e) < 3e-7 * math.e


def test_sigmoid_det_against_float64():
    x = np.linspace(-40, 40, 400_001, dtype=np.float32)
    s = O.sigmoid_det(x).astype(np.float64)
    ref = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(s - ref) / ref) < 6e-7
    assert O.sigmoid_det(np.array([100.0, -100.0], np.float32)).tolist() == [1.0, 0.0]


# ------------------------------------------------------------------ router --

def test_total_order_key():
    vals = np.array([-np.inf, -3.0, -1e-30, -0.0, 0.0, 1e-45, 2.0, np.inf], np.float32)
    k = O.total_order_key(vals)
    assert np.all(np.diff(k) > 0)                    # strictly increasing, -0 < +0
    rng = np.random.default_rng(3)
    a = rng.standard_normal(10_000).astype(np.float32)
    assert np.array_equal(np.argsort(O.total_order_key(a), kind="stable"),
                          np.argsort(a, kind="stable"))


def test_router_logits_is_correctly_rounded_dot():
    """Tiny case: the float64 d-ascending sum, rounded once, equals the float32
    rounding of the exact rational dot product."""
    rng = np.random.default_rng(4)
    x = O.bf16_round(rng.standard_normal((6, 16)).astype(np.float32))
    w = (0.02 * rng.standard_normal((16, 5))).astype(np.float32)
    got = O.router_logits(x, w)
    for t in range(6):
        for n in range(5):
            exact = sum(Fraction(float(x[t, d])) * Fraction(float(w[d, n])) for d in range(16))
            assert got[t, n] == np.float32(float(exact))   # float(Fraction) rounds once


def test_router_logits_bruteforce_and_blas():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((7, 33)).astype(np.float32)
    w = rng.standard_normal((33, 9)).astype(np.float32)
    got = O.router_logits(x, w, token_block=3)
    loop = np.empty_like(got)
    for t in range(7):
        for n in range(9):
            acc = 0.0
            for d in range(33):
                acc += float(x[t, d]) * float(w[d, n])
            loop[t, n] = np.float32(acc)
    assert np.array_equal(got, loop)
    blas = (x.astype(np.float64) @ w.astype(np.float64)).astype(np.float32)
    assert np.max(np.abs(got - blas)) <= np.max(np.abs(blas)) * 2e-7


def test_topk_matches_argsort_and_breaks_ties_low_index():
    rng = np.random.default_rng(6)
    key = rng.standard_normal((500, 64)).astype(np.float32)
    idx = O.topk_desc(key, 8)
    ref = np.argsort(-key, axis=1, kind="stable")[:, :8]
    assert np.array_equal(idx, ref)
    tied = np.zeros((2, 8), np.float32)
    tied[0, [1, 5, 6]] = 1.0
    tied[1, :] = 0.5
    got = O.topk_desc(tied, 4)
    assert got[0].tolist() == [1, 5, 6, 0]
    assert got[1].tolist() == [0, 1, 2, 3]
    signed_zero = np.array([[-0.0, 0.0, -0.0, 0.0]], np.float32)
    assert O.topk_desc(signed_zero, 4)[0].tolist() == [1, 3, 0, 2]


def test_route_softmax_gates_are_renormalised_softmax():
    rng = np.random.default_rng(7)
    logits = rng.standard_normal((300, 64)).astype(np.float32)
    idx, g = O.route_softmax(logits, 8)
    l64 = logits.astype(np.float64)
    p = np.exp(l64 - l64.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    sel = np.take_along_axis(p, idx, 1)
    assert np.allclose(g, sel / sel.sum(1, keepdims=True), rtol=2e-6, atol=0)
    assert np.all(np.diff(np.take_along_axis(logits, idx, 1), axis=1) <= 0)


def test_route_sigmoid_matches_reference_formula():
    rng = np.random.default_rng(8)
    logits = (rng.standard_normal((300, 16)) * 3).astype(np.float32)
    bias = (rng.standard_normal(16) * 0.1).astype(np.float32)
    idx, g, scores = O.route_sigmoid(logits, bias, 4, 2.5)
    s64 = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    assert np.allclose(scores, s64, rtol=1e-6, atol=0)
    key = scores + bias
    assert np.array_equal(idx, np.argsort(-key, axis=1, kind="stable")[:, :4])
    sel = np.take_along_axis(s64, idx, 1)
    assert np.allclose(g, sel / (sel.sum(1, keepdims=True) + 1e-9) * 2.5, rtol=2e-6)


# ----------------------------------------------------------- dispatch plan --

@pytest.mark.parametrize("T,K,N,C", [(1, 1, 1, 1), (5, 2, 3, 2), (16, 4, 8, 3), (33, 3, 5, 100),
                                     (64, 8, 64, 1), (40, 2, 4, 20)])
def test_plan_matches_bruteforce(T, K, N, C):
    rng = np.random.default_rng(T * 131 + N)
    top = rng.integers(0, N, size=(T, K)).astype(np.int32)
    a = O.dispatch_plan(top, N, C)
    b = O.dispatch_plan_bruteforce(top, N, C)
    for k in ("counts", "kept", "offsets", "slot_pos", "perm_src", "keep"):
        assert np.array_equal(a[k], b[k]), k


def test_plan_dropless_equals_stable_argsort_and_bincount():
    rng = np.random.default_rng(9)
    top = rng.integers(0, 64, size=(2048, 8)).astype(np.int32)
    R = top.size
    p = O.dispatch_plan(top, 64, R)
    assert np.array_equal(p["perm_src"], np.argsort(top.reshape(-1), kind="stable"))
    assert np.array_equal(p["counts"], np.bincount(top.reshape(-1), minlength=64))
    assert np.array_equal(p["slot_pos"], np.argsort(p["perm_src"], kind="stable"))
    assert p["keep"].all()


def test_plan_capacity_invariants():
    rng = np.random.default_rng(10)
    N, K, T = 16, 4, 1000
    # heavy skew: expert 0 gets far more than its capacity
    top = np.where(rng.random((T, K)) < 0.5, 0, rng.integers(0, N, (T, K))).astype(np.int32)
    C = O.capacity_of(T, K, N, 1.0)
    p = O.dispatch_plan(top, N, C)
    e = top.reshape(-1)
    assert p["counts"].sum() == T * K
    assert np.array_equal(p["kept"], np.minimum(p["counts"], C))
    assert p["keep"].sum() == np.minimum(p["counts"], C).sum()
    kept_idx = np.nonzero(p["keep"])[0]
    total = p["offsets"][-1]
    assert sorted(p["slot_pos"][kept_idx].tolist()) == list(range(total))  # bijection on kept
    assert np.all(p["perm_src"][total:] == -1)
    assert np.all(p["perm_src"][p["slot_pos"][kept_idx]] == kept_idx)
    for ex in range(N):                                  # first C slots of each expert win
        slots = np.nonzero(e == ex)[0]
        assert np.array_equal(np.nonzero(p["keep"][slots])[0], np.arange(min(len(slots), C)))
        seg = p["perm_src"][p["offsets"][ex]:p["offsets"][ex + 1]]
        assert np.all(np.diff(seg) > 0)                  # stable: ascending slot index
        assert np.all(e[seg] == ex)


def test_capacity_formula():
    assert O.capacity_of(16384, 8, 64, 1.25) == 2560
    assert O.capacity_of(32768, 8, 64, 1.0) == 4096
    assert O.capacity_of(65536, 8, 128, 1.25) == 5120
    assert O.capacity_of(8192, 4, 32, 1.25) == 1280
    assert O.capacity_of(2048, 2, 8, 1.25) == 640
    assert O.capacity_of(10, 3, 7, 1.0) == 5             # ceil(30/7)
    assert O.capacity_of(10, 3, 7, None) == 30


def test_permute_rows():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((20, 8)).astype(np.float32)
    top = rng.integers(0, 4, (20, 3)).astype(np.int32)
    p = O.dispatch_plan(top, 4, 6)
    xs = O.permute_rows(x, p["perm_src"], 3)
    for j, i in enumerate(p["perm_src"]):
        if i >= 0:
            assert np.array_equal(xs[j], x[i // 3])
        else:
            assert not xs[j].any()


# ---------------------------------------------------------- expert + combine --

def test_expert_ffn_is_per_expert_matmul():
    rng = np.random.default_rng(12)
    N, D, F = 4, 16, 8
    wg, wu = rng.standard_normal((2, N, D, F)).astype(np.float32)
    wd = rng.standard_normal((N, F, D)).astype(np.float32)
    offsets = np.array([0, 3, 3, 10, 12])               # expert 1 is empty
    xs = rng.standard_normal((14, D)).astype(np.float32)
    ys = O.expert_ffn(xs, offsets, wg, wu, wd, "fp32")
    for e in range(N):
        for r in range(offsets[e], offsets[e + 1]):
            g = xs[r].astype(np.float64) @ wg[e]
            u = xs[r].astype(np.float64) @ wu[e]
            h = g / (1 + np.exp(-g)) * u
            assert np.allclose(ys[r], h @ wd[e], rtol=1e-5, atol=1e-5)
    assert not ys[12:].any()
    yb = O.expert_ffn(xs, offsets, wg, wu, wd, "bf16")
    assert O.normwise_rel_err(yb[:12], ys[:12]) < 2e-2


def test_combine_identity_expert_closed_form():
    rng = np.random.default_rng(13)
    T, K, N, D = 64, 4, 8, 16
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    top = rng.integers(0, N, (T, K)).astype(np.int32)
    g = rng.random((T, K)).astype(np.float32)
    p = O.dispatch_plan(top, N, 20)                     # some drops
    xs = O.permute_rows(x, p["perm_src"], K)
    y = O.combine(xs, p["slot_pos"], g, T, K)
    keep = p["keep"].reshape(T, K).astype(np.float64)
    gb = O.bf16_round(g).astype(np.float64)
    ref = x.astype(np.float64) * (keep * gb).sum(1, keepdims=True)
    assert np.allclose(y, ref, rtol=1e-6, atol=1e-7)
    assert (p["keep"] == 0).any()


def test_whole_layer_with_identical_experts():
    """All experts equal => routed output = (sum_k bf16 gate_k) * expert(x)."""
    rng = np.random.default_rng(14)
    T, D, N, K, F = 32, 16, 6, 3, 8
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    wg1, wu1 = (0.3 * rng.standard_normal((2, D, F))).astype(np.float32)
    wd1 = (0.3 * rng.standard_normal((F, D))).astype(np.float32)
    params = {"router": (0.5 * rng.standard_normal((D, N))).astype(np.float32),
              "bias": np.zeros(N, np.float32),
              "expert_w_gate": np.repeat(wg1[None], N, 0), "expert_w_up": np.repeat(wu1[None], N, 0),
              "expert_w_down": np.repeat(wd1[None], N, 0)}
    r = O.moe_forward(x, params, top_k=K, routing="sigmoid", routed_scaling_factor=2.5)
    one = O.expert_ffn(x, np.array([0, T]), wg1[None], wu1[None], wd1[None], "fp32")
    gsum = O.bf16_round(r["gates"]).astype(np.float64).sum(1, keepdims=True)
    assert np.allclose(r["out"], one * gsum, rtol=1e-5, atol=1e-6)


def test_aux_closed_forms():
    B, S, N, K = 2, 8, 4, 2
    logits = np.zeros((B * S, N), np.float32)          # uniform router
    scores = O.sigmoid_det(logits)
    top = np.tile(np.array([[0, 1], [2, 3]], np.int32), (B * S // 2, 1))
    aux = O.aux_losses(logits, scores, top, B, S, N)
    assert math.isclose(aux["router_z_loss"], math.log(N) ** 2, rel_tol=1e-12)
    assert math.isclose(aux["balance_loss"], 1.0, rel_tol=1e-6)   # perfect balance
    assert math.isclose(aux["mean_entropy"], math.log(N), rel_tol=1e-6)
    assert aux["expert_counts"].tolist() == [B * S // 2] * N


def test_aux_hand_computed_non_uniform():
    """N = 2, logits [0, ln 3]: sigmoid scores [1/2, 3/4] normalise to
    p = [0.4, 0.6] (a softmax would give [0.25, 0.75]); logsumexp = ln 4.
    Worked by hand from moe.py:255-283, not from the oracle's formula."""
    logits = np.array([[0.0, math.log(3.0)]], np.float32)
    scores = np.array([[0.5, 0.75]], np.float32)
    aux = O.aux_losses(logits, scores, np.array([[1]], np.int32), 1, 1, 2)
    p0 = 0.5 / (1.25 + 1e-9)
    p1 = 0.75 / (1.25 + 1e-9)
    assert math.isclose(aux["router_z_loss"], math.log(4.0) ** 2, rel_tol=1e-6)
    ent = -(p0 * math.log(p0 + 1e-9) + p1 * math.log(p1 + 1e-9))
    assert math.isclose(aux["mean_entropy"], ent, rel_tol=1e-9)
    assert abs(aux["mean_entropy"] - 0.6730116670092565) < 1e-8    # -(0.4 ln 0.4 + 0.6 ln 0.6)
    # one token, top-1 on expert 1: fractions [0, 1], mean probs [0.4, 0.6]
    assert math.isclose(aux["balance_loss"], 2 * p1, rel_tol=1e-9)
    assert aux["expert_counts"].tolist() == [0.0, 1.0]


def test_aux_balance_is_per_sequence():
    """Two sequences that route to different experts: per sequence b,
    N * sum_n f[b,n] * mean_s p[b,s,n] (moe.py:268-277).  Sequence 0 sends
    both tokens to expert 0 with p = [0.6, 0.4]; sequence 1 sends them to
    expert 1 with p = [0.4, 0.6] and [0.2, 0.8]: 2 * 0.6 = 1.2 and
    2 * 0.7 = 1.4, mean 1.3.  Fractions or mean probabilities taken over the
    whole batch would give 2 * (0.5 * 0.4 + 0.5 * 0.6) = 1.0."""
    B, S, N = 2, 2, 2
    probs = np.array([[0.6, 0.4], [0.6, 0.4], [0.4, 0.6], [0.2, 0.8]])
    scores = probs.astype(np.float32)           # already normalised: sum 1
    logits = np.zeros((B * S, N), np.float32)
    top = np.array([[0], [0], [1], [1]], np.int32)
    aux = O.aux_losses(logits, scores, top, B, S, N)
    assert math.isclose(aux["balance_loss"], 1.3, rel_tol=1e-7)
    assert aux["expert_counts"].tolist() == [2.0, 2.0]


def test_aux_matches_python_loops():
    """Plain nested loops over (b, s, n) on a tiny random case, written from
    the text of moe.py:253-283 (logsumexp via max-shift, bincount by counting)."""
    rng = np.random.default_rng(17)
    B, S, N, K = 3, 5, 6, 2
    logits = (1.7 * rng.standard_normal((B * S, N))).astype(np.float32)
    scores = O.sigmoid_det(logits)
    top = np.stack([rng.choice(N, K, replace=False) for _ in range(B * S)]).astype(np.int32)
    aux = O.aux_losses(logits, scores, top, B, S, N)
    z = ent = bal = 0.0
    total = [0] * N
    for b in range(B):
        cnt = [0] * N
        mp = [0.0] * N
        for s_ in range(S):
            t = b * S + s_
            row = [float(v) for v in logits[t]]
            m = max(row)
            lse = m + math.log(sum(math.exp(v - m) for v in row))
            z += lse * lse
            sc = [float(v) for v in scores[t]]
            den = sum(sc) + 1e-9
            for n in range(N):
                p = sc[n] / den
                mp[n] += p / S
                ent -= p * math.log(p + 1e-9)
            for k in range(K):
                cnt[int(top[t, k])] += 1
        bal += N * sum(cnt[n] / (S * K) * mp[n] for n in range(N))
        total = [a + c for a, c in zip(total, cnt)]
    assert math.isclose(aux["router_z_loss"], z / (B * S), rel_tol=1e-12)
    assert math.isclose(aux["mean_entropy"], ent / (B * S), rel_tol=1e-12)
    assert math.isclose(aux["balance_loss"], bal / B, rel_tol=1e-12)
    assert aux["expert_counts"].tolist() == [float(c) for c in total]


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_shared_expert_is_one_segment_expert_ffn(precision):
    """One shared expert (moe.py:161-163) is the routed SwiGLU on a single
    segment holding every token (expert_ffn, pinned by numpy.matmul above);
    three shared experts (moe.py:164-168) are the mean of three such calls,
    and three identical experts equal one."""
    rng = np.random.default_rng(23)
    T, D, F = 40, 32, 24
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    wg, wu = (0.2 * rng.standard_normal((2, 3, D, F))).astype(np.float32)
    wd = (0.2 * rng.standard_normal((3, F, D))).astype(np.float32)
    seg = np.array([0, T])
    ones = [O.expert_ffn(x, seg, wg[i][None], wu[i][None], wd[i][None], precision) for i in range(3)]
    one = O.shared_expert(x, wg[0], wu[0], wd[0], 1, precision)
    np.testing.assert_array_equal(one, ones[0])
    three = O.shared_expert(x, wg, wu, wd, 3, precision)
    mean = (ones[0].astype(np.float64) + ones[1] + ones[2]) / 3
    np.testing.assert_allclose(three, mean, rtol=1e-6, atol=1e-7)
    same = O.shared_expert(x, np.stack([wg[0]] * 3), np.stack([wu[0]] * 3), np.stack([wd[0]] * 3),
                           3, precision)
    np.testing.assert_allclose(same, ones[0], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("n_shared", [1, 2])
def test_shared_expert_promoted_is_float32_swiglu_on_bf16_weights(n_shared):
    """A float32 x under bf16 compute reaches the shared expert as given
    (moe.py:249), so x @ w.astype(bf16) promotes to float32: the result is the
    float64 SwiGLU on the bf16-rounded weights up to float32 roundings. Both
    plausible mistakes, unrounded weights and the routed bf16 rounding points,
    are 100x further away. moe_forward picks this mode for a float32 x."""
    rng = np.random.default_rng(41 + n_shared)
    T, D, F = 48, 64, 40
    x = rng.standard_normal((T, D)).astype(np.float32)
    assert not np.array_equal(O.bf16_round(x), x)
    sh = (lambda *s: s) if n_shared == 1 else (lambda *s: (n_shared,) + s)
    wg, wu = (0.1 * rng.standard_normal((2,) + sh(D, F))).astype(np.float32)
    wd = (0.1 * rng.standard_normal(sh(F, D))).astype(np.float32)
    got = O.shared_expert(x, wg, wu, wd, n_shared, "bf16_promoted")
    ref = O.shared_expert(x, O.bf16_round(wg), O.bf16_round(wu), O.bf16_round(wd), n_shared, "fp32")
    assert O.normwise_rel_err(got, ref) < 1e-6
    assert O.normwise_rel_err(O.shared_expert(x, wg, wu, wd, n_shared, "fp32"), got) > 1e-4
    assert O.normwise_rel_err(O.shared_expert(x, wg, wu, wd, n_shared, "bf16"), got) > 1e-4
    # the layer: out with the shared expert minus out without it is that residual
    N, K = 4, 2
    params = {"router": (0.1 * rng.standard_normal((D, N))).astype(np.float32),
              "expert_w_gate": (0.1 * rng.standard_normal((N, D, F))).astype(np.float32),
              "expert_w_up": (0.1 * rng.standard_normal((N, D, F))).astype(np.float32),
              "expert_w_down": (0.1 * rng.standard_normal((N, F, D))).astype(np.float32),
              "shared_w_gate": wg, "shared_w_up": wu, "shared_w_down": wd}
    kw = dict(top_k=K, routing="softmax", dtype="bf16", precision="bf16", x_dtype="f32")
    with_sh = O.moe_forward(x, params, n_shared=n_shared, **kw)["out"]
    without = O.moe_forward(x, params, n_shared=0, **kw)["out"]
    assert O.normwise_rel_err(with_sh.astype(np.float64) - without, got) < 1e-5


@pytest.mark.parametrize("n_shared", [1, 2])
def test_shared_expert_promotion_follows_x_dtype_not_values(n_shared):
    """The promotion is decided by x's dtype (moe.py:249 against :198), not by
    its values: a float32 x whose values are all bf16-exact is still promoted
    (the float32 SwiGLU on bf16 weights, which keeps h and the output
    unrounded), and the same values declared bf16 take the bf16 path.  The two
    results differ, so a value-based rule fails one of the asserts."""
    rng = np.random.default_rng(77 + n_shared)
    T, D, F, N, K = 40, 64, 48, 4, 2
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))   # bf16-exact values
    sh = (lambda *s: s) if n_shared == 1 else (lambda *s: (n_shared,) + s)
    params = {"router": (0.1 * rng.standard_normal((D, N))).astype(np.float32),
              "expert_w_gate": (0.1 * rng.standard_normal((N, D, F))).astype(np.float32),
              "expert_w_up": (0.1 * rng.standard_normal((N, D, F))).astype(np.float32),
              "expert_w_down": (0.1 * rng.standard_normal((N, F, D))).astype(np.float32),
              "shared_w_gate": (0.1 * rng.standard_normal(sh(D, F))).astype(np.float32),
              "shared_w_up": (0.1 * rng.standard_normal(sh(D, F))).astype(np.float32),
              "shared_w_down": (0.1 * rng.standard_normal(sh(F, D))).astype(np.float32)}
    kw = dict(top_k=K, routing="softmax", dtype="bf16", precision="bf16", n_shared=n_shared)
    base = O.moe_forward(x, params, **{**kw, "n_shared": 0})["out"].astype(np.float64)
    f32 = O.moe_forward(x, params, x_dtype="f32", **kw)["out"] - base
    b16 = O.moe_forward(x, params, x_dtype="bf16", **kw)["out"] - base
    default = O.moe_forward(x, params, **kw)["out"] - base
    args = (params["shared_w_gate"], params["shared_w_up"], params["shared_w_down"], n_shared)
    promoted = O.shared_expert(x, *args, "bf16_promoted")
    plain = O.shared_expert(x, *args, "bf16")
    assert O.normwise_rel_err(promoted, plain) > 1e-4
    assert O.normwise_rel_err(f32, promoted) < 1e-5
    assert O.normwise_rel_err(b16, plain) < 1e-5
    assert np.array_equal(default, b16)
    with pytest.raises(ValueError):
        O.moe_forward(x, params, x_dtype="f16", **kw)


# ------------------------------------------------------------------- fp8 --

def test_quantize_rows_e4m3_rule_matches_torch_conversion():
    """Codes are torch's float8_e4m3fn conversion of clamp(a * (448/amax)),
    the row maximum maps to 448, and an all-zero row gets codes 0, scale 1."""
    rng = np.random.default_rng(80)
    a = (rng.standard_normal((16, 300)) * np.exp(rng.uniform(-12, 3, (16, 1)))).astype(np.float32)
    a[3] = 0.0
    a[5, :7] = [-0.0, 1e-30, -1e-30, 3e-5, -3e-5, 0.0, 1e-38]
    q, s = O.quantize_rows_e4m3(a)
    amax = np.abs(a).max(axis=1)
    inv = np.where(amax > 0, np.float32(448.0) / np.where(amax > 0, amax, 1), 1).astype(np.float32)
    ref = torch.from_numpy(np.clip((a * inv[:, None]).astype(np.float32), -448, 448)).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(q, ref)
    assert s[3] == 1.0 and not q[3].any()
    nz = amax > 0
    assert np.array_equal(np.abs(O.e4m3_decode(q[nz])).max(axis=1), np.full(nz.sum(), 448.0, np.float32))
    assert np.array_equal(s[nz], (amax[nz] / np.float32(448.0)).astype(np.float32))


def test_quantize_cols_e4m3_is_rowwise_on_the_transpose():
    rng = np.random.default_rng(81)
    w = (0.02 * rng.standard_normal((3, 64, 40))).astype(np.float32)
    q, s = O.quantize_cols_e4m3(w)
    qt, st = O.quantize_rows_e4m3(np.swapaxes(w, -1, -2))
    assert np.array_equal(q, np.swapaxes(qt, -1, -2)) and np.array_equal(s, st)


def test_quantization_error_bound():
    """e4m3 keeps 3 mantissa bits: dequantised values are within 2^-4 relative
    (normal range) or half a subnormal step times the scale."""
    rng = np.random.default_rng(82)
    a = rng.standard_normal((8, 1000)).astype(np.float32)
    q, s = O.quantize_rows_e4m3(a)
    deq = O.e4m3_decode(q).astype(np.float64) * s[:, None]
    err = np.abs(deq - a)
    bound = np.maximum(np.abs(a) * 2.0 ** -4, s[:, None] * 2.0 ** -10) * 1.0001
    assert np.all(err <= bound)


def _min_exponent_bruteforce(amax):
    """Smallest integer e >= -127 with amax <= 448 * 2**e, by search in float64
    (exact: 448 * 2**e is a float64 for every e in range)."""
    e = -127
    if amax > 448.0 * 2.0 ** -127:
        e = int(np.floor(np.log2(amax / 448.0))) - 2
        while amax > np.ldexp(448.0, e):
            e += 1
    return e


def test_block_exponent_is_minimal_power_of_two_cover():
    """e is the smallest exponent whose 448 * 2**e covers the block maximum,
    on the edges the field formula turns on: exactly 448 * 2**k, one float32
    ulp either side, the 1.75 mantissa boundary, zero, subnormals, the
    largest float32."""
    rng = np.random.default_rng(90)
    vals = [0.0, 1e-45, 1e-40, 2.0 ** -126, 448.0, 3.4e38, 1.0, 1.75, 1.7500001, 2.0]
    for k in (-140, -130, -127, -20, -3, 0, 1, 9, 60, 118):
        base = np.float32(np.ldexp(448.0, k)) if k > -150 else np.float32(0)
        vals += [float(base), float(np.nextafter(base, np.float32(np.inf))),
                 float(np.nextafter(base, np.float32(0)))]
    vals += list(np.exp(rng.uniform(-95, 85, 4000)))
    amax = np.array(vals, dtype=np.float32)
    got = O.block_exponent_e8m0(amax)
    want = np.array([_min_exponent_bruteforce(float(v)) for v in amax])
    assert np.array_equal(got, want)
    assert got.min() >= -127 and got.max() <= 127


def test_quantize_blocks_e4m3_rule_against_torch_per_block():
    """Codes are torch's float8_e4m3fn conversion of a * 2**-e block by block
    (32 columns, e from the brute-force search), nothing saturates, every
    nonzero block's largest code lies in (224, 448], and an all-zero block
    gets exponent byte 0 and zero codes."""
    rng = np.random.default_rng(91)
    a = (rng.standard_normal((6, 256)) * np.exp(rng.uniform(-30, 30, (6, 8))).repeat(32, axis=1))
    a = a.astype(np.float32)
    a[2, 64:96] = 0.0
    a[3, 0:32] = -0.0
    a[4, 32:64] = 1e-40                        # subnormal block
    a[5, 96:128] = np.float32(448.0 * 2.0 ** 5)  # exactly on a power-of-two cover
    q, e8 = O.quantize_blocks_e4m3(a)
    assert q.shape == a.shape and e8.shape == (6, 8) and e8.dtype == np.uint8
    for r in range(a.shape[0]):
        for j in range(8):
            blk = a[r, 32 * j:32 * j + 32]
            e = _min_exponent_bruteforce(float(np.abs(blk).max()))
            assert e8[r, j] == e + 127
            scaled = (blk.astype(np.float64) * 2.0 ** -e).astype(np.float32)
            assert np.abs(scaled).max() <= 448.0
            ref = torch.from_numpy(scaled).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            assert np.array_equal(q[r, 32 * j:32 * j + 32], ref), (r, j)
            top = np.abs(O.e4m3_decode(q[r, 32 * j:32 * j + 32])).max()
            if np.abs(blk).max() > 448.0 * 2.0 ** -127:
                assert 224.0 <= top <= 448.0, (r, j, top)
    assert e8[2, 2] == 0 and not O.e4m3_decode(q[2, 64:96]).any()
    assert e8[5, 3] == 5 + 127 and (q[5, 96:128] == 0x7E).all()


def test_block_quantization_error_bound():
    """Dequantised values are within 2^-4 relative (e4m3 normal range) or half
    a subnormal step, 2^-10, times the block's power of two."""
    rng = np.random.default_rng(92)
    a = (rng.standard_normal((16, 512)) * np.exp(rng.uniform(-8, 8, (16, 1)))).astype(np.float32)
    q, e8 = O.quantize_blocks_e4m3(a)
    deq = O.dequantize_blocks_e4m3(q, e8)
    scale = np.repeat(2.0 ** (e8.astype(np.int64) - 127), 32, axis=1)
    assert np.all(np.abs(deq - a) <= np.maximum(np.abs(a) * 2.0 ** -4, scale * 2.0 ** -10))


def _e4m3_grid_matrix(rng, shape, axis):
    """Values on the e4m3 grid whose maximum |v| along `axis` is exactly 448,
    so per-row/column quantisation is the identity with scale 1."""
    grid = O.e4m3_decode(np.arange(0, 126, dtype=np.uint8))          # 0 .. 448
    v = rng.choice(grid[grid <= 64], size=shape) * rng.choice([-1.0, 1.0], size=shape)
    v = v.astype(np.float32)
    idx = [slice(None)] * len(shape)
    idx[axis] = 0
    v[tuple(idx)] = 448.0
    return v


def test_expert_ffn_fp8_reduces_to_library_matmul_on_exact_operands():
    rng = np.random.default_rng(83)
    N, D, F = 3, 64, 32
    offsets = np.array([0, 5, 5, 17], np.int64)
    R = int(offsets[-1])
    x = _e4m3_grid_matrix(rng, (R, D), axis=1)
    wg, wu = (_e4m3_grid_matrix(rng, (N, D, F), axis=1) for _ in range(2))
    wd = _e4m3_grid_matrix(rng, (N, F, D), axis=1)
    xq, xs = O.quantize_rows_e4m3(x)
    assert np.array_equal(O.e4m3_decode(xq), x) and np.all(xs == 1.0)
    wq = O.quantize_expert_weights({"expert_w_gate": wg, "expert_w_up": wu, "expert_w_down": wd})
    assert all(np.all(wq[k] == 1.0) for k in ("wg_s", "wu_s", "wd_s"))
    ys, h, hq, he = O.expert_ffn_fp8(xq, xs, offsets, wq["wg_q"], wq["wg_s"], wq["wu_q"],
                                     wq["wu_s"], wq["wd_q"], wq["wd_s"])
    ys_r, h_r, hq_r, hs = O.expert_ffn_fp8(xq, xs, offsets, wq["wg_q"], wq["wg_s"], wq["wu_q"],
                                           wq["wu_s"], wq["wd_q"], wq["wd_s"], h_rule="row")
    assert np.array_equal(h_r, h) and he.shape == (R, F // 32) and hs.shape == (R,)
    for e in range(N):
        a, b = offsets[e], offsets[e + 1]
        if b == a:
            continue
        # g and u are rounded to bf16 before the SwiGLU (moe.py:70-72's points)
        g = np.matmul(x[a:b].astype(np.float64), wg[e].astype(np.float64))
        u = np.matmul(x[a:b].astype(np.float64), wu[e].astype(np.float64))
        g = O.bf16_round(g.astype(np.float32)).astype(np.float64)
        u = O.bf16_round(u.astype(np.float32)).astype(np.float64)
        assert np.array_equal(h[a:b], O.bf16_round((g / (1 + np.exp(-g)) * u).astype(np.float32)))
        # block rule: each 32-column block of h times its power of two
        scale = np.repeat(2.0 ** (he[a:b].astype(np.int64) - 127), 32, axis=1)
        hh = O.e4m3_decode(hq[a:b]).astype(np.float64) * scale
        y = np.matmul(hh, wd[e].astype(np.float64))
        assert np.array_equal(ys[a:b], O.bf16_round(y.astype(np.float32)))
        hh = O.e4m3_decode(hq_r[a:b]).astype(np.float64) * hs[a:b, None]
        y = np.matmul(hh, wd[e].astype(np.float64))
        assert np.array_equal(ys_r[a:b], O.bf16_round(y.astype(np.float32)))


def test_fp8_layer_within_tolerance_of_fp32_on_dequantised_weights():
    """The fp8 rule's expected accuracy at a small shape: normwise error of the
    e4m3 layer against the float32 layer on the dequantised weights < 5e-2."""
    from hanuman_amd import workloads as W
    wl = W.WORKLOADS["fp8_experts"].scaled(128)
    wl = W.Workload(**{**wl.__dict__, "d_model": 512, "d_ff": 256})
    inp = W.make_inputs(wl, seed=0)
    params = {"router": inp.router, "expert_w_gate": inp.w_gate, "expert_w_up": inp.w_up,
              "expert_w_down": inp.w_down}
    r8 = O.moe_forward(inp.x, params, top_k=wl.top_k, routing="softmax",
                       capacity_factor=wl.capacity_factor, expert="swiglu_fp8", out_dtype="bf16")
    ref = O.moe_forward(inp.x, {**params, **O.dequantized_weights(r8["fp8"])}, top_k=wl.top_k,
                        routing="softmax", capacity_factor=wl.capacity_factor, precision="fp32")
    assert np.array_equal(r8["top_idx"], ref["top_idx"])
    err = O.normwise_rel_err(r8["out"], ref["out"])
    assert err < 5e-2, err
