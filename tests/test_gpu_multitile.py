"""Elementwise parity of the persistent grouped GEMMs on their multi-tile path
(needs an MI355X).

The persistent kernels run one workgroup per CU (256 on the MI355X) over the
grouped tile list; a workgroup that owns more than one tile carries its load
pipeline into the next tile (the next tile's first K steps are loaded during
the current tile's last ones), prefetches the next tile's gather sources one
tile ahead, and on an odd number of K steps runs one zero-filled padding step
per tile.  None of that runs below 257 tiles.  Every case here has at least
three tiles per workgroup (asserted from the plan), ragged expert segments of
0 to ~1200 rows, and checks every output element of every expert against
float64 products of the same rounded operands (``model/moe.py:70-74``):
``|got - ref| <= 8e-3 |ref| + 1e-3 max|ref|`` per expert, the bound the
single-tile kernel tests use.  The gathering gate/up GEMMs are compared bit
for bit with the unfused permutation + GEMM on the same multi-tile schedule.
"""
import os

import numpy as np
import pytest
import torch

import oracle as O
from hanuman_amd import kernels as K

pytestmark = pytest.mark.gpu

N_WORKGROUPS = 256     # one persistent workgroup per CU
TILE = 256


def _dev_f32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def _dev_bf16(a, dev):
    return _dev_f32(a, dev).to(torch.bfloat16)


def _host(t):
    return t.float().cpu().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()


def _blas_threads():
    from threadpoolctl import threadpool_limits
    return threadpool_limits(min(16, len(os.sched_getaffinity(0))))


def _skewed_top_idx(rng, T, N, Kk):
    """Top-k without repeats, drawn with graded expert popularity (weights
    e^(-2 i / N)), two experts never chosen and one rarely: segment sizes
    range over 0, a few rows, and ~150 to ~1200 rows (T 4096, N 64, top-8)."""
    p = np.exp(-2.0 * np.linspace(0.0, 1.0, N))
    p[[5, 40]] = 1e-12
    p[17] = 0.004
    p = p[rng.permutation(N)]
    p /= p.sum()
    keys = np.log(rng.random((T, N))) / p          # Efraimidis-Spirakis weighted sampling
    return np.argsort(-keys, axis=1, kind="stable")[:, :Kk].astype(np.int32)


def _n_tiles(offsets, n_cols):
    sizes = np.diff(np.asarray(offsets, np.int64))
    return int(((sizes + TILE - 1) // TILE).sum()) * (n_cols // TILE)


def _silu_mul(g, u):
    return g / (1 + np.exp(-g)) * u


def _bf16_near(v, rel=2e-5, floor=1e-5):
    """The bf16 roundings of every value within rel |v| + floor of v: (lo, hi),
    equal unless v lies that close to a rounding midpoint.  The kernel's float32
    accumulation differs from the float64 sum by far less than that, so its
    bf16 g (or u) is one of the two."""
    d = rel * np.abs(v) + floor
    lo = O.bf16_round((v - d).astype(np.float32)).astype(np.float64)
    hi = O.bf16_round((v + d).astype(np.float32)).astype(np.float64)
    return lo, hi


def _check_swiglu(got, g64, u64, what):
    """h = bf16(silu(bf16 g) * bf16 u) (moe.py:70-72) against float64 g, u.
    Where g or u sits at a bf16 rounding midpoint (to within the float32
    accumulation error), either rounding is correct, and one ulp of g moves
    silu(g) u by up to ~2 % where silu is small (g near -5): each element is
    compared with the nearest of the (up to four) candidates."""
    ref = _silu_mul(O.bf16_round(g64.astype(np.float32)).astype(np.float64),
                    O.bf16_round(u64.astype(np.float32)).astype(np.float64))
    g_lo, g_hi = _bf16_near(g64)
    u_lo, u_hi = _bf16_near(u64)
    err = np.abs(got - ref)
    for gc in (g_lo, g_hi):
        for uc in (u_lo, u_hi):
            err = np.minimum(err, np.abs(got - _silu_mul(gc, uc)))
    amb = int(((g_lo != g_hi) | (u_lo != u_hi)).sum())
    _check(got, ref, what, err=err, note=f"{amb} elements at a g/u rounding midpoint")


def _check(got, ref, what, err=None, note=""):
    err = np.abs(got - ref) if err is None else err
    bound = 8e-3 * np.abs(ref) + 1e-3 * np.abs(ref).max()
    bad = err > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} elements out of bound; "
                           f"first at {np.argwhere(bad)[:3].tolist()}, max err {err.max():.3e} "
                           f"{note}")


def _plan(gpu, T, N, Kk, seed):
    rng = np.random.default_rng(seed)
    top = _skewed_top_idx(rng, T, N, Kk)
    plan = K.dispatch_plan(torch.from_numpy(top).to(gpu), N, T * Kk)
    ref = O.dispatch_plan(top, N, T * Kk)
    assert np.array_equal(_host(plan.offsets), ref["offsets"])
    sizes = np.diff(ref["offsets"])
    return rng, plan, ref, sizes


@pytest.mark.parametrize("D,F", [(2048, 1024), (1216, 1024)], ids=["k32", "odd_k19"])
def test_bf16_gate_up_multitile(gpu, D, F):
    """Gate/up with SwiGLU, plain and gathering, >= 3 tiles per workgroup; D
    1216 is 19 K steps (one zero-filled padding step per tile)."""
    T, N, Kk = 4096, 64, 8
    rng, plan, ref, sizes = _plan(gpu, T, N, Kk, seed=500 + D)
    tiles = _n_tiles(ref["offsets"], 2 * F)
    print(f"bf16 gate/up multitile D={D} F={F}: segments {sizes.min()}-{sizes.max()} rows, "
          f"{tiles} tiles ({tiles / N_WORKGROUPS:.1f} per workgroup)", flush=True)
    assert sizes.min() == 0 and (sizes[sizes > 0] < 64).any() and sizes.max() > 700
    assert tiles >= 3 * N_WORKGROUPS
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
    xt = _dev_bf16(x, gpu)
    w = K.pack_gate_up(_dev_f32(wg, gpu), _dev_f32(wu, gpu))
    h_gather = K.grouped_gate_up_gather(xt, plan, w)
    xs = K.permute_rows(xt, plan, torch.bfloat16)
    h = K.grouped_gate_up(xs, plan.offsets, w)
    torch.cuda.synchronize()
    R = int(ref["offsets"][-1])
    assert torch.equal(h_gather[:R], h[:R]), "gathering gate/up differs from permute + gate/up"
    h_host = _host(h)
    xs_ref = x[ref["perm_src"][:R] // Kk]
    with _blas_threads():
        for e in range(N):
            a, b = int(ref["offsets"][e]), int(ref["offsets"][e + 1])
            if b == a:
                continue
            x64 = xs_ref[a:b].astype(np.float64)
            g = x64 @ O.bf16_round(wg[e]).astype(np.float64)
            u = x64 @ O.bf16_round(wu[e]).astype(np.float64)
            _check_swiglu(h_host[a:b], g, u, f"h expert {e} rows {a}-{b}")


@pytest.mark.parametrize("D,F", [(2048, 1024), (2048, 1216)], ids=["k16", "odd_k19"])
def test_bf16_down_multitile(gpu, D, F):
    """The down GEMM (K = d_ff), >= 3 tiles per workgroup; F 1216 is 19 K
    steps."""
    T, N, Kk = 4096, 64, 8
    rng, plan, ref, sizes = _plan(gpu, T, N, Kk, seed=600 + F)
    tiles = _n_tiles(ref["offsets"], D)
    print(f"bf16 down multitile D={D} F={F}: segments {sizes.min()}-{sizes.max()} rows, "
          f"{tiles} tiles ({tiles / N_WORKGROUPS:.1f} per workgroup)", flush=True)
    assert tiles >= 3 * N_WORKGROUPS
    R = int(ref["offsets"][-1])
    h = O.bf16_round(rng.standard_normal((R, F)).astype(np.float32))
    wd = (0.02 * rng.standard_normal((N, F, D))).astype(np.float32)
    ys = _host(K.grouped_down(_dev_bf16(h, gpu), plan.offsets, K.pack_down(_dev_f32(wd, gpu))))
    torch.cuda.synchronize()
    with _blas_threads():
        for e in range(N):
            a, b = int(ref["offsets"][e]), int(ref["offsets"][e + 1])
            if b == a:
                continue
            y = h[a:b].astype(np.float64) @ O.bf16_round(wd[e]).astype(np.float64)
            _check(ys[a:b], y, f"ys expert {e} rows {a}-{b}")


def test_fp8_gate_up_and_down_multitile(gpu):
    """The e4m3 gate/up GEMM (plain and gathering from the per-token codes of
    x) and the e4m3 down GEMM, >= 3 tiles per workgroup, against float64
    products of the decoded codes times their scales."""
    T, N, Kk, D, F = 4096, 64, 8, 2048, 1024
    rng, plan, ref, sizes = _plan(gpu, T, N, Kk, seed=700)
    tiles_gu, tiles_d = _n_tiles(ref["offsets"], 2 * F), _n_tiles(ref["offsets"], D)
    print(f"fp8 multitile: segments {sizes.min()}-{sizes.max()} rows, {tiles_gu} gate/up and "
          f"{tiles_d} down tiles", flush=True)
    assert min(tiles_gu, tiles_d) >= 3 * N_WORKGROUPS
    R = int(ref["offsets"][-1])
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
    wd = (0.02 * rng.standard_normal((N, F, D))).astype(np.float32)
    xt = _dev_bf16(x, gpu)
    pgu, sgu = K.pack_fp8_gate_up(_dev_f32(wg, gpu), _dev_f32(wu, gpu))
    pd, sd = K.pack_fp8_down(_dev_f32(wd, gpu))
    x_q, x_s = K.quantize_rows_fp8(xt)
    h_gather = K.grouped_gate_up_fp8_gather(x_q, x_s, plan, pgu, sgu)
    xs_q, xs_s = K.permute_rows_fp8(xt, plan)
    h = K.grouped_gate_up_fp8(xs_q, xs_s, plan.offsets, pgu, sgu)
    torch.cuda.synchronize()
    assert torch.equal(h_gather[:R], h[:R]), "gathering fp8 gate/up differs from the permuted one"
    h_host = _host(h)
    hq, hs = O.quantize_rows_e4m3(h_host[:R])
    ys = _host(K.grouped_down_fp8(torch.from_numpy(hq).to(gpu), torch.from_numpy(hs).to(gpu),
                                  plan.offsets, pd, sd))
    torch.cuda.synchronize()
    xq_ref, xsc_ref = O.quantize_rows_e4m3(x)
    src = ref["perm_src"][:R] // Kk
    assert np.array_equal(x_q.cpu().numpy(), xq_ref) and np.array_equal(x_s.cpu().numpy(), xsc_ref)
    wq = O.quantize_expert_weights({"expert_w_gate": wg, "expert_w_up": wu, "expert_w_down": wd})
    x64 = O.e4m3_decode(xq_ref[src]).astype(np.float64) * xsc_ref[src][:, None]
    h64 = O.e4m3_decode(hq).astype(np.float64) * hs[:, None]
    with _blas_threads():
        for e in range(N):
            a, b = int(ref["offsets"][e]), int(ref["offsets"][e + 1])
            if b == a:
                continue
            g = (x64[a:b] @ O.e4m3_decode(wq["wg_q"][e]).astype(np.float64)) * wq["wg_s"][e]
            u = (x64[a:b] @ O.e4m3_decode(wq["wu_q"][e]).astype(np.float64)) * wq["wu_s"][e]
            _check_swiglu(h_host[a:b], g, u, f"fp8 h expert {e} rows {a}-{b}")
            y = (h64[a:b] @ O.e4m3_decode(wq["wd_q"][e]).astype(np.float64)) * wq["wd_s"][e]
            _check(ys[a:b], y, f"fp8 ys expert {e} rows {a}-{b}")
