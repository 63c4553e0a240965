"""Block-scaled e4m3 h between the fp8 expert GEMMs (needs an MI355X).

The gate/up GEMM quantises h in its epilogue (32-column blocks, power-of-two
scales) and the down GEMM feeds the block exponents to the MFMA's operand
scales.  The codes and exponents are checked bit for bit against the oracle's
rule applied to the bf16 h of the unquantised epilogue (the same h values);
the down GEMM bit for bit where its arithmetic is exact (operands whose
products and partial sums are exact in float32, so the result cannot depend
on summation order), against the per-row kernel where the two must agree, and
within the GEMM tolerance on random operands.
"""
import numpy as np
import pytest
import torch

import oracle as O
from hanuman_amd import kernels as K

pytestmark = pytest.mark.gpu


def dev_f32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def dev_u8(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).to(dev)


def host(t):
    return t.float().cpu().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()


def _offsets(sizes):
    return np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)


QH_CASES = [
    # name, D, F, segment sizes
    ("ragged", 256, 128, [0, 1, 255, 256, 257, 600, 0, 31]),
    ("wide_f", 512, 1024, [300, 1024, 513]),
    # 8 column tiles x ~90 row tiles: several tiles per workgroup
    ("multitile", 1024, 1024, [700 + 37 * i for i in range(32)]),
]


@pytest.mark.parametrize("case", QH_CASES, ids=lambda c: c[0])
def test_gate_up_qh_codes_and_exponents_bit_exact(gpu, case):
    name, D, F, sizes = case
    print(f"fp8 qh case {name} D={D} F={F} rows={sum(sizes)}", flush=True)
    rng = np.random.default_rng(7 + D + F)
    N = len(sizes)
    offsets = _offsets(sizes)
    R = int(offsets[-1])
    x = rng.standard_normal((R, D)).astype(np.float32)
    x[::97] = 0.0                               # all-zero h rows: exponent byte 0
    xq, xs = O.quantize_rows_e4m3(x)
    wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
    pgu, sgu = K.pack_fp8_gate_up(dev_f32(wg, gpu), dev_f32(wu, gpu))
    off_t = torch.from_numpy(offsets).to(gpu)
    xq_t, xs_t = dev_u8(xq, gpu), dev_f32(xs, gpu)
    h = K.grouped_gate_up_fp8(xq_t, xs_t, off_t, pgu, sgu)
    h_q, h_exp = K.grouped_gate_up_fp8_qh(xq_t, xs_t, off_t, pgu, sgu)
    torch.cuda.synchronize()
    q_ref, e_ref = O.quantize_blocks_e4m3(host(h)[:R])
    got_q, got_e = host(h_q)[:R], host(h_exp)[:R]
    bad = np.argwhere(got_e != e_ref)
    assert bad.size == 0, f"exponents differ at {bad[:5].tolist()}"
    bad = np.argwhere(got_q != q_ref)
    assert bad.size == 0, f"codes differ at {bad[:5].tolist()}"
    assert (got_e[::97] == 0).all()


QH_GATHER_CASES = [
    # T, D, N, K, F, capacity (rows per expert; small values drop slots)
    (700, 256, 8, 2, 128, 10**6),
    (1000, 384, 6, 4, 256, 300),
    (333, 512, 16, 8, 128, 90),
]


@pytest.mark.parametrize("case", QH_GATHER_CASES,
                         ids=lambda c: f"T{c[0]}_D{c[1]}_N{c[2]}_K{c[3]}_cap{c[5]}")
def test_gate_up_gather_qh_matches_bf16_epilogue(gpu, case):
    T, D, N, Kk, F, cap = case
    print(f"fp8 gather qh case {case}", flush=True)
    rng = np.random.default_rng(31 + T)
    x = O.bf16_round(rng.standard_normal((T, D)).astype(np.float32))
    x_t = torch.from_numpy(x).to(gpu).to(torch.bfloat16)
    top = np.stack([rng.choice(N, Kk, replace=False) for _ in range(T)]).astype(np.int32)
    plan = K.dispatch_plan(torch.from_numpy(top).to(gpu), N, cap)
    wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
    w, ws = K.pack_fp8_gate_up(dev_f32(wg, gpu), dev_f32(wu, gpu))
    x_q, x_s = K.quantize_rows_fp8(x_t)
    h = K.grouped_gate_up_fp8_gather(x_q, x_s, plan, w, ws)
    h_q, h_exp = K.grouped_gate_up_fp8_gather_qh(x_q, x_s, plan, w, ws)
    torch.cuda.synchronize()
    R = int(plan.offsets[-1].item())
    assert R > 0
    q_ref, e_ref = O.quantize_blocks_e4m3(host(h)[:R])
    assert np.array_equal(host(h_exp)[:R], e_ref)
    assert np.array_equal(host(h_q)[:R], q_ref)


# values whose products and sums of up to 1024 terms are exact in float32:
# h in multiples of 2^-4 up to 32 (codes up to 4, exponents -3..3), weights
# in multiples of 2^-2 up to 2, |partial sums| <= 2^16 with lsb 2^-6
_H_GRID = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0], np.float32)
_W_GRID = np.array([0.0, 0.25, 0.5, 1.0, 2.0], np.float32)


def _signed_codes(rng, grid, shape):
    v = rng.choice(grid, size=shape) * rng.choice([-1.0, 1.0], size=shape)
    return O.e4m3_encode(v.astype(np.float32))


MX_CASES = [
    # name, F, D, segment sizes
    ("k2_steps", 128, 256, [0, 1, 255, 256, 257, 600, 0, 31]),
    ("k6_steps", 384, 512, [513, 0, 1000, 77]),
    ("k16_steps", 1024, 256, [4000, 1, 2222]),
    # 8 column tiles x 96 row tiles: three tiles per workgroup
    ("multitile", 1024, 2048, [580 + 3 * i for i in range(32)]),
]


@pytest.mark.parametrize("case", MX_CASES, ids=lambda c: c[0])
def test_down_mx_bit_exact_on_exact_operands(gpu, case):
    """Per-block exponents -3..3 on codes and weights whose arithmetic is
    exact: ys must equal the float64 product rounded to bf16 bit for bit, so
    any misplaced block exponent (wrong row, block, K step or half) shows."""
    name, F, D, sizes = case
    print(f"fp8 mx down exact case {name} F={F} D={D} rows={sum(sizes)}", flush=True)
    rng = np.random.default_rng(11 + F + D)
    N = len(sizes)
    offsets = _offsets(sizes)
    R = int(offsets[-1])
    hq = _signed_codes(rng, _H_GRID, (R, F))
    he = (127 + rng.integers(-3, 4, size=(R, F // 32))).astype(np.uint8)
    wq = _signed_codes(rng, _W_GRID, (N, D, F))          # packed layout [N, D, F]
    ys = K.grouped_down_fp8_mx(dev_u8(hq, gpu), dev_u8(he, gpu),
                               torch.from_numpy(offsets).to(gpu), dev_u8(wq, gpu),
                               torch.ones((N, D), dtype=torch.float32, device=gpu))
    got = host(ys)
    torch.cuda.synchronize()
    h64 = O.dequantize_blocks_e4m3(hq, he)
    for e in range(N):
        a, b = offsets[e], offsets[e + 1]
        if b == a:
            continue
        y = h64[a:b] @ O.e4m3_decode(wq[e]).astype(np.float64).T
        ref = O.bf16_round(y.astype(np.float32))
        bad = np.argwhere(got[a:b] != ref)
        assert bad.size == 0, f"expert {e}: first mismatches {bad[:5].tolist()}"


def test_down_mx_equals_per_row_kernel_on_row_uniform_exponents(gpu):
    """Exponents equal across a row's blocks: the block-scaled GEMM and the
    per-row GEMM with scale 2^e compute the same float32 sums scaled by the
    same power of two, so ys is bit-identical."""
    print("fp8 mx down vs per-row", flush=True)
    rng = np.random.default_rng(5)
    F, D, sizes = 512, 512, [900, 3, 0, 1500, 250]
    N = len(sizes)
    offsets = _offsets(sizes)
    R = int(offsets[-1])
    hq = O.e4m3_encode((rng.standard_normal((R, F)) * 60).astype(np.float32))
    k = rng.integers(-6, 7, size=R)
    he = np.repeat((127 + k)[:, None], F // 32, axis=1).astype(np.uint8)
    wd = (0.02 * rng.standard_normal((N, F, D))).astype(np.float32)
    pd, sd = K.pack_fp8_down(dev_f32(wd, gpu))
    off_t = torch.from_numpy(offsets).to(gpu)
    hq_t = dev_u8(hq, gpu)
    ys_mx = K.grouped_down_fp8_mx(hq_t, dev_u8(he, gpu), off_t, pd, sd)
    ys_row = K.grouped_down_fp8(hq_t, dev_f32(np.ldexp(1.0, k), gpu), off_t, pd, sd)
    torch.cuda.synchronize()
    assert torch.equal(ys_mx[:R], ys_row[:R])


def test_pipeline_matches_block_rule_oracle(gpu):
    """Gate/up with quantised h, then the block-scaled down GEMM, against the
    oracle's block rule (float64 dot products of the same codes) within the
    GEMM tolerance, on ragged segments with several tiles per workgroup."""
    print("fp8 block pipeline", flush=True)
    rng = np.random.default_rng(44)
    D, F = 1024, 512
    sizes = [0, 1, 900, 2048, 257, 3000, 31, 1700]
    N = len(sizes)
    offsets = _offsets(sizes)
    R = int(offsets[-1])
    xq, xs = O.quantize_rows_e4m3(rng.standard_normal((R, D)).astype(np.float32))
    wg, wu = (0.02 * rng.standard_normal((2, N, D, F))).astype(np.float32)
    wd = (0.02 * rng.standard_normal((N, F, D))).astype(np.float32)
    pgu, sgu = K.pack_fp8_gate_up(dev_f32(wg, gpu), dev_f32(wu, gpu))
    pd, sd = K.pack_fp8_down(dev_f32(wd, gpu))
    off_t = torch.from_numpy(offsets).to(gpu)
    h_q, h_exp = K.grouped_gate_up_fp8_qh(dev_u8(xq, gpu), dev_f32(xs, gpu), off_t, pgu, sgu)
    ys = K.grouped_down_fp8_mx(h_q, h_exp, off_t, pd, sd)
    got = host(ys)[:R]
    hq_g, he_g = host(h_q)[:R], host(h_exp)[:R]
    torch.cuda.synchronize()
    wq = O.quantize_expert_weights({"expert_w_gate": wg, "expert_w_up": wu, "expert_w_down": wd})
    ys_ref, h_ref, hq_ref, he_ref = O.expert_ffn_fp8(xq, xs, offsets, wq["wg_q"], wq["wg_s"],
                                                     wq["wu_q"], wq["wu_s"], wq["wd_q"], wq["wd_s"])
    # the kernel's h may sit one bf16 rounding step from the float64 h, which
    # can move a code; the down GEMM is checked on the kernel's own codes
    h64 = O.dequantize_blocks_e4m3(hq_g, he_g)
    for e in range(N):
        a, b = offsets[e], offsets[e + 1]
        if b == a:
            continue
        y = (h64[a:b] @ O.e4m3_decode(wq["wd_q"][e]).astype(np.float64)) * wq["wd_s"][e]
        err = np.abs(got[a:b] - y)
        assert np.all(err <= 8e-3 * np.abs(y) + 1e-3 * np.abs(y).max()), \
            f"ys expert {e}: max err {err.max()}"
    assert np.mean(hq_g == hq_ref[:R]) > 0.99 and np.mean(he_g == he_ref[:R]) > 0.99
    err = O.normwise_rel_err(got, ys_ref[:R])
    print(f"  ys normwise err vs the block-rule oracle {err:.2e}", flush=True)
    assert err < 1e-2


def test_entry_points_refuse_bad_shapes(gpu):
    rng = np.random.default_rng(1)
    off_t = torch.tensor([0, 10], dtype=torch.int32, device=gpu)
    hq = dev_u8(np.zeros((10, 128), np.uint8), gpu)
    bad_exp = dev_u8(np.zeros((10, 3), np.uint8), gpu)
    wq = dev_u8(rng.integers(0, 120, (1, 256, 128)).astype(np.uint8), gpu)
    with pytest.raises(ValueError):
        K.grouped_down_fp8_mx(hq, bad_exp, off_t, wq, torch.ones((1, 256), device=gpu))
    hq = dev_u8(np.zeros((10, 64), np.uint8), gpu)
    w = dev_u8(np.zeros((1, 256, 64), np.uint8), gpu)
    with pytest.raises(Exception, match="d_ff"):
        K.grouped_down_fp8_mx(hq, dev_u8(np.zeros((10, 2), np.uint8), gpu), off_t, w,
                              torch.ones((1, 256), device=gpu))
