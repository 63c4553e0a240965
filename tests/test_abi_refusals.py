"""Argument checks of every compute entry point of the C ABI, on the CPU.

Each call below is refused (or is a zero-size no-op) before the library
touches a device: the pointers are placeholders that are never dereferenced.
What is pinned is the contract a caller codes against: an unsupported shape
returns HMOE_ERR_UNSUPPORTED and names the dimension, a malformed argument
returns HMOE_ERR_INVALID, a short workspace HMOE_ERR_WORKSPACE, a null
pointer is refused once there is work, and zero rows is a no-op that needs
no pointers at all (except where the output is a whole gradient, which is
written even then, and the router weight gradient, which refuses zero tokens
rather than leave d_router unwritten).
"""
import ctypes

import pytest

from hanuman_amd import _lib

P = ctypes.c_void_p(16)  # never dereferenced: every call below fails its checks first
S = None                 # default stream
BF16, F32 = _lib.BF16, _lib.F32
OK, INVALID, UNSUPPORTED, WORKSPACE = _lib.OK, _lib.ERR_INVALID, _lib.ERR_UNSUPPORTED, _lib.ERR_WORKSPACE


@pytest.fixture(scope="module")
def lib():
    return _lib.lib()


def expect(lib, code, needle, name, *args):
    rc = getattr(lib, name)(*args)
    msg = lib.hmoe_last_error().decode()
    assert rc == code, f"{name}{args}: rc {rc}, expected {code} ({msg})"
    if needle:
        assert needle in msg, f"{name}: '{needle}' not in '{msg}'"


# ---- grouped GEMMs: (call builder, name of the K dimension, of the N dimension)
# Builders take (n_experts, rows, d_model, d_ff, pointer) and return the argument list.
def _gate_up(name):
    return name, lambda n, r, d, f, p: (p, p, n, r, d, f, p, p, S)


def _gate_up_gather(name):
    return name, lambda n, r, d, f, p: (p, 64, 2, p, p, n, r, d, f, p, p, S)


GEMMS = [
    # (name, builder, a bad d_model, a bad d_ff, d_model ok, d_ff ok)
    (*_gate_up("hmoe_grouped_gate_up"), 100, 100, 256, 128),
    (*_gate_up("hmoe_grouped_gate_up_raw"), 100, 100, 256, 128),
    (*_gate_up_gather("hmoe_grouped_gate_up_gather"), 100, 100, 256, 128),
    (*_gate_up_gather("hmoe_grouped_gate_up_raw_gather"), 100, 100, 256, 128),
    ("hmoe_grouped_gate_up_swiglu_bwd",
     lambda n, r, d, f, p: (p, p, n, r, d, f, p, p, p, S), 100, 100, 256, 128),
    ("hmoe_grouped_gate_up_swiglu_bwd_gather",
     lambda n, r, d, f, p: (p, 64, 2, p, p, n, r, d, f, p, p, p, S), 100, 100, 256, 128),
    ("hmoe_grouped_down", lambda n, r, d, f, p: (p, p, n, r, f, d, p, p, S), 300, 100, 256, 256),
    ("hmoe_grouped_dgrad_down", lambda n, r, d, f, p: (p, p, n, r, d, f, p, p, S), 100, 300, 256, 256),
    ("hmoe_grouped_dgrad_gate_up", lambda n, r, d, f, p: (p, p, n, r, d, f, p, p, S), 300, 100, 256, 128),
    ("hmoe_grouped_gate_up_fp8", lambda n, r, d, f, p: (p, p, p, n, r, d, f, p, p, p, S),
     64, 100, 256, 128),
    ("hmoe_grouped_gate_up_fp8_qh", lambda n, r, d, f, p: (p, p, p, n, r, d, f, p, p, p, p, S),
     64, 100, 256, 128),
    ("hmoe_grouped_gate_up_fp8_gather",
     lambda n, r, d, f, p: (p, p, 64, 2, p, p, n, r, d, f, p, p, p, S), 64, 100, 256, 128),
    ("hmoe_grouped_gate_up_fp8_gather_qh",
     lambda n, r, d, f, p: (p, p, 64, 2, p, p, n, r, d, f, p, p, p, p, S), 64, 100, 256, 128),
    ("hmoe_grouped_down_fp8", lambda n, r, d, f, p: (p, p, p, n, r, f, d, p, p, p, S), 300, 64, 256, 256),
    ("hmoe_grouped_down_fp8_mx", lambda n, r, d, f, p: (p, p, p, n, r, f, d, p, p, p, S), 300, 64, 256, 256),
    ("hmoe_grouped_gate_up_f32", lambda n, r, d, f, p: (p, p, n, r, d, f, p, p, p, S), 100, 100, 256, 128),
    ("hmoe_grouped_down_f32", lambda n, r, d, f, p: (p, p, n, r, f, d, p, p, S), 100, 100, 256, 128),
    ("hmoe_grouped_dgrad_down_f32", lambda n, r, d, f, p: (p, p, n, r, d, f, p, p, S), 100, 100, 256, 128),
    ("hmoe_grouped_gate_up_swiglu_bwd_f32",
     lambda n, r, d, f, p: (p, p, n, r, d, f, p, p, p, p, S), 100, 100, 256, 128),
    ("hmoe_grouped_dgrad_gate_up_f32",
     lambda n, r, d, f, p: (p, p, n, r, d, f, p, p, p, S), 100, 100, 256, 128),
]


@pytest.mark.parametrize("name,build,bad_d,bad_f,d_ok,f_ok", GEMMS, ids=[g[0] for g in GEMMS])
def test_grouped_gemm_checks(lib, name, build, bad_d, bad_f, d_ok, f_ok):
    expect(lib, INVALID, "n_experts", name, *build(0, 10, d_ok, f_ok, P))
    expect(lib, UNSUPPORTED, "d_model", name, *build(4, 10, bad_d, f_ok, P))
    expect(lib, UNSUPPORTED, "d_ff", name, *build(4, 10, d_ok, bad_f, P))
    expect(lib, INVALID, "rows_cap", name, *build(4, -1, d_ok, f_ok, P))
    # zero rows: nothing to do, and no pointer is looked at
    expect(lib, OK, None, name, *build(4, 0, d_ok, f_ok, None))
    # rows to compute and no buffers
    expect(lib, INVALID, "null", name, *build(4, 10, d_ok, f_ok, None))


def test_gathering_gemms_check_the_token_matrix(lib):
    for name in ("hmoe_grouped_gate_up_gather", "hmoe_grouped_gate_up_raw_gather",
                 "hmoe_grouped_gate_up_swiglu_bwd_gather"):
        tail = (P, P) if "bwd" in name else (P,)
        # rows to gather but no tokens
        expect(lib, INVALID, None, name, P, 0, 2, P, P, 4, 10, 256, 128, P, *tail, S)
        # x of 2 GiB or more: its byte offsets no longer fit the gather's 32-bit offsets
        expect(lib, INVALID, "2 GiB", name, P, 1 << 20, 2, P, P, 4, 10, 1024, 128, P, *tail, S)
    # the e4m3 gather: one byte per value
    expect(lib, INVALID, "2 GiB", "hmoe_grouped_gate_up_fp8_gather_qh",
           P, P, 1 << 22, 2, P, P, 4, 10, 1024, 128, P, P, P, P, S)
    expect(lib, INVALID, "null", "hmoe_grouped_gate_up_fp8_gather_qh",
           P, P, 64, 2, None, P, 4, 10, 256, 128, P, P, P, P, S)


def test_block_scaled_down_needs_its_exponents(lib):
    expect(lib, INVALID, "null", "hmoe_grouped_down_fp8_mx", P, None, P, 4, 10, 256, 256, P, P, P, S)


def test_weight_gradient_checks(lib):
    # the bf16 weight gradients: d_ff and d_model in whole 256-row / 256-column tiles
    expect(lib, UNSUPPORTED, None, "hmoe_grouped_wgrad_down", P, P, P, 4, 10, 100, 256, P, S)
    expect(lib, UNSUPPORTED, None, "hmoe_grouped_wgrad_down", P, P, P, 4, 10, 256, 300, P, S)
    expect(lib, INVALID, "n_experts", "hmoe_grouped_wgrad_down", P, P, P, 0, 10, 256, 256, P, S)
    expect(lib, INVALID, None, "hmoe_grouped_wgrad_down", P, P, P, 4, 1 << 31, 256, 256, P, S)
    expect(lib, UNSUPPORTED, None, "hmoe_grouped_wgrad_gate_up", P, P, P, 4, 10, 300, 128, P, P, S)
    expect(lib, UNSUPPORTED, None, "hmoe_grouped_wgrad_gate_up", P, P, P, 4, 10, 256, 100, P, P, S)
    # zero rows still owes every expert a zero gradient: the outputs are required
    expect(lib, INVALID, "null", "hmoe_grouped_wgrad_down", P, P, P, 4, 0, 256, 256, None, S)
    expect(lib, INVALID, "null", "hmoe_grouped_wgrad_gate_up", P, P, P, 4, 0, 256, 128, P, None, S)
    # float32: no rows argument; the outputs are required
    expect(lib, INVALID, "null", "hmoe_grouped_wgrad_gate_up_f32", P, P, P, 4, 256, 128, P, None, S)
    expect(lib, INVALID, "null", "hmoe_grouped_wgrad_down_f32", P, P, P, 4, 128, 256, None, S)
    expect(lib, INVALID, "n_experts", "hmoe_grouped_wgrad_down_f32", P, P, P, 0, 128, 256, P, S)


def test_fused_launch_checks(lib):
    name = "hmoe_grouped_swiglu_fused"

    def args(n=4, r=10, d=256, f=256, ws=1 << 20, extra=0, p=P, x=P):
        return (x, 64, 2, p, p, n, r, d, f, p, p, p, p, p, ws, 0, extra, S)

    expect(lib, INVALID, "n_experts", name, *args(n=0))
    expect(lib, UNSUPPORTED, "d_model", name, *args(d=128))
    expect(lib, UNSUPPORTED, "d_ff", name, *args(f=128))  # at least one 256-column tile of h
    expect(lib, INVALID, "extra_ready_needed", name, *args(extra=-1))
    expect(lib, OK, None, name, *args(r=0, p=None, x=None))
    expect(lib, INVALID, "null", name, *args(p=None))
    need = lib.hmoe_grouped_swiglu_fused_workspace_bytes(10, 4)
    expect(lib, WORKSPACE, "workspace", name, *args(ws=need - 4))
    # sync words, one ready count per 256-row m-tile, one claim counter per expert
    assert need == (16 + 1 + 4) * 4
    assert lib.hmoe_grouped_swiglu_fused_workspace_bytes(131072 + 1, 64) == (16 + 513 + 64) * 4
    assert lib.hmoe_grouped_swiglu_fused_workspace_bytes(10, 0) == 0


def test_pack_checks(lib):
    for name in ("hmoe_pack_gate_up", "hmoe_pack_gate_up_dgrad"):
        expect(lib, INVALID, "d_ff", name, P, P, F32, 4, 256, 48, P, S)
        expect(lib, INVALID, "dtype", name, P, P, 9, 4, 256, 64, P, S)
        expect(lib, INVALID, "sizes", name, P, P, F32, 0, 256, 64, P, S)
        expect(lib, INVALID, "null", name, P, None, F32, 4, 256, 64, P, S)
    for name in ("hmoe_pack_down", "hmoe_pack_down_dgrad"):
        expect(lib, INVALID, "dtype", name, P, 9, 4, 64, 256, P, S)
        expect(lib, INVALID, "sizes", name, P, F32, 4, 0, 256, P, S)
        expect(lib, INVALID, "null", name, None, F32, 4, 64, 256, P, S)
    expect(lib, INVALID, "d_model", "hmoe_pack_down_dgrad", P, F32, 4, 64, 100, P, S)
    expect(lib, INVALID, "d_ff", "hmoe_pack_fp8_gate_up", P, P, F32, 4, 256, 48, P, P, S)
    expect(lib, INVALID, "null", "hmoe_pack_fp8_gate_up", P, P, F32, 4, 256, 64, P, None, S)
    expect(lib, INVALID, "dtype", "hmoe_pack_fp8_down", P, 9, 4, 64, 256, P, P, S)
    expect(lib, INVALID, "null", "hmoe_pack_fp8_down", P, F32, 4, 64, 256, P, None, S)
    # packed sizes: bf16 [N, 2F, D] and [N, D, F]; e4m3 one byte per value
    assert lib.hmoe_packed_fp8_gate_up_bytes(32, 4096, 2048) == 32 * 2 * 2048 * 4096
    assert lib.hmoe_packed_fp8_down_bytes(32, 2048, 4096) == 32 * 2048 * 4096
    assert lib.hmoe_packed_fp8_gate_up_bytes(0, 4096, 2048) == 0


def test_dispatch_side_checks(lib):
    expect(lib, INVALID, "d_model", "hmoe_permute_rows_fp8", P, BF16, 10, 12, 2, P, P, P, S)
    expect(lib, INVALID, None, "hmoe_permute_rows_fp8", P, BF16, 10, 16, 0, P, P, P, S)
    expect(lib, INVALID, None, "hmoe_permute_rows_fp8", P, 9, 10, 16, 2, P, P, P, S)
    expect(lib, OK, None, "hmoe_permute_rows_fp8", None, BF16, 0, 16, 2, None, None, None, S)
    expect(lib, INVALID, "null", "hmoe_permute_rows_fp8", P, BF16, 10, 16, 2, P, P, None, S)
    expect(lib, INVALID, None, "hmoe_quantize_rows_fp8", P, 10, 12, None, 0, P, P, S)
    expect(lib, INVALID, None, "hmoe_quantize_rows_fp8", P, 10, 16, P, 0, P, P, S)
    expect(lib, OK, None, "hmoe_quantize_rows_fp8", None, 0, 16, None, 0, None, None, S)
    expect(lib, INVALID, "null", "hmoe_quantize_rows_fp8", P, 10, 16, None, 0, P, None, S)
    # the no-alloc plan's histogram holds ceil(T*K / 1024) * N <= 2^18 entries
    expect(lib, WORKSPACE, None, "hmoe_dispatch_plan_noalloc",
           P, 1 << 20, 8, 64, 1 << 20, P, P, P, P, P, S)
    expect(lib, INVALID, "capacity", "hmoe_dispatch_plan_noalloc", P, 1000, 8, 64, 0, P, P, P, P, P, S)


def test_backward_elementwise_checks(lib):
    for name, d_bad in (("hmoe_combine_bwd", 12), ("hmoe_combine_bwd_f32", 6)):
        expect(lib, INVALID, "top_k", name, P, P, P, P, 10, 0, 16, P, P, None, 1.0, S)
        expect(lib, INVALID, "top_k", name, P, P, P, P, 10, 17, 16, P, P, None, 1.0, S)
        expect(lib, INVALID, "d_model", name, P, P, P, P, 10, 2, d_bad, P, P, None, 1.0, S)
        expect(lib, OK, None, name, None, None, None, None, 0, 2, 16, None, None, None, 1.0, S)
        expect(lib, INVALID, "null", name, P, P, P, None, 10, 2, 16, P, P, None, 1.0, S)
        # the shared expert's cotangent is divided by the shared-expert count (>= 1)
        expect(lib, INVALID, None, name, P, P, P, P, 10, 2, 16, P, P, P, 0.5, S)
    expect(lib, INVALID, "d_ff", "hmoe_swiglu_bwd", P, P, P, 4, 10, 48, P, S)
    expect(lib, INVALID, None, "hmoe_swiglu_bwd", P, P, P, 0, 10, 64, P, S)
    expect(lib, OK, None, "hmoe_swiglu_bwd", None, None, None, 4, 0, 64, None, S)
    expect(lib, INVALID, "null", "hmoe_swiglu_bwd", P, None, P, 4, 10, 64, P, S)
    # gather_bwd is the combine with unit weights: its checks are the combine's
    expect(lib, INVALID, "d_model", "hmoe_gather_bwd", P, BF16, P, None, F32, 10, 2, 12, P, F32, S)
    expect(lib, OK, None, "hmoe_gather_bwd", None, BF16, None, None, F32, 0, 2, 16, None, F32, S)


def test_router_backward_checks(lib):
    sm, sg = _lib.ROUTE_SOFTMAX, _lib.ROUTE_SIGMOID_BIAS
    expect(lib, INVALID, None, "hmoe_router_bwd", P, P, P, P, 10, 8, 9, sm, 1.0, P, S)
    expect(lib, INVALID, "mode", "hmoe_router_bwd", P, P, P, P, 10, 8, 2, 5, 1.0, P, S)
    expect(lib, OK, None, "hmoe_router_bwd", None, None, None, None, 0, 8, 2, sm, 1.0, None, S)
    # softmax gates are differentiated through the gates, sigmoid ones through the logits
    expect(lib, INVALID, None, "hmoe_router_bwd", P, P, None, P, 10, 8, 2, sm, 1.0, P, S)
    expect(lib, INVALID, None, "hmoe_router_bwd", None, P, P, P, 10, 8, 2, sg, 1.0, P, S)
    expect(lib, INVALID, "d_model", "hmoe_router_dx", P, P, F32, 10, 100, 8, P, 0, S)
    expect(lib, INVALID, "dtype", "hmoe_router_dx", P, P, 9, 10, 128, 8, P, 0, S)
    expect(lib, OK, None, "hmoe_router_dx", None, None, F32, 0, 128, 8, None, 0, S)
    expect(lib, INVALID, "null", "hmoe_router_dx", P, None, F32, 10, 128, 8, P, 0, S)
    # the router weight gradient: zero tokens is refused (d_router would stay unwritten)
    expect(lib, INVALID, "tokens", "hmoe_router_dw", P, BF16, P, 0, 128, 8, P, P, 1 << 20, S)
    expect(lib, INVALID, "d_model", "hmoe_router_dw", P, BF16, P, 10, 100, 8, P, P, 1 << 20, S)
    expect(lib, INVALID, "dtype", "hmoe_router_dw", P, 9, P, 10, 128, 8, P, P, 1 << 20, S)
    need = lib.hmoe_router_dw_workspace_bytes(1000, 128, 8)
    assert need == 2 * 128 * 8 * 4  # float32 partial sums per 512-token chunk
    expect(lib, WORKSPACE, "workspace", "hmoe_router_dw", P, BF16, P, 1000, 128, 8, P, P, need - 4, S)
    expect(lib, INVALID, "null", "hmoe_router_dw", P, BF16, P, 1000, 128, 8, P, None, need, S)


def test_aux_checks(lib):
    ws = lib.hmoe_aux_workspace_bytes(2, 100, 8)
    expect(lib, INVALID, None, "hmoe_router_aux", P, P, 0, 100, 8, 2, P, P, P, ws, S)
    expect(lib, INVALID, "n_experts", "hmoe_router_aux", P, P, 2, 100, 300, 2, P, P, P, ws, S)
    expect(lib, INVALID, "top_k", "hmoe_router_aux", P, P, 2, 100, 8, 9, P, P, P, ws, S)
    expect(lib, WORKSPACE, None, "hmoe_router_aux", P, P, 2, 100, 8, 2, P, P, P, ws - 4, S)
    expect(lib, INVALID, "null", "hmoe_router_aux", P, P, 2, 100, 8, 2, P, None, P, ws, S)
    wb = lib.hmoe_aux_bwd_workspace_bytes(2, 100, 8)
    # per (sequence, 64-token chunk) expert counts, then per-sequence fractions
    assert wb == (2 * 2 + 2) * 8 * 4
    expect(lib, INVALID, None, "hmoe_router_aux_bwd", P, P, 2, 0, 8, 2, P, P, 0, P, wb, S)
    expect(lib, INVALID, "top_k", "hmoe_router_aux_bwd", P, P, 2, 100, 8, 9, P, P, 0, P, wb, S)
    expect(lib, WORKSPACE, None, "hmoe_router_aux_bwd", P, P, 2, 100, 8, 2, P, P, 0, P, wb - 4, S)
    expect(lib, INVALID, "null", "hmoe_router_aux_bwd", P, P, 2, 100, 8, 2, None, P, 0, P, wb, S)


def test_zero_fill_checks(lib):
    expect(lib, INVALID, "multiple of 4", "hmoe_zero_fill", P, 6, S)
    expect(lib, OK, None, "hmoe_zero_fill", None, 0, S)
    expect(lib, INVALID, "null", "hmoe_zero_fill", None, 8, S)
