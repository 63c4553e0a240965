"""C-ABI library checks that need no GPU: it loads, exports every symbol the
header declares, and rejects bad arguments with a status code and message
before touching the device."""
import ctypes

import numpy as np
import pytest

import oracle as O
from hanuman_amd import _lib


@pytest.fixture(scope="module")
def lib():
    return _lib.lib()


def test_exports_every_declared_symbol(lib):
    names = _lib.header_symbols()
    assert len(names) >= 18
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "binding signatures must cover the header"


def test_abi_version(lib):
    assert lib.hmoe_abi_version() == 1


@pytest.mark.parametrize("T,K,N,cf", [(16384, 8, 64, 1.25), (32768, 8, 64, 1.0),
                                      (65536, 8, 128, 1.25), (8192, 4, 32, 1.25),
                                      (2048, 2, 8, 1.25), (10, 3, 7, 1.0), (10, 3, 7, None),
                                      (1000, 4, 16, 0.001), (1, 1, 1, 7.0)])
def test_capacity_and_rows_cap_match_oracle(lib, T, K, N, cf):
    c = lib.hmoe_capacity(T, K, N, 0.0 if cf is None else cf)
    assert c == O.capacity_of(T, K, N, cf)
    assert lib.hmoe_rows_cap(T, K, N, c) == O.rows_cap_of(T, K, N, c)


def test_workspace_sizes(lib):
    # one int32 per (block of 1024 slots, expert)
    assert lib.hmoe_plan_workspace_bytes(16384, 8, 64) == 128 * 64 * 4
    assert lib.hmoe_plan_workspace_bytes(1000, 3, 7) == 3 * 7 * 4
    assert lib.hmoe_plan_workspace_bytes(0, 8, 64) == 0
    assert lib.hmoe_packed_gate_up_bytes(64, 2048, 1024) == 64 * 2048 * 2048 * 2
    assert lib.hmoe_packed_down_bytes(64, 1024, 2048) == 64 * 1024 * 2048 * 2
    assert lib.hmoe_aux_workspace_bytes(8, 2048, 64) == 8 * 32 * (2 * 64 + 2) * 4


def _err(lib):
    return lib.hmoe_last_error().decode()


def test_router_rejects_bad_arguments(lib):
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc = lib.hmoe_router(p, _lib.BF16, p, _lib.F32, None, 10, 64, 0, 2, 0, 1.0, p, p, p, None)
    assert rc == _lib.ERR_INVALID and "n_experts" in _err(lib)
    rc = lib.hmoe_router(p, _lib.BF16, p, _lib.F32, None, 10, 64, 8, 9, 0, 1.0, p, p, p, None)
    assert rc == _lib.ERR_INVALID and "top_k" in _err(lib)
    rc = lib.hmoe_router(p, 7, p, _lib.F32, None, 10, 64, 8, 2, 0, 1.0, p, p, p, None)
    assert rc == _lib.ERR_INVALID and "dtype" in _err(lib)
    rc = lib.hmoe_router(p, _lib.BF16, p, _lib.F32, None, 10, 64, 8, 2, 5, 1.0, p, p, p, None)
    assert rc == _lib.ERR_INVALID and "mode" in _err(lib)
    rc = lib.hmoe_router(None, _lib.BF16, p, _lib.F32, None, 10, 64, 8, 2, 0, 1.0, p, p, p, None)
    assert rc == _lib.ERR_INVALID and "null" in _err(lib)
    # zero tokens is a no-op
    assert lib.hmoe_router(None, _lib.BF16, None, _lib.F32, None, 0, 64, 8, 2, 0, 1.0,
                           None, None, None, None) == _lib.OK
    # the router with x's e4m3 quantisation: bf16 x only, every output given
    rc = lib.hmoe_router_quant_fp8(p, _lib.F32, p, _lib.F32, None, 10, 64, 8, 2, 0, 1.0,
                                   p, p, p, p, p, None)
    assert rc == _lib.ERR_INVALID and "BF16" in _err(lib)
    rc = lib.hmoe_router_quant_fp8(p, _lib.BF16, p, _lib.F32, None, 10, 64, 8, 2, 0, 1.0,
                                   p, p, p, p, None, None)
    assert rc == _lib.ERR_INVALID and "null" in _err(lib)
    rc = lib.hmoe_router_quant_fp8(p, _lib.BF16, p, _lib.F32, None, 10, 60, 8, 2, 0, 1.0,
                                   p, p, p, p, p, None)
    assert rc == _lib.ERR_INVALID and "d_model" in _err(lib)
    assert lib.hmoe_router_quant_fp8(None, _lib.BF16, None, _lib.F32, None, 0, 64, 8, 2, 0, 1.0,
                                     None, None, None, None, None, None) == _lib.OK


def test_plan_rejects_small_workspace_and_bad_sizes(lib):
    p = ctypes.c_void_p(16)
    rc = lib.hmoe_dispatch_plan(p, 1000, 8, 64, 100, p, p, p, p, p, p, 4, None)
    assert rc == _lib.ERR_WORKSPACE and "workspace" in _err(lib)
    rc = lib.hmoe_dispatch_plan(p, 1000, 8, 2000, 100, p, p, p, p, p, p, 1 << 30, None)
    assert rc == _lib.ERR_INVALID
    rc = lib.hmoe_dispatch_plan(p, 1000, 8, 64, 0, p, p, p, p, p, p, 1 << 30, None)
    assert rc == _lib.ERR_INVALID and "capacity" in _err(lib)


def test_gemm_rejects_unsupported_shapes(lib):
    p = ctypes.c_void_p(16)
    rc = lib.hmoe_grouped_gate_up(p, p, 8, 100, 200, 128, p, p, None)
    assert rc == _lib.ERR_UNSUPPORTED and "d_model" in _err(lib)
    rc = lib.hmoe_grouped_gate_up(p, p, 8, 100, 256, 100, p, p, None)
    assert rc == _lib.ERR_UNSUPPORTED and "d_ff" in _err(lib)
    rc = lib.hmoe_grouped_down(p, p, 8, 100, 128, 300, p, p, None)
    assert rc == _lib.ERR_UNSUPPORTED and "d_model" in _err(lib)
    rc = lib.hmoe_grouped_down(p, p, 0, 100, 128, 256, p, p, None)
    assert rc == _lib.ERR_INVALID
    assert lib.hmoe_grouped_down(None, None, 8, 0, 128, 256, None, None, None) == _lib.OK


def test_permute_and_combine_reject_bad_shapes(lib):
    p = ctypes.c_void_p(16)
    assert lib.hmoe_permute_rows(p, _lib.BF16, 10, 12, 2, p, p, _lib.BF16, None) == _lib.ERR_INVALID
    assert lib.hmoe_permute_rows(p, _lib.BF16, 10, 16, 2, p, p, 9, None) == _lib.ERR_INVALID
    assert lib.hmoe_combine(p, _lib.BF16, p, p, None, 0, 10, 17, 16, p, _lib.F32, None) == _lib.ERR_INVALID
    assert lib.hmoe_combine(p, _lib.BF16, p, p, None, 0, 10, 2, 12, p, _lib.F32, None) == _lib.ERR_INVALID
    assert lib.hmoe_combine(p, _lib.BF16, p, p, p, 5, 10, 2, 16, p, _lib.F32, None) == _lib.ERR_INVALID


def test_errors_raise_from_python_binding(lib):
    with pytest.raises(_lib.HmoeError) as ei:
        _lib.call("hmoe_router_from_logits", ctypes.c_void_p(16), None, 10, 300, 2, 1, 1.0,
                  ctypes.c_void_p(16), ctypes.c_void_p(16), None)
    assert ei.value.code == _lib.ERR_INVALID and "n_experts" in ei.value.msg
