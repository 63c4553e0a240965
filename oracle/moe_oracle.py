"""NumPy restatement of the MoE-layer forward (reference: ``model/moe.py``).

TEST INFRASTRUCTURE ONLY -- imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, never by the product.

Two families of rules live here:

* reference mode (``model/moe.py:170-294``): sigmoid scores, ``+bias`` top-k,
  gates ``sel/(sum+1e-9)*rsf``, dropless stable-argsort dispatch, bf16 expert
  SwiGLU, fp32 weighted combine, shared expert, aux losses;
* workload mode (rules with no reference code, frozen here and in the design
  notes): softmax routing with renormalised top-k gates, capacity-factor drops
  with token-order priority, an identity expert, and e4m3 quantisation.

Bit-exact contract with the HIP kernels (integer outputs and the fp32 values
that decide them):

* router logits: ``fp32( sum_d x[t,d]*W[d,n] )`` with the sum accumulated in
  float64, ascending ``d``, starting from +0.0.  Every product of a bf16/fp32
  activation and an fp32/bf16 weight has <= 48 significant bits, so it is exact
  in float64 and ``fma`` equals ``mul``-then-``add``: the GPU's fused form and
  NumPy's two-step form give the same bits.  One final round-to-nearest-even.
* ``exp_det``: Cody-Waite range reduction (Cody & Waite, "Software Manual for
  the Elementary Functions", 1980) plus a degree-7 Taylor polynomial in Horner
  form, evaluated in float32 with only correctly rounded ``+ - *`` and an exact
  ``ldexp``; no fused multiply-add.  ``sigmoid_det(l) = 1/(1+exp_det(-l))``.
* top-k: IEEE-754 totalOrder on float32 keys (-0 < +0), descending; equal keys
  put the lower expert index first (XLA ``TopK`` ordering, ``moe.py:183``).
* gate sums run over ``k`` ascending in float32.
* combine: ``y[t] = sum_k bf16(g[t,k]) * ys[pos(t,k)]`` in float32, ``k``
  ascending from +0.0, dropped slots skipped; the product of two bf16 values
  is exact in float32.
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32
F64 = np.float64

__all__ = [
    "bf16_round", "bf16_bits", "bf16_from_bits", "e4m3_encode", "e4m3_decode",
    "exp_det", "sigmoid_det", "total_order_key", "router_logits",
    "router_logits_fast", "topk_desc", "route_sigmoid", "route_softmax",
    "capacity_of", "rows_cap_of", "dispatch_plan", "dispatch_plan_bruteforce",
    "permute_rows", "silu", "expert_ffn", "combine", "combine_identity", "aux_losses",
    "shared_expert", "moe_forward", "quantize_rows_e4m3", "quantize_cols_e4m3",
    "block_exponent_e8m0", "quantize_blocks_e4m3", "dequantize_blocks_e4m3",
    "expert_ffn_fp8", "quantize_expert_weights", "dequantized_weights", "normwise_rel_err",
]


# --------------------------------------------------------------------------
# dtype helpers
# --------------------------------------------------------------------------

def bf16_round(a) -> np.ndarray:
    """Round float32 to the nearest bfloat16 value (ties to even), as float32.

    Mirrors ``.astype(bfloat16)`` (``moe.py:198,204-206,72``).  Overflow rounds
    to +-inf as IEEE round-to-nearest requires; NaN stays NaN.
    """
    a = np.ascontiguousarray(np.asarray(a, dtype=F32))
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(F32)
    return np.where(np.isnan(a), F32(np.nan), out).astype(F32)


def bf16_bits(a) -> np.ndarray:
    """bfloat16 bit patterns (uint16) of ``bf16_round(a)``."""
    return (bf16_round(a).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b) -> np.ndarray:
    """float32 values of bfloat16 bit patterns."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(F32)


_E4M3_LUT = None


def _e4m3_lut() -> np.ndarray:
    global _E4M3_LUT
    if _E4M3_LUT is None:
        vals = np.empty(256, dtype=F32)
        for c in range(256):
            s = -1.0 if c & 0x80 else 1.0
            e = (c >> 3) & 0xF
            m = c & 7
            if e == 0xF and m == 7:
                vals[c] = np.nan
            elif e == 0:
                vals[c] = s * (m / 8.0) * 2.0 ** -6
            else:
                vals[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
        _E4M3_LUT = vals
    return _E4M3_LUT


def e4m3_decode(q) -> np.ndarray:
    """float32 values of OCP e4m3fn codes (bias 7, max 448, 0x7F/0xFF NaN)."""
    return _e4m3_lut()[np.asarray(q, dtype=np.uint8)]


def e4m3_encode(a) -> np.ndarray:
    """Saturating round-to-nearest-even float32 -> OCP e4m3fn code (uint8).

    Values are clamped to +-448 first (the kernels clamp before the hardware
    convert, which would otherwise produce NaN for |a| >= 464).  The sign of
    zero and of values that round to zero is kept.
    """
    a = np.clip(np.asarray(a, dtype=F32), F32(-448.0), F32(448.0))
    sign = np.signbit(a).astype(np.uint8) << 7
    m = np.abs(a).astype(F64)
    _, ex = np.frexp(m)                       # m = f * 2**ex, f in [0.5, 1)
    e = np.maximum(ex - 1, -6)                # binade exponent, subnormals share -6
    quantum = np.ldexp(1.0, e - 3)            # 3 mantissa bits
    q = np.rint(m / quantum) * quantum        # exact power-of-two scaling; RNE
    _, ex2 = np.frexp(q)
    e2 = np.maximum(ex2 - 1, -6)
    sub = q < 2.0 ** -6
    mant_sub = np.rint(q / 2.0 ** -9)
    mant_norm = np.rint((q / np.ldexp(1.0, e2) - 1.0) * 8.0)
    code_norm = ((e2 + 7) << 3) + mant_norm
    code = np.where(sub, mant_sub, code_norm).astype(np.int64)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


# --------------------------------------------------------------------------
# deterministic transcendental functions (shared bit-for-bit with the kernels)
# --------------------------------------------------------------------------

def _f32_bits(u: int) -> np.float32:
    return np.array([u], dtype=np.uint32).view(F32)[0]


# Constants by exact float32 bit pattern (the HIP twin uses the same bits).
_LOG2E = _f32_bits(0x3FB8AA3B)
_LN2_HI = _f32_bits(0x3F317200)           # low 9 bits zero: n*LN2_HI is exact
_LN2_LO = _f32_bits(0x35BFBE8E)           # ln2 - LN2_HI rounded to float32
_EXP_C = [F32(1.0), F32(1.0), F32(0.5), _f32_bits(0x3E2AAAAB), _f32_bits(0x3D2AAAAB),
          _f32_bits(0x3C088889), _f32_bits(0x3AB60B61), _f32_bits(0x39500D01)]  # 1/k!
_EXP_HI = F32(88.5)
_EXP_LO = F32(-87.0)


def exp_det(x) -> np.ndarray:
    """Deterministic float32 exp (Cody-Waite reduction + degree-7 Taylor).

    ``x > 88.5`` returns +inf, ``x < -87`` returns +0 (no subnormal results),
    NaN propagates.  Relative error below 3e-7 on [-87, 88.5] (tested against
    float64 ``np.exp``).  Every operation is a single correctly rounded float32
    ``*``, ``+`` or ``-``; the HIP twin (``hmoe_exp_det``) evaluates the same
    sequence with floating-point contraction disabled.
    """
    x = np.asarray(x, dtype=F32)
    with np.errstate(over="ignore", invalid="ignore", under="ignore"):
        xc = np.clip(x, _EXP_LO, _EXP_HI)
        n = np.rint(xc * _LOG2E).astype(F32)
        r = (xc - n * _LN2_HI).astype(F32)
        r = (r - n * _LN2_LO).astype(F32)
        p = _EXP_C[7]
        for k in range(6, -1, -1):
            p = (p * r + _EXP_C[k]).astype(F32)
        y = np.ldexp(p, n.astype(np.int32)).astype(F32)
        y = np.where(x > _EXP_HI, F32(np.inf), y)
        y = np.where(x < _EXP_LO, F32(0.0), y)
        y = np.where(np.isnan(x), F32(np.nan), y)
    return y.astype(F32)


def sigmoid_det(x) -> np.ndarray:
    """``1/(1+exp_det(-x))`` in float32 (``jax.nn.sigmoid`` at ``moe.py:179``)."""
    x = np.asarray(x, dtype=F32)
    with np.errstate(over="ignore", divide="ignore"):
        return (F32(1.0) / (F32(1.0) + exp_det(-x))).astype(F32)


def total_order_key(a) -> np.ndarray:
    """int64 key whose order is IEEE-754 totalOrder of float32 ``a``."""
    b = np.ascontiguousarray(np.asarray(a, dtype=F32)).view(np.int32).astype(np.int64)
    return np.where(b < 0, -(b & 0x7FFFFFFF) - 1, b)


# --------------------------------------------------------------------------
# router (moe.py:175-192)
# --------------------------------------------------------------------------

def router_logits(x, w, token_block: int = 4096) -> np.ndarray:
    """fp32 router logits ``x_f @ router`` (``moe.py:175,178``), bit-exact recipe.

    ``x`` [T,D] holds bf16 or fp32 values (as float32), ``w`` [D,N] holds fp32
    or bf16 values.  Accumulates in float64, ``d`` ascending from +0.0, rounds
    once to float32 (see module docstring for why this is order-exact).
    """
    x = np.asarray(x, dtype=F32)
    w = np.asarray(w, dtype=F32)
    T, D = x.shape
    D2, N = w.shape
    assert D == D2
    out = np.empty((T, N), dtype=F32)
    w64 = w.astype(F64)
    for t0 in range(0, T, token_block):
        xb = x[t0:t0 + token_block].astype(F64)
        acc = np.zeros((xb.shape[0], N), dtype=F64)
        for d in range(D):
            acc += xb[:, d:d + 1] * w64[d]
        out[t0:t0 + token_block] = acc.astype(F32)
    return out


def router_logits_fast(x, w) -> np.ndarray:
    """BLAS float32 ``x @ w``: the CPU-baseline router (not bit-exact)."""
    return np.asarray(x, dtype=F32) @ np.asarray(w, dtype=F32)


def topk_desc(key, K: int) -> np.ndarray:
    """``lax.top_k`` indices (``moe.py:183``): descending totalOrder, lower index
    first on equal keys.  int32 [T,K]."""
    k = total_order_key(key)
    return np.argsort(-k, axis=1, kind="stable")[:, :K].astype(np.int32)


def _seq_sum_k(a) -> np.ndarray:
    """float32 sum over the last axis, ascending index, from +0.0."""
    acc = np.zeros(a.shape[:-1], dtype=F32)
    for k in range(a.shape[-1]):
        acc = (acc + a[..., k]).astype(F32)
    return acc


def route_sigmoid(logits, bias, K: int, rsf: float):
    """Reference routing (``moe.py:179-192``).

    ``scores = sigmoid(l)``; top-k of ``scores + bias``; gates
    ``sel / (sum_k sel + 1e-9) * rsf``.  Returns (top_idx int32 [T,K],
    gates float32 [T,K], scores float32 [T,N]).
    """
    logits = np.asarray(logits, dtype=F32)
    scores = sigmoid_det(logits)
    b = np.zeros(logits.shape[1], F32) if bias is None else np.asarray(bias, F32)
    key = (scores + b[None, :]).astype(F32)
    idx = topk_desc(key, K)
    sel = np.take_along_axis(scores, idx, axis=1)
    denom = (_seq_sum_k(sel) + F32(1e-9)).astype(F32)
    gates = ((sel / denom[:, None]).astype(F32) * F32(rsf)).astype(F32)
    return idx, gates, scores


def route_softmax(logits, K: int):
    """Workload routing: top-k of softmax(l), gates renormalised over the top-k.

    Selection runs on the logits (softmax is monotone), so it is exact; gates
    are ``exp_det(l_k - l_max) / sum_j exp_det(l_j - l_max)`` over the
    selected experts, which equals the renormalised top-k softmax
    probabilities.  Returns (top_idx, gates).
    """
    logits = np.asarray(logits, dtype=F32)
    idx = topk_desc(logits, K)
    sel = np.take_along_axis(logits, idx, axis=1)
    e = exp_det((sel - sel[:, :1]).astype(F32))
    denom = _seq_sum_k(e)
    gates = (e / denom[:, None]).astype(F32)
    return idx, gates


# --------------------------------------------------------------------------
# dispatch plan (moe.py:54-65) with the capacity rule
# --------------------------------------------------------------------------

def capacity_of(T: int, K: int, N: int, capacity_factor) -> int:
    """``C = ceil(CF * T * K / N)``; ``None`` -> dropless (C = T*K)."""
    if capacity_factor is None:
        return T * K
    return int(math.ceil(capacity_factor * T * K / N))


def rows_cap_of(T: int, K: int, N: int, capacity: int) -> int:
    """Static upper bound on kept rows: ``min(T*K, N*C)``."""
    return min(T * K, N * capacity)


def dispatch_plan(top_idx, N: int, capacity: int) -> dict:
    """Expert-grouped stable permutation with capacity drops.

    ``e_i = top_idx.flat[i]`` for ``i = t*K + k`` (``moe.py:54``).
    ``order = argsort(e, stable)`` (``moe.py:55``), ``counts = bincount(e)``
    (``moe.py:57``).  ``rank_i`` = number of ``i' < i`` with the same expert.
    Slot ``i`` is kept iff ``rank_i < C``; kept rows are packed per expert:
    ``offsets = exclusive_scan(min(counts, C))``, ``slot_pos[i] = offsets[e_i]
    + rank_i`` (or -1), ``perm_src[j] = i`` for the kept row ``j`` (-1 past the
    kept total).  Dropless (C >= T*K): ``perm_src == order`` and ``slot_pos ==
    argsort(order)`` (``moe.py:80``).
    """
    e = np.asarray(top_idx, dtype=np.int64).reshape(-1)
    R = e.size
    order = np.argsort(e, kind="stable")
    counts = np.bincount(e, minlength=N).astype(np.int64)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]])
    rank = np.empty(R, dtype=np.int64)
    rank[order] = np.arange(R) - starts[e[order]]
    keep = rank < capacity
    kept = np.minimum(counts, capacity)
    offsets = np.concatenate([[0], np.cumsum(kept)]).astype(np.int64)
    slot_pos = np.where(keep, offsets[e] + rank, -1)
    rows_cap = min(R, N * capacity)
    perm_src = np.full(rows_cap, -1, dtype=np.int64)
    perm_src[slot_pos[keep]] = np.nonzero(keep)[0]
    return {
        "counts": counts.astype(np.int32),
        "kept": kept.astype(np.int32),
        "offsets": offsets.astype(np.int32),
        "slot_pos": slot_pos.astype(np.int32),
        "perm_src": perm_src.astype(np.int32),
        "keep": keep.astype(np.uint8),
        "order": order.astype(np.int32),
        "rank": rank.astype(np.int32),
    }


def dispatch_plan_bruteforce(top_idx, N: int, capacity: int) -> dict:
    """Pure-Python loop version of :func:`dispatch_plan` for tiny inputs."""
    e = [int(v) for v in np.asarray(top_idx).reshape(-1)]
    R = len(e)
    counts = [0] * N
    rank = [0] * R
    for i, ei in enumerate(e):
        rank[i] = counts[ei]
        counts[ei] += 1
    kept = [min(c, capacity) for c in counts]
    offsets = [0]
    for c in kept:
        offsets.append(offsets[-1] + c)
    slot_pos = [offsets[e[i]] + rank[i] if rank[i] < capacity else -1 for i in range(R)]
    rows_cap = min(R, N * capacity)
    perm_src = [-1] * rows_cap
    for i, j in enumerate(slot_pos):
        if j >= 0:
            perm_src[j] = i
    return {
        "counts": np.array(counts, np.int32), "kept": np.array(kept, np.int32),
        "offsets": np.array(offsets, np.int32), "slot_pos": np.array(slot_pos, np.int32),
        "perm_src": np.array(perm_src, np.int32),
        "keep": np.array([r < capacity for r in rank], np.uint8),
    }


def permute_rows(x_flat, perm_src, K: int) -> np.ndarray:
    """``xs[j] = x_flat[perm_src[j] // K]`` for kept rows (``moe.py:56``);
    rows past the kept total are zero (``moe.py:62-65`` pads with zeros)."""
    x_flat = np.asarray(x_flat)
    perm_src = np.asarray(perm_src)
    xs = np.zeros((perm_src.size, x_flat.shape[1]), dtype=x_flat.dtype)
    valid = perm_src >= 0
    xs[valid] = x_flat[perm_src[valid] // K]
    return xs


# --------------------------------------------------------------------------
# experts (moe.py:23-29, 67-74)
# --------------------------------------------------------------------------

def silu(a):
    a = np.asarray(a)
    return a / (1.0 + np.exp(-a))


def expert_ffn(xs, offsets, wg, wu, wd, precision: str = "fp32") -> np.ndarray:
    """Grouped SwiGLU over expert segments (``moe.py:70-74``).

    Rows ``[offsets[e], offsets[e+1])`` use expert ``e``; rows past
    ``offsets[-1]`` are zero.  ``precision``:

    * ``"fp32"`` -- the fp32 result: float64 arithmetic on the given values
      (fp32 master weights), returned as float32;
    * ``"f32"`` -- float32 BLAS on the same values (the CPU-baseline path);
    * ``"bf16"`` -- ``moe.py``'s casts: bf16 weights (``:204-206``), g and u
      rounded to bf16 (``ragged_dot`` returns the input dtype, ``:70-71``),
      ``h = bf16(silu(g)*u)`` (``:72``), ``ys`` bf16 (``:73``).
    """
    xs = np.asarray(xs, dtype=F32)
    offsets = np.asarray(offsets, dtype=np.int64)
    N = len(offsets) - 1
    D = xs.shape[1]
    ys = np.zeros((xs.shape[0], wd.shape[2]), dtype=F32)
    for e in range(N):
        a, b = int(offsets[e]), int(offsets[e + 1])
        if b <= a:
            continue
        x = xs[a:b]
        if precision == "fp32":
            x64 = x.astype(F64)
            g = x64 @ np.asarray(wg[e], F64)
            u = x64 @ np.asarray(wu[e], F64)
            h = silu(g) * u
            ys[a:b] = (h @ np.asarray(wd[e], F64)).astype(F32)
        elif precision == "f32":
            g = x @ np.asarray(wg[e], F32)
            u = x @ np.asarray(wu[e], F32)
            ys[a:b] = ((silu(g) * u).astype(F32) @ np.asarray(wd[e], F32)).astype(F32)
        elif precision == "bf16":
            g = bf16_round(x @ bf16_round(wg[e]))
            u = bf16_round(x @ bf16_round(wu[e]))
            h = bf16_round(silu(g).astype(F32) * u)
            ys[a:b] = bf16_round(h @ bf16_round(wd[e]))
        else:
            raise ValueError(precision)
    assert ys.shape[1] == D or wd.shape[2] == ys.shape[1]
    return ys


def _e4m3_scales(amax):
    """Dequantisation scale ``amax/448`` and quantisation multiplier
    ``448/amax`` (both correctly rounded float32 divisions); an all-zero group
    gets 1 and 1."""
    amax = np.asarray(amax, dtype=F32)
    pos = amax > 0
    safe = np.where(pos, amax, F32(1.0)).astype(F32)
    s = np.where(pos, (safe / F32(448.0)).astype(F32), F32(1.0)).astype(F32)
    inv = np.where(pos, (F32(448.0) / safe).astype(F32), F32(1.0)).astype(F32)
    return s, inv


def quantize_rows_e4m3(a):
    """Per-row e4m3 quantisation (the fp8 workload rule for activations):
    ``amax`` = max |a| over the row, ``q = e4m3(clamp(a * (448/amax), +-448))``
    (one float32 multiply, round-to-nearest-even, saturating), dequantisation
    scale ``s = amax/448``.  Returns (codes uint8, scales float32)."""
    a = np.asarray(a, dtype=F32)
    amax = np.max(np.abs(a), axis=-1)
    s, inv = _e4m3_scales(amax)
    q = e4m3_encode((a * inv[..., None]).astype(F32))
    return q, s


def quantize_cols_e4m3(w):
    """Per-output-channel e4m3 quantisation of ``w [..., K, Ncols]``: one scale
    per column (max over K), same rule as :func:`quantize_rows_e4m3`.
    Returns (codes uint8, scales float32 [..., Ncols])."""
    w = np.asarray(w, dtype=F32)
    amax = np.max(np.abs(w), axis=-2)
    s, inv = _e4m3_scales(amax)
    q = e4m3_encode((w * inv[..., None, :]).astype(F32))
    return q, s


E4M3_BLOCK = 32          # columns per power-of-two scale block of h


def block_exponent_e8m0(amax) -> np.ndarray:
    """Smallest integer ``e`` with ``amax <= 448 * 2**e``, at least -127 (the
    bottom of the E8M0 scale range; an all-zero block gets -127).

    From the float32 fields of ``amax = 1.m * 2**(E-127)``: ``amax * 2**-e =
    1.m * 2**(8-c)`` for ``e = E - 135 + c``, which is at most 448 exactly when
    ``c = 0`` and ``1.m <= 1.75`` (mantissa field <= 0x600000), else ``c = 1``
    (``1.m * 2**7 < 256``); one less than that ``e`` exceeds 448 either way.
    Returns int64."""
    bits = np.asarray(amax, dtype=F32).view(np.uint32).astype(np.int64)
    E = (bits >> 23) & 0xFF
    e = E - 135 + ((bits & 0x7FFFFF) > 0x600000)
    return np.maximum(e, -127)


def quantize_blocks_e4m3(a, block: int = E4M3_BLOCK):
    """Block-scaled e4m3 (the fp8 workload's rule for ``h``): every ``block``
    consecutive columns of a row share a power-of-two scale ``2**e``,
    ``e = block_exponent_e8m0(max |a| over the block)``, and the codes are
    ``e4m3(a * 2**-e)`` (an exact scaling, then round-to-nearest-even; the
    scaled magnitudes are at most 448 by the choice of ``e``, so nothing
    saturates).  Returns (codes uint8 [..., C], biased exponents uint8
    [..., C/block] = ``e + 127``, the E8M0 encoding of ``2**e``)."""
    a = np.asarray(a, dtype=F32)
    C = a.shape[-1]
    if C % block:
        raise ValueError(f"{C} columns are not a whole number of {block}-column blocks")
    blk = a.reshape(a.shape[:-1] + (C // block, block))
    e = block_exponent_e8m0(np.max(np.abs(blk), axis=-1))
    scaled = (blk.astype(F64) * np.ldexp(1.0, -e)[..., None]).astype(F32)
    return e4m3_encode(scaled).reshape(a.shape), (e + 127).astype(np.uint8)


def dequantize_blocks_e4m3(q, e8, block: int = E4M3_BLOCK) -> np.ndarray:
    """float64 values of block-scaled codes: ``decode(q) * 2**(e8 - 127)``."""
    scale = np.ldexp(1.0, np.asarray(e8, np.int64) - 127)
    return e4m3_decode(q).astype(F64) * np.repeat(scale, block, axis=-1)


def expert_ffn_fp8(xs_q, xs_s, offsets, wg_q, wg_s, wu_q, wu_s, wd_q, wd_s, h_rule: str = "block32"):
    """Grouped SwiGLU on e4m3 operands (the fp8 workload's expert rule).

    ``xs_q [R, D]`` codes with per-row scales ``xs_s``; ``wg_q/wu_q [N, D, F]``
    codes with per-column scales ``[N, F]``; ``wd_q [N, F, D]`` with ``[N, D]``.
    ``g = bf16((x.wg) * sx * sg)``, ``u`` likewise (rounded to bf16 as the
    bf16 path's ``ragged_dot`` outputs are, ``moe.py:70-71``),
    ``h = bf16(silu(g) * u)``.  h is re-quantised for the down GEMM by
    ``h_rule``: ``"block32"`` (the workload's rule,
    :func:`quantize_blocks_e4m3`: a power-of-two scale per 32 columns, which
    the gate/up GEMM applies in its epilogue and the down GEMM's scaled MFMA
    consumes) or ``"row"`` (:func:`quantize_rows_e4m3`, one float32 scale per
    row; the per-row kernels' rule).  ``ys = bf16((deq(hq).wd) * sd)``.  Dot
    products of decoded codes in float64.  Returns (ys float32 of bf16 values,
    h, hq, h_scale) with ``h_scale`` the biased exponents ``[R, F/32]``
    (uint8) or the row scales ``[R]`` (float32)."""
    if h_rule not in ("block32", "row"):
        raise ValueError(h_rule)
    offsets = np.asarray(offsets, dtype=np.int64)
    N = len(offsets) - 1
    R = xs_q.shape[0]
    F = wg_q.shape[2]
    D = wd_q.shape[2]
    h = np.zeros((R, F), F32)
    for e in range(N):
        a, b = int(offsets[e]), int(offsets[e + 1])
        if b <= a:
            continue
        x = e4m3_decode(xs_q[a:b]).astype(F64) * np.asarray(xs_s[a:b], F64)[:, None]
        g = (x @ e4m3_decode(wg_q[e]).astype(F64)) * np.asarray(wg_s[e], F64)[None, :]
        u = (x @ e4m3_decode(wu_q[e]).astype(F64)) * np.asarray(wu_s[e], F64)[None, :]
        g = bf16_round(g.astype(F32)).astype(F64)
        u = bf16_round(u.astype(F32)).astype(F64)
        h[a:b] = bf16_round((silu(g) * u).astype(F32))
    total = int(offsets[-1])
    hq = np.zeros((R, F), np.uint8)
    if h_rule == "block32":
        hs = np.full((R, F // E4M3_BLOCK), 127, np.uint8)
        hq[:total], hs[:total] = quantize_blocks_e4m3(h[:total])
        hh_all = dequantize_blocks_e4m3(hq, hs)
    else:
        hs = np.ones(R, F32)
        hq[:total], hs[:total] = quantize_rows_e4m3(h[:total])
        hh_all = e4m3_decode(hq).astype(F64) * hs.astype(F64)[:, None]
    ys = np.zeros((R, D), F32)
    for e in range(N):
        a, b = int(offsets[e]), int(offsets[e + 1])
        if b <= a:
            continue
        y = (hh_all[a:b] @ e4m3_decode(wd_q[e]).astype(F64)) * np.asarray(wd_s[e], F64)[None, :]
        ys[a:b] = bf16_round(y.astype(F32))
    return ys, h, hq, hs


# --------------------------------------------------------------------------
# combine (moe.py:80-85)
# --------------------------------------------------------------------------

def combine(ys, slot_pos, gates, T: int, K: int, residual=None, ys_dtype: str = "bf16") -> np.ndarray:
    """``y[t] = sum_k g'[t,k] * ys[slot_pos[t*K+k]]`` in float32, ``g'`` the
    gates cast to the rows' dtype: ``bf16(g)`` for bf16 rows, ``g`` for
    float32 rows (``ys_dtype="f32"``, the float32 compute dtype).

    ``inv = argsort(order)``; ``out = ys[inv]``; ``einsum('tkd,tk->td',
    out, weights.astype(out.dtype), preferred_element_type=f32)``
    (``moe.py:80-85``).  ``k`` ascending from +0.0; slots with
    ``slot_pos < 0`` (dropped) are skipped.  ``residual`` (float32 [T,D]) is
    added last.
    """
    ys = np.asarray(ys, dtype=F32)
    slot_pos = np.asarray(slot_pos).reshape(T, K)
    g16 = np.asarray(gates, dtype=F32).reshape(T, K)
    if ys_dtype == "bf16":
        g16 = bf16_round(g16)
    D = ys.shape[1]
    acc = np.zeros((T, D), dtype=F32)
    for k in range(K):
        p = slot_pos[:, k]
        kept = p >= 0
        rows = ys[np.where(kept, p, 0)]
        term = (g16[:, k:k + 1] * rows).astype(F32)
        acc = np.where(kept[:, None], (acc + term).astype(F32), acc)
    if residual is not None:
        acc = (acc + np.asarray(residual, F32)).astype(F32)
    return acc


def combine_identity(x, slot_pos, gates, T: int, K: int) -> np.ndarray:
    """:func:`combine` for the identity expert, reading token rows of ``x``
    directly: ``ys[slot_pos[t*K+k]] == x[t]`` for kept slots, so this is the
    same float32 accumulation without materialising the dispatched buffer."""
    x = np.asarray(x, dtype=F32)
    keep = (np.asarray(slot_pos).reshape(T, K) >= 0)
    g16 = bf16_round(np.asarray(gates, dtype=F32).reshape(T, K))
    acc = np.zeros_like(x)
    for k in range(K):
        term = (g16[:, k:k + 1] * x).astype(F32)
        acc = np.where(keep[:, k:k + 1], (acc + term).astype(F32), acc)
    return acc


# --------------------------------------------------------------------------
# shared expert and aux (moe.py:161-168, 249-292)
# --------------------------------------------------------------------------

def shared_expert(x_flat, w_gate, w_up, w_down, n_shared: int, precision: str = "fp32"):
    """``_shared_ffn`` (``moe.py:161-168``): one SwiGLU (2-D weights) or the
    mean of ``n_shared`` SwiGLUs (3-D weights).  ``precision="bf16_promoted"``:
    a float32 ``x`` under bf16 compute, which ``moe.py:249`` passes as given,
    so ``x @ w.astype(bf16)`` (``moe.py:23-29``) promotes to float32: bf16
    weights, every product and SwiGLU value a float32 result (float64
    arithmetic rounded to float32 at each op)."""
    x = np.asarray(x_flat, F32)

    def one(wg, wu, wd):
        if precision == "bf16_promoted":
            x64 = x.astype(F64)
            g = (x64 @ bf16_round(wg).astype(F64)).astype(F32)
            u = (x64 @ bf16_round(wu).astype(F64)).astype(F32)
            h = (silu(g.astype(F64)) * u.astype(F64)).astype(F32)
            return (h.astype(F64) @ bf16_round(wd).astype(F64)).astype(F32)
        if precision == "f32":
            return ((silu(x @ np.asarray(wg, F32)) * (x @ np.asarray(wu, F32))).astype(F32)
                    @ np.asarray(wd, F32)).astype(F32)
        if precision == "fp32":
            x64 = x.astype(F64)
            return ((silu(x64 @ np.asarray(wg, F64)) * (x64 @ np.asarray(wu, F64)))
                    @ np.asarray(wd, F64)).astype(F32)
        # the routed experts' rounding points (expert_ffn "bf16")
        g = bf16_round(x @ bf16_round(wg))
        u = bf16_round(x @ bf16_round(wu))
        h = bf16_round(silu(g).astype(F32) * u)
        return bf16_round(h @ bf16_round(wd))

    if n_shared == 1:
        return one(w_gate, w_up, w_down)
    out = np.zeros((x.shape[0], np.asarray(w_down).shape[-1]), F64)
    for i in range(n_shared):
        out += one(w_gate[i], w_up[i], w_down[i])
    return (out / n_shared).astype(F32)


def aux_losses(logits, scores, top_idx, B: int, S: int, N: int) -> dict:
    """Aux outputs (``moe.py:253-292``), float64 arithmetic.

    ``router_z_loss = mean(logsumexp(l)^2)``; per-sequence ``counts [B,N]``;
    ``probs = s/(sum s + 1e-9)``; ``balance_loss = mean_b(N * sum_n
    counts/(S*K) * mean_s probs)``; ``mean_entropy = mean(-sum p log(p+1e-9))``;
    ``expert_counts = sum_b counts`` (integer valued).
    """
    l = np.asarray(logits, F64).reshape(B, S, N)
    s = np.asarray(scores, F64).reshape(B, S, N)
    K = np.asarray(top_idx).shape[-1]
    m = l.max(axis=-1, keepdims=True)
    lse = (m + np.log(np.exp(l - m).sum(axis=-1, keepdims=True)))[..., 0]
    z = np.mean(lse ** 2)
    idx = np.asarray(top_idx).reshape(B, S * K)
    counts = np.stack([np.bincount(idx[b], minlength=N) for b in range(B)]).astype(F64)
    frac = counts / (S * K)
    probs = s / (s.sum(axis=-1, keepdims=True) + 1e-9)
    mean_probs = probs.mean(axis=1)
    balance = np.mean(N * np.sum(frac * mean_probs, axis=-1))
    ent = -np.sum(probs * np.log(probs + 1e-9), axis=-1)
    return {
        "router_z_loss": float(z),
        "balance_loss": float(balance),
        "mean_entropy": float(np.mean(ent)),
        "expert_counts": counts.sum(axis=0).astype(F32),
    }


def quantize_expert_weights(params: dict) -> dict:
    """Per-output-channel e4m3 codes and scales of the stacked expert weights
    (``expert_w_gate/up [N,D,F]``: scale per F column; ``expert_w_down
    [N,F,D]``: scale per D column)."""
    wg_q, wg_s = quantize_cols_e4m3(params["expert_w_gate"])
    wu_q, wu_s = quantize_cols_e4m3(params["expert_w_up"])
    wd_q, wd_s = quantize_cols_e4m3(params["expert_w_down"])
    return {"wg_q": wg_q, "wg_s": wg_s, "wu_q": wu_q, "wu_s": wu_s, "wd_q": wd_q, "wd_s": wd_s}


def dequantized_weights(wq: dict) -> dict:
    """float32 expert weights that the e4m3 codes and scales represent (the
    weights of the fp8 workload's float32 tolerance reference)."""
    return {
        "expert_w_gate": (e4m3_decode(wq["wg_q"]) * wq["wg_s"][:, None, :]).astype(F32),
        "expert_w_up": (e4m3_decode(wq["wu_q"]) * wq["wu_s"][:, None, :]).astype(F32),
        "expert_w_down": (e4m3_decode(wq["wd_q"]) * wq["wd_s"][:, None, :]).astype(F32),
    }


# --------------------------------------------------------------------------
# full layer
# --------------------------------------------------------------------------

def normwise_rel_err(y, ref) -> float:
    """``||y - ref||_2 / ||ref||_2`` over the whole array (float64)."""
    y = np.asarray(y, F64)
    ref = np.asarray(ref, F64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(y - ref) / (den if den > 0 else 1.0))


def moe_forward(x, params: dict, *, top_k: int, routing: str = "sigmoid",
                routed_scaling_factor: float = 2.5, capacity_factor=None,
                expert: str = "swiglu", n_shared: int = 0, dtype: str = "bf16",
                precision: str = "fp32", logits=None, fast_router: bool = False,
                batch_shape=None, out_dtype: str = "f32", x_dtype: str | None = None,
                fp8_h_rule: str = "block32") -> dict:
    """Whole-layer forward (``MoE.__call__``, ``moe.py:170-294``).

    ``x`` [T,D] float32 values (bf16-representable when ``dtype="bf16"``).
    ``params``: ``router [D,N]``, ``bias [N]``, ``expert_w_gate/up [N,D,F]``,
    ``expert_w_down [N,F,D]`` and, when ``n_shared > 0``, ``shared_w_*``.
    ``routing``: ``"sigmoid"`` (reference) or ``"softmax"`` (workload).
    ``logits``: precomputed router logits (identity-expert workload).
    ``expert``: ``"swiglu"``, ``"identity"`` or ``"swiglu_fp8"`` (e4m3 operands,
    :func:`expert_ffn_fp8`; quantised weights from ``params["fp8"]`` or
    :func:`quantize_expert_weights`; ``fp8_h_rule`` picks how ``h`` is
    re-quantised, see there).  ``out_dtype="bf16"`` rounds the output.
    ``x_dtype``: the dtype ``x`` arrives in (``"bf16"`` or ``"f32"``; default
    the compute ``dtype``, as ``model/transformer.py`` passes it).  The
    routed path casts ``x`` to the compute dtype (``moe.py:198``); the shared
    expert sees it as given (``moe.py:249``), so a float32 ``x`` under bf16
    compute promotes the shared SwiGLU to float32.  The promotion follows the
    dtype, never ``x``'s values: a float32 ``x`` whose values happen to be
    bf16-exact is still promoted.
    Returns a dict with every intermediate the kernels produce.
    """
    x_dtype = dtype if x_dtype is None else x_dtype
    if x_dtype not in ("bf16", "f32"):
        raise ValueError(x_dtype)
    x = np.asarray(x, dtype=F32)
    T, D = x.shape
    if logits is None:
        logits = (router_logits_fast if fast_router else router_logits)(x, params["router"])
    logits = np.asarray(logits, F32)
    N = logits.shape[1]
    K = top_k
    scores = None
    if routing == "sigmoid":
        top_idx, gates, scores = route_sigmoid(logits, params.get("bias"), K, routed_scaling_factor)
    elif routing == "softmax":
        top_idx, gates = route_softmax(logits, K)
    else:
        raise ValueError(routing)
    C = capacity_of(T, K, N, capacity_factor)
    plan = dispatch_plan(top_idx, N, C)
    x_c = bf16_round(x) if dtype == "bf16" else x
    extra = {}
    if expert == "swiglu_fp8":
        xq, xsc = quantize_rows_e4m3(x_c)
        perm = plan["perm_src"]
        valid = perm >= 0
        xs_q = np.zeros((perm.size, D), np.uint8)
        xs_q[valid] = xq[perm[valid] // K]
        xs_s = np.ones(perm.size, F32)
        xs_s[valid] = xsc[perm[valid] // K]
        wq = params["fp8"] if "fp8" in params else quantize_expert_weights(params)
        ys, h, hq, hs = expert_ffn_fp8(xs_q, xs_s, plan["offsets"], wq["wg_q"], wq["wg_s"],
                                       wq["wu_q"], wq["wu_s"], wq["wd_q"], wq["wd_s"],
                                       h_rule=fp8_h_rule)
        xs = xs_q
        extra = {"x_q": xq, "x_s": xsc, "xs_s": xs_s, "h": h, "hq": hq, "hs": hs, "fp8": wq}
    elif expert == "identity":
        xs = permute_rows(x_c, plan["perm_src"], K)
        ys = xs
    elif expert == "swiglu":
        xs = permute_rows(x_c, plan["perm_src"], K)
        ys = expert_ffn(xs, plan["offsets"], params["expert_w_gate"], params["expert_w_up"],
                        params["expert_w_down"], precision=precision)
    else:
        raise ValueError(expert)
    residual = None
    if n_shared > 0:
        # moe.py:249 passes x as given (only the routed path casts, moe.py:198):
        # a float32 x under bf16 compute promotes the shared SwiGLU to float32
        promoted = dtype == "bf16" and x_dtype == "f32"
        residual = shared_expert(x if promoted else x_c, params["shared_w_gate"],
                                 params["shared_w_up"], params["shared_w_down"], n_shared,
                                 precision="bf16_promoted" if promoted and precision == "bf16"
                                 else precision)
    out = combine(ys, plan["slot_pos"], gates, T, K, residual=residual,
                  ys_dtype="f32" if (dtype == "f32" and expert == "swiglu") else "bf16")
    if out_dtype == "bf16":
        out = bf16_round(out)
    res = {"logits": logits, "top_idx": top_idx, "gates": gates, "plan": plan,
           "capacity": C, "xs": xs, "ys": ys, "out": out, "scores": scores, **extra}
    if routing == "sigmoid" and batch_shape is not None:
        Bb, Ss = batch_shape
        res["aux"] = aux_losses(logits, scores, top_idx, Bb, Ss, N)
    return res
