"""The measured MoE-layer workloads and their synthetic inputs.

Five shapes (tiny fp32 layer, routing+dispatch+combine with an identity
expert, full bf16 layer, load-skewed layer, fp8-expert layer).  Inputs come
from ``numpy.random.default_rng(seed)`` with a fixed draw order -- x (or the
router logits), router weight, per-expert bias, then w_gate, w_up, w_down --
all drawn as float32 standard normals and scaled.  bf16 tensors are the
round-to-nearest-even rounding of those draws.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field, replace

import numpy as np


@dataclass(frozen=True)
class Workload:
    name: str
    tokens: int
    d_model: int
    n_experts: int
    top_k: int
    d_ff: int                 # 0 for the identity expert
    capacity_factor: float | None
    routing: str = "softmax"  # "softmax" | "sigmoid"
    x_dtype: str = "bf16"     # activations as given to the layer
    router_from_logits: bool = False
    expert: str = "swiglu"    # "swiglu" | "identity"
    zipf_bias: bool = False   # per-expert logit bias 3 * rank^-1.1
    router_w_dtype: str = "f32"
    expert_dtype: str = "bf16"  # "bf16" | "fp8" | "f32" (float32 compute)
    out_dtype: str = "f32"
    batch: int = 1
    weight_std: float = 0.02
    router_std: float = 0.02

    @property
    def seq(self) -> int:
        return self.tokens // self.batch

    @property
    def capacity(self) -> int:
        if self.capacity_factor is None:
            return self.tokens * self.top_k
        return int(math.ceil(self.capacity_factor * self.tokens * self.top_k / self.n_experts))

    @property
    def rows_cap(self) -> int:
        return min(self.tokens * self.top_k, self.n_experts * self.capacity)

    def scaled(self, tokens: int) -> "Workload":
        """Same layer at another token count (one sequence per batch row kept)."""
        b = max(1, min(self.batch, tokens))
        while tokens % b:
            b -= 1
        return replace(self, tokens=tokens, batch=b)


WORKLOADS = {
    "tiny_fp32": Workload("tiny_fp32", tokens=2048, d_model=256, n_experts=8, top_k=2, d_ff=512,
                          capacity_factor=1.25, x_dtype="f32", expert_dtype="f32", batch=4),
    "dispatch_identity": Workload("dispatch_identity", tokens=32768, d_model=2048, n_experts=64,
                                  top_k=8, d_ff=0, capacity_factor=1.0, router_from_logits=True,
                                  expert="identity"),
    "full_bf16": Workload("full_bf16", tokens=16384, d_model=2048, n_experts=64, top_k=8,
                          d_ff=1024, capacity_factor=1.25, batch=8),
    "skewed_bf16": Workload("skewed_bf16", tokens=65536, d_model=2048, n_experts=128, top_k=8,
                            d_ff=768, capacity_factor=1.25, router_from_logits=True,
                            zipf_bias=True),
    "fp8_experts": Workload("fp8_experts", tokens=8192, d_model=4096, n_experts=32, top_k=4,
                            d_ff=2048, capacity_factor=1.25, router_w_dtype="bf16",
                            expert_dtype="fp8", out_dtype="bf16"),
}

# Workload the headline bench line is quoted on.
HEADLINE = "full_bf16"


def bf16_round_np(a: np.ndarray) -> np.ndarray:
    """Round float32 to bf16 (ties to even), returned as float32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16) & 0xFFFFFFFF
    return r.astype(np.uint32).view(np.float32)


def zipf_bias(n_experts: int, rng: np.random.Generator) -> np.ndarray:
    """Per-expert logit bias ``3 * r_e**-1.1`` with ``r`` a seeded permutation of
    1..N: heavy skew (the top expert +3, the median about +0.05)."""
    ranks = rng.permutation(n_experts) + 1
    return (3.0 * ranks.astype(np.float64) ** -1.1).astype(np.float32)


@dataclass
class Inputs:
    """Host (numpy float32) inputs of one workload instance."""
    wl: Workload
    x: np.ndarray                         # [T, D] float32 (bf16 values if x_dtype == bf16)
    logits: np.ndarray | None = None      # [T, N] float32 when routing from given logits
    router: np.ndarray | None = None      # [D, N]
    bias: np.ndarray | None = None        # [N]
    w_gate: np.ndarray | None = None      # [N, D, F]
    w_up: np.ndarray | None = None
    w_down: np.ndarray | None = None      # [N, F, D]
    extra: dict = field(default_factory=dict)


def make_inputs(wl: Workload, seed: int = 0, with_weights: bool = True) -> Inputs:
    rng = np.random.default_rng(seed)
    T, D, N, F = wl.tokens, wl.d_model, wl.n_experts, wl.d_ff
    x = rng.standard_normal((T, D), dtype=np.float32)
    if wl.x_dtype == "bf16":
        x = bf16_round_np(x)
    inp = Inputs(wl, x)
    if wl.router_from_logits:
        inp.logits = rng.standard_normal((T, N), dtype=np.float32)
    else:
        r = (wl.router_std * rng.standard_normal((D, N), dtype=np.float32)).astype(np.float32)
        inp.router = bf16_round_np(r) if wl.router_w_dtype == "bf16" else r
    if wl.zipf_bias:
        inp.bias = zipf_bias(N, rng)
        inp.logits = (inp.logits + inp.bias[None, :]).astype(np.float32)
    if with_weights and wl.expert == "swiglu":
        s = np.float32(wl.weight_std)
        inp.w_gate = (s * rng.standard_normal((N, D, F), dtype=np.float32)).astype(np.float32)
        inp.w_up = (s * rng.standard_normal((N, D, F), dtype=np.float32)).astype(np.float32)
        inp.w_down = (s * rng.standard_normal((N, F, D), dtype=np.float32)).astype(np.float32)
    return inp
