"""Writes the golden fixtures of the MoE-layer forward (run from the repo root:
``python tests/golden/make_fixtures.py``).

The reference (JAX/Flax, ``model/moe.py``) cannot run in this image, so the
vectors come from the oracle (``oracle/moe_oracle.py``), whose functions are
pinned by the checks in ``tests/test_oracle.py``.  They freeze the oracle's
outputs on two small seeded cases so that a change to the oracle or to a
kernel shows up as a fixture mismatch:

* ``tiny_fp32.npz`` -- the tiny fp32 layer (2048 tokens, d_model 256, 8 experts,
  top-2, d_ff 512, capacity factor 1.25, softmax routing, seed 0): logits,
  top_idx, gates, the dispatch plan, and the float32 output of the first
  ``OUT_ROWS`` tokens.
* ``dispatch_identity_256.npz`` -- the routing + dispatch + combine workload
  truncated to 256 tokens (given logits, 64 experts, top-8, capacity factor
  1.0, identity expert, seed 0): routing, plan and the output of the first 16
  tokens (bit-exact).
* ``reference_mode.npz`` -- sigmoid + bias routing with the routed scaling
  factor, dropless, one shared expert and the aux outputs, inputs included
  (2 x 32 tokens, d_model 64, 4 experts, top-2, d_ff 64, seed 3).
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402
from hanuman_amd import workloads as W  # noqa: E402

PLAN_KEYS = ("counts", "offsets", "slot_pos", "perm_src", "keep")
OUT_ROWS = 128


def tiny_fp32():
    wl = W.WORKLOADS["tiny_fp32"]
    inp = W.make_inputs(wl, seed=0)
    r = O.moe_forward(inp.x, {"router": inp.router, "expert_w_gate": inp.w_gate,
                              "expert_w_up": inp.w_up, "expert_w_down": inp.w_down},
                      top_k=wl.top_k, routing="softmax", capacity_factor=wl.capacity_factor,
                      dtype="bf16", precision="fp32")
    return {"logits": r["logits"], "top_idx": r["top_idx"], "gates": r["gates"],
            "out": r["out"][:OUT_ROWS], **{f"plan_{k}": r["plan"][k] for k in PLAN_KEYS}}


def dispatch_identity_256():
    wl = W.WORKLOADS["dispatch_identity"].scaled(256)
    inp = W.make_inputs(wl, seed=0)
    r = O.moe_forward(inp.x, {}, top_k=wl.top_k, routing="softmax",
                      capacity_factor=wl.capacity_factor, expert="identity", dtype="bf16",
                      logits=inp.logits)
    return {"top_idx": r["top_idx"], "gates": r["gates"], "out": r["out"][:16],
            **{f"plan_{k}": r["plan"][k] for k in PLAN_KEYS}}


def reference_mode():
    rng = np.random.default_rng(3)
    B, S, D, N, K, F = 2, 32, 64, 4, 2, 64
    x = O.bf16_round(rng.standard_normal((B * S, D)).astype(np.float32))
    std = np.float32(D ** -0.5)
    params = {
        "router": (0.05 * rng.standard_normal((D, N))).astype(np.float32),
        "bias": (0.02 * rng.standard_normal(N)).astype(np.float32),
        "expert_w_gate": (std * rng.standard_normal((N, D, F))).astype(np.float32),
        "expert_w_up": (std * rng.standard_normal((N, D, F))).astype(np.float32),
        "expert_w_down": (std * rng.standard_normal((N, F, D))).astype(np.float32),
        "shared_w_gate": (std * rng.standard_normal((D, F))).astype(np.float32),
        "shared_w_up": (std * rng.standard_normal((D, F))).astype(np.float32),
        "shared_w_down": (std * rng.standard_normal((F, D))).astype(np.float32),
    }
    r = O.moe_forward(x, params, top_k=K, routing="sigmoid", routed_scaling_factor=2.5,
                      n_shared=1, dtype="bf16", precision="fp32", batch_shape=(B, S))
    a = r["aux"]
    return {"x": x, **{f"param_{k}": v for k, v in params.items()},
            "logits": r["logits"], "top_idx": r["top_idx"], "gates": r["gates"], "out": r["out"],
            "aux_losses": np.array([a["router_z_loss"], a["balance_loss"], a["mean_entropy"]]),
            "aux_expert_counts": a["expert_counts"],
            **{f"plan_{k}": r["plan"][k] for k in PLAN_KEYS}}


FIXTURES = {"tiny_fp32": tiny_fp32, "dispatch_identity_256": dispatch_identity_256,
            "reference_mode": reference_mode}


def main():
    for name, fn in FIXTURES.items():
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **fn())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
