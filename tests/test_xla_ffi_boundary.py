"""Source completeness of the XLA FFI boundary (runs without JAX or a GPU).

JAX and its FFI headers are absent from this image, so the handlers
(``hanuman_amd/xla_ffi/hmoe_xla_ffi.cc``) and the JAX module
(``hanuman_amd/xla_ffi/moe_jax.py``) cannot be built or run here.  These
checks read their text: every compute entry point of the C ABI has a
handler, every step of the training sequence that the integration guide
at the repository root binds has one, and the JAX
module's target table, its calls and the handler symbols agree.
"""
import ast
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "hanuman_moe.h"
FFI_CC = ROOT / "hanuman_amd" / "xla_ffi" / "hmoe_xla_ffi.cc"
JAX_PY = ROOT / "hanuman_amd" / "xla_ffi" / "moe_jax.py"
INTEGRATION = ROOT / "INTEGRATION.md"

# Entry points with no handler, and why.
NO_HANDLER = {
    # XLA hands every call its buffers; the library-held scratch array is for
    # callers that cannot allocate.
    "hmoe_dispatch_plan_noalloc",
    # a host-side query, no device work
    "hmoe_abi_version",
}


def _header_entry_points():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"^int\s+(hmoe_\w+)\s*\(", text, flags=re.M))


def _handlers():
    """handler symbol -> set of hmoe_* functions its implementation calls."""
    text = FFI_CC.read_text()
    impls = {}
    for m in re.finditer(r"static ffi::Error (\w+Impl)\(.*?\n}\n", text, flags=re.S):
        impls[m.group(1)] = set(re.findall(r"\b(hmoe_\w+)\(", m.group(0)))
    out = {}
    for sym, impl in re.findall(r"XLA_FFI_DEFINE_HANDLER_SYMBOL\(\s*(\w+),\s*(\w+)", text):
        out[sym] = impls[impl]
    return out


def _jax_targets():
    tree = ast.parse(JAX_PY.read_text())
    for node in ast.walk(tree):
        if isinstance(node, ast.Assign) and any(getattr(t, "id", None) == "TARGETS" for t in node.targets):
            return {k.value: v.value for k, v in zip(node.value.keys, node.value.values)}
    raise AssertionError("TARGETS not found")


def test_every_compute_entry_point_has_a_handler():
    called = set().union(*_handlers().values())
    missing = sorted(_header_entry_points() - called - NO_HANDLER)
    assert not missing, f"entry points without an XLA FFI handler: {missing}"


def test_integration_training_steps_have_handlers():
    text = INTEGRATION.read_text()
    start = text.index("Training goes through a `jax.custom_vjp`")
    end = text.index("With the float32 compute dtype", start)
    bound = set(re.findall(r"`(hmoe_\w+)", text[start:end]))
    bound -= {n for n in bound if n.endswith("_bytes")}
    assert len(bound) >= 15, sorted(bound)
    called = set().union(*_handlers().values())
    assert not sorted(bound - called), f"training steps without handlers: {sorted(bound - called)}"


def test_jax_targets_match_handler_symbols():
    targets = _jax_targets()
    handlers = _handlers()
    assert set(targets.values()) == set(handlers), (
        f"only in moe_jax: {sorted(set(targets.values()) - set(handlers))}; "
        f"only in the .cc: {sorted(set(handlers) - set(targets.values()))}")
    for name, sym in targets.items():
        assert name in handlers[sym], f"target {name} -> {sym}, which calls {sorted(handlers[sym])}"


def test_jax_module_calls_only_registered_targets():
    targets = _jax_targets()
    used = set(re.findall(r'_call\(\s*"(hmoe_\w+)"', JAX_PY.read_text()))
    assert used, "no custom calls found"
    assert used <= set(targets), sorted(used - set(targets))
    # the backward the custom_vjp binds, step by step
    for step in ("hmoe_combine_bwd", "hmoe_grouped_dgrad_down",
                 "hmoe_grouped_gate_up_swiglu_bwd_gather", "hmoe_grouped_dgrad_gate_up",
                 "hmoe_gather_bwd", "hmoe_router_bwd", "hmoe_router_aux_bwd", "hmoe_router_dx",
                 "hmoe_grouped_wgrad_gate_up", "hmoe_grouped_wgrad_down", "hmoe_router_dw"):
        assert step in used, step
    tree = ast.parse(JAX_PY.read_text())
    names = {n.name for n in ast.walk(tree) if isinstance(n, ast.FunctionDef)}
    assert {"moe_layer", "moe_call", "register", "_forward", "_backward"} <= names
