"""CPU oracle for the MoE-layer forward of theorionic/hanuman (``model/moe.py``).

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``hanuman_amd``) imports this
package.  It is imported by ``tests/``, by ``__graft_entry__.smoke()`` (as the
checker of one small GPU invocation) and by ``bench.py``'s ``cpu_baseline`` leg
(as the timed CPU restatement).  It is never a fallback for the GPU path.

Every function cites the reference line it restates.  The reference itself
(JAX 0.11 / Flax 0.12.8, Python >= 3.12) cannot run in this image: jax, jaxlib
and flax are absent, so the oracle is pinned by closed forms, library routines
(``np.argsort(kind="stable")``, ``np.bincount``, ``np.matmul``), brute force on
tiny inputs and torch-CPU dtype conversions.  See ``tests/test_oracle.py``.
"""
from .moe_oracle import *  # noqa: F401,F403
