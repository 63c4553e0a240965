"""MI355X-native MoE layer of theorionic/hanuman (``model/moe.py``).

``MoE`` is exported here as the reference exports it from its model package
(``model/__init__.py:4``); it is imported on first use, so importing the
package loads neither torch nor the HIP library.
"""


def __getattr__(name):
    if name == "MoE":
        from .moe import MoE
        return MoE
    raise AttributeError(f"module 'hanuman_amd' has no attribute {name!r}")
