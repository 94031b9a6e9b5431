"""vllm_espalier on MI355X (gfx950): the plugin's Python surface over hand-written HIP kernels.

Registered with vLLM through the vllm.general_plugins entry point (register()); the kernels live in
libespalier_hip.so (C ABI: include/espalier.h) and are reached through the espalier_ext torch extension.
(The surface of vllm_espalier/__init__.py:1-112; the vLLM serving patches there are not part of this package.)
"""
import os

# the switches that change which custom ops a compiled graph calls (vllm_espalier/__init__.py:12)
SWITCHES = ("ESPALIER_FUSED_DENSE", "ESPALIER_GROUPED_EXPERTS", "ESPALIER_FUSED_ROUTING", "ESPALIER_PREFILL_MODE")


def switches_salt() -> str:
    """The switch settings, as mixed into vLLM's compile-cache hash (vllm_espalier/__init__.py:15-22)."""
    return ",".join(f"{k}={os.environ.get(k, '')}" for k in SWITCHES)


def register():
    """vLLM plugin entry point: registers the espalier::* custom ops (and, when vLLM is importable, the quantisation
    method's modules)."""
    from . import ops  # noqa: F401
