"""headshot_amd — headshot's fused per-layer ops as HIP kernels for MI355X.

``headshot_amd.context.HipContext`` is the op-dispatch surface (the
reference's ``GpuContext`` methods for LayerNorm, QK-norm + RoPE, GELU,
LayerScale + residual and token assembly); ``headshot_amd.rope`` builds the
RoPE tables. The kernels live in ``csrc/`` and are reached through the C ABI
declared in ``include/headshot_hip.h``.
"""
from . import _lib, rope  # noqa: F401

__all__ = ["HipContext", "rope"]


def __getattr__(name):
    # torch is imported only by users of the device surface.
    if name == "HipContext":
        from .context import HipContext
        return HipContext
    raise AttributeError(name)
