"""MI355X-native GL-SDM transactional sparse-memory operator.

``glsdm.memory`` mirrors the reference's ``gl_sdm.memory`` API (views,
proposals, merge, commit, routed reads); ``glsdm.memory.backends.hip`` holds
the native entry points.  All compute runs in libglsdm.so (hand-written HIP
kernels for gfx950) through its C ABI; there is no CPU or torch fallback.
"""
from . import _native

__all__ = ["_native"]
